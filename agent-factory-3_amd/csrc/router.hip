// Router logits of the gpt-oss MoE layer on bf16 MFMA.
//
// Reference behaviour (quantization.py:653-654, mlp_forward):
//   router_logits = nn.functional.linear(hidden_states, router.weight, router.bias)
// i.e. logits[t][e] = bf16(sum_k x[t][k] W[e][k] + b[e]) with fp32 sums, for
// hidden_states [T, H] bf16, W [E, H] bf16, b [E] bf16.  The logits then feed
// the top-k / replay routing (routing.hip).
//
// The product is skinny (E = 32 or 128 columns) and reads every activation
// row once, so it is HBM-bound on x: a block takes 64 rows (two waves of 32)
// by all E columns.  Each lane loads its A fragments straight from global
// memory (64 contiguous bytes of one row per 64-deep k-step, one k-step
// ahead in registers); the W tile of the k-step ([E][64] bf16, 16-byte chunks
// XOR-swizzled by row) is staged in LDS once per block and shared by both
// waves, double-buffered.  k is permuted identically on both operands, so
// lane (r, h) of v_mfma_f32_32x32x16_bf16 feeds k = 32 h + 8 s + (0..7) at
// sub-step s: a lane's four A fragments are one contiguous 64-byte run.
#include "af3_common.h"

namespace {

constexpr int kRtRows = 64;  // rows per block (2 waves x 32)
constexpr int kRtBK = 64;    // k per step

// LDS element offset of 16-byte chunk c of W-tile row n
__device__ __forceinline__ int rt_off(int n, int c) { return n * kRtBK + ((c ^ (n & 7)) << 3); }

template <int TN>
__global__ __launch_bounds__(128) void router_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                     const uint16_t* __restrict__ w, int64_t ldw,
                                                     const uint16_t* __restrict__ bias, int64_t T, int H, int E,
                                                     uint16_t* __restrict__ out, int64_t ldo) {
  constexpr int EP = TN * 32;                // columns computed (E rounded up to whole sub-tiles)
  constexpr int WPT = EP * kRtBK / 8 / 128;  // 16-byte W chunks per thread per k-step
  __shared__ __attribute__((aligned(16))) uint16_t ws[2][EP * kRtBK];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t row = (int64_t)blockIdx.x * kRtRows + wave * 32 + lr;
  const uint16_t* xr = x + (row < T ? row : T - 1) * ldx + lh * 32;
  const int nk = H / kRtBK;

  af3_u32x4 xa[4], wv[WPT];
  auto load_x = [&](int kk) {
#pragma unroll
    for (int s = 0; s < 4; ++s) xa[s] = *(const af3_u32x4*)(xr + kk * kRtBK + s * 8);
  };
  auto load_w = [&](int kk) {
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      const int id = j * 128 + threadIdx.x;
      const int n = min(id >> 3, E - 1);  // rows past E: any valid row (their columns are not stored)
      wv[j] = *(const af3_u32x4*)(w + (int64_t)n * ldw + kk * kRtBK + (id & 7) * 8);
    }
  };
  auto store_w = [&](int buf) {
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      const int id = j * 128 + threadIdx.x;
      *(af3_u32x4*)(ws[buf] + rt_off(id >> 3, id & 7)) = wv[j];
    }
  };

  af3_f32x16 acc[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;

  load_w(0);
  load_x(0);
  store_w(0);
  __syncthreads();
  for (int kk = 0; kk < nk; ++kk) {
    const int buf = kk & 1;
    af3_u32x4 xc[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) xc[s] = xa[s];
    if (kk + 1 < nk) {  // next k-step's operands in flight during this one's MFMAs
      load_w(kk + 1);
      load_x(kk + 1);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const af3_bf16x8 a = __builtin_bit_cast(af3_bf16x8, xc[s]);
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const af3_bf16x8 b = *(const af3_bf16x8*)(ws[buf] + rt_off(t * 32 + lr, lh * 4 + s));
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[t], 0, 0, 0);
      }
    }
    if (kk + 1 < nk) {
      store_w(buf ^ 1);  // the other buffer was last read in k-step kk - 1 (before the barrier below it)
      __syncthreads();
    }
  }
  // epilogue: lane (c, h) of sub-tile t holds rows 8 j + 4 h + q, column t * 32 + c
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int col = t * 32 + lr;
    if (col >= E) continue;
    const float b = bias ? af3_bf16_to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t r = (int64_t)blockIdx.x * kRtRows + wave * 32 + 8 * j + 4 * lh + q;
        if (r < T) out[r * ldo + col] = (uint16_t)af3_f32_to_bf16(acc[t][4 * j + q] + b);
      }
  }
}

}  // namespace

extern "C" int af3_router_logits(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw, const uint16_t* bias,
                                 int64_t n_tokens, int hidden, int n_expts, uint16_t* logits, int64_t ld_logits,
                                 void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_tokens >= 0 && hidden > 0 && n_expts > 0, "router_logits: bad sizes");
  AF3_REQUIRE(n_expts <= 256, "router_logits: E=%d above 256", n_expts);
  AF3_REQUIRE(hidden % kRtBK == 0, "router_logits: hidden size %d must be a multiple of %d", hidden, kRtBK);
  AF3_REQUIRE(ldx >= hidden && ldw >= hidden && ld_logits >= n_expts, "router_logits: bad leading dimensions");
  AF3_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0,
              "router_logits: x and W rows must be 16-byte aligned");
  if (n_tokens == 0) return 0;
  AF3_REQUIRE(x && w && logits, "router_logits: null pointer");
  const dim3 grid((unsigned)af3_cdiv(n_tokens, kRtRows)), block(128);
  switch ((n_expts + 31) / 32) {
#define AF3_RT(tn) \
  case tn:         \
    hipLaunchKernelGGL(router_kernel<tn>, grid, block, 0, stream, x, ldx, w, ldw, bias, n_tokens, hidden, n_expts, logits, ld_logits); \
    break;
    AF3_RT(1) AF3_RT(2) AF3_RT(3) AF3_RT(4) AF3_RT(5) AF3_RT(6) AF3_RT(7) AF3_RT(8)
#undef AF3_RT
  }
  return af3::check_launch("router_logits");
}
