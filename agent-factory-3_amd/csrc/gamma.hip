// Gradient of the routing weights (gammas) of the down projection.
//
// The reference's down projection scales each expert row by its routing weight,
// Y[t] = sum_j gamma[r] * (I[r] W[e]^T + b[e]) with r = the sorted row of slot j
// (quantization.py:532-541), and returns no gradient for gamma
// (quantization.py:421).  With y[r] = I[r] W[e]^T + b[e] (+ the expert-LoRA term),
//
//   d gamma[r] = <dY[t(r)], y[r]> = <dY[t(r)] W[e] (+ LoRA), I[r]> + <dY[t(r)], b[e]>
//
// and the first product is the input gradient of the down projection before its
// gamma scaling, dI[r] / gamma[r], which the backward computes anyway.  So
//
//   out[r] = <dI[r], I[r]> / gamma[r] + <dY[t(r)], b[e(r)]>
//
// in fp32: one wave per row, 16-byte loads, a fixed shuffle reduction
// (deterministic).  The expert of row r is found by a binary search of
// token_offs (rows are expert-sorted).  A row whose gamma is exactly zero has
// dI = 0 and gets only the bias term.  HBM-bound: per row 2·N·2 B (dI, I) +
// H·2 B (the gathered dY row) read, 4 B written.
#include "af3_common.h"

namespace {

__device__ __forceinline__ float dot8_bf16(af3_u32x4 a, af3_u32x4 b) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += af3_bf16_to_f32(a[i] & 0xFFFFu) * af3_bf16_to_f32(b[i] & 0xFFFFu);
    s += af3_bf16_to_f32(a[i] >> 16) * af3_bf16_to_f32(b[i] >> 16);
  }
  return s;
}

__global__ __launch_bounds__(256) void gamma_grad_kernel(const uint16_t* __restrict__ d_act, int64_t ld_d,
                                                         const uint16_t* __restrict__ act, int64_t ld_a, int N,
                                                         const uint16_t* __restrict__ dy, int64_t ld_dy,
                                                         const int32_t* __restrict__ gather, int gdiv,
                                                         const float* __restrict__ bias, int H,
                                                         const int32_t* __restrict__ token_offs, int n_expts,
                                                         const uint16_t* __restrict__ gammas, int64_t R,
                                                         float* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  float s1 = 0.f;
  const uint16_t* dr = d_act + r * ld_d;
  const uint16_t* ar = act + r * ld_a;
  for (int c = lane * 8; c < N; c += 512)
    s1 += dot8_bf16(__builtin_nontemporal_load((const af3_u32x4*)(dr + c)),
                    __builtin_nontemporal_load((const af3_u32x4*)(ar + c)));
  float s2 = 0.f;
  if (bias) {
    int lo = 0, hi = n_expts - 1;  // last e with token_offs[e] <= r
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (token_offs[mid] <= r) lo = mid; else hi = mid - 1;
    }
    const int64_t t = gather ? gather[r] / gdiv : r;
    const uint16_t* yr = dy + t * ld_dy;
    const float* br = bias + (int64_t)lo * H;
    for (int c = lane * 8; c < H; c += 512) {
      const af3_u32x4 y = *(const af3_u32x4*)(yr + c);
      const float4 b0 = *(const float4*)(br + c);
      const float4 b1 = *(const float4*)(br + c + 4);
      s2 += af3_bf16_to_f32(y[0] & 0xFFFFu) * b0.x + af3_bf16_to_f32(y[0] >> 16) * b0.y +
            af3_bf16_to_f32(y[1] & 0xFFFFu) * b0.z + af3_bf16_to_f32(y[1] >> 16) * b0.w +
            af3_bf16_to_f32(y[2] & 0xFFFFu) * b1.x + af3_bf16_to_f32(y[2] >> 16) * b1.y +
            af3_bf16_to_f32(y[3] & 0xFFFFu) * b1.z + af3_bf16_to_f32(y[3] >> 16) * b1.w;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    s1 += __shfl_xor(s1, o);
    s2 += __shfl_xor(s2, o);
  }
  if (lane == 0) {
    const float g = af3_bf16_to_f32(gammas[r]);
    out[r] = (g != 0.f ? s1 / g : 0.f) + s2;
  }
}

}  // namespace

extern "C" int af3_gamma_grad(const uint16_t* d_act, int64_t ld_d, const uint16_t* act, int64_t ld_a, int N,
                              const uint16_t* dy, int64_t ld_dy, const int32_t* gather, int gdiv, const float* bias,
                              int H, const int32_t* token_offs, int n_expts, const uint16_t* gammas, int64_t R,
                              float* out, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(R >= 0 && N > 0 && N % 8 == 0, "gamma_grad: N must be a positive multiple of 8");
  if (R == 0) return 0;
  AF3_REQUIRE(d_act && act && gammas && out, "gamma_grad: null pointer");
  AF3_REQUIRE(ld_d % 8 == 0 && ld_a % 8 == 0 && ((uintptr_t)d_act & 15) == 0 && ((uintptr_t)act & 15) == 0,
              "gamma_grad: dI / I rows must be 16-byte aligned");
  if (bias) {
    AF3_REQUIRE(dy && token_offs && n_expts > 0 && H > 0 && H % 8 == 0 && gdiv > 0, "gamma_grad: bad bias term");
    AF3_REQUIRE(ld_dy % 8 == 0 && ((uintptr_t)dy & 15) == 0 && ((uintptr_t)bias & 15) == 0,
                "gamma_grad: dY rows and bias must be 16-byte aligned");
  }
  const int64_t grid = af3_cdiv(R, 4);
  AF3_REQUIRE(grid <= 0x7fffffffLL, "gamma_grad: too many rows");
  hipLaunchKernelGGL(gamma_grad_kernel, dim3((unsigned)grid), dim3(256), 0, stream, d_act, ld_d, act, ld_a, N, dy,
                     ld_dy, gather, gdiv, bias, H, token_offs, n_expts, gammas, R, out);
  return af3::check_launch("gamma_grad");
}
