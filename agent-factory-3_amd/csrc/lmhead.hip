// LM-head log-probabilities and entropy without materialised logits.
//
// Restates the fused linear cross entropy of the reference's trainer
// (trainer/losses/kernels.py:157-385 forward, 704-880 backward logits,
// wrapper trainer/losses/linear_cross_entropy.py): with z = hidden @ W^T / T
// (hidden [M][H], W [V][H] bf16, fp32 accumulation),
//
//   logprob[m] = z[m][label[m]] - lse[m],   lse = max + log(sum exp(z - max))
//   entropy[m] = lse[m] - E_p[z][m],        E_p[z] = sum exp(z - max) z / sum exp(z - max)
//
// and, for the backward, the logits gradient
//
//   dz[m][v] = ( dlp[m] (onehot - p) - dent[m] p (z - E_p[z]) ) / T
//
// which two plain GEMMs turn into d_hidden = dz W and d_weight = dz^T hidden.
//
// lmh_gemm_kernel<MODE>: one 256 (rows) x 256 (vocabulary) tile per block of
// 8 waves (2 x 4, 128 x 64 each), v_mfma_f32_32x32x16_bf16, a 128 KB global->LDS
// ring (global_load_lds_dwordx4): 64-deep k-steps in 2 stages when H % 64 == 0,
// else 32-deep in 4 stages; one barrier per k-step; 16-byte chunks XOR-swizzled
// so the fragment reads of 16 lanes hit distinct banks.  Blocks are ordered
// vocabulary-tile-major and dealt to the XCDs in contiguous runs, so the row
// tiles that reuse one W tile run together on one L2.
//   MODE 0: per row and tile, (max, sum exp, sum exp * z) over the tile's 256
//   columns (wave-wide shuffle reductions, then the four column waves through
//   LDS) -> partials [n_vtiles][M] float4; the row's label logit is stored by
//   the one lane that holds it.
//   MODE 1: dz for the tile from the row statistics of the forward, bf16.
// lmh_reduce_kernel combines the partials of a row (running max rescaling).
#include "af3_common.h"

namespace {

constexpr int kLmBM = 256, kLmBN = 256;
constexpr int kLmLds = 128 * 1024;
// waves: 2 along the rows (128 each) x kLmWN along the vocabulary columns
constexpr int kLmWN = 4;
constexpr int kLmWaves = 2 * kLmWN, kLmThreads = 64 * kLmWaves;
constexpr int kLmTN = kLmBN / kLmWN / 32;  // 32-column sub-tiles per wave

// Ring geometry per k-step depth: 64 (H % 64 == 0; 2 stages, one k-step ahead)
// or 32 (4 stages, three ahead), 128 KB either way.
template <int BK>
struct LmRing {
  static constexpr int kRowB = BK * 2;                      // bytes per tile row and k-step
  static constexpr int kCh = kRowB / 16;                    // 16-byte chunks per row
  static constexpr int kStage = (kLmBM + kLmBN) * kRowB;    // bytes per stage (A then B)
  static constexpr int kStages = kLmLds / kStage;
  static constexpr int kCopies = kLmBM * kRowB / 1024 / kLmWaves;  // 1 KB copies per wave and operand
  static_assert(kLmBM == kLmBN && kCopies * kLmWaves * 1024 == kLmBM * kRowB, "copy plan covers each operand once");
  static_assert(kStages >= 2 && kStages <= 4, "ring depth");
  // 16-byte chunk position of (row, chunk) in an LDS row: rows that share banks
  // (4 apart for 64-byte rows, 2 apart for 128-byte rows) take different positions,
  // so 16 lanes reading one chunk of 16 rows hit distinct banks; an involution
  static __device__ __forceinline__ int swz(int row, int chunk) {
    return kCh == 4 ? chunk ^ ((row >> 2) & 3) : chunk ^ ((row >> 1) & 7);
  }
};

// global -> LDS copy of 16 bytes per lane (lane i lands at m0 + 16 i); issued by
// inline assembly with explicit vmcnt waits, so the compiler's wait-count pass
// places no wait for the whole ring before the first LDS read of a stage
__device__ __forceinline__ void lm_dma16(const void* gptr, uint32_t lds_byte_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds_byte_addr) : "memory");
}
template <int N>
__device__ __forceinline__ void lm_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
#define LM_BARRIER() asm volatile("s_barrier" ::: "memory")
__device__ __forceinline__ uint32_t lm_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Reductions over each 32-lane half of a wave, every lane receiving the result:
// DPP quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror (partners
// within 4, 8 and 16 lanes), then ds_swizzle xor 16 (bit mode, and 0x1f).
template <int CTRL>
__device__ __forceinline__ float lm_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lm_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

__device__ __forceinline__ float wave32_max(float v) {
  v = fmaxf(v, lm_dpp<0xB1>(v));
  v = fmaxf(v, lm_dpp<0x4E>(v));
  v = fmaxf(v, lm_dpp<0x141>(v));
  v = fmaxf(v, lm_dpp<0x140>(v));
  return fmaxf(v, lm_xor16(v));
}

__device__ __forceinline__ float wave32_sum(float v) {
  v += lm_dpp<0xB1>(v);
  v += lm_dpp<0x4E>(v);
  v += lm_dpp<0x141>(v);
  v += lm_dpp<0x140>(v);
  return v + lm_xor16(v);
}

template <int MODE, int BK>
__global__ __launch_bounds__(kLmThreads, 1) void lmh_gemm_kernel(
    const uint16_t* __restrict__ hidden, int64_t ldh, const uint16_t* __restrict__ weight, int64_t ldw, int M, int V,
    int H, float rcp_t, const int64_t* __restrict__ labels, int n_mtiles, int n_vtiles, int per_xcd,
    // MODE 0
    float4* __restrict__ partials, float* __restrict__ zlab,
    // MODE 1
    const float* __restrict__ lse, const float* __restrict__ ez, const float* __restrict__ dlp, int64_t dlp_stride,
    float dlp_scale, const float* __restrict__ dent, uint16_t* __restrict__ dz, int64_t lddz, int64_t voff) {
  using Ring = LmRing<BK>;
  constexpr int kLmBK = BK, kLmRowB = Ring::kRowB, kLmCh = Ring::kCh, kLmStage = Ring::kStage;
  constexpr int kLmStages = Ring::kStages, kLmCopies = Ring::kCopies;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLmLds];
  const int xcd = blockIdx.x & 7;
  const int tile = xcd * per_xcd + (int)(blockIdx.x >> 3);
  if (tile >= n_mtiles * n_vtiles || tile >= (xcd + 1) * per_xcd) return;
  const int vt = tile / n_mtiles;
  const int mt = tile % n_mtiles;
  const int m0 = mt * kLmBM, v0 = vt * kLmBN;
  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int wm0 = (w / kLmWN) * 128, wn0 = (w % kLmWN) * (kLmBN / kLmWN);

  // global -> LDS copies: stage slot q (16 bytes) of the A (B) half holds row q / 4,
  // chunk (q % 4) ^ swizzle(row); wave w copies slots (w * kLmCopies + j) * 64 + lane
  const uint16_t* src[2 * kLmCopies];
  uint32_t dst_off[2 * kLmCopies];
#pragma unroll
  for (int j = 0; j < kLmCopies; ++j) {
    const int q = (w * kLmCopies + j) * 64 + lane;
    const int row = q / kLmCh;
    const int ch = Ring::swz(row, q % kLmCh);  // the swizzle is an involution
    src[j] = hidden + (int64_t)min(m0 + row, M - 1) * ldh + ch * 8;             // clamped rows: results never stored
    src[kLmCopies + j] = weight + (int64_t)min(v0 + row, V - 1) * ldw + ch * 8;
    dst_off[j] = (uint32_t)((w * kLmCopies + j) * 1024);
    dst_off[kLmCopies + j] = (uint32_t)(kLmBM * kLmRowB + (w * kLmCopies + j) * 1024);
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lm_lds_addr(lds));
  const int nk = H / kLmBK;  // H % BK == 0 (the host picks BK)
  auto issue = [&](int kt) {
    const uint32_t base = lds0 + (uint32_t)((kt % kLmStages) * kLmStage);
#pragma unroll
    for (int j = 0; j < 2 * kLmCopies; ++j)
      lm_dma16(src[j] + kt * kLmBK, __builtin_amdgcn_readfirstlane(base + dst_off[j]));  // wave-uniform
  };

  af3_f32x16 acc[4][kLmTN];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kLmTN; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

#pragma unroll
  for (int kt = 0; kt < kLmStages - 1; ++kt)
    if (kt < nk) issue(kt);
  for (int kt = 0; kt < nk; ++kt) {
    // this wave's copies of k-step kt have landed once at most those of the (up to
    // kLmStages - 2) later k-steps already issued are in flight
    constexpr int kCpw = 2 * kLmCopies;
    const int newer = min(kLmStages - 2, nk - 1 - kt);
    if (newer >= 2)
      lm_wait_vm<2 * kCpw>();
    else if (newer == 1)
      lm_wait_vm<kCpw>();
    else
      lm_wait_vm<0>();
    LM_BARRIER();  // every wave's copies of kt visible; every wave done with kt-1's stage
    if (kt + kLmStages - 1 < nk) issue(kt + kLmStages - 1);
    const uint8_t* As = lds + (kt % kLmStages) * kLmStage;
    const uint8_t* Bs = As + kLmBM * kLmRowB;
#pragma unroll
    for (int ks = 0; ks < kLmBK / 16; ++ks) {
      const int ch = ks * 2 + (lane >> 5);
      af3_u32x4 af[4], bf[kLmTN];
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        const int row = wm0 + tm * 32 + (lane & 31);
        af[tm] = *(const af3_u32x4*)(As + row * kLmRowB + 16 * Ring::swz(row, ch));
      }
#pragma unroll
      for (int tn = 0; tn < kLmTN; ++tn) {
        const int row = wn0 + tn * 32 + (lane & 31);
        bf[tn] = *(const af3_u32x4*)(Bs + row * kLmRowB + 16 * Ring::swz(row, ch));
      }
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
#pragma unroll
        for (int tn = 0; tn < kLmTN; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(af3_bf16x8, af[tm]),
                                                                __builtin_bit_cast(af3_bf16x8, bf[tn]),
                                                                acc[tm][tn], 0, 0, 0);
    }
  }
  __syncthreads();  // all fragment reads done before the epilogue reuses the LDS

  const int c0 = v0 + wn0 + (lane & 31);  // this lane's columns c0 + 32 tn
  if constexpr (MODE == 0) {
    float* part = (float*)lds;  // [256 rows][kLmWN column waves][3]
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rl = wm0 + tm * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        const int row = m0 + rl;
        float z[kLmTN];
        bool ok[kLmTN];
        float lm = -INFINITY;
#pragma unroll
        for (int tn = 0; tn < kLmTN; ++tn) {
          z[tn] = acc[tm][tn][i] * rcp_t;
          ok[tn] = c0 + 32 * tn < V;
          lm = fmaxf(lm, ok[tn] ? z[tn] : -INFINITY);
        }
        const float mx = wave32_max(lm);
        float se = 0.f, te = 0.f;
#pragma unroll
        for (int tn = 0; tn < kLmTN; ++tn) {
          const float e = ok[tn] ? __expf(z[tn] - mx) : 0.f;
          se += e;
          te += ok[tn] ? e * z[tn] : 0.f;
        }
        const float s = wave32_sum(se);
        const float t = wave32_sum(te);
        if ((lane & 31) == 0) {
          float* pp = part + (rl * kLmWN + (w % kLmWN)) * 3;
          pp[0] = mx;
          pp[1] = s;
          pp[2] = t;
        }
        if (row < M) {
          const int64_t lab = labels[row];
#pragma unroll
          for (int tn = 0; tn < kLmTN; ++tn)
            if (ok[tn] && lab == c0 + 32 * tn) zlab[row] = z[tn];
        }
      }
    }
    __syncthreads();
    if (tid < kLmBM && m0 + tid < M) {
      const float* pp = part + tid * 3 * kLmWN;
      float mx = -INFINITY;
#pragma unroll
      for (int q = 0; q < kLmWN; ++q) mx = fmaxf(mx, pp[3 * q]);
      float s = 0.f, t = 0.f;
#pragma unroll
      for (int q = 0; q < kLmWN; ++q) {
        const float f = pp[3 * q] == -INFINITY ? 0.f : __expf(pp[3 * q] - mx);
        s += pp[3 * q + 1] * f;
        t += pp[3 * q + 2] * f;
      }
      partials[(int64_t)vt * M + m0 + tid] = make_float4(mx, s, t, 0.f);
    }
  } else {
    float* rs = (float*)lds;  // per row: lse, E_p[z], dlp, dent, label (as float bits)
    if (tid < kLmBM) {
      const int row = min(m0 + tid, M - 1);
      rs[tid * 5 + 0] = lse[row];
      rs[tid * 5 + 1] = ez[row];
      rs[tid * 5 + 2] = dlp[(int64_t)row * dlp_stride] * dlp_scale;
      rs[tid * 5 + 3] = dent[row];
      const int64_t lab = labels[row];
      // the tile's columns are vocabulary entries voff .. voff + V - 1
      rs[tid * 5 + 4] = __int_as_float(lab >= voff && lab < voff + V ? (int)(lab - voff) : -1);
    }
    __syncthreads();
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rl = wm0 + tm * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        const int row = m0 + rl;
        if (row >= M) continue;
        const float* r = rs + rl * 5;
        const float l_ = r[0], e_ = r[1], g_ = r[2], h_ = r[3];
        const int lab = __float_as_int(r[4]);
        uint16_t* drow = dz + (int64_t)row * lddz;
#pragma unroll
        for (int tn = 0; tn < kLmTN; ++tn) {
          const int c = c0 + tn * 32;
          if (c >= V) continue;
          const float z = acc[tm][tn][i] * rcp_t;
          const float p = __expf(z - l_);
          const float d = (g_ * ((c == lab ? 1.f : 0.f) - p) - h_ * p * (z - e_)) * rcp_t;
          drow[c] = (uint16_t)af3_f32_to_bf16(d);
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void lmh_reduce_kernel(const float4* __restrict__ partials, int M, int n_vtiles,
                                                         const float* __restrict__ zlab,
                                                         const int64_t* __restrict__ labels, int V,
                                                         float* __restrict__ logprobs, float* __restrict__ entropy,
                                                         float* __restrict__ lse, float* __restrict__ ez) {
  const int row = blockIdx.x * 256 + threadIdx.x;
  if (row >= M) return;
  float mx = -INFINITY, s = 0.f, t = 0.f;
  for (int j = 0; j < n_vtiles; ++j) {
    const float4 p = partials[(int64_t)j * M + row];
    if (p.x == -INFINITY) continue;
    if (p.x > mx) {
      const float f = __expf(mx - p.x);  // 0 on the first tile (mx = -inf)
      s = s * f + p.y;
      t = t * f + p.z;
      mx = p.x;
    } else {
      const float f = __expf(p.x - mx);
      s += p.y * f;
      t += p.z * f;
    }
  }
  const float l = mx + __logf(s);
  const float e = t / s;
  const int64_t lab = labels[row];
  const float zl = (lab >= 0 && lab < V) ? zlab[row] : 0.f;
  logprobs[row] = zl - l;
  entropy[row] = l - e;
  lse[row] = l;
  ez[row] = e;
}

int lmh_grid(int M, int V, int& n_mtiles, int& n_vtiles, int& per_xcd) {
  n_mtiles = (int)af3_cdiv(M, kLmBM);
  n_vtiles = (int)af3_cdiv(V, kLmBN);
  const int64_t tiles = (int64_t)n_mtiles * n_vtiles;
  per_xcd = (int)af3_cdiv(tiles, 8);
  return 8 * per_xcd;
}

}  // namespace

extern "C" size_t af3_lm_head_workspace_bytes(int M, int V) {
  return (size_t)af3_cdiv(V, kLmBN) * (size_t)(M > 0 ? M : 0) * sizeof(float4) + (size_t)(M > 0 ? M : 0) * 4;
}

extern "C" int af3_lm_head_logprobs(const uint16_t* hidden, int64_t ldh, const uint16_t* weight, int64_t ldw, int M,
                                    int V, int H, const int64_t* labels, float temperature, float* logprobs,
                                    float* entropy, float* lse, float* ez, void* workspace, size_t ws_bytes,
                                    void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M >= 0 && V > 0 && H > 0 && H % 32 == 0, "lm_head_logprobs: H must be a positive multiple of 32");
  if (M == 0) return 0;
  AF3_REQUIRE(hidden && weight && labels && logprobs && entropy && lse && ez && workspace,
              "lm_head_logprobs: null pointer");
  AF3_REQUIRE(temperature > 0.f, "lm_head_logprobs: temperature must be positive");
  AF3_REQUIRE(ldh % 8 == 0 && ldw % 8 == 0 && ((uintptr_t)hidden & 15) == 0 && ((uintptr_t)weight & 15) == 0,
              "lm_head_logprobs: rows must be 16-byte aligned");
  AF3_REQUIRE(ws_bytes >= af3_lm_head_workspace_bytes(M, V) && ((uintptr_t)workspace & 15) == 0,
              "lm_head_logprobs: workspace too small or misaligned");
  int nm, nv, px;
  const int grid = lmh_grid(M, V, nm, nv, px);
  float4* partials = (float4*)workspace;
  float* zlab = (float*)((uint8_t*)workspace + (size_t)nv * M * sizeof(float4));
  if (H % 64 == 0)
    hipLaunchKernelGGL((lmh_gemm_kernel<0, 64>), dim3(grid), dim3(kLmThreads), 0, stream, hidden, ldh, weight, ldw, M, V, H,
                       1.f / temperature, labels, nm, nv, px, partials, zlab, nullptr, nullptr, nullptr, 0, 0.f,
                       nullptr, nullptr, 0, 0);
  else
    hipLaunchKernelGGL((lmh_gemm_kernel<0, 32>), dim3(grid), dim3(kLmThreads), 0, stream, hidden, ldh, weight, ldw, M, V, H,
                       1.f / temperature, labels, nm, nv, px, partials, zlab, nullptr, nullptr, nullptr, 0, 0.f,
                       nullptr, nullptr, 0, 0);
  int rc = af3::check_launch("lm_head_logprobs (gemm)");
  if (rc) return rc;
  hipLaunchKernelGGL(lmh_reduce_kernel, dim3((unsigned)af3_cdiv(M, 256)), dim3(256), 0, stream, partials, M, nv, zlab,
                     labels, V, logprobs, entropy, lse, ez);
  return af3::check_launch("lm_head_logprobs (reduce)");
}

extern "C" int af3_lm_head_dlogits_range(const uint16_t* hidden, int64_t ldh, const uint16_t* weight, int64_t ldw,
                                         int M, int v_begin, int v_count, int H, const int64_t* labels,
                                         float temperature, const float* lse, const float* ez, const float* dlogprobs,
                                         int64_t dlp_stride, float dlp_scale, const float* dentropy, uint16_t* dz,
                                         int64_t lddz, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M >= 0 && v_begin >= 0 && v_count > 0 && H > 0 && H % 32 == 0,
              "lm_head_dlogits: need v_begin >= 0, v_count > 0 and H a positive multiple of 32");
  if (M == 0) return 0;
  AF3_REQUIRE(hidden && weight && labels && lse && ez && dlogprobs && dentropy && dz, "lm_head_dlogits: null pointer");
  AF3_REQUIRE(temperature > 0.f, "lm_head_dlogits: temperature must be positive");
  AF3_REQUIRE(ldh % 8 == 0 && ldw % 8 == 0 && ((uintptr_t)hidden & 15) == 0 && ((uintptr_t)weight & 15) == 0 &&
                  lddz >= v_count,
              "lm_head_dlogits: rows must be 16-byte aligned");
  const uint16_t* wr = weight + (int64_t)v_begin * ldw;  // vocabulary rows v_begin .. v_begin + v_count - 1
  int nm, nv, px;
  const int grid = lmh_grid(M, v_count, nm, nv, px);
  if (H % 64 == 0)
    hipLaunchKernelGGL((lmh_gemm_kernel<1, 64>), dim3(grid), dim3(kLmThreads), 0, stream, hidden, ldh, wr, ldw, M,
                       v_count, H, 1.f / temperature, labels, nm, nv, px, nullptr, nullptr, lse, ez, dlogprobs,
                       dlp_stride, dlp_scale, dentropy, dz, lddz, (int64_t)v_begin);
  else
    hipLaunchKernelGGL((lmh_gemm_kernel<1, 32>), dim3(grid), dim3(kLmThreads), 0, stream, hidden, ldh, wr, ldw, M,
                       v_count, H, 1.f / temperature, labels, nm, nv, px, nullptr, nullptr, lse, ez, dlogprobs,
                       dlp_stride, dlp_scale, dentropy, dz, lddz, (int64_t)v_begin);
  return af3::check_launch("lm_head_dlogits");
}

extern "C" int af3_lm_head_dlogits(const uint16_t* hidden, int64_t ldh, const uint16_t* weight, int64_t ldw, int M,
                                   int V, int H, const int64_t* labels, float temperature, const float* lse,
                                   const float* ez, const float* dlogprobs, int64_t dlp_stride, float dlp_scale,
                                   const float* dentropy, uint16_t* dz, int64_t lddz, void* stream) {
  return af3_lm_head_dlogits_range(hidden, ldh, weight, ldw, M, 0, V, H, labels, temperature, lse, ez, dlogprobs,
                                   dlp_stride, dlp_scale, dentropy, dz, lddz, stream);
}
