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
// lmh_reduce_kernel combines the partials of a row (running max rescaling,
// 16 lanes per row and a fixed merge tree).
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
// the same from a wave-uniform base (SGPRs) plus a 32-bit lane offset that stays
// in its register for the whole tile (only the scalar base advances per k-step)
__device__ __forceinline__ void lm_dma16_s(const void* sbase, uint32_t voff, uint32_t lds_byte_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_byte_addr) : "memory");
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

// SA: hidden's and weight's rows lie within 4 GiB of their bases (the host
// checks), so the copies take 32-bit lane offsets from scalar bases
template <int MODE, int BK, bool SA>
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
  uint32_t soff[2 * kLmCopies];  // SA: byte offsets from hidden / weight
  uint32_t dst_off[2 * kLmCopies];
#pragma unroll
  for (int j = 0; j < kLmCopies; ++j) {
    const int q = (w * kLmCopies + j) * 64 + lane;
    const int row = q / kLmCh;
    const int ch = Ring::swz(row, q % kLmCh);  // the swizzle is an involution
    const int64_t ea = (int64_t)min(m0 + row, M - 1) * ldh + ch * 8;  // clamped rows: results never stored
    const int64_t eb = (int64_t)min(v0 + row, V - 1) * ldw + ch * 8;
    src[j] = hidden + ea;
    src[kLmCopies + j] = weight + eb;
    soff[j] = (uint32_t)(ea * 2);
    soff[kLmCopies + j] = (uint32_t)(eb * 2);
    dst_off[j] = (uint32_t)((w * kLmCopies + j) * 1024);
    dst_off[kLmCopies + j] = (uint32_t)(kLmBM * kLmRowB + (w * kLmCopies + j) * 1024);
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lm_lds_addr(lds));
  const int nk = H / kLmBK;  // H % BK == 0 (the host picks BK)
  auto issue = [&](int kt) {
    const uint32_t base = lds0 + (uint32_t)((kt % kLmStages) * kLmStage);
#pragma unroll
    for (int j = 0; j < 2 * kLmCopies; ++j) {
      const uint32_t dst = __builtin_amdgcn_readfirstlane(base + dst_off[j]);  // wave-uniform
      if constexpr (SA)
        lm_dma16_s((const uint8_t*)(j < kLmCopies ? hidden : weight) + (int64_t)kt * kLmBK * 2, soff[j], dst);
      else
        lm_dma16(src[j] + kt * kLmBK, dst);
    }
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

// Combine of the per-tile (or per-chunk) partials of each row: block = 16 rows
// x 16 lanes; lane q of a row merges partials q, q + 16, ... in order, then the
// 16 lanes' results are merged pairwise by shuffles (a fixed tree, so the
// result does not depend on timing).  Merge of (m1, s1, t1) and (m2, s2, t2):
// m = max, s = s1 e^(m1 - m) + s2 e^(m2 - m), t likewise.
__device__ __forceinline__ void lmh_merge(float& m, float& s, float& t, float m2, float s2, float t2) {
  if (m2 == -INFINITY) return;
  if (m2 > m) {
    const float f = __expf(m - m2);  // 0 while m = -inf
    s = s * f + s2;
    t = t * f + t2;
    m = m2;
  } else {
    const float f = __expf(m2 - m);
    s += s2 * f;
    t += t2 * f;
  }
}

__global__ __launch_bounds__(256) void lmh_reduce_kernel(const float4* __restrict__ partials, int M, int n_vtiles,
                                                         const float* __restrict__ zlab,
                                                         const int64_t* __restrict__ labels, int V,
                                                         float* __restrict__ logprobs, float* __restrict__ entropy,
                                                         float* __restrict__ lse, float* __restrict__ ez) {
  const int q = threadIdx.x & 15;
  const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int rr = min(row, M - 1);  // rows past the end take part in the shuffles, store nothing
  float mx = -INFINITY, s = 0.f, t = 0.f;
  for (int j = q; j < n_vtiles; j += 16) {
    const float4 p = partials[(int64_t)j * M + rr];
    lmh_merge(mx, s, t, p.x, p.y, p.z);
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    const float m2 = __shfl_xor(mx, o), s2 = __shfl_xor(s, o), t2 = __shfl_xor(t, o);
    // both lanes of a pair merge in the same order (lower lane's values first)
    if (q & o) {
      float mm = m2, ss = s2, tt = t2;
      lmh_merge(mm, ss, tt, mx, s, t);
      mx = mm, s = ss, t = tt;
    } else {
      lmh_merge(mx, s, t, m2, s2, t2);
    }
  }
  if (q != 0 || row >= M) return;
  const float l = mx + __logf(s);
  const float e = t / s;
  const int64_t lab = labels[row];
  const float zl = (lab >= 0 && lab < V) ? zlab[row] : 0.f;
  logprobs[row] = zl - l;
  entropy[row] = l - e;
  lse[row] = l;
  ez[row] = e;
}

// Statistics of one vocabulary chunk of fp32 logits that a library GEMM wrote
// (logits [M][ldl], column j = entry v_begin + j): one wave per row, each lane
// a running (max, sum exp, sum exp * z) over its float4 groups (1 KB per wave
// load), then the wave's max, each lane's sums rescaled to it, and the wave's
// sums by shuffles; the row's label logit when its label lies in the chunk.
// Same partial as one column tile of lmh_gemm_kernel<0>, so lmh_reduce_kernel
// combines them.
__device__ __forceinline__ float lmh_wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float lmh_wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ __launch_bounds__(256) void lmh_chunk_stats_kernel(const float* __restrict__ logits, int64_t ldl, int M,
                                                              int n, int v_begin, const int64_t* __restrict__ labels,
                                                              float rcp_t, bool vec, float4* __restrict__ partial,
                                                              float* __restrict__ zlab) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float* zr = logits + (int64_t)row * ldl;
  float m = -INFINITY, s = 0.f, t = 0.f;
  auto add4 = [&](float x0, float x1, float x2, float x3) {
    const float lm = fmaxf(fmaxf(x0, x1), fmaxf(x2, x3));
    if (lm > m) {
      const float f = __expf(m - lm);  // 0 while m = -inf
      s *= f;
      t *= f;
      m = lm;
    }
    const float e0 = __expf(x0 - m), e1 = __expf(x1 - m), e2 = __expf(x2 - m), e3 = __expf(x3 - m);
    s += (e0 + e1) + (e2 + e3);
    t += (e0 * x0 + e1 * x1) + (e2 * x2 + e3 * x3);
  };
  int c0 = 0;
  if (vec) {  // 16-byte aligned rows: float4 groups, four in flight per lane, the tail below
    const int n4 = n >> 2;
    const float4* z4 = (const float4*)zr;
    int i = lane;
    for (; i + 192 < n4; i += 256) {
      const float4 a = z4[i], b = z4[i + 64], c = z4[i + 128], d = z4[i + 192];
      add4(a.x * rcp_t, a.y * rcp_t, a.z * rcp_t, a.w * rcp_t);
      add4(b.x * rcp_t, b.y * rcp_t, b.z * rcp_t, b.w * rcp_t);
      add4(c.x * rcp_t, c.y * rcp_t, c.z * rcp_t, c.w * rcp_t);
      add4(d.x * rcp_t, d.y * rcp_t, d.z * rcp_t, d.w * rcp_t);
    }
    for (; i < n4; i += 64) {
      const float4 a = z4[i];
      add4(a.x * rcp_t, a.y * rcp_t, a.z * rcp_t, a.w * rcp_t);
    }
    c0 = n4 * 4;
  }
  for (int c = c0 + lane; c < n; c += 64) {
    const float x = zr[c] * rcp_t;
    if (x > m) {
      const float f = __expf(m - x);
      s *= f;
      t *= f;
      m = x;
    }
    const float e = __expf(x - m);
    s += e;
    t += e * x;
  }
  const float mw = lmh_wave_max(m);
  const float f = m == -INFINITY ? 0.f : __expf(m - mw);
  const float sw = lmh_wave_sum(s * f);
  const float tw = lmh_wave_sum(t * f);
  if (lane == 0) {
    partial[row] = make_float4(mw, sw, tw, 0.f);
    const int64_t lab = labels[row];
    if (lab >= v_begin && lab < (int64_t)v_begin + n) zlab[row] = zr[lab - v_begin] * rcp_t;
  }
}

// Logits gradient of one vocabulary chunk from its fp32 logits (the formula of
// lmh_gemm_kernel<1>'s epilogue): block = (row, 2048 columns), 8 columns per
// thread, one 16-byte store of bf16 where the row allows it.
__global__ __launch_bounds__(256) void lmh_chunk_dz_kernel(const float* __restrict__ logits, int64_t ldl, int n,
                                                           int v_begin, int n_cb, const int64_t* __restrict__ labels,
                                                           float rcp_t, const float* __restrict__ lse,
                                                           const float* __restrict__ ez,
                                                           const float* __restrict__ dlp, int64_t dlp_stride,
                                                           float dlp_scale, const float* __restrict__ dent,
                                                           uint16_t* __restrict__ dz, int64_t lddz, bool vec) {
  const int row = blockIdx.x / n_cb;
  const int c = (blockIdx.x % n_cb) * 2048 + threadIdx.x * 8;
  if (c >= n) return;
  const float l_ = lse[row], e_ = ez[row], g_ = dlp[(int64_t)row * dlp_stride] * dlp_scale, h_ = dent[row];
  const int64_t lab64 = labels[row];
  const int lab = lab64 >= v_begin && lab64 < (int64_t)v_begin + n ? (int)(lab64 - v_begin) : -1;
  const float* zr = logits + (int64_t)row * ldl;
  uint16_t* dr = dz + (int64_t)row * lddz;
  auto grad = [&](float zv, int j) {
    const float x = zv * rcp_t;
    const float p = __expf(x - l_);
    return (g_ * ((j == lab ? 1.f : 0.f) - p) - h_ * p * (x - e_)) * rcp_t;
  };
  if (vec && c + 8 <= n) {
    const float4 a = *(const float4*)(zr + c), b = *(const float4*)(zr + c + 4);
    af3_u32x4 o;
    o[0] = af3_f32_to_bf16(grad(a.x, c)) | (af3_f32_to_bf16(grad(a.y, c + 1)) << 16);
    o[1] = af3_f32_to_bf16(grad(a.z, c + 2)) | (af3_f32_to_bf16(grad(a.w, c + 3)) << 16);
    o[2] = af3_f32_to_bf16(grad(b.x, c + 4)) | (af3_f32_to_bf16(grad(b.y, c + 5)) << 16);
    o[3] = af3_f32_to_bf16(grad(b.z, c + 6)) | (af3_f32_to_bf16(grad(b.w, c + 7)) << 16);
    *(af3_u32x4*)(dr + c) = o;
  } else {
    for (int j = c; j < min(c + 8, n); ++j) dr[j] = (uint16_t)af3_f32_to_bf16(grad(zr[j], j));
  }
}

// every copy of `rows` rows of stride ld (H columns) lies within 4 GiB of the base:
// the copies' lane offsets fit 32 bits
bool lm_off32(int rows, int64_t ld, int H) {
  return rows <= 0 || ((int64_t)(rows - 1) * ld + H) * 2 <= ((int64_t)1 << 32);
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
  const bool sa = lm_off32(M, ldh, H) && lm_off32(V, ldw, H);
#define AF3_LMH_FWD(BK, SA)                                                                                          \
  hipLaunchKernelGGL((lmh_gemm_kernel<0, BK, SA>), dim3(grid), dim3(kLmThreads), 0, stream, hidden, ldh, weight, ldw, M, \
                     V, H, 1.f / temperature, labels, nm, nv, px, partials, zlab, nullptr, nullptr, nullptr, 0, 0.f,  \
                     nullptr, nullptr, 0, 0)
  if (H % 64 == 0) {
    if (sa) AF3_LMH_FWD(64, true); else AF3_LMH_FWD(64, false);
  } else {
    if (sa) AF3_LMH_FWD(32, true); else AF3_LMH_FWD(32, false);
  }
#undef AF3_LMH_FWD
  int rc = af3::check_launch("lm_head_logprobs (gemm)");
  if (rc) return rc;
  hipLaunchKernelGGL(lmh_reduce_kernel, dim3((unsigned)af3_cdiv(M, 16)), dim3(256), 0, stream, partials, M, nv, zlab,
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
  const bool sa = lm_off32(M, ldh, H) && lm_off32(v_count, ldw, H);
#define AF3_LMH_DZ(BK, SA)                                                                                         \
  hipLaunchKernelGGL((lmh_gemm_kernel<1, BK, SA>), dim3(grid), dim3(kLmThreads), 0, stream, hidden, ldh, wr, ldw, M, \
                     v_count, H, 1.f / temperature, labels, nm, nv, px, nullptr, nullptr, lse, ez, dlogprobs,       \
                     dlp_stride, dlp_scale, dentropy, dz, lddz, (int64_t)v_begin)
  if (H % 64 == 0) {
    if (sa) AF3_LMH_DZ(64, true); else AF3_LMH_DZ(64, false);
  } else {
    if (sa) AF3_LMH_DZ(32, true); else AF3_LMH_DZ(32, false);
  }
#undef AF3_LMH_DZ
  return af3::check_launch("lm_head_dlogits");
}

extern "C" int af3_lm_head_dlogits(const uint16_t* hidden, int64_t ldh, const uint16_t* weight, int64_t ldw, int M,
                                   int V, int H, const int64_t* labels, float temperature, const float* lse,
                                   const float* ez, const float* dlogprobs, int64_t dlp_stride, float dlp_scale,
                                   const float* dentropy, uint16_t* dz, int64_t lddz, void* stream) {
  return af3_lm_head_dlogits_range(hidden, ldh, weight, ldw, M, 0, V, H, labels, temperature, lse, ez, dlogprobs,
                                   dlp_stride, dlp_scale, dentropy, dz, lddz, stream);
}

extern "C" int af3_lm_head_chunk_stats(const float* logits, int64_t ldl, int M, int v_begin, int v_count,
                                       const int64_t* labels, float temperature, void* partial, float* zlab,
                                       void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M >= 0 && v_begin >= 0 && v_count > 0 && ldl >= v_count, "lm_head_chunk_stats: bad shape");
  if (M == 0) return 0;
  AF3_REQUIRE(logits && labels && partial && zlab, "lm_head_chunk_stats: null pointer");
  AF3_REQUIRE(temperature > 0.f, "lm_head_chunk_stats: temperature must be positive");
  AF3_REQUIRE(((uintptr_t)partial & 15) == 0, "lm_head_chunk_stats: partials must be 16-byte aligned");
  const bool vec = ((uintptr_t)logits & 15) == 0 && ldl % 4 == 0;
  hipLaunchKernelGGL(lmh_chunk_stats_kernel, dim3((unsigned)af3_cdiv(M, 4)), dim3(256), 0, stream, logits, ldl, M,
                     v_count, v_begin, labels, 1.f / temperature, vec, (float4*)partial, zlab);
  return af3::check_launch("lm_head_chunk_stats");
}

extern "C" int af3_lm_head_reduce(const void* partials, int M, int n_parts, const float* zlab, const int64_t* labels,
                                  int V, float* logprobs, float* entropy, float* lse, float* ez, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M >= 0 && n_parts > 0 && V > 0, "lm_head_reduce: bad shape");
  if (M == 0) return 0;
  AF3_REQUIRE(partials && zlab && labels && logprobs && entropy && lse && ez, "lm_head_reduce: null pointer");
  AF3_REQUIRE(((uintptr_t)partials & 15) == 0, "lm_head_reduce: partials must be 16-byte aligned");
  hipLaunchKernelGGL(lmh_reduce_kernel, dim3((unsigned)af3_cdiv(M, 16)), dim3(256), 0, stream,
                     (const float4*)partials, M, n_parts, zlab, labels, V, logprobs, entropy, lse, ez);
  return af3::check_launch("lm_head_reduce");
}

extern "C" int af3_lm_head_dz_chunk(const float* logits, int64_t ldl, int M, int v_begin, int v_count,
                                    const int64_t* labels, float temperature, const float* lse, const float* ez,
                                    const float* dlogprobs, int64_t dlp_stride, float dlp_scale,
                                    const float* dentropy, uint16_t* dz, int64_t lddz, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M >= 0 && v_begin >= 0 && v_count > 0 && ldl >= v_count && lddz >= v_count,
              "lm_head_dz_chunk: bad shape");
  if (M == 0) return 0;
  AF3_REQUIRE(logits && labels && lse && ez && dlogprobs && dentropy && dz, "lm_head_dz_chunk: null pointer");
  AF3_REQUIRE(temperature > 0.f, "lm_head_dz_chunk: temperature must be positive");
  const int n_cb = (int)af3_cdiv(v_count, 2048);
  AF3_REQUIRE((int64_t)M * n_cb <= 0x7fffffffLL, "lm_head_dz_chunk: too many rows");
  const bool vec = ((uintptr_t)logits & 15) == 0 && ldl % 4 == 0 && ((uintptr_t)dz & 15) == 0 && lddz % 8 == 0;
  hipLaunchKernelGGL(lmh_chunk_dz_kernel, dim3((unsigned)(M * n_cb)), dim3(256), 0, stream, logits, ldl, v_count,
                     v_begin, n_cb, labels, 1.f / temperature, lse, ez, dlogprobs, dlp_stride, dlp_scale, dentropy, dz,
                     lddz, vec);
  return af3::check_launch("lm_head_dz_chunk");
}
