// Expert-LoRA kernels (rank 16 or 32) on the streaming path.
//
// The expert LoRA of this build (no reference counterpart: the reference puts
// LoRA on attention only; convention W_eff = W + s * B @ A from PEFT as used at
// model_trainer.py:665,711) needs, per projection:
//   rows   out[r][j]  = s * sum_k X[a(r)][k] * Wl[e][j][k]      (L = s X A^T, u = s dY B)
//   wgrad  G[e]       = sum_{r in e} rs(r) * Big[b(r)][:]^T  (x)  Small[r][:]
//                        (dB = dY^T L  and  dA = u^T X)
// Both are skinny (the rank is the narrow side) and bound by reading the wide
// activation matrix once.  Both kernels stream that matrix through LDS with
// global->LDS copies (inline assembly, explicit vmcnt waits) a few k-steps
// ahead and keep the MFMA work on v_mfma_f32_32x32x16_bf16.  For the weight
// gradient the reduction runs over rows, so both MFMA operands come out of
// LDS through the gfx950 transposing read ds_read_b64_tr_b16: in a group of 16
// lanes, lane q points at 4 consecutive 16-bit values of row q / 4, columns
// 4 (q % 4) ..; lane i of the group receives the 4 values of column i of the
// 4 rows.
//
// Entry points (host side) return AF3_EUNSUPPORTED for shapes they do not
// cover; the callers in moe_gemm.hip then use the general kernels.
#include "af3_common.h"

namespace {

typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ void l_dma16(const void* gptr, uint32_t lds_byte_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds_byte_addr) : "memory");
}
// the same from a wave-uniform base (SGPRs) plus a 32-bit lane offset: the
// 32-bit offset arithmetic replaces a 64-bit address per copy
__device__ __forceinline__ void l_dma16_s(const void* sbase, uint32_t voff, uint32_t lds_byte_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_byte_addr) : "memory");
}
#define L_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")
// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 31] (the count is an immediate)
__device__ __forceinline__ void l_wait_vm(int n) {
  switch (n) {
    case 1: L_WAIT_VM(1); break;
    case 2: L_WAIT_VM(2); break;
    case 3: L_WAIT_VM(3); break;
    case 4: L_WAIT_VM(4); break;
    case 5: L_WAIT_VM(5); break;
    case 6: L_WAIT_VM(6); break;
    case 7: L_WAIT_VM(7); break;
    case 8: L_WAIT_VM(8); break;
    case 9: L_WAIT_VM(9); break;
    case 10: L_WAIT_VM(10); break;
    case 11: L_WAIT_VM(11); break;
    case 12: L_WAIT_VM(12); break;
    case 13: L_WAIT_VM(13); break;
    case 14: L_WAIT_VM(14); break;
    case 15: L_WAIT_VM(15); break;
    case 16: L_WAIT_VM(16); break;
    case 17: L_WAIT_VM(17); break;
    case 18: L_WAIT_VM(18); break;
    case 19: L_WAIT_VM(19); break;
    case 20: L_WAIT_VM(20); break;
    case 21: L_WAIT_VM(21); break;
    case 22: L_WAIT_VM(22); break;
    case 23: L_WAIT_VM(23); break;
    case 24: L_WAIT_VM(24); break;
    case 25: L_WAIT_VM(25); break;
    case 26: L_WAIT_VM(26); break;
    case 27: L_WAIT_VM(27); break;
    case 28: L_WAIT_VM(28); break;
    case 29: L_WAIT_VM(29); break;
    case 30: L_WAIT_VM(30); break;
    case 31: L_WAIT_VM(31); break;
    default: L_WAIT_VM(0); break;
  }
}
#define L_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

__device__ __forceinline__ uint32_t l_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// two transposing reads (rows r0..r0+3 and r0+4..r0+7 of the caller's lane
// pattern) -> the 8 consecutive-row values of one column
__device__ __forceinline__ af3_bf16x8 l_tr8(const uint8_t* p0, const uint8_t* p1) {
  const bf16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p0);
  const bf16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1);
  return af3_bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ int l_swz(int row) { return (row ^ (row >> 3)) & 7; }

// ---------------------------------------------------------------------------
// rows: out[r][j] = scale * sum_k X[a(r)][k] Wl[e][j][k]   (TRANS: Wl[e][k][j])
// Block = 128 expert-sorted rows (tile map of 128-row blocks), 4 waves of
// 32 rows x 32 columns.  X k-steps (128 rows x 64 k, 16-byte chunks swizzled
// as the GEMMs) and the Wl k-step ([32 j][64 k], or [64 k][SR bytes] when
// TRANS) go global->LDS through a 2-stage ring, one k-step ahead: 40 KB of
// LDS, so four blocks fit a CU and the ~640 blocks of a 65,536-row layer run
// in one round instead of 1.25 rounds of two blocks per CU.
// ---------------------------------------------------------------------------
struct LrParams {
  const uint16_t* x;
  int64_t ldx;
  const int32_t* gather;
  int gdiv;
  const uint16_t* wl;
  int64_t wl_estride;  // elements per expert
  float scale;
  const int32_t* offs;
  const int32_t* tile_map;
  int K, r;
  uint16_t* out;
  int64_t ld_out;
};

constexpr int kLrA = 128 * 64 * 2;  // A bytes per stage
constexpr int kLrB = 64 * 64;       // B bytes per stage (<= 32 x 64 bf16)
constexpr int kLrStage = kLrA + kLrB;

constexpr int kLrStages = 2;

template <bool TRANS, int SR>
__global__ __launch_bounds__(256) void lrows_kernel(LrParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLrStages * kLrStage];
  const int32_t ent = p.tile_map[blockIdx.x];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * 128;
  const int nrows = min(128, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int nk = p.K / 64;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  constexpr int NB = TRANS ? (64 * SR) / 1024 : 4;  // B copies per stage (block)
  const bool has_b = wave < NB;

  // A: 4 copies per wave (8 rows each)
  const uint16_t* arow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (wave * 4 + i) * 8 + (lane >> 3);
    int64_t src = row_lo + (row < nrows ? row : 0);
    if (p.gather) src = p.gather[src] / p.gdiv;
    arow[i] = p.x + src * p.ldx + (((lane & 7) ^ l_swz(row)) << 3);
  }
  // B: copy `wave` (when has_b)
  const uint8_t* bsrc;
  {
    const uint8_t* wb = (const uint8_t*)(p.wl + e * p.wl_estride);
    if (TRANS) {  // [K][r] rows of SR bytes; copy w covers bytes [1024 w, 1024 w + 1024) of the k-step
      const int off = (has_b ? wave : 0) * 1024 + lane * 16;
      bsrc = wb + (int64_t)(off / SR) * (p.r * 2) + (off % SR);
    } else {      // [r][K]: copy w covers j rows 8 w .. 8 w + 7 (128 B of k each)
      int j = (has_b ? wave : 0) * 8 + (lane >> 3);
      if (j >= p.r) j = 0;
      bsrc = wb + (int64_t)j * p.K * 2 + ((((lane & 7) ^ l_swz(j))) << 4);
    }
  }
  const int64_t bstep = TRANS ? (int64_t)64 * p.r * 2 : 128;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(l_lds_addr(lds));
  auto issue = [&](int kt) {
    const uint32_t st = lds0 + (uint32_t)((kt % kLrStages) * kLrStage);
#pragma unroll
    for (int i = 0; i < 4; ++i) l_dma16(arow[i] + kt * 64, st + (uint32_t)((wave * 4 + i) * 1024));
    if (has_b) l_dma16(bsrc + kt * bstep, st + (uint32_t)(kLrA + wave * 1024));
  };
  af3_f32x16 acc;
#pragma unroll
  for (int q = 0; q < 16; ++q) acc[q] = 0.f;

  issue(0);
  for (int kt = 0; kt < nk; ++kt) {
    // this k-step's copies are the only ones in flight; the barrier also orders
    // every wave's reads of the other stage (k-step kt - 1) before its refill
    L_WAIT_VM(0);
    L_BARRIER();
    if (kt + 1 < nk) issue(kt + 1);
    const uint8_t* as = lds + (kt % kLrStages) * kLrStage;
    const uint8_t* bs = as + kLrA;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = wave * 32 + lr;
      const af3_bf16x8 a = *(const af3_bf16x8*)(as + row * 128 + (((s * 2 + lh) ^ l_swz(row)) << 4));
      af3_bf16x8 b;
      if (TRANS) {  // [64 k][SR]: rows k = 16 s + 8 lh + (0..7), column j = lr
        const int gi = lane >> 4, q = lane & 15;
        const int kr = s * 16 + (gi >> 1) * 8 + (q >> 2);
        const int col = (gi & 1) * 16 + 4 * (q & 3);
        b = l_tr8(bs + kr * SR + col * 2, bs + (kr + 4) * SR + col * 2);
      } else {
        b = *(const af3_bf16x8*)(bs + lr * 128 + (((s * 2 + lh) ^ l_swz(lr)) << 4));
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
    }
  }
  const int j = lr;
  if (j < p.r) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int row = wave * 32 + (q >> 2) * 8 + lh * 4 + (q & 3);
      if (row < nrows) p.out[(int64_t)(row_lo + row) * p.ld_out + j] = (uint16_t)af3_f32_to_bf16(acc[q] * p.scale);
    }
  }
}

// ---------------------------------------------------------------------------
// wgrad partials: P[chunk] = sum_{r in chunk} Big[b(r)][c0 + (0..255)]^T (x) Small[r][0..r)
// with the entry point's row scale rs(r) folded into operand A of the entry
// point (the Small side in MODE 1, the Big side in MODE 0) as bf16(rs(r) * A).
// Block = (chunk of chunk_rows expert-sorted rows, 256 Big columns); 4 waves of
// 64 columns x 32.  Per 32-row step: Big rows [32][256] (512 B rows, 16-byte
// chunks XOR-swizzled by lw_swz(row) so the transposing reads hit distinct
// banks) and Small rows [32][SR bytes] go global->LDS through a
// 4-stage ring, three steps ahead.  The gather indices and the per-row scales
// of the chunk are staged in LDS once, so no copy waits on an index load.
// The row scales are applied in registers to the MFMA operands (each lane
// holds 8 consecutive rows of one column of either operand); rows past the
// chunk get scale 0 on the Small side.  MODE 0 writes P as [W][r] (dB),
// MODE 1 as [r][W] (dA; transposed through LDS so the stores are row runs).
// The chunk of an expert that has only one writes bf16(scale * P) into G
// directly (what lwg_reduce_kernel would compute from it) and no partial.
// ---------------------------------------------------------------------------
struct LwParams {
  const uint16_t* big;
  int64_t ld_big;
  const int32_t* big_gather;
  int big_div;
  const uint16_t* small;  // [rows][r], compact
  const uint16_t* rowscale;
  const int32_t* offs;
  const int32_t* chunk_map;
  const int32_t* chunk_offs;  // per-expert chunk ranges: an expert of one chunk skips the partials
  int chunk_rows;
  int W, r, nbb;
  float scale;
  float* partials;
  uint16_t* g;  // output, written here directly for one-chunk experts
};

constexpr int kLwRows = 32;               // rows per pipeline step
constexpr int kLwStages = 4;
constexpr int kLwBig = kLwRows * 512;     // Big bytes per step
constexpr int kLwSmall = kLwRows * 64;    // Small bytes per step (<= 32 columns)
constexpr int kLwStage = kLwBig + kLwSmall;
constexpr int kLwMaxChunk = 512;          // rows per chunk (gather indices and scales staged in LDS)
constexpr int kLwTPad = 260;              // floats per row of the MODE 1 output transpose

// XOR applied to the 16-byte chunk index of a 512-byte Big row: bits 2-3 are
// row & 3 and bits 0-1 are (row >> 2) & 3, so the transposing reads (4 rows x
// 4 consecutive chunks per half wave) and row reads (16 rows x 1 chunk per
// quarter wave) both touch 16 distinct 16-byte bank groups
__device__ __forceinline__ int lw_swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }

__device__ __forceinline__ int lw_big_off(int row, int col) {  // byte offset of Big[row][col] (col % 4 == 0)
  return row * 512 + (((col >> 3) ^ lw_swz(row)) << 4) + ((col & 7) << 1);
}

// bf16(rs[i] * v[i]) for the 8 values of an MFMA operand
__device__ __forceinline__ af3_bf16x8 lw_scale8(af3_bf16x8 v, const float4 r0, const float4 r1) {
  af3_u32x4 w = __builtin_bit_cast(af3_u32x4, v);
  const float rs[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
  for (int h = 0; h < 4; ++h)
    w[h] = af3_pack_bf16x2(af3_bf16_to_f32(w[h] & 0xFFFFu) * rs[2 * h], af3_bf16_to_f32(w[h] >> 16) * rs[2 * h + 1]);
  return __builtin_bit_cast(af3_bf16x8, w);
}

template <int SR, int MODE>
__global__ __launch_bounds__(256, 2) void lwg_kernel(LwParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLwStages * kLwStage];
  __shared__ int32_t gsrc[kLwMaxChunk];                             // source row of each chunk row
  __shared__ __attribute__((aligned(16))) float rs_small[kLwMaxChunk];  // 0 past the chunk's rows
  __shared__ __attribute__((aligned(16))) float rs_big[kLwMaxChunk];    // MODE 0 row scale
  const int chunk = blockIdx.x / p.nbb, bb = blockIdx.x % p.nbb;
  const int32_t ent = p.chunk_map[chunk];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, cb = ent >> 16;
  const int kb = p.offs[e] + cb * p.chunk_rows;
  const int kend = min(p.chunk_rows, p.offs[e + 1] - kb);
  if (kend <= 0) return;
  const int nsteps = (kend + kLwRows - 1) / kLwRows;
  const bool big_rs = MODE == 0 && p.rowscale != nullptr;
  const bool small_rs = MODE == 1 && p.rowscale != nullptr;
  bool wide = false;
  for (int i = threadIdx.x; i < nsteps * kLwRows; i += 256) {
    const bool valid = i < kend;
    const int64_t src = kb + (valid ? i : 0);  // rows past the chunk read its first row
    gsrc[i] = p.big_gather ? p.big_gather[src] / p.big_div : (int32_t)src;
    const float rs = p.rowscale ? af3_bf16_to_f32(p.rowscale[src]) : 1.f;
    rs_small[i] = valid ? (small_rs ? rs : 1.f) : 0.f;
    rs_big[i] = rs;
    wide |= ((int64_t)gsrc[i] * p.ld_big + p.W) * 2 > (1LL << 32);
  }
  // every copy of the block addresses Big and Small by 32-bit byte offsets
  // from their bases unless a row lies beyond 4 GiB
  wide = __syncthreads_or(wide) || (int64_t)(kb + kend) * SR > (1LL << 32);
  const int c0 = bb * 256;
  const int ncols = min(256, p.W - c0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int NS = (kLwRows * SR) / 1024;  // Small copies per step (block)
  constexpr int NB = kLwBig / 1024 / 4;      // Big copies per step and wave
  const bool has_s = wave < NS;

  // Big: NB copies per wave, copy c = NB wave + i covers rows 2 c, 2 c + 1
  const uint16_t* bcol[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int rr = (wave * NB + i) * 2 + (lane >> 5);
    const int lc = (lane & 31) ^ lw_swz(rr);
    bcol[i] = p.big + (lc * 8 < ncols ? c0 + lc * 8 : c0);  // row part added per step (rows are gathered)
  }
  const uint8_t* ssrc = (const uint8_t*)p.small;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(l_lds_addr(lds));
  auto issue = [&](int st_i) {
    const uint32_t st = lds0 + (uint32_t)((st_i % kLwStages) * kLwStage);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int rr = (wave * NB + i) * 2 + (lane >> 5);
      const int64_t src = gsrc[st_i * kLwRows + rr];
      const uint32_t dst = st + (uint32_t)((wave * NB + i) * 1024);
      if (wide)
        l_dma16(bcol[i] + src * p.ld_big, dst);
      else
        l_dma16_s(p.big, (uint32_t)(bcol[i] - p.big) * 2u + (uint32_t)src * (uint32_t)(p.ld_big * 2), dst);
    }
    if (has_s) {
      const int off = wave * 1024 + lane * 16;  // byte offset inside the step's Small rows
      const int rl = st_i * kLwRows + off / SR;
      const int64_t srow = kb + (rl < kend ? rl : 0);
      const uint32_t dst = st + (uint32_t)(kLwBig + wave * 1024);
      if (wide)
        l_dma16(ssrc + srow * SR + (off % SR), dst);
      else
        l_dma16_s(ssrc, (uint32_t)srow * SR + (off % SR), dst);
    }
  };
  af3_f32x16 acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[t][q] = 0.f;

  issue(0);
  if (nsteps > 1) issue(1);
  if (nsteps > 2) issue(2);
  const int gi = lane >> 4, q = lane & 15;
  const int lrow = 8 * (lane >> 5);  // first of the lane's 8 operand rows inside a 16-row slice
  for (int st_i = 0; st_i < nsteps; ++st_i) {
    // this step's copies are in once at most the (up to two) later issued steps are outstanding
    const int ahead = min(2, nsteps - 1 - st_i);
    if (has_s) {
      if (ahead == 2)
        L_WAIT_VM(10);
      else if (ahead == 1)
        L_WAIT_VM(5);
      else
        L_WAIT_VM(0);
    } else {
      if (ahead == 2)
        L_WAIT_VM(8);
      else if (ahead == 1)
        L_WAIT_VM(4);
      else
        L_WAIT_VM(0);
    }
    L_BARRIER();
    // the slot of step st_i + 3 was last read in step st_i - 1 (all waves are past it)
    if (st_i + 3 < nsteps) issue(st_i + 3);
    const uint8_t* bs = lds + (st_i % kLwStages) * kLwStage;
    const uint8_t* ss = bs + kLwBig;
    const bool scale_s = small_rs || (st_i + 1) * kLwRows > kend;
#pragma unroll
    for (int s = 0; s < kLwRows / 16; ++s) {
      const int kr = s * 16 + (gi >> 1) * 8 + (q >> 2);
      const int scol = (gi & 1) * 16 + 4 * (q & 3);
      const int r0 = st_i * kLwRows + s * 16 + lrow;
      af3_bf16x8 b = l_tr8(ss + kr * SR + scol * 2, ss + (kr + 4) * SR + scol * 2);
      if (scale_s) b = lw_scale8(b, *(const float4*)&rs_small[r0], *(const float4*)&rs_small[r0 + 4]);
      float4 g0, g1;
      if (big_rs) {
        g0 = *(const float4*)&rs_big[r0];
        g1 = *(const float4*)&rs_big[r0 + 4];
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int bc = wave * 64 + t * 32 + (gi & 1) * 16 + 4 * (q & 3);
        af3_bf16x8 a = l_tr8(bs + lw_big_off(kr, bc), bs + lw_big_off(kr + 4, bc));
        if (big_rs) a = lw_scale8(a, g0, g1);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[t], 0, 0, 0);
      }
    }
  }
  // acc[t][qq]: Big column c0 + 64 wave + 32 t + 8 (qq / 4) + 4 lh + qq % 4, Small column j = lane % 32
  const int lr = lane & 31, lh = lane >> 5;
  const int j = lr;
  float* P = p.partials + (int64_t)chunk * p.W * p.r;
  const bool direct = p.chunk_offs[e + 1] - p.chunk_offs[e] == 1;
  uint16_t* G = p.g + (int64_t)e * p.W * p.r;
  if (MODE == 0) {
    if (j >= p.r) return;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int qq = 0; qq < 16; ++qq) {
        const int col = wave * 64 + t * 32 + (qq >> 2) * 8 + lh * 4 + (qq & 3);
        if (col < ncols) {
          const int64_t o = (int64_t)(c0 + col) * p.r + j;
          if (direct)
            G[o] = (uint16_t)af3_f32_to_bf16(acc[t][qq] * p.scale);
          else
            P[o] = acc[t][qq];
        }
      }
    }
  } else {
    // [r][256] through LDS (rows padded to kLwTPad floats), then row runs of ncols floats
    float* T = (float*)lds;
    L_BARRIER();  // every wave is done with the ring
    if (j < p.r) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int qq = 0; qq < 16; ++qq)
          T[j * kLwTPad + wave * 64 + t * 32 + (qq >> 2) * 8 + lh * 4 + (qq & 3)] = acc[t][qq];
    }
    L_BARRIER();
    for (int i = threadIdx.x; i < p.r * 64; i += 256) {
      const int jj = i >> 6, c = (i & 63) * 4;
      if (c >= ncols) continue;
      const float4 v = *(const float4*)(T + jj * kLwTPad + c);
      const int64_t o = (int64_t)jj * p.W + c0 + c;
      if (direct) {
        uint2 b;
        b.x = af3_pack_bf16x2(v.x * p.scale, v.y * p.scale);
        b.y = af3_pack_bf16x2(v.z * p.scale, v.w * p.scale);
        *(uint2*)(G + o) = b;
      } else {
        *(float4*)(P + o) = v;
      }
    }
  }
}

__global__ __launch_bounds__(256) void lwg_reduce_kernel(const float* __restrict__ partials,
                                                         const int32_t* __restrict__ chunk_offs, int64_t MN,
                                                         float scale, uint16_t* __restrict__ g) {
  const int e = blockIdx.y;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= MN) return;
  const int c0 = chunk_offs[e], c1 = chunk_offs[e + 1];
  if (c1 - c0 == 1) return;  // the chunk's kernel wrote G itself
  // chunks in order, eight partial loads in flight per lane
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int cb = c0; cb < c1; cb += 8) {
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[j] = cb + j < c1 ? *(const float4*)(partials + (int64_t)(cb + j) * MN + i) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (cb + j < c1) {
        a0 += v[j].x;
        a1 += v[j].y;
        a2 += v[j].z;
        a3 += v[j].w;
      }
    }
  }
  uint2 o;
  o.x = af3_pack_bf16x2(a0 * scale, a1 * scale);
  o.y = af3_pack_bf16x2(a2 * scale, a3 * scale);
  *(uint2*)(g + (int64_t)e * MN + i) = o;
}

// ---------------------------------------------------------------------------
// One pass over the wide gradient Big for both LoRA backward products that
// read it (the two products otherwise stream Big separately):
//   u[i][n]  = scale_u * sum_k Big[b(i)][k] Bl[e][k][n]            (rows, Bl = B [E][W][r])
//   P[chunk] = sum_{i in chunk} bf16(rs(i) Big[b(i)][k]) (x) Small[i][n]   (dB partials, [W][r])
// Block = (chunk of <= 512 expert-sorted rows, group of kLuG 256-column
// slices); two blocks per CU.  Row steps of 32 rows outer, slices inner: ring
// step g = s kLuG + j copies Big[32 rows of step s][256 columns of slice j] and
// the step's Small rows global->LDS through a kLuStages-stage ring (the stage
// layout of lwg_kernel), kLuStages - 1 steps ahead.
// dB: the slice's 4 waves x 64 columns x r accumulate over all row steps in
//   registers (one accumulator pair per slice), as in lwg_kernel MODE 0.
// u:  on v_mfma_f32_16x16x32_bf16, one 16-row x 16-column tile of a row step
//   per wave over all the group's columns (r = 32: four tiles, every wave,
//   every step; r = 16: two tiles, waves 0-1 on even steps and 2-3 on odd
//   ones), so no partial sums cross waves.  A wave's Bl operands for its 16
//   columns of u are loaded once per block and stay in registers; after the
//   kLuG slices of a row step the tile goes to u_part[group][row][n] (fp32)
//   and lu_sum_kernel adds the groups in order.
// The Big tile has lwg_kernel's layout (lw_big_off), which keeps both the
// transposing reads (dB) and the row reads (u) free of bank conflicts.
// ---------------------------------------------------------------------------
struct LuParams {
  const uint16_t* big;
  int64_t ld_big;
  const int32_t* big_gather;
  int big_div;
  const uint16_t* small;     // [rows][r], compact
  const uint16_t* rowscale;  // Big-side row scale of dB (u has none), optional
  const uint16_t* bl;        // [E][W][r]
  const int32_t* offs;
  const int32_t* chunk_map;
  const int32_t* chunk_offs;  // per-expert chunk ranges: an expert of one chunk skips the dB partials
  int chunk_rows, W, r, ngrp;
  int64_t n_rows;
  float* partials;  // [chunk][W][r]
  float* u_part;    // [ngrp][n_rows][r]
  uint16_t* g;      // dB, written here directly for one-chunk experts
};

typedef __attribute__((ext_vector_type(4))) float lu_f32x4;

constexpr int kLuG = 2;          // 256-column slices per block
constexpr int kLuStages = 4;     // ring stages (three steps in flight per block)
constexpr int kLuMinBlocks = 2;  // resident blocks per CU (registers <= 256, LDS <= 80 KB per block)

template <int SR>
__global__ __launch_bounds__(256, kLuMinBlocks) void lug_kernel(LuParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLuStages * kLwStage];
  __shared__ int32_t gsrc[kLwMaxChunk];
  __shared__ __attribute__((aligned(16))) float rs_small[kLwMaxChunk];
  __shared__ __attribute__((aligned(16))) float rs_big[kLwMaxChunk];
  static_assert(256 * SR <= kLwStage && kLuStages >= 2 && kLuStages <= 7,
                "a Bl slice must fit a ring slot; the waits below cover up to 6 steps in flight");
  static_assert(kLuStages * kLwStage + 3 * kLwMaxChunk * 4 <= 80 * 1024, "two blocks per CU");
  constexpr bool R32 = SR == 64;  // r = 32 (else 16)
  const int chunk = blockIdx.x / p.ngrp, cg = blockIdx.x % p.ngrp;
  const int32_t ent = p.chunk_map[chunk];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, cb = ent >> 16;
  const int kb = p.offs[e] + cb * p.chunk_rows;
  const int kend = min(p.chunk_rows, p.offs[e + 1] - kb);
  if (kend <= 0) return;
  const int nsteps = (kend + kLwRows - 1) / kLwRows;
  const int NT = nsteps * kLuG;  // ring steps
  const bool big_rs = p.rowscale != nullptr;
  bool wide = false;
  for (int i = threadIdx.x; i < nsteps * kLwRows; i += 256) {
    const bool valid = i < kend;
    const int64_t src = kb + (valid ? i : 0);  // rows past the chunk read its first row
    gsrc[i] = p.big_gather ? p.big_gather[src] / p.big_div : (int32_t)src;
    rs_small[i] = valid ? 1.f : 0.f;
    rs_big[i] = big_rs ? af3_bf16_to_f32(p.rowscale[src]) : 1.f;
    wide |= ((int64_t)gsrc[i] * p.ld_big + p.W) * 2 > (1LL << 32);
  }
  // gsrc / rs_* published; every copy of the block addresses Big and Small by
  // 32-bit byte offsets from their bases unless a row lies beyond 4 GiB
  wide = __syncthreads_or(wide) || (int64_t)(kb + kend) * SR > (1LL << 32);
  const int gc0 = cg * (kLuG * 256);  // first column of the group (< W)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gi = lane >> 4, q = lane & 15, lr = lane & 31, lh = lane >> 5;
  // the wave's u tile: rows 16 uh of a row step, columns 16 un
  const int uh = R32 ? wave >> 1 : wave & 1;
  const int un = R32 ? wave & 1 : 0;

  constexpr int NS = (kLwRows * SR) / 1024;  // Small copies per step (block)
  constexpr int NB = kLwBig / 1024 / 4;      // Big copies per step and wave
  static_assert((kLuStages - 2) * (NB + 1) + 4 <= 31, "wait counts within l_wait_vm");
  const bool has_s = wave < NS;
  int lcs[NB];  // logical 16-byte chunk of each Big copy of this lane
#pragma unroll
  for (int i = 0; i < NB; ++i) lcs[i] = (lane & 31) ^ lw_swz((wave * NB + i) * 2 + lh);
  const uint8_t* ssrc = (const uint8_t*)p.small;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(l_lds_addr(lds));
  auto issue = [&](int g, int slot) {
    const int s = g / kLuG, j = g % kLuG;
    const uint32_t st = lds0 + (uint32_t)(slot * kLwStage);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int rr = (wave * NB + i) * 2 + lh;
      const int64_t src = gsrc[s * kLwRows + rr];
      int col = gc0 + j * 256 + lcs[i] * 8;
      col = col < p.W ? col : 0;
      const uint32_t dst = st + (uint32_t)((wave * NB + i) * 1024);
      if (wide)
        l_dma16(p.big + src * p.ld_big + col, dst);
      else
        l_dma16_s(p.big, (uint32_t)src * (uint32_t)(p.ld_big * 2) + (uint32_t)col * 2u, dst);
    }
    if (has_s) {
      const int off = wave * 1024 + lane * 16;  // byte offset inside the step's Small rows
      const int rl = s * kLwRows + off / SR;
      const int64_t srow = kb + (rl < kend ? rl : 0);
      const uint32_t dst = st + (uint32_t)(kLwBig + wave * 1024);
      if (wide)
        l_dma16(ssrc + srow * SR + (off % SR), dst);
      else
        l_dma16_s(ssrc, (uint32_t)srow * SR + (off % SR), dst);
    }
  };

  af3_f32x16 accb[kLuG][2];
  lu_f32x4 accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q2 = 0; q2 < 16; ++q2)
#pragma unroll
    for (int j = 0; j < kLuG; ++j) accb[j][0][q2] = accb[j][1][q2] = 0.f;
  constexpr int D = kLuStages - 1;  // steps in flight
#pragma unroll
  for (int g = 0; g < D; ++g)
    if (g < NT) issue(g, g);
  // Bl[e][gc0 + 256 j ..][0 .. r), one slice at a time -> the ring slot D, which the copies issued so far
  // leave free (rows past W zero) -> registers:
  // bw[j][kk] = Bl rows 256 j + 32 kk + 8 gi + (0..7), column 16 un + q (the 16x16x32 B operand)
  af3_bf16x8 bw[kLuG][8];
  {
    uint8_t* slab = lds + D * kLwStage;
    const int col = un * 16 + 4 * (q & 3);
#pragma unroll
    for (int j = 0; j < kLuG; ++j) {
      const int nbytes = min(256, p.W - gc0 - 256 * j) * SR;  // <= 0 for a slice past W
      const uint8_t* src = (const uint8_t*)(p.bl + ((int64_t)e * p.W + gc0 + 256 * j) * p.r);
      for (int o = threadIdx.x * 16; o < 256 * SR; o += 256 * 16) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (o < nbytes) v = *(const uint4*)(src + o);
        *(uint4*)(slab + o) = v;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int kr = kk * 32 + gi * 8 + (q >> 2);
        bw[j][kk] = l_tr8(slab + kr * SR + col * 2, slab + (kr + 4) * SR + col * 2);
      }
      __syncthreads();  // slot D is rewritten (next slice, then the ring's step D)
    }
  }

  int slot = 0;             // ring slot of step g
  const int lrow = 8 * lh;  // first of the lane's 8 operand rows inside a 16-row slice
  const int urow = uh * 16 + q;  // the lane's row of the u A operand
  for (int s = 0; s < nsteps; ++s) {
    const bool scale_s = (s + 1) * kLwRows > kend;
    const bool u_here = R32 || (wave >> 1) == (s & 1);  // this wave owns a u tile of step s
#pragma unroll
    for (int j = 0; j < kLuG; ++j) {
      const int g = s * kLuG + j;
      // this step's copies are in once at most those of the later issued steps are outstanding
      // (NB + has_s copies per step and wave; stores issued since only make the wait stricter)
      // (plus the previous row step's 4 u stores, issued after every copy of
      // the steps waited for in this row step: vmcnt counts stores too)
      const int ahead = min(D - 1, NT - 1 - g);
      const bool stored = s > 0 && (R32 || (wave >> 1) == ((s - 1) & 1));
      l_wait_vm(__builtin_amdgcn_readfirstlane(ahead * (NB + (has_s ? 1 : 0)) + (stored ? 4 : 0)));
      L_BARRIER();
      // the slot of step g + D is the one step g - 1 read (all waves are past it)
      const int prev = slot == 0 ? D : slot - 1;
      if (g + D < NT) issue(g + D, prev);
      const uint8_t* bs = lds + slot * kLwStage;
      slot = slot == D ? 0 : slot + 1;
      const uint8_t* ss = bs + kLwBig;
#pragma unroll
      for (int h = 0; h < kLwRows / 16; ++h) {
        const int kr = h * 16 + (gi >> 1) * 8 + (q >> 2);
        const int scol = (gi & 1) * 16 + 4 * (q & 3);
        const int r0 = s * kLwRows + h * 16 + lrow;
        af3_bf16x8 b = l_tr8(ss + kr * SR + scol * 2, ss + (kr + 4) * SR + scol * 2);
        if (scale_s) b = lw_scale8(b, *(const float4*)&rs_small[r0], *(const float4*)&rs_small[r0 + 4]);
        float4 g0, g1;
        if (big_rs) {
          g0 = *(const float4*)&rs_big[r0];
          g1 = *(const float4*)&rs_big[r0 + 4];
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int bc = wave * 64 + t * 32 + (gi & 1) * 16 + 4 * (q & 3);
          af3_bf16x8 a = l_tr8(bs + lw_big_off(kr, bc), bs + lw_big_off(kr + 4, bc));
          if (big_rs) a = lw_scale8(a, g0, g1);
          accb[j][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, accb[j][t], 0, 0, 0);
        }
      }
      if (u_here) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {  // columns 32 kk .. 32 kk + 31 of the slice; lane: 8 of them
          const int c = kk * 4 + gi;
          const af3_bf16x8 a = *(const af3_bf16x8*)(bs + urow * 512 + ((c ^ lw_swz(urow)) << 4));
          accu = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bw[j][kk], accu, 0, 0, 0);
        }
      }
    }
    // accu[i]: row 16 uh + 4 gi + i of row step s, column 16 un + q
    if (u_here) {
      float* up = p.u_part + ((int64_t)cg * p.n_rows + kb) * p.r + un * 16 + q;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = s * kLwRows + uh * 16 + gi * 4 + i;
        if (row < kend) up[(int64_t)row * p.r] = accu[i];
      }
      accu = lu_f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // accb[j][t][qq]: Big column gc0 + 256 j + 64 wave + 32 t + 8 (qq / 4) + 4 lh + qq % 4, Small column lr
  // (an expert of one chunk: bf16 straight into dB, as lwg_kernel)
  if (lr >= p.r) return;
  float* P = p.partials + (int64_t)chunk * p.W * p.r;
  uint16_t* G = p.g + (int64_t)e * p.W * p.r;
  const bool direct = p.chunk_offs[e + 1] - p.chunk_offs[e] == 1;
#pragma unroll
  for (int j = 0; j < kLuG; ++j)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int qq = 0; qq < 16; ++qq) {
        const int col = gc0 + j * 256 + wave * 64 + t * 32 + (qq >> 2) * 8 + lh * 4 + (qq & 3);
        if (col < p.W) {
          if (direct)
            G[(int64_t)col * p.r + lr] = (uint16_t)af3_f32_to_bf16(accb[j][t][qq]);
          else
            P[(int64_t)col * p.r + lr] = accb[j][t][qq];
        }
      }
}

// u[i][n] = bf16(scale * sum_g u_part[g][i][n]), groups in order, for the
// routed rows i < offs[E]; rows past them (entries dropped for an expert id
// outside [0, E)) have no partials and are written as zeros
__global__ __launch_bounds__(256) void lu_sum_kernel(const float* __restrict__ u_part, int64_t n_elems, int ngrp,
                                                     const int32_t* __restrict__ offs, int E, int r, float scale,
                                                     uint16_t* __restrict__ u) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n_elems) return;
  if (i >= (int64_t)offs[E] * r) {  // r % 4 == 0: the 4 elements lie in one row
    *(uint2*)(u + i) = uint2{0u, 0u};
    return;
  }
  float4 a = *(const float4*)(u_part + i);
  for (int g = 1; g < ngrp; ++g) {
    const float4 v = *(const float4*)(u_part + (int64_t)g * n_elems + i);
    a.x += v.x;
    a.y += v.y;
    a.z += v.z;
    a.w += v.w;
  }
  uint2 o;
  o.x = af3_pack_bf16x2(a.x * scale, a.y * scale);
  o.y = af3_pack_bf16x2(a.z * scale, a.w * scale);
  *(uint2*)(u + i) = o;
}

inline bool l_al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

namespace af3 {

int lora_rows_fast(const uint16_t* x, int64_t ldx, const int32_t* gather, int gdiv, const uint16_t* wl, int trans_b,
                   float scale, const int32_t* token_offs, const int32_t* block_pid_map, int max_tiles, int n_out,
                   int K, uint16_t* out, int64_t ld_out, hipStream_t stream) {
  if (!(n_out == 16 || n_out == 32) || K % 64 != 0 || ldx % 8 != 0 || !l_al16(x) || !l_al16(wl)) return AF3_EUNSUPPORTED;
  LrParams p{};
  p.x = x;
  p.ldx = ldx;
  p.gather = gather;
  p.gdiv = gdiv > 0 ? gdiv : 1;
  p.wl = wl;
  p.wl_estride = (int64_t)n_out * K;
  p.scale = scale;
  p.offs = token_offs;
  p.tile_map = block_pid_map;
  p.K = K;
  p.r = n_out;
  p.out = out;
  p.ld_out = ld_out;
  const dim3 grid(max_tiles), block(256);
  if (trans_b == 0)
    hipLaunchKernelGGL((lrows_kernel<false, 64>), grid, block, 0, stream, p);
  else if (n_out == 32)
    hipLaunchKernelGGL((lrows_kernel<true, 64>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((lrows_kernel<true, 32>), grid, block, 0, stream, p);
  return check_launch("lora_rows");
}

int lora_wgrad_fast(const uint16_t* big, int64_t ld_big, const int32_t* big_gather, int big_div,
                    const uint16_t* small, int64_t ld_small, const uint16_t* rowscale, int small_is_a, int W, int r,
                    float scale, const int32_t* token_offs, const int32_t* chunk_map, const int32_t* chunk_offs,
                    int max_chunks, int chunk_rows, int n_expts, float* partials, uint16_t* g, hipStream_t stream) {
  if (!(r == 16 || r == 32) || ld_small != r || W % 8 != 0 || ld_big % 8 != 0 || !l_al16(big) || !l_al16(small) ||
      !l_al16(partials) || !l_al16(g) || chunk_rows > kLwMaxChunk || chunk_rows % kLwRows != 0)
    return AF3_EUNSUPPORTED;
  LwParams p{};
  p.big = big;
  p.ld_big = ld_big;
  p.big_gather = big_gather;
  p.big_div = big_div > 0 ? big_div : 1;
  p.small = small;
  p.rowscale = rowscale;
  p.offs = token_offs;
  p.chunk_map = chunk_map;
  p.chunk_offs = chunk_offs;
  p.chunk_rows = chunk_rows;
  p.W = W;
  p.r = r;
  p.nbb = (W + 255) / 256;
  p.scale = scale;
  p.partials = partials;
  p.g = g;
  if (max_chunks > 0) {
    const dim3 grid((unsigned)max_chunks * p.nbb), block(256);
    // small_is_a: G = Small^T Big ([r][W], the dA form); else G = Big^T Small ([W][r], dB)
    if (r == 32) {
      if (small_is_a)
        hipLaunchKernelGGL((lwg_kernel<64, 1>), grid, block, 0, stream, p);
      else
        hipLaunchKernelGGL((lwg_kernel<64, 0>), grid, block, 0, stream, p);
    } else {
      if (small_is_a)
        hipLaunchKernelGGL((lwg_kernel<32, 1>), grid, block, 0, stream, p);
      else
        hipLaunchKernelGGL((lwg_kernel<32, 0>), grid, block, 0, stream, p);
    }
    const int rc = check_launch("lora_wgrad/partial");
    if (rc) return rc;
  }
  const int64_t MN = (int64_t)W * r;
  hipLaunchKernelGGL(lwg_reduce_kernel, dim3((unsigned)af3_cdiv(MN / 4, 256), n_expts), dim3(256), 0, stream,
                     partials, chunk_offs, MN, scale, g);
  return check_launch("lora_wgrad/reduce");
}

}  // namespace af3

namespace {
constexpr int kLuGroupCols = kLuG * 256;
int64_t lu_ngrp(int W) { return (W + kLuGroupCols - 1) / kLuGroupCols; }
size_t lu_align(size_t n) { return (n + 255) & ~(size_t)255; }
}  // namespace

extern "C" size_t af3_lora_u_wgrad_workspace_bytes(int max_chunks, int64_t n_rows, int W, int r) {
  if (W <= 0 || r <= 0 || n_rows < 0) return 0;
  const size_t part = (size_t)(max_chunks > 0 ? max_chunks : 1) * (size_t)W * (size_t)r * sizeof(float);
  return lu_align(part) + (size_t)lu_ngrp(W) * (size_t)n_rows * (size_t)r * sizeof(float);
}

extern "C" int af3_lora_u_wgrad(const uint16_t* big, int64_t ld_big, const int32_t* big_gather, int big_div,
                                const uint16_t* big_rowscale, const uint16_t* small, const uint16_t* bl,
                                float scale_u, const int32_t* token_offs, int n_expts, int64_t n_rows, int W, int r,
                                const int32_t* chunk_map, const int32_t* chunk_offs, int max_chunks, int chunk_rows,
                                void* workspace, size_t ws_bytes, uint16_t* u, uint16_t* g, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(W > 0 && r > 0 && n_expts > 0 && n_rows >= 0 && max_chunks >= 0 && chunk_rows > 0,
              "lora_u_wgrad: bad sizes");
  if (!(r == 16 || r == 32) || W % 8 != 0 || ld_big % 8 != 0 || chunk_rows > kLwMaxChunk ||
      chunk_rows % kLwRows != 0 || !l_al16(big) || !l_al16(small) || !l_al16(bl) || !l_al16(u) || !l_al16(g) ||
      !l_al16(workspace))
    return AF3_EUNSUPPORTED;
  AF3_REQUIRE(workspace && ws_bytes >= af3_lora_u_wgrad_workspace_bytes(max_chunks, n_rows, W, r),
              "lora_u_wgrad: workspace too small");
  LuParams p{};
  p.big = big;
  p.ld_big = ld_big;
  p.big_gather = big_gather;
  p.big_div = big_div > 0 ? big_div : 1;
  p.small = small;
  p.rowscale = big_rowscale;
  p.bl = bl;
  p.offs = token_offs;
  p.chunk_map = chunk_map;
  p.chunk_offs = chunk_offs;
  p.chunk_rows = chunk_rows;
  p.W = W;
  p.r = r;
  p.ngrp = (int)lu_ngrp(W);
  p.g = g;
  p.n_rows = n_rows;
  p.partials = (float*)workspace;
  p.u_part = (float*)((uint8_t*)workspace +
                      lu_align((size_t)(max_chunks > 0 ? max_chunks : 1) * (size_t)W * (size_t)r * sizeof(float)));
  if (max_chunks > 0 && n_rows > 0) {
    const dim3 grid((unsigned)max_chunks * (unsigned)p.ngrp), block(256);
    if (r == 32)
      hipLaunchKernelGGL((lug_kernel<64>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((lug_kernel<32>), grid, block, 0, stream, p);
    int rc = af3::check_launch("lora_u_wgrad/partial");
    if (rc) return rc;
    const int64_t nu = n_rows * r;  // multiple of 16
    hipLaunchKernelGGL(lu_sum_kernel, dim3((unsigned)af3_cdiv(nu / 4, 256)), dim3(256), 0, stream, p.u_part, nu,
                       p.ngrp, token_offs, n_expts, r, scale_u, u);
    rc = af3::check_launch("lora_u_wgrad/u");
    if (rc) return rc;
  }
  const int64_t MN = (int64_t)W * r;
  hipLaunchKernelGGL(lwg_reduce_kernel, dim3((unsigned)af3_cdiv(MN / 4, 256), n_expts), dim3(256), 0, stream,
                     p.partials, chunk_offs, MN, 1.f, g);
  return af3::check_launch("lora_u_wgrad/reduce");
}
