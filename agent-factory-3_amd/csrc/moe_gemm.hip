// Grouped (per-expert) GEMMs of the gpt-oss MoE expert path on bf16 MFMA.
//
// Reference behaviour (the reference calls triton_kernels.matmul_ogs after
// materialising the bf16 weights of every expert, quantization.py:358-362 and
// 409-418; matmul_ogs semantics: for each expert e,
//   Y[rows(e)] = X[gather(rows(e))] @ W[e] (+ bias[e]) (* gammas[rows(e)])
// followed by a scatter-sum over the K slots of each token):
//   A6  gate_up forward  quantization.py:516-525   trans_w = 0, gather, bias
//   A8  down forward     quantization.py:532-541   trans_w = 0, bias, gammas
//   A9  down dX          quantization.py:409-418   trans_w = 1, gather, gammas
//   A11 gate_up dX       quantization.py:409-418   trans_w = 1 (then combine)
// Here the MXFP4 weight is never materialised: each k-step of the B tile is
// read packed from HBM and converted to bf16 on its way into LDS.
//
// One kernel template covers every GEMM of the path.  C[m][n] = sum_k A(m,k) *
// B(n,k) with a 64-deep k-step staged through LDS as [rows][64] bf16 tiles
// (k contiguous, 16-byte chunks XOR-swizzled by row), read by
// v_mfma_f32_32x32x16_bf16.  Operands are produced by loaders:
//   RowsBf16   A[m][k] / B[n][k] with k contiguous (optionally row-gathered)
//   RowsFp4    B = MXFP4 W[e][n][k/32][16]     (nibbles packed along k)
//   ColsBf16   operand stored [k][rows]: 8x8 register transpose before LDS
//   ColsFp4    B = MXFP4 W[e][k][n/32][16]     (nibbles packed along n)
// Grid modes:
//   row tiles  blockIdx.x -> block_pid_map entry (expert e, BM-row block b) of
//              the expert-sorted rows; blockIdx.y -> BN-column block.  An
//              optional second k segment (the expert LoRA term) is appended.
//   wgrad      blockIdx.x -> (expert, m block, n block); the k range is the
//              expert's rows: G[e] = A(rows(e))^T B(rows(e)).
#include <type_traits>

#include "af3_common.h"

namespace {

constexpr int kBK = 64;
constexpr int kThreads = 256;

enum Kind { ROWS_BF16 = 0, ROWS_FP4 = 1, COLS_BF16 = 2, COLS_FP4 = 3, NONE = 4 };

struct Operand {
  const void* ptr;         // bf16 elements or MXFP4 blocks
  const uint8_t* scales;   // MXFP4 scales
  int64_t ld;              // row stride: elements (bf16) / bytes (fp4 blocks)
  int64_t sld;             // scale row stride (bytes)
  int64_t estride;         // per-expert stride (elements / bytes), 0 = shared
  int64_t sestride;        // per-expert scale stride
  const int32_t* gather;   // optional row indirection (index / gdiv)
  int gdiv;
  const uint16_t* rowscale;  // optional bf16 per-row multiplier (COLS_BF16 A only)
  int extent;              // number of valid tile rows along the operand's non-k axis (N or M)
};

struct Params {
  Operand a, b;       // main segment
  Operand ax, bx;     // extension segment (row tiles only)
  int K;              // main reduction length (row tiles)
  int kx;             // extension reduction length (0 = none)
  const int32_t* offs;      // expert row offsets [E+1]
  const int32_t* tile_map;  // block_pid_map (row tiles)
  const int32_t* tile_offs; // token_offs_pad of the same block size ([E] = number of m-tiles)
  int E;
  int n_mblk, n_nblk;       // wgrad tiling
  const float* bias;        // [E][N] fp32
  int64_t bias_estride;
  const void* gammas;       // [rows] bf16 or fp32
  int gammas_f32;
  float scale;
  uint16_t* c;
  int64_t ldc;
  int64_t c_estride;        // wgrad output per-expert stride
  int chunk_rows;           // wgrad rows per chunk
  float* partials;          // wgrad fp32 partials [chunk][M][N]
  int M, N;                 // output extents (M used by wgrad; rows come from offs in row tiles)
  int group_m;              // work-item grouping (m-tiles per group), gemm4
  // fused SwiGLU epilogue (gemm4 forward / gemm5 dgrad): 0 none;
  // 1 backward: c receives dGU [rows][2N] from the bf16 product dI and the
  //   saved interleaved pre-activation glu [rows][2N];
  // 2 forward: besides the bf16 product (the interleaved pre-activation), glu
  //   receives its SwiGLU output [rows][N / 2]
  int epi;
  void* glu;
  int64_t ld_glu;
  float alpha, limit;
  // per-row scale of the A operand (fp8 mode: per-token activation scale),
  // indexed like the A rows (gather[r] / gdiv, or r); the default epilogues
  // then store (acc * ascale + bias) * gammas
  const float* ascale;
  // forward weights (gemm7): 0 = the packed blocks row-major [E][N][K/32][16];
  // 1 = the forward-tiled copy of af3_mxfp4_tile_fwd, [E][N/32][K/64][2][32][16]
  // (one KB per 32 weight rows and 64-deep k-step, in the order the wave's
  // lanes take them)
  int b_tiled;
  // the caller's guarantee that every A row the call reads lies within 4 GiB
  // of a.ptr (tile_cfg | AF3_X_OFFSETS_32)
  int a_off32;
  // input gradient (gemm8): b.scales is the af3_mxfp4_tile_dx_scales copy,
  // [E][K/64][s_nt][8][64] bytes (s_nt = 256-column n-tiles)
  int s_tiled, s_nt;
};

// scale of A row a(r) for output row r (1 without a row scale)
__device__ __forceinline__ float g4_ascale(const Params& p, int64_t r) {
  if (!p.ascale) return 1.f;
  const int64_t ar = p.a.gather ? p.a.gather[r] / p.a.gdiv : r;
  return p.ascale[ar];
}

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

// LDS offset (in bf16 elements) of the 16-byte chunk `ch` of tile row `row`
__device__ __forceinline__ int lds_off(int row, int ch) { return row * kBK + ((ch ^ swz(row)) << 3); }

__device__ __forceinline__ af3_u32x4 zero4() { return af3_u32x4{0u, 0u, 0u, 0u}; }

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {  // lo16(a) | lo16(b) << 16
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {  // hi16(a) | hi16(b) << 16
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// in[j] = row j (k index) holding 8 consecutive tile-row values; out[i] =
// tile row i holding 8 consecutive k values.
__device__ __forceinline__ void transpose8x8(const af3_u32x4 in[8], af3_u32x4 out[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      uint32_t a = in[2 * p][q], b = in[2 * p + 1][q];
      lo[p] = perm_lo(a, b);
      hi[p] = perm_hi(a, b);
    }
    out[2 * q] = af3_u32x4{lo[0], lo[1], lo[2], lo[3]};
    out[2 * q + 1] = af3_u32x4{hi[0], hi[1], hi[2], hi[3]};
  }
}

// ---------------------------------------------------------------------------
// Loaders.  TR = tile rows (BM for A, BN for B).  `row0` is the first tile row
// in the operand's row space (expert-sorted row for gathered/row operands,
// column for cols operands); k ranges over [k0, k0+64) limited by `kend`.
// ---------------------------------------------------------------------------
template <int TR, int KIND, int NT = kThreads>
struct Loader;

// k-contiguous bf16 rows
template <int TR, int NT>
struct Loader<TR, ROWS_BF16, NT> {
  static constexpr int kUnits = TR * 8;
  static constexpr int kUPT = (kUnits + NT - 1) / NT;
  const uint16_t* rp[kUPT];
  af3_u32x4 v[kUPT];
  int kend;

  __device__ __forceinline__ void init(const Operand& op, int e, int row0, int nvalid, int kend_) {
    kend = kend_;
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      int r = u >> 3;
      rp[i] = nullptr;
      if (u < kUnits && r < nvalid) {
        int64_t src = row0 + r;
        if (op.gather) src = op.gather[src] / op.gdiv;
        rp[i] = (const uint16_t*)op.ptr + e * op.estride + src * op.ld;
      }
    }
  }
  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      int k = k0 + ((u & 7) << 3);
      v[i] = (rp[i] && k < kend) ? *(const af3_u32x4*)(rp[i] + k) : zero4();
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      if (u < kUnits) *(af3_u32x4*)(lds + lds_off(u >> 3, u & 7)) = v[i];
    }
  }
};

// MXFP4 rows packed along k: W[e][n][k/32][16]
template <int TR, int NT>
struct Loader<TR, ROWS_FP4, NT> {
  static constexpr int kUnits = TR * 2;  // two 32-element groups per 64-deep k-step
  static constexpr int kUPT = (kUnits + NT - 1) / NT;
  const uint8_t* bp[kUPT];
  const uint8_t* sp[kUPT];
  af3_u32x4 v[kUPT];
  uint32_t s[kUPT];
  int kend;

  __device__ __forceinline__ void init(const Operand& op, int e, int row0, int nvalid, int kend_) {
    kend = kend_;
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      int r = u >> 1;
      bp[i] = nullptr;
      sp[i] = nullptr;
      if (u < kUnits && r < nvalid) {
        int64_t n = row0 + r;
        bp[i] = (const uint8_t*)op.ptr + e * op.estride + n * op.ld;
        sp[i] = op.scales + e * op.sestride + n * op.sld;
      }
    }
  }
  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      int k = k0 + ((u & 1) << 5);
      bool ok = bp[i] && k < kend;
      v[i] = ok ? *(const af3_u32x4*)(bp[i] + (k >> 1)) : zero4();
      s[i] = ok ? (uint32_t)sp[i][k >> 5] : 127u;
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      if (u >= kUnits) continue;
      int r = u >> 1, ch0 = (u & 1) << 2;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t o[4];
        af3_dequant_u32(v[i][q], s[i], o);
        *(af3_u32x4*)(lds + lds_off(r, ch0 + q)) = af3_u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
};

// bf16 operand stored [k][rows] (rows contiguous): unit = 8 k x 8 rows
template <int TR, int NT>
struct Loader<TR, COLS_BF16, NT> {
  static constexpr int kCO = TR / 8;  // 8-column groups per k-row
  static constexpr int kUnits = 8 * kCO;
  static constexpr int kUPT = (kUnits + NT - 1) / NT;
  const uint16_t* base;
  const int32_t* gather;
  const uint16_t* rowscale;
  int64_t ld;
  int gdiv, kb, kend, col0, ncols;
  af3_u32x4 v[kUPT][8];

  __device__ __forceinline__ void init(const Operand& op, int e, int col0_, int ncols_, int kb_, int kend_) {
    base = (const uint16_t*)op.ptr + e * op.estride;
    gather = op.gather;
    gdiv = op.gdiv;
    rowscale = op.rowscale;
    ld = op.ld;
    kb = kb_;
    kend = kend_;
    col0 = col0_;
    ncols = ncols_;
  }
  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      int ko = u / kCO, co = u % kCO;
      int c = co * 8;
      bool cok = u < kUnits && c < ncols;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int k = k0 + ko * 8 + j;
        af3_u32x4 x = zero4();
        if (cok && k < kend) {
          int64_t r = kb + k;
          int64_t src = gather ? (int64_t)(gather[r] / gdiv) : r;
          x = *(const af3_u32x4*)(base + src * ld + col0 + c);
          if (rowscale) {
            float sc = af3_bf16_to_f32(rowscale[r]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              x[q] = af3_pack_bf16x2(af3_bf16_to_f32(x[q] & 0xFFFFu) * sc, af3_bf16_to_f32(x[q] >> 16) * sc);
          }
        }
        v[i][j] = x;
      }
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      if (u >= kUnits) continue;
      int ko = u / kCO, co = u % kCO;
      af3_u32x4 t[8];
      transpose8x8(v[i], t);
#pragma unroll
      for (int j = 0; j < 8; ++j) *(af3_u32x4*)(lds + lds_off(co * 8 + j, ko)) = t[j];
    }
  }
};

// MXFP4 operand packed along the tile-row axis: W[e][k][n/32][16]
template <int TR, int NT>
struct Loader<TR, COLS_FP4, NT> {
  static constexpr int kCO = TR / 8;  // 8-column groups per k-row
  static constexpr int kUnits = 8 * kCO;
  static constexpr int kUPT = (kUnits + NT - 1) / NT;
  const uint8_t* bbase;
  const uint8_t* sbase;
  int64_t ld, sld;
  int kend, col0, ncols;
  uint32_t w[kUPT][8];
  uint32_t s[kUPT][8];

  __device__ __forceinline__ void init(const Operand& op, int e, int col0_, int ncols_, int kb_, int kend_) {
    bbase = (const uint8_t*)op.ptr + e * op.estride;
    sbase = op.scales + e * op.sestride;
    ld = op.ld;
    sld = op.sld;
    kend = kend_;
    col0 = col0_;
    ncols = ncols_;
  }
  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      int ko = u / kCO, co = u % kCO;
      int c = col0 + co * 8;  // first of 8 columns = 4 packed bytes
      bool cok = u < kUnits && co * 8 < ncols;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int k = k0 + ko * 8 + j;
        bool ok = cok && k < kend;
        w[i][j] = ok ? *(const uint32_t*)(bbase + (int64_t)k * ld + (c >> 1)) : 0u;
        s[i][j] = ok ? (uint32_t)sbase[(int64_t)k * sld + (c >> 5)] : 127u;
      }
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) {
#pragma unroll
    for (int i = 0; i < kUPT; ++i) {
      int u = threadIdx.x + i * NT;
      if (u >= kUnits) continue;
      int ko = u / kCO, co = u % kCO;
      af3_u32x4 x[8], t[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t o[4];
        af3_dequant_u32(w[i][j], s[i][j], o);
        x[j] = af3_u32x4{o[0], o[1], o[2], o[3]};
      }
      transpose8x8(x, t);
#pragma unroll
      for (int j = 0; j < 8; ++j) *(af3_u32x4*)(lds + lds_off(co * 8 + j, ko)) = t[j];
    }
  }
};

// ---------------------------------------------------------------------------
// MFMA compute on one LDS k-step
// ---------------------------------------------------------------------------
template <int TM, int TN>
__device__ __forceinline__ void mma_kstep(const uint16_t* As, const uint16_t* Bs, int wm0, int wn0,
                                          af3_f32x16 acc[TM][TN], int nks = kBK / 16) {
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lk = lane >> 5;
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) {
    if (ks >= nks) break;  // (wave-uniform) sub-steps past a short k segment hold only zero padding
    af3_bf16x8 af[TM], bf[TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
      af[tm] = *(const af3_bf16x8*)(As + lds_off(wm0 + tm * 32 + lr, ks * 2 + lk));
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
      bf[tn] = *(const af3_bf16x8*)(Bs + lds_off(wn0 + tn * 32 + lr, ks * 2 + lk));
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[tm], bf[tn], acc[tm][tn], 0, 0, 0);
  }
}

template <class LA, class LB, int TM, int TN>
__device__ __forceinline__ void run_segment(LA& la, LB& lb, int k_len, uint16_t* As, uint16_t* Bs, int wm0, int wn0,
                                            af3_f32x16 acc[TM][TN]) {
  const int nk = (k_len + kBK - 1) / kBK;
  if (nk <= 0) return;
  la.load(0);
  lb.load(0);
  for (int kt = 0; kt < nk; ++kt) {
    __syncthreads();
    la.store(As);
    lb.store(Bs);
    __syncthreads();
    if (kt + 1 < nk) {
      la.load((kt + 1) * kBK);
      lb.load((kt + 1) * kBK);
    }
    mma_kstep<TM, TN>(As, Bs, wm0, wn0, acc);
  }
}

// ---------------------------------------------------------------------------
// A operand through direct global->LDS loads (global_load_lds_dwordx4):
// k-contiguous bf16 rows, optionally gathered.  One wave instruction fills 8
// LDS tile rows (1 KiB, lane l -> bytes [16 l, 16 l + 16)); lane l fetches the
// logical chunk (l % 8) ^ swz(row) of row l / 8, which realises the swizzled
// layout of lds_off.  Requires K % 64 == 0.  Padding rows (>= nvalid) read the
// tile's first row; their results are never stored.
// ---------------------------------------------------------------------------
template <int TR, int NW>
struct DmaRows {
  static_assert(TR % (8 * NW) == 0, "tile rows must split evenly over the waves");
  static constexpr int kIPW = TR / 8 / NW;  // 1 KiB instructions per wave per k-step
  const uint16_t* rp[kIPW];

  __device__ __forceinline__ void init(const Operand& op, int row0, int nvalid) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint16_t* base = (const uint16_t*)op.ptr;
    int64_t src0 = row0;
    if (op.gather) src0 = op.gather[row0] / op.gdiv;
#pragma unroll
    for (int i = 0; i < kIPW; ++i) {
      const int row = (wave * kIPW + i) * 8 + (lane >> 3);
      int64_t src = src0;
      if (row < nvalid) {
        src = row0 + row;
        if (op.gather) src = op.gather[src] / op.gdiv;
      }
      rp[i] = base + src * op.ld + (((lane & 7) ^ swz(row)) << 3);
    }
  }
  __device__ __forceinline__ void issue(uint16_t* lds, int k0) {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < kIPW; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(rp[i] + k0),
                                       (__attribute__((address_space(3))) void*)(lds + (wave * kIPW + i) * 8 * kBK),
                                       16, 0, 0);
  }
};

// ---------------------------------------------------------------------------
// main grouped GEMM through MXFP4 weights: double-buffered LDS (one barrier
// per k-step), A by direct loads, B (MXFP4, dequantised in registers) by the
// loaders above, optional LoRA extension segment, epilogue as rowtile_kernel.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN, int BK_, int BXK>
__global__ __launch_bounds__(WM * WN * 64) void gemm2_kernel(Params p) {
  constexpr int NW = WM * WN, NT = NW * 64;
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile at least 32x32");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * (BM + BN) * kBK];
  uint16_t* const A0 = lds;
  uint16_t* const B0 = lds + BM * kBK;
  uint16_t* const A1 = lds + (BM + BN) * kBK;
  uint16_t* const B1 = A1 + BM * kBK;

  // 1-D grid over (valid m-tile, n-tile) work items, n-tile fastest.  The
  // hardware deals consecutive workgroups to the 8 XCDs in turn, so workgroup
  // b is remapped to work item (b % 8) * (W8 / 8) + b / 8: each XCD walks a
  // contiguous range and keeps an m-tile's activation rows in its own L2
  // while it sweeps that tile's n-tiles.
  const int NN = p.n_nblk;
  const int W = p.tile_offs[p.E] * NN;  // number of valid m-tiles from the device-side scan
  const int b = blockIdx.x;
  if (b >= W) return;
  const int W8 = W & ~7;
  const int w = b < W8 ? (b & 7) * (W8 >> 3) + (b >> 3) : b;
  const int32_t ent = p.tile_map[w / NN];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * BM;
  const int nrows = min(BM, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = (w % NN) * BN;
  const int ncols = min(BN, p.N - n0);

  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave / WN) * (BM / WM), wn0 = (wave % WN) * (BN / WN);
  af3_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  {
    DmaRows<BM, NW> la;
    la.init(p.a, row_lo, nrows);
    Loader<BN, BK_, NT> lb;
    if constexpr (BK_ == ROWS_FP4)
      lb.init(p.b, e, n0, ncols, p.K);
    else
      lb.init(p.b, e, n0, ncols, 0, p.K);
    const int nk = p.K / kBK;
    la.issue(A0, 0);
    lb.load(0);
    lb.store(B0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      uint16_t* const Ac = (kt & 1) ? A1 : A0;
      uint16_t* const Bc = (kt & 1) ? B1 : B0;
      uint16_t* const An = (kt & 1) ? A0 : A1;
      uint16_t* const Bn = (kt & 1) ? B0 : B1;
      const bool more = kt + 1 < nk;
      if (more) {
        la.issue(An, (kt + 1) * kBK);
        lb.load((kt + 1) * kBK);
      }
      mma_kstep<TM, TN>(Ac, Bc, wm0, wn0, acc);
      if (more) lb.store(Bn);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  if constexpr (BXK != NONE) {
    if (p.kx > 0) {
      Loader<BM, ROWS_BF16, NT> la;
      Loader<BN, BXK, NT> lb;
      la.init(p.ax, 0, row_lo, nrows, p.kx);
      if constexpr (BXK == ROWS_BF16)
        lb.init(p.bx, e, n0, ncols, p.kx);
      else
        lb.init(p.bx, e, n0, ncols, 0, p.kx);
      run_segment<Loader<BM, ROWS_BF16, NT>, Loader<BN, BXK, NT>, TM, TN>(la, lb, p.kx, A0, B0, wm0, wn0, acc);
    }
  }

  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int col = wn0 + tn * 32 + (lane & 31);
      if (col >= ncols) continue;
      const int n = n0 + col;
      const float bv = p.bias ? p.bias[e * p.bias_estride + n] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm0 + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (row >= nrows) continue;
        const int64_t gr = row_lo + row;
        float v = acc[tm][tn][r] + bv;
        if (p.gammas)
          v *= p.gammas_f32 ? ((const float*)p.gammas)[gr] : af3_bf16_to_f32(((const uint16_t*)p.gammas)[gr]);
        p.c[gr * p.ldc + n] = (uint16_t)af3_f32_to_bf16(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// gemm4: forward grouped GEMM through MXFP4 weights packed along k
// (W[e][n][k/32][16]).  512 threads = 8 waves (two per SIMD) in a 2x4
// arrangement of 128x64 wave tiles over a 256x256 output tile (tiles of
// <= 128 rows: 128x512, waves 1x8).
//   * A (activation rows, optionally gathered) goes global->LDS directly
//     (global_load_lds_dwordx4) into a 3-stage ring of [256][64] bf16 tiles
//     (16-byte chunks XOR-swizzled by row, as lds_off);
//   * B stays packed in LDS: per 64-deep k-step the two MXFP4 blocks (32 B)
//     of each of the 256 weight rows, also loaded global->LDS, 3-stage ring;
//   * the e8m0 scale bytes of the tile's weight rows are loaded once per
//     work item;
//   * each wave dequantises its own 128 columns in registers
//     (v_cvt_scalef32_pk_bf16_fp4) straight into MFMA B fragments, so the bf16
//     weight never exists in LDS or HBM.
// k is permuted inside a k-step so that a lane's B fragment is one whole MXFP4
// block: lane (r, h) of v_mfma_f32_32x32x16_bf16 feeds k = 32 h + 8 s + (0..7)
// at sub-step s, i.e. A chunk 4 h + s and dword s of block 2 kt + h.  Both
// operands use the same permutation, so the dot products are unchanged.
// Loads run two k-steps ahead; each wave waits for its own loads of the
// current stage (exact vmcnt: 10 DMA instructions per wave per stage), then
// one barrier per k-step publishes the stage and frees the oldest one.
// Rows / columns past the tile's valid extent are loaded from valid addresses
// and their 32x32 MFMA sub-tiles are skipped (wave-uniform), so a short tail
// tile of an expert costs about its valid rows, not 256.
// ---------------------------------------------------------------------------
constexpr int kG4Stages = 3;
constexpr int kG4Rows = 256;               // BM = BN
constexpr int kG4AStage = kG4Rows * kBK;   // bf16 elements per A stage (32 KB)
constexpr int kG4BStage = kG4Rows * 32;    // bytes per packed-B stage (8 KB)
constexpr int kG4MaxG = 128;               // scale bytes per weight row (K <= 4096)
constexpr int kG4LdsBytes = kG4Stages * (kG4AStage * 2 + kG4BStage) + kG4Rows * kG4MaxG;  // 152 KB
static_assert(kG4LdsBytes >= 256 * 512 + 2048, "the epilogue reuses the LDS for the bf16 tile + row gammas / scales");
static_assert(kG4LdsBytes <= 160 * 1024, "gfx950 LDS per workgroup");

// Work item (m-tile, n-tile) of workgroup b.  Work goes in groups of GM
// m-tiles x all NN n-tiles (m-tile fastest inside a group, so the ~32 items an
// XCD runs at once share GM activation tiles and 32 / GM weight tiles through
// its L2); the groups are dealt to the 8 XCDs in turn (workgroup b runs on XCD
// b % 8), so with the m-tiles listed full tiles first and partial tiles by
// decreasing rows every XCD receives the same mix of expensive and cheap work.
// Returns false for workgroups past the work (the grid is rounded up to whole
// groups per XCD).
__device__ __forceinline__ bool g4_work_item(const Params& p, int& mt, int& nt) {
  const int NN = p.n_nblk;
  const int Mt = p.tile_offs[p.E];
  const int GM = p.group_m > 0 ? p.group_m : 1;
  const int per_group = GM * NN;
  const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int q = j / per_group, r = j - q * per_group;
  const int first_m = (x + 8 * q) * GM;
  if (first_m >= Mt) return false;
  const int gsz = min(GM, Mt - first_m);
  if (r >= gsz * NN) return false;
  mt = first_m + r % gsz;
  nt = r / gsz;
  return true;
}

// grid of g4_work_item for up to max_tiles m-tiles
static inline unsigned g4_grid(int max_tiles, int NN, int GM) {
  const long long groups = (max_tiles + GM - 1) / GM;
  return (unsigned)(8 * ((groups + 7) / 8) * GM * NN);
}

// Epilogue of a 256x256 (or CN = 512: 128x512) tile computed by waves of 32x32 MFMA
// sub-tiles: v = (acc + bias[n]) * gamma[row] -> bf16, staged through LDS as
// a [256][256] bf16 tile (16-byte chunks XOR-swizzled so the two row groups
// of an MFMA output store hit disjoint banks), then written out with one
// 16-byte store per chunk (a wave writes two whole 512-byte rows at a time).
// `lds` must hold >= 129 KB; every wave must have finished reading its
// operands from it.
template <int CN = 256>
__device__ __forceinline__ int g4_c_off(int row, int col) {  // byte offset of C[row][col] in the LDS tile
  return row * (CN * 2) + ((((col >> 3) ^ (((row >> 2) & 1) << 2))) << 4) + ((col & 7) << 1);
}

// Column of MFMA sub-tile tn, lane column lr inside a wave's 128 columns:
// plain (32 consecutive columns per sub-tile) or PAIRED (sub-tiles 2t and
// 2t + 1 hold the even / odd columns of 64 consecutive columns).
template <bool PAIRED>
__device__ __forceinline__ int g4_col(int tn, int lr) {
  return PAIRED ? 64 * (tn >> 1) + 2 * lr + (tn & 1) : tn * 32 + lr;
}

template <bool PAIRED = false, int TM = 4, int TN = 4, int NT = 256, int CN = 256, int RM = 256>
__device__ __forceinline__ void g4_epilogue(const Params& p, uint8_t* lds, af3_f32x16 acc[TM][TN], int e, int row_lo,
                                            int nrows, int n0, int ncols, int wm0, int wn0) {
  constexpr int CH = CN / 8;  // 16-byte chunks per tile row
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  float* const gl = (float*)(lds + RM * CN * 2);  // per-row gammas
  float* const al = gl + RM;                        // per-row A scales
  __syncthreads();
  for (int t = threadIdx.x; t < RM; t += NT) {
    float gv = 1.f;
    if (p.gammas && t < nrows) {
      const int64_t gr = row_lo + t;
      gv = p.gammas_f32 ? ((const float*)p.gammas)[gr] : af3_bf16_to_f32(((const uint16_t*)p.gammas)[gr]);
    }
    gl[t] = gv;
    al[t] = t < nrows ? g4_ascale(p, row_lo + t) : 1.f;
  }
  float bv[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int col = wn0 + g4_col<PAIRED>(tn, lr);
    bv[tn] = (p.bias && col < ncols) ? p.bias[e * p.bias_estride + n0 + col] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row0 = wm0 + tm * 32 + j * 8 + lh * 4;
      const float4 g = *(const float4*)(gl + row0);
      const float gq[4] = {g.x, g.y, g.z, g.w};
      const float4 a = *(const float4*)(al + row0);
      const float aq[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int col = wn0 + g4_col<PAIRED>(tn, lr);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x = acc[tm][tn][j * 4 + q];
          const float v = p.ascale ? (x * aq[q] + bv[tn]) * gq[q] : (x + bv[tn]) * gq[q];
          *(uint16_t*)(lds + g4_c_off<CN>(row0 + q, col)) = (uint16_t)af3_f32_to_bf16(v);
        }
      }
    }
  }
  __syncthreads();
#pragma unroll 4
  for (int i = 0; i < RM * CH / NT; ++i) {
    const int id = i * NT + threadIdx.x;
    const int row = id / CH, ch = id % CH;
    if (row < nrows && ch * 8 < ncols) {
      const af3_u32x4 v = *(const af3_u32x4*)(lds + row * (CN * 2) + ((ch ^ (((row >> 2) & 1) << 2)) << 4));
      *(af3_u32x4*)(p.c + (int64_t)(row_lo + row) * p.ldc + n0 + ch * 8) = v;
      if (p.epi == 2) {  // SwiGLU of the chunk's 4 (gate, up) pairs, from the bf16 values just stored
        uint32_t o[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float r0, r1, g, u;
          af3_swiglu_fwd_elem(af3_bf16_to_f32(v[2 * h] & 0xFFFFu), af3_bf16_to_f32(v[2 * h] >> 16), p.alpha,
                              p.limit, r0, g, u);
          af3_swiglu_fwd_elem(af3_bf16_to_f32(v[2 * h + 1] & 0xFFFFu), af3_bf16_to_f32(v[2 * h + 1] >> 16),
                              p.alpha, p.limit, r1, g, u);
          o[h] = af3_pack_bf16x2(r0, r1);
        }
        *(uint2*)((uint16_t*)p.glu + (int64_t)(row_lo + row) * p.ld_glu + ((n0 + ch * 8) >> 1)) = uint2{o[0], o[1]};
      }
    }
  }
}

// byte offset of (weight row n, block h) inside a packed-B stage: four rows
// share a 128-byte line, the block bit is flipped every 8 rows, so the 16
// lanes of an MFMA fragment read hit 16 distinct 16-byte bank groups
__device__ __forceinline__ int g4_b_off(int n, int h) {
  return (n >> 2) * 128 + (((h << 2) | (n & 3)) ^ (((n >> 3) & 1) << 2)) * 16;
}

// The k-loop's global->LDS copies are issued through inline assembly so that
// the compiler's wait-count insertion, which cannot tell the LDS stages apart
// and would wait for every copy in flight before any LDS read, leaves them
// alone; the loop waits for them explicitly (vmcnt) and publishes a stage with
// a bare s_barrier.  All three are compiler memory barriers.
__device__ __forceinline__ void g4_dma16(const void* gptr, uint32_t lds_byte_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds_byte_addr) : "memory");
}
// The same with the address split into a wave-uniform 64-bit base (SGPRs) and
// a per-lane 32-bit byte offset: the k-loop advances only the scalar base, so
// the lanes' offsets stay in the same registers for the whole work item (no
// per-copy 64-bit address arithmetic, and no register the copy has yet to read
// is rewritten right after it is issued).
__device__ __forceinline__ void g4_dma16_s(const void* sbase, uint32_t voff, uint32_t lds_byte_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_byte_addr) : "memory");
}
#define AF3_ASM_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")
#define AF3_ASM_BARRIER() asm volatile("s_barrier" ::: "memory")
// the same after this wave's own LDS stores have completed
#define AF3_ASM_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ af3_bf16x8 g4_cvt(uint32_t v, float sc) {
  af3_u32x4 o;
  o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 0));
  o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 1));
  o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 2));
  o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 3));
  return __builtin_bit_cast(af3_bf16x8, o);
}

__device__ __forceinline__ af3_bf16x8 g4_int(uint32_t v, uint32_t scale) {
  uint32_t o[4];
  af3_dequant_u32_int(v, scale, o);
  return __builtin_bit_cast(af3_bf16x8, af3_u32x4{o[0], o[1], o[2], o[3]});
}

// B fragment of sub-step s: dword s of the lane's MXFP4 block -> 8 bf16.
// EXACT (work items whose tile holds a scale byte outside [2, 252], which
// normal quantisers never produce): the integer restatement for those lanes.
template <bool EXACT>
__device__ __forceinline__ af3_bf16x8 g4_bfrag(uint32_t v, uint32_t sc, float scf) {
  if constexpr (EXACT) {
    if (sc - 2u > 250u) return g4_int(v, sc);
  }
  return g4_cvt(v, scf);
}

// one 64-deep k-step of a wave's (32 TM) x (32 TN) tile, software-pipelined
// by one sub-step: af[1] / bf[1] enter holding the previous k-step's last
// sub-step (zeros before the first k-step), whose MFMAs run first and cover
// the LDS reads and B conversions of this k-step's sub-step 0; this k-step's
// sub-step 3 leaves in af[1] / bf[1].  FULL: every sub-tile live.
// sc[] enters holding this k-step's e8m0 bytes and leaves holding the next
// k-step's (the scales stay in LDS for the whole work item, so they are read
// a k-step ahead and the k-step starts without waiting for them).
// Instruction order is fixed by scheduling barriers: the conversions of the
// next sub-step's B fragments take the last TN MFMA slots of a sub-step (so
// the packed B bytes read after the k-step's barrier have the sub-step's
// first MFMAs to land), the k-step's DPW global->LDS copies are spread
// between the MFMAs, and the A-fragment LDS reads of sub-step s + 1 are
// issued ahead of the MFMAs of sub-step s.
template <int TM, int TN, int DPW, bool FULL, bool EXACT, bool BG, class Dma>
__device__ __forceinline__ void g4_kstep(const uint16_t* as, const uint8_t* bs, const af3_u32x4 (&bqv)[TN],
                                         const uint8_t* ss, int G, int kt,
                                         bool more, int wm0, int wn0, int tm_live, int tn_live,
                                         af3_f32x16 acc[TM][TN], af3_bf16x8 af[2][TM], af3_bf16x8 bf[2][TN],
                                         uint32_t sc[TN], Dma&& dma) {
  constexpr int NM = TM * TN * 4;      // MFMAs per k-step
  constexpr int GAP = NM / (DPW + 1);  // MFMAs between copies
  constexpr int NS = TM * TN;          // MFMAs per sub-step
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  af3_u32x4 bp[TN];
  float scf[TN];
  uint32_t sc_next[TN];
  // (partial tiles: no LDS reads or conversions for dead sub-tiles)
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int n = wn0 + tn * 32 + lr;
    if constexpr (BG)
      bp[tn] = (FULL || tn < tn_live) ? bqv[tn] : zero4();
    else
      bp[tn] = (FULL || tn < tn_live) ? *(const af3_u32x4*)(bs + g4_b_off(n, lh)) : zero4();
    scf[tn] = __uint_as_float(sc[tn] << 23);
    sc_next[tn] = 127u;
  }
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
    if (FULL || tm < tm_live) af[0][tm] = *(const af3_bf16x8*)(as + lds_off(wm0 + tm * 32 + lr, lh * 4));
  // sub-step -1 (the carried one) and sub-steps 0..2; the k-step's copies
  // are spread over all of their MFMAs
#pragma unroll
  for (int s = -1; s < 3; ++s) {
    const int c = s < 0 ? 1 : (s & 1);  // fragments used by this sub-step
    const int nx = s < 0 ? 0 : (c ^ 1);  // fragments of sub-step s + 1
    __builtin_amdgcn_sched_barrier(0);
    if (s >= 0) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        if (FULL || tm < tm_live) af[nx][tm] = *(const af3_bf16x8*)(as + lds_off(wm0 + tm * 32 + lr, lh * 4 + s + 1));
    }
    if (s == 0 && more) {  // the next k-step's scale bytes
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        if (FULL || tn < tn_live) sc_next[tn] = ss[(wn0 + tn * 32 + lr) * G + 2 * (kt + 1) + lh];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int tm = i / TN, tn = i % TN;
      if (FULL || (tm < tm_live && tn < tn_live))
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[c][tm], bf[c][tn], acc[tm][tn], 0, 0, 0);
      if (i >= NS - TN) {  // B fragment t of sub-step s + 1 in each of the last TN slots
        const int t = i - (NS - TN);
        if (FULL || t < tn_live) bf[nx][t] = g4_bfrag<EXACT>(bp[t][s + 1], sc[t], scf[t]);
      }
      const int q = (s + 1) * NS + i;
      if (q % GAP == GAP / 2 && q / GAP < DPW) dma(q / GAP);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) sc[tn] = sc_next[tn];
}

// Packed weight words global -> registers (inline assembly, counted by the
// k-loop's explicit vmcnt waits), and the marker that ties the registers to
// the wait that covers them: every later use depends on its output.
template <int TN>
__device__ __forceinline__ void g7_load_words(af3_u32x4 (&dst)[TN], const uint8_t* const (&src)[TN], int off) {
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(dst[tn]) : "v"(src[tn] + off) : "memory");
}
template <int TN>
__device__ __forceinline__ void g7_load_words_s(af3_u32x4 (&dst)[TN], const uint32_t (&voff)[TN], const void* sbase) {
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(dst[tn]) : "v"(voff[tn]), "s"(sbase) : "memory");
}
template <int TN>
__device__ __forceinline__ void g7_landed(af3_u32x4 (&r)[TN]) {
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) asm volatile("" : "+v"(r[tn]));
}

// One work item of the forward kernel: a RM x CN output tile (256 x 256, or
// NARROW 128 x 512 for the partial tiles of short experts, so a tail tile of
// <= 128 rows converts each weight byte once per 128 rows instead of per 256).
// The 8 waves are WM x WN (NARROW: 1 x 8) of the same 128 x 64 wave tile.
// SHAPE 0: 256 x 256 (WM x WN waves), 1 (NARROW): 128 x 512 (8 waves side by
// side), 2 (HALF): 128 x 256 (4 waves side by side; two blocks per CU)
template <int WM, int WN, int BXK, int SHAPE, bool BG = false, int NB = 2, bool SA = false>
__device__ __forceinline__ void g4f_tile(const Params& p, uint8_t* lds, int e, int row_lo, int nrows, int n0,
                                         int ncols) {
  constexpr bool NARROW = SHAPE == 1, HALF = SHAPE == 2;
  static_assert(NB == 2 || (NB == 3 && BG), "weight register buffers: 2, or 3 (BG, k-steps a multiple of 3)");
  // SA (BG): the k-loop's A copies and weight loads address a scalar base
  // plus a 32-bit per-lane offset (a_off32; the expert's packed weights < 4 GiB)
  static_assert(!SA || BG, "scalar-base addressing in the register-weight kernel");
  static_assert(!HALF || BG, "the 128 x 256 shape takes the packed weights from registers");
  constexpr int NW = HALF ? 4 : WM * WN, NT = NW * 64;
  constexpr int RM = (NARROW || HALF) ? 128 : kG4Rows, CN = NARROW ? 512 : kG4Rows;
  constexpr int WMX = (NARROW || HALF) ? 1 : WM, WNX = (NARROW || HALF) ? NW : WN;
  constexpr int TM = RM / WMX / 32, TN = CN / WNX / 32;
  constexpr int ASTAGE = RM * kBK;  // bf16 elements per A stage
  constexpr int BSTAGE = CN * 32;   // bytes per packed-B stage
  // copies per wave per k-step (BG: the packed weights go straight to registers, no B copies)
  constexpr int API = RM / 8 / NW, BPI = BG ? 0 : CN / 32 / NW, DPW = API + BPI;
  static_assert(API >= 1 && (BG || BPI >= 1) && (DPW == 10 || DPW == 8 || DPW == 5 || DPW == 4 || DPW == 2),
                "copy schedule");
  static_assert(kG4Stages * (ASTAGE * 2 + BSTAGE) <= kG4Stages * (kG4AStage * 2 + kG4BStage), "LDS ring");
  uint16_t* const As = (uint16_t*)lds;                    // 3 x RM x 64 bf16
  uint8_t* const Bs = lds + kG4Stages * ASTAGE * 2;       // 3 x CN x 32 bytes (not with BG)
  uint8_t* const Ss = BG ? Bs : Bs + kG4Stages * BSTAGE;  // CN x G scale bytes
  const int G = p.K >> 5;
  const int nk = p.K / kBK;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar)
  const int lr = lane & 31, lh = lane >> 5;
  const int wm0 = (wave / WNX) * (32 * TM), wn0 = (wave % WNX) * (32 * TN);
  const int tm_live = min(TM, max(0, (nrows - wm0 + 31) >> 5));
  const int tn_live = min(TN, max(0, (ncols - wn0 + 31) >> 5));
  const bool full = tm_live == TM && tn_live == TN;

  // DMA sources: A rows (API instructions per wave per stage, 8 rows each);
  // SA: byte offsets from a.ptr
  const uint16_t* arow[API];
  uint32_t aoff[API];
#pragma unroll
  for (int i = 0; i < API; ++i) {
    const int row = (wave * API + i) * 8 + (lane >> 3);
    int64_t src = row_lo + (row < nrows ? row : 0);
    if (p.a.gather) src = p.a.gather[src] / p.a.gdiv;
    const int64_t el = src * p.a.ld + (((lane & 7) ^ swz(row)) << 3);
    arow[i] = (const uint16_t*)p.a.ptr + el;
    aoff[i] = (uint32_t)(el * 2);
  }
  // packed B (BPI instructions per wave per stage, 32 weight rows each)
  const uint8_t* bsrc[BPI > 0 ? BPI : 1];
#pragma unroll
  for (int j = 0; j < BPI; ++j) {
    const int row4 = (wave * BPI + j) * 8 + (lane >> 3);
    const int lc = (lane & 7) ^ (((row4 >> 1) & 1) << 2);
    int nn = row4 * 4 + (lc & 3);
    if (nn >= ncols) nn = 0;
    bsrc[j] = (const uint8_t*)p.b.ptr + e * p.b.estride + (int64_t)(n0 + nn) * p.b.ld + (lc >> 2) * 16;
  }
  // scales of the tile's weight rows: [ncols][G] bytes, contiguous in memory
  {
    const uint8_t* sbase = p.b.scales + e * p.b.sestride + (int64_t)n0 * G;
    const int nbytes = ncols * G;  // multiple of 32: ncols % 32 == 0
    const int ninstr = (nbytes + 1023) >> 10;
    for (int i = wave; i < ninstr; i += NW) {
      int off = i * 1024 + lane * 16;
      const int src = off < nbytes ? off : 0;
      g4_dma16(sbase + src, __builtin_amdgcn_readfirstlane(lds_addr(Ss)) + (uint32_t)(i * 1024));
    }
  }
  // copy j (0..DPW-1) of k-step kt: API A instructions (8 rows each), then BPI packed-B
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));  // LDS byte address of the block's area
  auto issue_one = [&](int kt, int j) {
    const int st = kt % kG4Stages;
    // BG: the k-steps past the end copy the last k-step's rows again (into a stage no wave reads again)
    const int ks = BG ? min(kt, nk - 1) : kt;
    if (j < API) {
      const uint32_t dst = lds0 + (uint32_t)(st * ASTAGE * 2 + (wave * API + j) * 8 * kBK * 2);
      if constexpr (SA)
        g4_dma16_s((const uint8_t*)p.a.ptr + (int64_t)ks * kBK * 2, aoff[j], dst);
      else
        g4_dma16(arow[j] + ks * kBK, dst);
    } else if constexpr (BPI > 0)
      g4_dma16(bsrc[j - API] + kt * 32,
               lds0 + (uint32_t)(kG4Stages * ASTAGE * 2 + st * BSTAGE + (wave * BPI + j - API) * 1024));
  };
  auto issue = [&](int kt) {
#pragma unroll
    for (int j = 0; j < DPW; ++j) issue_one(kt, j);
  };
  // k-step kt's stage is complete once this wave's copies for it have landed
  // (at most DPW newer ones outstanding, none for the last k-step)
  auto wait_stage = [&](bool last) {
    if (last)
      AF3_ASM_WAIT_VM(0);
    else if constexpr (DPW == 10)
      AF3_ASM_WAIT_VM(10);
    else if constexpr (DPW == 8)
      AF3_ASM_WAIT_VM(8);
    else if constexpr (DPW == 5)
      AF3_ASM_WAIT_VM(5);
    else if constexpr (DPW == 4)
      AF3_ASM_WAIT_VM(4);
    else
      AF3_ASM_WAIT_VM(2);
  };
  // BG: the lane's packed weight words of a k-step (row wn0 + 32 tn + lr, MXFP4 block 2 kt + lh: the
  // 16 bytes of its B fragments for the whole k-step) go global -> registers NB - 1 k-steps ahead,
  // into bq[kt % NB] (NB = 3 needs nk % 3 == 0, so the loop runs whole triples); the loads are
  // issued by inline assembly like the copies (so the k-step waits stay exact) and each k-step's
  // registers pass through an empty asm after the vmcnt wait, so no use of them can be scheduled
  // before it.  Rows past the tile read row 0 (their sub-tiles are skipped).
  // With the forward-tiled copy (p.b_tiled) the words of one k-step of the
  // wave's 32 rows of sub-tile tn are one contiguous KB, lane l's at 16 l, so
  // each load instruction reads 8 whole 128-byte lines (row-major, it takes 32
  // bytes of 32 different lines, each line re-read over four k-steps).
  af3_u32x4 bq[NB][TN];
  const uint8_t* bgp[TN];
  uint32_t boff[TN];  // SA: byte offsets from the expert's weights
  const int bstep = BG && p.b_tiled ? 1024 : 32;  // bytes between a lane's words of consecutive k-steps
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const uint8_t* eb = (const uint8_t*)p.b.ptr + e * p.b.estride;
    int64_t o;
    if (BG && p.b_tiled) {  // ncols % 32 == 0: a 32-row group is live or dead as a whole
      const int nb = wn0 + tn * 32 < ncols ? n0 + wn0 + tn * 32 : 0;
      o = (int64_t)nb * p.b.ld + lane * 16;  // the group's tiles start at row nb's byte offset
    } else {
      int nr = wn0 + tn * 32 + lr;
      if (nr >= ncols) nr = 0;
      o = (int64_t)(n0 + nr) * p.b.ld + lh * 16;
    }
    bgp[tn] = eb + o;
    boff[tn] = (uint32_t)o;
#pragma unroll
    for (int b = 0; b < NB; ++b) bq[b][tn] = zero4();
  }
  auto load_b = [&](int kt, auto par) {
    if constexpr (SA)
      g7_load_words_s<TN>(bq[decltype(par)::value], boff,
                          (const uint8_t*)p.b.ptr + e * p.b.estride + (int64_t)kt * bstep);
    else
      g7_load_words<TN>(bq[decltype(par)::value], bgp, kt * bstep);
  };
  const bool live = tm_live > 0 && tn_live > 0;

  af3_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // two blocks share each CU: while one runs its epilogue (VALU and memory
  // work), the other's k-loop keeps issue priority for its MFMAs and copies
  if constexpr (HALF) __builtin_amdgcn_s_setprio(2);
  // BG: the weight words of k-step 0 (NB = 3: and 1), each before its
  // k-step's copies (the order every later k-step keeps: its weight loads
  // first, then its copies)
  if constexpr (BG) {
    if (live) load_b(0, std::integral_constant<int, 0>{});
  }
  issue(0);
  if constexpr (NB == 3) {
    if (live) load_b(1, std::integral_constant<int, 1>{});
  }
  if (BG || nk > 1) issue(1);
  // does the tile hold a scale byte outside [2, 252]?  (then the whole work
  // item takes the exact integer dequantisation)
  bool odd = false;
  {
    AF3_ASM_WAIT_VM(0);
    AF3_ASM_BARRIER();
    const int nbytes = ncols * G;
    for (int i = threadIdx.x * 16; i < nbytes; i += NT * 16) {
      const af3_u32x4 v = *(const af3_u32x4*)(Ss + i);
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) odd |= ((v[q] >> (8 * j)) & 0xFFu) - 2u > 250u;
    }
  }
  odd = __syncthreads_or(odd);

  // FULL: every sub-tile of the wave's first TMV row groups is live (TMV < TM:
  // a partial m-tile whose columns are all live, compiled per row-group count
  // so the k-loop holds no registers for the dead row groups); otherwise the
  // live sub-tiles are chosen at run time
  auto kloop = [&](auto full_c, auto exact_c, auto rows_c) {
    constexpr bool FULL = decltype(full_c)::value, EXACT = decltype(exact_c)::value;
    constexpr int TMV = decltype(rows_c)::value;
    static_assert(FULL || TMV == TM, "run-time sub-tile selection covers all row groups");
    af3_bf16x8 af[2][TMV], bf[2][TN];
    const af3_bf16x8 zf = __builtin_bit_cast(af3_bf16x8, zero4());
#pragma unroll
    for (int tm = 0; tm < TMV; ++tm) af[1][tm] = zf;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) bf[1][tn] = zf;
    // the barrier after the wait also orders the carried fragment reads of
    // stage kt - 1 before the copies into that stage (issued for kt + 2 during kt)
    uint32_t sc[TN];  // the e8m0 bytes of the lane's B rows for the current k-step
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
      sc[tn] = (FULL || tn < tn_live) ? Ss[(wn0 + tn * 32 + lr) * G + lh] : 127u;
    auto step = [&](int kt, auto last_c, auto par, auto&& dma) {
      constexpr int P = decltype(par)::value;
      constexpr bool last = decltype(last_c)::value;
      if constexpr (BG) {
        // uniform k-steps: every earlier k-step issued TN weight loads (for
        // NB - 1 k-steps later) and then API copies (for two k-steps later), so
        // this k-step's data is everything but the newest API operations (NB =
        // 2) or the newest TN + API (NB = 3: the previous k-step's loads too)
        if constexpr (NB == 3) {
          static_assert(DPW + TN == 6, "wait count");
          AF3_ASM_WAIT_VM(6);
        } else {
          wait_stage(false);
        }
        g7_landed<TN>(bq[P]);
        AF3_ASM_LDS_BARRIER();
        load_b(min(kt + NB - 1, nk - 1), std::integral_constant<int, (P + NB - 1) % NB>{});
      } else {
        wait_stage(last);
        AF3_ASM_LDS_BARRIER();
      }
      const int st = kt % kG4Stages;
      g4_kstep<TMV, TN, DPW, FULL, EXACT, BG>(As + st * ASTAGE, Bs + st * BSTAGE, bq[P], Ss, G, kt, BG || !last,
                                              wm0, wn0, tm_live, tn_live, acc, af, bf, sc, dma);
    };
    constexpr std::integral_constant<int, 0> I0{};
    constexpr std::integral_constant<int, 1> I1{};
    constexpr std::false_type MORE{};
    constexpr std::true_type LAST{};
    int kt = 0;
    if constexpr (BG) {
      if constexpr (NB == 3) {
        // whole triples (nk % 3 == 0; the register buffer of each k-step is
        // static and no path of the compiled loop skips a k-step)
        for (; kt < nk; kt += 3) {
          step(kt, MORE, I0, [&](int j) { issue_one(kt + 2, j); });
          step(kt + 1, MORE, I1, [&](int j) { issue_one(kt + 3, j); });
          step(kt + 2, MORE, std::integral_constant<int, 2>{}, [&](int j) { issue_one(kt + 4, j); });
        }
      } else {
        // pairs of k-steps (the register parity is static)
        for (; kt < nk; kt += 2) {
          step(kt, MORE, I0, [&](int j) { issue_one(kt + 2, j); });
          if (kt + 1 < nk) step(kt + 1, MORE, I1, [&](int j) { issue_one(kt + 3, j); });
        }
      }
      // the redundant copies and weight loads past the end have landed before
      // the LDS is reused; all weight-register buffers stay allocated until
      // this wait (a dead load's registers handed to another value before its
      // data lands would be overwritten by it)
      AF3_ASM_WAIT_VM(0);
#pragma unroll
      for (int b = 0; b < NB; ++b) g7_landed<TN>(bq[b]);
    } else {
      for (; kt + 2 < nk; ++kt) step(kt, MORE, I0, [&](int j) { issue_one(kt + 2, j); });
      if (nk - kt == 2) step(kt++, MORE, I0, [](int) {});
      step(kt, LAST, I0, [](int) {});
    }
    // the last k-step's sub-step 3
#pragma unroll
    for (int i = 0; i < TMV * TN; ++i) {
      const int tm = i / TN, tn = i % TN;
      if (FULL || (tm < tm_live && tn < tn_live))
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][tm], bf[1][tn], acc[tm][tn], 0, 0, 0);
    }
  };
  constexpr std::integral_constant<int, TM> ALL_ROWS{};
  // NB = 3 (N % 64 == 0: a live wave's columns are all live): every k-loop
  // is compiled for its wave's live row groups, with the exact conversion or
  // without, and none selects sub-tiles at run time
  auto by_rows = [&](auto exact_c) {
    if constexpr (NB == 3 && TM == 4) {
      if (tm_live >= 4)
        kloop(std::true_type{}, exact_c, ALL_ROWS);
      else if (tm_live == 3)
        kloop(std::true_type{}, exact_c, std::integral_constant<int, 3>{});
      else if (tm_live == 2)
        kloop(std::true_type{}, exact_c, std::integral_constant<int, 2>{});
      else
        kloop(std::true_type{}, exact_c, std::integral_constant<int, 1>{});
    }
  };
  if (NB == 3 && tm_live > 0 && tn_live > 0) {
    if (odd)
      by_rows(std::true_type{});
    else
      by_rows(std::false_type{});
  } else if (NB == 2 && odd) {
    if constexpr (NB == 2) kloop(std::false_type{}, std::true_type{}, ALL_ROWS);
  } else if (NB == 2 && full) {
    if constexpr (NB == 2) kloop(std::true_type{}, std::false_type{}, ALL_ROWS);
  } else if (NB == 2 && BG && TM == 4 && tn_live == TN && tm_live > 0) {  // tm_live < TM: a partial m-tile
    if constexpr (NB == 2 && BG && TM == 4) {
      if (tm_live == 3)
        kloop(std::true_type{}, std::false_type{}, std::integral_constant<int, 3>{});
      else if (tm_live == 2)
        kloop(std::true_type{}, std::false_type{}, std::integral_constant<int, 2>{});
      else
        kloop(std::true_type{}, std::false_type{}, std::integral_constant<int, 1>{});
    }
  } else if (NB == 2 && tm_live > 0 && tn_live > 0) {
    if constexpr (NB == 2) kloop(std::false_type{}, std::false_type{}, ALL_ROWS);
  } else {
    // a wave with no live sub-tile (rows or columns past the end of a
    // partial tile) only keeps the copy / barrier protocol of the k-loop, so
    // the live wave sharing its SIMD runs alone
    for (int kt = 0; kt < nk; ++kt) {
      if constexpr (BG) {
        wait_stage(false);
        AF3_ASM_LDS_BARRIER();
        issue(kt + 2);
      } else {
        wait_stage(kt + 1 == nk);
        AF3_ASM_LDS_BARRIER();
        if (kt + 2 < nk) issue(kt + 2);
      }
    }
    if constexpr (BG) AF3_ASM_WAIT_VM(0);
  }

  if constexpr (BXK != NONE) {
    if (p.kx > 0) {  // expert-LoRA segment: + L[r] . Bx[e][n]^T, both bf16 through LDS
      Loader<RM, ROWS_BF16, NT> la;
      Loader<CN, ROWS_BF16, NT> lb;
      la.init(p.ax, 0, row_lo, nrows, p.kx);
      lb.init(p.bx, e, n0, ncols, p.kx);
      for (int k0 = 0; k0 < p.kx; k0 += kBK) {
        la.load(k0);
        lb.load(k0);
        __syncthreads();
        la.store(As);
        lb.store(As + RM * kBK);
        __syncthreads();
        mma_kstep<TM, TN>(As, As + RM * kBK, wm0, wn0, acc, (min(kBK, p.kx - k0) + 15) / 16);
      }
    }
  }

  if constexpr (HALF) __builtin_amdgcn_s_setprio(0);  // the k-loop's waves first (see the k-loop's start)
  g4_epilogue<false, TM, TN, NT, CN, RM>(p, lds, acc, e, row_lo, nrows, n0, ncols, wm0, wn0);
}

// scale bytes of a NARROW work item (512 weight rows x G) fit behind its rings
constexpr int kG4NarrowMaxG = (kG4LdsBytes - kG4Stages * (128 * kBK * 2 + 512 * 32)) / 512;

template <int WM, int WN, int BXK>
__global__ __launch_bounds__(WM * WN * 64) void gemm4_fwd_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kG4LdsBytes];
  int mt, nt;
  if (!g4_work_item(p, mt, nt)) return;
  const int32_t ent = p.tile_map[mt];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * kG4Rows;
  const int nrows = min(kG4Rows, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = nt * kG4Rows;
  if constexpr (WM * WN == 8) {
    if (nrows <= 128 && (p.K >> 5) <= kG4NarrowMaxG) {
      // tiles of <= 128 rows take n-tiles nt and nt + 1 as one 128 x 512 item
      if (nt & 1) return;
      g4f_tile<WM, WN, BXK, 1>(p, lds, e, row_lo, nrows, n0, min(512, p.N - n0));
      return;
    }
  }
  g4f_tile<WM, WN, BXK, 0>(p, lds, e, row_lo, nrows, n0, min(kG4Rows, p.N - n0));
}

// Two independent blocks per CU: 128 x 256 items of 4 waves (one per SIMD per
// block) on the 128-row tile map, packed weights from registers, so one
// block's epilogue and barriers overlap the other block's k-loop.
constexpr int kG7MaxG = 96;  // scale bytes per weight row (K <= 3072)
constexpr int kG7LdsBytes = kG4Stages * 128 * kBK * 2 + 256 * kG7MaxG;  // 72 KB
static_assert(kG7LdsBytes >= 128 * 256 * 2 + 1024, "the epilogue reuses the LDS for the bf16 tile + row gammas / scales");

template <int BXK, int NB, bool SA>
__global__ __launch_bounds__(256, 2) void gemm7_fwd_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kG7LdsBytes];
  int mt, nt;
  if (!g4_work_item(p, mt, nt)) return;
  const int32_t ent = p.tile_map[mt];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * 128;
  const int nrows = min(128, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = nt * 256;
  g4f_tile<1, 4, BXK, 2, true, NB, SA>(p, lds, e, row_lo, nrows, n0, min(256, p.N - n0));
}

// ---------------------------------------------------------------------------
// fp8-mode forward: A = per-token E4M3 codes [rows][K] bytes, B = the packed
// MXFP4 weights fed to the block-scaled MFMA v_mfma_scale_f32_32x32x64_f8f6f4
// (A format E4M3 with block scale 2^0, B format E2M1 with the group's e8m0
// byte), so the weights are never converted: one 16-byte MXFP4 group is the B
// operand of a lane (lanes 32 h + n hold weight row n, k block h of the
// 64-deep step).  The A operand of lane 32 h + r holds row r's k 16 h .. 16 h
// + 15 in bytes 0-15 and k 32 + 16 h .. in bytes 16-31 (measured on gfx950).
// The per-token scale multiplies the fp32 accumulator in the epilogue.
// Same work items, ring and epilogue as g4f_tile (8 waves of 128 x 64).
// ---------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(8))) int af3_i32x8;

__device__ __forceinline__ int f8_chunk(int row, int c) { return c ^ ((row >> 2) & 3); }  // physical 16-B chunk

template <bool NARROW>
__device__ __forceinline__ void g4f8_tile(const Params& p, uint8_t* lds, int e, int row_lo, int nrows, int n0,
                                          int ncols) {
  constexpr int WM = 2, WN = 4, NW = 8, NT = 512;
  constexpr int RM = NARROW ? 128 : kG4Rows, CN = NARROW ? 512 : kG4Rows;
  constexpr int WMX = NARROW ? 1 : WM, WNX = NARROW ? NW : WN;
  constexpr int TM = RM / WMX / 32, TN = CN / WNX / 32;
  constexpr int ASTAGE = RM * kBK;  // bytes per A stage (1 byte per code)
  constexpr int BSTAGE = CN * 32;   // bytes per packed-B stage
  constexpr int API = RM / 16 / NW, BPI = CN / 32 / NW, DPW = API + BPI;  // copies per wave per k-step
  static_assert(API >= 1 && BPI >= 1 && (DPW == 3), "copy schedule");
  uint8_t* const As = lds;
  uint8_t* const Bs = lds + kG4Stages * ASTAGE;
  uint8_t* const Ss = Bs + kG4Stages * BSTAGE;  // [ncols][G] scale bytes
  const int G = p.K >> 5;
  const int nk = p.K / kBK;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int wm0 = (wave / WNX) * (32 * TM), wn0 = (wave % WNX) * (32 * TN);
  const int tm_live = min(TM, max(0, (nrows - wm0 + 31) >> 5));
  const int tn_live = min(TN, max(0, (ncols - wn0 + 31) >> 5));

  // A copies: 16 rows x 64 bytes each
  const uint8_t* arow[API];
#pragma unroll
  for (int i = 0; i < API; ++i) {
    const int row = (wave * API + i) * 16 + (lane >> 2);
    int64_t src = row_lo + (row < nrows ? row : 0);
    if (p.a.gather) src = p.a.gather[src] / p.a.gdiv;
    arow[i] = (const uint8_t*)p.a.ptr + src * p.a.ld + (f8_chunk(row, lane & 3) << 4);
  }
  const uint8_t* bsrc[BPI];
#pragma unroll
  for (int j = 0; j < BPI; ++j) {
    const int row4 = (wave * BPI + j) * 8 + (lane >> 3);
    const int lc = (lane & 7) ^ (((row4 >> 1) & 1) << 2);
    int nn = row4 * 4 + (lc & 3);
    if (nn >= ncols) nn = 0;
    bsrc[j] = (const uint8_t*)p.b.ptr + e * p.b.estride + (int64_t)(n0 + nn) * p.b.ld + (lc >> 2) * 16;
  }
  {
    const uint8_t* sbase = p.b.scales + e * p.b.sestride + (int64_t)n0 * G;
    const int nbytes = ncols * G;
    const int ninstr = (nbytes + 1023) >> 10;
    for (int i = wave; i < ninstr; i += NW) {
      const int off = i * 1024 + lane * 16;
      g4_dma16(sbase + (off < nbytes ? off : 0), __builtin_amdgcn_readfirstlane(lds_addr(Ss)) + (uint32_t)(i * 1024));
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  auto issue_one = [&](int kt, int j) {
    const int st = kt % kG4Stages;
    if (j < API)
      g4_dma16(arow[j] + kt * kBK, lds0 + (uint32_t)(st * ASTAGE + (wave * API + j) * 1024));
    else
      g4_dma16(bsrc[j - API] + kt * 32,
               lds0 + (uint32_t)(kG4Stages * ASTAGE + st * BSTAGE + (wave * BPI + j - API) * 1024));
  };
  af3_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  // fragments of k-step kt from its stage (A: two 16-byte chunks per row, B: one MXFP4 group)
  auto read_frags = [&](int kt, af3_i32x8 (&af)[TM], af3_i32x8 (&bfr)[TN], int (&sc)[TN]) {
    const int st = kt % kG4Stages;
    const uint8_t* as = As + st * ASTAGE;
    const uint8_t* bs = Bs + st * BSTAGE;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = wn0 + tn * 32 + lr;
      const af3_u32x4 b4 = (tn < tn_live) ? *(const af3_u32x4*)(bs + g4_b_off(n, lh)) : zero4();
      bfr[tn] = af3_i32x8{(int)b4[0], (int)b4[1], (int)b4[2], (int)b4[3], 0, 0, 0, 0};
      sc[tn] = (tn < tn_live) ? (int)Ss[n * G + 2 * kt + lh] : 127;
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      if (tm < tm_live) {
        const int row = wm0 + tm * 32 + lr;
        const af3_u32x4 lo = *(const af3_u32x4*)(as + row * 64 + (f8_chunk(row, lh) << 4));
        const af3_u32x4 hi = *(const af3_u32x4*)(as + row * 64 + (f8_chunk(row, 2 + lh) << 4));
        af[tm] = af3_i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2],
                           (int)hi[3]};
      } else {
        af[tm] = af3_i32x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };
  auto mfmas = [&](const af3_i32x8 (&af)[TM], const af3_i32x8 (&bfr)[TN], const int (&sc)[TN]) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        if (tm < tm_live && tn < tn_live)
          acc[tm][tn] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[tm], bfr[tn], acc[tm][tn], 0, 4, 0, 127, 0,
                                                                         sc[tn]);
  };
  // three stages in flight: k-steps 0, 1, 2; the fragments of a k-step are read
  // one k-step early (right after its stage is published) and its slot is
  // refilled (k-step + 3) as soon as they are read
#pragma unroll
  for (int j = 0; j < DPW; ++j) issue_one(0, j);
  if (nk > 1) {
#pragma unroll
    for (int j = 0; j < DPW; ++j) issue_one(1, j);
  }
  if (nk > 2) {
#pragma unroll
    for (int j = 0; j < DPW; ++j) issue_one(2, j);
  }
  // stage 0 in: every wave waits for its own copies of k-step 0 (<= two later k-steps outstanding)
  if (nk > 2)
    AF3_ASM_WAIT_VM(6);
  else if (nk > 1)
    AF3_ASM_WAIT_VM(3);
  else
    AF3_ASM_WAIT_VM(0);
  AF3_ASM_LDS_BARRIER();
  af3_i32x8 afA[TM], bfA[TN], afB[TM], bfB[TN];
  int scA[TN], scB[TN];
  read_frags(0, afA, bfA, scA);
  // k-step kt: fragments of kt in (af, bf); publish stage kt + 1, read its fragments
  // into the other buffer, refill slot kt % 3 with k-step kt + 3, then kt's MFMAs
  auto step = [&](int kt, af3_i32x8 (&af)[TM], af3_i32x8 (&bfr)[TN], int (&sc)[TN], af3_i32x8 (&afn)[TM],
                  af3_i32x8 (&bfn)[TN], int (&scn)[TN]) {
    if (kt + 1 < nk) {
      // copies outstanding after k-step kt + 1's: those of kt + 2 (if issued)
      if (kt + 2 < nk)
        AF3_ASM_WAIT_VM(3);
      else
        AF3_ASM_WAIT_VM(0);
      AF3_ASM_LDS_BARRIER();  // also: every wave has its k-step kt fragments (slot kt % 3 is free)
      read_frags(kt + 1, afn, bfn, scn);
      if (kt + 3 < nk) {
#pragma unroll
        for (int j = 0; j < DPW; ++j) issue_one(kt + 3, j);
      }
    }
    mfmas(af, bfr, sc);
  };
  int kt = 0;
#pragma nounroll
  for (; kt + 1 < nk; kt += 2) {
    step(kt, afA, bfA, scA, afB, bfB, scB);
    step(kt + 1, afB, bfB, scB, afA, bfA, scA);
  }
  if (kt < nk) step(kt, afA, bfA, scA, afB, bfB, scB);
  g4_epilogue<false, TM, TN, NT, CN, RM>(p, lds, acc, e, row_lo, nrows, n0, ncols, wm0, wn0);
}

template <int BXK>
__global__ __launch_bounds__(512) void gemm4_fwd_f8_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kG4LdsBytes];
  int mt, nt;
  if (!g4_work_item(p, mt, nt)) return;
  const int32_t ent = p.tile_map[mt];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * kG4Rows;
  const int nrows = min(kG4Rows, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = nt * kG4Rows;
  if (nrows <= 128 && (p.K >> 5) <= kG4NarrowMaxG) {
    if (nt & 1) return;
    g4f8_tile<true>(p, lds, e, row_lo, nrows, n0, min(512, p.N - n0));
    return;
  }
  g4f8_tile<false>(p, lds, e, row_lo, nrows, n0, min(kG4Rows, p.N - n0));
}

// ---------------------------------------------------------------------------
// gemm5 dgrad: the same products as gemm4 dgrad (weights packed along the
// output axis, W[e][k][n/32][16], scales [e][k][n/32]) with no transposing
// pass.  Each k-step stage holds, all copied global->LDS two k-steps ahead in
// a three-stage ring and published by one barrier per k-step:
//   A   [256 rows][64 k] bf16, 16-byte chunks XOR-swizzled by row (as gemm4);
//   B   the packed weight rows [64 k][128 B] (256 columns), 16-byte chunk c of
//       row k stored in slot c ^ (k & 7);
//   S   the e8m0 scales as zero-extended dwords [8 column blocks][64 k] (the
//       byte form of the LDS copy writes one dword per lane, which turns the
//       [k][block] bytes of HBM into block-major dwords on the way in).
// A lane's B fragment for one sub-step is one ds_read_b64_tr_b8 of the staged
// rows: within each 16-lane group, output lane j byte b comes from source lane
// 2b + j / 8, byte j % 8, so pointing source lanes 2b and 2b + 1 at row
// (k0 + b), 8-byte halves 0 and 1 of the group's 16 column pairs, hands lane
// j the byte of column pair (base + j) at the 8 rows k0 .. k0 + 7.  One
// v_cvt_scalef32_pk_bf16_fp4 per byte yields the (even, odd) column values
// (the cvt reads only the exponent field of its scale operand, so the scale
// dword shifted left by 23 is the operand); the even values feed one MFMA
// sub-tile and the odd values its partner, as in gemm4 dgrad.
// k inside a k-step is permuted as in gemm4 forward: lane (r, h) at sub-step
// s covers k = 32 h + 8 s + (0..7) (A chunk 4 h + s), so a lane's scales of a
// sub-step are 8 consecutive dwords of its block.
// Four waves (one per SIMD), wave w owns all 256 rows and columns 64 w ..
// 64 w + 63.  The last sub-step of each k-step is carried: its fragments are
// read before the barrier and its MFMAs run after it, covering the LDS reads
// and the B conversion of the next k-step's first sub-step.
// Scale bytes outside [2, 252] (never produced by normal quantisers) are
// detected per wave and k-step from the staged scales; such k-steps rebuild
// their B fragments with the integer rule after the fast conversion.
// ---------------------------------------------------------------------------
constexpr int kD5Stages = 3;
constexpr int kD5AOff = 0;
constexpr int kD5BOff = 256 * 64 * 2;           // 32 KB of A
constexpr int kD5SOff = kD5BOff + 64 * 128;     // + 8 KB of packed B
constexpr int kD5Stage = kD5SOff + 8 * 64 * 4;  // + 2 KB of scale dwords = 42 KB
constexpr int kD5LdsBytes = kD5Stages * kD5Stage > 256 * 512 + 2048 ? kD5Stages * kD5Stage : 256 * 512 + 2048;
static_assert(kD5LdsBytes <= 160 * 1024, "gemm5 dgrad LDS budget");
// HALF work items (128 rows x 256 columns, two blocks per CU): A 16 KB, packed
// B 8 KB and scales 2 KB per stage
constexpr int kD5HStage = 128 * 64 * 2 + 64 * 128 + 8 * 64 * 4;  // 26 KB
constexpr int kD5HLdsBytes = kD5Stages * kD5HStage;             // 78 KB
static_assert(kD5HLdsBytes >= 128 * 512 + 2048, "the HALF epilogue reuses the ring's LDS");
static_assert(2 * kD5HLdsBytes <= 160 * 1024, "two HALF blocks per CU");

typedef __attribute__((ext_vector_type(2))) int af3_i32x2;

// (even, odd) column fragments of one sub-step from the 8 packed bytes (w0:
// k 0..3, w1: k 4..7) and the 8 scale dwords of those k
__device__ __forceinline__ void d5_cvt(uint32_t w0, uint32_t w1, const uint32_t s[8], af3_bf16x8& ev,
                                       af3_bf16x8& od) {
  uint32_t dw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t src = i < 4 ? w0 : w1;
    const float sc = __uint_as_float(s[i] << 23);
    switch (i & 3) {
      case 0: dw[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, sc, 0)); break;
      case 1: dw[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, sc, 1)); break;
      case 2: dw[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, sc, 2)); break;
      default: dw[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, sc, 3)); break;
    }
  }
  af3_u32x4 e4, o4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    e4[j] = perm_lo(dw[2 * j], dw[2 * j + 1]);
    o4[j] = perm_hi(dw[2 * j], dw[2 * j + 1]);
  }
  ev = __builtin_bit_cast(af3_bf16x8, e4);
  od = __builtin_bit_cast(af3_bf16x8, o4);
}

// the same with the integer rule (exact for every scale byte)
__device__ __forceinline__ void d5_cvt_exact(uint32_t w0, uint32_t w1, const uint32_t s[8], af3_bf16x8& ev,
                                             af3_bf16x8& od) {
  uint32_t dw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t byte = ((i < 4 ? w0 : w1) >> (8 * (i & 3))) & 0xFFu;
    dw[i] = af3_e2m1_to_bf16_bits(byte & 0xFu, s[i]) | (af3_e2m1_to_bf16_bits(byte >> 4, s[i]) << 16);
  }
  af3_u32x4 e4, o4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    e4[j] = perm_lo(dw[2 * j], dw[2 * j + 1]);
    o4[j] = perm_hi(dw[2 * j], dw[2 * j + 1]);
  }
  ev = __builtin_bit_cast(af3_bf16x8, e4);
  od = __builtin_bit_cast(af3_bf16x8, o4);
}

// Epilogue of gemm5: the RM x CN tile of 4 waves (wave w owns columns
// CN / 4 * w .. + CN / 4, all RM rows; its MFMA sub-tile pairs hold the even /
// odd columns of 64 consecutive columns): v = (acc + bias[n]) * gamma[row] -> bf16, staged
// through LDS as [RM][CN] bf16 rows (16-byte chunks XOR-swizzled by row bit 2
// so the two row groups of an MFMA output store hit disjoint banks), then one
// 16-byte global store per chunk.
// acc[tm][tn] of a wave holds rows rb + 32 tm .. and the column pairs of
// sub-tile tn from column wn0 (TM row groups per wave)
template <int RM, int CN, int TM = RM / 32, int NBMAX = 16>
__device__ __forceinline__ void d5_epilogue(const Params& p, uint8_t* lds, af3_f32x16 (&acc)[TM][CN / 128],
                                            int e, int row_lo, int nrows, int n0, int ncols, int wn0, int rb = 0) {
  constexpr int TN = CN / 128, RB = CN * 2;
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  float* const gl = (float*)(lds + RM * RB);
  float* const al = gl + 256;  // per-row A scales
  auto coff = [&](int row, int col) { return row * RB + ((((col >> 3) ^ (((row >> 2) & 1) << 2))) << 4) + ((col & 7) << 1); };
  // SwiGLU backward (epi 1): the saved pre-activation of the lane's first NB
  // output chunks is loaded before the staging below and the rest as one more
  // batch, so a work item waits for NI / NB batches of loads instead of one
  // small group after another (chunks past the tile load from its first row
  // and column, valid addresses whose values are never used)
  constexpr int CH = CN / 8;              // 16-byte chunks per row
  constexpr int NI = RM * CH / 256;       // chunks per lane
  constexpr int NB = NI < NBMAX ? NI : NBMAX;  // chunks per prefetch batch
  const bool swb = p.epi == 1;
  af3_u32x4 gx[NB][2];
  auto gu_load = [&](int i, af3_u32x4 (&d)[2]) {
    const int id = i * 256 + threadIdx.x;
    const int row = id / CH, ch = id % CH;
    const bool ok = row < nrows && ch * 8 < ncols;
    const int64_t grow = row_lo + (ok ? row : 0);
    const int64_t col2 = 2 * (int64_t)(n0 + (ok ? ch * 8 : 0));
    const uint16_t* gu = (const uint16_t*)p.glu + grow * p.ld_glu + col2;
    d[0] = *(const af3_u32x4*)gu;
    d[1] = *(const af3_u32x4*)(gu + 8);
  };
  if (swb) {
#pragma unroll
    for (int j = 0; j < NB; ++j) gu_load(j, gx[j]);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < RM; t += 256) {
    float gv = 1.f;
    if (p.gammas && t < nrows) {
      const int64_t gr = row_lo + t;
      gv = p.gammas_f32 ? ((const float*)p.gammas)[gr] : af3_bf16_to_f32(((const uint16_t*)p.gammas)[gr]);
    }
    gl[t] = gv;
    al[t] = t < nrows ? g4_ascale(p, row_lo + t) : 1.f;
  }
  float bv[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int col = wn0 + 64 * (tn >> 1) + 2 * lr + (tn & 1);
    bv[tn] = (p.bias && col < ncols) ? p.bias[e * p.bias_estride + n0 + col] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row0 = rb + tm * 32 + j * 8 + lh * 4;
      const float4 g = *(const float4*)(gl + row0);
      const float gq[4] = {g.x, g.y, g.z, g.w};
      const float4 a = *(const float4*)(al + row0);
      const float aq[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int col = wn0 + 64 * (tn >> 1) + 2 * lr + (tn & 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x = acc[tm][tn][j * 4 + q];
          const float v = p.ascale ? (x * aq[q] + bv[tn]) * gq[q] : (x + bv[tn]) * gq[q];
          *(uint16_t*)(lds + coff(row0 + q, col)) = (uint16_t)af3_f32_to_bf16(v);
        }
      }
    }
  }
  __syncthreads();
  if (swb) {
    for (int b0 = 0; b0 < NI; b0 += NB) {
      if (b0 > 0) {
#pragma unroll
        for (int j = 0; j < NB; ++j) gu_load(b0 + j, gx[j]);
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int id = (b0 + j) * 256 + threadIdx.x;
        const int row = id / CH, ch = id % CH;
        if (row < nrows && ch * 8 < ncols) {  // dI (the bf16 values v) and the saved pre-activation -> dGU
          const af3_u32x4 v = *(const af3_u32x4*)(lds + row * RB + ((ch ^ (((row >> 2) & 1) << 2)) << 4));
          const int64_t grow = row_lo + row;
          const int64_t col2 = 2 * (int64_t)(n0 + ch * 8);
          const uint32_t xw[8] = {gx[j][0][0], gx[j][0][1], gx[j][0][2], gx[j][0][3],
                                  gx[j][1][0], gx[j][1][1], gx[j][1][2], gx[j][1][3]};
          uint32_t o[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const float d = af3_bf16_to_f32(q & 1 ? v[q >> 1] >> 16 : v[q >> 1] & 0xFFFFu);
            const float g = fminf(af3_bf16_to_f32(xw[q] & 0xFFFFu), p.limit);
            const float u = fminf(fmaxf(af3_bf16_to_f32(xw[q] >> 16), -p.limit), p.limit);
            float dg, du;
            af3_swiglu_bwd_elem(d, g, u, p.alpha, p.limit, dg, du);
            o[q] = af3_pack_bf16x2(dg, du);
          }
          af3_u32x4* dst = (af3_u32x4*)(p.c + grow * p.ldc + col2);
          dst[0] = af3_u32x4{o[0], o[1], o[2], o[3]};
          dst[1] = af3_u32x4{o[4], o[5], o[6], o[7]};
        }
      }
    }
    return;
  }
#pragma unroll 4
  for (int i = 0; i < NI; ++i) {
    const int id = i * 256 + threadIdx.x;
    const int row = id / CH, ch = id % CH;
    if (row < nrows && ch * 8 < ncols) {
      const af3_u32x4 v = *(const af3_u32x4*)(lds + row * RB + ((ch ^ (((row >> 2) & 1) << 2)) << 4));
      *(af3_u32x4*)(p.c + (row_lo + row) * p.ldc + n0 + ch * 8) = v;
    }
  }
}

// One work item of gemm5 dgrad.  NARROW = false: 256 rows x 256 columns, wave
// w owns all rows and columns 64 w .. 64 w + 63 (8 x 2 MFMA sub-tiles).
// NARROW = true (m-tiles of <= 128 rows): 128 rows x 512 columns (two n-tiles),
// wave w owns columns 128 w .. 128 w + 127 (4 x 4 sub-tiles, two pair groups),
// so a short expert tile still gives every wave 16 MFMAs per sub-step.  Both
// copy 12 instructions per wave per k-step (A / B / S = 8 / 2 / 2 or 4 / 4 / 4).
// SPLIT = 2 / 4 (256-row tiles with only 128 / 64 columns: the last n-tile
// when N % 256 is 128 / 64): SPLIT waves share a 64-column group, each taking
// 256 / SPLIT of the rows, so the tail tile's MFMAs are spread over all four
// SIMDs instead of running on one; copies, LDS layouts and the slot schedule
// are those of SPLIT = 1 (the A reads and MFMAs of the missing row groups
// drop out of their slots).
// RG > 0 (SPLIT = 1): only the first RG row groups of the tile hold rows (an
// expert's last, partial m-tile), so the waves run the MFMAs and A reads of
// those alone; the rows past them are never stored either way.
// SADDR: the copies address a scalar base plus 32-bit lane offsets (A: a_off32;
// the expert's packed weights and scales below 4 GiB), advancing only the base.
// TS (HALF): the scales are the af3_mxfp4_tile_dx_scales copy: a wave's two
// blocks x 64 rows of a k-step are 128 contiguous bytes, taken by one 2-byte
// copy per lane (rows 2 l, 2 l + 1 of block l / 32 in lane l's LDS dword)
// instead of two 1-byte copies that read 64 rows each.
template <bool NARROW, int BXK, int SPLIT = 1, int RG = 0, bool HALF = false, bool SADDR = false, bool TS = false>
__device__ __forceinline__ void d5_tile(const Params& p, uint8_t* lds, int e, int row_lo, int nrows, int n0, int ncols) {
  static_assert(!(NARROW && HALF), "one item shape");
  static_assert(!TS || HALF, "tiled input-gradient scales on the 128 x 256 items");
  static_assert(SPLIT == 1 || (!NARROW && !HALF && (SPLIT == 2 || SPLIT == 4)), "row split only for 256-row tiles");
  static_assert(RG == 0 || (SPLIT == 1 && RG >= 1 && RG <= ((NARROW || HALF) ? 4 : 8)), "row groups of a tile");
  constexpr int RM = (NARROW || HALF) ? 128 : 256;  // tile rows
  constexpr int CN = NARROW ? 512 : 256;  // tile columns
  constexpr int TM = RM / 32;             // row groups of the tile
  constexpr int TMW = RG ? RG : TM / SPLIT;  // row groups of one wave
  constexpr int PG = CN / 256;            // pair groups (64 columns each) per wave
  constexpr int TN = 2 * PG;
  constexpr int WC = CN / 4;              // columns per wave
  constexpr int BRB = CN / 2;             // packed bytes per weight row
  constexpr int NCH = BRB / 16;           // 16-byte chunks per weight row
  constexpr int NBLK = CN / 32;           // scale blocks
  constexpr int AI = RM / 32, BI = BRB / 64, SI = NBLK / 4;  // copies per wave per k-step
  constexpr int NCP = AI + BI + SI;
  static_assert(NCP == (HALF ? 8 : 12), "12 (HALF: 8) copies per wave per k-step");
  constexpr int AOFF = 0, BOFF = (NARROW || HALF) ? 16384 : 32768, SOFF = NARROW ? 32768 : HALF ? 24576 : 40960;
  constexpr int STAGE = HALF ? kD5HStage : kD5Stage;
  static_assert(SOFF + NBLK * 256 <= STAGE, "stage layout");
  // slot of chunk c in weight row k (keeps the transposing reads conflict-free)
  auto bswz = [](int k) { return NARROW ? ((k & 7) << 1) : (k & 7); };

  const int nk = p.K / kBK;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int wn0 = (wave / SPLIT) * WC;         // first column of the wave
  const int rb = (wave % SPLIT) * (RM / SPLIT);  // first row of the wave
  const int tm_live = min(TM, (nrows + 31) >> 5);
  const int pg_live = min(PG, max(0, (ncols - wn0) >> 6));  // ncols is a multiple of 64
  const bool wave_live = pg_live > 0;

  // ---- global -> LDS copy sources (SA: byte offsets from the scalar bases) ----
  const uint16_t* arow[AI];
  uint32_t aoff32[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int row = (wave * AI + i) * 8 + (lane >> 3);
    int64_t src = row_lo + (row < nrows ? row : 0);
    if (p.a.gather) src = p.a.gather[src] / p.a.gdiv;
    const int64_t el = src * p.a.ld + (((lane & 7) ^ swz(row)) << 3);
    arow[i] = (const uint16_t*)p.a.ptr + el;
    aoff32[i] = (uint32_t)(el * 2);
  }
  const uint8_t* bsrc[BI];  // 1 KB of weight rows per copy: 1024 / BRB rows, LDS slot lane % NCH
  uint32_t boff32[BI];
#pragma unroll
  for (int j = 0; j < BI; ++j) {
    const int kr = (wave * BI + j) * (1024 / BRB) + lane / NCH;
    int c = (lane % NCH) ^ bswz(kr);
    if (c * 32 >= ncols) c = 0;  // columns past the tile: any valid bytes (never read)
    const int64_t o = (int64_t)kr * p.b.ld + (n0 >> 1) + c * 16;
    bsrc[j] = (const uint8_t*)p.b.ptr + e * p.b.estride + o;
    boff32[j] = (uint32_t)o;
  }
  const uint8_t* ssrc[SI];  // block q = SI w + j, k row = lane
  uint32_t soff32[SI];
#pragma unroll
  for (int j = 0; j < SI; ++j) {
    int q = wave * SI + j;
    if (q * 32 >= ncols) q = 0;
    const int64_t o = (int64_t)lane * p.b.sld + (n0 >> 5) + q;
    ssrc[j] = p.b.scales + e * p.b.sestride + o;
    soff32[j] = (uint32_t)o;
  }
  const int64_t bstep = (int64_t)kBK * p.b.ld, sstep = (int64_t)kBK * p.b.sld;
  // TS: the wave's 128 bytes of k-step kc are at tsb + kc * tstep
  const uint8_t* const tsb = p.b.scales + ((int64_t)e * nk * p.s_nt + (n0 >> 8)) * 512 + wave * 128;
  const int64_t tstep = (int64_t)p.s_nt * 512;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  // copy j (0..11) of k-step kc: A, then B, then S (TS: one S copy, j = AI + BI)
  auto issue_one = [&](int kc, int j) {
    const uint32_t st = lds0 + (uint32_t)((kc % kD5Stages) * STAGE);
    if (j < AI) {
      const uint32_t dst = st + (uint32_t)(AOFF + (wave * AI + j) * 1024);
      if constexpr (SADDR)
        g4_dma16_s((const uint8_t*)p.a.ptr + (int64_t)kc * kBK * 2, aoff32[j], dst);
      else
        g4_dma16(arow[j] + kc * kBK, dst);
    } else if (j < AI + BI) {
      const uint32_t dst = st + (uint32_t)(BOFF + (wave * BI + j - AI) * 1024);
      if constexpr (SADDR)
        g4_dma16_s((const uint8_t*)p.b.ptr + e * p.b.estride + kc * bstep, boff32[j - AI], dst);
      else
        g4_dma16(bsrc[j - AI] + kc * bstep, dst);
    } else if constexpr (TS) {
      if (j == AI + BI)
        asm volatile("s_nop 0\n\tglobal_load_lds_ushort %0, %1" ::"v"((uint32_t)(lane * 2)), "s"(tsb + kc * tstep),
                     "{m0}"(st + (uint32_t)(SOFF + wave * 256)) : "memory");
    } else {
      const uint32_t dst = st + (uint32_t)(SOFF + (wave * SI + j - AI - BI) * 256);
      if constexpr (SADDR)
        asm volatile("s_nop 0\n\tglobal_load_lds_ubyte %0, %1" ::"v"(soff32[j - AI - BI]),
                     "s"(p.b.scales + e * p.b.sestride + kc * sstep), "{m0}"(dst) : "memory");
      else
        asm volatile("s_nop 0\n\tglobal_load_lds_ubyte %0, off" ::"v"(ssrc[j - AI - BI] + kc * sstep), "{m0}"(dst) : "memory");
    }
  };
  auto issue = [&](int kc) {
#pragma unroll
    for (int j = 0; j < NCP; ++j) issue_one(kc, j);
  };

  // ---- lane-fixed LDS byte offsets inside a stage ----
  const int ax = (lr ^ (lr >> 3)) & 7;
  // A fragment of the wave's row group tm at sub-step s: aoff[tm & 1][s] + 4096 tm
  // (the wave's first row group rb / 32 is even, so tm & 1 is the tile row group's parity)
  int aoff[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int s = 0; s < 4; ++s) aoff[t][s] = AOFF + rb * 128 + lr * 128 + ((((lh * 4 + s) ^ ax) ^ (t << 2)) << 4);
  // B transposed read of pair group pg: lane group g = lane / 16 (k half g / 2,
  // chunk (2 pg + g % 2) of the wave's columns), i = lane % 16
  const int gi = lane & 15, gg = lane >> 4;
  int boff[PG], soff[PG];
#pragma unroll
  for (int pg = 0; pg < PG; ++pg) {
    const int chunk = wn0 / 32 + 2 * pg + (gg & 1);
    const int kr = 32 * (gg >> 1) + (gi >> 1);
    boff[pg] = BOFF + kr * BRB + ((chunk ^ bswz(kr)) << 4) + (gi & 1) * 8;  // + 8 BRB s
    if constexpr (TS)  // the wave's dwords: block chunk - 2 wave, rows in pairs from 32 (gg / 2) + 8 s
      soff[pg] = SOFF + wave * 256 + (gg & 1) * 128 + (gg >> 1) * 64;       // + 16 s
    else
      soff[pg] = SOFF + (chunk * 64 + 32 * (gg >> 1)) * 4;                   // + 32 s
  }
  constexpr int CW = WC / 32;  // scale dwords per lane for the wave's check (its blocks x 64 k / 64 lanes)
  const int coff = TS ? SOFF + wave * 256 + lane * 4 : SOFF + (wn0 / 32 * 64 + CW * lane) * 4;

  af3_f32x16 acc[TMW][TN];
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // two blocks share each CU: while one runs its epilogue (VALU and memory
  // work), the other's k-loop keeps issue priority for its MFMAs and copies
  if constexpr (HALF) __builtin_amdgcn_s_setprio(2);
  issue(0);
  if (nk > 1) issue(1);

  // TS: the exact conversion is chosen per work item (the tiled scales carry a
  // flag per expert and n-tile: any scale byte outside [2, 252]), so the
  // k-loop of the usual items holds no range check and no exact path;
  // otherwise each k-step checks the wave's scale bytes (XC: run time)
  auto kloop = [&](auto full_c, auto exact_c) {
    constexpr bool FULL = decltype(full_c)::value;
    constexpr int XC = decltype(exact_c)::value;  // 0: never exact, 1: always, 2: per k-step check
    af3_bf16x8 af[2][TMW], bf[2][TN];
    // one k-step: iterations s = -1 (the carried sub-step of the previous
    // k-step, skipped at kt = 0) and 0..2; iteration s runs the MFMAs of
    // sub-step s while reading and converting the fragments of s + 1
    auto kstep = [&](int kt, bool first, bool pf) {
      const uint8_t* stg = lds + (kt % kD5Stages) * STAGE;
      const int nxt_copy = kt + 2;
      bool odd = false;
#pragma unroll
      for (int s = -1; s < 3; ++s) {
        const int c = s < 0 ? 1 : (s & 1);   // fragments of sub-step s
        const int nx = s < 0 ? 0 : (c ^ 1);  // fragments of sub-step s + 1
        const int o = s + 1;                 // sub-step whose operands are read
        uint32_t w[PG][2];
        uint32_t sc[PG][8];
        uint32_t chk[CW];
#pragma unroll
        for (int q = 0; q < CW; ++q) chk[q] = 2;
        uint32_t dw[PG][8];
        // 16 MFMAs of sub-step s, one LDS read or a slice of the B conversion
        // of sub-step s + 1 after each (a burst of reads would hold the wave at
        // issue while its MFMA pipe idles).  Slots (read order B, scales,
        // check, A; conversions once their operands have had time to land):
        //   PG 1: 0 B, 1-2 S, 3 check, 4-11 A, 6-13 convert, 14-15 fragments
        //   PG 2: 0-1 B, 2-5 S, 6 check, 7-10 A, 5-12 / 7-14 convert, 13 / 15
        // the copies of k-step kt + 2 after slots 2, 7, 12
        constexpr int SB = PG;             // first scale read slot
        constexpr int SC = SB + 2 * PG;    // check slot
        constexpr int SA = SC + 1;         // first A read slot
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // (HALF: the sub-step's 8 MFMAs in every other slot)
          const int mi = HALF ? (i >> 1) : i;
          const bool mslot = HALF ? ((i & 1) == 0 && mi < TMW * TN) : i < TMW * TN;
          const int tm = mi / TN, tn = mi % TN;
          if (mslot && !(s < 0 && first) && (FULL || (tm < tm_live && (tn >> 1) < pg_live)))
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[c][tm], bf[c][tn], acc[tm][tn], 0, 0, 0);
          if (FULL || wave_live) {
            if (i < SB) {
              const int pg = i;
              const af3_i32x2 wv = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                  (__attribute__((address_space(3))) af3_i32x2*)(stg + boff[pg] + 8 * BRB * o));
              w[pg][0] = (uint32_t)wv[0];
              w[pg][1] = (uint32_t)wv[1];
            } else if (i < SC) {
              const int pg = (i - SB) >> 1, h = (i - SB) & 1;
              if constexpr (TS) {  // 4 dwords = the 8 rows' bytes, two per dword
                if (h == 0) {
                  const af3_u32x4 sv = *(const af3_u32x4*)(stg + soff[pg] + 16 * o);
#pragma unroll
                  for (int q = 0; q < 4; ++q) {
                    sc[pg][2 * q] = sv[q] & 0xFFu;
                    sc[pg][2 * q + 1] = (sv[q] >> 8) & 0xFFu;
                  }
                }
              } else {
                const af3_u32x4 sv = *(const af3_u32x4*)(stg + soff[pg] + 32 * o + 16 * h);
#pragma unroll
                for (int q = 0; q < 4; ++q) sc[pg][4 * h + q] = sv[q];
              }
            } else if (i == SC) {
              if (s < 0 && XC == 2) {
                if constexpr (TS) {  // the lane's dword: two of the wave's scale bytes
                  const uint32_t cv = *(const uint32_t*)(stg + coff);
                  chk[0] = cv & 0xFFu;
                  chk[1] = (cv >> 8) & 0xFFu;
                } else if constexpr (CW == 2) {
                  const uint2 cv = *(const uint2*)(stg + coff);
                  chk[0] = cv.x;
                  chk[1] = cv.y;
                } else {
                  const af3_u32x4 cv = *(const af3_u32x4*)(stg + coff);
#pragma unroll
                  for (int q = 0; q < CW; ++q) chk[q] = cv[q];
                }
              }
            } else if (i < SA + TMW) {
              const int t = i - SA;
              if (FULL || t < tm_live) af[nx][t] = *(const af3_bf16x8*)(stg + aoff[t & 1][o] + 4096 * t);
            }
#pragma unroll
            for (int pg = 0; pg < PG; ++pg) {
              const int c0 = PG == 1 ? 6 : (pg ? 7 : 5);  // first conversion slot of this pair group
              if (i >= c0 && i < c0 + 8 && (FULL || pg < pg_live)) {
                const int q = i - c0;
                const uint32_t src = w[pg][q >> 2];
                const float scf = __uint_as_float(sc[pg][q] << 23);
                switch (q & 3) {
                  case 0: dw[pg][q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, scf, 0)); break;
                  case 1: dw[pg][q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, scf, 1)); break;
                  case 2: dw[pg][q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, scf, 2)); break;
                  default: dw[pg][q] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, scf, 3)); break;
                }
                asm volatile("" : "+v"(dw[pg][q]));  // keep the conversion in its slot
              }
              const int pe = PG == 1 ? 14 : (pg ? 15 : 13);  // even fragment slot (odd: next slot for PG 1)
              if ((i == pe) && (FULL || pg < pg_live)) {
                af3_u32x4 e4;
#pragma unroll
                for (int j = 0; j < 4; ++j) e4[j] = perm_lo(dw[pg][2 * j], dw[pg][2 * j + 1]);
                // materialise the fast conversion here, ahead of the rare exact
                // rebuild below (otherwise it is sunk past that branch)
                asm volatile("" : "+v"(e4));
                bf[nx][2 * pg] = __builtin_bit_cast(af3_bf16x8, e4);
              }
              if ((i == (PG == 1 ? 15 : pe)) && (FULL || pg < pg_live)) {
                af3_u32x4 o4;
#pragma unroll
                for (int j = 0; j < 4; ++j) o4[j] = perm_hi(dw[pg][2 * j], dw[pg][2 * j + 1]);
                asm volatile("" : "+v"(o4));
                bf[nx][2 * pg + 1] = __builtin_bit_cast(af3_bf16x8, o4);
              }
            }
          }
          if constexpr (HALF) {
            if (pf && (i == 3 || i == 10)) issue_one(nxt_copy, o * 2 + (i == 3 ? 0 : 1));
          } else {
            if (pf && (i == 2 || i == 7 || i == 12)) issue_one(nxt_copy, o * 3 + (i == 2 ? 0 : i == 7 ? 1 : 2));
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (FULL || wave_live) {
          if (XC == 2 && s < 0) {  // does this wave's part of k-step kt hold a scale byte outside [2, 252]?
            bool lane_odd = false;
#pragma unroll
            for (int q = 0; q < CW; ++q) lane_odd |= chk[q] - 2u > 250u;
            odd = __builtin_amdgcn_ballot_w64(lane_odd) != 0;
          }
          if (XC == 1 || (XC == 2 && odd)) {
#pragma unroll
            for (int pg = 0; pg < PG; ++pg)
              if (FULL || pg < pg_live) d5_cvt_exact(w[pg][0], w[pg][1], sc[pg], bf[nx][2 * pg], bf[nx][2 * pg + 1]);
          }
        }
      }
    };
    const af3_bf16x8 zf = __builtin_bit_cast(af3_bf16x8, zero4());
#pragma unroll
    for (int tm = 0; tm < TMW; ++tm) af[1][tm] = zf;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) bf[1][tn] = zf;
    // a k-step's stage is complete once this wave's copies for it have landed
    // (NCP newer ones outstanding (TS: 7), none for the last k-step)
    if constexpr (HALF && TS) {
      if (nk > 1)
        AF3_ASM_WAIT_VM(7);
      else
        AF3_ASM_WAIT_VM(0);
    } else if constexpr (HALF) {
      if (nk > 1)
        AF3_ASM_WAIT_VM(8);
      else
        AF3_ASM_WAIT_VM(0);
    } else {
      if (nk > 1)
        AF3_ASM_WAIT_VM(12);
      else
        AF3_ASM_WAIT_VM(0);
    }
    AF3_ASM_LDS_BARRIER();
    kstep(0, true, nk > 2);
#pragma nounroll
    for (int kt = 1; kt < nk; ++kt) {
      if constexpr (HALF && TS) {
        if (kt + 1 < nk)
          AF3_ASM_WAIT_VM(7);
        else
          AF3_ASM_WAIT_VM(0);
      } else if constexpr (HALF) {
        if (kt + 1 < nk)
          AF3_ASM_WAIT_VM(8);
        else
          AF3_ASM_WAIT_VM(0);
      } else {
        if (kt + 1 < nk)
          AF3_ASM_WAIT_VM(12);
        else
          AF3_ASM_WAIT_VM(0);
      }
      AF3_ASM_LDS_BARRIER();
      kstep(kt, false, kt + 2 < nk);
    }
    // the last k-step's sub-step 3
#pragma unroll
    for (int i = 0; i < TMW * TN; ++i) {
      const int tm = i / TN, tn = i % TN;
      if (FULL || (tm < tm_live && (tn >> 1) < pg_live))
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][tm], bf[1][tn], acc[tm][tn], 0, 0, 0);
    }
  };
  // every tile runs all of its MFMAs: rows and columns past the tile read
  // valid addresses and are never stored (the k-step is not MFMA-bound, and a
  // variant that skips dead sub-tiles needs more scalar registers than a wave
  // has)
  if constexpr (TS) {
    const int64_t flags = (int64_t)p.E * nk * p.s_nt * 512;  // the per-(expert, n-tile) flags after the bytes
    if (p.b.scales[flags + (int64_t)e * p.s_nt + (n0 >> 8)])
      kloop(std::true_type{}, std::integral_constant<int, 1>{});
    else
      kloop(std::true_type{}, std::integral_constant<int, 0>{});
  } else {
    kloop(std::true_type{}, std::integral_constant<int, 2>{});
  }

  if constexpr (BXK != NONE) {
    if (p.kx > 0) {  // expert-LoRA segment: + L[r] . Bx[e][:, n] (Bx [r][N], n contiguous)
      uint16_t* const As = (uint16_t*)lds;
      uint16_t* const Bs = As + RM * kBK;
      Loader<RM, ROWS_BF16, 256> la;
      Loader<CN, COLS_BF16, 256> lb;
      la.init(p.ax, 0, row_lo, nrows, p.kx);
      lb.init(p.bx, e, n0, ncols, 0, p.kx);
      for (int k0 = 0; k0 < p.kx; k0 += kBK) {
        la.load(k0);
        lb.load(k0);
        __syncthreads();
        la.store(As);
        lb.store(Bs);
        __syncthreads();
        const int nks = (min(kBK, p.kx - k0) + 15) / 16;  // sub-steps past the rank hold only zero padding
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
          if (ks >= nks) break;
          af3_bf16x8 af[TMW], bf[TN];
#pragma unroll
          for (int tm = 0; tm < TMW; ++tm) af[tm] = *(const af3_bf16x8*)(As + lds_off(rb + tm * 32 + lr, ks * 2 + lh));
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            bf[tn] = *(const af3_bf16x8*)(Bs + lds_off(wn0 + 64 * (tn >> 1) + 2 * lr + (tn & 1), ks * 2 + lh));
#pragma unroll
          for (int tm = 0; tm < TMW; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
              acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[tm], bf[tn], acc[tm][tn], 0, 0, 0);
        }
      }
    }
  }
  // (HALF: smaller batches of the SwiGLU-backward prefetch, within 256 registers)
  if constexpr (HALF) __builtin_amdgcn_s_setprio(0);  // the k-loop's waves first (see the k-loop's start)
  d5_epilogue<RM, CN, TMW, HALF ? 4 : 16>(p, lds, acc, e, row_lo, nrows, n0, ncols, wn0, rb);
}

template <int BXK>
__global__ __launch_bounds__(256) void gemm5_dgrad_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kD5LdsBytes];
  int mt, nt;
  if (!g4_work_item(p, mt, nt)) return;
  const int32_t ent = p.tile_map[mt];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * kG4Rows;
  const int nrows = min(kG4Rows, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = nt * kG4Rows;
  if (nrows <= 128) {
    // short tile: even n-tiles take the next n-tile too, odd ones have no work
    if (nt & 1) return;
    const int ncols = min(2 * kG4Rows, p.N - n0);
    if (nrows <= 64)
      d5_tile<true, BXK, 1, 2>(p, lds, e, row_lo, nrows, n0, ncols);
    else
      d5_tile<true, BXK>(p, lds, e, row_lo, nrows, n0, ncols);
  } else {
    // N % 64 == 0: the last n-tile of N % 256 == 64 / 128 splits its columns' rows over the waves
    const int ncols = min(kG4Rows, p.N - n0);
    if (ncols <= 64)
      d5_tile<false, BXK, 4>(p, lds, e, row_lo, nrows, n0, ncols);
    else if (ncols <= 128)
      d5_tile<false, BXK, 2>(p, lds, e, row_lo, nrows, n0, ncols);
    else if (nrows <= 160)  // a partial m-tile: only its live row groups
      d5_tile<false, BXK, 1, 5>(p, lds, e, row_lo, nrows, n0, ncols);
    else if (nrows <= 192)
      d5_tile<false, BXK, 1, 6>(p, lds, e, row_lo, nrows, n0, ncols);
    else if (nrows <= 224)
      d5_tile<false, BXK, 1, 7>(p, lds, e, row_lo, nrows, n0, ncols);
    else
      d5_tile<false, BXK, 1>(p, lds, e, row_lo, nrows, n0, ncols);
  }
}

// Input gradient on HALF work items: 128 x 256 tiles of the 128-row map, four
// waves of 128 x 64 (each weight byte converted once per 128 rows), two blocks
// per CU, so one block's epilogue (the fused SwiGLU backward's VALU work in
// the down projection) overlaps the other block's k-loop.
template <int BXK, bool SA, bool TS>
__global__ __launch_bounds__(256, 2) void gemm8_dgrad_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kD5HLdsBytes];
  int mt, nt;
  if (!g4_work_item(p, mt, nt)) return;
  const int32_t ent = p.tile_map[mt];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * 128;
  const int nrows = min(128, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = nt * 256;
  const int ncols = min(256, p.N - n0);
  if (nrows <= 32)
    d5_tile<false, BXK, 1, 1, true, SA, TS>(p, lds, e, row_lo, nrows, n0, ncols);
  else if (nrows <= 64)
    d5_tile<false, BXK, 1, 2, true, SA, TS>(p, lds, e, row_lo, nrows, n0, ncols);
  else if (nrows <= 96)
    d5_tile<false, BXK, 1, 3, true, SA, TS>(p, lds, e, row_lo, nrows, n0, ncols);
  else
    d5_tile<false, BXK, 1, 0, true, SA, TS>(p, lds, e, row_lo, nrows, n0, ncols);
}

// ---------------------------------------------------------------------------
// fp8-mode input gradient (the reference's fp8 backward, quantization.py:382-408:
// per-token E4M3 gradient x the weights' E5M2 form): A = E4M3 codes [rows][K]
// bytes, B = the packed MXFP4 weights of gemm5 (W[e][k][n/32][16], scales
// [e][k][n/32]), converted to E5M2 in registers, on the block-scaled MFMA
// v_mfma_scale_f32_32x32x64_f8f6f4 (A format E4M3, B format E5M2, block scales
// 2^0); the per-token scale multiplies the fp32 accumulator in gemm5's epilogue.
// Work items, wave layout (wave w: all rows x columns 64 w .. 64 w + 63, or the
// NARROW 128 x 512 item with 128 columns per wave) and the epilogue are gemm5's.
// The k permutation is the MFMA's own: lane (r, h) holds k 16 h .. 16 h + 15 in
// bytes 0-15 and 32 + 16 h .. in bytes 16-31 of its 32-byte operand.
//   A   [RM rows][64 k] codes, 16-byte chunk c of row r in slot c ^ ((r >> 2) & 3)
//       (the fp8 forward's layout); a lane's operand is two 16-byte reads.
//   B   gemm5's packed rows; four ds_read_b64_tr_b8 per pair group (rows 16 h +
//       {0, 8, 32, 40} .. + 7) give a lane the bytes of its column pair at the 32
//       k of its operand; per byte (one k row) v_cvt_scalef32_pk_f32_fp4 with the
//       row's scale yields the (even, odd) column values and v_cvt_pk_bf8_f32
//       packs four rows of each into E5M2 bytes.  That is exact and equal to the
//       reference's integer rule for scale bytes 114 .. 140 (every value an E5M2
//       normal); a wave's k-step holding another scale byte rebuilds its
//       fragments with the integer rule (af3_e2m1_to_e5m2_byte).
//   S   the scales as zero-extended dwords [blocks][64 k] (gemm5's copy).
// Four-stage ring, copies issued three k-steps ahead; the barrier at k-step kt
// publishes stage kt + 1, whose B fragments are read and converted during the
// MFMAs of k-step kt (double-buffered B), and the A operands are read one row
// group ahead of their MFMAs.
// ---------------------------------------------------------------------------
constexpr int kD8Stages = 4;
constexpr int kD8Stage = 28 * 1024;  // A 16 + B 8 + S 2 KB, NARROW A 8 + B 16 + S 4 KB
static_assert(kD8Stages * kD8Stage <= kD5LdsBytes, "fp8 dgrad ring inside gemm5's LDS area");

typedef __attribute__((ext_vector_type(2))) float af3_f32x2;

// E5M2 bytes of the 8 packed bytes (w0: k rows 0..3, w1: rows 4..7) of one
// transposing read: even columns -> e[0..1], odd -> o[0..1]; s[q] = scale dword of row q
template <bool EXACT>
__device__ __forceinline__ void d8_cvt(uint32_t w0, uint32_t w1, const uint32_t s[8], uint32_t e[2], uint32_t o[2]) {
  if constexpr (EXACT) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t ev = 0, od = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t byte = ((h ? w1 : w0) >> (8 * q)) & 0xFFu;
        ev |= af3_e2m1_to_e5m2_byte(byte & 0xFu, s[4 * h + q]) << (8 * q);
        od |= af3_e2m1_to_e5m2_byte(byte >> 4, s[4 * h + q]) << (8 * q);
      }
      e[h] = ev;
      o[h] = od;
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t src = h ? w1 : w0;
      af3_f32x2 r[4];
      r[0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(src, __uint_as_float(s[4 * h + 0] << 23), 0);
      r[1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(src, __uint_as_float(s[4 * h + 1] << 23), 1);
      r[2] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(src, __uint_as_float(s[4 * h + 2] << 23), 2);
      r[3] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(src, __uint_as_float(s[4 * h + 3] << 23), 3);
      int ev = __builtin_amdgcn_cvt_pk_bf8_f32(r[0][0], r[1][0], 0, false);
      ev = __builtin_amdgcn_cvt_pk_bf8_f32(r[2][0], r[3][0], ev, true);
      int od = __builtin_amdgcn_cvt_pk_bf8_f32(r[0][1], r[1][1], 0, false);
      od = __builtin_amdgcn_cvt_pk_bf8_f32(r[2][1], r[3][1], od, true);
      e[h] = (uint32_t)ev;
      o[h] = (uint32_t)od;
    }
  }
}

template <bool NARROW>
__device__ __forceinline__ void d8_tile(const Params& p, uint8_t* lds, int e, int row_lo, int nrows, int n0, int ncols) {
  constexpr int RM = NARROW ? 128 : 256;  // tile rows
  constexpr int CN = NARROW ? 512 : 256;  // tile columns
  constexpr int TM = RM / 32;
  constexpr int WC = CN / 4;              // columns per wave
  constexpr int PG = WC / 64;             // pair groups (64 columns each) per wave
  constexpr int TN = 2 * PG;
  constexpr int BRB = CN / 2;             // packed bytes per weight row
  constexpr int NCH = BRB / 16;           // 16-byte chunks per weight row
  constexpr int NBLK = CN / 32;           // scale blocks
  constexpr int AI = RM / 64, BI = BRB / 64, SI = NBLK / 4;  // copies per wave per k-step
  constexpr int DPW = AI + BI + SI;
  static_assert(DPW == 8 || DPW == 10, "copy schedule");
  constexpr int AOFF = 0, BOFF = RM * 64, SOFF = BOFF + 64 * BRB;
  static_assert(SOFF + NBLK * 256 <= kD8Stage, "stage layout");
  auto bswz = [](int k) { return NARROW ? ((k & 7) << 1) : (k & 7); };

  const int nk = p.K / kBK;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int wn0 = wave * WC;

  // ---- global -> LDS copy sources ----
  const uint8_t* arow[AI];  // 16 rows of 64 codes per copy
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int row = (wave * AI + i) * 16 + (lane >> 2);
    int64_t src = row_lo + (row < nrows ? row : 0);
    if (p.a.gather) src = p.a.gather[src] / p.a.gdiv;
    arow[i] = (const uint8_t*)p.a.ptr + src * p.a.ld + (f8_chunk(row, lane & 3) << 4);
  }
  const uint8_t* bsrc[BI];
#pragma unroll
  for (int j = 0; j < BI; ++j) {
    const int kr = (wave * BI + j) * (1024 / BRB) + lane / NCH;
    int c = (lane % NCH) ^ bswz(kr);
    if (c * 32 >= ncols) c = 0;  // columns past the tile: any valid bytes (never stored)
    bsrc[j] = (const uint8_t*)p.b.ptr + e * p.b.estride + (int64_t)kr * p.b.ld + (n0 >> 1) + c * 16;
  }
  const uint8_t* ssrc[SI];
#pragma unroll
  for (int j = 0; j < SI; ++j) {
    int q = wave * SI + j;
    if (q * 32 >= ncols) q = 0;
    ssrc[j] = p.b.scales + e * p.b.sestride + (int64_t)lane * p.b.sld + (n0 >> 5) + q;
  }
  const int64_t bstep = (int64_t)kBK * p.b.ld, sstep = (int64_t)kBK * p.b.sld;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  auto issue_one = [&](int kc, int j) {
    const uint32_t st = lds0 + (uint32_t)((kc % kD8Stages) * kD8Stage);
    if (j < AI) {
      g4_dma16(arow[j] + kc * kBK, st + (uint32_t)(AOFF + (wave * AI + j) * 1024));
    } else if (j < AI + BI) {
      g4_dma16(bsrc[j - AI] + kc * bstep, st + (uint32_t)(BOFF + (wave * BI + j - AI) * 1024));
    } else {
      asm volatile("s_nop 0\n\tglobal_load_lds_ubyte %0, off" ::"v"(ssrc[j - AI - BI] + kc * sstep), "{m0}"(st + (uint32_t)(SOFF + (wave * SI + j - AI - BI) * 256)) : "memory");
    }
  };

  // ---- lane-fixed LDS byte offsets inside a stage ----
  const int ach = (lr >> 2) & 3;
  const int aoff_lo = AOFF + lr * 64 + ((lh ^ ach) << 4), aoff_hi = AOFF + lr * 64 + (((2 + lh) ^ ach) << 4);
  const int gi = lane & 15, gg = lane >> 4;
  int boff[PG], soff[PG];
#pragma unroll
  for (int pg = 0; pg < PG; ++pg) {
    const int chunk = wn0 / 32 + 2 * pg + (gg & 1);
    const int kr = 16 * (gg >> 1) + (gi >> 1);
    boff[pg] = BOFF + kr * BRB + ((chunk ^ bswz(kr)) << 4) + (gi & 1) * 8;  // + BRB (8 (i & 1) + 32 (i >> 1))
    soff[pg] = SOFF + (chunk * 64 + 16 * (gg >> 1)) * 4;                   // + 4 (8 (i & 1) + 32 (i >> 1))
  }
  constexpr int CW = WC / 32;  // scale dwords per lane for the wave's range check
  const int coff = SOFF + (wn0 / 32 * 64 + CW * lane) * 4;

  af3_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // B operands of the stage at stg: tr reads, scales, range check, conversion
  auto load_b = [&](const uint8_t* stg, af3_i32x8 (&bf)[TN]) {
    uint32_t chk[CW];
    if constexpr (CW == 2) {
      const uint2 cv = *(const uint2*)(stg + coff);
      chk[0] = cv.x;
      chk[1] = cv.y;
    } else {
      const af3_u32x4 cv = *(const af3_u32x4*)(stg + coff);
#pragma unroll
      for (int q = 0; q < CW; ++q) chk[q] = cv[q];
    }
    bool lane_odd = false;
#pragma unroll
    for (int q = 0; q < CW; ++q) lane_odd |= chk[q] - 114u > 26u;
    const bool odd = __builtin_amdgcn_ballot_w64(lane_odd) != 0;
#pragma unroll
    for (int pg = 0; pg < PG; ++pg) {
      uint32_t ev[8], od[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int radd = 8 * (i & 1) + 32 * (i >> 1);
        const af3_i32x2 wv = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) af3_i32x2*)(stg + boff[pg] + BRB * radd));
        const af3_u32x4 s0 = *(const af3_u32x4*)(stg + soff[pg] + 4 * radd);
        const af3_u32x4 s1 = *(const af3_u32x4*)(stg + soff[pg] + 4 * radd + 16);
        const uint32_t sc[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        if (odd)
          d8_cvt<true>((uint32_t)wv[0], (uint32_t)wv[1], sc, ev + 2 * i, od + 2 * i);
        else
          d8_cvt<false>((uint32_t)wv[0], (uint32_t)wv[1], sc, ev + 2 * i, od + 2 * i);
      }
      bf[2 * pg] = af3_i32x8{(int)ev[0], (int)ev[1], (int)ev[2], (int)ev[3], (int)ev[4], (int)ev[5], (int)ev[6],
                             (int)ev[7]};
      bf[2 * pg + 1] = af3_i32x8{(int)od[0], (int)od[1], (int)od[2], (int)od[3], (int)od[4], (int)od[5], (int)od[6],
                                 (int)od[7]};
    }
  };
  auto load_a = [&](const uint8_t* stg, int tm) {
    const af3_u32x4 lo = *(const af3_u32x4*)(stg + aoff_lo + tm * 2048);
    const af3_u32x4 hi = *(const af3_u32x4*)(stg + aoff_hi + tm * 2048);
    return af3_i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };

  // prologue: stages 0..2 in flight, stage 0 published, its B operands converted
#pragma unroll
  for (int kc = 0; kc < 3; ++kc)
    if (kc < nk) {
#pragma unroll
      for (int j = 0; j < DPW; ++j) issue_one(kc, j);
    }
  if (nk > 2) {
    if constexpr (DPW == 8) AF3_ASM_WAIT_VM(16); else AF3_ASM_WAIT_VM(20);
  } else if (nk > 1) {
    if constexpr (DPW == 8) AF3_ASM_WAIT_VM(8); else AF3_ASM_WAIT_VM(10);
  } else {
    AF3_ASM_WAIT_VM(0);
  }
  AF3_ASM_LDS_BARRIER();
  af3_i32x8 bfA[TN], bfB[TN];
  load_b(lds, bfA);
  // k-step kt: publish stage kt + 1 (its copies in, those of kt + 2 still in flight),
  // issue k-step kt + 3 into the slot of kt - 1, then the MFMAs of kt with the A
  // operands read one row group ahead, while stage kt + 1's B operands are converted
  auto kstep = [&](int kt, af3_i32x8 (&bcur)[TN], af3_i32x8 (&bnxt)[TN]) {
    if (kt + 2 < nk) {
      if constexpr (DPW == 8) AF3_ASM_WAIT_VM(8); else AF3_ASM_WAIT_VM(10);
    } else {
      AF3_ASM_WAIT_VM(0);
    }
    AF3_ASM_LDS_BARRIER();
    if (kt + 3 < nk) {
#pragma unroll
      for (int j = 0; j < DPW; ++j) issue_one(kt + 3, j);
    }
    const uint8_t* stg = lds + (kt % kD8Stages) * kD8Stage;
    af3_i32x8 a0 = load_a(stg, 0), a1;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      if (tm + 1 < TM) a1 = load_a(stg, tm + 1);
      if (tm == TM / 2 && kt + 1 < nk) load_b(lds + ((kt + 1) % kD8Stages) * kD8Stage, bnxt);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        acc[tm][tn] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a0, bcur[tn], acc[tm][tn], 0, 1, 0, 127, 0,
                                                                       127);
      a0 = a1;
    }
  };
  int kt = 0;
#pragma nounroll
  for (; kt + 1 < nk; kt += 2) {
    kstep(kt, bfA, bfB);
    kstep(kt + 1, bfB, bfA);
  }
  if (kt < nk) kstep(kt, bfA, bfB);
  d5_epilogue<RM, CN>(p, lds, acc, e, row_lo, nrows, n0, ncols, wn0);
}

__global__ __launch_bounds__(256) void gemm5_f8_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kD5LdsBytes];
  int mt, nt;
  if (!g4_work_item(p, mt, nt)) return;
  const int32_t ent = p.tile_map[mt];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * kG4Rows;
  const int nrows = min(kG4Rows, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = nt * kG4Rows;
  if (nrows <= 128) {
    if (nt & 1) return;
    d8_tile<true>(p, lds, e, row_lo, nrows, n0, min(2 * kG4Rows, p.N - n0));
  } else {
    d8_tile<false>(p, lds, e, row_lo, nrows, n0, min(kG4Rows, p.N - n0));
  }
}

// ---------------------------------------------------------------------------
// row-tile kernel: main GEMMs and the skinny LoRA row products
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN, int AK, int BK_, int AXK, int BXK>
__global__ __launch_bounds__(kThreads) void rowtile_kernel(Params p) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * kBK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * kBK];

  const int32_t ent = p.tile_map[blockIdx.x];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int row_lo = p.offs[e] + blk * BM;
  const int nrows = min(BM, p.offs[e + 1] - row_lo);
  if (nrows <= 0) return;
  const int n0 = blockIdx.y * BN;
  const int ncols = min(BN, p.N - n0);

  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave / WN) * (BM / WM), wn0 = (wave % WN) * (BN / WN);
  af3_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  {
    Loader<BM, AK> la;
    Loader<BN, BK_> lb;
    la.init(p.a, 0, row_lo, nrows, p.K);
    if constexpr (BK_ == ROWS_BF16 || BK_ == ROWS_FP4)
      lb.init(p.b, e, n0, ncols, p.K);
    else
      lb.init(p.b, e, n0, ncols, 0, p.K);
    run_segment<Loader<BM, AK>, Loader<BN, BK_>, TM, TN>(la, lb, p.K, As, Bs, wm0, wn0, acc);
  }
  if constexpr (AXK != NONE) {
    if (p.kx > 0) {
      Loader<BM, AXK> la;
      Loader<BN, BXK> lb;
      la.init(p.ax, 0, row_lo, nrows, p.kx);
      if constexpr (BXK == ROWS_BF16)
        lb.init(p.bx, e, n0, ncols, p.kx);
      else
        lb.init(p.bx, e, n0, ncols, 0, p.kx);
      run_segment<Loader<BM, AXK>, Loader<BN, BXK>, TM, TN>(la, lb, p.kx, As, Bs, wm0, wn0, acc);
    }
  }

  // epilogue: (acc + bias) * gamma * scale -> bf16
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int col = wn0 + tn * 32 + (lane & 31);
      if (col >= ncols) continue;
      const int n = n0 + col;
      const float bv = p.bias ? p.bias[e * p.bias_estride + n] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm0 + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (row >= nrows) continue;
        const int64_t gr = row_lo + row;
        float v = acc[tm][tn][r] + bv;
        if (p.gammas)
          v *= p.gammas_f32 ? ((const float*)p.gammas)[gr] : af3_bf16_to_f32(((const uint16_t*)p.gammas)[gr]);
        v *= p.scale;
        p.c[gr * p.ldc + n] = (uint16_t)af3_f32_to_bf16(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// weight-gradient kernels: G[e][m][n] = scale * sum_{r in rows(e)} A[r][m] B[r][n]
// Pass 1: blockIdx.x -> chunk (expert e, chunk_rows-row block b) of the
// expert-sorted rows (the chunk map has the block_pid_map format),
// blockIdx.y -> (m block, n block); writes the fp32 partial of its rows.
// Pass 2: per expert, sums its chunks' partials in chunk order (deterministic).
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(kThreads) void wgrad_partial_kernel(Params p) {
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * kBK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * kBK];

  const int32_t ent = p.tile_map[blockIdx.x];
  if (ent < 0) return;
  const int e = ent & 0xFFFF, blk = ent >> 16;
  const int kb = p.offs[e] + blk * p.chunk_rows;
  const int kend = min(p.chunk_rows, p.offs[e + 1] - kb);
  if (kend <= 0) return;
  const int m0 = (blockIdx.y / p.n_nblk) * BM, n0 = (blockIdx.y % p.n_nblk) * BN;
  const int mcols = min(BM, p.M - m0), ncols = min(BN, p.N - n0);

  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave / WN) * (BM / WM), wn0 = (wave % WN) * (BN / WN);
  af3_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  Loader<BM, COLS_BF16> la;
  Loader<BN, COLS_BF16> lb;
  la.init(p.a, 0, m0, mcols, kb, kend);
  lb.init(p.b, 0, n0, ncols, kb, kend);
  run_segment<Loader<BM, COLS_BF16>, Loader<BN, COLS_BF16>, TM, TN>(la, lb, kend, As, Bs, wm0, wn0, acc);

  const int lane = threadIdx.x & 63;
  float* out = p.partials + (int64_t)blockIdx.x * p.M * p.N;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int col = wn0 + tn * 32 + (lane & 31);
      if (col >= ncols) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm0 + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (row >= mcols) continue;
        out[(int64_t)(m0 + row) * p.N + n0 + col] = acc[tm][tn][r];
      }
    }
  }
}

// one thread per 4 output elements of one expert
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* __restrict__ partials,
                                                           const int32_t* __restrict__ chunk_offs, int64_t MN,
                                                           float scale, uint16_t* __restrict__ g) {
  const int e = blockIdx.y;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= MN) return;
  const int c0 = chunk_offs[e], c1 = chunk_offs[e + 1];
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  for (int c = c0; c < c1; ++c) {
    const float4 v = *(const float4*)(partials + (int64_t)c * MN + i);
    a0 += v.x;
    a1 += v.y;
    a2 += v.z;
    a3 += v.w;
  }
  uint2 o;
  o.x = af3_pack_bf16x2(a0 * scale, a1 * scale);
  o.y = af3_pack_bf16x2(a2 * scale, a3 * scale);
  *(uint2*)(g + (int64_t)e * MN + i) = o;
}

// ---------------------------------------------------------------------------
// combine: out[t] = sum_j rows[src[t*K + j]] (fp32 sum, bf16 out), -1 skipped
// ---------------------------------------------------------------------------
// KU > 0: K <= KU, the K row indices and then the K rows loaded before any
// sum (KU rows in flight per lane); KU = 0: any K, one row at a time.  The
// fp32 sum runs over j = 0 .. K - 1 in order either way.
template <int KU>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ rows, int64_t ld_rows,
                                                      const int32_t* __restrict__ src, int K, int N,
                                                      uint16_t* __restrict__ out, int64_t ld_out, int vec_per_row,
                                                      int64_t n_vec) {
  int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= n_vec) return;
  int64_t t = v / vec_per_row;
  int c = (int)(v - t * vec_per_row) * 8;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add = [&](const af3_u32x4 x) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += af3_bf16_to_f32(x[q] & 0xFFFFu);
      acc[2 * q + 1] += af3_bf16_to_f32(x[q] >> 16);
    }
  };
  if constexpr (KU > 0) {
    int32_t r[KU];
#pragma unroll
    for (int j = 0; j < KU; ++j) r[j] = j < K ? src[t * K + j] : -1;
    af3_u32x4 x[KU];
#pragma unroll
    for (int j = 0; j < KU; ++j)
      x[j] = r[j] >= 0 ? __builtin_nontemporal_load((const af3_u32x4*)(rows + (int64_t)r[j] * ld_rows + c)) : zero4();
#pragma unroll
    for (int j = 0; j < KU; ++j)
      if (r[j] >= 0) add(x[j]);
  } else {
    for (int j = 0; j < K; ++j) {
      int32_t r = src[t * K + j];
      if (r < 0) continue;
      add(*(const af3_u32x4*)(rows + (int64_t)r * ld_rows + c));
    }
  }
  af3_u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = af3_pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  __builtin_nontemporal_store(o, (af3_u32x4*)(out + t * ld_out + c));
}

Operand make_bf16(const uint16_t* ptr, int64_t ld, int64_t estride, const int32_t* gather, int gdiv,
                  const uint16_t* rowscale = nullptr) {
  Operand o{};
  o.ptr = ptr;
  o.ld = ld;
  o.estride = estride;
  o.gather = gather;
  o.gdiv = gdiv > 0 ? gdiv : 1;
  o.rowscale = rowscale;
  return o;
}

inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// ---------------------------------------------------------------------------
// exported entry points
// ---------------------------------------------------------------------------

static void launch_gemm8_dgrad(int max_tiles, int N, hipStream_t stream, Params p) {
  p.n_nblk = (N + 255) / 256;
  dim3 grid(g4_grid(max_tiles, p.n_nblk, p.group_m));
  // scalar-base addressing where the caller vouches for 32-bit A offsets and
  // an expert's packed weights (K x N / 2 bytes) are below 4 GiB
  const bool sa = p.a_off32 && (int64_t)p.K * (N / 2) < (1LL << 32);
  if (sa && p.s_tiled)
    hipLaunchKernelGGL((gemm8_dgrad_kernel<COLS_BF16, true, true>), grid, dim3(256), 0, stream, p);
  else if (sa)
    hipLaunchKernelGGL((gemm8_dgrad_kernel<COLS_BF16, true, false>), grid, dim3(256), 0, stream, p);
  else if (p.s_tiled)
    hipLaunchKernelGGL((gemm8_dgrad_kernel<COLS_BF16, false, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((gemm8_dgrad_kernel<COLS_BF16, false, false>), grid, dim3(256), 0, stream, p);
}

static void launch_gemm5_dgrad(int max_tiles, int N, hipStream_t stream, Params p) {
  p.n_nblk = (N + kG4Rows - 1) / kG4Rows;
  dim3 grid(g4_grid(max_tiles, p.n_nblk, p.group_m));
  hipLaunchKernelGGL((gemm5_dgrad_kernel<COLS_BF16>), grid, dim3(256), 0, stream, p);
}

template <int WM, int WN>
static void launch_gemm4_fwd(int max_tiles, int N, hipStream_t stream, Params p) {
  p.n_nblk = (N + kG4Rows - 1) / kG4Rows;
  dim3 grid(g4_grid(max_tiles, p.n_nblk, p.group_m));
  hipLaunchKernelGGL((gemm4_fwd_kernel<WM, WN, ROWS_BF16>), grid, dim3(WM * WN * 64), 0, stream, p);
}

static void launch_gemm7_fwd(int max_tiles, int N, hipStream_t stream, Params p) {
  p.n_nblk = (N + 255) / 256;
  dim3 grid(g4_grid(max_tiles, p.n_nblk, p.group_m));
  // weight words two k-steps ahead where the k-steps come in whole triples
  // and every n-tile's columns come in whole 64-column wave slices; scalar-base
  // addressing where the caller vouches for 32-bit A offsets and an expert's
  // packed weights are below 4 GiB
  const bool sa = p.a_off32 && (int64_t)N * (p.K / 2) < (1LL << 32);
  if ((p.K / kBK) % 3 == 0 && N % 64 == 0) {
    if (sa)
      hipLaunchKernelGGL((gemm7_fwd_kernel<ROWS_BF16, 3, true>), grid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((gemm7_fwd_kernel<ROWS_BF16, 3, false>), grid, dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL((gemm7_fwd_kernel<ROWS_BF16, 2, false>), grid, dim3(256), 0, stream, p);
  }
}

template <int BM, int BN, int WM, int WN>
static void launch_gemm2(bool trans, int max_tiles, int N, hipStream_t stream, Params p) {
  p.n_nblk = (N + BN - 1) / BN;
  dim3 grid(max_tiles * p.n_nblk);
  if (!trans)
    hipLaunchKernelGGL((gemm2_kernel<BM, BN, WM, WN, ROWS_FP4, ROWS_BF16>), grid, dim3(WM * WN * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((gemm2_kernel<BM, BN, WM, WN, COLS_FP4, COLS_BF16>), grid, dim3(WM * WN * 64), 0, stream, p);
}

// Grouped GEMM through frozen MXFP4 expert weights (A6/A8/A9/A11).
//   trans_w = 0: Y[r][n] = sum_k X[a(r)][k] W[e][n][k]   W blocks [E][N][K/32][16]
//   trans_w = 1: Y[r][n] = sum_k X[a(r)][k] W[e][k][n]   W blocks [E][K][N/32][16]
//   optional extension (expert LoRA):  + sum_j L[r][j] Bx[e][n][j] (trans 0) or Bx[e][j][n] (trans 1)
//   then v = (acc + bias[e][n]) * gammas[r] -> bf16 Y[r][n]
// a(r) = gather ? gather[r] / gather_div : r.  Rows r are expert-sorted; expert
// e owns rows [token_offs[e], token_offs[e+1]); block_pid_map is the map of
// af3_expt_data for BM = block_m; grid.x = max_tiles.  tile_cfg selects the
// block tile (0 = default for block_m; see the table below).
static int moe_gemm_impl(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                         const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                         const void* gammas, int gammas_f32, const uint16_t* lora_l, int64_t ld_l,
                         const uint16_t* lora_b, int lora_r, const int32_t* token_offs, const int32_t* block_pid_map,
                         const int32_t* tile_offs, int max_tiles, int block_m, int tile_cfg, int n_expts, int N,
                         int K, uint16_t* y, int64_t ldy, int epi, void* glu, int64_t ld_glu, float alpha,
                         float limit, const float* a_row_scale, void* stream_, int a_fp8 = 0) {
  hipStream_t stream = (hipStream_t)stream_;
  const bool w_tiled = (tile_cfg & AF3_W_FWD_TILED) != 0;  // w_blocks is the af3_mxfp4_tile_fwd copy
  const bool x_off32 = (tile_cfg & AF3_X_OFFSETS_32) != 0;  // x's rows within 4 GiB of x (caller's word)
  const bool s_tiled = (tile_cfg & AF3_S_DX_TILED) != 0;    // w_scales is the af3_mxfp4_tile_dx_scales copy
  tile_cfg &= ~(AF3_W_FWD_TILED | AF3_X_OFFSETS_32 | AF3_S_DX_TILED);
  AF3_REQUIRE(tile_cfg >= 0, "moe_gemm: bad tile_cfg %d", tile_cfg);
  AF3_REQUIRE(N > 0 && K > 0 && n_expts > 0 && max_tiles >= 0, "moe_gemm: bad sizes N=%d K=%d E=%d", N, K, n_expts);
  if (max_tiles == 0) return 0;
  AF3_REQUIRE(x && w_blocks && w_scales && token_offs && block_pid_map && tile_offs && y, "moe_gemm: null pointer");
  AF3_REQUIRE((int64_t)max_tiles * ((N + 127) / 128) < 0x7fffffffLL, "moe_gemm: grid too large");
  AF3_REQUIRE(K % 32 == 0 && N % 32 == 0, "moe_gemm: N and K must be multiples of 32 (N=%d K=%d)", N, K);
  AF3_REQUIRE(ldx % 8 == 0 && al16(x), "moe_gemm: x must be 16-byte aligned with ld % 8 == 0");
  AF3_REQUIRE(lora_r >= 0 && lora_r <= 64, "moe_gemm: lora rank %d unsupported (max 64)", lora_r);
  AF3_REQUIRE(lora_r == 0 || (lora_l && lora_b && ld_l % 8 == 0 && lora_r % 8 == 0 && al16(lora_l) && al16(lora_b)),
              "moe_gemm: LoRA operands must be 16-byte aligned, rank % 8 == 0");
  AF3_REQUIRE(al16(w_blocks), "moe_gemm: weight blocks must be 16-byte aligned");
  AF3_REQUIRE(block_m == 128 || block_m == 256, "moe_gemm: block_m must be 128 or 256 (got %d)", block_m);
  Params p{};
  const int G_k = K / 32, G_n = N / 32;
  p.a = make_bf16(x, ldx, 0, gather_indx, gather_div);
  p.a_off32 = x_off32;
  p.b.ptr = w_blocks;
  p.b.scales = w_scales;
  if (trans_w == 0) {
    p.b.ld = (int64_t)G_k * 16;
    p.b.sld = G_k;
    p.b.estride = (int64_t)N * G_k * 16;
    p.b.sestride = (int64_t)N * G_k;
  } else {
    p.b.ld = (int64_t)G_n * 16;
    p.b.sld = G_n;
    p.b.estride = (int64_t)K * G_n * 16;
    p.b.sestride = (int64_t)K * G_n;
  }
  p.K = K;
  p.kx = lora_r;
  if (lora_r) {
    p.ax = make_bf16(lora_l, ld_l, 0, nullptr, 1);
    // trans 0: Bx[e] is [N][r] (k contiguous); trans 1: Bx[e] is [r][N] (n contiguous)
    p.bx = trans_w == 0 ? make_bf16(lora_b, lora_r, (int64_t)N * lora_r, nullptr, 1)
                        : make_bf16(lora_b, N, (int64_t)N * lora_r, nullptr, 1);
  }
  p.offs = token_offs;
  p.tile_map = block_pid_map;
  p.tile_offs = tile_offs;
  p.E = n_expts;
  p.bias = bias;
  p.bias_estride = N;
  p.gammas = gammas;
  p.gammas_f32 = gammas_f32;
  p.scale = 1.0f;
  p.c = y;
  p.ldc = ldy;
  p.N = N;
  p.epi = epi;
  p.glu = glu;
  p.ascale = a_row_scale;
  p.ld_glu = ld_glu;
  p.alpha = alpha;
  p.limit = limit;
  const bool trans = trans_w != 0;
  // tile configurations:
  //   26: gemm7 forward (128x256 work items on the 128-row map, 4 waves of
  //       128x64, two blocks per CU; activation rows through a three-stage
  //       global->LDS ring, the packed MXFP4 words straight into registers and
  //       converted there); default for trans_w 0 with block_m 128
  //   22: gemm4 forward (256x256 work items, 8 waves of 128x64, two per SIMD,
  //       packed MXFP4 through a three-stage global->LDS ring, converted in
  //       registers); default for trans_w 0 with block_m 256
  //   28: gemm8 input gradient (gemm5's k-loop on 128x256 items of the 128-row
  //       map, 4 waves of 128x64, two blocks per CU); default for trans_w 1
  //       with block_m 128
  //   23: gemm5 input gradient (packed weight rows read with transposing LDS
  //       loads, one three-stage ring for A, B and scales; 4 waves of 256x64);
  //       default for trans_w 1 with block_m 256
  //   4 / 2: gemm2, 256x256 / 128x256 tiles with the weight dequantised into
  //       LDS (general fallback for block_m 256 / 128)
  //   9: single-buffered 128x128 row tiles (any K % 32 == 0; used when K % 64 != 0)
  //   tile_cfg / 100 = m-tiles per group of the 22 / 23 / 26 / 28 work order (default 4; 2 for 26 / 28)
  int cfg = tile_cfg % 100;
  const int group_m = tile_cfg / 100 > 0 ? tile_cfg / 100 : 4;
  if (cfg == 0) {
    const bool g4_fwd = !trans && block_m == 256 && K % kBK == 0 && K / 32 <= kG4MaxG && al16(w_scales) && al16(y) &&
                        ldy % 8 == 0;
    const bool g7_fwd = !trans && block_m == 128 && K % kBK == 0 && K / 32 <= kG7MaxG && al16(w_scales) && al16(y) &&
                        ldy % 8 == 0;
    const bool g4_dgrad = trans && block_m == 256 && K % kBK == 0 && N % 64 == 0 && al16(y) && ldy % 8 == 0;
    const bool g8_dgrad = trans && block_m == 128 && K % kBK == 0 && N % 64 == 0 && al16(y) && ldy % 8 == 0;
    cfg = g4_fwd ? 22 : g7_fwd ? 26 : g4_dgrad ? 23 : g8_dgrad ? 28 : (block_m == 256 ? 4 : 2);
  }
  const bool bm_ok = (cfg == 4 || cfg == 22 || cfg == 23) ? block_m == 256 : block_m == 128;
  AF3_REQUIRE(bm_ok, "moe_gemm: tile_cfg %d does not match block_m %d", cfg, block_m);
  if (w_tiled) {  // only the two-blocks-per-CU forward reads the forward-tiled weights
    if (a_fp8 || trans || cfg != 26 || K % kBK != 0) {
      af3::set_error("moe_gemm: forward-tiled weights need the tile_cfg 26 forward (got cfg %d, trans_w %d)", cfg,
                     trans_w);
      return AF3_EUNSUPPORTED;
    }
    p.b_tiled = 1;
  }
  if (s_tiled) {  // only the two-blocks-per-CU input gradient reads the tiled scales
    if (a_fp8 || !trans || cfg != 28 || K % kBK != 0 || N % 64 != 0) {
      af3::set_error("moe_gemm: tiled input-gradient scales need tile_cfg 28 with trans_w 1 (got cfg %d, trans_w %d)",
                     cfg, trans_w);
      return AF3_EUNSUPPORTED;
    }
    p.s_tiled = 1;
    p.s_nt = (N + 255) / 256;
  }
  if (a_fp8) {  // E4M3 activations x MXFP4 weights on the block-scaled MFMA (256-row map)
    if (trans) {  // input gradient: the weights converted to E5M2 in registers
      if (block_m != 256 || K % kBK != 0 || N % 64 != 0 || !al16(y) || ldy % 8 != 0 || ldx % 16 != 0 || !al16(x) ||
          !a_row_scale || lora_r != 0 || epi != 0 || !(cfg == 23 || cfg == 0)) {
        af3::set_error("moe_gemm_f8 (trans_w 1): needs block_m 256, K %% 64 == 0, N %% 64 == 0, 16-byte aligned "
                       "rows, a row scale");
        return AF3_EUNSUPPORTED;
      }
      p.group_m = group_m;
      p.n_nblk = (N + kG4Rows - 1) / kG4Rows;
      dim3 grid(g4_grid(max_tiles, p.n_nblk, p.group_m));
      hipLaunchKernelGGL(gemm5_f8_kernel, grid, dim3(256), 0, stream, p);
      return af3::check_launch("moe_gemm_f8 (input gradient)");
    }
    if (block_m != 256 || K % kBK != 0 || K / 32 > kG4MaxG || !al16(w_scales) || !al16(y) || ldy % 8 != 0 ||
        ldx % 16 != 0 || !al16(x) || !a_row_scale || lora_r != 0 || epi != 0 || !(cfg == 22 || cfg == 0)) {
      af3::set_error("moe_gemm_f8: needs block_m 256, K %% 64 == 0, 16-byte aligned rows, a row scale");
      return AF3_EUNSUPPORTED;
    }
    p.group_m = group_m;
    p.n_nblk = (N + kG4Rows - 1) / kG4Rows;
    dim3 grid(g4_grid(max_tiles, p.n_nblk, p.group_m));
    hipLaunchKernelGGL((gemm4_fwd_f8_kernel<NONE>), grid, dim3(512), 0, stream, p);
    return af3::check_launch("moe_gemm_f8");
  }
  if (K % kBK != 0) cfg = 9;  // direct A loads need whole 64-deep k-steps (never with forward-tiled weights)
  if (epi != 0) {
    AF3_REQUIRE(glu && (epi == 1 || epi == 2), "moe_gemm: bad SwiGLU epilogue %d", epi);
    const bool ok = epi == 1 ? (trans && (cfg == 23 || cfg == 28) && ld_glu % 8 == 0 && al16(glu) && ldy >= 2LL * N)
                             : (!trans && (cfg == 22 || cfg == 26) && N % 2 == 0 && ld_glu % 4 == 0 &&
                                ((uintptr_t)glu & 7) == 0);
    if (!ok) {
      af3::set_error("moe_gemm: the fused SwiGLU epilogue %d is not available for tile_cfg %d / these operands", epi,
                     cfg);
      return AF3_EUNSUPPORTED;
    }
  }
  if (a_row_scale) {
    AF3_REQUIRE(lora_r == 0, "moe_gemm: a row scale cannot be combined with the LoRA extension segment");
    if (!(cfg == 22 || cfg == 23 || cfg == 26 || cfg == 28)) {
      af3::set_error("moe_gemm: the A row scale needs tile_cfg 22, 23, 26 or 28 (got %d)", cfg);
      return AF3_EUNSUPPORTED;
    }
  }
  if (cfg == 9 && block_m != 128) {
    af3::set_error("moe_gemm: K %% 64 != 0 needs block_m 128");
    return AF3_EINVAL;
  }
  switch (cfg) {
    case 2: launch_gemm2<128, 256, 2, 2>(trans, max_tiles, N, stream, p); break;
    case 4: launch_gemm2<256, 256, 2, 4>(trans, max_tiles, N, stream, p); break;
    case 22:
      p.group_m = group_m;
      AF3_REQUIRE(!trans && block_m == 256 && K % kBK == 0 && K / 32 <= kG4MaxG && al16(w_scales) && al16(y) &&
                      ldy % 8 == 0,
                  "moe_gemm: tile_cfg 22 needs trans_w 0, block_m 256, K %% 64 == 0, K <= %d, 16-byte aligned scales/y",
                  kG4MaxG * 32);
      launch_gemm4_fwd<2, 4>(max_tiles, N, stream, p);
      break;
    case 26:
      p.group_m = tile_cfg / 100 > 0 ? tile_cfg / 100 : 2;
      AF3_REQUIRE(!trans && block_m == 128 && K % kBK == 0 && K / 32 <= kG7MaxG && al16(w_scales) && al16(y) &&
                      ldy % 8 == 0,
                  "moe_gemm: tile_cfg 26 needs trans_w 0, block_m 128, K %% 64 == 0, K <= %d, 16-byte aligned", kG7MaxG * 32);
      launch_gemm7_fwd(max_tiles, N, stream, p);
      break;
    case 28:
      p.group_m = tile_cfg / 100 > 0 ? tile_cfg / 100 : 2;
      AF3_REQUIRE(trans && block_m == 128 && K % kBK == 0 && N % 64 == 0 && al16(y) && ldy % 8 == 0,
                  "moe_gemm: tile_cfg 28 needs trans_w 1, block_m 128, K %% 64 == 0, N %% 64 == 0, 16-byte aligned y");
      launch_gemm8_dgrad(max_tiles, N, stream, p);
      break;
    case 23:
      p.group_m = group_m;
      AF3_REQUIRE(trans && block_m == 256 && K % kBK == 0 && N % 64 == 0 && al16(y) && ldy % 8 == 0,
                  "moe_gemm: tile_cfg 23 needs trans_w 1, block_m 256, K %% 64 == 0, N %% 64 == 0, 16-byte aligned y");
      launch_gemm5_dgrad(max_tiles, N, stream, p);
      break;
    case 9: {
      dim3 grid(max_tiles, (N + 127) / 128);
      if (!trans)
        hipLaunchKernelGGL((rowtile_kernel<128, 128, 2, 2, ROWS_BF16, ROWS_FP4, ROWS_BF16, ROWS_BF16>), grid,
                           dim3(kThreads), 0, stream, p);
      else
        hipLaunchKernelGGL((rowtile_kernel<128, 128, 2, 2, ROWS_BF16, COLS_FP4, ROWS_BF16, COLS_BF16>), grid,
                           dim3(kThreads), 0, stream, p);
      break;
    }
    default:
      af3::set_error("moe_gemm: unknown tile_cfg %d", tile_cfg);
      return AF3_EINVAL;
  }
  return af3::check_launch("moe_gemm");
}

extern "C" int af3_moe_gemm(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                            const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                            const void* gammas, int gammas_f32, const uint16_t* lora_l, int64_t ld_l,
                            const uint16_t* lora_b, int lora_r, const int32_t* token_offs, const int32_t* block_pid_map,
                            const int32_t* tile_offs, int max_tiles, int block_m, int tile_cfg, int n_expts, int N,
                            int K, uint16_t* y, int64_t ldy, void* stream) {
  return moe_gemm_impl(x, ldx, gather_indx, gather_div, w_blocks, w_scales, trans_w, bias, gammas, gammas_f32, lora_l,
                       ld_l, lora_b, lora_r, token_offs, block_pid_map, tile_offs, max_tiles, block_m, tile_cfg,
                       n_expts, N, K, y, ldy, 0, nullptr, 0, 0.f, 0.f, nullptr, stream);
}

// fp8-mode forward: A = per-token E4M3 codes [rows][ldx bytes] (ldx % 16 == 0),
// y = bf16((acc * a_row_scale[a(r)] + bias) * gammas) with acc the fp32 sum of
// E4M3 codes x MXFP4 weights on the block-scaled MFMA.  trans_w 0, block_m
// 256, no LoRA; AF3_EUNSUPPORTED when a requirement fails.
extern "C" int af3_moe_gemm_f8(const uint8_t* x_e4m3, int64_t ldx, const int32_t* gather_indx, int gather_div,
                               const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                               const void* gammas, int gammas_f32, const int32_t* token_offs,
                               const int32_t* block_pid_map, const int32_t* tile_offs, int max_tiles, int block_m,
                               int tile_cfg, int n_expts, int N, int K, uint16_t* y, int64_t ldy,
                               const float* a_row_scale, void* stream) {
  AF3_REQUIRE(a_row_scale, "moe_gemm_f8: null row scale");
  return moe_gemm_impl((const uint16_t*)x_e4m3, ldx, gather_indx, gather_div, w_blocks, w_scales, trans_w, bias, gammas,
                       gammas_f32, nullptr, 0, nullptr, 0, token_offs, block_pid_map, tile_offs, max_tiles, block_m,
                       tile_cfg, n_expts, N, K, y, ldy, 0, nullptr, 0, 0.f, 0.f, a_row_scale, stream, 1);
}

// af3_moe_gemm with a per-row scale of the A operand applied to the
// accumulator: y = bf16((acc * a_row_scale[a(r)] + bias) * gammas), a(r) the
// A row of output row r.  The fp8 mode's per-token activation scale.
// AF3_EUNSUPPORTED when the selected tile configuration has no such epilogue.
extern "C" int af3_moe_gemm_rowscale(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                                     const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                                     const void* gammas, int gammas_f32, const int32_t* token_offs,
                                     const int32_t* block_pid_map, const int32_t* tile_offs, int max_tiles,
                                     int block_m, int tile_cfg, int n_expts, int N, int K, uint16_t* y, int64_t ldy,
                                     const float* a_row_scale, void* stream) {
  AF3_REQUIRE(a_row_scale, "moe_gemm_rowscale: null row scale");
  return moe_gemm_impl(x, ldx, gather_indx, gather_div, w_blocks, w_scales, trans_w, bias, gammas, gammas_f32, nullptr,
                       0, nullptr, 0, token_offs, block_pid_map, tile_offs, max_tiles, block_m, tile_cfg, n_expts, N,
                       K, y, ldy, 0, nullptr, 0, 0.f, 0.f, a_row_scale, stream);
}

// af3_moe_gemm with the gpt-oss clamped SwiGLU fused into the epilogue
// (epi 1: trans_w 1, y <- dGU [rows][2N] from dI and the saved pre-activation
// glu [rows][2N]; epi 2: trans_w 0, y <- the pre-activation [rows][N] and glu
// <- its SwiGLU [rows][N / 2]).  AF3_EUNSUPPORTED when the selected tile
// configuration has no fused epilogue.
extern "C" int af3_moe_gemm_swiglu(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                                   const uint8_t* w_blocks, const uint8_t* w_scales, int trans_w, const float* bias,
                                   const void* gammas, int gammas_f32, const uint16_t* lora_l, int64_t ld_l,
                                   const uint16_t* lora_b, int lora_r, const int32_t* token_offs,
                                   const int32_t* block_pid_map, const int32_t* tile_offs, int max_tiles, int block_m,
                                   int tile_cfg, int n_expts, int N, int K, uint16_t* y, int64_t ldy, int epi,
                                   void* glu, int64_t ld_glu, float alpha, float limit, void* stream) {
  AF3_REQUIRE(epi == 1 || epi == 2, "moe_gemm_swiglu: epi must be 1 or 2 (got %d)", epi);
  return moe_gemm_impl(x, ldx, gather_indx, gather_div, w_blocks, w_scales, trans_w, bias, gammas, gammas_f32, lora_l,
                       ld_l, lora_b, lora_r, token_offs, block_pid_map, tile_offs, max_tiles, block_m, tile_cfg,
                       n_expts, N, K, y, ldy, epi, glu, ld_glu, alpha, limit, nullptr, stream);
}

// Skinny per-expert row product for the LoRA terms (BM = 128 map):
//   trans_b = 0: out[r][j] = scale * sum_k X[a(r)][k] Wl[e][j][k]   Wl [E][n_out][K]
//   trans_b = 1: out[r][j] = scale * sum_k X[a(r)][k] Wl[e][k][j]   Wl [E][K][n_out]
extern "C" int af3_lora_rows(const uint16_t* x, int64_t ldx, const int32_t* gather_indx, int gather_div,
                             const uint16_t* wl, int trans_b, float scale, const int32_t* token_offs,
                             const int32_t* block_pid_map, int max_tiles, int n_expts, int n_out, int K,
                             uint16_t* out, int64_t ld_out, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_out > 0 && n_out <= 64 && K > 0, "lora_rows: bad sizes n_out=%d K=%d", n_out, K);
  if (max_tiles == 0) return 0;
  AF3_REQUIRE(K % 8 == 0 && n_out % 8 == 0 && ldx % 8 == 0 && al16(x) && al16(wl),
              "lora_rows: operands must be 16-byte aligned with sizes % 8 == 0");
  {
    const int rc = af3::lora_rows_fast(x, ldx, gather_indx, gather_div, wl, trans_b, scale, token_offs, block_pid_map,
                                       max_tiles, n_out, K, out, ld_out, stream);
    if (rc != AF3_EUNSUPPORTED) return rc;
  }
  Params p{};
  p.a = make_bf16(x, ldx, 0, gather_indx, gather_div);
  p.b = trans_b == 0 ? make_bf16(wl, K, (int64_t)n_out * K, nullptr, 1)
                     : make_bf16(wl, n_out, (int64_t)n_out * K, nullptr, 1);
  p.K = K;
  p.offs = token_offs;
  p.tile_map = block_pid_map;
  p.E = n_expts;
  p.scale = scale;
  p.c = out;
  p.ldc = ld_out;
  p.N = n_out;
  if (n_out <= 32) {
    dim3 grid(max_tiles, 1);
    if (trans_b == 0)
      hipLaunchKernelGGL((rowtile_kernel<128, 32, 4, 1, ROWS_BF16, ROWS_BF16, NONE, NONE>), grid, dim3(kThreads), 0,
                         stream, p);
    else
      hipLaunchKernelGGL((rowtile_kernel<128, 32, 4, 1, ROWS_BF16, COLS_BF16, NONE, NONE>), grid, dim3(kThreads), 0,
                         stream, p);
  } else {
    dim3 grid(max_tiles, 1);
    if (trans_b == 0)
      hipLaunchKernelGGL((rowtile_kernel<128, 64, 2, 2, ROWS_BF16, ROWS_BF16, NONE, NONE>), grid, dim3(kThreads), 0,
                         stream, p);
    else
      hipLaunchKernelGGL((rowtile_kernel<128, 64, 2, 2, ROWS_BF16, COLS_BF16, NONE, NONE>), grid, dim3(kThreads), 0,
                         stream, p);
  }
  return af3::check_launch("lora_rows");
}

// Per-expert weight gradient over the expert's rows:
//   G[e][m][n] = scale * sum_{r in rows(e)} (rs(r) * A[a(r)][m]) * B[b(r)][n]
// with a(r) = a_gather ? a_gather[r] / a_div : r (same for b) and rs the
// optional bf16 per-row multiplier.  G is bf16 [E][M][N] row-major.  The rows
// are split into chunk_rows-row chunks described by chunk_map / chunk_offs
// (block_pid_map / token_offs_pad of af3_expt_data for that block size); each
// chunk writes an fp32 partial into `partials`, then the partials of an expert
// are summed in chunk order.
extern "C" size_t af3_lora_wgrad_workspace_bytes(int max_chunks, int M, int N) {
  return (size_t)(max_chunks > 0 ? max_chunks : 1) * (size_t)M * (size_t)N * sizeof(float);
}

extern "C" int af3_lora_wgrad(const uint16_t* a, int64_t lda, const int32_t* a_gather, int a_div,
                              const uint16_t* a_rowscale, const uint16_t* b, int64_t ldb, const int32_t* b_gather,
                              int b_div, float scale, const int32_t* token_offs, int n_expts, int M, int N,
                              const int32_t* chunk_map, const int32_t* chunk_offs, int max_chunks, int chunk_rows,
                              float* partials, size_t partial_bytes, uint16_t* g, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M > 0 && N > 0 && n_expts > 0 && max_chunks >= 0 && chunk_rows > 0, "lora_wgrad: bad sizes");
  AF3_REQUIRE(M % 8 == 0 && N % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && al16(a) && al16(b) && al16(g),
              "lora_wgrad: operands must be 16-byte aligned with sizes % 8 == 0");
  AF3_REQUIRE(partial_bytes >= af3_lora_wgrad_workspace_bytes(max_chunks, M, N) && partials && al16(partials),
              "lora_wgrad: partials workspace too small");
  {
    int rc = AF3_EUNSUPPORTED;
    if ((N == 16 || N == 32) && b_gather == nullptr)  // G = A^T B with B the rank side: [M][r]
      rc = af3::lora_wgrad_fast(a, lda, a_gather, a_div, b, ldb, a_rowscale, 0, M, N, scale, token_offs, chunk_map,
                                chunk_offs, max_chunks, chunk_rows, n_expts, partials, g, stream);
    else if ((M == 16 || M == 32) && a_gather == nullptr)  // A the rank side: [r][N]
      rc = af3::lora_wgrad_fast(b, ldb, b_gather, b_div, a, lda, a_rowscale, 1, N, M, scale, token_offs, chunk_map,
                                chunk_offs, max_chunks, chunk_rows, n_expts, partials, g, stream);
    if (rc != AF3_EUNSUPPORTED) return rc;
  }
  Params p{};
  p.a = make_bf16(a, lda, 0, a_gather, a_div, a_rowscale);
  p.b = make_bf16(b, ldb, 0, b_gather, b_div);
  p.offs = token_offs;
  p.tile_map = chunk_map;
  p.E = n_expts;
  p.scale = scale;
  p.M = M;
  p.N = N;
  p.chunk_rows = chunk_rows;
  p.partials = partials;
  if (max_chunks > 0) {
    if (N <= 32) {  // tall output (e.g. dB: [N_out][r])
      p.n_mblk = (M + 127) / 128;
      p.n_nblk = 1;
      hipLaunchKernelGGL((wgrad_partial_kernel<128, 32, 4, 1>), dim3(max_chunks, p.n_mblk), dim3(kThreads), 0,
                         stream, p);
    } else if (M <= 32) {  // wide output (e.g. dA: [r][K])
      p.n_mblk = 1;
      p.n_nblk = (N + 127) / 128;
      hipLaunchKernelGGL((wgrad_partial_kernel<32, 128, 1, 4>), dim3(max_chunks, p.n_nblk), dim3(kThreads), 0,
                         stream, p);
    } else {
      p.n_mblk = (M + 127) / 128;
      p.n_nblk = (N + 127) / 128;
      hipLaunchKernelGGL((wgrad_partial_kernel<128, 128, 2, 2>), dim3(max_chunks, p.n_mblk * p.n_nblk),
                         dim3(kThreads), 0, stream, p);
    }
    int rc = af3::check_launch("lora_wgrad/partial");
    if (rc) return rc;
  }
  const int64_t MN = (int64_t)M * N;  // multiple of 64: M % 8 == 0 and N % 8 == 0
  hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)af3_cdiv(MN / 4, 256), n_expts), dim3(256), 0, stream,
                     partials, chunk_offs, MN, scale, g);
  return af3::check_launch("lora_wgrad/reduce");
}

// out[t][:] = sum_{j<K} rows[src[t*K+j]][:]  (the scatter-sum of matmul_ogs)
// Forward-tiled copy of packed MXFP4 weights (Params::b_tiled): 16-byte unit
// u of out [n_mats * N / 32][K / 64][2][32][16] is block 2 kt + h of row
// 32 (u >> 6) / nk + r, with r = u & 31, h = (u >> 5) & 1, kt = (u >> 6) % nk.
// One wave writes one KB tile; its 32 rows are read 32 bytes each, and the
// tiles of consecutive k-steps of the same rows follow each other, so every
// 128-byte line of the source comes from HBM once and is re-read from L2.
__global__ __launch_bounds__(256) void tile_fwd_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                       int64_t n_units, int nk, int64_t ld) {
  for (int64_t u = blockIdx.x * 256LL + threadIdx.x; u < n_units; u += (int64_t)gridDim.x * 256) {
    const int l = (int)(u & 63);
    const int64_t t = u >> 6;
    const int64_t row = (t / nk) * 32 + (l & 31);  // t / nk = the 32-row group over all matrices
    const int kt = (int)(t % nk);
    *(af3_u32x4*)(out + u * 16) = *(const af3_u32x4*)(in + row * ld + (2 * kt + (l >> 5)) * 16);
  }
}

extern "C" int af3_mxfp4_tile_fwd(const uint8_t* blocks, int64_t n_mats, int N, int K, uint8_t* out, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_mats >= 0 && N > 0 && K > 0, "mxfp4_tile_fwd: bad sizes E=%lld N=%d K=%d", (long long)n_mats, N, K);
  AF3_REQUIRE(N % 32 == 0 && K % 64 == 0, "mxfp4_tile_fwd: needs N %% 32 == 0 and K %% 64 == 0 (N=%d K=%d)", N, K);
  if (n_mats == 0) return 0;
  AF3_REQUIRE(blocks && out && al16(blocks) && al16(out), "mxfp4_tile_fwd: blocks / out must be 16-byte aligned");
  const int64_t n_units = n_mats * N * (int64_t)(K / 32);
  const int64_t bytes = n_units * 16;
  AF3_REQUIRE(out + bytes <= blocks || blocks + bytes <= out, "mxfp4_tile_fwd: out must not overlap blocks");
  const int64_t nblk = af3_cdiv(n_units, 256);
  const unsigned grid = (unsigned)(nblk < 16384 ? nblk : 16384);
  hipLaunchKernelGGL(tile_fwd_kernel, dim3(grid), dim3(256), 0, stream, blocks, out, n_units, K / 64,
                     (int64_t)(K / 2));
  return af3::check_launch("mxfp4_tile_fwd");
}

// Tiled input-gradient scales (Params::s_tiled): byte (e, kc, nt, b, r) of out
// [n_mats][K/64][NT][8][64] is scale byte (row 64 kc + r, block 8 nt + b) of
// matrix e, [n_mats][K][N/32] row-major; blocks past N/32 (the last n-tile of
// N % 256 != 0) hold 127 (a unit scale, never used).
__global__ __launch_bounds__(256) void tile_dx_scales_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                             int64_t n_out, int nk, int nt, int G) {
  for (int64_t o = blockIdx.x * 256LL + threadIdx.x; o < n_out; o += (int64_t)gridDim.x * 256) {
    const int r = (int)(o & 63), b = (int)((o >> 6) & 7);
    const int64_t t = o >> 9;  // (e nk + kc) nt + n
    const int n = (int)(t % nt);
    const int64_t ek = t / nt;  // e nk + kc
    const int blk = n * 8 + b;
    out[o] = blk < G ? in[(ek * 64 + r) * G + blk] : (uint8_t)127;
  }
}

// flag (e, nt) of the tiled scales: 1 when a scale byte of matrix e in the
// columns of n-tile nt lies outside [2, 252] (the input gradient then runs
// the exact integer conversion for that work item)
__global__ __launch_bounds__(256) void tile_dx_flags_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ flags,
                                                            int K, int nt, int G) {
  const int e = blockIdx.x / nt, n = blockIdx.x % nt;
  const int b0 = n * 8, nb = min(8, G - b0);
  bool odd = false;
  for (int i = threadIdx.x; i < K * nb; i += 256) {
    const uint8_t v = in[((int64_t)e * K + i / nb) * G + b0 + i % nb];
    odd |= (uint32_t)v - 2u > 250u;
  }
  odd = __syncthreads_or(odd);
  if (threadIdx.x == 0) flags[blockIdx.x] = odd ? 1 : 0;
}

extern "C" int af3_mxfp4_tile_dx_scales(const uint8_t* scales, int64_t n_mats, int K, int N, uint8_t* out,
                                        void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_mats >= 0 && N > 0 && K > 0, "mxfp4_tile_dx_scales: bad sizes E=%lld K=%d N=%d", (long long)n_mats,
              K, N);
  AF3_REQUIRE(K % 64 == 0 && N % 32 == 0, "mxfp4_tile_dx_scales: needs K %% 64 == 0 and N %% 32 == 0 (K=%d N=%d)", K,
              N);
  if (n_mats == 0) return 0;
  AF3_REQUIRE(scales && out, "mxfp4_tile_dx_scales: null pointer");
  const int nt = (N + 255) / 256;
  const int64_t n_out = n_mats * (K / 64) * (int64_t)nt * 512;
  const int64_t n_in = n_mats * (int64_t)K * (N / 32);
  AF3_REQUIRE(out + n_out + n_mats * nt <= scales || scales + n_in <= out,
              "mxfp4_tile_dx_scales: out must not overlap scales");
  AF3_REQUIRE(n_mats * nt < 0x7fffffffLL, "mxfp4_tile_dx_scales: too many matrices");
  const int64_t nblk = af3_cdiv(n_out, 256);
  hipLaunchKernelGGL(tile_dx_scales_kernel, dim3((unsigned)(nblk < 16384 ? nblk : 16384)), dim3(256), 0, stream, scales,
                     out, n_out, K / 64, nt, N / 32);
  hipLaunchKernelGGL(tile_dx_flags_kernel, dim3((unsigned)(n_mats * nt)), dim3(256), 0, stream, scales, out + n_out, K,
                     nt, N / 32);
  return af3::check_launch("mxfp4_tile_dx_scales");
}

extern "C" int af3_moe_combine(const uint16_t* rows, int64_t ld_rows, const int32_t* src_indx, int64_t n_tokens,
                               int K, int N, uint16_t* out, int64_t ld_out, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_tokens >= 0 && K > 0 && N > 0, "moe_combine: bad sizes");
  if (n_tokens == 0) return 0;
  AF3_REQUIRE(N % 8 == 0 && ld_rows % 8 == 0 && ld_out % 8 == 0 && al16(rows) && al16(out),
              "moe_combine: rows/out must be 16-byte aligned with N % 8 == 0");
  int vpr = N / 8;
  int64_t nv = n_tokens * vpr;
  if (K <= 4)
    hipLaunchKernelGGL(combine_kernel<4>, dim3((unsigned)af3_cdiv(nv, 256)), dim3(256), 0, stream, rows, ld_rows,
                       src_indx, K, N, out, ld_out, vpr, nv);
  else if (K <= 8)
    hipLaunchKernelGGL(combine_kernel<8>, dim3((unsigned)af3_cdiv(nv, 256)), dim3(256), 0, stream, rows, ld_rows,
                       src_indx, K, N, out, ld_out, vpr, nv);
  else
    hipLaunchKernelGGL(combine_kernel<0>, dim3((unsigned)af3_cdiv(nv, 256)), dim3(256), 0, stream, rows, ld_rows,
                       src_indx, K, N, out, ld_out, vpr, nv);
  return af3::check_launch("moe_combine");
}
