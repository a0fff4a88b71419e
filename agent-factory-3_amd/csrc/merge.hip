// Expert-LoRA merge for weight sync: one bf16 weight per expert with the
// adapter folded in,
//
//   W'[e][n][k] = bf16( float(deq(W[e])[n][k]) + s * sum_j B[e][n][j] * A[e][j][k] )
//
// deq = the MXFP4 -> bf16 rule of the dequant kernel (kernels.py:120-158),
// A [E][r][K] and B [E][N][r] bf16 (the adapter layout of the experts module),
// s = lora_alpha / r.  The arithmetic follows the reference's LoRA merge for
// sglang sync (model_trainer.py:653-719, arithmetic at 710-712): base and delta in fp32, the product
// B @ A scaled after the sum, one rounding to bf16 (round to nearest even).
//
// Output layouts: 0 = [E][N][K] (the frozen weight's own row order),
// 1 = [E][K][N] (transformers' GptOssExperts parameter, modeling_gpt_oss.py:75-77,
// the layout a bf16 gpt-oss checkpoint holds).
//
// A tile = 64(n) x 64(k) of one expert; persistent blocks of 4 waves walk the tiles.  The rank-r delta
// runs on v_mfma_f32_32x32x16_bf16 (products of bf16 are exact in fp32), each
// wave one 32x32 sub-tile (A's k-slice staged in LDS with 16-byte loads), the
// result staged in LDS as fp32.  Then each thread
// dequantises a quarter MXFP4 block (8 values) of two rows, adds the delta and
// writes 16 B of bf16 per row: straight to HBM for layout 0, through an LDS
// transpose for layout 1 (64-column runs of 128 B, whole lines per store).  HBM-bound: per output element 2 B written
// and 17/32 B of packed weight read; the adapters are re-read from L2.
#include "af3_common.h"

namespace {

constexpr int kMgN = 64;
constexpr int kMgK = 64;
constexpr int kMgDP = 68;  // fp32 pitch of the delta tile (16-lane groups of the row reads hit distinct banks)
constexpr int kMgMP = 66;  // u16 pitch of the merged tile (transposed reads hit distinct banks)
constexpr int kMgLP = 72;  // u16 pitch of the staged A slice (16-byte rows; the half-waves' rows 32 banks apart)
static_assert(kMgN * kMgMP <= kMgN * kMgLP, "merged tile must fit the staging buffer");
constexpr int kMgBlocksPerXcd = 32 * 6;

struct MergeTile {
  int e, n0, k0;
};

__device__ __forceinline__ MergeTile merge_tile(int64_t tile, int n_tiles_n, int n_tiles_k) {
  const int64_t rest = tile / n_tiles_k;
  return {(int)(rest / n_tiles_n), (int)(rest % n_tiles_n) * kMgN, (int)(tile % n_tiles_k) * kMgK};
}

// The packed dword (8 consecutive k) of rows p*32 + tid/8, p = 0, 1, of a tile.
__device__ __forceinline__ void merge_load_packed(const uint8_t* __restrict__ blocks,
                                                  const uint8_t* __restrict__ scales, MergeTile t, int N, int K,
                                                  int tid, uint32_t v[2], uint32_t sc[2]) {
  const int k = t.k0 + (tid & 7) * 8;
  const int G = K >> 5;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int n = t.n0 + p * 32 + (tid >> 3);
    v[p] = 0u;
    sc[p] = 0u;
    if (n < N && k < K) {
      const int64_t grp = ((int64_t)t.e * N + n) * G + (k >> 5);
      v[p] = __builtin_nontemporal_load((const uint32_t*)(blocks + grp * 16 + ((k & 31) >> 1)));
      sc[p] = scales[grp];
    }
  }
}

// Persistent blocks: block b serves XCD b % 8 and walks that XCD's contiguous run of
// tiles (k fastest) with stride blocks_per_xcd, so the neighbouring k-tiles of a row,
// which share lines of the packed weight and its scales, are in flight together in one
// L2.  The next tile's packed dwords are loaded while the current tile is computed.
__global__ __launch_bounds__(256, 6) void lora_merge_generic_kernel(const uint8_t* __restrict__ blocks,
                                                         const uint8_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ la,
                                                         const uint16_t* __restrict__ lb, float s,
                                                         uint16_t* __restrict__ out, int N, int K, int r,
                                                         int layout, int n_tiles_n, int n_tiles_k, int64_t n_tiles,
                                                         int64_t per_xcd, int blocks_per_xcd) {
  __shared__ __attribute__((aligned(16))) float D[kMgN * kMgDP];
  // A's k-slice (up to 64 of its r rows at a time) before the MFMA, the merged tile after it
  __shared__ __attribute__((aligned(16))) uint16_t LM[kMgN * kMgLP];
  uint16_t* const La = LM;
  uint16_t* const Mt = LM;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int xcd = blockIdx.x & 7;
  const int64_t t_end = min(n_tiles, (int64_t)(xcd + 1) * per_xcd);
  int64_t tile = (int64_t)xcd * per_xcd + (blockIdx.x >> 3);
  uint32_t v[2] = {0u, 0u}, sc[2] = {0u, 0u};
  if (tile < t_end) merge_load_packed(blocks, scales, merge_tile(tile, n_tiles_n, n_tiles_k), N, K, tid, v, sc);

  for (; tile < t_end; tile += blocks_per_xcd) {
    const MergeTile t = merge_tile(tile, n_tiles_n, n_tiles_k);
    const int e = t.e, n0 = t.n0, k0 = t.k0;
    uint32_t vn[2] = {0u, 0u}, scn[2] = {0u, 0u};
    if (tile + blocks_per_xcd < t_end)
      merge_load_packed(blocks, scales, merge_tile(tile + blocks_per_xcd, n_tiles_n, n_tiles_k), N, K, tid, vn, scn);

    // ---- delta = B[e][n0.., :] @ A[e][:, k0..] on the MFMA, one 32x32 sub-tile per wave
    {
      const int nr = n0 + (w >> 1) * 32 + (lane & 31);
      const int kcl = (w & 1) * 32 + (lane & 31);
      af3_f32x16 acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.f;
      for (int jc = 0; jc < r; jc += 64) {
        // stage A[e][jc .. jc+64)[k0 .. k0+64) in LDS with 16-byte loads (the MFMA wants
        // 8 consecutive j per lane, which run down A's columns); the barrier also ends
        // the previous tile's reads of the merged tile that shares this buffer
        const int rc = min(64, r - jc);
        __syncthreads();
        for (int j = tid >> 3; j < rc; j += 32) {
          const int kk = k0 + (tid & 7) * 8;
          af3_u32x4 val = {0u, 0u, 0u, 0u};
          if (kk < K) val = *(const af3_u32x4*)(la + ((int64_t)e * r + jc + j) * K + kk);
          *(af3_u32x4*)(La + j * kMgLP + (tid & 7) * 8) = val;
        }
        __syncthreads();
        for (int j0 = 0; j0 < rc; j0 += 16) {
          const int jl = j0 + (lane >> 5) * 8;  // this lane's 8 reduction indices (r % 8 == 0)
          af3_u32x4 aw = {0u, 0u, 0u, 0u};
          uint32_t bw[4] = {0u, 0u, 0u, 0u};
          if (jl < rc) {
            if (nr < N) aw = *(const af3_u32x4*)(lb + ((int64_t)e * N + nr) * r + jc + jl);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              bw[q] = (uint32_t)La[(jl + 2 * q) * kMgLP + kcl] | ((uint32_t)La[(jl + 2 * q + 1) * kMgLP + kcl] << 16);
          }
          const af3_bf16x8 a = __builtin_bit_cast(af3_bf16x8, aw);
          const af3_bf16x8 b = __builtin_bit_cast(af3_bf16x8, (af3_u32x4){bw[0], bw[1], bw[2], bw[3]});
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = (w >> 1) * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        D[row * kMgDP + kcl] = acc[i] * s;
      }
    }
    __syncthreads();

    // ---- dequantise + add; thread = 8 consecutive k of rows p*32 + tid/8 (eight lanes
    // span a 128-byte output run, so each 16-byte store instruction writes whole lines)
    const int kl = (tid & 7) * 8;
    const int k = k0 + kl;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int nl = p * 32 + (tid >> 3);
      const bool live = n0 + nl < N && k < K;
      uint32_t m[4] = {0u, 0u, 0u, 0u};
      if (live) {
        uint32_t q[4];
        af3_dequant_u32(v[p], sc[p], q);
        const float4* d4 = (const float4*)(D + nl * kMgDP + kl);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float4 d = d4[c];
          const uint32_t lo = q[2 * c], hi = q[2 * c + 1];
          m[2 * c] = af3_pack_bf16x2(af3_bf16_to_f32(lo & 0xFFFFu) + d.x, af3_bf16_to_f32(lo >> 16) + d.y);
          m[2 * c + 1] = af3_pack_bf16x2(af3_bf16_to_f32(hi & 0xFFFFu) + d.z, af3_bf16_to_f32(hi >> 16) + d.w);
        }
      }
      if (layout == 0) {
        if (live)
          __builtin_nontemporal_store((af3_u32x4){m[0], m[1], m[2], m[3]},
                                      (af3_u32x4*)(out + ((int64_t)e * N + n0 + nl) * K + k));
      } else {
        uint32_t* mrow = (uint32_t*)(Mt + nl * kMgMP + kl);
#pragma unroll
        for (int c = 0; c < 4; ++c) mrow[c] = m[c];
      }
    }

    if (layout != 0) {
      // ---- layout 1: transposed through LDS; thread = 8 consecutive n of k row p*32 + tid/8
      __syncthreads();
      const int nt = (tid & 7) * 8;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int kt = p * 32 + (tid >> 3);
        const int kk = k0 + kt;
        if (kk >= K) break;
        uint32_t t4[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          t4[c] = (uint32_t)Mt[(nt + 2 * c) * kMgMP + kt] | ((uint32_t)Mt[(nt + 2 * c + 1) * kMgMP + kt] << 16);
        uint16_t* o = out + ((int64_t)e * K + kk) * N + n0 + nt;
        if ((N & 7) == 0 && n0 + nt + 8 <= N) {
          __builtin_nontemporal_store((af3_u32x4){t4[0], t4[1], t4[2], t4[3]}, (af3_u32x4*)o);
        } else {
          for (int c = 0; c < 8 && n0 + nt + c < N; ++c) o[c] = (uint16_t)(t4[c >> 1] >> (16 * (c & 1)));
        }
      }
    }
    v[0] = vn[0];
    v[1] = vn[1];
    sc[0] = scn[0];
    sc[1] = scn[1];
  }
}

// The merge for r <= 64.  A block owns one (expert, 64-column k-tile, run of up to
// kMgRun n-tiles) unit: A's k-slice is staged once, transposed (At[k][j], so a lane's
// MFMA fragment is one 16-byte read), then the block walks down its n-tiles.  For
// each tile the next tile's packed dwords and B fragments are loaded into registers
// while the current tile is computed; every pointer is a per-tile uniform base plus a
// per-thread 32-bit offset that does not change along the walk.  Units are dealt to
// the XCDs in contiguous runs (k-tile fastest), so the blocks sharing the lines of a
// packed row run on one L2.
constexpr int kMgRun = 16;
constexpr int kMgAtP = 72;  // u16 pitch of At (16-byte rows)

__global__ __launch_bounds__(256, 4) void lora_merge_kernel(const uint8_t* __restrict__ blocks,
                                                            const uint8_t* __restrict__ scales,
                                                            const uint16_t* __restrict__ la,
                                                            const uint16_t* __restrict__ lb, float s,
                                                            uint16_t* __restrict__ out, int N, int K, int r,
                                                            int layout, int n_tiles_n, int n_tiles_k, int n_runs,
                                                            int n_units, int per_xcd) {
  __shared__ __attribute__((aligned(16))) uint16_t At[kMgK * kMgAtP];
  __shared__ __attribute__((aligned(16))) float D[kMgN * kMgDP];
  __shared__ __attribute__((aligned(16))) uint16_t Mt[kMgN * kMgMP];
  const int unit = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (unit >= n_units || unit >= ((int)(blockIdx.x & 7) + 1) * per_xcd) return;
  const int kt_i = unit % n_tiles_k;
  const int rest = unit / n_tiles_k;
  const int run = rest % n_runs;
  const int e = rest / n_runs;
  const int k0 = kt_i * kMgK;
  const int t_first = run * kMgRun;
  const int t_last = min(n_tiles_n, t_first + kMgRun);
  const int G = K >> 5;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;

  // ---- At[k][j] = A[e][j][k0 + k]
  {
    const uint16_t* a_e = la + (int64_t)e * r * K + k0;
    const int c = tid & 7;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = h * 32 + (tid >> 3);
      if (j < r) {
        af3_u32x4 val = {0u, 0u, 0u, 0u};
        if (k0 + c * 8 < K) val = *(const af3_u32x4*)(a_e + j * K + c * 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          At[(c * 8 + 2 * i) * kMgAtP + j] = (uint16_t)(val[i] & 0xFFFFu);
          At[(c * 8 + 2 * i + 1) * kMgAtP + j] = (uint16_t)(val[i] >> 16);
        }
      }
    }
  }

  // per-thread offsets, fixed along the walk
  const int kl = (tid & 7) * 8;            // 8 consecutive k of rows p*32 + tid/8
  const bool k_live = k0 + kl < K;
  const int kcl = (w & 1) * 32 + (lane & 31);
  const int nsub = (w >> 1) * 32 + (lane & 31);
  const int jh = (lane >> 5) * 8;
  uint32_t off_b[2], off_s[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int nl = p * 32 + (tid >> 3);
    off_b[p] = (uint32_t)(nl * G * 16 + (kl >> 1));
    off_s[p] = (uint32_t)(nl * G + (kl >> 5));
  }
  const uint32_t off_lb = (uint32_t)(nsub * r + jh);

  uint32_t v[2], sc[2];
  af3_u32x4 bv[4];
  auto fetch = [&](int ti, uint32_t v_[2], uint32_t sc_[2], af3_u32x4 bv_[4]) {
    const int n0 = ti * kMgN;
    const int64_t row0 = (int64_t)e * N + n0;
    const uint8_t* bt = blocks + (row0 * G + (k0 >> 5)) * 16;
    const uint8_t* st = scales + row0 * G + (k0 >> 5);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      v_[p] = 0u;
      sc_[p] = 0u;
      if (n0 + p * 32 + (tid >> 3) < N && k_live) {
        v_[p] = __builtin_nontemporal_load((const uint32_t*)(bt + off_b[p]));
        sc_[p] = st[off_s[p]];
      }
    }
    const uint16_t* lt = lb + row0 * r;
    const bool n_ok = n0 + nsub < N;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bv_[q] = (af3_u32x4){0u, 0u, 0u, 0u};
      if (q * 16 + jh < r && n_ok) bv_[q] = *(const af3_u32x4*)(lt + off_lb + q * 16);
    }
  };
  fetch(t_first, v, sc, bv);

  for (int ti = t_first; ti < t_last; ++ti) {
    const int n0 = ti * kMgN;
    // consume the registers the previous fetch filled before the next fetch is issued,
    // so that no wait for the new loads is needed before the end of this tile
    uint32_t qd[2][4];
#pragma unroll
    for (int p = 0; p < 2; ++p) af3_dequant_u32(v[p], sc[p], qd[p]);
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(bv[q]));
    uint32_t vn[2] = {0u, 0u}, scn[2] = {0u, 0u};
    af3_u32x4 bvn[4] = {};
    if (ti + 1 < t_last) fetch(ti + 1, vn, scn, bvn);
    __syncthreads();  // At staged (first tile); the previous tile's reads of D and Mt are done

    af3_f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q * 16 >= r) break;
      af3_u32x4 bw = {0u, 0u, 0u, 0u};
      if (q * 16 + jh < r) bw = *(const af3_u32x4*)(At + kcl * kMgAtP + q * 16 + jh);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(af3_bf16x8, bv[q]),
                                                    __builtin_bit_cast(af3_bf16x8, bw), acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = (w >> 1) * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      D[row * kMgDP + kcl] = acc[i] * s;
    }
    __syncthreads();

#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int nl = p * 32 + (tid >> 3);
      const bool live = n0 + nl < N && k_live;
      uint32_t m[4] = {0u, 0u, 0u, 0u};
      if (live) {
        const float4* d4 = (const float4*)(D + nl * kMgDP + kl);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float4 d = d4[c];
          const uint32_t lo = qd[p][2 * c], hi = qd[p][2 * c + 1];
          m[2 * c] = af3_pack_bf16x2(af3_bf16_to_f32(lo & 0xFFFFu) + d.x, af3_bf16_to_f32(lo >> 16) + d.y);
          m[2 * c + 1] = af3_pack_bf16x2(af3_bf16_to_f32(hi & 0xFFFFu) + d.z, af3_bf16_to_f32(hi >> 16) + d.w);
        }
      }
      if (layout == 0) {
        if (live)
          __builtin_nontemporal_store((af3_u32x4){m[0], m[1], m[2], m[3]},
                                      (af3_u32x4*)(out + ((int64_t)e * N + n0) * K + k0 + (uint32_t)(nl * K + kl)));
      } else {
        uint32_t* mrow = (uint32_t*)(Mt + nl * kMgMP + kl);
#pragma unroll
        for (int c = 0; c < 4; ++c) mrow[c] = m[c];
      }
    }
    if (layout != 0) {
      __syncthreads();
      const int nt = (tid & 7) * 8;
      uint16_t* ot = out + ((int64_t)e * K + k0) * N + n0;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int kt = p * 32 + (tid >> 3);
        if (k0 + kt >= K) break;
        uint32_t t4[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          t4[c] = (uint32_t)Mt[(nt + 2 * c) * kMgMP + kt] | ((uint32_t)Mt[(nt + 2 * c + 1) * kMgMP + kt] << 16);
        uint16_t* o = ot + (uint32_t)(kt * N + nt);
        if ((N & 7) == 0 && n0 + nt + 8 <= N) {
          __builtin_nontemporal_store((af3_u32x4){t4[0], t4[1], t4[2], t4[3]}, (af3_u32x4*)o);
        } else {
          for (int c = 0; c < 8 && n0 + nt + c < N; ++c) o[c] = (uint16_t)(t4[c >> 1] >> (16 * (c & 1)));
        }
      }
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      v[p] = vn[p];
      sc[p] = scn[p];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = bvn[q];
  }
}

}  // namespace

extern "C" int af3_mxfp4_lora_merge(const uint8_t* blocks, const uint8_t* scales, const uint16_t* lora_a,
                                    const uint16_t* lora_b, float scaling, uint16_t* out, int E, int N, int K, int r,
                                    int layout, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(E >= 0 && N >= 0 && K >= 0 && E <= 65535, "mxfp4_lora_merge: bad sizes");
  AF3_REQUIRE(K % 32 == 0, "mxfp4_lora_merge: K must be a multiple of 32 (one MXFP4 block)");
  AF3_REQUIRE(r > 0 && r % 8 == 0 && r <= 256, "mxfp4_lora_merge: rank must be a positive multiple of 8, <= 256");
  AF3_REQUIRE(layout == 0 || layout == 1, "mxfp4_lora_merge: layout must be 0 ([E,N,K]) or 1 ([E,K,N])");
  if ((int64_t)E * N * K == 0) return 0;
  AF3_REQUIRE(blocks && scales && lora_a && lora_b && out, "mxfp4_lora_merge: null pointer");
  AF3_REQUIRE(((uintptr_t)blocks & 3) == 0 && ((uintptr_t)lora_b & 15) == 0 && ((uintptr_t)lora_a & 15) == 0 &&
                  ((uintptr_t)out & 15) == 0,
              "mxfp4_lora_merge: blocks must be 4-byte, lora_a, lora_b and out 16-byte aligned");
  const int ntn = (int)af3_cdiv(N, kMgN), ntk = (int)af3_cdiv(K, kMgK);
  const int64_t tiles = (int64_t)E * ntn * ntk;
  const int64_t per_xcd = af3_cdiv(tiles, 8);
  // resident blocks per XCD: 32 CUs x 6 blocks of 26 KB LDS
  if (r <= 64) {
    const int runs = (int)af3_cdiv(ntn, kMgRun);
    const int64_t units = (int64_t)E * runs * ntk;
    AF3_REQUIRE(units <= 0x7ffffff0LL && (int64_t)kMgN * N <= 0x7fffffffLL && (int64_t)kMgK * N <= 0x7fffffffLL,
                "mxfp4_lora_merge: tensor too large");
    const int upx = (int)af3_cdiv(units, 8);
    hipLaunchKernelGGL(lora_merge_kernel, dim3((unsigned)(8 * upx)), dim3(256), 0, stream, blocks, scales, lora_a,
                       lora_b, scaling, out, N, K, r, layout, ntn, ntk, runs, (int)units, upx);
  } else {
    const int bpx = (int)(per_xcd < kMgBlocksPerXcd ? per_xcd : kMgBlocksPerXcd);
    hipLaunchKernelGGL(lora_merge_generic_kernel, dim3((unsigned)(8 * bpx)), dim3(256), 0, stream, blocks, scales,
                       lora_a, lora_b, scaling, out, N, K, r, layout, ntn, ntk, tiles, per_xcd, bpx);
  }
  return af3::check_launch("mxfp4_lora_merge");
}
