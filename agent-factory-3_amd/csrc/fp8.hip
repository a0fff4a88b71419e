// fp8 mode of the expert path (dequant_dtype="fp8"):
//   * MXFP4 -> fp8 E5M2 dequantisation, row-major and column-major, with the
//     reference's integer rule (kernels.py:20-37) bit for bit, including what
//     it does for scale bytes whose E5M2 exponent leaves the format;
//   * per-token dynamic quantisation of bf16 activations to fp8 E4M3FN with a
//     per-row fp32 scale (kernels.py:343-388).
// The fp8 grouped GEMM itself runs through the MXFP4 grouped GEMM: E4M3 codes
// are exact in bf16 and the E5M2 weights equal the MXFP4 values, so the
// products are the same; the per-row scale is applied to the accumulator in
// the epilogue (af3_moe_gemm_rowscale).
#include "af3_common.h"

namespace {

// E2M1 nibble + e8m0 byte -> E5M2 bits as the reference computes them in
// int32 (kernels.py:21-37): exponent field ee + S - 113, mantissa m << 1 for
// ee > 0; |n| == 0 or exponent < 1 -> signed zero.  The exponent is not
// clamped above: for S > 140 the result spills past 8 bits, and the callers
// truncate the way the reference's stores do.
__device__ __forceinline__ uint32_t f8_e5m2_bits(uint32_t nib, int scale_adj) {
  const uint32_t sign = (nib >> 3) & 1u, ee = (nib >> 1) & 3u, m = nib & 1u;
  const int exp = (int)ee + scale_adj;
  const uint32_t mant = ee ? (m << 1) : 0u;
  uint32_t r = (sign << 7) | ((uint32_t)exp << 2) | mant;
  if ((nib & 7u) == 0u || exp < 1) r = sign << 7;
  return r;
}

// row-major: group g, byte j -> out[g][2j] (lo nibble), out[g][2j+1] (hi), as
// the uint16 (lo | hi << 8) the reference stores (kernels.py:80-84).  A lane
// converts 4 packed bytes into one 8-byte store, four words per lane; scale
// bytes 114..141 take a byte-table path, the others the integer rule above.
__device__ __forceinline__ void e5m2_word(uint32_t v, uint32_t S, uint32_t& o0, uint32_t& o1) {
  if (S - 114u <= 27u) {
    // every nonzero code lands inside E5M2 (exponent 1..31): the magnitude byte is a
    // table of the 3-bit code, (S - 113) * 4 + {0, 0, 4, 6, 8, 10, 12, 14} (0 for
    // code 0), looked up for four nibbles at once with v_perm_b32; the sign bit is
    // the nibble's bit 3 moved to bit 7
    const uint32_t a = (S - 113u) << 2;
    const uint32_t tlo = a * 0x01010100u + 0x06040000u, thi = a * 0x01010101u + 0x0E0C0A08u;
    const uint32_t lo = __builtin_amdgcn_perm(thi, tlo, v & 0x07070707u) | ((v & 0x08080808u) << 4);
    const uint32_t hi = __builtin_amdgcn_perm(thi, tlo, (v >> 4) & 0x07070707u) | (v & 0x80808080u);
    o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    return;
  }
  const int adj = (int)S - 113;
  uint32_t h[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t byte = (v >> (8 * b)) & 0xFFu;
    h[b] = (f8_e5m2_bits(byte & 0xFu, adj) | (f8_e5m2_bits(byte >> 4, adj) << 8)) & 0xFFFFu;
  }
  o0 = h[0] | (h[1] << 16);
  o1 = h[2] | (h[3] << 16);
}

constexpr int kE5Words = 4;

__global__ __launch_bounds__(256) void e5m2_rows_kernel(const uint32_t* __restrict__ blocks,
                                                       const uint8_t* __restrict__ scales, uint2* __restrict__ out,
                                                       int64_t n_words) {
  typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
  const int64_t base = (int64_t)blockIdx.x * (256 * kE5Words) + threadIdx.x;
  uint32_t v[kE5Words], S[kE5Words];
#pragma unroll
  for (int i = 0; i < kE5Words; ++i) {
    const int64_t w = base + (int64_t)i * 256;
    const bool ok = w < n_words;
    v[i] = ok ? __builtin_nontemporal_load(blocks + w) : 0u;
    S[i] = ok ? (uint32_t)scales[w >> 2] : 127u;
  }
#pragma unroll
  for (int i = 0; i < kE5Words; ++i) {
    const int64_t w = base + (int64_t)i * 256;
    if (w >= n_words) break;
    uint32_t o0, o1;
    e5m2_word(v[i], S[i], o0, o1);
    __builtin_nontemporal_store((u32x2){o0, o1}, (u32x2*)(out + w));
  }
}

// column-major: out[e][k][n] (n contiguous), each value truncated to a byte
// (kernels.py:272-285).  A block takes 256 weight rows n of one (expert,
// group); a lane converts its row's 16-byte block and writes one byte per k
// row, so every store instruction writes 64 consecutive n.
__global__ __launch_bounds__(256) void e5m2_cols_kernel(const uint8_t* __restrict__ blocks,
                                                       const uint8_t* __restrict__ scales, uint8_t* __restrict__ out,
                                                       int N, int G) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int g = blockIdx.y, e = blockIdx.z;
  if (n >= N) return;
  const int64_t row = (int64_t)e * N + n;
  const af3_u32x4 blk = *(const af3_u32x4*)(blocks + (row * G + g) * 16);
  const int adj = (int)scales[row * G + g] - 113;
  const int64_t K = (int64_t)G * 32;
  uint8_t* o = out + (int64_t)e * K * N + (int64_t)(g * 32) * N + n;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (blk[q] >> (8 * b)) & 0xFFu;
      const int k = 2 * (4 * q + b);
      o[(int64_t)k * N] = (uint8_t)f8_e5m2_bits(byte & 0xFu, adj);
      o[(int64_t)(k + 1) * N] = (uint8_t)f8_e5m2_bits(byte >> 4, adj);
    }
  }
}

// fp32 -> fp8 E4M3FN (bias 7, no infinities, 0x7F = NaN, largest finite 448),
// round to nearest even, saturating at +-448: the conversion of kernels.py:383
// for the values it meets.  Normal results drop 20 mantissa bits of the
// rebiased fp32 pattern with round-to-nearest-even; results below 2^-6 are
// multiples of 2^-9, rounded with v_rndne_f32 on the exact product by 512.
__device__ __forceinline__ uint32_t f8_e4m3_rne_sat(float v) {
  // every case computed and selected (no divergent branches in the caller's loop)
  const uint32_t u = __float_as_uint(v);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t sub = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);  // |v| < 2^-6: 0..8 (8 = 0x08)
  const uint32_t nrm = ((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - (120u << 3);  // RNE to 3 mantissa bits, rebias
  uint32_t r = a < 0x3C800000u ? sub : nrm;
  r = a >= 0x43E80000u ? 0x7Eu : r;  // >= 464 (and inf): saturate to 448
  r = a > 0x7F800000u ? 0x7Fu : r;   // NaN
  return sign | r;
}

// E4M3FN code -> bf16 bits (exact)
__device__ __forceinline__ uint32_t f8_e4m3_to_bf16(uint32_t c) {
  const uint32_t sign = (c & 0x80u) << 8, ex = (c >> 3) & 0xFu, m = c & 7u;
  const uint32_t sub = __float_as_uint((float)m * (1.0f / 512.0f)) >> 16;  // exact; 0 for m = 0
  const uint32_t nrm = ((ex + 120u) << 7) | (m << 4);
  return sign | (ex == 0 ? sub : nrm);
}

// Four values -> their E4M3FN codes in bytes 0..3 (v_cvt_pk_fp8_f32: round to
// nearest even, subnormals kept; equal to f8_e4m3_rne_sat for every finite value
// below 464 in magnitude, the only values the quantizer feeds it: x / scale with
// scale = amax / 448 stays within 448 (1 + 2^-22)).
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// the bf16 values of four E4M3FN codes (bytes 0..3 of w) as two bf16 pairs (exact:
// every E4M3 value is a bf16 value, so the fp32 conversion's high half is it)
__device__ __forceinline__ void e4m3x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false), b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  lo = __builtin_amdgcn_perm(__float_as_uint(a[1]), __float_as_uint(a[0]), 0x07060302u);
  hi = __builtin_amdgcn_perm(__float_as_uint(b[1]), __float_as_uint(b[0]), 0x07060302u);
}

// One row per block: amax over the row (fp32), scale = max(amax, 1e-12) / 448,
// codes = E4M3(x * (1 / scale)).  Optionally also the codes' values as bf16
// (the activation operand of the MXFP4 grouped GEMM in fp8 mode).
// One wave per row, the whole row held in registers (up to CPL 8-element chunks
// per lane, K <= 512 * CPL): a single HBM pass, the row maximum by a wave
// shuffle reduction, then the codes from the registers.  Four rows per block.
template <int CPL>
__global__ __launch_bounds__(256) void quant_e4m3_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M,
                                                              int K, uint8_t* __restrict__ out, int64_t ld_out,
                                                              float* __restrict__ scale,
                                                              uint16_t* __restrict__ out_bf16, int64_t ld_bf16) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int nch = K >> 3;
  const uint16_t* xr = x + row * ldx;
  af3_u32x4 v[CPL];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    v[j] = c < nch ? __builtin_nontemporal_load((const af3_u32x4*)(xr + c * 8)) : (af3_u32x4){0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int h = 0; h < 4; ++h)
      amax = fmaxf(amax, fmaxf(fabsf(af3_bf16_to_f32(v[j][h] & 0xFFFFu)), fabsf(af3_bf16_to_f32(v[j][h] >> 16))));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const float sc = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
  const float inv = __fdiv_rn(1.0f, sc);
  if (lane == 0) scale[row] = sc;
  uint8_t* orow = out + row * ld_out;
  uint16_t* brow = out_bf16 ? out_bf16 + row * ld_bf16 : nullptr;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c >= nch) break;
    float f[8];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      f[2 * h] = af3_bf16_to_f32(v[j][h] & 0xFFFFu) * inv;
      f[2 * h + 1] = af3_bf16_to_f32(v[j][h] >> 16) * inv;
    }
    const uint32_t w0 = e4m3x4(f[0], f[1], f[2], f[3]), w1 = e4m3x4(f[4], f[5], f[6], f[7]);
    typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
    __builtin_nontemporal_store((u32x2){w0, w1}, (u32x2*)(orow + c * 8));
    if (brow) {
      uint32_t b0, b1, b2, b3;
      e4m3x4_to_bf16(w0, b0, b1);
      e4m3x4_to_bf16(w1, b2, b3);
      __builtin_nontemporal_store(af3_u32x4{b0, b1, b2, b3}, (af3_u32x4*)(brow + c * 8));
    }
  }
}

__global__ __launch_bounds__(256) void quant_e4m3_kernel(const uint16_t* __restrict__ x, int64_t ldx, int K,
                                                        uint8_t* __restrict__ out, int64_t ld_out,
                                                        float* __restrict__ scale, uint16_t* __restrict__ out_bf16,
                                                        int64_t ld_bf16) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  float amax = 0.f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    if (k + 8 <= K) {
      const af3_u32x4 v = *(const af3_u32x4*)(xr + k);
#pragma unroll
      for (int h = 0; h < 4; ++h)
        amax = fmaxf(amax, fmaxf(fabsf(af3_bf16_to_f32(v[h] & 0xFFFFu)), fabsf(af3_bf16_to_f32(v[h] >> 16))));
    } else {
      for (int j = k; j < K; ++j) amax = fmaxf(amax, fabsf(af3_bf16_to_f32(xr[j])));
    }
  }
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
  const float inv = __fdiv_rn(1.0f, sc);
  if (threadIdx.x == 0) scale[row] = sc;
  uint8_t* orow = out + row * ld_out;
  uint16_t* brow = out_bf16 ? out_bf16 + row * ld_bf16 : nullptr;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    const int n = min(8, K - k);
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = j < n ? f8_e4m3_rne_sat(af3_bf16_to_f32(xr[k + j]) * inv) : 0u;
    if (n == 8) {
      *(uint2*)(orow + k) = uint2{c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                                  c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)};
      if (brow)
        *(af3_u32x4*)(brow + k) = af3_u32x4{f8_e4m3_to_bf16(c[0]) | (f8_e4m3_to_bf16(c[1]) << 16),
                                            f8_e4m3_to_bf16(c[2]) | (f8_e4m3_to_bf16(c[3]) << 16),
                                            f8_e4m3_to_bf16(c[4]) | (f8_e4m3_to_bf16(c[5]) << 16),
                                            f8_e4m3_to_bf16(c[6]) | (f8_e4m3_to_bf16(c[7]) << 16)};
    } else {
      for (int j = 0; j < n; ++j) {
        orow[k + j] = (uint8_t)c[j];
        if (brow) brow[k + j] = (uint16_t)f8_e4m3_to_bf16(c[j]);
      }
    }
  }
}

}  // namespace

extern "C" int af3_mxfp4_to_fp8_e5m2(const uint8_t* blocks, const uint8_t* scales, uint8_t* out, int64_t n_groups,
                                     void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_groups >= 0, "mxfp4_to_fp8_e5m2: n_groups must be >= 0");
  if (n_groups == 0) return 0;
  AF3_REQUIRE(blocks && scales && out, "mxfp4_to_fp8_e5m2: null pointer");
  AF3_REQUIRE(((uintptr_t)blocks & 3) == 0 && ((uintptr_t)out & 7) == 0,
              "mxfp4_to_fp8_e5m2: blocks must be 4-byte and out 8-byte aligned");
  const int64_t n_words = n_groups * 4;
  const int64_t grid = af3_cdiv(n_words, 256 * kE5Words);
  AF3_REQUIRE(grid <= 0x7fffffffLL, "mxfp4_to_fp8_e5m2: tensor too large");
  hipLaunchKernelGGL(e5m2_rows_kernel, dim3((unsigned)grid), dim3(256), 0, stream, (const uint32_t*)blocks, scales,
                     (uint2*)out, n_words);
  return af3::check_launch("mxfp4_to_fp8_e5m2");
}

extern "C" int af3_mxfp4_to_fp8_e5m2_colmajor(const uint8_t* blocks, const uint8_t* scales, uint8_t* out, int E,
                                              int N, int G, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(E >= 0 && N >= 0 && G >= 0 && G <= 65535 && E <= 65535, "mxfp4_to_fp8_e5m2_colmajor: bad sizes");
  if ((int64_t)E * N * G == 0) return 0;
  AF3_REQUIRE(blocks && scales && out && ((uintptr_t)blocks & 15) == 0,
              "mxfp4_to_fp8_e5m2_colmajor: null pointer or blocks not 16-byte aligned");
  hipLaunchKernelGGL(e5m2_cols_kernel, dim3((unsigned)af3_cdiv(N, 256), G, E), dim3(256), 0, stream, blocks, scales,
                     out, N, G);
  return af3::check_launch("mxfp4_to_fp8_e5m2_colmajor");
}

extern "C" int af3_quantize_per_token_e4m3(const uint16_t* x, int64_t ldx, int64_t M, int K, uint8_t* out,
                                           int64_t ld_out, float* scale, uint16_t* out_bf16, int64_t ld_bf16,
                                           void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M >= 0 && K > 0, "quantize_per_token_e4m3: bad sizes");
  if (M == 0) return 0;
  AF3_REQUIRE(x && out && scale, "quantize_per_token_e4m3: null pointer");
  AF3_REQUIRE(ldx % 8 == 0 && ((uintptr_t)x & 15) == 0 && ld_out % 8 == 0 && ((uintptr_t)out & 7) == 0 &&
                  (!out_bf16 || (ld_bf16 % 8 == 0 && ((uintptr_t)out_bf16 & 15) == 0)),
              "quantize_per_token_e4m3: rows must be 16-byte aligned (bf16) / 8-byte aligned (fp8)");
  AF3_REQUIRE(M <= 0x7fffffffLL, "quantize_per_token_e4m3: too many rows");
  if (K % 8 == 0 && K <= 512 * 12) {
    const unsigned grid = (unsigned)af3_cdiv(M, 4);
    if (K <= 512 * 6)
      hipLaunchKernelGGL(quant_e4m3_rows_kernel<6>, dim3(grid), dim3(256), 0, stream, x, ldx, M, K, out, ld_out,
                         scale, out_bf16, ld_bf16);
    else
      hipLaunchKernelGGL(quant_e4m3_rows_kernel<12>, dim3(grid), dim3(256), 0, stream, x, ldx, M, K, out, ld_out,
                         scale, out_bf16, ld_bf16);
  } else {
    hipLaunchKernelGGL(quant_e4m3_kernel, dim3((unsigned)M), dim3(256), 0, stream, x, ldx, K, out, ld_out, scale,
                       out_bf16, ld_bf16);
  }
  return af3::check_launch("quantize_per_token_e4m3");
}
