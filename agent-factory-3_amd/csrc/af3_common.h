// Shared device/host helpers for the gfx950 MXFP4 MoE expert path.
//
// Storage conventions used by every kernel in this library:
//   * bf16 tensors travel as raw 16-bit patterns (uint16_t); arithmetic is fp32.
//   * MXFP4 weights are two e2m1 nibbles per byte (low nibble = even element)
//     in 16-byte blocks of 32 elements, with one e8m0 scale byte per block.
//   * Element/byte offsets that can exceed 2^31 are computed in int64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define AF3_ABI_VERSION 2

// ---------------------------------------------------------------------------
// error reporting (host side)
// ---------------------------------------------------------------------------
namespace af3 {
void set_error(const char* fmt, ...);
int check_launch(const char* what);

// streaming expert-LoRA kernels (lora.hip); AF3_EUNSUPPORTED when the shape is
// not covered (the entry points then use the general kernels)
int lora_rows_fast(const uint16_t* x, int64_t ldx, const int32_t* gather, int gdiv, const uint16_t* wl, int trans_b,
                   float scale, const int32_t* token_offs, const int32_t* block_pid_map, int max_tiles, int n_out,
                   int K, uint16_t* out, int64_t ld_out, hipStream_t stream);
int lora_wgrad_fast(const uint16_t* big, int64_t ld_big, const int32_t* big_gather, int big_div,
                    const uint16_t* small, int64_t ld_small, const uint16_t* rowscale, int small_is_a, int W, int r,
                    float scale, const int32_t* token_offs, const int32_t* chunk_map, const int32_t* chunk_offs,
                    int max_chunks, int chunk_rows, int n_expts, float* partials, uint16_t* g, hipStream_t stream);
}  // namespace af3

// argument errors are negative, HIP errors positive (the hipError_t value)
#define AF3_EINVAL (-1)
#define AF3_EUNSUPPORTED (-2)
// OR-ed into af3_moe_gemm's tile_cfg: w_blocks is the af3_mxfp4_tile_fwd copy
#ifndef AF3_W_FWD_TILED
#define AF3_W_FWD_TILED 0x10000
#endif
// OR-ed into af3_moe_gemm's tile_cfg: every row of x the call reads lies
// within 4 GiB of x (row * ldx * 2 + K * 2 <= 2^32)
#ifndef AF3_X_OFFSETS_32
#define AF3_X_OFFSETS_32 0x20000
#endif
// OR-ed into af3_moe_gemm's tile_cfg: w_scales is the af3_mxfp4_tile_dx_scales copy
#ifndef AF3_S_DX_TILED
#define AF3_S_DX_TILED 0x40000
#endif

#define AF3_REQUIRE(cond, ...)            \
  do {                                    \
    if (!(cond)) {                        \
      af3::set_error(__VA_ARGS__);        \
      return AF3_EINVAL;                  \
    }                                     \
  } while (0)

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(2))) __bf16 af3_bf16x2;
typedef __attribute__((ext_vector_type(8))) __bf16 af3_bf16x8;
typedef __attribute__((ext_vector_type(16))) float af3_f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned int af3_u32x4;

// bf16 bits (the low 16 of h) -> fp32: exact, a shift.  Written as the bf16
// -> float conversion so the compiler treats the result as canonical and
// drops the quieting v_max it otherwise puts before every fminf / fmaxf of a
// loaded value (a signaling-NaN input then clamps to NaN instead of to the
// bound; such inputs never come out of the kernels that write these operands)
__device__ __forceinline__ float af3_bf16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(__bf16, (unsigned short)(h & 0xFFFFu));
}

// fp32 -> bf16 bits, round to nearest even (hardware v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint32_t af3_f32_to_bf16(float f) {
  __bf16 b = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(unsigned short, b);
}

// two fp32 -> one dword of bf16 (lo in bits 0-15), round to nearest even:
// one v_cvt_pk_bf16_f32 (bit-identical to two af3_f32_to_bf16)
__device__ __forceinline__ uint32_t af3_pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, af3_bf16x2));
}

// One e2m1 nibble + e8m0 scale byte -> bf16 bits, integer-only.
// Restates kernels.py:120-158 (_convert_nibble_to_bf16): normal e2m1
// (ee>0) gives bf16 exponent ee-1+S and mantissa bit6 = m; the e2m1
// subnormal (ee=0, m=1) gives exponent S-1; |n|==0, exponent > 254 and
// exponent < 1 all give a signed zero.
__device__ __forceinline__ uint32_t af3_e2m1_to_bf16_bits(uint32_t nib, uint32_t scale) {
  uint32_t sign = (nib >> 3) & 1u;
  uint32_t ee = (nib >> 1) & 3u;
  uint32_t m = nib & 1u;
  int exp = ee ? (int)(ee - 1 + scale) : (int)scale - 1;
  uint32_t mant = ee ? (m << 6) : 0u;
  uint32_t r = (sign << 15) | ((uint32_t)exp << 7) | mant;
  bool zero = ((nib & 7u) == 0u) || exp > 254 || exp < 1;
  return zero ? (sign << 15) : (r & 0xFFFFu);
}

// Four packed bytes (8 nibbles) with one scale -> 8 bf16 (4 dwords, element
// order lo0,hi0,lo1,hi1,...), exact for every scale byte 0..255.
// Scales in [2, 252] keep every exponent inside bf16's normal range, where the
// gfx950 hardware converter (v_cvt_scalef32_pk_bf16_fp4: fp4 pair * 2^(S-127))
// is exact; other scales take the integer restatement above so that the
// overflow/underflow flush-to-zero rule is honoured bit for bit.
__device__ __forceinline__ void af3_dequant_u32(uint32_t v, uint32_t scale, uint32_t out[4]) {
  if (scale - 2u <= 250u) {
    float sc = __uint_as_float(scale << 23);
    out[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 0));
    out[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 1));
    out[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 2));
    out[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 3));
  } else {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      uint32_t byte = (v >> (8 * b)) & 0xFFu;
      out[b] = af3_e2m1_to_bf16_bits(byte & 0xFu, scale) |
               (af3_e2m1_to_bf16_bits(byte >> 4, scale) << 16);
    }
  }
}

// integer-only variant of af3_dequant_u32 (used as the in-kernel cross-check
// path and for the exhaustive known-answer entry point)
__device__ __forceinline__ void af3_dequant_u32_int(uint32_t v, uint32_t scale, uint32_t out[4]) {
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    uint32_t byte = (v >> (8 * b)) & 0xFFu;
    out[b] = af3_e2m1_to_bf16_bits(byte & 0xFu, scale) |
             (af3_e2m1_to_bf16_bits(byte >> 4, scale) << 16);
  }
}

// E5M2 byte of one e2m1 nibble under e8m0 scale byte S by the reference's
// integer rule (kernels.py:21-37: exponent field ee + S - 113, mantissa m << 1
// for ee > 0; zero magnitude or an exponent below 1 gives the signed zero),
// truncated to a byte as its column-major store does (kernels.py:272-285)
__device__ __forceinline__ uint32_t af3_e2m1_to_e5m2_byte(uint32_t nib, uint32_t scale) {
  const uint32_t sign = (nib >> 3) & 1u, ee = (nib >> 1) & 3u, m = nib & 1u;
  const int exp = (int)ee + (int)scale - 113;
  const uint32_t r = (sign << 7) | ((uint32_t)exp << 2) | (ee ? (m << 1) : 0u);
  return ((nib & 7u) == 0u || exp < 1) ? (sign << 7) : (r & 0xFFu);
}

__host__ __device__ __forceinline__ int64_t af3_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// gpt-oss clamped SwiGLU per element (kernels.py:431-441 forward, 533-545
// backward): g = min(G, limit), u = clamp(U, -limit, limit),
// s = 1 / (1 + 2^(-alpha g log2 e)); out = g s (u + 1);
// dg = dO (u + 1) s (1 + alpha g (1 - s)) where g < limit, else 0;
// du = dO g s where -limit < u < limit, else 0.  exp2 is v_exp_f32 and the
// reciprocal v_rcp_f32.  Shared by the standalone SwiGLU kernels and the
// grouped-GEMM epilogues that fuse it, so both round identically.
__device__ __forceinline__ float af3_sigmoid_alpha(float g, float alpha) {
  const float e = __builtin_amdgcn_exp2f(-alpha * g * 1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ void af3_swiglu_fwd_elem(float graw, float uraw, float alpha, float limit, float& out,
                                                    float& g, float& u) {
  g = fminf(graw, limit);
  u = fminf(fmaxf(uraw, -limit), limit);
  const float s = af3_sigmoid_alpha(g, alpha);
  out = g * s * (u + 1.0f);
}

__device__ __forceinline__ void af3_swiglu_bwd_elem(float dout, float g, float u, float alpha, float limit, float& dg,
                                                    float& du) {
  const float s = af3_sigmoid_alpha(g, alpha);
  dg = dout * (u + 1.0f) * s * (1.0f + alpha * g * (1.0f - s));
  dg = (g < limit) ? dg : 0.0f;
  du = dout * g * s;
  du = (fabsf(u) < limit) ? du : 0.0f;  // -limit < u < limit (false for NaN either way)
}
