// gpt-oss clamped SwiGLU, forward and backward (HBM-bound elementwise).
//
// Reference behaviour:
//   forward  kernels.py:394-490 (_swiglu_fwd_kernel / _swiglu_forward_triton):
//     g = min(G, limit), u = clamp(U, -limit, limit),
//     s = 1 / (1 + 2^(-alpha*g*log2 e)), out = g*s*(u+1)   (fp32, stored bf16)
//     input is interleaved [.., 2N] (even = gate, odd = up); optionally stores
//     the clamped g and u for backward.
//   backward kernels.py:493-582 (_swiglu_bwd_kernel / _swiglu_backward):
//     dg = dO*(u+1)*s*(1 + alpha*g*(1-s))  where g < limit, else 0
//     du = dO*g*s                          where -limit < u < limit, else 0
//     output interleaved [.., 2N] bf16.
// The backward exists in two forms: from the saved clamped (g, u) pair (the
// reference's form) and from the raw interleaved pre-activation, which lets
// the autograd function keep the GEMM output instead of writing g and u.
//
// exp2 is v_exp_f32 and the reciprocal v_rcp_f32 (both about 1 ulp); the
// reference uses an approximate ex2 too, so results agree to bf16 tolerance.
//
// Vector path: one lane owns 8 consecutive output columns of one row (16-byte
// loads/stores; the interleaved input is two 16-byte loads).  Rows may have a
// stride; every row offset is int64.
#include "af3_common.h"

namespace {

constexpr int kThreads = 256;
__device__ __forceinline__ void swiglu_fwd_elem(float graw, float uraw, float alpha, float limit, float& out,
                                                float& g, float& u) {
  af3_swiglu_fwd_elem(graw, uraw, alpha, limit, out, g, u);
}

__device__ __forceinline__ void swiglu_bwd_elem(float dout, float g, float u, float alpha, float limit, float& dg,
                                                float& du) {
  af3_swiglu_bwd_elem(dout, g, u, alpha, limit, dg, du);
}

// ---- forward ---------------------------------------------------------------
template <bool kSave>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_vec8(const uint16_t* __restrict__ in, int64_t ld_in,
                                                            uint16_t* __restrict__ out, int64_t ld_out,
                                                            uint16_t* __restrict__ gsave,
                                                            uint16_t* __restrict__ usave, int64_t ld_save,
                                                            uint32_t vec_per_row, uint32_t n_vec, float alpha,
                                                            float limit) {
  uint32_t v = blockIdx.x * kThreads + threadIdx.x;
  if (v >= n_vec) return;
  uint32_t row = v / vec_per_row;
  uint32_t c8 = (v - row * vec_per_row) * 8;
  const af3_u32x4* src = (const af3_u32x4*)(in + (int64_t)row * ld_in + 2 * (int64_t)c8);
  af3_u32x4 a = __builtin_nontemporal_load(src);
  af3_u32x4 b = __builtin_nontemporal_load(src + 1);
  uint32_t words[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t o[4], go[4], uo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float r0, r1, g0, g1, u0, u1;
    uint32_t w0 = words[2 * i], w1 = words[2 * i + 1];
    swiglu_fwd_elem(af3_bf16_to_f32(w0 & 0xFFFFu), af3_bf16_to_f32(w0 >> 16), alpha, limit, r0, g0, u0);
    swiglu_fwd_elem(af3_bf16_to_f32(w1 & 0xFFFFu), af3_bf16_to_f32(w1 >> 16), alpha, limit, r1, g1, u1);
    o[i] = af3_pack_bf16x2(r0, r1);
    if (kSave) {
      go[i] = af3_pack_bf16x2(g0, g1);
      uo[i] = af3_pack_bf16x2(u0, u1);
    }
  }
  int64_t ooff = (int64_t)row * ld_out + c8;
  af3_u32x4 ov = {o[0], o[1], o[2], o[3]};
  *(af3_u32x4*)(out + ooff) = ov;
  if (kSave) {
    int64_t soff = (int64_t)row * ld_save + c8;
    af3_u32x4 gv = {go[0], go[1], go[2], go[3]};
    af3_u32x4 uv = {uo[0], uo[1], uo[2], uo[3]};
    *(af3_u32x4*)(gsave + soff) = gv;
    *(af3_u32x4*)(usave + soff) = uv;
  }
}

__global__ __launch_bounds__(kThreads) void swiglu_fwd_scalar(const uint16_t* __restrict__ in, int64_t ld_in,
                                                              uint16_t* __restrict__ out, int64_t ld_out,
                                                              uint16_t* __restrict__ gsave,
                                                              uint16_t* __restrict__ usave, int64_t ld_save,
                                                              int64_t M, int64_t N, float alpha, float limit) {
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= M * N) return;
  int64_t row = i / N, col = i - row * N;
  const uint16_t* p = in + row * ld_in + 2 * col;
  float r, g, u;
  swiglu_fwd_elem(af3_bf16_to_f32(p[0]), af3_bf16_to_f32(p[1]), alpha, limit, r, g, u);
  out[row * ld_out + col] = (uint16_t)af3_f32_to_bf16(r);
  if (gsave) {
    gsave[row * ld_save + col] = (uint16_t)af3_f32_to_bf16(g);
    usave[row * ld_save + col] = (uint16_t)af3_f32_to_bf16(u);
  }
}

// ---- backward --------------------------------------------------------------
// kRaw: gate/up come from the raw interleaved pre-activation (clamped here);
// otherwise from the saved clamped tensors.
template <bool kRaw>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_vec8(const uint16_t* __restrict__ dout, int64_t ld_dout,
                                                            const uint16_t* __restrict__ a_ptr,
                                                            const uint16_t* __restrict__ b_ptr, int64_t ld_ab,
                                                            uint16_t* __restrict__ dgu, int64_t ld_dgu,
                                                            uint32_t vec_per_row, uint32_t n_vec, float alpha,
                                                            float limit) {
  uint32_t v = blockIdx.x * kThreads + threadIdx.x;
  if (v >= n_vec) return;
  uint32_t row = v / vec_per_row;
  uint32_t c8 = (v - row * vec_per_row) * 8;
  af3_u32x4 d = __builtin_nontemporal_load((const af3_u32x4*)(dout + (int64_t)row * ld_dout + c8));
  float g[8], u[8];
  if (kRaw) {
    const af3_u32x4* src = (const af3_u32x4*)(a_ptr + (int64_t)row * ld_ab + 2 * (int64_t)c8);
    af3_u32x4 x0 = __builtin_nontemporal_load(src);
    af3_u32x4 x1 = __builtin_nontemporal_load(src + 1);
    uint32_t w[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      g[i] = fminf(af3_bf16_to_f32(w[i] & 0xFFFFu), limit);
      u[i] = fminf(fmaxf(af3_bf16_to_f32(w[i] >> 16), -limit), limit);
    }
  } else {
    int64_t off = (int64_t)row * ld_ab + c8;
    af3_u32x4 gv = __builtin_nontemporal_load((const af3_u32x4*)(a_ptr + off));
    af3_u32x4 uv = __builtin_nontemporal_load((const af3_u32x4*)(b_ptr + off));
    uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g[2 * i] = af3_bf16_to_f32(gw[i] & 0xFFFFu);
      g[2 * i + 1] = af3_bf16_to_f32(gw[i] >> 16);
      u[2 * i] = af3_bf16_to_f32(uw[i] & 0xFFFFu);
      u[2 * i + 1] = af3_bf16_to_f32(uw[i] >> 16);
    }
  }
  uint32_t dw[4] = {d.x, d.y, d.z, d.w};
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float dd = af3_bf16_to_f32(i & 1 ? dw[i >> 1] >> 16 : dw[i >> 1] & 0xFFFFu);
    float dg, du;
    swiglu_bwd_elem(dd, g[i], u[i], alpha, limit, dg, du);
    o[i] = af3_pack_bf16x2(dg, du);
  }
  af3_u32x4* dst = (af3_u32x4*)(dgu + (int64_t)row * ld_dgu + 2 * (int64_t)c8);
  af3_u32x4 o0 = {o[0], o[1], o[2], o[3]}, o1 = {o[4], o[5], o[6], o[7]};
  dst[0] = o0;
  dst[1] = o1;
}

template <bool kRaw>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_scalar(const uint16_t* __restrict__ dout, int64_t ld_dout,
                                                              const uint16_t* __restrict__ a_ptr,
                                                              const uint16_t* __restrict__ b_ptr, int64_t ld_ab,
                                                              uint16_t* __restrict__ dgu, int64_t ld_dgu,
                                                              int64_t M, int64_t N, float alpha, float limit) {
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= M * N) return;
  int64_t row = i / N, col = i - row * N;
  float g, u;
  if (kRaw) {
    const uint16_t* p = a_ptr + row * ld_ab + 2 * col;
    g = fminf(af3_bf16_to_f32(p[0]), limit);
    u = fminf(fmaxf(af3_bf16_to_f32(p[1]), -limit), limit);
  } else {
    g = af3_bf16_to_f32(a_ptr[row * ld_ab + col]);
    u = af3_bf16_to_f32(b_ptr[row * ld_ab + col]);
  }
  float dg, du;
  swiglu_bwd_elem(af3_bf16_to_f32(dout[row * ld_dout + col]), g, u, alpha, limit, dg, du);
  uint16_t* q = dgu + row * ld_dgu + 2 * col;
  q[0] = (uint16_t)af3_f32_to_bf16(dg);
  q[1] = (uint16_t)af3_f32_to_bf16(du);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int af3_swiglu_fwd(const uint16_t* gate_up, int64_t ld_in, uint16_t* out, int64_t ld_out,
                              uint16_t* gate_save, uint16_t* up_save, int64_t ld_save, int64_t M, int64_t N,
                              float alpha, float limit, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(M >= 0 && N >= 0, "swiglu_fwd: negative shape");
  if (M == 0 || N == 0) return 0;
  AF3_REQUIRE(gate_up && out, "swiglu_fwd: null pointer");
  AF3_REQUIRE((gate_save == nullptr) == (up_save == nullptr), "swiglu_fwd: gate_save/up_save must both be set");
  AF3_REQUIRE(ld_in >= 2 * N && ld_out >= N && (!gate_save || ld_save >= N), "swiglu_fwd: bad leading dims");
  const bool save = gate_save != nullptr;
  const bool vec = (N % 8 == 0) && (ld_in % 8 == 0) && (ld_out % 8 == 0) && aligned16(gate_up) &&
                   aligned16(out) && (!save || (ld_save % 8 == 0 && aligned16(gate_save) && aligned16(up_save))) &&
                   (M * (N / 8) < 0xffffffffLL);
  if (vec) {
    uint32_t vpr = (uint32_t)(N / 8);
    uint32_t nv = (uint32_t)(M * (N / 8));
    dim3 grid((unsigned)af3_cdiv(nv, kThreads));
    if (save)
      hipLaunchKernelGGL(swiglu_fwd_vec8<true>, grid, dim3(kThreads), 0, stream, gate_up, ld_in, out, ld_out,
                         gate_save, up_save, ld_save, vpr, nv, alpha, limit);
    else
      hipLaunchKernelGGL(swiglu_fwd_vec8<false>, grid, dim3(kThreads), 0, stream, gate_up, ld_in, out, ld_out,
                         gate_save, up_save, ld_save, vpr, nv, alpha, limit);
  } else {
    int64_t grid = af3_cdiv(M * N, kThreads);
    AF3_REQUIRE(grid <= 0x7fffffffLL, "swiglu_fwd: tensor too large");
    hipLaunchKernelGGL(swiglu_fwd_scalar, dim3((unsigned)grid), dim3(kThreads), 0, stream, gate_up, ld_in, out,
                       ld_out, gate_save, up_save, ld_save, M, N, alpha, limit);
  }
  return af3::check_launch("swiglu_fwd");
}

static int swiglu_bwd_common(bool raw, const uint16_t* dout, int64_t ld_dout, const uint16_t* a,
                             const uint16_t* b, int64_t ld_ab, uint16_t* dgu, int64_t ld_dgu, int64_t M,
                             int64_t N, float alpha, float limit, hipStream_t stream) {
  AF3_REQUIRE(M >= 0 && N >= 0, "swiglu_bwd: negative shape");
  if (M == 0 || N == 0) return 0;
  AF3_REQUIRE(dout && a && dgu && (raw || b), "swiglu_bwd: null pointer");
  AF3_REQUIRE(ld_dout >= N && ld_dgu >= 2 * N && ld_ab >= (raw ? 2 * N : N), "swiglu_bwd: bad leading dims");
  const bool vec = (N % 8 == 0) && (ld_dout % 8 == 0) && (ld_ab % 8 == 0) && (ld_dgu % 8 == 0) &&
                   aligned16(dout) && aligned16(a) && (raw || aligned16(b)) && aligned16(dgu) &&
                   (M * (N / 8) < 0xffffffffLL);
  if (vec) {
    uint32_t vpr = (uint32_t)(N / 8);
    uint32_t nv = (uint32_t)(M * (N / 8));
    dim3 grid((unsigned)af3_cdiv(nv, kThreads));
    if (raw)
      hipLaunchKernelGGL(swiglu_bwd_vec8<true>, grid, dim3(kThreads), 0, stream, dout, ld_dout, a, b, ld_ab, dgu,
                         ld_dgu, vpr, nv, alpha, limit);
    else
      hipLaunchKernelGGL(swiglu_bwd_vec8<false>, grid, dim3(kThreads), 0, stream, dout, ld_dout, a, b, ld_ab, dgu,
                         ld_dgu, vpr, nv, alpha, limit);
  } else {
    int64_t grid = af3_cdiv(M * N, kThreads);
    AF3_REQUIRE(grid <= 0x7fffffffLL, "swiglu_bwd: tensor too large");
    if (raw)
      hipLaunchKernelGGL(swiglu_bwd_scalar<true>, dim3((unsigned)grid), dim3(kThreads), 0, stream, dout, ld_dout,
                         a, b, ld_ab, dgu, ld_dgu, M, N, alpha, limit);
    else
      hipLaunchKernelGGL(swiglu_bwd_scalar<false>, dim3((unsigned)grid), dim3(kThreads), 0, stream, dout,
                         ld_dout, a, b, ld_ab, dgu, ld_dgu, M, N, alpha, limit);
  }
  return af3::check_launch("swiglu_bwd");
}

extern "C" int af3_swiglu_bwd(const uint16_t* grad_out, int64_t ld_grad, const uint16_t* gate,
                              const uint16_t* up, int64_t ld_save, uint16_t* grad_gu, int64_t ld_gu, int64_t M,
                              int64_t N, float alpha, float limit, void* stream) {
  return swiglu_bwd_common(false, grad_out, ld_grad, gate, up, ld_save, grad_gu, ld_gu, M, N, alpha, limit,
                           (hipStream_t)stream);
}

extern "C" int af3_swiglu_bwd_raw(const uint16_t* grad_out, int64_t ld_grad, const uint16_t* gate_up,
                                  int64_t ld_in, uint16_t* grad_gu, int64_t ld_gu, int64_t M, int64_t N,
                                  float alpha, float limit, void* stream) {
  return swiglu_bwd_common(true, grad_out, ld_grad, gate_up, nullptr, ld_in, grad_gu, ld_gu, M, N, alpha, limit,
                           (hipStream_t)stream);
}
