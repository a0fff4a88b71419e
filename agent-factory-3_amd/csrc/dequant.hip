// MXFP4 -> bf16 dequantisation (standalone, HBM-bound).
//
// Reference behaviour: kernels.py:161-235 (_mxfp4_to_bf16_kernel /
// mxfp4_to_bf16_triton): byte j of a 16-byte block g becomes output elements
// 32g+2j (low nibble) and 32g+2j+1 (high nibble), scaled by the block's e8m0
// byte, with the flush-to-zero rule of kernels.py:137-158.
//
// Layout: one lane owns one 4-byte word of packed nibbles (8 outputs, one
// 16-byte store).  Consecutive lanes own consecutive words, so every load is a
// 256-byte contiguous wave access and every store a 1 KiB contiguous one.  The
// scale byte is shared by the four lanes of a block.
#include "af3_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWordsPerThread = 8;

__global__ __launch_bounds__(kThreads) void mxfp4_to_bf16_kernel(const uint32_t* __restrict__ blocks,
                                                                 const uint8_t* __restrict__ scales,
                                                                 af3_u32x4* __restrict__ out,
                                                                 int64_t n_words) {
  const int64_t base = (int64_t)blockIdx.x * (kThreads * kWordsPerThread) + threadIdx.x;
  uint32_t w[kWordsPerThread];
  uint32_t s[kWordsPerThread];
#pragma unroll
  for (int i = 0; i < kWordsPerThread; ++i) {
    int64_t idx = base + (int64_t)i * kThreads;
    bool ok = idx < n_words;
    w[i] = ok ? __builtin_nontemporal_load(blocks + idx) : 0u;
    s[i] = ok ? (uint32_t)scales[idx >> 2] : 127u;
  }
#pragma unroll
  for (int i = 0; i < kWordsPerThread; ++i) {
    int64_t idx = base + (int64_t)i * kThreads;
    if (idx < n_words) {
      uint32_t o[4];
      af3_dequant_u32(w[i], s[i], o);
      af3_u32x4 v = {o[0], o[1], o[2], o[3]};
      __builtin_nontemporal_store(v, out + idx);
    }
  }
}

}  // namespace

extern "C" int af3_mxfp4_to_bf16(const uint8_t* blocks, const uint8_t* scales, uint16_t* out,
                                 int64_t n_groups, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_groups >= 0, "mxfp4_to_bf16: n_groups must be >= 0 (got %lld)", (long long)n_groups);
  if (n_groups == 0) return 0;
  AF3_REQUIRE(blocks && scales && out, "mxfp4_to_bf16: null pointer");
  AF3_REQUIRE(((uintptr_t)blocks & 3) == 0, "mxfp4_to_bf16: blocks must be 4-byte aligned");
  AF3_REQUIRE(((uintptr_t)out & 15) == 0, "mxfp4_to_bf16: out must be 16-byte aligned");
  const int64_t n_words = n_groups * 4;
  const int64_t per_block = kThreads * kWordsPerThread;
  const int64_t grid = af3_cdiv(n_words, per_block);
  AF3_REQUIRE(grid <= 0x7fffffffLL, "mxfp4_to_bf16: tensor too large");
  hipLaunchKernelGGL(mxfp4_to_bf16_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                       (const uint32_t*)blocks, scales, (af3_u32x4*)out, n_words);
  return af3::check_launch("mxfp4_to_bf16");
}
