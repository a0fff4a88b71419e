// Token -> expert permutation (routing metadata) for the grouped expert GEMMs.
//
// Reference behaviour:
//   routing_replay   quantization.py:593-636: softmax over the K gathered
//                    logits of each token; stable sort of the flat [T*K]
//                    expert ids; gate_indx = inverse permutation; gate_scal =
//                    softmax weights in sorted order; hist = bincount.
//   top-k routing    quantization.py:551-590 (routing_torch_dist at world size
//                    1, the torch restatement of triton_kernels' routing):
//                    top-K logits per token by a stable descending sort (ties
//                    go to the lower expert id), softmax over those K, then
//                    the K (id, weight) pairs of a token sorted by expert id.
//   expt data        triton_kernels.routing.compute_expt_data_torch (called at
//                    quantization.py:588,627): token_offs_raw = exclusive scan
//                    of hist; per block size BM, token_offs_pad = exclusive
//                    scan of ceil(hist/BM) and block_pid_map[i] = (b<<16)|e for
//                    the b-th BM-row block of expert e, -1 for unused slots.
//
// The sort is a stable counting sort: per 256-entry chunk histograms, a scan
// over (expert, chunk), then a scatter where each entry's rank among equal ids
// earlier in its chunk keeps the order of the flat index.  Entries whose
// expert id is outside [0, E) are dropped (gate_indx = -1), the same shape the
// reference gives expert-parallel-masked entries.
#include <mutex>

#include "af3_common.h"

namespace {

constexpr int kChunk = 256;

__device__ __forceinline__ uint32_t bf16_bits_rne(float f) { return af3_f32_to_bf16(f); }

// one thread per token: ids/weights of its K slots (replay form)
__global__ void replay_token_kernel(const uint16_t* __restrict__ logits, int64_t ld, const int32_t* __restrict__ idx,
                                    int64_t T, int E, int K, int32_t* __restrict__ ids,
                                    uint16_t* __restrict__ scal) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  float v[16];
  int e[16];
  float mx = -INFINITY;
  for (int j = 0; j < K; ++j) {
    e[j] = idx[t * K + j];
    bool ok = e[j] >= 0 && e[j] < E;
    v[j] = ok ? af3_bf16_to_f32(logits[t * ld + e[j]]) : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
  float den = 0.f;
  for (int j = 0; j < K; ++j) {
    v[j] = (e[j] >= 0 && e[j] < E) ? expf(v[j] - mx) : 0.f;
    den += v[j];
  }
  for (int j = 0; j < K; ++j) {
    bool ok = e[j] >= 0 && e[j] < E;
    ids[t * K + j] = ok ? e[j] : -1;
    scal[t * K + j] = (uint16_t)bf16_bits_rne(v[j] / den);
  }
}

// one thread per token: top-K selection + softmax + sort of the K by expert id
__global__ void topk_token_kernel(const uint16_t* __restrict__ logits, int64_t ld, int64_t T, int E, int K,
                                  int32_t* __restrict__ ids, uint16_t* __restrict__ scal) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  float v[16];
  int e[16];
  for (int j = 0; j < K; ++j) {
    v[j] = -INFINITY;
    e[j] = E;  // sentinel larger than any id
  }
  const uint16_t* row = logits + t * ld;
  for (int x = 0; x < E; ++x) {
    float f = af3_bf16_to_f32(row[x]);
    // strict > keeps the earlier (lower) id on ties, matching a stable sort of -logits
    if (f > v[K - 1] || (e[K - 1] == E)) {
      int p = K - 1;
      while (p > 0 && (f > v[p - 1] || e[p - 1] == E)) {
        v[p] = v[p - 1];
        e[p] = e[p - 1];
        --p;
      }
      v[p] = f;
      e[p] = x;
    }
  }
  float mx = v[0];
  float w[16], den = 0.f;
  for (int j = 0; j < K; ++j) {
    w[j] = expf(v[j] - mx);
    den += w[j];
  }
  // softmax output is rounded to the logits dtype (bf16) before reordering
  uint16_t wb[16];
  for (int j = 0; j < K; ++j) wb[j] = (uint16_t)bf16_bits_rne(w[j] / den);
  // insertion sort of the K pairs by expert id (ids are distinct)
  for (int a = 1; a < K; ++a) {
    int ek = e[a];
    uint16_t wk = wb[a];
    int b = a - 1;
    while (b >= 0 && e[b] > ek) {
      e[b + 1] = e[b];
      wb[b + 1] = wb[b];
      --b;
    }
    e[b + 1] = ek;
    wb[b + 1] = wk;
  }
  for (int j = 0; j < K; ++j) {
    ids[t * K + j] = e[j];
    scal[t * K + j] = wb[j];
  }
}

// per-chunk histogram: counts[e * n_chunks + c]
__global__ void chunk_hist_kernel(const int32_t* __restrict__ ids, int64_t R, int E, int n_chunks,
                                  int32_t* __restrict__ counts) {
  extern __shared__ int32_t sh[];
  for (int e = threadIdx.x; e < E; e += blockDim.x) sh[e] = 0;
  __syncthreads();
  int64_t i = (int64_t)blockIdx.x * kChunk + threadIdx.x;
  if (i < R) {
    int e = ids[i];
    if (e >= 0) atomicAdd(&sh[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) counts[(int64_t)e * n_chunks + blockIdx.x] = sh[e];
}

// one block per expert: exclusive scan of its per-chunk counts (in place) and hist[e]
__global__ __launch_bounds__(256) void chunk_scan_kernel(int32_t* __restrict__ counts, int n_chunks,
                                                         int32_t* __restrict__ hist) {
  __shared__ int32_t sh[256];
  const int e = blockIdx.x, t = threadIdx.x;
  int32_t* row = counts + (int64_t)e * n_chunks;
  int32_t carry = 0;
  for (int base = 0; base < n_chunks; base += 256) {
    const int c = base + t;
    const int32_t v = c < n_chunks ? row[c] : 0;
    sh[t] = v;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      int32_t add = t >= off ? sh[t - off] : 0;
      __syncthreads();
      sh[t] += add;
      __syncthreads();
    }
    if (c < n_chunks) row[c] = carry + sh[t] - v;
    carry += sh[255];
    __syncthreads();
  }
  if (t == 0) hist[e] = carry;
}

// single block: token_offs_raw = exclusive scan of hist over experts
__global__ __launch_bounds__(1024) void expert_scan_kernel(const int32_t* __restrict__ hist, int E,
                                                           int32_t* __restrict__ offs) {
  __shared__ int32_t sh[1024];
  const int t = threadIdx.x;
  int32_t carry = 0;
  for (int base = 0; base < E; base += 1024) {
    const int e = base + t;
    const int32_t v = e < E ? hist[e] : 0;
    sh[t] = v;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      int32_t add = t >= off ? sh[t - off] : 0;
      __syncthreads();
      sh[t] += add;
      __syncthreads();
    }
    if (e < E) offs[e] = carry + sh[t] - v;
    carry += sh[1023];
    __syncthreads();
  }
  if (t == 0) offs[E] = carry;
}

// stable scatter of each chunk into expert-sorted order
__global__ void scatter_kernel(const int32_t* __restrict__ ids, const uint16_t* __restrict__ scal, int64_t R,
                               int n_chunks, const int32_t* __restrict__ offs, const int32_t* __restrict__ base,
                               int32_t* __restrict__ topk_indx,
                               int32_t* __restrict__ gate_indx, uint16_t* __restrict__ gate_scal) {
  __shared__ int32_t sid[kChunk];
  int64_t i = (int64_t)blockIdx.x * kChunk + threadIdx.x;
  int e = (i < R) ? ids[i] : -1;
  sid[threadIdx.x] = e;
  __syncthreads();
  if (i >= R) return;
  if (e < 0) {
    gate_indx[i] = -1;
    return;
  }
  int rank = 0;
  for (int j = 0; j < (int)threadIdx.x; ++j) rank += (sid[j] == e);
  int32_t pos = offs[e] + base[(int64_t)e * n_chunks + blockIdx.x] + rank;
  topk_indx[pos] = (int32_t)i;
  gate_indx[i] = pos;
  gate_scal[pos] = scal[i];
}

__global__ void zero_kernel(int32_t* __restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

// sorted slots past the number of valid entries (only when some ids were dropped)
__global__ void fill_tail_kernel(const int32_t* __restrict__ offs, int E, int64_t R, int32_t* __restrict__ topk_indx,
                                 uint16_t* __restrict__ gate_scal) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R) return;
  if (i >= offs[E]) {
    topk_indx[i] = -1;
    gate_scal[i] = 0;
  }
}

// ---- expert data: padded tile offsets and block -> (block, expert) map -----
// per tile size (one 1024-thread block each): the exclusive prefix of the
// experts' tile counts -> offs_pad, then the tile -> (expert, tile) map
constexpr int kScanMaxE = 4096;

__global__ __launch_bounds__(1024) void tile_scan_map_kernel(const int32_t* __restrict__ hist, int E,
                                                             const int32_t* __restrict__ block_ms, int max_tiles,
                                                             int32_t* __restrict__ offs_pad /* n_bm x (E+1) */,
                                                             int32_t* __restrict__ map /* n_bm x max_tiles */) {
  __shared__ int32_t op[kScanMaxE + 1];
  __shared__ int32_t part[1024];
  const int b = blockIdx.x, t = threadIdx.x;
  const int bm = block_ms[b];
  // thread t owns experts [t * per, (t + 1) * per)
  const int per = (E + 1023) / 1024;
  int32_t run = 0;
  for (int i = 0; i < per; ++i) {
    const int e = t * per + i;
    if (e < E) {
      const int32_t n = (hist[e] + bm - 1) / bm;
      op[e] = n;
      run += n;
    }
  }
  part[t] = run;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int32_t pos = part[t] - run;
  for (int i = 0; i < per; ++i) {
    const int e = t * per + i;
    if (e < E) {
      const int32_t n = op[e];
      op[e] = pos;
      pos += n;
    }
  }
  if (t == 1023) op[E] = part[1023];
  __syncthreads();
  for (int e = t; e <= E; e += 1024) offs_pad[b * (E + 1) + e] = op[e];
  for (int i = t; i < max_tiles; i += 1024) {
    int32_t val = -1;
    if (i < op[E]) {
      // largest e with op[e] <= i (experts with zero tiles have op[e] == op[e+1])
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (op[mid] <= i)
          lo = mid;
        else
          hi = mid - 1;
      }
      val = ((i - op[lo]) << 16) | lo;
    }
    map[(int64_t)b * max_tiles + i] = val;
  }
}

// ---- grouped-GEMM tile order: full tiles first (expert order), then the
// experts' partial last tiles by decreasing row count (ties: lower expert first)
constexpr int kSchedMaxE = 4096;
constexpr int kSchedMaxBM = 512;

__global__ __launch_bounds__(1024) void tile_order_kernel(const int32_t* __restrict__ hist, int E, int bm,
                                                          int max_tiles, int32_t* __restrict__ order) {
  __shared__ int32_t nfull[kSchedMaxE];
  __shared__ int32_t tail[kSchedMaxE];
  __shared__ int32_t start[kSchedMaxBM + 1];  // tails of size s start at start[s]
  __shared__ int32_t part[1024];               // prefix of full-tile counts
  __shared__ int32_t suf[1024];                // suffix of the tail-size histogram
  const int t = threadIdx.x;
  for (int e = t; e < E; e += 1024) {
    const int h = hist[e];
    nfull[e] = h / bm;
    tail[e] = h % bm;
  }
  for (int s = t; s <= kSchedMaxBM; s += 1024) start[s] = 0;
  __syncthreads();
  for (int e = t; e < E; e += 1024)
    if (tail[e]) atomicAdd(&start[tail[e]], 1);
  // exclusive prefix of full-tile counts over experts: thread t owns experts
  // [t * per, (t + 1) * per)
  const int per = (E + 1023) / 1024;
  int32_t run = 0;
  for (int i = 0; i < per; ++i) {
    const int e = t * per + i;
    if (e < E) run += nfull[e];
  }
  part[t] = run;
  __syncthreads();
  // thread t holds the count of tail size t (sizes 1 .. bm - 1; bm <= 1024)
  const int32_t cnt = (t >= 1 && t < bm) ? start[t] : 0;
  suf[t] = cnt;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t v = t >= off ? part[t - off] : 0;
    const int32_t w = t + off < 1024 ? suf[t + off] : 0;
    __syncthreads();
    part[t] += v;
    suf[t] += w;
    __syncthreads();
  }
  const int32_t total_full = part[1023];
  const int32_t n_tiles = total_full + suf[0];  // full tiles + one partial tile per expert with a tail
  // partial tiles by decreasing size: size s starts after every larger one
  if (t >= 1 && t < bm) start[t] = suf[t] - cnt;
  __syncthreads();
  int32_t pos = part[t] - run;
  for (int i = 0; i < per; ++i) {
    const int e = t * per + i;
    if (e >= E) break;
    // (a max_tiles below the real tile count truncates the order instead of
    // writing past it)
    for (int b = 0; b < nfull[e]; ++b)
      if (pos + b < max_tiles) order[pos + b] = (b << 16) | e;
    pos += nfull[e];
    const int s = tail[e];
    if (s) {
      int rank = start[s];
      for (int f = 0; f < e; ++f) rank += tail[f] == s;
      if (total_full + rank < max_tiles) order[total_full + rank] = (nfull[e] << 16) | e;
    }
  }
  for (int i = n_tiles + t; i < max_tiles; i += 1024) order[i] = -1;
}

}  // namespace

extern "C" size_t af3_routing_workspace_bytes(int64_t n_tokens, int n_expts_tot, int n_expts_act) {
  int64_t R = n_tokens * n_expts_act;
  int64_t n_chunks = af3_cdiv(R, kChunk);
  size_t b = 0;
  b += (size_t)R * 4;                       // ids
  b = (b + 255) & ~(size_t)255;
  b += (size_t)R * 2;                       // scal
  b = (b + 255) & ~(size_t)255;
  b += (size_t)n_chunks * n_expts_tot * 4;  // counts
  return b + 256;
}

static int routing_common(bool topk, const uint16_t* logits, int64_t ld, const int32_t* expt_indx, int64_t T, int E,
                          int K, uint16_t* gate_scal, int32_t* hist, int32_t* topk_indx, int32_t* gate_indx,
                          int32_t* token_offs_raw, void* workspace, size_t ws_bytes, hipStream_t stream) {
  AF3_REQUIRE(T >= 0 && E > 0 && K > 0, "routing: bad sizes T=%lld E=%d K=%d", (long long)T, E, K);
  AF3_REQUIRE(K <= 16, "routing: K=%d > 16 unsupported", K);
  AF3_REQUIRE(E <= 0x7fff, "routing: E=%d too large", E);
  AF3_REQUIRE(E * 4 <= 48 * 1024, "routing: E=%d exceeds the per-chunk LDS histogram", E);
  AF3_REQUIRE(!topk || K <= E, "routing: K=%d > E=%d", K, E);
  AF3_REQUIRE(ld >= E, "routing: logits leading dim %lld < E", (long long)ld);
  AF3_REQUIRE(ws_bytes >= af3_routing_workspace_bytes(T, E, K), "routing: workspace too small");
  const int64_t R = T * K;
  AF3_REQUIRE(R < 0x7fffffffLL, "routing: T*K too large");
  char* ws = (char*)workspace;
  size_t o = 0;
  int32_t* ids = (int32_t*)(ws + o);
  o += (size_t)R * 4;
  o = (o + 255) & ~(size_t)255;
  uint16_t* scal = (uint16_t*)(ws + o);
  o += (size_t)R * 2;
  o = (o + 255) & ~(size_t)255;
  int32_t* counts = (int32_t*)(ws + o);
  const int n_chunks = (int)af3_cdiv(R, kChunk);

  if (T > 0) {
    dim3 g((unsigned)af3_cdiv(T, 128));
    if (topk)
      hipLaunchKernelGGL(topk_token_kernel, g, dim3(128), 0, stream, logits, ld, T, E, K, ids, scal);
    else
      hipLaunchKernelGGL(replay_token_kernel, g, dim3(128), 0, stream, logits, ld, expt_indx, T, E, K, ids, scal);
    int rc = af3::check_launch("routing/token");
    if (rc) return rc;
    hipLaunchKernelGGL(chunk_hist_kernel, dim3(n_chunks), dim3(kChunk), E * 4, stream, ids, R, E, n_chunks, counts);
    rc = af3::check_launch("routing/hist");
    if (rc) return rc;
    hipLaunchKernelGGL(chunk_scan_kernel, dim3(E), dim3(256), 0, stream, counts, n_chunks, hist);
    rc = af3::check_launch("routing/chunk_scan");
    if (rc) return rc;
  } else {
    hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(256), 0, stream, hist, E);
    int rc = af3::check_launch("routing/zero");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(expert_scan_kernel, dim3(1), dim3(1024), 0, stream, hist, E, token_offs_raw);
  int rc = af3::check_launch("routing/expert_scan");
  if (rc) return rc;
  if (T > 0) {
    hipLaunchKernelGGL(scatter_kernel, dim3(n_chunks), dim3(kChunk), 0, stream, ids, scal, R, n_chunks, token_offs_raw,
                       counts, topk_indx, gate_indx, gate_scal);
    rc = af3::check_launch("routing/scatter");
    if (rc) return rc;
    hipLaunchKernelGGL(fill_tail_kernel, dim3((unsigned)af3_cdiv(R, 256)), dim3(256), 0, stream, token_offs_raw, E,
                       R, topk_indx, gate_scal);
    rc = af3::check_launch("routing/tail");
  }
  return rc;
}

extern "C" int af3_routing_replay(const uint16_t* logits, int64_t ld_logits, const int32_t* expt_indx, int64_t n_tokens,
                                  int n_expts_tot, int n_expts_act, uint16_t* gate_scal, int32_t* hist,
                                  int32_t* topk_indx, int32_t* gate_indx, int32_t* token_offs_raw, void* workspace,
                                  size_t ws_bytes, void* stream) {
  AF3_REQUIRE(expt_indx || n_tokens == 0, "routing_replay: null expt_indx");
  return routing_common(false, logits, ld_logits, expt_indx, n_tokens, n_expts_tot, n_expts_act, gate_scal, hist,
                        topk_indx, gate_indx, token_offs_raw, workspace, ws_bytes, (hipStream_t)stream);
}

// ---- allocation-free routing replay --------------------------------------
// The workspace of af3_routing_replay (ids, softmax weights, per-chunk counts;
// every byte is written before it is read, so nothing needs clearing) lives in
// this file-scope device array.  Each device holds its own copy; host code
// never passes the array's name to a kernel (on the host it only names the
// symbol), it passes the device address taken once per device with
// hipGetSymbolAddress.
constexpr size_t kRoutingScratchBytes = size_t(4) << 20;
static __device__ __align__(256) unsigned char scratch[kRoutingScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

extern "C" size_t af3_routing_scratch_bytes(void) { return kRoutingScratchBytes; }

extern "C" int af3_routing_replay_noalloc(const uint16_t* logits, int64_t ld_logits, const int32_t* expt_indx,
                                          int64_t n_tokens, int n_expts_tot, int n_expts_act, uint16_t* gate_scal,
                                          int32_t* hist, int32_t* topk_indx, int32_t* gate_indx,
                                          int32_t* token_offs_raw, void* stream) {
  AF3_REQUIRE(expt_indx || n_tokens == 0, "routing_replay_noalloc: null expt_indx");
  AF3_REQUIRE(n_tokens >= 0 && n_expts_tot > 0 && n_expts_act > 0, "routing_replay_noalloc: bad sizes");
  const size_t need = af3_routing_workspace_bytes(n_tokens, n_expts_tot, n_expts_act);
  AF3_REQUIRE(need <= kRoutingScratchBytes,
              "routing_replay_noalloc: T=%lld E=%d K=%d needs %zu scratch bytes, the built-in buffer holds %zu "
              "(use af3_routing_replay with a workspace)",
              (long long)n_tokens, n_expts_tot, n_expts_act, need, kRoutingScratchBytes);
  // the array of the device the stream belongs to (the null stream: the
  // current device), taken with that device current
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) {
    af3::set_error("routing_replay_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return (int)e;
  }
  hipDevice_t dev = cur;
  if (stream) {
    e = hipStreamGetDevice((hipStream_t)stream, &dev);
    if (e != hipSuccess) {
      af3::set_error("routing_replay_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
      return (int)e;
    }
  }
  AF3_REQUIRE(dev >= 0 && dev < kMaxDevices, "routing_replay_noalloc: device %d out of range", (int)dev);
  if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
    af3::set_error("routing_replay_noalloc: hipSetDevice(%d): %s", (int)dev, hipGetErrorString(e));
    return (int)e;
  }
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {  // first call on this device: its copy of the array
      e = hipGetSymbolAddress(&g_scratch_ptr[dev], HIP_SYMBOL(scratch));
      if (e != hipSuccess) g_scratch_ptr[dev] = nullptr;
    }
    ws = g_scratch_ptr[dev];
  }
  int rc = 0;
  if (!ws) {
    af3::set_error("routing_replay_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    rc = (int)e;
  } else {
    rc = routing_common(false, logits, ld_logits, expt_indx, n_tokens, n_expts_tot, n_expts_act, gate_scal, hist,
                        topk_indx, gate_indx, token_offs_raw, ws, kRoutingScratchBytes, (hipStream_t)stream);
  }
  if (dev != cur) hipSetDevice(cur);  // the caller's current device, as it was
  return rc;
}

extern "C" int af3_routing_topk(const uint16_t* logits, int64_t ld_logits, int64_t n_tokens, int n_expts_tot,
                                int n_expts_act, uint16_t* gate_scal, int32_t* hist, int32_t* topk_indx,
                                int32_t* gate_indx, int32_t* token_offs_raw, void* workspace, size_t ws_bytes,
                                void* stream) {
  return routing_common(true, logits, ld_logits, nullptr, n_tokens, n_expts_tot, n_expts_act, gate_scal, hist,
                        topk_indx, gate_indx, token_offs_raw, workspace, ws_bytes, (hipStream_t)stream);
}

extern "C" int af3_expt_data(const int32_t* hist, int n_expts_tot, const int32_t* block_ms_dev, int n_block_ms,
                             int max_tiles, int32_t* token_offs_pad, int32_t* block_pid_map, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_expts_tot > 0 && n_expts_tot <= kScanMaxE && n_block_ms > 0 && n_block_ms <= 64 && max_tiles >= 0,
              "expt_data: bad sizes (E=%d, block sizes %d, max_tiles %d)", n_expts_tot, n_block_ms, max_tiles);
  hipLaunchKernelGGL(tile_scan_map_kernel, dim3(n_block_ms), dim3(1024), 0, stream, hist, n_expts_tot, block_ms_dev,
                     max_tiles, token_offs_pad, block_pid_map);
  return af3::check_launch("expt_data");
}

// Order of the BM-row tiles for the grouped GEMM's work list (same entries as
// the block_pid_map of af3_expt_data for this BM, permuted): full tiles in
// expert order, then each expert's partial last tile by decreasing rows.
extern "C" int af3_tile_order(const int32_t* hist, int n_expts_tot, int block_m, const int32_t* token_offs_pad,
                              int max_tiles, int32_t* order, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  AF3_REQUIRE(n_expts_tot > 0 && n_expts_tot <= kSchedMaxE, "tile_order: E=%d outside [1, %d]", n_expts_tot,
              kSchedMaxE);
  AF3_REQUIRE(block_m > 0 && block_m <= kSchedMaxBM && max_tiles >= 0, "tile_order: bad block_m %d / max_tiles %d",
              block_m, max_tiles);
  AF3_REQUIRE(max_tiles == 0 || (hist && token_offs_pad && order), "tile_order: null pointer");
  if (max_tiles == 0) return 0;
  (void)token_offs_pad;  // the kernel counts the tiles itself (the same total as token_offs_pad[E])
  hipLaunchKernelGGL(tile_order_kernel, dim3(1), dim3(1024), 0, stream, hist, n_expts_tot, block_m, max_tiles, order);
  return af3::check_launch("tile_order");
}
