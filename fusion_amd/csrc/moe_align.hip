// Token -> expert dispatch layout (sglang `moe_align_block_size`), on the device, gfx950.
//
// Semantics restate `glm52/reference.py:85-128` and the convention written down in
// `glm52/kernels/REFERENCES.md:41-51`:
//
//   flat      = topk_ids.flatten()                      (numel = T * top_k entries)
//   count[e]  = #{i : flat[i] == e},  padded[e] = ceil(count[e] / BM) * BM
//   start[e]  = sum_{e' < e} padded[e']
//   sorted_token_ids[start[e] + j] = the j-th smallest i with flat[i] == e     (stable)
//   sorted_token_ids[start[e] + count[e] .. start[e] + padded[e]) = numel      (sentinel)
//   expert_ids[b] = e for every BM-block b of [start[e], start[e] + padded[e])
//   num_tokens_post_padded = sum_e padded[e]
//
// The reference allocates exactly `num_tokens_post_padded` slots after a device->host
// sync.  Here the caller passes buffers sized for the worst case
// (numel + E * (BM - 1) slots) and the count stays on the device, so the whole block
// is graph-capturable.  Slots past the count hold the sentinel and blocks past it hold
// expert id -1; consumers stop at `num_tokens_post_padded`.
//
// One workgroup builds the layout (select.h, align_body_waves): per-wave LDS histograms
// over contiguous index ranges, padded prefix, sentinel fill, then a stable scatter in
// which every wave walks its own range in index order, ranking equal keys inside each
// 64-id step with ballots.
//
// For larger inputs (glm52_moe_align_ws, more than one chunk of 2048 ids) the layout is
// built by one workgroup per chunk in two launches, with the same result:
//   align_hist_kernel     hist[c][e] = the ids of expert e in chunk c (LDS histogram)
//   align_scatter_kernel  every workgroup sums hist into the totals (and the ids of each
//                         expert in earlier chunks), takes the padded prefix, gives each of
//                         its waves a cursor per expert (chunk base + earlier waves of the
//                         chunk), and scatters its chunk as the single workgroup does; the
//                         sentinel, expert-id and tail fills are split over the workgroups.
//
// For decode the router's top-k and the layout run as one launch
// (`router_topk_align_kernel`): one workgroup selects the experts of every token, keeps
// the ids in LDS and builds the layout from them.
#include "select.h"

#include <mutex>

using namespace glm52;

namespace {

constexpr int kThreads = 1024;

__global__ __launch_bounds__(kThreads) void moe_align_kernel(
    const int32_t* __restrict__ ids, int numel, int E, int BM, int capacity,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ ntp_out) {
  __shared__ AlignLds<kThreads> sh;
  align_body_waves<kThreads>(ids, numel, E, BM, capacity, sorted_ids, expert_ids, ntp_out, sh);
}

constexpr int kFusedThreads = 256;

__global__ __launch_bounds__(kFusedThreads) void router_topk_align_kernel(
    const float* __restrict__ logits, int64_t sl, const float* __restrict__ bias,
    float* __restrict__ topw, int64_t stw, int32_t* __restrict__ topi, int64_t sti, int T,
    int E, int topk, float scale, int norm_prob, int BM, int capacity,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ ntp_out) {
  __shared__ TopkAlignLds sh;
  float bv[4];
  load_bias(bias, E, bv);
  topk_align_block(logits, sl, bv, bias != nullptr, topw, stw, topi, sti, T, E, topk, scale,
                   norm_prob, BM, capacity, sorted_ids, expert_ids, ntp_out, sh);
}

constexpr int kChunkThreads = 256;
constexpr int kChunkIds = 8 * kChunkThreads;  // ids per chunk: 8 per lane
constexpr int kChunkWaves = kChunkThreads / kWave;
constexpr int kMaxChunks = 512;               // numel <= 1M

__global__ __launch_bounds__(kChunkThreads) void align_hist_kernel(
    const int32_t* __restrict__ ids, int numel, int E, int32_t* __restrict__ hist) {
  __shared__ int cnt[kMaxE];
  const int tid = threadIdx.x;
  for (int e = tid; e < kMaxE; e += kChunkThreads) cnt[e] = 0;
  __syncthreads();
  const int lo = blockIdx.x * kChunkIds;
  int ev[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int i = lo + u * kChunkThreads + tid;
    ev[u] = i < numel ? ids[i] : -1;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (ev[u] >= 0 && ev[u] < E) atomicAdd(&cnt[ev[u]], 1);
  __syncthreads();
  for (int e = tid; e < E; e += kChunkThreads) hist[(int64_t)blockIdx.x * E + e] = cnt[e];
}

__global__ __launch_bounds__(kChunkThreads) void align_scatter_kernel(
    const int32_t* __restrict__ ids, int numel, int E, int BM, int capacity,
    const int32_t* __restrict__ hist, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp_out) {
  __shared__ int wcur[kChunkWaves][kMaxE];
  __shared__ int cnt[kMaxE];
  __shared__ int start[kMaxE];
  __shared__ int total_s;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wid = tid / kWave;
  const int c = blockIdx.x;
  const int P = gridDim.x;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));

  // the wave's 512 ids of the chunk, in index order (step u: ids lo + 64 u .. + 63)
  const int lo = c * kChunkIds + wid * 8 * kWave;
  int ev[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int i = lo + u * kWave + lane;
    const int e = i < numel ? ids[i] : -1;
    ev[u] = (e >= 0 && e < E) ? e : -1;
  }
  // thread e: the total of expert e and its ids in earlier chunks
  int tot = 0, before = 0;
  if (tid < E) {
    for (int q = 0; q < P; ++q) {
      const int h = hist[(int64_t)q * E + tid];
      tot += h;
      before += q < c ? h : 0;
    }
  }
  for (int q = tid; q < kChunkWaves * kMaxE; q += kChunkThreads) (&wcur[0][0])[q] = 0;
  if (tid < kMaxE) cnt[tid] = tid < E ? tot : 0;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (ev[u] >= 0) atomicAdd(&wcur[wid][ev[u]], 1);
  if (wid == 0) {  // padded exclusive prefix over the experts, 4 a lane
    int pad[4], incl = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = cnt[lane * 4 + j];
      pad[j] = ((n + BM - 1) / BM) * BM;
      incl += pad[j];
    }
    int scan = incl;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int o = __shfl_up(scan, off, kWave);
      if (lane >= off) scan += o;
    }
    int run = scan - incl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      start[lane * 4 + j] = run;
      run += pad[j];
    }
    if (lane == kWave - 1) total_s = scan;
  }
  __syncthreads();
  const int total = total_s;
  if (tid < E) {  // each wave's first slot per expert
    int run = start[tid] + before;
#pragma unroll
    for (int w = 0; w < kChunkWaves; ++w) {
      const int k = wcur[w][tid];
      wcur[w][tid] = run;
      run += k;
    }
  }
  // sentinels and expert ids of experts c, c + P, ...; this workgroup's share of the tail
  for (int e = c; e < E; e += P) {
    const int n = cnt[e];
    const int s0 = start[e];
    const int pd = ((n + BM - 1) / BM) * BM;
    for (int j = n + tid; j < pd; j += kChunkThreads) sorted_ids[s0 + j] = numel;
    for (int b = tid; b < pd / BM; b += kChunkThreads) expert_ids[s0 / BM + b] = e;
  }
  for (int j = total + c * kChunkThreads + tid; j < capacity; j += P * kChunkThreads)
    sorted_ids[j] = numel;
  for (int b = total / BM + c * kChunkThreads + tid; b < capacity / BM; b += P * kChunkThreads)
    expert_ids[b] = -1;
  if (c == 0 && tid == 0) ntp_out[0] = total;
  __syncthreads();

  // stable scatter of the wave's ids: rank among equal experts inside each 64-id step
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int base = lo + u * kWave;
    if (base >= numel) break;  // wave-uniform
    const int e = ev[u];
    const bool valid = e >= 0;
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t bm = __ballot(bit);
      m &= bit ? bm : ~bm;
    }
    const int rank = __popcll(m & lt_mask);
    if (valid) sorted_ids[wcur[wid][e] + rank] = base + lane;
    if (valid && rank == 0) wcur[wid][e] += __popcll(m);  // after every lane's read
  }
}

int check_layout_args(int numel, int block_m, int num_experts, int capacity,
                      const int32_t* sorted_token_ids, const int32_t* expert_ids,
                      const int32_t* ntp) {
  if (numel < 0 || block_m <= 0 || num_experts <= 0 || num_experts > kMaxE) return GLM52_EINVAL;
  if (!sorted_token_ids || !expert_ids || !ntp) return GLM52_EINVAL;
  const int64_t need = (int64_t)numel + (int64_t)num_experts * (block_m - 1);
  if (capacity < need || (capacity % block_m) != 0) return GLM52_EINVAL;
  return GLM52_OK;
}

}  // namespace

extern "C" int glm52_moe_align(const int32_t* topk_ids, int numel, int block_m,
                               int num_experts, int capacity, int32_t* sorted_token_ids,
                               int32_t* expert_ids, int32_t* num_tokens_post_padded,
                               hipStream_t stream) {
  int rc = check_layout_args(numel, block_m, num_experts, capacity, sorted_token_ids, expert_ids,
                             num_tokens_post_padded);
  if (rc != GLM52_OK) return rc;
  if (numel > 0 && !topk_ids) return GLM52_EINVAL;
  moe_align_kernel<<<1, kThreads, 0, stream>>>(topk_ids, numel, num_experts, block_m, capacity,
                                                sorted_token_ids, expert_ids,
                                                num_tokens_post_padded);
  GLM52_RETURN_LAUNCH();
}

// the chunk histograms' bytes, or 0 where the chunked build does not apply
int64_t chunk_hist_bytes(int numel, int num_experts) {
  if (numel <= kChunkIds || num_experts <= 0 || num_experts > kMaxE) return 0;
  const int64_t P = ((int64_t)numel + kChunkIds - 1) / kChunkIds;
  return P > kMaxChunks ? 0 : P * num_experts * (int64_t)sizeof(int32_t);
}

// Below this many ids one workgroup is as fast (measured at T = 512 and 2048 with top-8:
// 15 vs 38 us and 25 vs 20 us), so the query asks for no workspace there.
constexpr int kChunkedMinIds = 16384;

extern "C" int64_t glm52_moe_align_workspace_bytes(int numel, int num_experts) {
  return numel < kChunkedMinIds ? 0 : chunk_hist_bytes(numel, num_experts);
}

extern "C" int glm52_moe_align_ws(const int32_t* topk_ids, int numel, int block_m,
                                  int num_experts, int capacity, int32_t* sorted_token_ids,
                                  int32_t* expert_ids, int32_t* num_tokens_post_padded,
                                  void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  const int64_t need = chunk_hist_bytes(numel, num_experts);
  if (need == 0 || !workspace || workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return glm52_moe_align(topk_ids, numel, block_m, num_experts, capacity, sorted_token_ids,
                           expert_ids, num_tokens_post_padded, stream);
  int rc = check_layout_args(numel, block_m, num_experts, capacity, sorted_token_ids, expert_ids,
                             num_tokens_post_padded);
  if (rc != GLM52_OK) return rc;
  if (!topk_ids) return GLM52_EINVAL;
  const int P = (numel + kChunkIds - 1) / kChunkIds;
  auto* hist = static_cast<int32_t*>(workspace);
  align_hist_kernel<<<P, kChunkThreads, 0, stream>>>(topk_ids, numel, num_experts, hist);
  align_scatter_kernel<<<P, kChunkThreads, 0, stream>>>(topk_ids, numel, num_experts, block_m,
                                                        capacity, hist, sorted_token_ids,
                                                        expert_ids, num_tokens_post_padded);
  GLM52_RETURN_LAUNCH();
}

// ------------------------------------------------------------------------------------
// glm52_moe_align_noalloc: glm52_moe_align_ws with its chunk histograms in a scratch array
// of the library's own, for callers that cannot allocate.  The array holds the histograms
// of up to kMaxChunks chunks of kMaxE experts (512 KB); each GPU the library runs on holds
// its own copy until the process ends.  Host code never passes the array's name (a host
// stand-in) to a kernel: the first call on a device, with that device current, looks up
// the device copy's address once and keeps it per device.  align_hist_kernel writes every
// (chunk, expert) entry it later reads, so nothing needs clearing between calls; calls
// that overlap on one GPU share the array and race.
// ------------------------------------------------------------------------------------
static __device__ __align__(256) int32_t scratch[kMaxChunks * kMaxE];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// the current device's copy of `scratch` (looked up on the first call on that device)
int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  if (dev < 0 || dev >= kMaxDevices) return GLM52_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return (int)err;
    if (!p) return GLM52_EUNSUPPORTED;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GLM52_OK;
}
}  // namespace

extern "C" int glm52_moe_align_noalloc(const int32_t* topk_ids, int numel, int block_m,
                                       int num_experts, int capacity, int32_t* sorted_token_ids,
                                       int32_t* expert_ids, int32_t* num_tokens_post_padded,
                                       hipStream_t stream) {
  if (numel < 0 || numel > kMaxChunks * kChunkIds || num_experts <= 0 || num_experts > kMaxE)
    return GLM52_EINVAL;
  const int64_t need = chunk_hist_bytes(numel, num_experts);
  if (need == 0)  // one chunk or less: the single-workgroup build, which needs no scratch
    return glm52_moe_align(topk_ids, numel, block_m, num_experts, capacity, sorted_token_ids,
                           expert_ids, num_tokens_post_padded, stream);
  if (need > (int64_t)sizeof(scratch)) return GLM52_EINVAL;
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc != GLM52_OK) return rc;
  return glm52_moe_align_ws(topk_ids, numel, block_m, num_experts, capacity, sorted_token_ids,
                            expert_ids, num_tokens_post_padded, ws, need, stream);
}

extern "C" int glm52_router_topk_align(const float* logits, int64_t stride_l, const float* bias,
                                       float* topw, int64_t stride_w, int32_t* topi,
                                       int64_t stride_i, int T, int E, int topk, float scale,
                                       int norm_prob, int block_m, int capacity,
                                       int32_t* sorted_token_ids, int32_t* expert_ids,
                                       int32_t* num_tokens_post_padded, hipStream_t stream) {
  if (T < 0 || E <= 0 || E > kMaxE || (E % 4) != 0 || topk <= 0 || topk > 8 || topk > E ||
      (int64_t)T * topk > kTopkAlignSlots)
    return GLM52_EINVAL;
  if (!logits || !topw || !topi || stride_l < E || stride_w < topk || stride_i < topk)
    return GLM52_EINVAL;
  int rc = check_layout_args(T * topk, block_m, E, capacity, sorted_token_ids, expert_ids,
                             num_tokens_post_padded);
  if (rc != GLM52_OK) return rc;
  router_topk_align_kernel<<<1, kFusedThreads, 0, stream>>>(
      logits, stride_l, bias, topw, stride_w, topi, stride_i, T, E, topk, scale, norm_prob,
      block_m, capacity, sorted_token_ids, expert_ids, num_tokens_post_padded);
  GLM52_RETURN_LAUNCH();
}
