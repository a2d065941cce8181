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
// One workgroup of 1024 threads:
//   1. LDS histogram of the ids,
//   2. padded exclusive prefix over experts (one wave, shuffle scan),
//   3. sentinel fill of the padding and of the tail, expert_ids fill,
//   4. stable scatter: the ids are walked in chunks of 1024 in index order; inside a
//      chunk each wave ranks equal keys with ballots, and a per-wave count table in LDS
//      gives each wave its offset, so the order of equal ids is their index order.
#include "common.h"

using namespace glm52;

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxE = 256;

__global__ __launch_bounds__(kThreads) void moe_align_kernel(
    const int32_t* __restrict__ ids, int numel, int E, int BM, int capacity,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ ntp_out) {
  __shared__ int cnt[kMaxE];
  __shared__ int start[kMaxE];
  __shared__ int running[kMaxE];
  __shared__ int wcnt[kWaves][kMaxE];
  __shared__ int total_s;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wid = tid / kWave;

  for (int e = tid; e < kMaxE; e += kThreads) {
    cnt[e] = 0;
    running[e] = 0;
  }
  for (int q = tid; q < kWaves * kMaxE; q += kThreads) (&wcnt[0][0])[q] = 0;
  __syncthreads();

  // 1. histogram (ids outside [0, E) are ignored: they get no slot)
  for (int i = tid; i < numel; i += kThreads) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();

  // 2. padded exclusive prefix, one wave, 4 experts per lane (E <= 256)
  if (wid == 0) {
    int pad[4], incl = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      const int c = e < E ? cnt[e] : 0;
      pad[j] = ((c + BM - 1) / BM) * BM;
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
      const int e = lane * 4 + j;
      if (e < kMaxE) start[e] = run;
      run += pad[j];
    }
    if (lane == kWave - 1) total_s = scan;
  }
  __syncthreads();
  const int total = total_s;

  // 3. sentinels, expert ids, tail
  for (int e = wid; e < E; e += kWaves) {
    const int c = cnt[e];
    const int s = start[e];
    const int p = ((c + BM - 1) / BM) * BM;
    for (int j = c + lane; j < p; j += kWave) sorted_ids[s + j] = numel;
    for (int b = lane; b < p / BM; b += kWave) expert_ids[s / BM + b] = e;
  }
  for (int j = total + tid; j < capacity; j += kThreads) sorted_ids[j] = numel;
  for (int b = total / BM + tid; b < capacity / BM; b += kThreads) expert_ids[b] = -1;
  if (tid == 0) ntp_out[0] = total;

  // 4. stable scatter
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  for (int base = 0; base < numel; base += kThreads) {
    const int i = base + tid;
    int e = i < numel ? ids[i] : -1;
    const bool valid = e >= 0 && e < E;
    if (!valid) e = -1;
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t bm = __ballot(bit);
      m &= bit ? bm : ~bm;
    }
    const int rank = __popcll(m & lt_mask);
    if (valid && rank == 0) wcnt[wid][e] = __popcll(m);
    __syncthreads();
    if (valid) {
      int off = running[e];
      for (int w = 0; w < wid; ++w) off += wcnt[w][e];
      sorted_ids[start[e] + off + rank] = i;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += kThreads) {
      int s = 0;
      for (int w = 0; w < kWaves; ++w) {
        s += wcnt[w][ee];
        wcnt[w][ee] = 0;
      }
      running[ee] += s;
    }
    __syncthreads();
  }
}

}  // namespace

extern "C" int glm52_moe_align(const int32_t* topk_ids, int numel, int block_m,
                               int num_experts, int capacity, int32_t* sorted_token_ids,
                               int32_t* expert_ids, int32_t* num_tokens_post_padded,
                               hipStream_t stream) {
  if (numel < 0 || block_m <= 0 || num_experts <= 0 || num_experts > kMaxE) return GLM52_EINVAL;
  if (!sorted_token_ids || !expert_ids || !num_tokens_post_padded) return GLM52_EINVAL;
  if (numel > 0 && !topk_ids) return GLM52_EINVAL;
  const int64_t need = (int64_t)numel + (int64_t)num_experts * (block_m - 1);
  if (capacity < need || (capacity % block_m) != 0) return GLM52_EINVAL;
  moe_align_kernel<<<1, kThreads, 0, stream>>>(topk_ids, numel, num_experts, block_m, capacity,
                                                sorted_token_ids, expert_ids,
                                                num_tokens_post_padded);
  GLM52_RETURN_LAUNCH();
}
