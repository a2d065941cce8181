// Device pieces shared by the router top-k and the dispatch layout kernels.
//
//  * topk_token: the top-k selection of one token by one wave, under the rule of
//    `glm52/reference.py:62-79`: s = fp32(sigmoid(logit)) evaluated in fp64, key =
//    s + bias (NaN keys sort last), ids by descending key with the lower index first on
//    ties; weights s[id] / max(sum s, 1e-20) * scale with the k scores summed in slot
//    order.  Each expert's rank is the number of experts that beat it, so the experts of
//    rank < k land in slot = rank already sorted, without sequential selection rounds.
//  * align_body: the sglang dispatch layout of `glm52/reference.py:85-128` built by one
//    workgroup of NT threads (histogram, padded prefix, sentinel fill, stable scatter).
#pragma once

#include "common.h"

namespace glm52 {

constexpr int kMaxE = 256;

GLM52_DEV bool beats(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// Stage 1 (every lane): scores and keys of the token's experts lane + 64 j into `keys`.
GLM52_DEV void topk_keys(const float lg[4], const float* __restrict__ bias, int E, bool active,
                         float sc[4], float key[4], float* keys) {
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    key[j] = -INFINITY;
    sc[j] = 0.f;
    if (active && e < E) {
      const float s = (float)(1.0 / (1.0 + exp(-(double)lg[j])));
      sc[j] = s;
      const float k = bias ? s + bias[e] : s;
      key[j] = (k != k) ? -INFINITY : k;
    }
    keys[lane + j * kWave] = key[j];
  }
}

// Stage 2 (after a barrier): ranks against all keys; winners to sel_s / sel_i.
GLM52_DEV void topk_rank(const float* keys, const float sc[4], const float key[4], int E, int topk,
                         float* sel_s, int* sel_i) {
  const int lane = threadIdx.x % kWave;
  const int nk = (E + 3) / 4;
  int rank[4] = {0, 0, 0, 0};
  for (int q = 0; q < nk; ++q) {
    const float4 kv = *reinterpret_cast<const float4*>(&keys[4 * q]);
    const float o[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int oi = 4 * q + i;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        rank[j] += (oi < E && beats(o[i], oi, key[j], lane + j * kWave)) ? 1 : 0;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    if (e < E && rank[j] < topk) {
      sel_s[rank[j]] = sc[j];
      sel_i[rank[j]] = e;
    }
  }
}

// Stage 3 (after a barrier): lane k < topk returns slot k's weight and id.
GLM52_DEV void topk_weight(const float* sel_s, const int* sel_i, int topk, float scale,
                           int norm_prob, float* w, int* id) {
  const int lane = threadIdx.x % kWave;
  float sum = 0.f;
  for (int k = 0; k < topk; ++k) sum += sel_s[k];
  const float denom = fmaxf(sum, 1e-20f);
  const float s = sel_s[lane];
  *w = norm_prob ? (s / denom) * scale : s * scale;
  *id = sel_i[lane];
}

template <int NT>
struct AlignLds {
  int cnt[kMaxE];
  int start[kMaxE];
  int running[kMaxE];
  int wcnt[NT / kWave][kMaxE];
  int total;
};

// Dispatch layout by one workgroup of NT threads.  `ids` may point to global or LDS
// memory.  Entries outside [0, E) get no slot.
template <int NT>
GLM52_DEV void align_body(const int32_t* ids, int numel, int E, int BM, int capacity,
                          int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                          int32_t* __restrict__ ntp_out, AlignLds<NT>& sh) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wid = tid / kWave;

  for (int e = tid; e < kMaxE; e += NT) {
    sh.cnt[e] = 0;
    sh.running[e] = 0;
  }
  for (int q = tid; q < NW * kMaxE; q += NT) (&sh.wcnt[0][0])[q] = 0;
  __syncthreads();

  // 1. histogram
  for (int i = tid; i < numel; i += NT) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&sh.cnt[e], 1);
  }
  __syncthreads();

  // 2. padded exclusive prefix, one wave, 4 experts per lane
  if (wid == 0) {
    int pad[4], incl = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      const int c = e < E ? sh.cnt[e] : 0;
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
      sh.start[lane * 4 + j] = run;
      run += pad[j];
    }
    if (lane == kWave - 1) sh.total = scan;
  }
  __syncthreads();
  const int total = sh.total;

  // 3. sentinels, expert ids, tail
  for (int e = wid; e < E; e += NW) {
    const int c = sh.cnt[e];
    const int s = sh.start[e];
    const int p = ((c + BM - 1) / BM) * BM;
    for (int j = c + lane; j < p; j += kWave) sorted_ids[s + j] = numel;
    for (int b = lane; b < p / BM; b += kWave) expert_ids[s / BM + b] = e;
  }
  for (int j = total + tid; j < capacity; j += NT) sorted_ids[j] = numel;
  for (int b = total / BM + tid; b < capacity / BM; b += NT) expert_ids[b] = -1;
  if (tid == 0) ntp_out[0] = total;

  // 4. stable scatter, NT ids per chunk in index order
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  for (int base = 0; base < numel; base += NT) {
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
    if (valid && rank == 0) sh.wcnt[wid][e] = __popcll(m);
    __syncthreads();
    if (valid) {
      int off = sh.running[e];
      for (int w = 0; w < wid; ++w) off += sh.wcnt[w][e];
      sorted_ids[sh.start[e] + off + rank] = i;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += NT) {
      int s = 0;
      for (int w = 0; w < NW; ++w) {
        s += sh.wcnt[w][ee];
        sh.wcnt[w][ee] = 0;
      }
      sh.running[ee] += s;
    }
    __syncthreads();
  }
}

}  // namespace glm52
