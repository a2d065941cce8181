// Device pieces shared by the router top-k and the dispatch layout kernels.
//
//  * topk_keys / topk_rank / topk_weight: the top-k selection of one token by one wave,
//    under the rule of `glm52/reference.py:62-79`: s = fp32(sigmoid(logit)) evaluated in
//    fp64, key = s + bias (NaN keys sort last), ids by descending key with the lower
//    index first on ties; weights s[id] / max(sum s, 1e-20) * scale with the k scores
//    summed in slot order.  Selection is k rounds of a wave-wide argmax.
//  * align_body: the sglang dispatch layout of `glm52/reference.py:85-128` built by one
//    workgroup of NT threads (histogram, padded prefix, sentinel fill, stable scatter).
#pragma once

#include "common.h"

namespace glm52 {

constexpr int kMaxE = 256;

// The correction bias of experts lane + 64 j (zero if there is none), for topk_keys.
GLM52_DEV void load_bias(const float* __restrict__ bias, int E, float bv[4]) {
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    bv[j] = (bias && e < E) ? bias[e] : 0.f;
  }
}

// Stage 1 (every lane): scores and keys of the token's experts lane + 64 j.
// The fp64 sigmoid is long code; it is kept in one copy inside a rolled loop, because
// right after a cache flush every instruction line of a kernel is fetched from HBM and
// four unrolled copies cost microseconds of fetch latency.
GLM52_DEV void topk_keys(const float lg[4], const float bv[4], bool has_bias, int E, bool active,
                         float sc[4], float key[4]) {
  const int lane = threadIdx.x % kWave;
  float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int j = 0; j < 4; ++j) {
    const float x = j == 0 ? lg[0] : j == 1 ? lg[1] : j == 2 ? lg[2] : lg[3];
    const float s = (float)(1.0 / (1.0 + exp(-(double)x)));
    s4[0] = j == 0 ? s : s4[0];
    s4[1] = j == 1 ? s : s4[1];
    s4[2] = j == 2 ? s : s4[2];
    s4[3] = j == 3 ? s : s4[3];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    key[j] = -INFINITY;
    sc[j] = 0.f;
    if (active && e < E) {
      sc[j] = s4[j];
      const float k = has_bias ? s4[j] + bv[j] : s4[j];
      key[j] = (k != k) ? -INFINITY : k;
    }
  }
}

// Order-preserving map of an fp32 key (not NaN) to uint32, shifted so that every real
// key maps above 0, which marks an expert already taken (or absent).
GLM52_DEV uint32_t key_order(float k) {
  const uint32_t u = __float_as_uint(k);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return o == 0u ? 1u : o;  // -NaN patterns never reach here; keep 0 free
}

// Wave-wide max of a uint32 (result in a scalar register): xor-1 and xor-2 quad swaps,
// half-row and row mirrors leave every lane with its 16-lane row's maximum, then the four
// row maxima meet through readlane.  DPP moves cost a few cycles; xor shuffles go through
// the LDS crossbar.
GLM52_DEV uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false));   // quad [1,0,3,2]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false));   // quad [2,3,0,1]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));  // row half mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));  // row mirror
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}

// Stage 2: the wave selects its token's top-k in k rounds of a wave-wide argmax under
// (key descending, expert index ascending) and writes slot r of sel_s / sel_i.  Each
// lane keeps its four experts' order keys; a round takes the wave maximum of the lane
// maxima, finds the lanes that hold it with a ballot and, on a tie between lanes, takes
// the lowest expert index.  Slot j of a lane whose bit j of `absent` is set takes no
// part (it is never selected).  Every lane of the wave must call it.
GLM52_DEV void topk_rank(const float sc[4], const float key[4], int E, int topk, float* sel_s,
                         int* sel_i, uint32_t absent = 0u) {
  const int lane = threadIdx.x % kWave;
  uint32_t ou[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    ou[j] = (lane + j * kWave < E && !((absent >> j) & 1u)) ? key_order(key[j]) : 0u;
  for (int r = 0; r < topk; ++r) {
    // lane-local best: strict > keeps the lower j (the lower expert index) on ties
    uint32_t bu = ou[0];
    int bj = 0;
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (ou[j] > bu) {
        bu = ou[j];
        bj = j;
      }
    const uint32_t m = wave_max_u32(bu);
    const uint64_t holders = __ballot(bu == m);
    int wl;  // winning lane (wave-uniform)
    if (__popcll(holders) == 1) {
      wl = __ffsll((unsigned long long)holders) - 1;
    } else {
      int idx = bu == m ? lane + bj * kWave : 0x7fffffff;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) idx = min(idx, __shfl_xor(idx, off, kWave));
      wl = idx % kWave;
    }
    wl = __builtin_amdgcn_readfirstlane(wl);
    const int wj = __builtin_amdgcn_readlane(bj, wl);
    float ws = sc[0];
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (wj == j) ws = sc[j];
    const float win_s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(ws), wl));
    if (lane == wl) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j == wj) ou[j] = 0u;
    }
    if (lane == 0) {
      sel_s[r] = win_s;
      sel_i[r] = wl + wj * kWave;
    }
  }
}

// Stage 3 (after a barrier, lanes k < topk): slot k's weight and id.
GLM52_DEV void topk_weight(const float* sel_s, const int* sel_i, int topk, float scale,
                           int norm_prob, float* w, int* id) {
  const int lane = threadIdx.x % kWave;
  float sum = 0.f;
  for (int k = 0; k < topk; ++k) sum += sel_s[k];
  const float denom = sum < 1e-20f ? 1e-20f : sum;  // clamp_min: a NaN sum stays NaN
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

// The dispatch layout by one workgroup of NT threads for many ids: wave w owns the
// contiguous index range [w L, (w + 1) L).  Pass 1 counts each wave's ids per expert in
// LDS; a prefix over experts (padded starts) and over waves turns the counts into each
// wave's first slot per expert; pass 2 lets every wave scatter its range in index order,
// ranking equal experts inside each 64-id step with ballots and advancing its own
// per-expert cursor -- no workgroup barrier inside the passes.  Same result as
// align_body (ids of one expert in ascending index order).
template <int NT>
GLM52_DEV void align_body_waves(const int32_t* __restrict__ ids, int numel, int E, int BM,
                                int capacity, int32_t* __restrict__ sorted_ids,
                                int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp_out,
                                AlignLds<NT>& sh) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wid = tid / kWave;
  const int L = ((numel + NW * kWave - 1) / (NW * kWave)) * kWave;  // ids per wave
  const int lo = wid * L;
  const int hi = min(numel, lo + L);
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));

  for (int q = tid; q < NW * kMaxE; q += NT) (&sh.wcnt[0][0])[q] = 0;
  __syncthreads();

  // 1. per-wave histograms; eight loads of a lane in flight before its first atomic
  for (int i0 = lo; i0 < hi; i0 += 8 * kWave) {
    int ev[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * kWave + lane;
      ev[u] = i < hi ? ids[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (ev[u] >= 0 && ev[u] < E) atomicAdd(&sh.wcnt[wid][ev[u]], 1);
  }
  __syncthreads();

  // 2. totals, padded exclusive prefix (one wave, 4 experts per lane)
  for (int e = tid; e < kMaxE; e += NT) {
    int c = 0;
    for (int w = 0; w < NW; ++w) c += sh.wcnt[w][e];
    sh.cnt[e] = e < E ? c : 0;
  }
  __syncthreads();
  if (wid == 0) {
    int pad[4], incl = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = sh.cnt[lane * 4 + j];
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
  // each wave's first slot per expert: start[e] + the ids of e held by earlier waves
  for (int e = tid; e < E; e += NT) {
    int run = sh.start[e];
    for (int w = 0; w < NW; ++w) {
      const int c = sh.wcnt[w][e];
      sh.wcnt[w][e] = run;
      run += c;
    }
  }

  // 3. sentinels, expert ids, tail (independent of the cursors)
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
  __syncthreads();

  // 4. stable scatter, every wave over its own range in index order, 64 ids a step; the
  //    ids of eight steps are loaded before the first of them is ranked
  for (int b0 = lo; b0 < hi; b0 += 8 * kWave) {
    int ev[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = b0 + u * kWave + lane;
      ev[u] = i < hi ? ids[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int base = b0 + u * kWave;
      if (base >= hi) break;  // wave-uniform
      const int i = base + lane;
      int e = ev[u];
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
      int pos = 0;
      if (valid) {
        pos = sh.wcnt[wid][e] + rank;
        sorted_ids[pos] = i;
      }
      if (valid && rank == 0) sh.wcnt[wid][e] += __popcll(m);  // after every lane's read
    }
  }
}

// The dispatch layout for few ids, by the first wave of the workgroup (all NT threads
// call it; they help with the sentinel tail).  Valid when no expert can receive more
// than BM ids (numel <= 64 and every expert at most once per token with T <= BM): then
// every expert that is hit owns exactly one block, the blocks follow in expert order, and
// an id's slot is (its expert's rank among the distinct experts) * BM + (the number of
// smaller flat indices routed to the same expert).  Same result as align_body.
template <int NT>
GLM52_DEV void align_few(const int32_t* ids, int numel, int E, int BM, int capacity,
                         int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                         int32_t* __restrict__ ntp_out, int* s_nblk) {
  const int tid = threadIdx.x;
  if (tid < kWave) {
    const int lane = tid;
    int e = lane < numel ? ids[lane] : -1;
    if (e >= E) e = -1;
    const bool valid = e >= 0;
    int earlier_same = 0, distinct_below = 0, cnt_same = 0;
    bool first = valid;
    for (int j = 0; j < numel; ++j) {  // uniform loop, at most 64 rounds
      const int ej = __builtin_amdgcn_readlane(e, j);
      if (ej < 0) continue;
      if (ej == e) {
        ++cnt_same;
        if (j < lane) {
          ++earlier_same;
          first = false;
        }
      }
    }
    // distinct experts below mine: count first occurrences with a smaller expert id
    const uint64_t firsts = __ballot(first);
    for (int j = 0; j < numel; ++j) {
      if (!((firsts >> j) & 1ull)) continue;
      const int ej = __builtin_amdgcn_readlane(e, j);
      distinct_below += (valid && ej < e) ? 1 : 0;
    }
    const int nblk = __popcll(firsts);
    if (valid) {
      const int slot = distinct_below * BM + earlier_same;
      sorted_ids[slot] = lane;
      if (first) {
        expert_ids[distinct_below] = e;
        for (int q = cnt_same; q < BM; ++q) sorted_ids[distinct_below * BM + q] = numel;
      }
    }
    if (lane == 0) {
      ntp_out[0] = nblk * BM;
      *s_nblk = nblk;
    }
  }
  __syncthreads();
  const int nblk = *s_nblk;
  for (int j = nblk * BM + tid; j < capacity; j += NT) sorted_ids[j] = numel;
  for (int b = nblk + tid; b < capacity / BM; b += NT) expert_ids[b] = -1;
}

// Top-k of every token (four at a time, a wave each) and the dispatch layout of the
// selected ids, by one workgroup of 256 threads (decode: T * topk <= 256).  The ids are
// kept in LDS between the two.
constexpr int kTopkAlignSlots = 256;

struct TopkAlignLds {
  float sel_s[4][8];
  int sel_i[4][8];
  int ids[kTopkAlignSlots];
  int nblk;
  AlignLds<256> al;
};

// `bv` holds the lane's four bias values (load_bias), `has_bias` whether there is a bias.
GLM52_DEV void topk_align_block(const float* logits, int64_t sl, const float bv[4], bool has_bias,
                                float* __restrict__ topw, int64_t stw, int32_t* __restrict__ topi,
                                int64_t sti, int T, int E, int topk, float scale, int norm_prob,
                                int BM, int capacity, int32_t* __restrict__ sorted_ids,
                                int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp_out,
                                TopkAlignLds& sh) {
  const int lane = threadIdx.x % kWave;
  const int wv = threadIdx.x / kWave;
  for (int t0 = 0; t0 < T; t0 += 4) {
    const int t = t0 + wv;
    const bool active = t < T;
    float lg[4], sc[4], key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + j * kWave;
      lg[j] = (active && e < E) ? logits[(int64_t)t * sl + e] : 0.f;
    }
    topk_keys(lg, bv, has_bias, E, active, sc, key);
    topk_rank(sc, key, E, active ? topk : 0, sh.sel_s[wv], sh.sel_i[wv]);
    __syncthreads();
    if (active && lane < topk) {
      float w;
      int id;
      topk_weight(sh.sel_s[wv], sh.sel_i[wv], topk, scale, norm_prob, &w, &id);
      topw[(int64_t)t * stw + lane] = w;
      topi[(int64_t)t * sti + lane] = id;
      sh.ids[t * topk + lane] = id;
    }
    __syncthreads();
  }
  if (T <= BM && T * topk <= kWave)
    align_few<256>(sh.ids, T * topk, E, BM, capacity, sorted_ids, expert_ids, ntp_out, &sh.nblk);
  else
    align_body<256>(sh.ids, T * topk, E, BM, capacity, sorted_ids, expert_ids, ntp_out, sh.al);
}

}  // namespace glm52
