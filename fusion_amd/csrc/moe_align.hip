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
// For decode the router's top-k and the layout run as one launch
// (`router_topk_align_kernel`): one workgroup selects the experts of every token, keeps
// the ids in LDS and builds the layout from them.
#include "select.h"

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
