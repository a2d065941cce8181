// Token-major down GEMV: the accumulation strategy (b) of fusions #8 / #9
// (`glm52/kernels/moe_down_merge.py:165-293`, `moe_down_token_major_kernel`):
//
//   out[t, n] = bf16( sum_k w[t, k] * (a[t * top_k + k] . w2[ids[t, k], n])  (+ r[t, n]) )
//
// one fp32 accumulation over all of a token's experts, no [T, top_k, H] tensor, no
// atomics, one rounding.  Optionally a shared expert joins as one more unit with weight 1
// (its activation row a_s[t], its weight w2_s), which makes the kernel the whole tail of
// the MoE block at decode sizes: out = bf16(routed + shared + h).
//
// Mapping for gfx950: workgroup (g, t) owns output rows n0 .. n0 + 4 * kNR - 1 of token t,
// a wave kNR consecutive W2 rows (at T = 1 and N = 6144: 512 workgroups, two per CU).  A
// W2 row (K bf16) is read by the wave as K / 512 coalesced 1 KB pieces, lane l taking the 16-byte chunks l, l + 64, ...; the lane keeps
// one fp32 partial per row across all units, and the 64 lane partials meet in a fixed
// butterfly at the end.  The rows of the next unit are loaded (non-temporal: the weights
// are read once) before the current unit's FMAs, so two units' rows are in flight.
#include "moe_gemm.h"

using namespace glm52;

namespace {

constexpr int kNR = 3;  // W2 rows per wave (4 waves x 3 = 12 output columns per workgroup)

template <int QC>
__global__ __launch_bounds__(256) void down_tokmaj_kernel(
    const uint16_t* __restrict__ a, int64_t sam, const uint16_t* __restrict__ w2, int64_t swe,
    int64_t swn, const float* __restrict__ topw, const int32_t* __restrict__ topi, int64_t stk,
    int topk, int E, const uint16_t* __restrict__ a_s, int64_t sas,
    const uint16_t* __restrict__ w2_s, int64_t sws, const uint16_t* __restrict__ res, int64_t srm,
    uint16_t* __restrict__ out, int64_t som, int N) {
  const int lane = threadIdx.x % kWave;
  const int wv = threadIdx.x / kWave;
  const int t = blockIdx.y;
  const int n0 = (blockIdx.x * 4 + wv) * kNR;
  if (n0 >= N) return;  // no barriers below: a wave may leave on its own
  const int nunits = topk + (w2_s ? 1 : 0);

  // unit u: routed expert u of the token, or (u == topk) the shared expert
  auto load_unit = [&](int u, uint4 (&wr)[kNR][QC], uint4 (&ar)[QC], float& wk) {
    const uint16_t* wbase = nullptr;
    const uint16_t* arow = nullptr;
    wk = 0.f;
    if (u < topk) {
      const int e = topi[(int64_t)t * stk + u];
      if (e >= 0 && e < E) {  // an id outside [0, E) contributes nothing
        wbase = w2 + (int64_t)e * swe;
        arow = a + ((int64_t)t * topk + u) * sam;
        wk = topw[(int64_t)t * stk + u];
      }
    } else {
      wbase = w2_s;
      arow = a_s + (int64_t)t * sas;
      wk = 1.f;
    }
#pragma unroll
    for (int q = 0; q < QC; ++q)
      ar[q] = arow ? ldg(arow + (lane + kWave * q) * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < kNR; ++r)
#pragma unroll
      for (int q = 0; q < QC; ++q)
        wr[r][q] = (wbase && n0 + r < N)
                       ? ldg_nt(wbase + (int64_t)(n0 + r) * swn + (lane + kWave * q) * 8)
                       : make_uint4(0, 0, 0, 0);
  };

  float acc[kNR];
#pragma unroll
  for (int r = 0; r < kNR; ++r) acc[r] = 0.f;
  auto fma_unit = [&](const uint4 (&wr)[kNR][QC], const uint4 (&ar)[QC], float wk) {
    float af[QC][8];
#pragma unroll
    for (int q = 0; q < QC; ++q) unpack8(ar[q], af[q]);
#pragma unroll
    for (int r = 0; r < kNR; ++r) {
      float p = 0.f;
#pragma unroll
      for (int q = 0; q < QC; ++q) {
        float wf[8];
        unpack8(wr[r][q], wf);
#pragma unroll
        for (int i = 0; i < 8; ++i) p = fmaf(af[q][i], wf[i], p);
      }
      acc[r] = fmaf(wk, p, acc[r]);
    }
  };

  uint4 wc[kNR][QC], wn[kNR][QC], ac[QC], an[QC];
  float kc, kn;
  load_unit(0, wc, ac, kc);
  for (int u = 0; u < nunits; ++u) {
    const bool more = u + 1 < nunits;
    if (more) load_unit(u + 1, wn, an, kn);
    fma_unit(wc, ac, kc);
    if (more) {
#pragma unroll
      for (int q = 0; q < QC; ++q) {
        ac[q] = an[q];
#pragma unroll
        for (int r = 0; r < kNR; ++r) wc[r][q] = wn[r][q];
      }
      kc = kn;
    }
  }

#pragma unroll
  for (int r = 0; r < kNR; ++r) {
    float v = wave_sum(acc[r]);
    if (lane == r && n0 + r < N) {
      if (res) v = v + bf16_to_f32(res[(int64_t)t * srm + n0 + r]);
      out[(int64_t)t * som + n0 + r] = f32_to_bf16(v);
    }
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// Token-major down GEMV + expert merge (+ residual), for T tokens: a [T * top_k, K] bf16
// (rows t * top_k + k), w2 [E, N, K] bf16 (K contiguous), topk_weights fp32 / topk_ids
// int32 [T, top_k] (row stride stride_tk); a_shared [T, K] and w2_shared [N, K] (row
// strides stride_as, stride_ws) add a shared expert with weight 1 when w2_shared is
// non-null; residual [T, N] may be null.  K must be 1024 or 2048.
extern "C" int glm52_down_token_major(const void* a, int64_t stride_am, const void* w2,
                                      int64_t stride_we, int64_t stride_wn,
                                      const float* topk_weights, const int32_t* topk_ids,
                                      int64_t stride_tk, int top_k, int num_experts,
                                      const void* a_shared, int64_t stride_as,
                                      const void* w2_shared, int64_t stride_ws,
                                      const void* residual, int64_t stride_rm, void* out,
                                      int64_t stride_om, int T, int N, int K,
                                      hipStream_t stream) {
  if (T < 0 || T > 65535 || N <= 0 || top_k < 1 || num_experts < 1 || stride_tk < top_k)
    return GLM52_EINVAL;
  if (K != 1024 && K != 2048) return GLM52_EUNSUPPORTED;
  if (T == 0) return GLM52_OK;
  if (!a || !w2 || !topk_weights || !topk_ids || !out) return GLM52_EINVAL;
  if (!al16(a) || !al16(w2) || (stride_am % 8) || stride_am < K || (stride_wn % 8) ||
      stride_wn < K || (stride_we % 8) || stride_we < (int64_t)N * stride_wn - stride_wn + K ||
      stride_om < N)
    return GLM52_EINVAL;
  if (w2_shared && (!a_shared || !al16(a_shared) || !al16(w2_shared) || (stride_as % 8) ||
                    stride_as < K || (stride_ws % 8) || stride_ws < K))
    return GLM52_EINVAL;
  if (residual && stride_rm < N) return GLM52_EINVAL;
  const dim3 grid((N + 4 * kNR - 1) / (4 * kNR), T);
  auto* aa = static_cast<const uint16_t*>(a);
  auto* ww = static_cast<const uint16_t*>(w2);
  auto* as = static_cast<const uint16_t*>(a_shared);
  auto* ws = static_cast<const uint16_t*>(w2_shared);
  auto* rr = static_cast<const uint16_t*>(residual);
  auto* oo = static_cast<uint16_t*>(out);
  if (K == 1024)
    down_tokmaj_kernel<2><<<grid, 256, 0, stream>>>(aa, stride_am, ww, stride_we, stride_wn,
        topk_weights, topk_ids, stride_tk, top_k, num_experts, as, stride_as, ws, stride_ws, rr,
        stride_rm, oo, stride_om, N);
  else
    down_tokmaj_kernel<4><<<grid, 256, 0, stream>>>(aa, stride_am, ww, stride_we, stride_wn,
        topk_weights, topk_ids, stride_tk, top_k, num_experts, as, stride_as, ws, stride_ws, rr,
        stride_rm, oo, stride_om, N);
  GLM52_RETURN_LAUNCH();
}
