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
// are read once) before the current unit's FMAs, so two units' rows are in flight.  The
// shared expert's unit, when there is one, comes first: its weights need no routing, so
// its loads leave before the token's expert ids arrive (the packed form below: T = 1 tail
// 41.5 -> 40.0 us, block 119.6 -> 118.9 us, one process).
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
  auto unit_at = [&](int j) { return w2_s ? (j == 0 ? topk : j - 1) : j; };  // shared first
  load_unit(unit_at(0), wc, ac, kc);
  for (int u = 0; u < nunits; ++u) {
    const bool more = u + 1 < nunits;
    if (more) load_unit(unit_at(u + 1), wn, an, kn);
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

// The same sum on packed weights (glm52_pack_w512 of w2 for N plain outputs).  The 16 rows
// of packed load slot q of 512-row tile P are rows P * 512 + (q / 8) * 128 + (q % 8 / 2) * 32
// + (q % 2) * 8 + phi32(p), p = 0 .. 15; the slot holds their K / 32 stages of 1 KB each,
// kPackStride apart (packed_slot_off), lane l's 16 bytes holding row p = l / 4, 8-k chunk
// (l % 4) ^ (p / 4 % 4).  Workgroup (s, t) owns slot s (tile s / 32, slot s % 32) of token
// t: wave w takes the pieces of QS stages that start at stages QS b and QS (b + 4) with
// b = (w + g) % 8 for the workgroup's group of 8 slots g = s / 8, so the four waves read
// 4 QS stages of the slot at a time; every load reads one stage's whole 1 KB, and a lane
// keeps one fp32 partial of its row over all pieces.  The 4 lanes of a row, then the 4
// waves, meet in a fixed order.  The pieces flow through two register buffers, so a wave
// has two pieces' loads in flight; four waves per workgroup let two workgroups share a CU
// (about 210 VGPRs), so at T = 1 and N = 6144 the 384 workgroups run in a single round.
// The rotation by g: the workgroups advance in step, and without it every group would
// read the same stages of the same expert at once, at addresses a power of two apart (the
// group stride, NK * 8 KB), which the HBM serves from fewer channels at a time (T = 1
// tail 44.0 -> 41.3 us; the row-major tail 40.5 us).
template <int QS>
__global__ __launch_bounds__(256) void down_tokmaj_packed_kernel(
    const uint16_t* __restrict__ a, int64_t sam, const uint16_t* __restrict__ w2p,
    const float* __restrict__ topw, const int32_t* __restrict__ topi, int64_t stk, int topk,
    int E, const uint16_t* __restrict__ a_s, int64_t sas, const uint16_t* __restrict__ w2sp,
    const uint16_t* __restrict__ res, int64_t srm, uint16_t* __restrict__ out, int64_t som,
    int N) {
  __shared__ float red[4][16];
  const int lane = threadIdx.x % kWave;
  const int wv = threadIdx.x / kWave;
  const int t = blockIdx.y;
  const int P = blockIdx.x >> 5, q = blockIdx.x & 31;
  constexpr int NK = 8 * QS;                // 32-k stages of a row (K / 32)
  const int num_n512 = N / 512;
  const int pr = lane >> 2;                      // the lane's row in the slot
  const int kc = (lane & 3) ^ ((pr >> 2) & 3);   // and its 8-k chunk of every stage
  const int64_t toff = P * packed_tile_elems(NK) + packed_slot_off(NK, q) + lane * 8;
  const int npieces = 2 * (topk + (w2sp ? 1 : 0));

  // piece c: half c % 2 of the wave's stages of the (c / 2)-th unit -- the shared expert
  // first (u == topk), when there is one, then routed expert u of the token
  auto load_piece = [&](int c, uint4 (&wr)[QS], uint4 (&ar)[QS], float& wk) {
    const int u = w2sp ? ((c >> 1) == 0 ? topk : (c >> 1) - 1) : (c >> 1);
    const int kt0 = ((((c & 1) * 4 + wv) + (int)(blockIdx.x >> 3)) & 7) * QS;
    const uint16_t* wb = nullptr;
    const uint16_t* arow = nullptr;
    wk = 0.f;
    if (u < topk) {
      const int e = topi[(int64_t)t * stk + u];
      if (e >= 0 && e < E) {  // an id outside [0, E) contributes nothing
        wb = w2p + (int64_t)e * num_n512 * packed_tile_elems(NK) + toff;
        arow = a + ((int64_t)t * topk + u) * sam;
        wk = topw[(int64_t)t * stk + u];
      }
    } else {
      wb = w2sp + toff;
      arow = a_s + (int64_t)t * sas;
      wk = 1.f;
    }
#pragma unroll
    for (int i = 0; i < QS; ++i)
      ar[i] = arow ? ldg(arow + (kt0 + i) * 32 + kc * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < QS; ++i)
      wr[i] = wb ? ldg_nt(wb + (int64_t)(kt0 + i) * kPackStride) : make_uint4(0, 0, 0, 0);
  };

  float acc = 0.f;
  auto fma_piece = [&](const uint4 (&wr)[QS], const uint4 (&ar)[QS], float wk) {
    float pd = 0.f;
#pragma unroll
    for (int i = 0; i < QS; ++i) {
      float af[8], wf[8];
      unpack8(ar[i], af);
      unpack8(wr[i], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) pd = fmaf(af[j], wf[j], pd);
    }
    acc = fmaf(wk, pd, acc);
  };

  uint4 wc[QS], wn[QS], ac[QS], an[QS];
  float kc_w, kn_w;
  load_piece(0, wc, ac, kc_w);
  for (int c = 0; c < npieces; ++c) {
    const bool more = c + 1 < npieces;
    if (more) load_piece(c + 1, wn, an, kn_w);
    fma_piece(wc, ac, kc_w);
    if (more) {
#pragma unroll
      for (int i = 0; i < QS; ++i) {
        ac[i] = an[i];
        wc[i] = wn[i];
      }
      kc_w = kn_w;
    }
  }

  acc += __shfl_xor(acc, 1, kWave);
  acc += __shfl_xor(acc, 2, kWave);
  if ((lane & 3) == 0) red[wv][pr] = acc;
  __syncthreads();
  if (threadIdx.x < 16) {
    const int i = threadIdx.x;
    const float v0 = ((red[0][i] + red[1][i]) + red[2][i]) + red[3][i];
    const int n = P * 512 + (q >> 3) * 128 + ((q & 7) >> 1) * 32 + (q & 1) * 8 + phi32(i);
    const float v = res ? v0 + bf16_to_f32(res[(int64_t)t * srm + n]) : v0;
    out[(int64_t)t * som + n] = f32_to_bf16(v);
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

// glm52_down_token_major on packed weights: w2_packed = glm52_pack_w512 of w2 ([E, N, K],
// plain, n_out = N), w2_shared_packed (may be null) the same of the [1, N, K] shared w2.
// N must be a multiple of 512, K 1024 or 2048.  Same sum; the adds run in another order.
extern "C" int glm52_down_token_major_packed(const void* a, int64_t stride_am,
                                             const void* w2_packed, const float* topk_weights,
                                             const int32_t* topk_ids, int64_t stride_tk,
                                             int top_k, int num_experts, const void* a_shared,
                                             int64_t stride_as, const void* w2_shared_packed,
                                             const void* residual, int64_t stride_rm, void* out,
                                             int64_t stride_om, int T, int N, int K,
                                             hipStream_t stream) {
  if (T < 0 || T > 65535 || N <= 0 || (N % 512) || top_k < 1 || num_experts < 1 ||
      stride_tk < top_k)
    return GLM52_EINVAL;
  if (K != 1024 && K != 2048) return GLM52_EUNSUPPORTED;
  if (T == 0) return GLM52_OK;
  if (!a || !w2_packed || !topk_weights || !topk_ids || !out) return GLM52_EINVAL;
  if (!al16(a) || !al16(w2_packed) || (stride_am % 8) || stride_am < K || stride_om < N)
    return GLM52_EINVAL;
  if (w2_shared_packed && (!a_shared || !al16(a_shared) || !al16(w2_shared_packed) ||
                           (stride_as % 8) || stride_as < K))
    return GLM52_EINVAL;
  if (residual && stride_rm < N) return GLM52_EINVAL;
  const dim3 grid(N / 16, T);
  auto* aa = static_cast<const uint16_t*>(a);
  auto* ww = static_cast<const uint16_t*>(w2_packed);
  auto* as = static_cast<const uint16_t*>(a_shared);
  auto* ws = static_cast<const uint16_t*>(w2_shared_packed);
  auto* rr = static_cast<const uint16_t*>(residual);
  auto* oo = static_cast<uint16_t*>(out);
  if (K == 1024)
    down_tokmaj_packed_kernel<4><<<grid, 256, 0, stream>>>(aa, stride_am, ww, topk_weights,
        topk_ids, stride_tk, top_k, num_experts, as, stride_as, ws, rr, stride_rm, oo,
        stride_om, N);
  else
    down_tokmaj_packed_kernel<8><<<grid, 256, 0, stream>>>(aa, stride_am, ww, topk_weights,
        topk_ids, stride_tk, top_k, num_experts, as, stride_as, ws, rr, stride_rm, oo,
        stride_om, N);
  GLM52_RETURN_LAUNCH();
}
