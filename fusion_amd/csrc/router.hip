// GLM-5.2 router: fp32 logits, sigmoid scores, noaux_tc bias-corrected top-8, gfx950.
//
// Semantics restate `glm52/reference.py:46-79` (n_group = topk_group = 1, so there is no
// group mask):
//
//   logits = y . Wg^T                          (fp32 result)
//   s      = sigmoid(logits)                   (fp32)
//   choice = s + bias                          (fp32 add; bias may be absent)
//   ids    = the 8 largest choices, in descending order, lower index first on ties
//   w      = s[ids] / max(sum_k s[ids], 1e-20) * scale      (or s[ids] * scale)
//
// Bit-exact routing.  A 6144-term fp32 dot product depends on summation order, so two
// implementations that sum differently can disagree on an id whenever the 8th and 9th
// choices are within an ulp or two.  This kernel therefore pins the arithmetic to a rule
// that does not depend on order: every bf16 x bf16 product is exact in fp64, the sum is
// carried in fp64 (its rounding error, ~2^-53 relative, is far below half an fp32 ulp),
// and the result is rounded once to fp32.  The sigmoid is evaluated in fp64 and rounded
// once to fp32 as well.  The CPU oracle applies the same rule, so ids agree bit for bit.
//
// The reference kernel's layout for the gate weight is [H, E] (`wgt_from_gate`,
// `glm52/kernels/norm_router.py:251-255`); it is what `router_gemm` consumes here too.
#include "common.h"

using namespace glm52;

namespace {

constexpr int KC = 32;  // k-chunk staged in LDS per wave

// grid = (ceil(T / BT), ceil(E / 64)); block = 256 (4 waves, each a quarter of K).
template <int BT, bool WG_F32>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ y, int64_t sy, const void* __restrict__ wg_raw, int64_t swg,
    float* __restrict__ logits, int64_t sl, int T, int H, int E) {
  constexpr int NACC = BT >= 4 ? 1 : 4 / BT;  // independent chains for small BT
  __shared__ double ys[4][BT][KC];
  __shared__ double red[4][BT][kWave];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int t0 = blockIdx.x * BT;
  const int e = blockIdx.y * kWave + lane;
  const bool e_ok = e < E;
  const int kq = H / 4;
  const int kbeg = wv * kq;

  double acc[BT][NACC];
#pragma unroll
  for (int t = 0; t < BT; ++t)
#pragma unroll
    for (int q = 0; q < NACC; ++q) acc[t][q] = 0.0;

  for (int k0 = kbeg; k0 < kbeg + kq; k0 += KC) {
    // stage y[t0 .. t0+BT)[k0 .. k0+KC) as fp64 in this wave's LDS slice
    for (int idx = lane; idx < BT * KC; idx += kWave) {
      const int t = idx / KC, kk = idx % KC;
      double v = 0.0;
      if (t0 + t < T) v = (double)bf16_to_f32(y[(int64_t)(t0 + t) * sy + k0 + kk]);
      ys[wv][t][kk] = v;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < KC; ++kk) {
      double wvv = 0.0;
      if (e_ok) {
        const int64_t off = (int64_t)(k0 + kk) * swg + e;
        wvv = WG_F32 ? (double)static_cast<const float*>(wg_raw)[off]
                     : (double)bf16_to_f32(static_cast<const uint16_t*>(wg_raw)[off]);
      }
#pragma unroll
      for (int t = 0; t < BT; ++t) acc[t][kk % NACC] = fma(ys[wv][t][kk], wvv, acc[t][kk % NACC]);
    }
    __syncthreads();
  }

#pragma unroll
  for (int t = 0; t < BT; ++t) {
    double s = 0.0;
#pragma unroll
    for (int q = 0; q < NACC; ++q) s += acc[t][q];
    red[wv][t][lane] = s;
  }
  __syncthreads();
  for (int t = wv; t < BT; t += 4) {
    if (t0 + t < T && e_ok) {
      const double s = ((red[0][t][lane] + red[1][t][lane]) + red[2][t][lane]) + red[3][t][lane];
      logits[(int64_t)(t0 + t) * sl + e] = (float)s;
    }
  }
}

// One wave per token; E <= 256 experts, four per lane.
struct Cand {
  float v;  // selection key (score + bias)
  int i;    // expert index
  float s;  // unbiased score
};

GLM52_DEV bool better(const Cand& a, const Cand& b) {
  return a.v > b.v || (a.v == b.v && a.i < b.i);
}

__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, int64_t sl, const float* __restrict__ bias,
    float* __restrict__ topw, int64_t stw, int32_t* __restrict__ topi, int64_t sti, int T,
    int E, int topk, float scale, int norm_prob) {
  const int lane = threadIdx.x % kWave;
  const int64_t t = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (t >= T) return;

  float key[4], sc[4];
  bool taken[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    taken[j] = !(e < E);
    key[j] = -INFINITY;
    sc[j] = 0.f;
    if (e < E) {
      const double lg = (double)logits[t * sl + e];
      const float s = (float)(1.0 / (1.0 + exp(-lg)));
      sc[j] = s;
      key[j] = bias ? s + bias[e] : s;
    }
  }

  float sel_s[8];
  int sel_i[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sel_s[k] = 0.f;
    sel_i[k] = 0;
    if (k >= topk) continue;
    Cand best{-INFINITY, 0x7fffffff, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Cand c{key[j], lane + j * kWave, sc[j]};
      if (!taken[j] && (best.i == 0x7fffffff || better(c, best))) best = c;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      Cand o;
      o.v = __shfl_xor(best.v, off, kWave);
      o.i = __shfl_xor(best.i, off, kWave);
      o.s = __shfl_xor(best.s, off, kWave);
      if (o.i != 0x7fffffff && (best.i == 0x7fffffff || better(o, best))) best = o;
    }
    sel_s[k] = best.s;
    sel_i[k] = best.i;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (lane + j * kWave == best.i) taken[j] = true;
  }

  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < topk) sum += sel_s[k];
  const float denom = fmaxf(sum, 1e-20f);
  if (lane < topk) {
    float s = 0.f;
    int id = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k == lane) {
        s = sel_s[k];
        id = sel_i[k];
      }
    const float wgt = norm_prob ? (s / denom) * scale : s * scale;
    topw[t * stw + lane] = wgt;
    topi[t * sti + lane] = id;
  }
}

}  // namespace

extern "C" int glm52_router_logits(const void* y, int64_t stride_y, const void* wgt,
                                   int64_t stride_wg, int wg_is_f32, float* logits,
                                   int64_t stride_l, int T, int H, int E, hipStream_t stream) {
  if (T < 0 || H <= 0 || E <= 0 || E > 256 || (H % (4 * KC)) != 0) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  if (!y || !wgt || !logits || stride_wg < E || stride_l < E || stride_y < H) return GLM52_EINVAL;
  auto* yy = static_cast<const uint16_t*>(y);
  dim3 block(256);
  if (T <= 2) {
    dim3 grid((T + 0) / 1, (E + kWave - 1) / kWave);
    if (wg_is_f32)
      router_logits_kernel<1, true><<<grid, block, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, T, H, E);
    else
      router_logits_kernel<1, false><<<grid, block, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, T, H, E);
  } else if (T <= 64) {
    dim3 grid((T + 3) / 4, (E + kWave - 1) / kWave);
    if (wg_is_f32)
      router_logits_kernel<4, true><<<grid, block, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, T, H, E);
    else
      router_logits_kernel<4, false><<<grid, block, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, T, H, E);
  } else {
    dim3 grid((T + 15) / 16, (E + kWave - 1) / kWave);
    if (wg_is_f32)
      router_logits_kernel<16, true><<<grid, block, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, T, H, E);
    else
      router_logits_kernel<16, false><<<grid, block, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, T, H, E);
  }
  GLM52_RETURN_LAUNCH();
}

extern "C" int glm52_router_topk(const float* logits, int64_t stride_l, const float* bias,
                                 float* topw, int64_t stride_w, int32_t* topi,
                                 int64_t stride_i, int T, int E, int topk, float scale,
                                 int norm_prob, hipStream_t stream) {
  if (T < 0 || E <= 0 || E > 256 || topk <= 0 || topk > 8 || topk > E) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  if (!logits || !topw || !topi || stride_l < E || stride_w < topk || stride_i < topk)
    return GLM52_EINVAL;
  dim3 grid((T + 3) / 4);
  router_topk_kernel<<<grid, 256, 0, stream>>>(logits, stride_l, bias, topw, stride_w, topi,
                                               stride_i, T, E, topk, scale, norm_prob);
  GLM52_RETURN_LAUNCH();
}
