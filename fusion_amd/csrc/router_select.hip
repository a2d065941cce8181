// Router for T > 16 tokens on the gate's rows ([E, H], K contiguous), gfx950: logits on
// bf16 MFMA with a rigorous error bound, then the exact rule only where it decides.
//
// The exact rule (router.hip): logit = fp32(sum_k y[k] * w[e, k]) with the exact
// products summed in fp64; s = fp32(sigmoid) in fp64; key = fp32(s + bias); the k largest
// keys in descending order, lower index first on ties; weights from the selected s.
// Evaluating every logit that way costs an fp64 GEMM.  Here:
//
// 1. router_approx_kernel: L~[t, e] on `v_mfma_f32_32x32x16_bf16`.  The products are exact
//    in fp32; each accumulator runs a chain of eight MFMAs (128 k) and is then added into
//    an fp64 sum.  An MFMA adds 16 products to its accumulator with at most 16 roundings
//    of a partial sum no larger than |acc| + its |products|, so a chain of eight errs by
//    at most 16 * 9 * 2^-23 times the chain's sum of |products|, and |L~ - sum| <=
//    1.125 * 2^-16 * sum_k |y_k w_k| over the
//    row, and sum_k |y_k w_k| <= ||y|| ||w_e|| (Cauchy-Schwarz).  The kernel also returns
//    the sums of squares of every gate row (those of y come from the token's row in 2.).  A workgroup owns 64 tokens x all
//    experts of one K slice (K is split until about 256 workgroups run; fp32 partials).
// 2. router_select_kernel, one wave per token: from L~ and the bound
//    B = 2.5 * 2^-16 * ||y|| ||w_e|| + 2^-21 |L~| (over twice the chain bound, plus the fp32
//    roundings of L~ and of the exact logit), each expert's exact key lies in
//    [lo, hi] = [sig(L~ - B) + b - d, sig(L~ + B) + b + d] (d covers the fp32 roundings
//    and the fast sigmoid).  Every expert of the exact top k has key >= the k-th largest
//    lo, so the candidates {e : hi_e >= that} hold the whole top k, and no other expert
//    can tie with its k-th key.  Only the candidates (about k per token) get the exact
//    logit -- an fp64 dot product of y and the gate row -- and the exact top k is taken
//    among them: the same ids, order and weights as the exact rule over all experts.
//    Non-finite values make every expert a candidate.
//
// The logits written are exact for the candidates (so for every selected expert) and
// L~ rounded to fp32 elsewhere (within B of the exact logit).
#include "moe_gemm.h"
#include "select.h"

using namespace glm52;

namespace {

constexpr int kTok = 64;                 // tokens per workgroup of the approximate pass
constexpr int kBk = 32;                  // k per LDS stage
constexpr int kStages = 7;               // LDS ring
constexpr int kRows = kMaxE + kTok;      // gate rows (E padded to 256) + token rows
constexpr int kStageElems = kRows * kBk; // 20 KB per stage
constexpr int kIps = 5;                  // loads per wave and stage: 4 gate + 1 token
constexpr int kMaxH = 8192;

GLM52_DEV float sumsq8(const uint4& v) {
  float f[8];
  unpack8(v, f);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s = fmaf(f[i], f[i], s);
  return s;
}

// grid = (ceil(T / 64), KS); block = 256.  Wave w computes expert blocks 2w, 2w + 1 (of
// 32) against both 32-token blocks.  out: KS == 1: L~ into logits [T, E] (row stride
// so); else fp32 partials part[ks][T][E].  ssw[ks][E]: the gate rows' sums of squares
// over slice ks.
__global__ __launch_bounds__(256) void router_approx_kernel(
    const uint16_t* __restrict__ y, int64_t sy, const uint16_t* __restrict__ gate, int64_t sg,
    int T, int H, int E, float* __restrict__ out, int64_t so, float* __restrict__ ssw) {
  __shared__ __attribute__((aligned(1024))) uint16_t ring[kStages * kStageElems];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int l32 = lane % 32, h = lane / 32;
  const int t0 = blockIdx.x * kTok;
  const int ks = blockIdx.y, KS = gridDim.y;
  const int ksl = H / KS;
  const int kbeg = ks * ksl;
  const int nk = ksl / kBk;

  // load slots: lane -> row lane / 4 of a 16-row slab, physical chunk lane % 4 holding
  // logical chunk dc (the read side applies the same swizzle)
  const int dr = lane >> 2;
  const int dc = (lane & 3) ^ ((dr >> 2) & 3);
  uint32_t goff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int er = min((wv * 4 + i) * 16 + dr, E - 1);  // padded experts re-read a real row
    goff[i] = (uint32_t)((er * sg + dc * 8) * 2);
  }
  const int yrow = wv * 16 + dr;
  const uint16_t* ybase = y + (int64_t)t0 * sy;
  const uint32_t yoff = (uint32_t)((min(yrow, T - 1 - t0) * sy + dc * 8) * 2);
  const uint32_t ring_base = lds_addr(ring);

  auto issue = [&](int s) {
    const int kc = kbeg + min(s, nk - 1) * kBk;
    const uint32_t sb = ring_base + (uint32_t)((s % kStages) * kStageElems * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16s(gate + kc, goff[i], sb + (uint32_t)((wv * 4 + i) * 16 * kBk * 2));
    dma16s(ybase + kc, yoff, sb + (uint32_t)((kMaxE + wv * 16) * kBk * 2));
  };

  const int rd0 = l32 * kBk + (((0 + h) ^ ((l32 >> 2) & 3)) * 8);
  const int rd1 = l32 * kBk + (((2 + h) ^ ((l32 >> 2) & 3)) * 8);

  floatx16_t acc[2][2];   // [expert block][token block]
  double dacc[2][2][16];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[f][tb][i] = 0.f;
        dacc[f][tb][i] = 0.0;
      }
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue(s);
#pragma unroll 1
  for (int s = 0; s < nk; ++s) {
    GLM52_WAIT_VMCNT((kStages - 2) * kIps);  // stage s landed for this wave
    __syncthreads();                          // ... for every wave; buffer s - 1 is free
    issue(s + kStages - 1);
    const uint16_t* sb = ring + (s % kStages) * kStageElems;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int rd = kk ? rd1 : rd0;
      uint4 a[2], b[2];
#pragma unroll
      for (int f = 0; f < 2; ++f)
        a[f] = *reinterpret_cast<const uint4*>(sb + ((wv * 2 + f) * 32) * kBk + rd);
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
        b[tb] = *reinterpret_cast<const uint4*>(sb + (kMaxE + tb * 32) * kBk + rd);
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) acc[f][tb] = mfma32(a[f], b[tb], acc[f][tb]);
    }
    if ((s & 3) == 3 || s == nk - 1) {  // chains of at most eight MFMAs, then into fp64
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            dacc[f][tb][i] += (double)acc[f][tb][i];
            acc[f][tb][i] = 0.f;
          }
    }
  }
  GLM52_WAIT_VMCNT(0);  // the clamped loads past the slice

  // sums of squares of the gate rows over this K slice: row e by workgroup e % nblocks,
  // a wave per row, from global memory (the rows were just streamed: L2 hits)
  for (int e = blockIdx.x + wv * gridDim.x; e < E; e += 4 * gridDim.x) {
    const uint16_t* grow = gate + (int64_t)e * sg + kbeg;
    float q = 0.f;
    for (int c = lane; c < ksl / 8; c += kWave) q += sumsq8(*reinterpret_cast<const uint4*>(grow + c * 8));
    q = wave_sum(q);
    if (lane == 0) ssw[(int64_t)ks * E + e] = q;
  }

  // result i of lane (l32, h) in block (f, tb): expert (2 wv + f) * 32 + 8 (i / 4) + 4 h +
  // i % 4, token t0 + 32 tb + l32
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const int t = t0 + tb * 32 + l32;
    if (t < T) {
      float* orow = KS == 1 ? out + (int64_t)t * so : out + ((int64_t)ks * T + t) * E;
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int e = (wv * 2 + f) * 32 + 8 * (i / 4) + 4 * h + (i % 4);
          if (e < E) orow[e] = (float)dacc[f][tb][i];
        }
    }
  }
}

// fp32 logistic with __expf: within a few 2^-24 of the exact value
GLM52_DEV float sig_fast(float x) { return 1.f / (1.f + __expf(-x)); }

GLM52_DEV double dpp_f64(double v, int ctrl_sel) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  int lo = (int)(uint32_t)u, hi = (int)(uint32_t)(u >> 32);
  switch (ctrl_sel) {  // the DPP control must be an immediate
    case 0:
      lo = __builtin_amdgcn_update_dpp(0, lo, 0xb1, 0xf, 0xf, false);
      hi = __builtin_amdgcn_update_dpp(0, hi, 0xb1, 0xf, 0xf, false);
      break;
    case 1:
      lo = __builtin_amdgcn_update_dpp(0, lo, 0x4e, 0xf, 0xf, false);
      hi = __builtin_amdgcn_update_dpp(0, hi, 0x4e, 0xf, 0xf, false);
      break;
    case 2:
      lo = __builtin_amdgcn_update_dpp(0, lo, 0x141, 0xf, 0xf, false);
      hi = __builtin_amdgcn_update_dpp(0, hi, 0x141, 0xf, 0xf, false);
      break;
    default:
      lo = __builtin_amdgcn_update_dpp(0, lo, 0x140, 0xf, 0xf, false);
      hi = __builtin_amdgcn_update_dpp(0, hi, 0x140, 0xf, 0xf, false);
      break;
  }
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Wave-wide fp64 sum (uniform result): xor-1 and xor-2 quad swaps and the half-row and row
// mirrors give every lane its 16-lane row's sum; the four rows are added in row order.
GLM52_DEV double wave_sum_f64_dpp(double v) {
  v += dpp_f64(v, 0);
  v += dpp_f64(v, 1);
  v += dpp_f64(v, 2);
  v += dpp_f64(v, 3);
  auto row = [&](int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
  };
  return ((row(0) + row(16)) + row(32)) + row(48);
}

// fp64 dot products of the token row (held as yr) with two gate rows, each as four
// interleaved partial sums (any order of exact products rounds to the same fp32)
template <int NQ>
GLM52_DEV void dot2_f64(const uint4 (&yr)[NQ], const uint16_t* g0, const uint16_t* g1,
                        double* out0, double* out1) {
  const int lane = threadIdx.x % kWave;
  uint4 a[NQ], b[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {  // every load in flight before the first product
    a[q] = *reinterpret_cast<const uint4*>(g0 + (lane + kWave * q) * 8);
    b[q] = *reinterpret_cast<const uint4*>(g1 + (lane + kWave * q) * 8);
  }
  double s0[4] = {0.0, 0.0, 0.0, 0.0}, s1[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    float yf[8], af[8], bf[8];
    unpack8(yr[q], yf);
    unpack8(a[q], af);
    unpack8(b[q], bf);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s0[i % 4] = fma((double)yf[i], (double)af[i], s0[i % 4]);
      s1[i % 4] = fma((double)yf[i], (double)bf[i], s1[i % 4]);
    }
  }
  *out0 = wave_sum_f64_dpp((s0[0] + s0[1]) + (s0[2] + s0[3]));
  *out1 = wave_sum_f64_dpp((s1[0] + s1[1]) + (s1[2] + s1[3]));
}

// One wave per token, four tokens per workgroup; H = NQ * 512.  part: the KS fp32
// partials, or null when KS == 1 (the logits array then holds L~).
template <int NQ>
__global__ __launch_bounds__(256) void router_select_kernel(
    const uint16_t* __restrict__ y, int64_t sy, const uint16_t* __restrict__ gate, int64_t sg,
    const float* __restrict__ part, int KS, const float* __restrict__ ssw,
    const float* __restrict__ bias, float* __restrict__ logits,
    int64_t sl, float* __restrict__ topw, int64_t stw, int32_t* __restrict__ topi, int64_t sti,
    int T, int E, int topk, float scale, int norm_prob) {
  __shared__ float sel_s[4][8];
  __shared__ int sel_i[4][8];
  __shared__ int cand[4][kMaxE];
  const int lane = threadIdx.x % kWave;
  const int wv = threadIdx.x / kWave;
  const int64_t t = (int64_t)blockIdx.x * 4 + wv;
  const bool t_ok = t < T;  // wave-uniform

  // the token's y row, 16-byte chunk lane + 64 q per lane
  uint4 yr[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    yr[q] = t_ok ? *reinterpret_cast<const uint4*>(y + t * sy + (lane + kWave * q) * 8)
                 : make_uint4(0, 0, 0, 0);

  float bv[4];
  load_bias(bias, E, bv);
  float sy2 = 0.f;  // the row's sum of squares, from the registers
#pragma unroll
  for (int q = 0; q < NQ; ++q) sy2 += sumsq8(yr[q]);
  sy2 = wave_sum(sy2) * (1.0f + 0x1p-10f);  // an upper bound of the exact sum

  // L~ and the gate-row sums of squares of the lane's experts, the K slices' values
  // loaded eight at a time (all in flight) and summed in slice order
  double la[4] = {0.0, 0.0, 0.0, 0.0};
  float sw[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < KS; k0 += 8) {
    float pv[8][4], wv8[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = lane + j * kWave;
        const bool ok = t_ok && e < E && k0 + i < KS;
        pv[i][j] = ok ? (part ? part[((int64_t)(k0 + i) * T + t) * E + e] : logits[t * sl + e]) : 0.f;
        wv8[i][j] = ok ? ssw[(int64_t)(k0 + i) * E + e] : 0.f;
      }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        la[j] += (double)pv[i][j];
        sw[j] += wv8[i][j];
      }
  }

  float sc[4], key[4];
  uint32_t ol[4], oh[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    sc[j] = 0.f;
    key[j] = -INFINITY;
    ol[j] = 0u;
    oh[j] = 0u;
    if (t_ok && e < E) {
      const float l = (float)la[j];
      if (part) logits[t * sl + e] = l;
      const float sw2 = sw[j] * (1.0f + 0x1p-10f);
      const float bnd = 2.5f * 0x1p-16f * __fsqrt_rn(sy2 * sw2) * (1.0f + 0x1p-20f) +
                        0x1p-21f * fabsf(l) + 1e-30f;
      const float b = bv[j];
      const float d = 0x1p-17f + fabsf(b) * 0x1p-22f;
      float lo = -INFINITY, hi = INFINITY;
      if (__builtin_isfinite(l) && __builtin_isfinite(b) && __builtin_isfinite(bnd)) {
        lo = (sig_fast(l - bnd) + b) - d;
        hi = (sig_fast(l + bnd) + b) + d;
      }
      ol[j] = key_order(lo);
      oh[j] = key_order(hi);
    }
  }

  // the k-th largest lower bound (as an order key): k rounds of a wave-wide max
  uint32_t kth = 0u;
  {
    uint32_t ou[4] = {ol[0], ol[1], ol[2], ol[3]};
    for (int r = 0; r < topk; ++r) {
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
      const int wl = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)holders) - 1);
      if (lane == wl) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (j == bj) ou[j] = 0u;
      }
      kth = m;
    }
  }

  // the candidates, listed in expert order
  uint32_t absent = 0u;
  int nc = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool c = t_ok && lane + j * kWave < E && oh[j] >= kth;
    if (!c) absent |= 1u << j;
    const uint64_t m = __ballot(c);
    if (c) cand[wv][nc + __popcll(m & ((1ull << lane) - 1ull))] = lane + j * kWave;
    nc += __popcll(m);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the list is written (one wave)

  // exact logits of the candidates, two at a time; the owner lane of each takes its score
  // and key
  for (int i = 0; i < nc; i += 2) {
    const int e0 = cand[wv][i];
    const int e1 = i + 1 < nc ? cand[wv][i + 1] : e0;
    double d0, d1;
    dot2_f64<NQ>(yr, gate + (int64_t)e0 * sg, gate + (int64_t)e1 * sg, &d0, &d1);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = u ? e1 : e0;
      const float lx = (float)(u ? d1 : d0);
      const float s = (float)(1.0 / (1.0 + exp(-(double)lx)));
      if (lane == e % kWave) {
        const int j = e / kWave;
        const float b = j == 0 ? bv[0] : j == 1 ? bv[1] : j == 2 ? bv[2] : bv[3];
        const float k2 = bias ? s + b : s;
        const float kk = (k2 != k2) ? -INFINITY : k2;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (q == j) {
            sc[q] = s;
            key[q] = kk;
          }
        logits[t * sl + e] = lx;
      }
    }
  }
  topk_rank(sc, key, E, t_ok ? topk : 0, sel_s[wv], sel_i[wv], absent);
  __syncthreads();
  if (t_ok && lane < topk) {
    float w;
    int id;
    topk_weight(sel_s[wv], sel_i[wv], topk, scale, norm_prob, &w, &id);
    topw[t * stw + lane] = w;
    topi[t * sti + lane] = id;
  }
}

// K split for T tokens: about 256 workgroups (one per CU), at most 32 slices, each a
// multiple of 64 k
int select_ks(int T, int H) {
  const int tblocks = (T + kTok - 1) / kTok;
  int ks = 1;
  while (tblocks * ks < 256 && ks < 32 && (H % (64 * ks * 2)) == 0) ks *= 2;
  return ks;
}

}  // namespace

namespace glm52 {

int64_t router_select_workspace_bytes(int T, int H, int E) {
  if (T <= 0 || H <= 0 || E <= 0) return 0;
  const int ks = select_ks(T, H);
  int64_t b = (int64_t)ks * E * 4 + 256;
  if (ks > 1) b += (int64_t)ks * T * E * 4;
  return b;
}

// The two launches; the caller has checked the operands.
int launch_router_select(const uint16_t* y, int64_t sy, const uint16_t* gate, int64_t sg,
                         float* logits, int64_t sl, void* workspace, int64_t workspace_bytes,
                         const float* bias, float* topw, int64_t stw, int32_t* topi, int64_t sti,
                         int T, int H, int E, int topk, float scale, int norm_prob,
                         hipStream_t st) {
  if ((H != 4096 && H != 6144 && H != 8192) || E > kMaxE || E < topk || (E % 4) ||
      (sg % 8) || sg < H || (reinterpret_cast<uintptr_t>(gate) & 15u))
    return GLM52_EUNSUPPORTED;
  if (T == 0) return GLM52_OK;
  const int ks = select_ks(T, H);
  if (!workspace || workspace_bytes < router_select_workspace_bytes(T, H, E) ||
      (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return GLM52_EINVAL;
  float* ssw = static_cast<float*>(workspace);
  float* part = ks > 1 ? reinterpret_cast<float*>(
                             (reinterpret_cast<uintptr_t>(ssw + (int64_t)ks * E) + 255) & ~uintptr_t(255))
                       : nullptr;
  dim3 grid((T + kTok - 1) / kTok, ks);
  router_approx_kernel<<<grid, 256, 0, st>>>(y, sy, gate, sg, T, H, E, ks > 1 ? part : logits,
                                             ks > 1 ? (int64_t)E : sl, ssw);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  const unsigned nb = (unsigned)((T + 3) / 4);
  switch (H / 512) {
    case 8:
      router_select_kernel<8><<<nb, 256, 0, st>>>(y, sy, gate, sg, part, ks, ssw, bias, logits,
                                                  sl, topw, stw, topi, sti, T, E, topk, scale, norm_prob);
      break;
    case 12:
      router_select_kernel<12><<<nb, 256, 0, st>>>(y, sy, gate, sg, part, ks, ssw, bias, logits,
                                                   sl, topw, stw, topi, sti, T, E, topk, scale, norm_prob);
      break;
    default:
      router_select_kernel<16><<<nb, 256, 0, st>>>(y, sy, gate, sg, part, ks, ssw, bias, logits,
                                                   sl, topw, stw, topi, sti, T, E, topk, scale, norm_prob);
      break;
  }
  GLM52_RETURN_LAUNCH();
}

}  // namespace glm52
