// Router for T > 16 tokens on the gate's rows ([E, H], K contiguous), gfx950: logits on
// bf16 MFMA with a rigorous error bound, then the exact rule only where it decides.
//
// The exact rule (router.hip): logit = fp32(sum_k y[k] * w[e, k]) with the exact
// products summed in fp64; s = fp32(sigmoid) in fp64; key = fp32(s + bias); the k largest
// keys in descending order, lower index first on ties; weights from the selected s.
// Evaluating every logit that way costs an fp64 GEMM.  Here:
//
// 1. router_approx_kernel: L~[t, e] on `v_mfma_f32_32x32x16_bf16`.  The products are exact
//    in fp32; each accumulator runs a chain of eight MFMAs (128 k), and the chains of a K
//    slice are summed in fp32.  An MFMA adds 16 products to its accumulator with at most 16
//    roundings of a partial sum no larger than |acc| + its |products|, so a chain of eight
//    errs by at most 16 * 9 * 2^-23 = 1.125 * 2^-16 times the chain's sum of |products|;
//    each of the m <= H / 128 additions of a chain into the slice sum errs by at most
//    2^-24 times the slice's sum of |products| (m * 2^-24 <= 0.25 * 2^-16 at H = 8192).
//    The slices' fp32 sums are added in fp64 and rounded once, so |L~ - sum| <=
//    1.375 * 2^-16 * sum_k |y_k w_k| + 2^-24 |L~|, and sum_k |y_k w_k| <= ||y|| ||w_e||
//    (Cauchy-Schwarz).  The kernel also returns the sums of squares of the token rows and
//    of the gate rows over each slice.  A workgroup owns 64 tokens (128 from 4096 tokens)
//    x all experts of one K slice (K is split until about 256 workgroups run; fp32
//    partials), its eight waves reading 2 x 2 (2 x 1) blocks of 32 x 32 from a three-stage
//    LDS ring of 64-k stages (one 128-byte segment per row and stage).
// 2. router_select_kernel, one wave per token: from L~ and the bound
//    B = 2.5 * 2^-16 * ||y|| ||w_e|| + 2^-21 |L~| (above the bound of 1. plus the fp32
//    rounding of the exact logit), each expert's exact key lies in
//    [lo, hi] = [sig(L~ - B) + b - d, sig(L~ + B) + b + d] (d covers the fp32 roundings
//    and the fast sigmoid).  Every expert of the exact top k has key >= the k-th largest
//    lo, so the candidates {e : hi_e >= that} hold the whole top k, and no other expert
//    can tie with its k-th key.  Only the candidates (about k per token) get the exact
//    logit -- an fp64 dot product of y and the gate row, eight (then four) rows per pass
//    over the token row -- and the exact top k is taken among them by rank: the same ids,
//    order and weights as the exact rule over all experts.  Non-finite values make every
//    expert a candidate.
//
// The logits written are exact for the candidates (so for every selected expert) and
// L~ rounded to fp32 elsewhere (within B of the exact logit).
#include "moe_gemm.h"
#include "select.h"

using namespace glm52;

namespace {

constexpr int kBk = 64;                  // k per LDS stage (one 128-byte segment of a row)
constexpr int kStages = 3;               // LDS ring
constexpr int kWaves = 8;                // waves per workgroup of the approximate pass
constexpr int kGateIps = kMaxE / (8 * kWaves);  // loads per wave and stage: 8 rows each

// tokens per workgroup of the approximate pass: 128 from 4096 tokens, else 64 (more
// workgroups for the smaller batches)
constexpr int kBigTokT = 4096;
inline int approx_tok(int T) { return T >= kBigTokT ? 128 : 64; }

GLM52_DEV float sumsq8(const uint4& v) {
  float f[8];
  unpack8(v, f);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s = fmaf(f[i], f[i], s);
  return s;
}

// grid = ceil(T / TOK) * KS; block = 512.  With TB = TOK / 64 token blocks (of 32) per
// wave, wave w computes expert blocks 2 (w % 4) + f (of 32, f < 2) against token blocks
// TB (w / 4) + j (j < TB).  out: KS == 1: L~ into logits [T, E] (row stride so); else
// fp32 partials part[ks][T][E].  ssw[ks][E] / ssy[ks][T]: the gate rows' / the token rows'
// sums of squares over slice ks (fp32, one chain of at most H / 2 fused multiply-adds per
// lane: within 2^-11 relative of the exact sums).
template <int TOK>
__global__ __launch_bounds__(512) void router_approx_kernel(
    const uint16_t* __restrict__ y, int64_t sy, const uint16_t* __restrict__ gate, int64_t sg,
    int T, int H, int E, int KS, float* __restrict__ out, int64_t so, float* __restrict__ ssw,
    float* __restrict__ ssy) {
  constexpr int kTok = TOK;
  constexpr int TB = TOK / 64;                      // token blocks per wave
  constexpr int kStageElems = (kMaxE + kTok) * kBk; // gate rows (E padded to 256) + token rows
  constexpr int kTokIps = kTok / (8 * kWaves);      // token-row loads per wave and stage
  constexpr int kIps = kGateIps + kTokIps;
  __shared__ __attribute__((aligned(1024))) uint16_t ring[kStages * kStageElems];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int l32 = lane % 32, h = lane / 32;
  // the workgroups of one K slice run on the same XCDs (hardware workgroup h runs on XCD
  // h % 8), so the slice's gate rows are shared through those XCDs' L2: logical index L,
  // slice L / nb, token block L % nb
  const int nb = (T + kTok - 1) / kTok;
  const int nwg = nb * KS;
  const int xcd = blockIdx.x % 8, q8 = nwg / 8, r8 = nwg % 8;
  const int L = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + blockIdx.x / 8;
  const int ks = L / nb, tb = L % nb;
  const int t0 = tb * kTok;
  const int ksl = H / KS;
  const int kbeg = ks * ksl;
  const int nk = ksl / kBk;

  // load slots: lane -> row lane / 8 of an 8-row slab (a 128-byte segment per row),
  // physical 16-byte chunk lane % 8 holding logical chunk (lane % 8) ^ ((row / 2) % 8): the
  // MFMA operand reads of 16 consecutive rows then hit 16 different bank groups
  const int dr = lane >> 3;
  auto chunk_of = [&](int slab) { return (lane & 7) ^ ((((slab & 1) << 2) + (dr >> 1)) & 7); };
  uint32_t goff[kGateIps];
#pragma unroll
  for (int i = 0; i < kGateIps; ++i) {
    const int slab = wv * kGateIps + i;
    const int er = min(slab * 8 + dr, E - 1);  // padded experts re-read a real row
    goff[i] = (uint32_t)((er * sg + chunk_of(slab) * 8) * 2);
  }
  const uint16_t* ybase = y + (int64_t)t0 * sy;
  uint32_t yoff[kTokIps];
#pragma unroll
  for (int i = 0; i < kTokIps; ++i) {
    const int slab = wv * kTokIps + i;  // kMaxE / 8 is even: same parity as its ring row
    yoff[i] = (uint32_t)((min(slab * 8 + dr, T - 1 - t0) * sy + chunk_of(slab) * 8) * 2);
  }
  const uint32_t ring_base = lds_addr(ring);

  // past the slice's last stage the loads keep their count (the waits stay constant) but
  // every lane reads the same 16 bytes
  auto issue = [&](int s) {
    const bool past = s >= nk;  // wave-uniform
    const int kc = kbeg + min(s, nk - 1) * kBk;
    const uint32_t sb = ring_base + (uint32_t)((s % kStages) * kStageElems * 2);
#pragma unroll
    for (int i = 0; i < kGateIps; ++i)
      dma16s(gate + kc, past ? 0u : goff[i], sb + (uint32_t)((wv * kGateIps + i) * 8 * kBk * 2));
#pragma unroll
    for (int i = 0; i < kTokIps; ++i)
      dma16s(ybase + kc, past ? 0u : yoff[i],
             sb + (uint32_t)((kMaxE + (wv * kTokIps + i) * 8) * kBk * 2));
  };

  const int eb0 = (wv % 4) * 2, tb0 = (wv / 4) * TB;
  floatx16_t acc[2][TB];   // [expert block][token block]: chains of at most eight MFMAs
  floatx16_t acc2[2][TB];  // the chains' sum
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[f][tb][i] = 0.f;
        acc2[f][tb][i] = 0.f;
      }
  float ysq = 0.f;  // waves w % 4 < TB: the sum of squares of token block tb0 + w % 4's row l32 (half h)
  // the gate rows' sums of squares over the slice: with at least 8 token blocks, workgroup
  // tb < 8 takes expert block tb from the operands of wave tb / 2 (f = tb % 2); else a
  // loop over global memory after the main loop
  const bool gsq_on = nb >= 8 && tb < 8 && wv == tb / 2;
  float gsq = 0.f;
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue(s);
#pragma unroll 1
  for (int s = 0; s < nk; ++s) {
    GLM52_WAIT_VMCNT((kStages - 2) * kIps);  // stage s landed for this wave
    __syncthreads();                          // ... for every wave; buffer s - 1 is free
    issue(s + kStages - 1);
    const uint16_t* sb = ring + (s % kStages) * kStageElems;
#pragma unroll
    for (int kk = 0; kk < kBk / 16; ++kk) {
      const int rd = l32 * kBk + (((2 * kk + h) ^ ((l32 >> 1) & 7)) * 8);
      uint4 a[2], b[TB];
#pragma unroll
      for (int f = 0; f < 2; ++f)
        a[f] = *reinterpret_cast<const uint4*>(sb + ((eb0 + f) * 32) * kBk + rd);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb)
        b[tb] = *reinterpret_cast<const uint4*>(sb + (kMaxE + (tb0 + tb) * 32) * kBk + rd);
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[f][tb] = mfma32(a[f], b[tb], acc[f][tb]);
      // both sums, then a select of the result: a runtime choice between array elements
      // becomes a dynamically indexed private array (LDS or scratch), and a scratch load
      // inside this loop would wait for the ring's loads
      if (wv % 4 < TB) {
        const float q0 = sumsq8(b[0]), q1 = TB == 2 ? sumsq8(b[TB - 1]) : 0.f;
        ysq += (TB == 2 && wv % 4 == 1) ? q1 : q0;
      }
      if (gsq_on) {
        const float q0 = sumsq8(a[0]), q1 = sumsq8(a[1]);
        gsq += (tb & 1) ? q1 : q0;
      }
    }
    if ((s & 1) == 1 || s == nk - 1) {  // chains of at most eight MFMAs, then into the sum
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            acc2[f][tb][i] += acc[f][tb][i];
            acc[f][tb][i] = 0.f;
          }
    }
  }
  GLM52_WAIT_VMCNT(0);  // the clamped loads past the slice
  if (wv % 4 < TB) {
    ysq += __shfl_xor(ysq, 32, kWave);
    const int t = t0 + (tb0 + wv % 4) * 32 + l32;
    if (h == 0 && t < T) ssy[(int64_t)ks * T + t] = ysq;
  }

  if (gsq_on) {
    gsq += __shfl_xor(gsq, 32, kWave);
    const int e = tb * 32 + l32;
    if (h == 0 && e < E) ssw[(int64_t)ks * E + e] = gsq;
  }
  // fewer than 8 token blocks: row e by workgroup e % nb, a wave per row, from global
  // memory (the rows were just streamed: L2 hits)
  for (int e = tb + wv * nb; nb < 8 && e < E; e += kWaves * nb) {
    const uint16_t* grow = gate + (int64_t)e * sg + kbeg;
    float q = 0.f;
    for (int c = lane; c < ksl / 8; c += kWave) q += sumsq8(*reinterpret_cast<const uint4*>(grow + c * 8));
    q = wave_sum(q);
    if (lane == 0) ssw[(int64_t)ks * E + e] = q;
  }

  // result i of lane (l32, h) in block (f, tb): expert (eb0 + f) * 32 + 8 (i / 4) + 4 h +
  // i % 4, token t0 + 32 (tb0 + tb) + l32
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int t = t0 + (tb0 + tb) * 32 + l32;
    if (t < T) {
      float* orow = KS == 1 ? out + (int64_t)t * so : out + ((int64_t)ks * T + t) * E;
      const bool al16 = (reinterpret_cast<uintptr_t>(orow) & 15u) == 0;
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e = (eb0 + f) * 32 + 8 * q + 4 * h;  // E % 4 == 0: e < E covers e + 3
          if (e < E) {
            if (al16) {
              *reinterpret_cast<float4*>(orow + e) =
                  make_float4(acc2[f][tb][4 * q], acc2[f][tb][4 * q + 1], acc2[f][tb][4 * q + 2],
                              acc2[f][tb][4 * q + 3]);
            } else {
#pragma unroll
              for (int u = 0; u < 4; ++u) orow[e + u] = acc2[f][tb][4 * q + u];
            }
          }
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

// Exact logits of G candidate experts of one token, by one wave: fp64 dot products of
// the token row and the gate rows ids[0, G) (an LDS list), lane l holding the 16-byte
// chunks l + 64 q of every row, one fp64 accumulator per row (any order of the exact
// products rounds to the same fp32).  One K step loads the token chunk and the G gate
// chunks, then converts the token chunk once for all G rows.  Results are wave-uniform.
template <int NQ, int G>
GLM52_DEV void dots_f64(const uint16_t* __restrict__ yrow, const uint16_t* __restrict__ gate,
                        int64_t sg, const int* ids, double (&out)[G]) {
  const int lane = threadIdx.x % kWave;
  const uint16_t* g[G];
#pragma unroll
  for (int c = 0; c < G; ++c) g[c] = gate + (int64_t)__builtin_amdgcn_readfirstlane(ids[c]) * sg;
  double acc[G];
#pragma unroll
  for (int c = 0; c < G; ++c) acc[c] = 0.0;
#pragma unroll 2
  for (int q = 0; q < NQ; ++q) {
    const int off = (lane + kWave * q) * 8;
    const uint4 yv = *reinterpret_cast<const uint4*>(yrow + off);
    uint4 gv[G];
#pragma unroll
    for (int c = 0; c < G; ++c) gv[c] = *reinterpret_cast<const uint4*>(g[c] + off);
    float yf[8];
    unpack8(yv, yf);
    double yd[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) yd[i] = (double)yf[i];
#pragma unroll
    for (int c = 0; c < G; ++c) {
      float gf[8];
      unpack8(gv[c], gf);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[c] = fma(yd[i], (double)gf[i], acc[c]);
    }
  }
#pragma unroll
  for (int c = 0; c < G; ++c) out[c] = wave_sum_f64_dpp(acc[c]);
}

// One wave per token, four tokens per workgroup; H = NQ * 512.  part: the KS fp32
// partials, or null when KS == 1 (the logits array then holds L~).  ssy[ks][t] / ssw[ks][e]:
// the token rows' / gate rows' sums of squares over slice ks (from router_approx_kernel).
// rstd (optional, the half-fused pre-norm epilogue): every logit is the dot product's fp32
// value times rstd[t] (one fp32 product) -- the exact rule's logit fl(fl(dot) * r) for the
// candidates, fl(L~ * r) elsewhere.  With |L~ - dot| <= B, |fl(L~ r) - fl(fl(dot) r)| <=
// r B (1 + 2^-23) + 3 * 2^-24 |L~ r|, which B' = r B (1 + 2^-20) + 2^-21 |fl(L~ r)| covers;
// the candidates are then chosen from B' exactly as from B.
template <int NQ>
__global__ __launch_bounds__(256) void router_select_kernel(
    const uint16_t* __restrict__ y, int64_t sy, const uint16_t* __restrict__ gate, int64_t sg,
    const float* __restrict__ part, int KS, const float* __restrict__ ssw,
    const float* __restrict__ ssy, const float* __restrict__ bias, float* __restrict__ logits,
    int64_t sl, float* __restrict__ topw, int64_t stw, int32_t* __restrict__ topi, int64_t sti,
    int T, int E, int topk, float scale, int norm_prob, const float* __restrict__ rstd) {
  __shared__ float sel_s[4][8];
  __shared__ int sel_i[4][8];
  __shared__ int cand[4][kMaxE];
  __shared__ float clg[4][kMaxE];          // the candidates' exact logits (fp32)
  __shared__ uint64_t cord[4][kMaxE];      // (key order, 0xffff - expert): larger ranks first
  const int lane = threadIdx.x % kWave;
  const int wv = threadIdx.x / kWave;
  const int64_t t = (int64_t)blockIdx.x * 4 + wv;
  const bool t_ok = t < T;  // wave-uniform

  float bv[4];
  load_bias(bias, E, bv);
  const float rs = rstd && t_ok ? rstd[t] : 1.0f;

  // L~, the gate rows' sums of squares of the lane's experts and the token row's sum of
  // squares: the K slices' values loaded eight at a time (all in flight), summed in order
  double la[4] = {0.0, 0.0, 0.0, 0.0};
  float sw[4] = {0.f, 0.f, 0.f, 0.f};
  float sy2 = 0.f;
  for (int k0 = 0; k0 < KS; k0 += 4) {
    float pv[4][4], wv8[4][4], yv8[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      yv8[i] = t_ok && k0 + i < KS ? ssy[(int64_t)(k0 + i) * T + t] : 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = lane + j * kWave;
        const bool ok = t_ok && e < E && k0 + i < KS;
        pv[i][j] = ok ? (part ? part[((int64_t)(k0 + i) * T + t) * E + e] : logits[t * sl + e]) : 0.f;
        wv8[i][j] = ok ? ssw[(int64_t)(k0 + i) * E + e] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sy2 += yv8[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        la[j] += (double)pv[i][j];
        sw[j] += wv8[i][j];
      }
    }
  }
  sy2 *= 1.0f + 0x1p-10f;  // an upper bound of the exact sum

  uint32_t ol[4], oh[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    ol[j] = 0u;
    oh[j] = 0u;
    if (t_ok && e < E) {
      const float l0 = (float)la[j];
      const float l = rstd ? l0 * rs : l0;
      if (part || rstd) logits[t * sl + e] = l;
      const float sw2 = sw[j] * (1.0f + 0x1p-10f);
      float bnd = 2.5f * 0x1p-16f * __fsqrt_rn(sy2 * sw2) * (1.0f + 0x1p-20f) +
                  0x1p-21f * fabsf(l0) + 1e-30f;
      if (rstd) bnd = bnd * rs * (1.0f + 0x1p-20f) + 0x1p-21f * fabsf(l) + 1e-30f;
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
  int nc = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool c = t_ok && lane + j * kWave < E && oh[j] >= kth;
    const uint64_t m = __ballot(c);
    if (c) cand[wv][nc + __popcll(m & ((1ull << lane) - 1ull))] = lane + j * kWave;
    nc += __popcll(m);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the list is written (one wave)

  // exact logits of the candidates, eight at a time, then four at a time (the last group
  // repeats its first row where the list runs out)
  const uint16_t* yrow = y + t * sy;
  int i = 0;
  for (; i + 8 <= nc; i += 8) {
    double d[8];
    dots_f64<NQ, 8>(yrow, gate, sg, &cand[wv][i], d);
    if (lane < 8) {
      double v = d[0];
#pragma unroll
      for (int c = 1; c < 8; ++c) v = lane == c ? d[c] : v;
      clg[wv][i + lane] = rstd ? (float)v * rs : (float)v;
    }
  }
  for (; i < nc; i += 4) {
    if (lane < 4 && i + lane >= nc) cand[wv][i + lane] = cand[wv][i];
    __builtin_amdgcn_s_waitcnt(0xc07f);
    double d[4];
    dots_f64<NQ, 4>(yrow, gate, sg, &cand[wv][i], d);
    if (lane < 4 && i + lane < nc) {
      double v = d[0];
#pragma unroll
      for (int c = 1; c < 4; ++c) v = lane == c ? d[c] : v;
      clg[wv][i + lane] = rstd ? (float)v * rs : (float)v;
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);

  // each candidate's score and key (fp64 sigmoid, one rounding), its logit stored
  for (int c = lane; c < nc; c += kWave) {
    const int e = cand[wv][c];
    const float lx = clg[wv][c];
    const float s = (float)(1.0 / (1.0 + exp(-(double)lx)));
    const float k2 = bias ? s + bias[e] : s;
    const float kk = (k2 != k2) ? -INFINITY : k2;
    logits[t * sl + e] = lx;
    clg[wv][c] = s;
    cord[wv][c] = ((uint64_t)key_order(kk) << 32) | (uint32_t)(0xffff - e);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);

  // slot of each candidate: the number of candidates ahead of it under (key descending,
  // expert ascending); the top k take slots 0 .. k-1
  for (int c = lane; c < nc; c += kWave) {
    const uint64_t me = cord[wv][c];
    int rank = 0;
    for (int c2 = 0; c2 < nc; ++c2) rank += cord[wv][c2] > me ? 1 : 0;
    if (rank < topk) {
      sel_s[wv][rank] = clg[wv][c];
      sel_i[wv][rank] = cand[wv][c];
    }
  }
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
  const int tok = approx_tok(T);
  const int tblocks = (T + tok - 1) / tok;
  int ks = 1;
  while (tblocks * ks < 256 && ks < 32 && (H % (64 * ks * 2)) == 0) ks *= 2;
  return ks;
}

}  // namespace

namespace glm52 {

int64_t router_select_workspace_bytes(int T, int H, int E) {
  if (T <= 0 || H <= 0 || E <= 0) return 0;
  const int ks = select_ks(T, H);
  int64_t b = (int64_t)ks * (E + T) * 4 + 256;
  if (ks > 1) b += (int64_t)ks * T * E * 4;
  return b;
}

// The two launches; the caller has checked the operands.
int launch_router_select(const uint16_t* y, int64_t sy, const uint16_t* gate, int64_t sg,
                         float* logits, int64_t sl, void* workspace, int64_t workspace_bytes,
                         const float* bias, float* topw, int64_t stw, int32_t* topi, int64_t sti,
                         int T, int H, int E, int topk, float scale, int norm_prob,
                         hipStream_t st, const float* rstd) {
  if ((H != 4096 && H != 6144 && H != 8192) || E > kMaxE || E < topk || (E % 4) ||
      (sg % 8) || sg < H || (reinterpret_cast<uintptr_t>(gate) & 15u))
    return GLM52_EUNSUPPORTED;
  if (T == 0) return GLM52_OK;
  const int ks = select_ks(T, H);
  // a workspace sized for the exact path only: the caller falls back to it
  if (!workspace || workspace_bytes < router_select_workspace_bytes(T, H, E) ||
      (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return GLM52_EUNSUPPORTED;
  float* ssw = static_cast<float*>(workspace);
  float* ssy = ssw + (int64_t)ks * E;
  float* part = ks > 1 ? reinterpret_cast<float*>(
                             (reinterpret_cast<uintptr_t>(ssy + (int64_t)ks * T) + 255) & ~uintptr_t(255))
                       : nullptr;
  const int tok = approx_tok(T);
  const unsigned grid = (unsigned)(((T + tok - 1) / tok) * ks);
  if (tok == 128)
    router_approx_kernel<128><<<grid, 64 * kWaves, 0, st>>>(
        y, sy, gate, sg, T, H, E, ks, ks > 1 ? part : logits, ks > 1 ? (int64_t)E : sl, ssw, ssy);
  else
    router_approx_kernel<64><<<grid, 64 * kWaves, 0, st>>>(
        y, sy, gate, sg, T, H, E, ks, ks > 1 ? part : logits, ks > 1 ? (int64_t)E : sl, ssw, ssy);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  const unsigned nb = (unsigned)((T + 3) / 4);
  switch (H / 512) {
    case 8:
      router_select_kernel<8><<<nb, 256, 0, st>>>(y, sy, gate, sg, part, ks, ssw, ssy, bias, logits,
                                                  sl, topw, stw, topi, sti, T, E, topk, scale, norm_prob, rstd);
      break;
    case 12:
      router_select_kernel<12><<<nb, 256, 0, st>>>(y, sy, gate, sg, part, ks, ssw, ssy, bias, logits,
                                                   sl, topw, stw, topi, sti, T, E, topk, scale, norm_prob, rstd);
      break;
    default:
      router_select_kernel<16><<<nb, 256, 0, st>>>(y, sy, gate, sg, part, ks, ssw, ssy, bias, logits,
                                                   sl, topw, stw, topi, sti, T, E, topk, scale, norm_prob, rstd);
      break;
  }
  GLM52_RETURN_LAUNCH();
}

}  // namespace glm52
