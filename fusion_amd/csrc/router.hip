// GLM-5.2 router: fp32 logits, sigmoid scores, noaux_tc bias-corrected top-k, gfx950.
//
// Semantics restate `glm52/reference.py:46-79` (n_group = topk_group = 1, so there is no
// group mask):
//
//   logits = y . Wg^T                          (fp32 result)
//   s      = sigmoid(logits)                   (fp32)
//   choice = s + bias                          (fp32 add; bias may be absent)
//   ids    = the k largest choices, in descending order, lower index first on ties
//   w      = s[ids] / max(sum_k s[ids], 1e-20) * scale      (or s[ids] * scale)
//
// Bit-exact routing.  A 6144-term fp32 dot product depends on summation order, so two
// implementations that sum differently can disagree on an id whenever the 8th and 9th
// choices are within an ulp or two.  The arithmetic is therefore pinned to a rule that
// does not depend on order: every bf16 x bf16 product is exact in fp64, the sum is
// carried in fp64 (its rounding error is far below half an fp32 ulp), and the result is
// rounded once to fp32.  The sigmoid is evaluated in fp64 and rounded once to fp32.  The
// CPU oracle applies the same rule, so ids agree bit for bit.
//
// Two mappings, picked by the gate's layout.  Rows ([E, H], K contiguous, used at small
// T): a workgroup per expert row and group of 4 tokens (`router_rows_kernel`).  Columns
// ([H, E], the reference kernel's layout): the logits run on the fp64 matrix cores
// (`v_mfma_f64_16x16x4_f64`), a workgroup per 32 tokens x all experts of a K slice, gate
// and token chunks staged through two LDS buffers (`router_logits_kernel`).  Small T
// splits K over KS workgroups; their fp64 partials land in a caller-provided workspace
// and are summed in a fixed order (by `router_reduce_kernel`, or inside the top-k kernel)
// before the single rounding to fp32.
//
// Top-k: one wave per token, k rounds of a wave-wide argmax under the (choice
// descending, index ascending) order (select.h).
//
// The gate weight layout is the reference kernel's [H, E] (`wgt_from_gate`,
// `glm52/kernels/norm_router.py:251-255`).
#include "select.h"

using namespace glm52;

typedef double doublex4_t __attribute__((ext_vector_type(4)));

namespace {

constexpr int KC = 64;    // K split granularity: every split slice is a multiple of it
constexpr int TB = 32;    // tokens per workgroup of the [H, E] mapping
constexpr int EMAX = kMaxE;

GLM52_DEV doublex4_t mfma64(double a, double b, doublex4_t c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Bank spread of the gate rows in LDS: expert column c's slot in a row holds two halves
// (experts c*16 .. +7 and c*16+8 .. +15); half h is stored at position h ^ gsw(c), so the 16
// lanes of one operand read cover distinct bank groups.
GLM52_DEV int gsw(int c) { return ((c >> 2) ^ (c >> 3)) & 1; }

// [H, E] mapping on `v_mfma_f64_16x16x4f64`.  grid = (ceil(T / 32), KS); block = 256.
// A workgroup owns 32 tokens x all (<= 256) experts of one K slice; wave (th, eh) owns
// tokens th*16 .. +15 and the experts c*16 + eh*8 + j (c < 16 the MFMA column, j < 8 its
// tile), so a lane's 8 B operands of one MFMA step are 8 adjacent gate entries (one
// 16-byte LDS read).  K is walked in chunks of KCH through two LDS buffers; inside a
// chunk, lane group g of an MFMA takes k = g * KCH/4 + s at step s (the sum is order-
// free, the same k feeds both operands), so a lane's token operands of the whole chunk
// are KCH/4 adjacent y entries.  The next chunk is loaded into registers while the
// current one is multiplied.  Results are staged through LDS for coalesced stores: fp32
// logits when KS == 1, else fp64 partials part[ks, t, e].
template <bool WG_F32>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ y, int64_t sy, const void* __restrict__ wg_raw, int64_t swg,
    float* __restrict__ logits, int64_t sl, double* __restrict__ part, int T, int H, int E,
    const float* __restrict__ rstd) {
  using WT = typename std::conditional<WG_F32, float, uint16_t>::type;
  constexpr int EPV = 16 / sizeof(WT);        // gate entries per 16-byte vector
  constexpr int CPR = EMAX / EPV;              // 16-byte vectors per gate row (32 or 64)
  constexpr int KCH = 2048 / CPR;              // k per chunk (64 bf16, 32 fp32): 32 KB / 64 KB
  constexpr int SPG = KCH / 4;                 // MFMA steps per chunk
  constexpr int YC = KCH / 8;                  // 16-byte y vectors per token row and chunk
  constexpr int YLD = KCH + 8;                 // y row pitch in LDS (bf16)
  constexpr int GSZ = KCH * EMAX * sizeof(WT); // bytes of one gate chunk: 32 KB
  static_assert(2 * GSZ >= TB * EMAX * 8, "the epilogue stage fits in the gate buffers");
  __shared__ __attribute__((aligned(16))) WT gs[2][KCH * EMAX];
  __shared__ __attribute__((aligned(16))) uint16_t ys[2][TB * YLD];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int c = lane % 16, g = lane / 16;
  const int th = wv & 1, eh = wv >> 1;
  const int t0 = blockIdx.x * TB;
  const int KS = gridDim.y;
  const int ksl = H / KS;
  const int kbeg = blockIdx.y * ksl;
  const int nch = ksl / KCH;
  const WT* wg = static_cast<const WT*>(wg_raw);

  // LDS element offset, inside a gate row, of 16-byte vector m (entries m*EPV .. +EPV-1)
  auto gpos = [](int m) {
    const int per_col = 16 / EPV;  // vectors per expert column (2 bf16, 4 fp32)
    const int cc = m / per_col, w = m % per_col;
    const int half = w / (per_col / 2), q = w % (per_col / 2);
    return (cc * per_col + ((half ^ gsw(cc)) * (per_col / 2)) + q) * EPV;
  };

  uint4 rg[8], ry = make_uint4(0, 0, 0, 0);
  auto gload = [&](int ch) {
    const int k0 = kbeg + ch * KCH;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = tid + i * 256;
      const int kk = q / CPR, m = q % CPR;
      rg[i] = m * EPV < E ? *reinterpret_cast<const uint4*>(wg + (int64_t)(k0 + kk) * swg + m * EPV)
                          : make_uint4(0, 0, 0, 0);
    }
    if (tid < TB * YC) {
      const int t = tid / YC, kc = tid % YC;
      ry = t0 + t < T ? *reinterpret_cast<const uint4*>(y + (int64_t)(t0 + t) * sy + k0 + kc * 8)
                      : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int b) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = tid + i * 256;
      const int kk = q / CPR, m = q % CPR;
      *reinterpret_cast<uint4*>(&gs[b][kk * EMAX + gpos(m)]) = rg[i];
    }
    if (tid < TB * YC) {
      const int t = tid / YC, kc = tid % YC;
      *reinterpret_cast<uint4*>(&ys[b][t * YLD + kc * 8]) = ry;
    }
  };

  doublex4_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = doublex4_t{0.0, 0.0, 0.0, 0.0};
  // the lane's 8 gate entries of a row: experts c*16 + eh*8 .. +7
  const int boff = gpos((c * 16 + eh * 8) / EPV);

  gload(0);
  sstore(0);
  __syncthreads();
  for (int ch = 0; ch < nch; ++ch) {
    const int cur = ch & 1;
    if (ch + 1 < nch) gload(ch + 1);
    float af[SPG];
    {
      const uint16_t* yr = &ys[cur][(th * 16 + c) * YLD + g * SPG];
#pragma unroll
      for (int v = 0; v < SPG / 8; ++v) unpack8(*reinterpret_cast<const uint4*>(yr + v * 8), af + v * 8);
    }
    const WT* gb = &gs[cur][(g * SPG) * EMAX + boff];
#pragma unroll
    for (int s = 0; s < SPG; ++s) {
      float wf[8];
      if constexpr (WG_F32) {
        const float4 w0 = *reinterpret_cast<const float4*>(gb + s * EMAX);
        const float4 w1 = *reinterpret_cast<const float4*>(gb + s * EMAX + 4);
        wf[0] = w0.x; wf[1] = w0.y; wf[2] = w0.z; wf[3] = w0.w;
        wf[4] = w1.x; wf[5] = w1.y; wf[6] = w1.z; wf[7] = w1.w;
      } else {
        unpack8(*reinterpret_cast<const uint4*>(gb + s * EMAX), wf);
      }
      const double a = (double)af[s];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = mfma64(a, (double)wf[j], acc[j]);
    }
    if (ch + 1 < nch) sstore(cur ^ 1);
    __syncthreads();
  }

  // fp64 MFMA result layout: register v of lane (c, g) is row g + 4 v (token), column c
  double* st = reinterpret_cast<double*>(&gs[0][0]);  // [TB][EMAX]
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int tl = th * 16 + g + 4 * v;
#pragma unroll
    for (int j = 0; j < 8; ++j) st[tl * EMAX + c * 16 + eh * 8 + j] = acc[j][v];
  }
  __syncthreads();
  const int nt = min(TB, T - t0);
  for (int q = tid; q < nt * E; q += 256) {
    const int tl = q / E, e = q % E;
    const double s = st[tl * EMAX + e];
    if (KS == 1) logits[(int64_t)(t0 + tl) * sl + e] = rstd ? (float)s * rstd[t0 + tl] : (float)s;
    else part[((int64_t)blockIdx.y * T + t0 + tl) * E + e] = s;
  }
}

// Row layout (gate as [E, H], rows contiguous), for small T: a workgroup per (gate row e,
// group of RT tokens).  Thread (w, l) owns the 16-byte chunks w * H/32 + l + 64 j of the
// gate row and of each token row (a wave takes a quarter of the row), and issues all of
// its loads before its first FMA, so a workgroup waits for one round of memory latency.
// fp64 FMAs; each token's four wave sums meet in wave order.
// grid = (E, ceil(T / RT)); block = 256.
constexpr int RT = 4;
constexpr int HMAX = 8192;
constexpr int RNJ = HMAX / 32 / kWave;  // chunks per lane of a quarter row (H <= HMAX)

template <bool WG_F32>
__global__ __launch_bounds__(256) void router_rows_kernel(
    const uint16_t* __restrict__ y, int64_t sy, const void* __restrict__ wg_raw, int64_t swe,
    float* __restrict__ logits, int64_t sl, int T, int H, int E, const float* __restrict__ rstd) {
  __shared__ double part[RT][4];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int e = blockIdx.x;
  const int t0 = blockIdx.y * RT;
  const int nt = min(RT, T - t0);
  const int qc = H / 32;
  uint4 yr[RT][RNJ];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int j = 0; j < RNJ; ++j) {
      const int c = wv * qc + lane + kWave * j;
      const bool ok = t < nt && lane + kWave * j < qc;
      yr[t][j] = ok ? *reinterpret_cast<const uint4*>(y + (int64_t)(t0 + t) * sy + c * 8)
                    : make_uint4(0, 0, 0, 0);
    }
  float wf[RNJ][8];
  if constexpr (WG_F32) {
    float4 g0[RNJ], g1[RNJ];
    const float* wr = static_cast<const float*>(wg_raw) + (int64_t)e * swe;
#pragma unroll
    for (int j = 0; j < RNJ; ++j) {
      const int c = wv * qc + lane + kWave * j;
      const bool ok = lane + kWave * j < qc;
      g0[j] = ok ? *reinterpret_cast<const float4*>(wr + c * 8) : make_float4(0.f, 0.f, 0.f, 0.f);
      g1[j] = ok ? *reinterpret_cast<const float4*>(wr + c * 8 + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < RNJ; ++j) {
      wf[j][0] = g0[j].x; wf[j][1] = g0[j].y; wf[j][2] = g0[j].z; wf[j][3] = g0[j].w;
      wf[j][4] = g1[j].x; wf[j][5] = g1[j].y; wf[j][6] = g1[j].z; wf[j][7] = g1[j].w;
    }
  } else {
    uint4 gr[RNJ];
    const uint16_t* wr = static_cast<const uint16_t*>(wg_raw) + (int64_t)e * swe;
#pragma unroll
    for (int j = 0; j < RNJ; ++j) {
      const int c = wv * qc + lane + kWave * j;
      gr[j] = lane + kWave * j < qc ? *reinterpret_cast<const uint4*>(wr + c * 8)
                                    : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < RNJ; ++j) unpack8(gr[j], wf[j]);
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    if (t < nt) {  // each reduction is 12 cross-lane moves: only the tokens that exist
      double acc = 0.0;
#pragma unroll
      for (int j = 0; j < RNJ; ++j) {
        float yf[8];
        unpack8(yr[t][j], yf);  // chunks past the row are zero
#pragma unroll
        for (int q = 0; q < 8; ++q) acc = fma((double)yf[q], (double)wf[j][q], acc);
      }
      acc = wave_sum_f64(acc);
      if (lane == 0) part[t][wv] = acc;
    }
  }
  __syncthreads();
  if (tid < nt) {
    const int t = tid;
    const double s = ((part[t][0] + part[t][1]) + part[t][2]) + part[t][3];
    logits[(int64_t)(t0 + t) * sl + e] = rstd ? (float)s * rstd[t0 + t] : (float)s;
  }
}

// logits[t, e] = fp32(sum_ks part[ks, t, e]), ks in order (times rstd[t] if given).
__global__ __launch_bounds__(256) void router_reduce_kernel(const double* __restrict__ part,
                                                            float* __restrict__ logits,
                                                            int64_t sl, int T, int E, int KS,
                                                            const float* __restrict__ rstd) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= (int64_t)T * E) return;
  const int64_t t = q / E;
  const int e = (int)(q % E);
  double s = 0.0;
  for (int ks0 = 0; ks0 < KS; ks0 += 8) {  // 8 loads in flight, adds in ks order
    double v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = ks0 + i < KS ? part[(int64_t)(ks0 + i) * T * E + q] : 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (ks0 + i < KS) s += v[i];
  }
  logits[t * sl + e] = rstd ? (float)s * rstd[t] : (float)s;
}

// One wave per token, four tokens per workgroup.  If `part` is non-null the fp64
// partials are reduced here in ks order (and the logits written); else logits are read.
__global__ __launch_bounds__(256) void router_topk_kernel(
    float* __restrict__ logits, int64_t sl, const double* __restrict__ part, int KS,
    const float* __restrict__ bias, float* __restrict__ topw, int64_t stw,
    int32_t* __restrict__ topi, int64_t sti, int T, int E, int topk, float scale,
    int norm_prob) {
  __shared__ float sel_s[4][8];
  __shared__ int sel_i[4][8];
  const int lane = threadIdx.x % kWave;
  const int wv = threadIdx.x / kWave;
  const int64_t t = (int64_t)blockIdx.x * 4 + wv;
  const bool t_ok = t < T;

  float lg[4], sc[4], key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + j * kWave;
    lg[j] = 0.f;
    if (t_ok && e < E) {
      if (part) {
        double s = 0.0;
        for (int ks0 = 0; ks0 < KS; ks0 += 8) {  // 8 loads in flight, adds in ks order
          double v[8];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            v[i] = ks0 + i < KS ? part[((int64_t)(ks0 + i) * T + t) * E + e] : 0.0;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (ks0 + i < KS) s += v[i];
        }
        lg[j] = (float)s;
        logits[t * sl + e] = lg[j];
      } else {
        lg[j] = logits[t * sl + e];
      }
    }
  }
  float bv[4];
  load_bias(bias, E, bv);
  topk_keys(lg, bv, bias != nullptr, E, t_ok, sc, key);
  topk_rank(sc, key, E, t_ok ? topk : 0, sel_s[wv], sel_i[wv]);
  __syncthreads();
  if (t_ok && lane < topk) {
    float w;
    int id;
    topk_weight(sel_s[wv], sel_i[wv], topk, scale, norm_prob, &w, &id);
    topw[t * stw + lane] = w;
    topi[t * sti + lane] = id;
  }
}

// K split for T tokens: enough workgroups for two per CU (512), at most 32 slices.
int choose_ks(int T, int H) {
  const int tblocks = (T + TB - 1) / TB;
  int ks = 1;
  while (tblocks * ks < 512 && ks < 32 && (H % (KC * ks * 2)) == 0) ks *= 2;
  return ks;
}

}  // namespace

namespace glm52 {
// router_select.hip: the bf16-MFMA logits with an error bound and the exact rule on the
// candidates, for T > 16 tokens on the gate's rows
int64_t router_select_workspace_bytes(int T, int H, int E);
int launch_router_select(const uint16_t* y, int64_t sy, const uint16_t* gate, int64_t sg,
                         float* logits, int64_t sl, void* workspace, int64_t workspace_bytes,
                         const float* bias, float* topw, int64_t stw, int32_t* topi, int64_t sti,
                         int T, int H, int E, int topk, float scale, int norm_prob,
                         hipStream_t st, const float* rstd = nullptr);
}  // namespace glm52

// Above this many tokens glm52_router on the gate's rows takes the bounded bf16 path.
constexpr int kSelectMinT = 17;

extern "C" int64_t glm52_router_select_workspace_bytes(int T, int H, int E) {
  return T >= kSelectMinT ? router_select_workspace_bytes(T, H, E) : 0;
}

extern "C" int64_t glm52_router_workspace_bytes(int T, int H, int E) {
  const int ks = choose_ks(T, H);
  return ks == 1 ? 0 : (int64_t)ks * T * E * (int64_t)sizeof(double);
}

namespace {
int launch_logits(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                  int64_t stride_we, int wg_is_f32, float* logits, int64_t stride_l,
                  void* workspace, int64_t workspace_bytes, int T, int H, int E, int* ks_out,
                  hipStream_t stream, const float* rstd = nullptr) {
  if (T < 0 || H <= 0 || E <= 0 || E > EMAX || (E % 16) != 0 || (H % KC) != 0) return GLM52_EINVAL;
  if (!y || !wgt || !logits || stride_l < E || stride_y < H || (stride_y % 8) ||
      (reinterpret_cast<uintptr_t>(y) & 15u))
    return GLM52_EINVAL;
  // the gate is read with 16-byte vectors along its contiguous dim
  if (reinterpret_cast<uintptr_t>(wgt) & 15u) return GLM52_EINVAL;
  const int vec = wg_is_f32 ? 4 : 8;
  if (stride_wk == 1) {  // rows layout [E, H]
    if (stride_we < H || (stride_we % vec) || H > HMAX) return GLM52_EINVAL;
    *ks_out = 1;
    if (T == 0) return GLM52_OK;
    dim3 grid(E, (T + RT - 1) / RT);
    auto* yy = static_cast<const uint16_t*>(y);
    if (wg_is_f32)
      router_rows_kernel<true><<<grid, 256, 0, stream>>>(yy, stride_y, wgt, stride_we, logits, stride_l, T, H, E, rstd);
    else
      router_rows_kernel<false><<<grid, 256, 0, stream>>>(yy, stride_y, wgt, stride_we, logits, stride_l, T, H, E, rstd);
    GLM52_RETURN_LAUNCH();
  }
  if (stride_we != 1 || stride_wk < E || (stride_wk % vec)) return GLM52_EINVAL;
  const int64_t stride_wg = stride_wk;
  const int ks = choose_ks(T, H);
  *ks_out = ks;
  if (T == 0) return GLM52_OK;
  if (ks > 1 && (!workspace || workspace_bytes < glm52_router_workspace_bytes(T, H, E)))
    return GLM52_EINVAL;
  dim3 grid((T + TB - 1) / TB, ks);
  auto* yy = static_cast<const uint16_t*>(y);
  auto* part = static_cast<double*>(workspace);
  if (wg_is_f32)
    router_logits_kernel<true><<<grid, 256, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, part, T, H, E, rstd);
  else
    router_logits_kernel<false><<<grid, 256, 0, stream>>>(yy, stride_y, wgt, stride_wg, logits, stride_l, part, T, H, E, rstd);
  GLM52_RETURN_LAUNCH();
}
}  // namespace

namespace {
int logits_entry(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                 int64_t stride_we, int wg_is_f32, float* logits, int64_t stride_l,
                 void* workspace, int64_t workspace_bytes, int T, int H, int E,
                 const float* rstd, hipStream_t stream) {
  int ks = 1;
  int rc = launch_logits(y, stride_y, wgt, stride_wk, stride_we, wg_is_f32, logits, stride_l,
                         workspace, workspace_bytes, T, H, E, &ks, stream, rstd);
  if (rc != GLM52_OK || T == 0 || ks == 1) return rc;
  const int64_t n = (int64_t)T * E;
  router_reduce_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
      static_cast<const double*>(workspace), logits, stride_l, T, E, ks, rstd);
  GLM52_RETURN_LAUNCH();
}
}  // namespace

extern "C" int glm52_router_logits(const void* y, int64_t stride_y, const void* wgt,
                                   int64_t stride_wk, int64_t stride_we, int wg_is_f32,
                                   float* logits, int64_t stride_l, void* workspace,
                                   int64_t workspace_bytes, int T, int H, int E,
                                   hipStream_t stream) {
  return logits_entry(y, stride_y, wgt, stride_wk, stride_we, wg_is_f32, logits, stride_l,
                      workspace, workspace_bytes, T, H, E, nullptr, stream);
}

// The router GEMM with the half-fused pre-norm epilogue: each logit is rounded to fp32 as
// in glm52_router_logits, then multiplied by rstd[t] (one fp32 product) before its store.
extern "C" int glm52_router_logits_rstd(const void* y, int64_t stride_y, const void* wgt,
                                        int64_t stride_wk, int64_t stride_we, int wg_is_f32,
                                        const float* rstd, float* logits, int64_t stride_l,
                                        void* workspace, int64_t workspace_bytes, int T, int H,
                                        int E, hipStream_t stream) {
  if (T > 0 && !rstd) return GLM52_EINVAL;
  return logits_entry(y, stride_y, wgt, stride_wk, stride_we, wg_is_f32, logits, stride_l,
                      workspace, workspace_bytes, T, H, E, rstd, stream);
}

extern "C" int glm52_router_topk(const float* logits, int64_t stride_l, const float* bias,
                                 float* topw, int64_t stride_w, int32_t* topi,
                                 int64_t stride_i, int T, int E, int topk, float scale,
                                 int norm_prob, hipStream_t stream) {
  if (T < 0 || E <= 0 || E > EMAX || (E % 4) != 0 || topk <= 0 || topk > 8 || topk > E)
    return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  if (!logits || !topw || !topi || stride_l < E || stride_w < topk || stride_i < topk)
    return GLM52_EINVAL;
  router_topk_kernel<<<(T + 3) / 4, 256, 0, stream>>>(const_cast<float*>(logits), stride_l,
                                                      nullptr, 1, bias, topw, stride_w, topi,
                                                      stride_i, T, E, topk, scale, norm_prob);
  GLM52_RETURN_LAUNCH();
}

namespace {
// Logits (times rstd[t] when rstd is given) + top-k.  Gate rows and many tokens: the
// bounded bf16 logits with the exact rule on each token's candidates (two launches); an
// operand that path cannot take (misaligned y, a workspace sized for the exact path only)
// falls through to the exact logits.  Exact path: two launches (the split-K partials are
// reduced inside top-k), three with rstd (the partials reduced with the epilogue first).
int router_entry(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                 int64_t stride_we, int wg_is_f32, float* logits, int64_t stride_l,
                 void* workspace, int64_t workspace_bytes, const float* bias, float* topw,
                 int64_t stride_w, int32_t* topi, int64_t stride_i, int T, int H, int E,
                 int topk, float scale, int norm_prob, const float* rstd, hipStream_t stream) {
  if (topk <= 0 || topk > 8 || topk > E || (E % 4) != 0 || !topw || !topi || stride_w < topk ||
      stride_i < topk)
    return GLM52_EINVAL;
  if (T < 0 || H <= 0 || E <= 0 || E > EMAX || !y || !wgt || !logits || stride_l < E)
    return GLM52_EINVAL;
  if (stride_wk == 1 && !wg_is_f32 && T >= kSelectMinT && stride_y >= H && (stride_y % 8) == 0 &&
      (reinterpret_cast<uintptr_t>(y) & 15u) == 0) {
    // gate rows, many tokens: bf16 MFMA logits, the exact rule on each token's candidates
    const int rc = launch_router_select(static_cast<const uint16_t*>(y), stride_y,
                                        static_cast<const uint16_t*>(wgt), stride_we, logits,
                                        stride_l, workspace, workspace_bytes, bias, topw,
                                        stride_w, topi, stride_i, T, H, E, topk, scale, norm_prob,
                                        stream, rstd);
    if (rc != GLM52_EUNSUPPORTED) return rc;
  }
  if (rstd) {
    const int rc = logits_entry(y, stride_y, wgt, stride_wk, stride_we, wg_is_f32, logits,
                                stride_l, workspace, workspace_bytes, T, H, E, rstd, stream);
    if (rc != GLM52_OK || T == 0) return rc;
    router_topk_kernel<<<(T + 3) / 4, 256, 0, stream>>>(logits, stride_l, nullptr, 1, bias, topw,
                                                        stride_w, topi, stride_i, T, E, topk,
                                                        scale, norm_prob);
    GLM52_RETURN_LAUNCH();
  }
  int ks = 1;
  int rc = launch_logits(y, stride_y, wgt, stride_wk, stride_we, wg_is_f32, logits, stride_l,
                         workspace, workspace_bytes, T, H, E, &ks, stream);
  if (rc != GLM52_OK || T == 0) return rc;
  router_topk_kernel<<<(T + 3) / 4, 256, 0, stream>>>(
      logits, stride_l, ks > 1 ? static_cast<const double*>(workspace) : nullptr, ks, bias,
      topw, stride_w, topi, stride_i, T, E, topk, scale, norm_prob);
  GLM52_RETURN_LAUNCH();
}
}  // namespace

// Logits + top-k (`norm_router.router_gemm` + `topk_only`).
extern "C" int glm52_router(const void* y, int64_t stride_y, const void* wgt, int64_t stride_wk,
                            int64_t stride_we, int wg_is_f32, float* logits, int64_t stride_l,
                            void* workspace, int64_t workspace_bytes, const float* bias,
                            float* topw, int64_t stride_w, int32_t* topi, int64_t stride_i, int T,
                            int H, int E, int topk, float scale, int norm_prob,
                            hipStream_t stream) {
  return router_entry(y, stride_y, wgt, stride_wk, stride_we, wg_is_f32, logits, stride_l,
                      workspace, workspace_bytes, bias, topw, stride_w, topi, stride_i, T, H, E,
                      topk, scale, norm_prob, nullptr, stream);
}

// The same with the half-fused pre-norm epilogue: each logit is its fp32 value times
// rstd[t] (one fp32 product), and the top-k is taken on those logits.
extern "C" int glm52_router_rstd(const void* y, int64_t stride_y, const void* wgt,
                                 int64_t stride_wk, int64_t stride_we, int wg_is_f32,
                                 const float* rstd, float* logits, int64_t stride_l,
                                 void* workspace, int64_t workspace_bytes, const float* bias,
                                 float* topw, int64_t stride_w, int32_t* topi, int64_t stride_i,
                                 int T, int H, int E, int topk, float scale, int norm_prob,
                                 hipStream_t stream) {
  if (T > 0 && !rstd) return GLM52_EINVAL;
  return router_entry(y, stride_y, wgt, stride_wk, stride_we, wg_is_f32, logits, stride_l,
                      workspace, workspace_bytes, bias, topw, stride_w, topi, stride_i, T, H, E,
                      topk, scale, norm_prob, rstd, stream);
}
