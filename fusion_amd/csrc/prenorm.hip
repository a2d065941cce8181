// Half-fused pre-norm (`glm52/kernels/lazy_prenorm.py`, fusion #11b'): the RMSNorm of the
// block's input is not materialised for a consumer GEMM.  Its weight w is folded into the
// consumer's weight once, and the per-row scale rstd is applied to the consumer's
// accumulator in the epilogue:
//
//   ((h * rstd) * w) @ B  ==  (h @ (w[:, None] * B)) * rstd
//
// This file holds the statistic the consumers need, and the router's decode mapping:
//   rstd       rstd[t] = fp32(1 / sqrt(sum_k h[t, k]^2 / N + eps)) -- `rstd_kernel`
//              (`lazy_prenorm.py:346-368`); the squares (exact in fp32 for bf16 h) are
//              summed in fp64 and rounded once, the statistic of this build's RMSNorm
//              (add_rmsnorm.hip), so rstd here equals the one inside that kernel.  It
//              can also write rstd repeated `repeat` times per row, the per-slot scale
//              of a grouped GEMM whose slot f gathers row f / repeat.
//   prenorm_router_rows  the router of T <= 4 tokens in one launch, the statistic
//              (unless given) and the dot computed in the same pass over h.
// Elsewhere the consumers apply rstd in their epilogues: the router GEMM (router.hip,
// glm52_router_logits_rstd) and the grouped GEMM, which takes the repeated rstd as its
// per-slot scale.
#include "common.h"

using namespace glm52;

namespace {

constexpr int kRJ = 16;  // 16-byte chunks a lane has in flight at once (a full 8192 row)

// One wave per row; each lane issues all its loads of a row before the first add.
__global__ __launch_bounds__(256) void rstd_kernel(const uint16_t* __restrict__ x, int64_t sx,
                                                   int T, int N, float eps,
                                                   float* __restrict__ rstd,
                                                   float* __restrict__ flat, int repeat) {
  const int lane = threadIdx.x % kWave;
  const int t = blockIdx.x * 4 + threadIdx.x / kWave;
  if (t >= T) return;
  const uint16_t* row = x + (int64_t)t * sx;
  const int nch = N / 8;
  double ss = 0.0;
  for (int base = 0; base < nch; base += kRJ * kWave) {
    uint4 v[kRJ];
#pragma unroll
    for (int j = 0; j < kRJ; ++j) {
      const int c = base + lane + j * kWave;
      v[j] = c < nch ? *reinterpret_cast<const uint4*>(row + c * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kRJ; ++j) {
      float f[8];
      unpack8(v[j], f);  // zero chunks past the row add nothing
#pragma unroll
      for (int q = 0; q < 8; ++q) ss += (double)(f[q] * f[q]);
    }
  }
  ss = wave_sum_f64(ss);
  const float r = (float)(1.0 / sqrt(ss / (double)N + (double)eps));
  if (lane == 0 && rstd) rstd[t] = r;
  if (flat)
    for (int j = lane; j < repeat; j += kWave) flat[(int64_t)t * repeat + j] = r;
}

// The pre-norm router at decode sizes (T <= 4), one workgroup per gate row e: thread
// (w, l) owns the same 16-byte chunks of every token row and of the gate row, so one
// pass over registers gives both the dot h[t] . gate_fold[e] and, unless rstd is given,
// the sum of squares of h[t] -- the fully fused form, one launch.  Wave partials (fp64)
// meet in wave order; logits[t, e] = fp32(dot) * rstd[t].
constexpr int kPTmax = 4;
constexpr int kPHmax = 8192;
constexpr int kPNJ = kPHmax / 32 / kWave;  // chunks per lane of a wave's quarter row

__global__ __launch_bounds__(256) void prenorm_router_rows_kernel(
    const uint16_t* __restrict__ h, int64_t sh, const uint16_t* __restrict__ gate, int64_t sg,
    const float* __restrict__ rstd_in, float eps, float* __restrict__ logits, int64_t sl,
    float* __restrict__ rstd_out, int T, int H) {
  __shared__ double spart[kPTmax][4];
  __shared__ double dpart[kPTmax][4];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int e = blockIdx.x;
  const int qc = H / 32;
  uint4 hr[kPTmax][kPNJ], gr[kPNJ];
#pragma unroll
  for (int t = 0; t < kPTmax; ++t)
#pragma unroll
    for (int j = 0; j < kPNJ; ++j) {
      const int c = wv * qc + lane + kWave * j;
      const bool ok = t < T && lane + kWave * j < qc;
      hr[t][j] = ok ? *reinterpret_cast<const uint4*>(h + t * sh + c * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
  for (int j = 0; j < kPNJ; ++j) {
    const int c = wv * qc + lane + kWave * j;
    gr[j] = lane + kWave * j < qc ? *reinterpret_cast<const uint4*>(gate + (int64_t)e * sg + c * 8)
                                  : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int t = 0; t < kPTmax; ++t) {
    if (t < T) {
      double ss = 0.0, dot = 0.0;
#pragma unroll
      for (int j = 0; j < kPNJ; ++j) {
        float hv[8], gv[8];
        unpack8(hr[t][j], hv);
        unpack8(gr[j], gv);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          ss += (double)(hv[q] * hv[q]);
          dot = fma((double)hv[q], (double)gv[q], dot);
        }
      }
      dot = wave_sum_f64(dot);
      if (!rstd_in) ss = wave_sum_f64(ss);
      if (lane == 0) {
        spart[t][wv] = ss;
        dpart[t][wv] = dot;
      }
    }
  }
  __syncthreads();
  if (tid < T) {
    const int t = tid;
    const double d = ((dpart[t][0] + dpart[t][1]) + dpart[t][2]) + dpart[t][3];
    float r;
    if (rstd_in) {
      r = rstd_in[t];
    } else {
      const double ss = ((spart[t][0] + spart[t][1]) + spart[t][2]) + spart[t][3];
      r = (float)(1.0 / sqrt(ss / (double)H + (double)eps));
    }
    logits[(int64_t)t * sl + e] = (float)d * r;
    if (rstd_out && e == 0) rstd_out[t] = r;
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// rstd of T rows of x [T, N] bf16; rstd and/or flat (rstd repeated `repeat` times per row)
// may be null.
extern "C" int glm52_rstd(const void* x, int64_t stride_x, int T, int N, float eps, float* rstd,
                          float* rstd_flat, int repeat, hipStream_t stream) {
  if (T < 0 || N <= 0 || (N % 8) || (rstd_flat && repeat < 1)) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  if (!x || !al16(x) || (stride_x % 8) || stride_x < N) return GLM52_EINVAL;
  rstd_kernel<<<(T + 3) / 4, 256, 0, stream>>>(static_cast<const uint16_t*>(x), stride_x, T, N,
                                               eps, rstd, rstd_flat, repeat);
  GLM52_RETURN_LAUNCH();
}

// The pre-norm router for T <= 4 tokens on a gate read as rows ([E, H], row stride sg):
// logits[t, e] = fp32(h[t] . gate[e]) * rstd[t], with rstd from `rstd_in` when given and
// computed in the same pass otherwise (then also written to `rstd_out` if non-null).
extern "C" int glm52_prenorm_router_rows(const void* h, int64_t stride_h, const void* gate,
                                         int64_t stride_g, const float* rstd_in, float eps,
                                         float* logits, int64_t stride_l, float* rstd_out,
                                         int T, int H, int E, hipStream_t stream) {
  if (T < 0 || T > kPTmax || H <= 0 || (H % 32) || H > kPHmax || E <= 0) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  if (!h || !gate || !logits || !al16(h) || !al16(gate) || (stride_h % 8) || stride_h < H ||
      (stride_g % 8) || stride_g < H || stride_l < E)
    return GLM52_EINVAL;
  prenorm_router_rows_kernel<<<E, 256, 0, stream>>>(
      static_cast<const uint16_t*>(h), stride_h, static_cast<const uint16_t*>(gate), stride_g,
      rstd_in, eps, logits, stride_l, rstd_out, T, H);
  GLM52_RETURN_LAUNCH();
}
