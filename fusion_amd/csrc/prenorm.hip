// Half-fused pre-norm (`glm52/kernels/lazy_prenorm.py`, fusion #11b'): the RMSNorm of the
// block's input is not materialised for a consumer GEMM.  Its weight w is folded into the
// consumer's weight once, and the per-row scale rstd is applied to the consumer's
// accumulator in the epilogue:
//
//   ((h * rstd) * w) @ B  ==  (h @ (w[:, None] * B)) * rstd
//
// This file holds the two pieces the consumers need:
//   rstd       rstd[t] = fp32(1 / sqrt(sum_k h[t, k]^2 / N + eps)) -- `rstd_kernel`
//              (`lazy_prenorm.py:346-368`); the squares (exact in fp32 for bf16 h) are
//              summed in fp64 and rounded once, the statistic of this build's RMSNorm
//              (add_rmsnorm.hip), so rstd here equals the one inside that kernel.  It
//              can also write rstd repeated `repeat` times per row, the per-slot scale
//              of a grouped GEMM whose slot f gathers row f / repeat.
//   scale_rows c[t, :] *= rstd[t] on fp32 rows -- the USE_RSTD epilogue of the router
//              GEMM (`lazy_prenorm.py:323-325`), applied after the logits are rounded.
#include "common.h"

using namespace glm52;

namespace {

__global__ __launch_bounds__(256) void rstd_kernel(const uint16_t* __restrict__ x, int64_t sx,
                                                   int T, int N, float eps,
                                                   float* __restrict__ rstd,
                                                   float* __restrict__ flat, int repeat) {
  const int lane = threadIdx.x % kWave;
  const int t = blockIdx.x * 4 + threadIdx.x / kWave;  // one wave per row
  if (t >= T) return;
  const uint16_t* row = x + (int64_t)t * sx;
  double ss = 0.0;
  for (int c = lane; c < N / 8; c += kWave) {
    float v[8];
    unpack8(*reinterpret_cast<const uint4*>(row + c * 8), v);
#pragma unroll
    for (int q = 0; q < 8; ++q) ss += (double)(v[q] * v[q]);
  }
  ss = wave_sum_f64(ss);
  const float r = (float)(1.0 / sqrt(ss / (double)N + (double)eps));
  if (lane == 0 && rstd) rstd[t] = r;
  if (flat)
    for (int j = lane; j < repeat; j += kWave) flat[(int64_t)t * repeat + j] = r;
}

__global__ __launch_bounds__(256) void scale_rows_kernel(float* __restrict__ c, int64_t sc, int T,
                                                         int N, const float* __restrict__ rstd) {
  const int64_t total = (int64_t)T * N;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * 256) {
    const int64_t t = q / N;
    c[t * sc + q % N] *= rstd[t];
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

extern "C" int glm52_scale_rows(float* c, int64_t stride_c, int T, int N, const float* rstd,
                                hipStream_t stream) {
  if (T < 0 || N <= 0) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  if (!c || !rstd || stride_c < N) return GLM52_EINVAL;
  const int64_t total = (int64_t)T * N;
  const int grid = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  scale_rows_kernel<<<grid, 256, 0, stream>>>(c, stride_c, T, N, rstd);
  GLM52_RETURN_LAUNCH();
}
