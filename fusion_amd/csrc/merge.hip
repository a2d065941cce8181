// HBM-bound vector kernels of the GLM-5.2 MoE block, gfx950.
//
//   silu_and_mul  : y = bf16(silu(fp32 g) * fp32 u) for x = [g | u]
//                   (`glm52/reference.py:36-40`; kernel `glm52/kernels/moe_gateup.py:154-182`)
//   moe_sum       : out = bf16(sum_k fp32 Y[t, k] (+ fp32 res)), k in order
//                   (`glm52/kernels/moe_down_merge.py:300-349`)
//   resadd        : o = bf16(fp32 x + fp32 r)   (`glm52/kernels/moe_down_merge.py:355-381`)
//   merge_resadd  : m = sum_k w[t, k] * fp32 Y[t, k];  out = bf16(bf16?(m) + fp32 res)
//                   (`glm52/kernels/merge_resadd.py:59-196`, ROUND_MID optional); each
//                   product is rounded before its add (no FMA contraction), k in order
//   block_merge   : out = bf16((sum_k fp32 Y[t, k] + fp32 h) + fp32 s)  -- the tail of the
//                   block in one pass: routed merge, the residual h and the shared expert
//                   output s (nullable), one rounding at the end.
//
// Every kernel walks (row, 8-column chunk) pairs with a grid-stride loop and moves each
// byte with one 128-bit access; all top-k loads of a chunk are issued before any add.
#include "moe_gemm.h"

using namespace glm52;

namespace {

constexpr int kBlock = 256;

int grid_for(int64_t work) {
  int64_t g = (work + kBlock - 1) / kBlock;
  const int64_t cap = 256 * 32;  // 32 workgroups per CU on 256 CUs
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return (int)g;
}

__global__ __launch_bounds__(kBlock) void silu_and_mul_kernel(const uint16_t* __restrict__ x,
                                                              int64_t sx, uint16_t* __restrict__ y,
                                                              int64_t sy, int M, int I) {
  const int cpr = I / 8;
  const int64_t total = (int64_t)M * cpr;
  for (int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kBlock) {
    const int64_t m = q / cpr;
    const int c = (int)(q % cpr);
    float gf[8], uf[8], of[8];
    unpack8(*reinterpret_cast<const uint4*>(x + m * sx + c * 8), gf);
    unpack8(*reinterpret_cast<const uint4*>(x + m * sx + I + c * 8), uf);
#pragma unroll
    for (int j = 0; j < 8; ++j) of[j] = silu_mul(gf[j], uf[j]);
    *reinterpret_cast<uint4*>(y + m * sy + c * 8) = pack8(of);
  }
}

template <int TOPK, bool ADD_RES>
__global__ __launch_bounds__(kBlock) void moe_sum_kernel(const uint16_t* __restrict__ yin,
                                                         int64_t s0, int64_t s1,
                                                         uint16_t* __restrict__ out, int64_t so,
                                                         const uint16_t* __restrict__ res,
                                                         int64_t sr, int T, int N, int topk) {
  const int cpr = N / 8;
  const int64_t total = (int64_t)T * cpr;
  for (int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kBlock) {
    const int64_t t = q / cpr;
    const int c = (int)(q % cpr);
    const int kk = TOPK > 0 ? TOPK : topk;
    uint4 v[TOPK > 0 ? TOPK : 8];
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (TOPK > 0) {
#pragma unroll
      for (int k = 0; k < (TOPK > 0 ? TOPK : 1); ++k)
        v[k] = *reinterpret_cast<const uint4*>(yin + t * s0 + k * s1 + c * 8);
#pragma unroll
      for (int k = 0; k < (TOPK > 0 ? TOPK : 1); ++k) {
        float f[8];
        unpack8(v[k], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += f[j];
      }
    } else {
      for (int k = 0; k < kk; ++k) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(yin + t * s0 + k * s1 + c * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += f[j];
      }
    }
    if (ADD_RES) {
      float r[8];
      unpack8(*reinterpret_cast<const uint4*>(res + t * sr + c * 8), r);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += r[j];
    }
    *reinterpret_cast<uint4*>(out + t * so + c * 8) = pack8(acc);
  }
}

__global__ __launch_bounds__(kBlock) void resadd_kernel(const uint16_t* __restrict__ x, int64_t sx,
                                                        const uint16_t* __restrict__ r, int64_t sr,
                                                        uint16_t* __restrict__ o, int64_t so,
                                                        int M, int N) {
  const int cpr = N / 8;
  const int64_t total = (int64_t)M * cpr;
  for (int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kBlock) {
    const int64_t m = q / cpr;
    const int c = (int)(q % cpr);
    float a[8], b[8];
    unpack8(*reinterpret_cast<const uint4*>(x + m * sx + c * 8), a);
    unpack8(*reinterpret_cast<const uint4*>(r + m * sr + c * 8), b);
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = a[j] + b[j];
    *reinterpret_cast<uint4*>(o + m * so + c * 8) = pack8(a);
  }
}

// do_merge / do_resadd / round_mid follow `merge_resadd_kernel`'s flags.
template <bool DO_MERGE, bool DO_RESADD>
__global__ __launch_bounds__(kBlock) void merge_resadd_kernel(
    const uint16_t* __restrict__ y, int64_t syt, int64_t syk, const float* __restrict__ wt,
    int64_t swt, const uint16_t* __restrict__ res, int64_t sr, uint16_t* __restrict__ m,
    int64_t sm, uint16_t* __restrict__ out, int64_t so, int T, int N, int topk, int round_mid) {
#pragma clang fp contract(off)
  const int cpr = N / 8;
  const int64_t total = (int64_t)T * cpr;
  for (int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kBlock) {
    const int64_t t = q / cpr;
    const int c = (int)(q % cpr);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (DO_MERGE) {
      uint4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < topk) v[k] = *reinterpret_cast<const uint4*>(y + t * syt + k * syk + c * 8);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k < topk) {
          const float w = wt[t * swt + k];
          float f[8];
          unpack8(v[k], f);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] = acc[j] + f[j] * w;  // contraction off: no FMA
        }
      }
      if (!DO_RESADD) {
        *reinterpret_cast<uint4*>(m + t * sm + c * 8) = pack8(acc);
        continue;
      }
      if (round_mid) {
        uint4 rb = pack8(acc);
        unpack8(rb, acc);
      }
    } else {
      unpack8(*reinterpret_cast<const uint4*>(m + t * sm + c * 8), acc);
    }
    float r[8];
    unpack8(*reinterpret_cast<const uint4*>(res + t * sr + c * 8), r);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += r[j];
    *reinterpret_cast<uint4*>(out + t * so + c * 8) = pack8(acc);
  }
}

template <bool HAS_SHARED>
__global__ __launch_bounds__(kBlock) void block_merge_kernel(
    const uint16_t* __restrict__ y, int64_t syt, int64_t syk, const uint16_t* __restrict__ h,
    int64_t sh, const uint16_t* __restrict__ s, int64_t ss, uint16_t* __restrict__ out,
    int64_t so, int T, int N) {
  const int cpr = N / 8;
  const int64_t total = (int64_t)T * cpr;
  for (int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kBlock) {
    const int64_t t = q / cpr;
    const int c = (int)(q % cpr);
    uint4 v[8];
#pragma unroll
    // every input is read once and the output is not read again in the block: all
    // non-temporal (T = 8192, 1.1 GB moved: 257 -> 195 us after the benchmark's flush)
    for (int k = 0; k < 8; ++k) v[k] = ldg_nt(y + t * syt + k * syk + c * 8);
    const uint4 hv = ldg_nt(h + t * sh + c * 8);
    uint4 sv = make_uint4(0, 0, 0, 0);
    if (HAS_SHARED) sv = ldg_nt(s + t * ss + c * 8);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float f[8];
      unpack8(v[k], f);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += f[j];
    }
    float f[8];
    unpack8(hv, f);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += f[j];
    if (HAS_SHARED) {
      unpack8(sv, f);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += f[j];
    }
    stg_nt(out + t * so + c * 8, pack8(acc));
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool st8(int64_t s) { return (s % 8) == 0; }

}  // namespace

extern "C" int glm52_silu_and_mul(const void* x, int64_t stride_x, void* y, int64_t stride_y,
                                  int M, int I, hipStream_t stream) {
  if (M < 0 || I <= 0 || (I % 8) || !x || !y || !al16(x) || !al16(y) || !st8(stride_x) || !st8(stride_y))
    return GLM52_EINVAL;
  if (M == 0) return GLM52_OK;
  silu_and_mul_kernel<<<grid_for((int64_t)M * (I / 8)), kBlock, 0, stream>>>(
      static_cast<const uint16_t*>(x), stride_x, static_cast<uint16_t*>(y), stride_y, M, I);
  GLM52_RETURN_LAUNCH();
}

extern "C" int glm52_moe_sum(const void* y, int64_t stride_t, int64_t stride_k, void* out,
                             int64_t stride_o, const void* residual, int64_t stride_r, int T,
                             int N, int topk, int add_residual, hipStream_t stream) {
  if (T < 0 || N <= 0 || (N % 8) || topk <= 0 || !y || !out) return GLM52_EINVAL;
  if (!al16(y) || !al16(out) || !st8(stride_t) || !st8(stride_k) || !st8(stride_o)) return GLM52_EINVAL;
  if (add_residual && (!residual || !al16(residual) || !st8(stride_r))) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  const int g = grid_for((int64_t)T * (N / 8));
  auto* yy = static_cast<const uint16_t*>(y);
  auto* oo = static_cast<uint16_t*>(out);
  auto* rr = static_cast<const uint16_t*>(residual);
  if (topk == 8) {
    if (add_residual)
      moe_sum_kernel<8, true><<<g, kBlock, 0, stream>>>(yy, stride_t, stride_k, oo, stride_o, rr, stride_r, T, N, topk);
    else
      moe_sum_kernel<8, false><<<g, kBlock, 0, stream>>>(yy, stride_t, stride_k, oo, stride_o, rr, stride_r, T, N, topk);
  } else {
    if (add_residual)
      moe_sum_kernel<0, true><<<g, kBlock, 0, stream>>>(yy, stride_t, stride_k, oo, stride_o, rr, stride_r, T, N, topk);
    else
      moe_sum_kernel<0, false><<<g, kBlock, 0, stream>>>(yy, stride_t, stride_k, oo, stride_o, rr, stride_r, T, N, topk);
  }
  GLM52_RETURN_LAUNCH();
}

extern "C" int glm52_resadd(const void* x, int64_t stride_x, const void* r, int64_t stride_r,
                            void* o, int64_t stride_o, int M, int N, hipStream_t stream) {
  if (M < 0 || N <= 0 || (N % 8) || !x || !r || !o) return GLM52_EINVAL;
  if (!al16(x) || !al16(r) || !al16(o) || !st8(stride_x) || !st8(stride_r) || !st8(stride_o))
    return GLM52_EINVAL;
  if (M == 0) return GLM52_OK;
  resadd_kernel<<<grid_for((int64_t)M * (N / 8)), kBlock, 0, stream>>>(
      static_cast<const uint16_t*>(x), stride_x, static_cast<const uint16_t*>(r), stride_r,
      static_cast<uint16_t*>(o), stride_o, M, N);
  GLM52_RETURN_LAUNCH();
}

extern "C" int glm52_merge_resadd(const void* y, int64_t stride_yt, int64_t stride_yk,
                                  const float* wt, int64_t stride_wt, const void* res,
                                  int64_t stride_r, void* m, int64_t stride_m, void* out,
                                  int64_t stride_o, int T, int N, int topk, int do_merge,
                                  int do_resadd, int round_mid, hipStream_t stream) {
  if (T < 0 || N <= 0 || (N % 8) || topk <= 0 || topk > 8) return GLM52_EINVAL;
  if (!do_merge && !do_resadd) return GLM52_EINVAL;
  if (do_merge && (!y || !wt || !al16(y) || !st8(stride_yt) || !st8(stride_yk))) return GLM52_EINVAL;
  if (do_resadd && (!res || !out || !al16(res) || !al16(out) || !st8(stride_r) || !st8(stride_o)))
    return GLM52_EINVAL;
  if ((!do_merge || !do_resadd) && (!m || !al16(m) || !st8(stride_m))) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  const int g = grid_for((int64_t)T * (N / 8));
  auto* yy = static_cast<const uint16_t*>(y);
  auto* rr = static_cast<const uint16_t*>(res);
  auto* mm = static_cast<uint16_t*>(m);
  auto* oo = static_cast<uint16_t*>(out);
  if (do_merge && do_resadd)
    merge_resadd_kernel<true, true><<<g, kBlock, 0, stream>>>(yy, stride_yt, stride_yk, wt, stride_wt, rr, stride_r, mm, stride_m, oo, stride_o, T, N, topk, round_mid);
  else if (do_merge)
    merge_resadd_kernel<true, false><<<g, kBlock, 0, stream>>>(yy, stride_yt, stride_yk, wt, stride_wt, rr, stride_r, mm, stride_m, oo, stride_o, T, N, topk, round_mid);
  else
    merge_resadd_kernel<false, true><<<g, kBlock, 0, stream>>>(yy, stride_yt, stride_yk, wt, stride_wt, rr, stride_r, mm, stride_m, oo, stride_o, T, N, topk, round_mid);
  GLM52_RETURN_LAUNCH();
}

extern "C" int glm52_block_merge(const void* y, int64_t stride_yt, int64_t stride_yk,
                                 const void* h, int64_t stride_h, const void* shared_out,
                                 int64_t stride_s, void* out, int64_t stride_o, int T, int N,
                                 hipStream_t stream) {
  if (T < 0 || N <= 0 || (N % 8) || !y || !h || !out) return GLM52_EINVAL;
  if (!al16(y) || !al16(h) || !al16(out) || !st8(stride_yt) || !st8(stride_yk) || !st8(stride_h) ||
      !st8(stride_o))
    return GLM52_EINVAL;
  if (shared_out && (!al16(shared_out) || !st8(stride_s))) return GLM52_EINVAL;
  if (T == 0) return GLM52_OK;
  const int g = grid_for((int64_t)T * (N / 8));
  auto* yy = static_cast<const uint16_t*>(y);
  auto* hh = static_cast<const uint16_t*>(h);
  auto* ss = static_cast<const uint16_t*>(shared_out);
  auto* oo = static_cast<uint16_t*>(out);
  if (shared_out)
    block_merge_kernel<true><<<g, kBlock, 0, stream>>>(yy, stride_yt, stride_yk, hh, stride_h, ss, stride_s, oo, stride_o, T, N);
  else
    block_merge_kernel<false><<<g, kBlock, 0, stream>>>(yy, stride_yt, stride_yk, hh, stride_h, ss, stride_s, oo, stride_o, T, N);
  GLM52_RETURN_LAUNCH();
}

// ------------------------------------------------------------------------------------
// Read-bandwidth probe: grid-stride 16-byte loads over `bytes` of device memory, U = 4
// loads in flight per lane, normal or non-temporal.  It measures the HBM ceiling the
// weight-streaming kernels are held to; `sink` is written only if the xor of all words
// equals a magic value (never, for a real buffer), which keeps the loads alive.
// ------------------------------------------------------------------------------------
namespace {

template <bool NT>
__global__ __launch_bounds__(kBlock) void stream_read_kernel(const uint4* __restrict__ p,
                                                             int64_t n16,
                                                             uint32_t* __restrict__ sink) {
  constexpr int U = 4;
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (NT) {
        const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p + i + u * stride));
        v[u] = make_uint4(t[0], t[1], t[2], t[3]);
      } else {
        v[u] = p[i + u * stride];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}
}  // namespace

extern "C" int glm52_stream_read(const void* buf, int64_t bytes, int nontemporal, int grid,
                                 uint32_t* sink, hipStream_t stream) {
  if (!buf || !sink || bytes < 0 || (bytes % 16) || !al16(buf) || grid <= 0 || grid > 65536)
    return GLM52_EINVAL;
  if (bytes == 0) return GLM52_OK;
  auto* p = static_cast<const uint4*>(buf);
  if (nontemporal)
    stream_read_kernel<true><<<grid, kBlock, 0, stream>>>(p, bytes / 16, sink);
  else
    stream_read_kernel<false><<<grid, kBlock, 0, stream>>>(p, bytes / 16, sink);
  GLM52_RETURN_LAUNCH();
}
