// Decode front end of the GLM-5.2 MoE block in one launch, gfx950: ResAdd + RMSNorm,
// router logits, sigmoid + noaux_tc top-k, and the dispatch layout, for T <= 4 tokens.
//
// It computes exactly what the separate kernels compute (add_rmsnorm.hip, router.hip's
// row mapping, select.h), so its outputs are bit-identical to that chain:
//   h = bf16(x + r); y = bf16(fp32(bf16(h * rstd)) * w), rstd from the fp64 sum of the
//   exact squares (`glm52/reference.py:22-33`);
//   logits[t, e] = fp32(sum_k y[t, k] * gate[e, k]) with exact products summed in fp64
//   (`glm52/reference.py:61`);
//   ids / weights and the layout as `glm52/reference.py:62-128`.
//
// Mapping: E / 4 workgroups of four waves.  Each wave owns one gate row ([E, H] layout)
// and issues all of its 16-byte loads first, with the norm weight's, so that they land
// while the workgroup recomputes the T normalised rows into LDS (x, r and the norm weight
// come from L2 after the first workgroup; workgroup 0 also writes h and y); then the
// wave dots its row with the staged rows.  The workgroups publish their logits, then count themselves
// on a device-scope counter; the last one to arrive runs the top-k of every token and
// builds the layout, then resets the counter to zero for the next launch.  The counter
// is the only state and must be zero before the first launch.
//
// glm52_decode_norm_logits computes the first two steps only (the routed decode GEMM
// derives the routing from the logits itself) with its own mapping, norm_logits_kernel:
// one workgroup per gate row.
#include "select.h"

using namespace glm52;

namespace {

constexpr int kTmax = 4;
constexpr int kHmax = 8192;
constexpr int kChunks = kHmax / 8 / 256;  // 16-byte chunks per thread of one row

__global__ __launch_bounds__(256) void decode_front_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ wn, uint16_t* __restrict__ h_out, uint16_t* __restrict__ y_out,
    int64_t sx, int64_t sr, int64_t sh_, int64_t sy, const uint16_t* __restrict__ gate,
    int64_t sg, const float* __restrict__ bias, float* logits, int64_t sl,
    float* __restrict__ topw, int64_t stw, int32_t* __restrict__ topi, int64_t sti, int T, int H,
    int E, int topk, float eps, float scale, int norm_prob, int BM, int capacity,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ ntp_out, int32_t* counter) {
  __shared__ __attribute__((aligned(16))) uint16_t ys[kTmax][kHmax];
  __shared__ double part[4];
  __shared__ int is_last;
  __shared__ TopkAlignLds tsh;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int nchunk = H / 8;
  const int e = blockIdx.x * 4 + wv;  // the gate row this wave owns

  // ---- 0. loads, in the order they are needed (loads complete in order) --------------
  // token 0's x and r chunks, then the norm weight, the bias, and the wave's gate row
  uint4 xr0[kChunks][2];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c = tid + j * 256;
    xr0[j][0] = c < nchunk ? *reinterpret_cast<const uint4*>(x + c * 8) : make_uint4(0, 0, 0, 0);
    xr0[j][1] = c < nchunk ? *reinterpret_cast<const uint4*>(res + c * 8) : make_uint4(0, 0, 0, 0);
  }
  // the norm weight chunks this thread applies
  uint4 wraw[kChunks];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c = tid + j * 256;
    wraw[j] = c < nchunk ? *reinterpret_cast<const uint4*>(wn + c * 8) : make_uint4(0, 0, 0, 0);
  }
  float bv[4];  // the correction bias, for the top-k (read here, off the critical path)
  load_bias(bias, E, bv);
  // the wave's gate row, 16 bytes per lane per step (H <= 8192: at most 16 steps)
  constexpr int kG = kHmax / 8 / kWave;
  uint4 graw[kG];
  const uint16_t* grow = gate + (int64_t)(e < E ? e : 0) * sg;
#pragma unroll
  for (int i = 0; i < kG; ++i) {
    const int c = lane + i * kWave;
    graw[i] = c < nchunk ? *reinterpret_cast<const uint4*>(grow + c * 8) : make_uint4(0, 0, 0, 0);
  }

  // ---- 1. the T normalised rows into LDS ----------------------------------------------
  for (int t = 0; t < T; ++t) {
    float hv[kChunks][8];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int c = tid + j * 256;
      if (c < nchunk) {
        float xf[8], rf[8];
        if (t == 0) {
          unpack8(xr0[j][0], xf);
          unpack8(xr0[j][1], rf);
        } else {
          unpack8(*reinterpret_cast<const uint4*>(x + t * sx + c * 8), xf);
          unpack8(*reinterpret_cast<const uint4*>(res + t * sr + c * 8), rf);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) xf[q] = xf[q] + rf[q];
        const uint4 hb = pack8(xf);
        if (blockIdx.x == 0) *reinterpret_cast<uint4*>(h_out + t * sh_ + c * 8) = hb;
        unpack8(hb, hv[j]);
#pragma unroll
        for (int q = 0; q < 8; ++q) ss += (double)(hv[j][q] * hv[j][q]);
      }
    }
    ss = wave_sum_f64(ss);
    if (lane == 0) part[wv] = ss;
    __syncthreads();
    ss = ((part[0] + part[1]) + part[2]) + part[3];  // add_rmsnorm's order: same bits
    const float rstd = (float)(1.0 / sqrt(ss / (double)H + (double)eps));
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int c = tid + j * 256;
      if (c < nchunk) {
        float wf[8], yf[8];
        unpack8(wraw[j], wf);
#pragma unroll
        for (int q = 0; q < 8; ++q) yf[q] = bf16_to_f32(f32_to_bf16(hv[j][q] * rstd)) * wf[q];
        const uint4 yb = pack8(yf);
        *reinterpret_cast<uint4*>(&ys[t][c * 8]) = yb;
        if (blockIdx.x == 0) *reinterpret_cast<uint4*>(y_out + t * sy + c * 8) = yb;
      }
    }
    __syncthreads();  // part[] is reused by the next token; ys is complete
  }

  // ---- 2. the wave's gate row against the staged rows ----------------------------------
  if (e < E) {
    double acc[kTmax];
#pragma unroll
    for (int t = 0; t < kTmax; ++t) acc[t] = 0.0;
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      const int c = lane + i * kWave;
      if (c < nchunk) {
        float gf[8];
        unpack8(graw[i], gf);
#pragma unroll
        for (int t = 0; t < kTmax; ++t) {
          if (t < T) {
            float yf[8];
            unpack8(*reinterpret_cast<const uint4*>(&ys[t][c * 8]), yf);
#pragma unroll
            for (int q = 0; q < 8; ++q) acc[t] = fma((double)yf[q], (double)gf[q], acc[t]);
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kTmax; ++t) {
      if (t < T) {  // each reduction is 12 cross-lane moves: only the tokens that exist
        const double s = wave_sum_f64(acc[t]);
        if (lane == 0) logits[(int64_t)t * sl + e] = (float)s;
      }
    }
  }

  // ---- 3. the last workgroup to arrive selects and builds the layout -----------------
  __threadfence();  // publish this workgroup's logits (and h, y) device-wide
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(counter, 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();  // acquire the other workgroups' logits
  topk_align_block(logits, sl, bv, bias != nullptr, topw, stw, topi, sti, T, E, topk, scale,
                   norm_prob, BM, capacity, sorted_ids, expert_ids, ntp_out, tsh);
  if (tid == 0) atomicExch(counter, 0);
}

// Norm and router logits only (glm52_decode_norm_logits): one workgroup per gate row, so
// all CUs stream the gate.  Thread (wave w, lane l) owns the 16-byte chunks
// c = w * H / 32 + l + 64 j of every token row: it adds x and r there, squares h for the
// row's statistic, forms y there once rstd is known, and dots y with the same chunks of
// the workgroup's gate row -- y never goes through LDS.  The statistic and the logit each
// meet as four wave partials added in wave order.
constexpr int kNJ = kHmax / 32 / kWave;  // chunks per thread (H <= 8192)

__global__ __launch_bounds__(256) void norm_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ wn, uint16_t* __restrict__ h_out, uint16_t* __restrict__ y_out,
    int64_t sx, int64_t sr, int64_t sh_, int64_t sy, const uint16_t* __restrict__ gate,
    int64_t sg, float* __restrict__ logits, int64_t sl, int T, int H, float eps) {
  __shared__ double part[kTmax][4];
  __shared__ double lpart[kTmax][4];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int e = blockIdx.x;
  const int qc = H / 32;  // chunks of one wave's quarter of a row

  // loads, in the order they are needed: x and r of every token, the norm weight, the gate
  uint4 xr[kTmax][kNJ][2];
  uint4 wraw[kNJ], graw[kNJ];
#pragma unroll
  for (int t = 0; t < kTmax; ++t)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      const int c = wv * qc + lane + 64 * j;
      const bool ok = t < T && lane + 64 * j < qc;
      xr[t][j][0] = ok ? *reinterpret_cast<const uint4*>(x + t * sx + c * 8) : make_uint4(0, 0, 0, 0);
      xr[t][j][1] = ok ? *reinterpret_cast<const uint4*>(res + t * sr + c * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const int c = wv * qc + lane + 64 * j;
    const bool ok = lane + 64 * j < qc;
    wraw[j] = ok ? *reinterpret_cast<const uint4*>(wn + c * 8) : make_uint4(0, 0, 0, 0);
    graw[j] = ok ? *reinterpret_cast<const uint4*>(gate + (int64_t)e * sg + c * 8) : make_uint4(0, 0, 0, 0);
  }

  // h = bf16(x + r) and the sum of its exact squares in fp64, per token
  uint4 hb[kTmax][kNJ];
#pragma unroll
  for (int t = 0; t < kTmax; ++t) {
    if (t < T) {
      double ss = 0.0;
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        float xf[8], rf[8], hv[8];
        unpack8(xr[t][j][0], xf);
        unpack8(xr[t][j][1], rf);
#pragma unroll
        for (int q = 0; q < 8; ++q) xf[q] = xf[q] + rf[q];
        hb[t][j] = pack8(xf);
        unpack8(hb[t][j], hv);
        if (lane + 64 * j < qc) {
#pragma unroll
          for (int q = 0; q < 8; ++q) ss += (double)(hv[q] * hv[q]);
          if (e == 0) *reinterpret_cast<uint4*>(h_out + t * sh_ + (wv * qc + lane + 64 * j) * 8) = hb[t][j];
        }
      }
      ss = wave_sum_f64(ss);
      if (lane == 0) part[t][wv] = ss;
    }
  }
  __syncthreads();

  // y = bf16(fp32(bf16(h * rstd)) * w) on the thread's chunks, dotted with the gate row
  double acc[kTmax];
#pragma unroll
  for (int t = 0; t < kTmax; ++t) {
    acc[t] = 0.0;
    if (t < T) {
      const double ssum = ((part[t][0] + part[t][1]) + part[t][2]) + part[t][3];
      const float rstd = (float)(1.0 / sqrt(ssum / (double)H + (double)eps));
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        if (lane + 64 * j < qc) {
          float hv[8], wf[8], gf[8], yf[8];
          unpack8(hb[t][j], hv);
          unpack8(wraw[j], wf);
#pragma unroll
          for (int q = 0; q < 8; ++q) yf[q] = bf16_to_f32(f32_to_bf16(hv[q] * rstd)) * wf[q];
          const uint4 yb = pack8(yf);
          if (e == 0) *reinterpret_cast<uint4*>(y_out + t * sy + (wv * qc + lane + 64 * j) * 8) = yb;
          unpack8(yb, yf);
          unpack8(graw[j], gf);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[t] = fma((double)yf[q], (double)gf[q], acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kTmax; ++t) {
    if (t < T) {
      const double s = wave_sum_f64(acc[t]);
      if (lane == 0) lpart[t][wv] = s;
    }
  }
  __syncthreads();
  if (tid < T)
    logits[(int64_t)tid * sl + e] =
        (float)(((lpart[tid][0] + lpart[tid][1]) + lpart[tid][2]) + lpart[tid][3]);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int glm52_decode_front(const void* x, int64_t stride_x, const void* res,
                                  int64_t stride_r, const void* w_norm, void* h1,
                                  int64_t stride_h, void* y, int64_t stride_y, const void* gate,
                                  int64_t stride_g, const float* bias, float* logits,
                                  int64_t stride_l, float* topw, int64_t stride_w, int32_t* topi,
                                  int64_t stride_i, int T, int H, int E, int topk, float eps,
                                  float scale, int norm_prob, int block_m, int capacity,
                                  int32_t* sorted_token_ids, int32_t* expert_ids,
                                  int32_t* num_tokens_post_padded, int32_t* counter,
                                  hipStream_t stream) {
  if (T < 1 || T > kTmax || H <= 0 || H > kHmax || (H % 8) || E <= 0 || E > kMaxE || (E % 4) ||
      topk <= 0 || topk > 8 || topk > E)
    return GLM52_EINVAL;
  if (!x || !res || !w_norm || !h1 || !y || !gate || !logits || !topw || !topi || !counter)
    return GLM52_EINVAL;
  if (!al16(x) || !al16(res) || !al16(w_norm) || !al16(h1) || !al16(y) || !al16(gate) ||
      (stride_x % 8) || (stride_r % 8) || (stride_h % 8) || (stride_y % 8) || (stride_g % 8) ||
      stride_g < H || stride_l < E || stride_w < topk || stride_i < topk)
    return GLM52_EINVAL;
  if (block_m <= 0 || !sorted_token_ids || !expert_ids || !num_tokens_post_padded)
    return GLM52_EINVAL;
  const int64_t need = (int64_t)T * topk + (int64_t)E * (block_m - 1);
  if (capacity < need || (capacity % block_m)) return GLM52_EINVAL;
  decode_front_kernel<<<(E + 3) / 4, 256, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(res),
      static_cast<const uint16_t*>(w_norm), static_cast<uint16_t*>(h1), static_cast<uint16_t*>(y),
      stride_x, stride_r, stride_h, stride_y, static_cast<const uint16_t*>(gate), stride_g, bias,
      logits, stride_l, topw, stride_w, topi, stride_i, T, H, E, topk, eps, scale, norm_prob,
      block_m, capacity, sorted_token_ids, expert_ids, num_tokens_post_padded, counter);
  GLM52_RETURN_LAUNCH();
}

// The first part of glm52_decode_front alone: ResAdd + RMSNorm and the router logits of
// T <= 4 tokens in one launch, no top-k (glm52_moe_gemm_route_shared derives the routing).
extern "C" int glm52_decode_norm_logits(const void* x, int64_t stride_x, const void* res,
                                        int64_t stride_r, const void* w_norm, void* h1,
                                        int64_t stride_h, void* y, int64_t stride_y,
                                        const void* gate, int64_t stride_g, float* logits,
                                        int64_t stride_l, int T, int H, int E, float eps,
                                        hipStream_t stream) {
  if (T < 1 || T > kTmax || H <= 0 || H > kHmax || (H % 32) || E <= 0 || E > kMaxE)
    return GLM52_EINVAL;
  if (!x || !res || !w_norm || !h1 || !y || !gate || !logits) return GLM52_EINVAL;
  if (!al16(x) || !al16(res) || !al16(w_norm) || !al16(h1) || !al16(y) || !al16(gate) ||
      (stride_x % 8) || (stride_r % 8) || (stride_h % 8) || (stride_y % 8) || (stride_g % 8) ||
      stride_g < H || stride_l < E)
    return GLM52_EINVAL;
  norm_logits_kernel<<<E, 256, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(res),
      static_cast<const uint16_t*>(w_norm), static_cast<uint16_t*>(h1), static_cast<uint16_t*>(y),
      stride_x, stride_r, stride_h, stride_y, static_cast<const uint16_t*>(gate), stride_g,
      logits, stride_l, T, H, eps);
  GLM52_RETURN_LAUNCH();
}
