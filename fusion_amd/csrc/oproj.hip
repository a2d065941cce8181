// o_proj + ResAdd1 of the GLM-5.2 decoder layer on gfx950: the dense GEMM feeding the MoE
// block, h1 = A @ B + r, with the epilogue variants of `glm52/kernels/oproj_resadd.py`:
//
//   epilogue 0 : c = bf16(A @ B)                     (oproj_gemm_kernel, FUSE_RESADD off)
//   epilogue 1 : c = bf16(fp32(A @ B) + fp32 r)      (FUSE_RESADD on: beta = 1)
//   epilogue 2 : c32 += fp32(A @ B) (+ fp32 r)        (ATOMIC_OUT: split-K into fp32)
//   cast_add   : o = bf16(fp32 c + fp32 r) or bf16(c) (epilogue_kernel)
//
// A is [M, K] bf16 (K contiguous), B is [K, N] bf16 -- the reference feeds its kernels the
// nn.Linear weight transposed and made contiguous, N contiguous.  K is 32768 at decode
// (absorbed MLA) and 16384 at prefill.
//
// Decode (M <= 16, N contiguous): a weight stream.  Split K: workgroup (g, s) multiplies
// k rows [s KC, (s + 1) KC) of B by the matching columns of A, for a slice of the N
// columns, each thread owning 16-byte column chunks of every k row; so every workgroup
// reads whole contiguous rows of B, with non-temporal loads (B is read once: a stream the
// size of one o_proj right after other work reads about 3 TB/s with normal loads and over
// 5 TB/s non-temporal on MI355X).  A's slice is staged in LDS as fp32.  Partial sums go
// to an fp32 workspace [S][M][N]; the reduction gives one wave to each 8-column chunk of
// a row: lane l adds splits l, l + 64, ... in order, then the 64 lane sums meet in a fixed
// butterfly.  No atomics: the result does not depend on timing.
//
// Prefill: the 512-row tile GEMM of the MoE block (moe_gemm_wide.hip) as a one-expert
// grouped GEMM over an identity row layout, on a packed copy of B (made once per weight,
// glm52_oproj_pack), with epilogue 1 or 2 fused.
#include "moe_gemm.h"

using namespace glm52;

namespace {

constexpr int kCols = 8;       // columns per 16-byte chunk
constexpr int kMaxKC = 512;    // k rows per split (LDS: M x KC fp32)

template <int TM, int CPT, int U>
__global__ __launch_bounds__(256) void oproj_splitk_kernel(
    const uint16_t* __restrict__ a, int64_t sam, const uint16_t* __restrict__ b, int64_t sbk,
    int M, int N, int K, int KC, float* __restrict__ ws) {
  __shared__ float as[TM][kMaxKC];
  const int tid = threadIdx.x;
  const int g = blockIdx.x, s = blockIdx.y;
  const int k0 = s * KC, k1 = min(K, k0 + KC), nk = k1 - k0;
  for (int q = tid; q < M * nk; q += 256) {
    const int t = q / nk, kk = q % nk;
    as[t][kk] = bf16_to_f32(a[(int64_t)t * sam + k0 + kk]);
  }
  __syncthreads();
  const int nchunk = N / kCols;
  int cj[CPT];
  bool ok[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    cj[j] = (g * CPT + j) * 256 + tid;
    ok[j] = cj[j] < nchunk;
  }
  float acc[TM][CPT][kCols];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int q = 0; q < kCols; ++q) acc[t][j][q] = 0.f;
  // U k rows per step; the next step's rows are loaded before this step's FMAs, so
  // 2 U rows of this thread's chunks are in flight
  auto load_rows = [&](uint4 (&bv)[U][CPT], int kk) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPT; ++j)
        bv[u][j] = (ok[j] && kk + u < nk)
                       ? ldg_nt(b + (int64_t)(k0 + kk + u) * sbk + cj[j] * kCols)  // read once
                       : make_uint4(0, 0, 0, 0);
  };
  auto fma_rows = [&](const uint4 (&bv)[U][CPT], int kk) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        float bf[kCols];
        unpack8(bv[u][j], bf);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
          if (t < M) {
            const float av = kk + u < nk ? as[t][kk + u] : 0.f;
#pragma unroll
            for (int q = 0; q < kCols; ++q) acc[t][j][q] = fmaf(av, bf[q], acc[t][j][q]);
          }
        }
      }
    }
  };
  uint4 cur[U][CPT], nxt[U][CPT];
  load_rows(cur, 0);
  for (int kk = 0; kk < nk; kk += U) {
    const bool more = kk + U < nk;
    if (more) load_rows(nxt, kk + U);
    fma_rows(cur, kk);
    if (more) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < CPT; ++j) cur[u][j] = nxt[u][j];
    }
  }
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    if (t < M) {
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        if (ok[j]) {
          float4* dst = reinterpret_cast<float4*>(ws + ((int64_t)s * M + t) * N + cj[j] * kCols);
          dst[0] = make_float4(acc[t][j][0], acc[t][j][1], acc[t][j][2], acc[t][j][3]);
          dst[1] = make_float4(acc[t][j][4], acc[t][j][5], acc[t][j][6], acc[t][j][7]);
        }
      }
    }
  }
}

// The epilogue of a reduced 8-column chunk of row t (0: bf16; 1: + r, bf16; 2: c32 += sum
// (+ r)).
__device__ inline void reduce_store(float (&v)[kCols], int t, int ch,
                                    const uint16_t* __restrict__ r, int64_t srm,
                                    uint16_t* __restrict__ c, float* __restrict__ c32,
                                    int64_t scm, int epi) {
  if (r && epi != 0) {
    float rf[kCols];
    unpack8(*reinterpret_cast<const uint4*>(r + (int64_t)t * srm + ch * kCols), rf);
#pragma unroll
    for (int q = 0; q < kCols; ++q) v[q] = v[q] + rf[q];
  }
  if (epi == 2) {
    float4* dst = reinterpret_cast<float4*>(c32 + (int64_t)t * scm + ch * kCols);
    float4 o0 = dst[0], o1 = dst[1];
    o0.x += v[0]; o0.y += v[1]; o0.z += v[2]; o0.w += v[3];
    o1.x += v[4]; o1.y += v[5]; o1.z += v[6]; o1.w += v[7];
    dst[0] = o0;
    dst[1] = o1;
  } else {
    *reinterpret_cast<uint4*>(c + (int64_t)t * scm + ch * kCols) = pack8(v);
  }
}

// Many splits (decode): one wave per (row t, 8-column chunk); lane l adds the partials
// l, l + 64, ... (split sp of row t at ws + sp s_split + t s_tok), then a fixed butterfly.
__global__ __launch_bounds__(256) void oproj_reduce_kernel(
    const float* __restrict__ ws, int64_t s_split, int64_t s_tok, int S, int M, int N,
    const uint16_t* __restrict__ r, int64_t srm, uint16_t* __restrict__ c,
    float* __restrict__ c32, int64_t scm, int epi) {
  const int lane = threadIdx.x % kWave;
  const int64_t w = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  const int nchunk = N / kCols;
  if (w >= (int64_t)M * nchunk) return;
  const int t = (int)(w / nchunk), ch = (int)(w % nchunk);
  float v[kCols] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int sp = lane; sp < S; sp += kWave) {
    const float4* src = reinterpret_cast<const float4*>(ws + sp * s_split + t * s_tok + ch * kCols);
    const float4 p0 = src[0], p1 = src[1];
    v[0] += p0.x; v[1] += p0.y; v[2] += p0.z; v[3] += p0.w;
    v[4] += p1.x; v[5] += p1.y; v[6] += p1.z; v[7] += p1.w;
  }
#pragma unroll
  for (int q = 0; q < kCols; ++q)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v[q] += __shfl_xor(v[q], off, kWave);
  if (lane != 0) return;
  reduce_store(v, t, ch, r, srm, c, c32, scm, epi);
}

// Few splits (the prefill K slices): one thread per (row t, 8-column chunk), the S
// partials added in split order, 8 of them loaded before the first add.
constexpr int kSeqSplits = 32;  // at most this many splits take this kernel

__global__ __launch_bounds__(256) void oproj_reduce_seq_kernel(
    const float* __restrict__ ws, int64_t s_split, int64_t s_tok, int S, int M, int N,
    const uint16_t* __restrict__ r, int64_t srm, uint16_t* __restrict__ c,
    float* __restrict__ c32, int64_t scm, int epi) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nchunk = N / kCols;
  if (q >= (int64_t)M * nchunk) return;
  const int t = (int)(q / nchunk), ch = (int)(q % nchunk);
  const float* base = ws + t * s_tok + ch * kCols;
  float v[kCols] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int sp0 = 0; sp0 < S; sp0 += 8) {
    float4 p[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (sp0 + i < S) {
        const float4* src = reinterpret_cast<const float4*>(base + (int64_t)(sp0 + i) * s_split);
        p[i][0] = src[0];
        p[i][1] = src[1];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (sp0 + i < S) {
        v[0] += p[i][0].x; v[1] += p[i][0].y; v[2] += p[i][0].z; v[3] += p[i][0].w;
        v[4] += p[i][1].x; v[5] += p[i][1].y; v[6] += p[i][1].z; v[7] += p[i][1].w;
      }
    }
  }
  reduce_store(v, t, ch, r, srm, c, c32, scm, epi);
}

// The fixed-order sum of S split partials with the epilogue; the mapping is a function of
// S alone, so a shape always sums in the same order.
hipError_t launch_reduce(const float* ws, int64_t s_split, int64_t s_tok, int S, int M, int N,
                         const void* r, int64_t srm, void* c, int64_t scm, int epi,
                         hipStream_t stream) {
  const int64_t items = (int64_t)M * (N / kCols);
  const auto* rr = static_cast<const uint16_t*>(r);
  if (S <= kSeqSplits)
    oproj_reduce_seq_kernel<<<(int)((items + 255) / 256), 256, 0, stream>>>(
        ws, s_split, s_tok, S, M, N, rr, srm, static_cast<uint16_t*>(c), static_cast<float*>(c),
        scm, epi);
  else
    oproj_reduce_kernel<<<(int)((items + 3) / 4), 256, 0, stream>>>(
        ws, s_split, s_tok, S, M, N, rr, srm, static_cast<uint16_t*>(c), static_cast<float*>(c),
        scm, epi);
  return hipGetLastError();
}

// The row layout of an M-row dense GEMM split S ways along K, on block size BM: "expert"
// s (k slice s) owns the rows m S + s of A viewed as [M S, K / S] (row m S + s is row m's
// slice s); its blocks hold them in m order, padded with the sentinel M S.  S = 1 is the
// identity layout.
__global__ __launch_bounds__(256) void split_layout_kernel(int M, int S, int BM, int per,
                                                           int32_t* __restrict__ sti,
                                                           int32_t* __restrict__ eids,
                                                           int32_t* __restrict__ ntp) {
  const int cap = S * per;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < cap; i += gridDim.x * 256) {
    const int sp = i / per, m = i % per;
    sti[i] = m < M ? m * S + sp : M * S;
    if (i % BM == 0) eids[i / BM] = sp;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) ntp[0] = cap;
}

// o = bf16(c (+ r)), c bf16 or fp32, r bf16 or absent: `epilogue_kernel`.
template <bool F32, bool RES>
__global__ __launch_bounds__(256) void cast_add_kernel(const void* __restrict__ c,
                                                       int64_t sc, const uint16_t* __restrict__ r,
                                                       int64_t sr, uint16_t* __restrict__ o,
                                                       int64_t so, int M, int N) {
  const int nchunk = N / kCols;
  const int64_t total = (int64_t)M * nchunk;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * 256) {
    const int64_t t = q / nchunk;
    const int ch = (int)(q % nchunk);
    float v[kCols];
    if (F32) {
      const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(c) + t * sc + ch * kCols);
      const float4 p0 = src[0], p1 = src[1];
      v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
      v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
    } else {
      unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(c) + t * sc + ch * kCols), v);
    }
    if (RES) {
      float rf[kCols];
      unpack8(*reinterpret_cast<const uint4*>(r + t * sr + ch * kCols), rf);
#pragma unroll
      for (int q2 = 0; q2 < kCols; ++q2) v[q2] = v[q2] + rf[q2];
    }
    *reinterpret_cast<uint4*>(o + t * so + ch * kCols) = pack8(v);
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// decode split: (column groups, k splits, k rows per split, chunks per thread, token rows)
struct Split {
  int ng, S, KC, cpt, tm;
};
Split decode_split(int M, int N, int K) {
  Split sp;
  sp.tm = M == 1 ? 1 : (M <= 4 ? 4 : 16);
  sp.cpt = M == 1 ? 3 : 1;  // acc registers: tm x cpt x 8
  const int cols = 256 * sp.cpt * kCols;
  sp.ng = (N + cols - 1) / cols;
  int S = 512 / sp.ng;  // two workgroups per CU: twice the rows in flight
  if (S < 1) S = 1;
  int KC = (K + S - 1) / S;
  if (KC < 64) KC = 64;
  if (KC > kMaxKC) KC = kMaxKC;
  KC = (KC + 3) / 4 * 4;
  sp.KC = KC;
  sp.S = (K + KC - 1) / KC;
  return sp;
}

// Rows per tile of the prefill mapping: the 256 x 256 tile for 256 .. 2048 rows (it stages
// a fifth fewer bytes through LDS per flop than 128 rows x 512 columns: o_proj at M = 256
// 188 -> 148 us, at M = 2048 483 -> 458 us), else 128 rows.  At M = 8192 its twice as many
// column tiles re-read the 268 MB of A twice as often from HBM (1701 -> 2014 us).
int prefill_bm(int M) { return M >= 256 && M <= 2048 ? 256 : 128; }

// K slices of the prefill mapping: enough (1 .. 16, powers of two) to give the 256 CUs
// about one tile each, keeping every slice a multiple of 64 and at least 1024 k.
int prefill_splits(int M, int N, int K) {
  const int bm = prefill_bm(M);
  const int64_t items = (int64_t)((M + bm - 1) / bm) * (N / (bm == 256 ? 256 : 512));
  int S = 1;
  while (S < 16 && items * S * 2 <= 256 && K % (64 * S * 2) == 0 && K / (S * 2) >= 1024) S *= 2;
  return S;
}

int64_t layout_bytes(int M, int S) {
  const int bm = prefill_bm(M);
  const int64_t per = ((int64_t)M + bm - 1) / bm * bm;
  const int64_t cap = per * S;
  return (cap + cap / bm + 1 + 64) * 4;
}

int64_t round256(int64_t b) { return (b + 255) / 256 * 256; }

}  // namespace

// Workspace the o_proj GEMM needs for M rows: the decode split-K partials, or the identity
// row layout of the prefill mapping.
extern "C" int64_t glm52_oproj_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const Split sp = decode_split(M, N, K);
  const int64_t dec = M <= 16 ? (int64_t)sp.S * M * N * 4 : 0;
  const int S = prefill_splits(M, N, K);
  const int64_t pre = round256(layout_bytes(M, S)) + (S > 1 ? (int64_t)M * S * N * 4 : 0);
  return (dec > pre ? dec : pre) + 256;
}

// The number of K slices glm52_oproj_gemm runs the prefill mapping with for this shape;
// B must be packed with the same count (glm52_oproj_pack).
extern "C" int glm52_oproj_splits(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 1;
  return prefill_splits(M, N, K);
}

extern "C" int64_t glm52_oproj_packed_bytes(int K, int N) {
  return pack_wide512(nullptr, 0, 0, 1, N, K, 0, false, nullptr, nullptr);
}

// B [K, N] (strides in elements) packed for the prefill mapping, as W = B^T cut into
// `splits` K slices (experts of K / splits each).
extern "C" int glm52_oproj_pack(const void* b, int64_t stride_bk, int64_t stride_bn, int K, int N,
                                int splits, void* packed, hipStream_t stream) {
  if (!b || !packed || !al16(packed) || stride_bk <= 0 || stride_bn <= 0 || splits < 1 ||
      (K % splits))
    return GLM52_EINVAL;
  const int Ks = K / splits;
  const int64_t rc = pack_wide512(static_cast<const uint16_t*>(b), (int64_t)Ks * stride_bk,
                                  stride_bn, splits, N, Ks, 0, false,
                                  static_cast<uint16_t*>(packed), stream, stride_bk);
  if (rc == GLM52_EUNSUPPORTED) return GLM52_EUNSUPPORTED;
  return rc < 0 ? (int)(-rc) : GLM52_OK;
}

// c = A @ B with epilogue: r non-null adds the residual row; c_f32 != 0 accumulates into an
// fp32 c (c += result), else c is bf16.  Decode (M <= 16, B with N contiguous) streams B;
// otherwise b_packed (glm52_oproj_pack with the same `splits`) is required.  splits > 1
// runs the K slices as separate experts into fp32 partials (A rows must be contiguous),
// summed in slice order with the epilogue.
extern "C" int glm52_oproj_gemm(const void* a, int64_t stride_am, const void* b, int64_t stride_bk,
                                int64_t stride_bn, const void* b_packed, int splits,
                                const void* r, int64_t stride_rm, void* c, int64_t stride_cm,
                                int c_f32, int M, int N, int K, void* workspace,
                                int64_t workspace_bytes, hipStream_t stream) {
  if (M < 0 || N <= 0 || K <= 0 || (N % 16) || !a || !c || !workspace) return GLM52_EINVAL;
  if (!al16(a) || (stride_am % 8) || stride_am < K || !al16(c) || (stride_cm % 8) ||
      stride_cm < N || !al16(workspace))
    return GLM52_EINVAL;
  if (r && (!al16(r) || (stride_rm % 8) || stride_rm < N)) return GLM52_EINVAL;
  if (M == 0) return GLM52_OK;
  if (workspace_bytes < glm52_oproj_workspace_bytes(M, N, K)) return GLM52_EINVAL;
  const int epi = c_f32 ? 2 : (r ? 1 : 0);
  if (M <= 16 && b && stride_bn == 1 && al16(b) && (stride_bk % 8) == 0 && stride_bk >= N) {
    const Split sp = decode_split(M, N, K);
    float* ws = static_cast<float*>(workspace);
    const dim3 grid(sp.ng, sp.S);
    const auto* aa = static_cast<const uint16_t*>(a);
    const auto* bb = static_cast<const uint16_t*>(b);
    if (sp.tm == 1)
      oproj_splitk_kernel<1, 3, 8><<<grid, 256, 0, stream>>>(aa, stride_am, bb, stride_bk, M, N, K, sp.KC, ws);
    else if (sp.tm == 4)
      oproj_splitk_kernel<4, 1, 8><<<grid, 256, 0, stream>>>(aa, stride_am, bb, stride_bk, M, N, K, sp.KC, ws);
    else
      oproj_splitk_kernel<16, 1, 8><<<grid, 256, 0, stream>>>(aa, stride_am, bb, stride_bk, M, N, K, sp.KC, ws);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return (int)err;
    const hipError_t rerr = launch_reduce(ws, (int64_t)M * N, N, sp.S, M, N, r, stride_rm, c,
                                          stride_cm, epi, stream);
    return rerr == hipSuccess ? GLM52_OK : (int)rerr;
  }
  if (!b_packed || !al16(b_packed)) return GLM52_EUNSUPPORTED;
  const int S = splits;
  if (S < 1 || (N % 512) || (K % (64 * S))) return GLM52_EUNSUPPORTED;
  if (S > 1 && stride_am != K) return GLM52_EINVAL;  // A is viewed as [M S, K / S]
  if (workspace_bytes < round256(layout_bytes(M, S)) + (S > 1 ? (int64_t)M * S * N * 4 : 0))
    return GLM52_EINVAL;
  const int Ks = K / S;
  // one "expert" per K slice over the split row layout, written into the workspace
  const int BM = prefill_bm(M);
  const int per = (M + BM - 1) / BM * BM;
  const int cap = per * S;
  int32_t* sti = static_cast<int32_t*>(workspace);
  int32_t* eids = sti + cap;
  int32_t* ntp = eids + cap / BM + 16;
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + round256(layout_bytes(M, S)));
  split_layout_kernel<<<(cap + 255) / 256 < 1024 ? (cap + 255) / 256 : 1024, 256, 0, stream>>>(
      M, S, BM, per, sti, eids, ntp);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  const int64_t sam = S > 1 ? Ks : stride_am;
  const int64_t ab = ((int64_t)M * S - 1) * sam * 2 + (int64_t)Ks * 2;
  if (ab >= 0x7ffffff0) return GLM52_EUNSUPPORTED;
  GemmArgs g{static_cast<const uint16_t*>(a), sam, 1, static_cast<const uint16_t*>(b_packed),
             0, 0, 0, nullptr, stride_cm, nullptr, sti, eids, ntp, BM, N, Ks, M * S, 4, 64,
             nullptr, 0, nullptr, nullptr, 0, 0, (int)ab, 0};
  g.Wp = static_cast<const uint16_t*>(b_packed);
  if (S == 1) {
    g.epi = epi;
    g.C = epi == 2 ? nullptr : static_cast<uint16_t*>(c);
    g.R = static_cast<const uint16_t*>(r);
    g.srm = stride_rm;
    g.C32 = epi == 2 ? static_cast<float*>(c) : nullptr;
    return launch_wide512(g, cap, false, false, stream);
  }
  // fp32 partials [M S][N], then the fixed-order sum over the slices with the epilogue
  g.epi = 3;
  g.C32 = part;
  g.scm = N;
  const int rc = launch_wide512(g, cap, false, false, stream);
  if (rc != GLM52_OK) return rc;
  const hipError_t rerr = launch_reduce(part, N, (int64_t)S * N, S, M, N, r, stride_rm, c,
                                        stride_cm, epi, stream);
  return rerr == hipSuccess ? GLM52_OK : (int)rerr;
}

// o = bf16(c (+ r)): `epilogue_kernel` (c bf16 or fp32).
extern "C" int glm52_cast_add(const void* c, int c_f32, int64_t stride_c, const void* r,
                              int64_t stride_r, void* o, int64_t stride_o, int M, int N,
                              hipStream_t stream) {
  if (M < 0 || N <= 0 || (N % 8) || !c || !o || !al16(c) || !al16(o) || (stride_c % 8) ||
      (stride_o % 8) || (r && (!al16(r) || (stride_r % 8))))
    return GLM52_EINVAL;
  if (M == 0) return GLM52_OK;
  const int64_t total = (int64_t)M * (N / kCols);
  const int grid = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  const auto* rr = static_cast<const uint16_t*>(r);
  auto* oo = static_cast<uint16_t*>(o);
  if (c_f32) {
    if (r) cast_add_kernel<true, true><<<grid, 256, 0, stream>>>(c, stride_c, rr, stride_r, oo, stride_o, M, N);
    else cast_add_kernel<true, false><<<grid, 256, 0, stream>>>(c, stride_c, rr, stride_r, oo, stride_o, M, N);
  } else {
    if (r) cast_add_kernel<false, true><<<grid, 256, 0, stream>>>(c, stride_c, rr, stride_r, oo, stride_o, M, N);
    else cast_add_kernel<false, false><<<grid, 256, 0, stream>>>(c, stride_c, rr, stride_r, oo, stride_o, M, N);
  }
  GLM52_RETURN_LAUNCH();
}
