// Grouped expert GEMMs of the GLM-5.2 MoE block on bf16 MFMA, gfx950.
//
// One source serves both expert GEMMs, like `moe_gateup_kernel`
// (`glm52/kernels/moe_gateup.py:34-148`) and `moe_down_kernel`
// (`glm52/kernels/moe_down_merge.py:66-169`), which mirror sglang's `fused_moe_kernel`:
//
//   for every padded row slot r of the dispatch layout with token f = sorted_ids[r] < num_valid
//   and expert e = expert_ids[r / BM]:
//     gated (w13 + SwiGLU): g = A[f / a_div] . W[e, n, :],  u = A[f / a_div] . W[e, off + n, :]
//                           C[f, n] = bf16(silu(g) * u)
//     plain              :  c = A[f / a_div] . W[e, n, :]
//                           C[f, n] = bf16(c * topk_w[f])   if weighted, else bf16(c)
//
// Both operands are K-contiguous (A rows and W rows), which is the native operand layout
// of `v_mfma_f32_16x16x32_bf16`: a lane supplies 8 consecutive k of one row of A and 8 of
// one row of W.  Accumulation is fp32.
//
// Two mappings, chosen by the host from the number of rows per expert:
//
//  * stream (decode): the GEMM is a weight stream.  An item is one 16-row slice of the
//    layout times 16 output columns; the four waves of a workgroup each take a quarter of
//    K, load their W fragments straight from HBM into registers (128-bit non-temporal
//    loads, U steps of 64 k in flight), read the token rows through a range-checked
//    buffer (padding rows read zeros without a memory access), and meet in LDS for the
//    split-K sum and the epilogue.
//
//  * tiled (prefill): LDS-staged BM x BN tiles with a register-staged double buffer; a
//    workgroup of four waves computes a BM x BN block with 16x16x32 MFMAs.  Items are
//    ordered so that the workgroups on one XCD (consecutive ids modulo 8 share an XCD)
//    walk consecutive row blocks of the same expert, so a W tile is fetched from HBM once
//    and served from that XCD's L2 to the other row blocks of the expert.
//
// Both kernels are persistent: the grid is sized on the host for the worst-case layout
// and every workgroup loops over the items that exist for the layout the device holds
// (`num_tokens_post_padded` is read on the device), so no host sync is needed.
#include "moe_gemm.h"

using namespace glm52;

namespace {

// ------------------------------------------------------------------------------------
// stream mapping
// ------------------------------------------------------------------------------------
template <bool GATED, bool WEIGHTED, int U>
__global__ __launch_bounds__(256) void moe_gemm_stream_kernel(GemmArgs p) {
  __shared__ float red[4][GATED ? 2 : 1][4][kWave];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int r = lane % 16;  // A row / W row within the 16 x 16 tile
  const int g = lane / 16;  // k group

  const int ntp = *p.ntp;
  const int num_m = ntp / 16;
  const int num_n = p.n_out / 16;
  const int items_r = num_m * num_n;
  const int items = items_r + ((p.x_rows + 15) / 16) * num_n;  // + the extra expert's
  const int kq = p.K / 4;
  const int kbeg = wv * kq;

  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    // n fastest: consecutive workgroups stream different W rows of the same expert
    const bool extra = it >= items_r;
    const int li = extra ? it - items_r : it;
    const int pid_m = li / num_n;
    const int pid_n = li % num_n;
    const int row0 = pid_m * 16;
    int tok;
    bool tok_ok;
    const uint16_t* wbase;
    if (extra) {  // the extra expert: rows are tokens 0 .. x_rows - 1, A row = token
      tok = row0 + r;
      tok_ok = tok < p.x_rows;
      wbase = p.Wx;
    } else {
      if (p.sti[row0] >= p.num_valid) continue;  // an all-padding slice (BM > 16)
      tok = p.sti[row0 + r];
      tok_ok = tok < p.num_valid;
      wbase = p.W + (int64_t)p.eids[row0 / p.BM] * p.swe;
    }
    const int n0 = pid_n * 16;
    // token rows through a range-checked buffer: padding rows read zeros at no cost
    const __amdgpu_buffer_rsrc_t arsrc = extra ? buffer_rsrc(p.Ax, p.ax_bytes) : buffer_rsrc(p.A, p.a_bytes);
    const uint32_t abad = (uint32_t)(extra ? p.ax_bytes : p.a_bytes);
    const uint32_t aoff = tok_ok ? (uint32_t)(((int64_t)(extra ? tok : tok / p.a_div) *
                                               (extra ? p.sax : p.sam) + 16 * g) * 2)
                                 : abad;
    const uint16_t* wg = wbase + (int64_t)(n0 + r) * p.swn + 16 * g;
    const uint16_t* wu = wg + (int64_t)p.gu_off * p.swn;

    floatx4_t accg = {0.f, 0.f, 0.f, 0.f};
    floatx4_t accu = {0.f, 0.f, 0.f, 0.f};
    // U steps of 64 k in flight per lane (W: non-temporal 16-byte loads), then their MFMAs
    int k = kbeg;
    const int kend = kbeg + kq;
    for (; k < kend; k += 64 * U) {
      uint4 bg[U][2], bu[U][2], av[U][2];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kk = k + u * 64;
        if (kk < kend) {
          bg[u][0] = ldg_nt(wg + kk);
          bg[u][1] = ldg_nt(wg + kk + 8);
          if (GATED) {
            bu[u][0] = ldg_nt(wu + kk);
            bu[u][1] = ldg_nt(wu + kk + 8);
          }
          av[u][0] = ldb(arsrc, aoff + kk * 2);
          av[u][1] = ldb(arsrc, aoff + kk * 2 + 16);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (k + u * 64 < kend) {
          accg = mfma16(av[u][0], bg[u][0], accg);
          accg = mfma16(av[u][1], bg[u][1], accg);
          if (GATED) {
            accu = mfma16(av[u][0], bu[u][0], accu);
            accu = mfma16(av[u][1], bu[u][1], accu);
          }
        }
      }
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[wv][0][i][lane] = accg[i];
      if (GATED) red[wv][GATED ? 1 : 0][i][lane] = accu[i];
    }
    __syncthreads();
    if (wv == 0) {
      // lane holds rows 4*g + i of column r of the 16 x 16 output tile
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int orow = 4 * g + i;
        const int otok = extra ? row0 + orow : p.sti[row0 + orow];
        const float sg = ((red[0][0][i][lane] + red[1][0][i][lane]) + red[2][0][i][lane]) + red[3][0][i][lane];
        float v;
        if (GATED) {
          const float su = ((red[0][GATED ? 1 : 0][i][lane] + red[1][GATED ? 1 : 0][i][lane]) +
                            red[2][GATED ? 1 : 0][i][lane]) + red[3][GATED ? 1 : 0][i][lane];
          v = silu_mul(sg, su);
        } else {
          v = sg;
        }
        if (extra) {
          if (otok < p.x_rows) p.Cx[(int64_t)otok * p.scx + n0 + r] = f32_to_bf16(v);
        } else if (otok < p.num_valid) {
          if (WEIGHTED) v = v * p.topw[otok];
          p.C[(int64_t)otok * p.scm + n0 + r] = f32_to_bf16(v);
        }
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------
// tiled mapping
// ------------------------------------------------------------------------------------
template <int BM, int BN, int BK, int WM, int WN, bool GATED, bool WEIGHTED>
__global__ __launch_bounds__(256) void moe_gemm_tiled_kernel(GemmArgs p) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int NB = GATED ? 2 * BN : BN;  // W rows staged per tile
  constexpr int LDK = BK + 8;              // +16 B row pad: conflict-free 128-bit reads
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  static_assert(TM >= 1 && TN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "wave tile");
  constexpr int CPR = BK / 8;  // 16-byte chunks per tile row
  constexpr int CH_A = BM * CPR, CH_B = NB * CPR;
  constexpr int QA = (CH_A + 255) / 256, QB = (CH_B + 255) / 256;
  constexpr int NG = GATED ? 2 : 1;

  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][NB][LDK];
  __shared__ int toks[BM];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int wm = wv / WN, wn = wv % WN;
  const int l16 = lane % 16, lg = lane / 16;

  const int ntp = *p.ntp;
  const int num_m = ntp / BM;
  const int num_n = p.n_out / BN;
  const int items = num_m * num_n;
  const int nk = p.K / BK;

  // XCD-aware order: ids congruent mod 8 run on one XCD; give each XCD a contiguous
  // range of logical items.
  const int per_xcd = (items + 7) / 8;
  const int span = per_xcd * 8;

  for (int it = blockIdx.x; it < span; it += gridDim.x) {
    const int L = (it % 8) * per_xcd + it / 8;
    if (L >= items) continue;
    // grouped swizzle: GROUP_M row blocks x all column tiles, row block fastest, so a
    // W tile is reused by the group's row blocks and their A rows stay in L2
    const int in_group = p.group_m * num_n;
    const int first_m = (L / in_group) * p.group_m;
    const int gsz = min(num_m - first_m, p.group_m);
    const int pid_m = first_m + (L % in_group) % gsz;
    const int pid_n = (L % in_group) / gsz;
    const int row0 = pid_m * BM;
    if (p.sti[row0] >= p.num_valid) continue;  // uniform: an all-padding block
    const int e = p.eids[pid_m];
    const int n0 = pid_n * BN;

    for (int q = tid; q < BM; q += 256) toks[q] = p.sti[row0 + q];
    __syncthreads();

    // per-thread global sources for the A and W chunks it copies
    const uint16_t* asrc[QA];
    bool aok[QA];
    int arow_l[QA], akc[QA];
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int c = tid + q * 256;
      const int rr = c / CPR, kc = c % CPR;
      arow_l[q] = rr;
      akc[q] = kc;
      bool ok = c < CH_A;
      int t = ok ? toks[rr] : 0;
      ok = ok && t < p.num_valid;
      aok[q] = ok;
      asrc[q] = p.A + (int64_t)(ok ? t / p.a_div : 0) * p.sam + kc * 8;
    }
    const uint16_t* bsrc[QB];
    int brow_l[QB], bkc[QB];
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const int c = tid + q * 256;
      const int nn = c / CPR, kc = c % CPR;
      brow_l[q] = nn;
      bkc[q] = kc;
      int grow = n0 + nn;
      if (GATED && nn >= BN) grow = p.gu_off + n0 + (nn - BN);
      bsrc[q] = p.W + (int64_t)e * p.swe + (int64_t)(c < CH_B ? grow : n0) * p.swn + kc * 8;
    }

    uint4 ra[QA], rb[QB];
    auto gload = [&](int kt) {
      const int koff = kt * BK;
#pragma unroll
      for (int q = 0; q < QA; ++q) ra[q] = aok[q] ? ldg(asrc[q] + koff) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int q = 0; q < QB; ++q)
        if (tid + q * 256 < CH_B) rb[q] = ldg(bsrc[q] + koff);
    };
    auto sstore = [&](int buf) {
#pragma unroll
      for (int q = 0; q < QA; ++q)
        if (tid + q * 256 < CH_A) *reinterpret_cast<uint4*>(&As[buf][arow_l[q]][akc[q] * 8]) = ra[q];
#pragma unroll
      for (int q = 0; q < QB; ++q)
        if (tid + q * 256 < CH_B) *reinterpret_cast<uint4*>(&Bs[buf][brow_l[q]][bkc[q] * 8]) = rb[q];
    };

    floatx4_t acc[NG][TM][TN];
#pragma unroll
    for (int h = 0; h < NG; ++h)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[h][i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        uint4 af[TM], bf[NG][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const uint4*>(&As[cur][wm * WTM + i * 16 + l16][ks * 32 + lg * 8]);
#pragma unroll
        for (int h = 0; h < NG; ++h)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            bf[h][j] = *reinterpret_cast<const uint4*>(&Bs[cur][h * BN + wn * WTN + j * 16 + l16][ks * 32 + lg * 8]);
#pragma unroll
        for (int h = 0; h < NG; ++h)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[h][i][j] = mfma16(af[i], bf[h][j], acc[h][i][j]);
      }
      if (kt + 1 < nk) sstore(cur ^ 1);
      __syncthreads();
    }

    // epilogue: lane holds rows 4*lg + q of column l16 of each 16 x 16 sub-tile
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int rl = wm * WTM + i * 16 + lg * 4 + q;
          const int t = toks[rl];
          if (t < p.num_valid) {
            float v = GATED ? silu_mul(acc[0][i][j][q], acc[NG - 1][i][j][q]) : acc[0][i][j][q];
            if (WEIGHTED) v = v * p.topw[t];
            p.C[(int64_t)t * p.scm + n0 + wn * WTN + j * 16 + l16] = f32_to_bf16(v);
          }
        }
    __syncthreads();
  }
}

template <bool GATED, bool WEIGHTED>
int launch_stream(const GemmArgs& a, int capacity, hipStream_t st) {
  const int items_max = (capacity / 16 + (a.x_rows + 15) / 16) * (a.n_out / 16);
  int grid = items_max < 4096 ? items_max : 4096;
  if (grid < 1) grid = 1;
  moe_gemm_stream_kernel<GATED, WEIGHTED, 4><<<grid, 256, 0, st>>>(a);
  GLM52_RETURN_LAUNCH();
}

template <int BM, int BN, int BK, int WM, int WN, bool GATED, bool WEIGHTED>
int launch_tiled(const GemmArgs& a, int capacity, hipStream_t st) {
  if (a.BM != BM || (a.n_out % BN) || (a.K % BK)) return GLM52_EUNSUPPORTED;
  const int items_max = (capacity / BM) * (a.n_out / BN);
  int grid = items_max < 2048 ? items_max : 2048;
  grid = ((grid + 7) / 8) * 8;
  moe_gemm_tiled_kernel<BM, BN, BK, WM, WN, GATED, WEIGHTED><<<grid, 256, 0, st>>>(a);
  GLM52_RETURN_LAUNCH();
}

template <bool GATED, bool WEIGHTED>
int launch_tiled_bm(const GemmArgs& a, int capacity, hipStream_t st) {
  // gated tiles stage 2 * BN W rows; plain tiles stage BN
  if constexpr (GATED) {
    switch (a.BM) {
      case 32: return launch_tiled<32, 64, 64, 1, 4, GATED, WEIGHTED>(a, capacity, st);
      case 64: return launch_tiled<64, 64, 64, 2, 2, GATED, WEIGHTED>(a, capacity, st);
      case 128: return launch_tiled<128, 64, 64, 2, 2, GATED, WEIGHTED>(a, capacity, st);
      default: return GLM52_EUNSUPPORTED;
    }
  } else {
    switch (a.BM) {
      case 32: return launch_tiled<32, 128, 64, 1, 4, GATED, WEIGHTED>(a, capacity, st);
      case 64: return launch_tiled<64, 128, 64, 2, 2, GATED, WEIGHTED>(a, capacity, st);
      case 128: return launch_tiled<128, 128, 64, 2, 2, GATED, WEIGHTED>(a, capacity, st);
      default: return GLM52_EUNSUPPORTED;
    }
  }
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// Output rows take 8-byte stores in the contiguous-run mapping.
bool c_ok8(const void* c, int64_t stride) {
  return (reinterpret_cast<uintptr_t>(c) & 7u) == 0 && (stride % 4) == 0;
}

// Bytes spanned by the A rows a layout can address: row f / a_div of every valid flat
// index f, each K elements long at stride sa (the buffer range of the token loads).
int a_bytes(int num_valid, int a_div, int64_t sa, int k) {
  const int64_t rows = ((int64_t)num_valid + a_div - 1) / a_div;
  const int64_t b = rows == 0 ? 0 : ((rows - 1) * sa + k) * 2;
  return b > 0x7ffffff0 ? 0x7ffffff0 : (int)b;
}

}  // namespace

// variant: 0 = choose: block_m 16 runs the contiguous-run weight stream (6), and the
// stream mapping (1) for what it does not cover (k % 512 != 0, output rows not 8-byte
// aligned); block_m 64, 128 and 256 run the 512-row W tiles (5; 256: 256 x 256 tiles), and
// at 64 and 128 the 256-row wide mapping (3) for what those do not cover (gated n_out %
// 256 != 0, plain n_out % 512 != 0, token rows past 2^31 bytes); any other block_m (32)
// runs the tiled mapping (2).  1 = stream, 2 = tiled, 3 = wide (64-k stages), 5 = 512-row W
// tiles (moe_gemm_wide.hip), 6 = contiguous-run weight stream (moe_gemm_runs.hip; block_m
// 16) force one mapping.
extern "C" int glm52_moe_gemm(const void* a, int64_t stride_am, int a_row_div, const void* w,
                              int64_t stride_we, int64_t stride_wn, int gate_up_offset,
                              void* c, int64_t stride_cm, const float* topk_weights,
                              const int32_t* sorted_token_ids, const int32_t* expert_ids,
                              const int32_t* num_tokens_post_padded, int capacity, int block_m,
                              int num_valid_tokens, int n_out, int k, int gated, int variant,
                              hipStream_t stream) {
  if (!a || !w || !c || !sorted_token_ids || !expert_ids || !num_tokens_post_padded)
    return GLM52_EINVAL;
  if (block_m <= 0 || (block_m % 16) != 0 || capacity < 0 || (capacity % block_m) != 0)
    return GLM52_EINVAL;
  if (n_out <= 0 || (n_out % 16) != 0 || k <= 0 || (k % 256) != 0 || a_row_div <= 0)
    return GLM52_EINVAL;
  if (!al16(a) || !al16(w) || (stride_am % 8) || (stride_we % 8) || (stride_wn % 8)) return GLM52_EINVAL;
  if (gated && (gate_up_offset < n_out)) return GLM52_EINVAL;
  if (capacity == 0) return GLM52_OK;
  GemmArgs g{static_cast<const uint16_t*>(a), stride_am, a_row_div,
             static_cast<const uint16_t*>(w), stride_we, stride_wn, gate_up_offset,
             static_cast<uint16_t*>(c), stride_cm, topk_weights, sorted_token_ids, expert_ids,
             num_tokens_post_padded, block_m, n_out, k, num_valid_tokens, 4, 64,
             nullptr, 0, nullptr, nullptr, 0, 0, a_bytes(num_valid_tokens, a_row_div, stride_am, k), 0};
  const bool weighted = topk_weights != nullptr;
  const bool auto_wide = variant == 0 && (block_m == 64 || block_m == 128 || block_m == 256);
  if (variant == 5 || auto_wide) {
    // the 512-row mapping addresses token rows with 32-bit byte offsets; shapes it has no
    // instance for fall back to the 256-row mapping when the mapping was not forced
    const int rc = g.a_bytes < 0x7ffffff0 ? launch_wide512(g, capacity, gated != 0, weighted, stream)
                                          : GLM52_EUNSUPPORTED;
    if (rc != GLM52_EUNSUPPORTED || variant == 5) return rc;
  }
  if (variant == 3 || auto_wide) {
    g.stage_k = 64;
    return launch_wide(g, capacity, gated != 0, weighted, stream);
  }
  if (variant == 4 || variant < 0 || variant > 6) return GLM52_EINVAL;
  if (variant == 6 || (variant == 0 && block_m == 16)) {
    // contiguous-run weight stream; shapes it has no instance for fall back to the stream
    // mapping unless it was forced
    const int rc = c_ok8(c, stride_cm) ? launch_runs(g, capacity, gated != 0, weighted, false, stream)
                                       : GLM52_EUNSUPPORTED;
    if (rc != GLM52_EUNSUPPORTED || variant == 6) return rc;
  }
  const bool use_stream = variant == 1 || (variant == 0 && block_m == 16);
  if (use_stream) {
    if (gated) return weighted ? launch_stream<true, true>(g, capacity, stream)
                               : launch_stream<true, false>(g, capacity, stream);
    return weighted ? launch_stream<false, true>(g, capacity, stream)
                    : launch_stream<false, false>(g, capacity, stream);
  }
  if (gated) return weighted ? launch_tiled_bm<true, true>(g, capacity, stream)
                             : launch_tiled_bm<true, false>(g, capacity, stream);
  return weighted ? launch_tiled_bm<false, true>(g, capacity, stream)
                  : launch_tiled_bm<false, false>(g, capacity, stream);
}

// Packed weights for the 512-row tile mapping (prefill, block_m 64 or 128).  The mapping
// reads every 32-k stage of a 512-row W tile as 512 runs of 64 bytes, one per row, which
// the HBM serves far below its streaming rate; packed, a stage is 32 KB of contiguous
// memory in exactly the order its loads fill LDS.  Same values, same arithmetic: the
// packed launch computes the same bits as glm52_moe_gemm on the unpacked weights.
extern "C" int64_t glm52_packed_w512_bytes(int num_experts, int n_out, int k, int gated) {
  return pack_wide512(nullptr, 0, 0, num_experts, n_out, k, 0, gated != 0, nullptr, nullptr);
}

extern "C" int glm52_pack_w512(const void* w, int64_t stride_we, int64_t stride_wn,
                               int num_experts, int n_out, int k, int gate_up_offset, int gated,
                               void* packed, hipStream_t stream) {
  if (!w || !packed || !al16(w) || !al16(packed) || (stride_we % 8) || (stride_wn % 8) ||
      stride_wn < k)
    return GLM52_EINVAL;
  if (gated && gate_up_offset < n_out) return GLM52_EINVAL;
  const int64_t rc = pack_wide512(static_cast<const uint16_t*>(w), stride_we, stride_wn,
                                  num_experts, n_out, k, gate_up_offset, gated != 0,
                                  static_cast<uint16_t*>(packed), stream);
  if (rc == GLM52_EUNSUPPORTED) return GLM52_EUNSUPPORTED;
  return rc < 0 ? (int)(-rc) : GLM52_OK;
}

// The down GEMM with the atomic expert merge (FUSE_MERGE): for every valid flat token f of
// the layout, out[f / top_k, :] += bf16(topk_weights[f] * (a[f] . w[e]^T)), each add a
// packed bf16 atomic (two outputs a word), so the order of a row's adds -- and with it the
// rounding -- depends on timing.  out [T, n_out] must be seeded by the caller (zeros, or
// the residual).  w_packed (glm52_pack_w512 of w, may be null) is read by the 512-row tile
// mapping.  block_m 16 (contiguous-run mapping) or 64 / 128 (512-row tiles).
extern "C" int glm52_moe_down_merge(const void* a, int64_t stride_am, const void* w,
                                    int64_t stride_we, int64_t stride_wn, const void* w_packed,
                                    void* out, int64_t stride_om, const float* topk_weights,
                                    const int32_t* sorted_token_ids, const int32_t* expert_ids,
                                    const int32_t* num_tokens_post_padded, int capacity,
                                    int block_m, int num_valid_tokens, int top_k, int n_out,
                                    int k, hipStream_t stream) {
  if (!a || !w || !out || !topk_weights || !sorted_token_ids || !expert_ids ||
      !num_tokens_post_padded || top_k < 1)
    return GLM52_EINVAL;
  if (capacity < 0 || (capacity % 16) != 0 || n_out <= 0 || (n_out % 16) || k <= 0 || (k % 256))
    return GLM52_EINVAL;
  if (!al16(a) || !al16(w) || (stride_am % 8) || (stride_we % 8) || (stride_wn % 8) ||
      (reinterpret_cast<uintptr_t>(out) & 3u) || (stride_om % 2) || stride_om < n_out ||
      (w_packed && !al16(w_packed)))
    return GLM52_EINVAL;
  if (block_m != 16 && block_m != 64 && block_m != 128 && block_m != 256)
    return GLM52_EUNSUPPORTED;
  if (capacity % block_m) return GLM52_EINVAL;
  if (capacity == 0) return GLM52_OK;
  GemmArgs g{static_cast<const uint16_t*>(a), stride_am, 1, static_cast<const uint16_t*>(w),
             stride_we, stride_wn, 0, static_cast<uint16_t*>(out), stride_om, topk_weights,
             sorted_token_ids, expert_ids, num_tokens_post_padded, block_m, n_out, k,
             num_valid_tokens, 4, 64, nullptr, 0, nullptr, nullptr, 0, 0,
             a_bytes(num_valid_tokens, 1, stride_am, k), 0};
  g.merge_topk = top_k;
  if (block_m == 16) {
    if (w_packed) return GLM52_EINVAL;  // the run mapping reads w in place
    return launch_runs(g, capacity, false, true, false, stream);
  }
  if (g.a_bytes >= 0x7ffffff0) return GLM52_EUNSUPPORTED;
  g.Wp = static_cast<const uint16_t*>(w_packed);
  return launch_wide512(g, capacity, false, true, stream);
}

extern "C" int glm52_moe_gemm_packed(const void* a, int64_t stride_am, int a_row_div,
                                     const void* w_packed, void* c, int64_t stride_cm,
                                     const float* topk_weights,
                                     const int32_t* sorted_token_ids, const int32_t* expert_ids,
                                     const int32_t* num_tokens_post_padded, int capacity,
                                     int block_m, int num_valid_tokens, int n_out, int k,
                                     int gated, hipStream_t stream) {
  if (!a || !w_packed || !c || !sorted_token_ids || !expert_ids || !num_tokens_post_padded)
    return GLM52_EINVAL;
  if ((block_m != 16 && block_m != 64 && block_m != 128 && block_m != 256) || capacity < 0 ||
      (capacity % block_m) != 0)
    return GLM52_EINVAL;
  if (n_out <= 0 || (n_out % (gated ? 256 : 512)) != 0 || k <= 0 ||
      (k % (block_m == 16 ? 512 : 64)) != 0 || a_row_div <= 0)
    return GLM52_EINVAL;
  if (!al16(a) || !al16(w_packed) || (stride_am % 8) || !al16(c) || (stride_cm % 8))
    return GLM52_EINVAL;
  if (capacity == 0) return GLM52_OK;
  const int ab = a_bytes(num_valid_tokens, a_row_div, stride_am, k);
  if (ab < 0 || ab >= 0x7ffffff0) return GLM52_EUNSUPPORTED;
  GemmArgs g{static_cast<const uint16_t*>(a), stride_am, a_row_div,
             static_cast<const uint16_t*>(w_packed), 0, 0, gated ? n_out : 0,
             static_cast<uint16_t*>(c), stride_cm, topk_weights, sorted_token_ids, expert_ids,
             num_tokens_post_padded, block_m, n_out, k, num_valid_tokens, 4, 64,
             nullptr, 0, nullptr, nullptr, 0, 0, ab, 0};
  g.Wp = static_cast<const uint16_t*>(w_packed);
  if (block_m == 16)  // the contiguous-run weight stream on the packed load slots
    return launch_runs(g, capacity, gated != 0, topk_weights != nullptr, false, stream);
  return launch_wide512(g, capacity, gated != 0, topk_weights != nullptr, stream);
}

// glm52_moe_gemm_packed with the shared expert in the same launch (prefill): an extra
// expert with its own packed weights (glm52_pack_w512 of the [1, N, K] shared weight, same
// n_out / k / gated) applied to rows 0 .. shared_rows - 1 of a_shared, without routing
// weight, written to c_shared.  Its items follow each XCD's share of the routed items.
extern "C" int glm52_moe_gemm_packed_shared(
    const void* a, int64_t stride_am, int a_row_div, const void* w_packed, void* c,
    int64_t stride_cm, const float* topk_weights, const int32_t* sorted_token_ids,
    const int32_t* expert_ids, const int32_t* num_tokens_post_padded, int capacity, int block_m,
    int num_valid_tokens, const void* a_shared, int64_t stride_as, const void* w_shared_packed,
    void* c_shared, int64_t stride_cs, int shared_rows, int n_out, int k, int gated,
    hipStream_t stream) {
  if (!a || !w_packed || !c || !sorted_token_ids || !expert_ids || !num_tokens_post_padded ||
      !a_shared || !w_shared_packed || !c_shared || shared_rows < 0)
    return GLM52_EINVAL;
  if ((block_m != 16 && block_m != 64 && block_m != 128 && block_m != 256) || capacity < 0 ||
      (capacity % block_m) != 0)
    return GLM52_EINVAL;
  if (n_out <= 0 || (n_out % (gated ? 256 : 512)) != 0 || k <= 0 ||
      (k % (block_m == 16 ? 512 : 64)) != 0 || a_row_div <= 0)
    return GLM52_EINVAL;
  if (!al16(a) || !al16(w_packed) || (stride_am % 8) || !al16(c) || (stride_cm % 8) ||
      !al16(a_shared) || (stride_as % 8) || !al16(w_shared_packed) || !al16(c_shared) ||
      (stride_cs % 8))
    return GLM52_EINVAL;
  if (capacity == 0 && shared_rows == 0) return GLM52_OK;
  const int ab = a_bytes(num_valid_tokens, a_row_div, stride_am, k);
  const int axb = a_bytes(shared_rows, 1, stride_as, k);
  if (ab < 0 || ab >= 0x7ffffff0 || axb < 0 || axb >= 0x7ffffff0) return GLM52_EUNSUPPORTED;
  GemmArgs g{static_cast<const uint16_t*>(a), stride_am, a_row_div,
             static_cast<const uint16_t*>(w_packed), 0, 0, gated ? n_out : 0,
             static_cast<uint16_t*>(c), stride_cm, topk_weights, sorted_token_ids, expert_ids,
             num_tokens_post_padded, block_m, n_out, k, num_valid_tokens, 4, 64,
             static_cast<const uint16_t*>(a_shared), stride_as,
             static_cast<const uint16_t*>(w_shared_packed), static_cast<uint16_t*>(c_shared),
             stride_cs, shared_rows, ab, axb};
  g.Wp = static_cast<const uint16_t*>(w_packed);
  if (block_m == 16)  // the contiguous-run weight stream on the packed load slots
    return launch_runs(g, capacity, gated != 0, topk_weights != nullptr, false, stream);
  return launch_wide512(g, capacity, gated != 0, topk_weights != nullptr, stream);
}

// The routed grouped GEMM and the shared expert's GEMM in one weight-streaming launch
// (decode): the shared expert is an extra expert whose rows are the tokens 0 .. T - 1 of
// its own input (no routing weight), written to its own output.  Same operand rules as
// glm52_moe_gemm with block_m = 16.
extern "C" int glm52_moe_gemm_shared(const void* a, int64_t stride_am, int a_row_div,
                                     const void* w, int64_t stride_we, int64_t stride_wn,
                                     int gate_up_offset, void* c, int64_t stride_cm,
                                     const float* topk_weights, const int32_t* sorted_token_ids,
                                     const int32_t* expert_ids,
                                     const int32_t* num_tokens_post_padded, int capacity,
                                     int block_m, int num_valid_tokens, const void* a_shared,
                                     int64_t stride_as, const void* w_shared, void* c_shared,
                                     int64_t stride_cs, int shared_rows, int n_out, int k,
                                     int gated, hipStream_t stream) {
  if (!a || !w || !c || !sorted_token_ids || !expert_ids || !num_tokens_post_padded ||
      !a_shared || !w_shared || !c_shared)
    return GLM52_EINVAL;
  if (!al16(a_shared) || (stride_as % 8)) return GLM52_EINVAL;
  if (block_m != 16 || capacity < 0 || (capacity % block_m) || shared_rows < 0) return GLM52_EINVAL;
  if (n_out <= 0 || (n_out % 16) != 0 || k <= 0 || (k % 256) != 0 || a_row_div <= 0)
    return GLM52_EINVAL;
  if (!al16(a) || !al16(w) || !al16(w_shared) || (stride_am % 8) || (stride_we % 8) ||
      (stride_wn % 8))
    return GLM52_EINVAL;
  if (gated && (gate_up_offset < n_out)) return GLM52_EINVAL;
  GemmArgs g{static_cast<const uint16_t*>(a), stride_am, a_row_div,
             static_cast<const uint16_t*>(w), stride_we, stride_wn, gate_up_offset,
             static_cast<uint16_t*>(c), stride_cm, topk_weights, sorted_token_ids, expert_ids,
             num_tokens_post_padded, block_m, n_out, k, num_valid_tokens, 4, 64,
             static_cast<const uint16_t*>(a_shared), stride_as,
             static_cast<const uint16_t*>(w_shared), static_cast<uint16_t*>(c_shared), stride_cs,
             shared_rows, a_bytes(num_valid_tokens, a_row_div, stride_am, k),
             a_bytes(shared_rows, 1, stride_as, k)};
  const bool weighted = topk_weights != nullptr;
  if (c_ok8(c, stride_cm) && c_ok8(c_shared, stride_cs)) {
    const int rc = launch_runs(g, capacity, gated != 0, weighted, false, stream);
    if (rc != GLM52_EUNSUPPORTED) return rc;
  }
  if (gated) return weighted ? launch_stream<true, true>(g, capacity, stream)
                             : launch_stream<true, false>(g, capacity, stream);
  return weighted ? launch_stream<false, true>(g, capacity, stream)
                  : launch_stream<false, false>(g, capacity, stream);
}

// Decode (T <= 4 tokens): the router's biased top-k and the dispatch layout (block_m 16),
// derived from the logits inside the routed w13 + SwiGLU launch with the shared expert --
// glm52_router_topk_align followed by glm52_moe_gemm_shared (gated), in one launch with no
// grid-wide wait (moe_gemm_runs.hip).
extern "C" int glm52_moe_gemm_route_shared(
    const float* logits, int64_t stride_l, const float* bias, int T, int E, int topk,
    float scale, int norm_prob, float* topw, int64_t stride_w, int32_t* topi, int64_t stride_i,
    int32_t* sorted_token_ids, int32_t* expert_ids, int32_t* num_tokens_post_padded,
    int capacity, const void* a, int64_t stride_am, const void* w, int64_t stride_we,
    int64_t stride_wn, int gate_up_offset, void* c, int64_t stride_cm, const void* a_shared,
    int64_t stride_as, const void* w_shared, void* c_shared, int64_t stride_cs, int n_out,
    int k, hipStream_t stream) {
  if (!logits || !topw || !topi || !sorted_token_ids || !expert_ids || !num_tokens_post_padded ||
      !a || !w || !c || !a_shared || !w_shared || !c_shared)
    return GLM52_EINVAL;
  if (T < 1 || T > 4 || E < 1 || topk < 1 || topk > 8 || topk > E || stride_l < E ||
      stride_w < topk || stride_i < topk || capacity < 0 || (capacity % 16))
    return GLM52_EINVAL;
  // logits rows and the bias are loaded 16 bytes per lane
  if (!al16(logits) || (stride_l % 4) || (bias && !al16(bias))) return GLM52_EINVAL;
  if (n_out <= 0 || (n_out % 16) != 0 || k <= 0 || (k % 256) != 0 || gate_up_offset < n_out)
    return GLM52_EINVAL;
  if (!al16(a) || !al16(w) || !al16(w_shared) || !al16(a_shared) || (stride_am % 8) ||
      (stride_as % 8) || (stride_we % 8) || (stride_wn % 8) || !c_ok8(c, stride_cm) ||
      !c_ok8(c_shared, stride_cs))
    return GLM52_EINVAL;
  GemmArgs g{static_cast<const uint16_t*>(a), stride_am, topk,
             static_cast<const uint16_t*>(w), stride_we, stride_wn, gate_up_offset,
             static_cast<uint16_t*>(c), stride_cm, nullptr, sorted_token_ids, expert_ids,
             num_tokens_post_padded, 16, n_out, k, T * topk, 4, 64,
             static_cast<const uint16_t*>(a_shared), stride_as,
             static_cast<const uint16_t*>(w_shared), static_cast<uint16_t*>(c_shared), stride_cs,
             T, 0, 0,
             logits, stride_l, bias, T, E, topk, norm_prob, scale, topw, stride_w, topi, stride_i,
             sorted_token_ids, expert_ids, num_tokens_post_padded, capacity};
  return launch_runs(g, capacity, true, false, true, stream);
}

// glm52_moe_gemm_route_shared on packed weights (glm52_pack_w512 of w13 for n_out gated
// outputs, and of the [1, 2 n_out, K] shared w13): the same routing, layout and bits.
extern "C" int glm52_moe_gemm_route_shared_packed(
    const float* logits, int64_t stride_l, const float* bias, int T, int E, int topk,
    float scale, int norm_prob, float* topw, int64_t stride_w, int32_t* topi, int64_t stride_i,
    int32_t* sorted_token_ids, int32_t* expert_ids, int32_t* num_tokens_post_padded,
    int capacity, const void* a, int64_t stride_am, const void* w_packed, void* c,
    int64_t stride_cm, const void* a_shared, int64_t stride_as, const void* w_shared_packed,
    void* c_shared, int64_t stride_cs, int n_out, int k, hipStream_t stream) {
  if (!logits || !topw || !topi || !sorted_token_ids || !expert_ids || !num_tokens_post_padded ||
      !a || !w_packed || !c || !a_shared || !w_shared_packed || !c_shared)
    return GLM52_EINVAL;
  if (T < 1 || T > 4 || E < 1 || topk < 1 || topk > 8 || topk > E || stride_l < E ||
      stride_w < topk || stride_i < topk || capacity < 0 || (capacity % 16))
    return GLM52_EINVAL;
  if (!al16(logits) || (stride_l % 4) || (bias && !al16(bias))) return GLM52_EINVAL;
  if (n_out <= 0 || (n_out % 256) != 0 || k <= 0 || (k % 512) != 0) return GLM52_EINVAL;
  if (!al16(a) || !al16(w_packed) || !al16(w_shared_packed) || !al16(a_shared) ||
      (stride_am % 8) || (stride_as % 8) || !c_ok8(c, stride_cm) || !c_ok8(c_shared, stride_cs))
    return GLM52_EINVAL;
  GemmArgs g{static_cast<const uint16_t*>(a), stride_am, topk,
             static_cast<const uint16_t*>(w_packed), 0, 0, n_out,
             static_cast<uint16_t*>(c), stride_cm, nullptr, sorted_token_ids, expert_ids,
             num_tokens_post_padded, 16, n_out, k, T * topk, 4, 64,
             static_cast<const uint16_t*>(a_shared), stride_as,
             static_cast<const uint16_t*>(w_shared_packed), static_cast<uint16_t*>(c_shared),
             stride_cs, T, 0, 0,
             logits, stride_l, bias, T, E, topk, norm_prob, scale, topw, stride_w, topi, stride_i,
             sorted_token_ids, expert_ids, num_tokens_post_padded, capacity};
  g.Wp = static_cast<const uint16_t*>(w_packed);
  return launch_runs(g, capacity, true, false, true, stream);
}

// Self-test of the MFMA result layouts this library assumes, for the bf16 16x16x32, the fp64
// 16x16x4 and the bf16 32x32x16 instructions.  16x16 probes: A[r][k] = r + 1 for the first 16
// k, B = identity on those k -> C[r][c] = r + 1.  Lane l supplies row / column l % 16 and k
// group l / 16; the result's register i of lane l is row 4 (l / 16) + i for bf16 and
// (l / 16) + 4 i for fp64, column l % 16 in both.  32x32 probe: A[r][0] = r, A[r][1] = 1,
// B[0][c] = 32, B[1][c] = c, so C[r][c] = 32 r + c; lane l supplies row / column l % 32 and
// the 8 k from 8 (l / 32); register i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4,
// column l % 32.  Writes 1536 floats to `out`: [0, 256) and [256, 512) the two 16 x 16
// matrices row-major (bf16, fp64 MFMA), [512, 1536) the raw 32x32 results, lane-major
// (out[512 + 16 l + i] = register i of lane l).
typedef double doublex4_t __attribute__((ext_vector_type(4)));
namespace {
__global__ void mfma_layout_probe(float* out) {
  const int lane = threadIdx.x;
  const int r = lane % 16, g = lane / 16;
  float af[8], bf[8];
  for (int j = 0; j < 8; ++j) {
    const int kk = 8 * g + j;
    af[j] = kk < 16 ? (float)(r + 1) : 0.f;
    bf[j] = (kk == r) ? 1.f : 0.f;  // B column r has a one at k == r
  }
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma16(pack8(af), pack8(bf), acc);
  for (int i = 0; i < 4; ++i) out[(4 * g + i) * 16 + r] = acc[i];
  // fp64: four k-steps of 4 cover k = 0..15; lane supplies A[r][k0 + g], B[k0 + g][r]
  doublex4_t d = {0.0, 0.0, 0.0, 0.0};
  for (int k0 = 0; k0 < 16; k0 += 4) {
    const double a = (double)(r + 1);
    const double b = (k0 + g == r) ? 1.0 : 0.0;
    d = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, d, 0, 0, 0);
  }
  // fp64 result layout: register i of lane (r, g) is row g + 4 i
  for (int i = 0; i < 4; ++i) out[256 + (g + 4 * i) * 16 + r] = (float)d[i];
  // bf16 32x32x16
  const int r32 = lane % 32, h = lane / 32;
  float a32[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, b32[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (h == 0) {
    a32[0] = (float)r32;
    a32[1] = 1.f;
    b32[0] = 32.f;
    b32[1] = (float)r32;
  }
  floatx16_t c32;
  for (int i = 0; i < 16; ++i) c32[i] = 0.f;
  c32 = mfma32(pack8(a32), pack8(b32), c32);
  for (int i = 0; i < 16; ++i) out[512 + lane * 16 + i] = c32[i];
}
}  // namespace

extern "C" int glm52_selftest_mfma_layout(float* out, hipStream_t stream) {
  if (!out) return GLM52_EINVAL;
  mfma_layout_probe<<<1, 64, 0, stream>>>(out);
  GLM52_RETURN_LAUNCH();
}
