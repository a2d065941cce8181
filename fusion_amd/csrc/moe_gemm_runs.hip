// Decode mapping of the grouped expert GEMMs (`glm52_moe_gemm` semantics, moe_gemm.hip):
// W streamed from HBM as contiguous 1 KB row runs, gfx950.
//
// At decode a layout slice holds a few real tokens, so the GEMM is a weight stream and its
// speed is the HBM read rate.  That rate depends on the access pattern: loads whose 64 lanes
// cover one contiguous 1 KB run read about 6.5 TB/s on MI355X, while loads spread over 16
// rows (64 B each) -- the layout the MFMA operand wants -- read about 4.5 TB/s.  So W is
// loaded in runs straight into LDS (`global_load_lds_dwordx4`, one 1 KB row run per
// instruction, non-temporal: W is read once) and read back from LDS in MFMA layout.
//
// Item.  One 16-row slice of the layout (an expert's block of BM = 16 slots, or 16 tokens of
// the extra expert) times 16 W rows: gated, 8 `gate` rows and the matching 8 `up` rows (8
// outputs); plain, 16 rows (16 outputs).  The four waves split K: wave w multiplies k-steps
// w*4 .. +3 of every 512-k stage with `v_mfma_f32_16x16x32_bf16` (W rows x tokens) and the
// partial sums meet in LDS in a fixed order at the item's end.
//
// Pipeline.  A stage is the 512-k run of the item's 16 W rows and its real token rows (up
// to 16; the rows of padding slots are not loaded, and whatever their LDS rows hold only
// reaches the discarded outputs of those slots).  Stages flow through a ring of four LDS
// buffers with three in flight, and the ring runs across item boundaries, so every
// workgroup streams continuously.  Each wave counts the loads it issued per stage, and a
// stage is waited for with the count of the two newer stages; stages past the workgroup's
// last one re-read its last stage into the free buffer.  Staged row R keeps global 16-byte
// chunk c at chunk c ^ (R & 15): the 16 lanes of an operand read hit 16 distinct bank
// groups.
#include "moe_gemm.h"

using namespace glm52;

namespace {

constexpr int KS = 512;            // k per stage: one 1 KB run of every staged row
constexpr int NSTAGE = 4;
constexpr int SROWS = 32;          // 16 W rows + 16 token rows
constexpr int SELEM = SROWS * KS;  // elements per stage

template <bool GATED, bool WEIGHTED>
__global__ __launch_bounds__(256) void moe_gemm_runs_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) uint16_t ring[NSTAGE * SELEM];
  __shared__ float red[4][4][kWave];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  const int r16 = lane % 16, g = lane / 16;

  constexpr int NOC = GATED ? 8 : 16;  // outputs per item
  const int num_m = *p.ntp / 16;
  const int xm = (p.x_rows + 15) / 16;
  const int num_n = p.n_out / NOC;
  const int items = (num_m + xm) * num_n;
  const int nks = p.K / KS;
  if ((int)blockIdx.x >= items) return;
  const int total = ((items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x) * nks;
  const uint32_t ring_base = lds_addr(ring);

  // ---- load side: the wave's 4 W rows and its real token rows (da_n of 4) of the item
  // being loaded -------------------------------------------------------------------------
  const uint16_t* dw[4];
  const uint16_t* da[4];
  int da_n = 0;
  auto dma_setup = [&](int it) {
    const int m = it / num_n;
    const int n0 = (it % num_n) * NOC;
    const bool extra = m >= num_m;
    const uint16_t* wbase = extra ? p.Wx : p.W + (int64_t)p.eids[m] * p.swe;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wvu * 4 + i;  // W tile row
      const int grow = GATED ? (row < 8 ? n0 + row : p.gu_off + n0 + row - 8) : n0 + row;
      dw[i] = wbase + (int64_t)grow * p.swn;
    }
    da_n = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tr = wvu * 4 + i;  // token row of the slice; real rows fill a prefix
      if (extra) {
        const int tok = (m - num_m) * 16 + tr;
        da[i] = p.Ax + (int64_t)(tok < p.x_rows ? tok : 0) * p.sax;
        da_n += tok < p.x_rows ? 1 : 0;
      } else {
        const int tok = __builtin_amdgcn_readfirstlane(p.sti[m * 16 + tr]);
        da[i] = p.A + (int64_t)(tok < p.num_valid ? tok / p.a_div : 0) * p.sam;
        da_n += tok < p.num_valid ? 1 : 0;
      }
    }
  };
  auto issue = [&](int s, int buf) {  // stage s (512-k run) of the item being loaded
    const uint32_t sb = ring_base + (uint32_t)(buf * SELEM * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int R = wvu * 4 + i;
      dma16s_nt(dw[i] + s * KS, (uint32_t)((lane ^ (R & 15)) * 16), sb + (uint32_t)(R * KS * 2));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int R = 16 + wvu * 4 + i;
      if (i < da_n)
        dma16s(da[i] + s * KS, (uint32_t)((lane ^ (R & 15)) * 16), sb + (uint32_t)(R * KS * 2));
    }
    return 4 + da_n;  // loads issued
  };
  int d_item = blockIdx.x, d_s = 0;
  auto dma_advance = [&]() {
    if (++d_s == nks) {
      d_s = 0;
      if (d_item + (int)gridDim.x < items) {
        d_item += gridDim.x;
        dma_setup(d_item);
      } else {
        d_s = nks - 1;  // past the last stage: keep re-reading the last one
      }
    }
  };

  // ---- multiply side ------------------------------------------------------------------
  auto compute = [&](int buf, floatx4_t acc) {
    const uint16_t* sb = ring + buf * SELEM;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = (wv * 4 + q) * 4 + g;  // logical 16-byte chunk of the 512-k run
      const uint4 wf = *reinterpret_cast<const uint4*>(sb + r16 * KS + ((c ^ r16) * 8));
      const uint4 af = *reinterpret_cast<const uint4*>(sb + (16 + r16) * KS + ((c ^ r16) * 8));
      acc = mfma16(wf, af, acc);  // C[W row 4 g + i][token r16]
    }
    return acc;
  };
  auto epilogue = [&](int it, floatx4_t acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wv][i][lane] = acc[i];
    __syncthreads();
    if (wv != 0) return;
    const int m = it / num_n;
    const int n0 = (it % num_n) * NOC;
    const bool extra = m >= num_m;
    int tok;
    bool ok;
    if (extra) {
      tok = (m - num_m) * 16 + r16;
      ok = tok < p.x_rows;
    } else {
      tok = p.sti[m * 16 + r16];
      ok = tok < p.num_valid;
    }
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = ((red[0][i][lane] + red[1][i][lane]) + red[2][i][lane]) + red[3][i][lane];
    if (GATED) {
      // rows 4 g + i (g < 2) are `gate` outputs 4 g + i; their `up` rows are held by lane + 32
      const int lu = (lane + 32) % kWave;
      float u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        u[i] = ((red[0][i][lu] + red[1][i][lu]) + red[2][i][lu]) + red[3][i][lu];
      if (!ok || g >= 2) return;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = silu_mul(v[i], u[i]);
    } else {
      if (!ok) return;
      if (WEIGHTED && !extra) {
        const float w = p.topw[tok];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = v[i] * w;
      }
    }
    uint16_t* dst = extra ? p.Cx + (int64_t)tok * p.scx : p.C + (int64_t)tok * p.scm;
    uint2 o;
    o.x = pack_bf16x2(v[0], v[1]);
    o.y = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<uint2*>(dst + n0 + 4 * g) = o;
  };

  // loads issued by this wave for the two stages after the one being waited for
  int n1, n2;
  dma_setup(d_item);
  issue(d_s, 0);
  dma_advance();
  n1 = issue(d_s, 1);
  dma_advance();
  n2 = issue(d_s, 2);
  dma_advance();
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
  int c_item = blockIdx.x, c_s = 0;
#pragma unroll 1
  for (int j = 0; j < total; ++j) {
    // stage j landed for this wave (stages j+1, j+2 may be in flight) and for every wave;
    // every wave is done with the buffer refilled next
    switch (n1 + n2) {
      case 8: GLM52_WAIT_VMCNT(8); break;
      case 9: GLM52_WAIT_VMCNT(9); break;
      case 10: GLM52_WAIT_VMCNT(10); break;
      case 11: GLM52_WAIT_VMCNT(11); break;
      case 12: GLM52_WAIT_VMCNT(12); break;
      case 13: GLM52_WAIT_VMCNT(13); break;
      case 14: GLM52_WAIT_VMCNT(14); break;
      case 15: GLM52_WAIT_VMCNT(15); break;
      default: GLM52_WAIT_VMCNT(16); break;
    }
    __syncthreads();
    n1 = n2;
    n2 = issue(d_s, (j + NSTAGE - 1) % NSTAGE);
    dma_advance();
    acc = compute(j % NSTAGE, acc);
    if (++c_s == nks) {
      epilogue(c_item, acc);
      acc = floatx4_t{0.f, 0.f, 0.f, 0.f};
      c_s = 0;
      c_item += gridDim.x;
    }
  }
  GLM52_WAIT_VMCNT(0);  // the re-reads past the last stage land before the workgroup ends
}

template <bool GATED, bool WEIGHTED>
int launch_runs_t(const GemmArgs& a, int capacity, hipStream_t st) {
  constexpr int NOC = GATED ? 8 : 16;
  if (a.BM != 16 || (a.n_out % NOC) || (a.K % KS) || a.K / KS < 1) return GLM52_EUNSUPPORTED;
  const int items_max = (capacity / 16 + (a.x_rows + 15) / 16) * (a.n_out / NOC);
  int grid = items_max < 256 ? items_max : 256;
  if (grid < 1) grid = 1;
  moe_gemm_runs_kernel<GATED, WEIGHTED><<<grid, 256, 0, st>>>(a);
  GLM52_RETURN_LAUNCH();
}

}  // namespace

namespace glm52 {
int launch_runs(const GemmArgs& a, int capacity, bool gated, bool weighted, hipStream_t st) {
  if (gated) return weighted ? launch_runs_t<true, true>(a, capacity, st) : launch_runs_t<true, false>(a, capacity, st);
  return weighted ? launch_runs_t<false, true>(a, capacity, st) : launch_runs_t<false, false>(a, capacity, st);
}
}  // namespace glm52
