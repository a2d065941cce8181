// LDS-tiled grouped expert GEMM for prefill (tens to thousands of rows per expert),
// gfx950.  Same semantics as the other mappings of `glm52_moe_gemm` (moe_gemm.hip):
// `moe_gateup_kernel` (`glm52/kernels/moe_gateup.py:34-148`) when gated and
// `moe_down_kernel` with MUL_ROUTED_WEIGHT (`glm52/kernels/moe_down_merge.py:66-169`) when
// weighted.
//
// Tile.  A workgroup owns one layout block of MT rows (tokens) of one expert and 256 rows
// of that expert's W:
//   gated: 128 `gate` rows n0 .. n0+127 and the matching 128 `up` rows -> 128 outputs;
//   plain: 256 rows n0 .. n0+255 -> 256 outputs.
// Four waves split the tile 2 x 2: wave (wn, wm) computes 128 W rows x MT/2 tokens with
// `v_mfma_f32_16x16x32_bf16`, W as the MFMA's first operand and the token rows as its
// second, so that a lane's four results of one 16 x 16 block are four consecutive output
// columns of one token.
//
// Output stores.  Inside each 32-row group of the W tile, LDS row 16 h + 4 g + i holds W
// row 8 g + 4 h + i (h < 2, g < 4, i < 4).  Then lane (g, c) holds, in the blocks h = 0
// and h = 1 of a group, the eight consecutive outputs 8 g .. 8 g + 7 of token c, which it
// writes with one 16-byte store.  A gated tile keeps `gate` row n and `up` row n in the
// same lane and register, so SwiGLU is applied in registers.
//
// Padding.  Real tokens fill a prefix of every layout block; 16-token groups past it are
// neither multiplied nor stored (their A rows re-read the block's first real row).
//
// Order.  The kernel is persistent (one workgroup per CU).  Workgroup ids congruent
// modulo 8 run on one XCD; each XCD takes a contiguous range of items, and the items of
// one expert are laid out column tile major, row block fastest, so all row blocks of the
// expert run against one W tile at the same time on one XCD: the tile is fetched from HBM
// once and served to the others from the XCD's L2.
#include "moe_gemm.h"

#include <atomic>
#include <type_traits>

using namespace glm52;

namespace {

constexpr int NT = 256;   // W rows per tile
constexpr int BK = 64;    // k per LDS stage
constexpr int LDK = BK + 8;
constexpr int CPR = BK / 8;  // 16-byte chunks per staged row

// LDS row of W row `n` (0 <= n < 32) inside its 32-row group.
GLM52_DEV int perm32(int n) { return ((n >> 2) & 1) * 16 + (n >> 3) * 4 + (n & 3); }

// ------------------------------------------------------------------------------------
// The same tile fed by direct global -> LDS loads (`global_load_lds_dwordx4`) through a
// ring of LDS stages (BK = 64: three stages of 64 k, two in flight while one is
// multiplied; BK = 32: four stages of 32 k, three in flight).  No staging registers are
// needed.  A staged row is BK bf16 (CPR 16-byte chunks); chunk c of row r is stored at
// chunk c ^ ((r >> SW) & (CPR - 1)) with SW = log2(16 / CPR), so the 16 lanes of one
// 128-bit operand read touch 16 distinct bank groups.  A wave's load instruction fills
// 1 KB of LDS (64 / CPR rows) in lane order, so each lane fetches the global chunk that
// belongs at its slot; with BK = 64 a W row is fetched 128 B at a time.
// ------------------------------------------------------------------------------------
// W row (0 <= n < 32) stored at LDS row perm32(n) of its group; the inverse.
GLM52_DEV int iperm32(int r) { return ((r >> 2) & 3) * 8 + ((r >> 4) & 1) * 4 + (r & 3); }

template <int MT, int BKS, bool GATED, bool WEIGHTED>
__global__ __launch_bounds__(256) void moe_gemm_dma_kernel(GemmArgs p) {
  constexpr int NSTAGE = BKS == 64 ? 3 : 4;
  constexpr int LATER = NSTAGE - 2;  // stages still in flight while one is multiplied
  constexpr int CPR_S = BKS / 8;     // chunks per staged row
  constexpr int SW = CPR_S == 8 ? 1 : 2;
  constexpr int RPI = 64 / CPR_S;    // rows per load instruction
  constexpr int TT = MT / 2;
  constexpr int TF = TT / 16;
  constexpr int NO = GATED ? NT / 2 : NT;
  constexpr int WI = NT / RPI / 4;   // W load instructions per wave per stage
  constexpr int AI = MT / RPI / 4;   // A load instructions per wave per stage
  constexpr int IPS = WI + AI;
  constexpr int SROWS = NT + MT;
  static_assert(TF >= 1 && AI >= 1, "tile");
  static_assert(LATER * IPS < 64, "vmcnt range");

  // one array per stage ([W rows | A rows])
  __shared__ __attribute__((aligned(1024))) uint16_t S0[SROWS * BKS];
  __shared__ __attribute__((aligned(1024))) uint16_t S1[SROWS * BKS];
  __shared__ __attribute__((aligned(1024))) uint16_t S2[SROWS * BKS];
  __shared__ __attribute__((aligned(1024))) uint16_t S3[NSTAGE == 4 ? SROWS * BKS : 8];
  __shared__ int toks[MT];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  const int wn = wv & 1, wm = wv >> 1;
  const int l16 = lane % 16, lg = lane / 16;

  const int ntp = *p.ntp;
  const int num_m = ntp / MT;
  const int num_n = p.n_out / NO;
  const int items = num_m * num_n;
  const int nk = p.K / BKS;
  const int per_xcd = (items + 7) / 8;
  const int span = per_xcd * 8;

  // operand reads: lane (l16, lg) reads logical chunk 4 ks + lg of row base + l16
  int rd_off[BKS / 32];
#pragma unroll
  for (int ks = 0; ks < BKS / 32; ++ks)
    rd_off[ks] = l16 * BKS + (((ks * 4 + lg) ^ ((l16 >> SW) & (CPR_S - 1))) * 8);
  int frow[8];
#pragma unroll
  for (int f = 0; f < 8; ++f)
    frow[f] = GATED ? ((f < 4) ? wn * 64 + f * 16 : 128 + wn * 64 + (f - 4) * 16)
                    : wn * 128 + f * 16;

  // load slots: lane -> row lane / CPR of the instruction's slab, physical chunk lane % CPR
  const int dr = lane / CPR_S;
  const int dpc = lane % CPR_S;

  for (int it = blockIdx.x; it < span; it += gridDim.x) {
    const int L = (it % 8) * per_xcd + it / 8;
    if (L >= items) continue;
    // Expert-aligned order: the items of expert e are [mb * num_n, (mb + cnt) * num_n)
    // for its row blocks mb .. mb + cnt - 1, column tile major and row block fastest, so
    // every row block of the expert runs against a W tile at the same time.
    const int b = L / num_n;
    const int eb = p.eids[b];
    int mb = b, me = b + 1;
    while (mb > 0 && p.eids[mb - 1] == eb) --mb;
    while (me < num_m && p.eids[me] == eb) ++me;
    const int cnt = me - mb;
    const int local = L - mb * num_n;
    const int pid_n = local / cnt;
    const int pid_m = mb + local % cnt;
    const int row0 = pid_m * MT;
    if (p.sti[row0] >= p.num_valid) continue;
    const int e = p.eids[pid_m];
    const int n0 = pid_n * NO;

    for (int q = tid; q < MT; q += 256) toks[q] = p.sti[row0 + q];
    __syncthreads();
    const int nv_rows = __builtin_amdgcn_readfirstlane(
        __syncthreads_count(tid < MT && toks[tid] < p.num_valid));
    const int nvf = __builtin_amdgcn_readfirstlane(max(0, min(TF, (nv_rows - wm * TT + 15) / 16)));

    const uint16_t* wsrc[WI];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int rl = wv * (NT / 4) + i * RPI + dr;  // LDS row of the W tile
      const int c = dpc ^ ((rl >> SW) & (CPR_S - 1));
      int grow;
      if (GATED) {
        const int half = rl >> 7, within = rl & 127;
        grow = (half ? p.gu_off : 0) + n0 + (within & ~31) + iperm32(within & 31);
      } else {
        grow = n0 + (rl & ~31) + iperm32(rl & 31);
      }
      wsrc[i] = p.W + (int64_t)e * p.swe + (int64_t)grow * p.swn + c * 8;
    }
    int asrc[AI];  // 32-bit element offsets into A (A holds < 2^31 elements)
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const int rl = wv * (MT / 4) + i * RPI + dr;
      const int c = dpc ^ ((rl >> SW) & (CPR_S - 1));
      asrc[i] = (toks[rl < nv_rows ? rl : 0] / p.a_div) * (int)p.sam + c * 8;
    }

    auto issue = [&](int kt, uint16_t* sbuf) {
      const uint32_t wb = lds_addr(sbuf) + (uint32_t)(wvu * (NT / 4) * BKS * 2);
      const uint32_t ab = lds_addr(sbuf + NT * BKS) + (uint32_t)(wvu * (MT / 4) * BKS * 2);
      const int koff = kt * BKS;
#pragma unroll
      for (int i = 0; i < WI; ++i) dma16(wsrc[i] + koff, wb + i * 1024);
#pragma unroll
      for (int i = 0; i < AI; ++i) dma16(p.A + asrc[i] + koff, ab + i * 1024);
    };

    floatx4_t acc[8][TF];
#pragma unroll
    for (int f = 0; f < 8; ++f)
#pragma unroll
      for (int t = 0; t < TF; ++t) acc[f][t] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const uint16_t* sbuf) {
      const uint16_t* abuf = sbuf + NT * BKS;
#pragma unroll
      for (int ks = 0; ks < BKS / 32; ++ks) {
        uint4 wf[8];
#pragma unroll
        for (int f = 0; f < 8; ++f)
          wf[f] = *reinterpret_cast<const uint4*>(sbuf + frow[f] * BKS + rd_off[ks]);
#pragma unroll
        for (int t = 0; t < TF; ++t) {
          if (t < nvf) {
            const uint4 af = *reinterpret_cast<const uint4*>(abuf + (wm * TT + t * 16) * BKS + rd_off[ks]);
#pragma unroll
            for (int f = 0; f < 8; ++f) acc[f][t] = mfma16(wf[f], af, acc[f][t]);
          }
        }
      }
    };

    // prologue: stages 0 .. NSTAGE - 2 in flight
    issue(0, S0);
    if (nk > 1) issue(1, S1);
    if (NSTAGE == 4 && nk > 2) issue(2, S2);
    for (int k0 = 0; k0 < nk; k0 += NSTAGE) {
#pragma unroll
      for (int j = 0; j < NSTAGE; ++j) {
        const int kt = k0 + j;
        if (kt < nk) {
          // stage kt landed (at most LATER later stages still in flight), for all waves
          const int later = min(LATER, nk - 1 - kt);
          if (later >= 2) GLM52_WAIT_VMCNT(2 * IPS);
          else if (later == 1) GLM52_WAIT_VMCNT(IPS);
          else GLM52_WAIT_VMCNT(0);
          __syncthreads();
          // refill the buffer every wave finished reading before this barrier
          const int nx = kt + NSTAGE - 1;
          if (nx < nk) {
            const int b = (j + NSTAGE - 1) % NSTAGE;
            if (b == 0) issue(nx, S0);
            if (b == 1) issue(nx, S1);
            if (b == 2) issue(nx, S2);
            if (NSTAGE == 4 && b == 3) issue(nx, S3);
          }
          if (j == 0) compute(S0);
          if (j == 1) compute(S1);
          if (j == 2) compute(S2);
          if (NSTAGE == 4 && j == 3) compute(S3);
        }
      }
    }

#pragma unroll
    for (int t = 0; t < TF; ++t) {
      if (t >= nvf) continue;
      const int tl = wm * TT + t * 16 + l16;
      const int tok = toks[tl];
      if (tok >= p.num_valid) continue;
      float wgt = 1.f;
      if (WEIGHTED) wgt = p.topw[tok];
      uint16_t* crow = p.C + (int64_t)tok * p.scm;
      if (GATED) {
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          float v[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[i] = silu_mul(acc[2 * pr][t][i], acc[4 + 2 * pr][t][i]);
            v[4 + i] = silu_mul(acc[2 * pr + 1][t][i], acc[5 + 2 * pr][t][i]);
          }
          *reinterpret_cast<uint4*>(crow + n0 + (wn * 2 + pr) * 32 + lg * 8) = pack8(v);
        }
      } else {
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          float v[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[i] = acc[2 * pr][t][i];
            v[4 + i] = acc[2 * pr + 1][t][i];
          }
          if (WEIGHTED) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = v[i] * wgt;
          }
          *reinterpret_cast<uint4*>(crow + n0 + (wn * 4 + pr) * 32 + lg * 8) = pack8(v);
        }
      }
    }
    __syncthreads();  // toks and the ring are reused by the next item
  }
}

template <int MT, int BKS, bool GATED, bool WEIGHTED>
int launch_dma(const GemmArgs& a, int capacity, hipStream_t st) {
  constexpr int NO = GATED ? NT / 2 : NT;
  if ((a.n_out % NO) || (a.K % BKS)) return GLM52_EUNSUPPORTED;
  const int items_max = (capacity / MT) * (a.n_out / NO);
  int grid = items_max < 256 ? items_max : 256;
  grid = ((grid + 7) / 8) * 8;
  moe_gemm_dma_kernel<MT, BKS, GATED, WEIGHTED><<<grid, 256, 0, st>>>(a);
  GLM52_RETURN_LAUNCH();
}

template <bool GATED, bool WEIGHTED>
int launch_bm(const GemmArgs& a, int capacity, hipStream_t st) {
  // a three-buffer ring of 64-k stages
  if (a.stage_k != 64) return GLM52_EUNSUPPORTED;
  switch (a.BM) {
    case 64: return launch_dma<64, 64, GATED, WEIGHTED>(a, capacity, st);
    case 128: return launch_dma<128, 64, GATED, WEIGHTED>(a, capacity, st);
    default: return GLM52_EUNSUPPORTED;
  }
}

}  // namespace

namespace glm52 {
int launch_wide(const GemmArgs& a, int capacity, bool gated, bool weighted, hipStream_t st) {
  if (gated) return weighted ? launch_bm<true, true>(a, capacity, st) : launch_bm<true, false>(a, capacity, st);
  return weighted ? launch_bm<false, true>(a, capacity, st) : launch_bm<false, false>(a, capacity, st);
}
}  // namespace glm52

// ------------------------------------------------------------------------------------
// 512-row W tiles on the 32x32x16 MFMA.  A workgroup owns MT tokens (one layout block) x 512
// rows of W[e]; wave w computes the W rows w*128 .. +127 (gated: 64 `gate` rows and the
// matching 64 `up` rows) against all MT tokens: a 128 x MT wave tile of 4 x MT/32 blocks of
// 32 x 32, W as the first MFMA operand.  All four waves share the staged token rows.
//
// Pipeline.  K advances in 32-k stages through a ring of four LDS buffers filled by direct
// global -> LDS loads.  While the MFMAs of stage kt run on fragments already in registers,
// the same instruction stream reads the fragments of stage kt+1 from LDS and issues the
// loads of stage kt+3; the three kinds are interleaved in a fixed order (scheduling
// barriers pin it), so neither the LDS reads nor the load issue stall the matrix core.
// Loads past the last stage re-read the last stage into the free buffer, so every stage
// has the same shape and the waits are the same constant.  Staged row r keeps its 16-byte
// chunk c at c ^ ((r >> 2) & 3): the 16 lanes served together read 16 distinct bank groups.
//
// Output.  Inside each 32-row group of the W tile, LDS row p holds W row
// ((p >> 2) & 1) * 16 + (p >> 3) * 4 + (p & 3); a lane's 16 results of a 32 x 32 block are
// then 16 consecutive outputs of one token, written with two 16-byte stores.  A gated tile
// pairs `gate` row n and `up` row n in the same lane and register, so SwiGLU runs in
// registers.  The tokens and routing weights of an item's rows are loaded once, before
// its first store, and kept in the ring buffer the last stage has freed.
//
// Registers.  The kernel holds 256 accumulators and the fragments of two stages: near the
// 512-register limit, a value the compiler hoists out of the item loop to keep live across
// it (the lane's load offsets, the ring's addresses) is spilled, and its reload waits for
// every load in flight.  Such values are formed per item from opaque copies of the lane
// index and the ring's address.
// ------------------------------------------------------------------------------------
namespace {

// Packed W (PACKED): expert e's 512-row tiles P follow each other; inside a tile its 32 load
// slots (slot w * 8 + i: what load instruction i of wave w fetches), nk stages of 1 KB each,
// lane l's 16 bytes at l * 16: exactly what the instruction writes to LDS.  The slots are
// interleaved a stage at a time in groups of 8 (packed_slot_off): every load reads 1 KB of
// contiguous memory, a stage of the tile is four 8 KB runs, and the decode weight stream
// (one slot per item) reads a slot's stages 8 KB apart.

// W row (relative to the tile's first `gate` row, or to n0) and k chunk of packed lane l of
// load instruction i of wave w: the row and chunk the unpacked loads of that slot fetch.
GLM52_DEV int w512_row(bool gated, int gu_rel, int w, int i, int l) {
  const int f = i >> 1;
  const int base = gated ? (f >= 2 ? gu_rel : 0) + w * 64 + (f & 1) * 32 : w * 128 + f * 32;
  return base + (i & 1) * 8 + phi32(l >> 2);
}
GLM52_DEV int w512_chunk(int l) { return (l & 3) ^ (((l >> 2) >> 2) & 3); }

// EPI (non-gated): 0 bf16 store; 1 bf16(acc + R); 2 C32 += acc (+ R); 3 C32 = acc (fp32
// partials); 4 the atomic expert merge, bf16 packed atomic adds into row tok / merge_topk.
//
// NTW = 512: the tile above (4 waves along W, each 128 W rows x all MT tokens).
// NTW = 256 (MT = 256): a 256-token x 256-row tile, the waves 2 x 2 (wave (wn, wm): W rows
// wn * 128 .. +127 against tokens wm * 128 .. +127).  Its W tile is half of a 512-row tile
// -- gated: `gate` and `up` rows of 128 consecutive outputs -- which the packed layout
// keeps as 16 KB of contiguous memory per stage (512-row waves 2s and 2s + 1), so both
// tile heights read one packed copy.  A stage is 32 KB, so five fit in LDS: four in flight
// while one is multiplied.  A tile of 256 tokens covers most experts' rows at prefill
// sizes in one item, so most W tiles are streamed by one workgroup only.
//
// Dealing.  Each XCD owns a contiguous share of the items (its routed items, then its
// share of the extra expert's), so the W tiles and token rows its workgroups share stay in
// its L2.  A workgroup (XCD blockIdx.x % 8) takes its first item by its index and each
// next one from its XCD's counter, fetched while the current item runs; once its XCD's
// items are all taken it takes those of the next XCDs.  The items differ in cost (L2
// hits, non-temporal tiles, real rows), so a fixed round-robin deal left the workgroups of
// one XCD finishing hundreds of microseconds apart.  Every item writes its own outputs:
// the results do not depend on which workgroup runs it.  The counters of one launch are a
// set of kDealSets; the launcher gives consecutive launches consecutive sets, and the
// last workgroup out clears its set, so launches that overlap on one GPU use different
// sets unless kDealSets launches apart (a captured graph keeps the set it was captured
// with: replays of one graph must not overlap).
constexpr int kDealSets = 64;
constexpr int kDealStride = 256;  // ints per set: XCD x's counter at 16 x, the exits at 128
__device__ __align__(256) int g_w512_deal[kDealSets * kDealStride];

// The host side of glm52_debug_item_trace: the record the next launches write, or null.
std::atomic<unsigned long long*> g_item_trace{nullptr};

template <int MT, int NTW, bool GATED, bool WEIGHTED, bool PACKED, int EPI = 0>
__global__ __launch_bounds__(256) void moe_gemm_w512_kernel(GemmArgs p) {
  const unsigned long long t_start = p.wg_trace ? __builtin_amdgcn_s_memrealtime() : 0ull;
  int n_run = 0;  // items this workgroup ran (the trace record)
  constexpr int BKS = 32;          // k per stage
  constexpr int WN = NTW / 128;    // waves along W
  constexpr int WM = 4 / WN;       // waves along the tokens
  constexpr int TPW = MT / WM;     // tokens per wave
  constexpr int RPI = 16;          // staged rows per load instruction (64 lanes x 16 B / 64 B)
  constexpr int TF = TPW / 32;     // token blocks of 32 per wave
  constexpr int NO = GATED ? NTW / 2 : NTW;
  constexpr int NO512 = GATED ? 256 : 512;  // outputs of a packed 512-row tile
  constexpr int SPLIT = 512 / NTW;          // W tiles per packed 512-row tile
  constexpr int WI = NTW / RPI / 4;  // W load instructions per wave and stage
  constexpr int AI = MT / RPI / 4;   // token-row load instructions per wave and stage
  constexpr int IPS = WI + AI;
  constexpr int SROWS = NTW + MT;
  constexpr int SELEM = SROWS * BKS;  // elements per stage
  constexpr int NSTAGE = 5 * SELEM * 2 <= 163840 ? 5 : 4;
  static_assert(WN * WM == 4 && AI >= 1 && TF >= 1 && TF <= 4, "tile");
  static_assert((NSTAGE - 2) * IPS < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) uint16_t ring[NSTAGE * SELEM];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  const int wn = wvu % WN, wm = wvu / WN;
  const int l32 = lane % 32, h = lane / 32;

  const int ntp = *p.ntp;
  const int num_m = ntp / MT;
  const int num_n = p.n_out / NO;
  const int num_n512 = p.n_out / NO512;
  const int items = num_m * num_n;
  const int nk = p.K / BKS;
  const int per_xcd = (items + 7) / 8;
  // the extra (shared) expert, packed weights only: rows are tokens 0 .. x_rows - 1 of Ax,
  // its row blocks' items follow each XCD's share of the routed items
  const bool has_x = PACKED && EPI == 0 && p.Wx && p.x_rows > 0;
  const int nbx = has_x ? (p.x_rows + MT - 1) / MT : 0;
  const int items_x = nbx * num_n;
  const int per_xcd_x = (items_x + 7) / 8;
  int* const deal = g_w512_deal + p.deal_set * kDealStride;
  const int wg_xcd = gridDim.x / 8;  // workgroups per XCD (the launcher rounds to 8)
  int xcd = blockIdx.x % 8;  // the XCD whose items this workgroup takes: its own first
  int tried = 1;

  // fragment reads: lane (l32, h) reads logical chunk 2 ks + h of row base + l32 (base % 32 == 0)
  const int rd0 = l32 * BKS + (((0 + h) ^ ((l32 >> 2) & 3)) * 8);
  const int rd1 = l32 * BKS + (((2 + h) ^ ((l32 >> 2) & 3)) * 8);
  const uint32_t ring_base = lds_addr(ring);
  // the next item's index passes from wave 0 to the others through the first word of the
  // ring buffer of the last stage: no load issued past the last stage lands there, and
  // every wave has read that stage's fragments before the stage's barrier
  int* const slot = reinterpret_cast<int*>(ring + ((nk - 1) % NSTAGE) * SELEM);
  auto fetch_now = [&]() {  // the next index of XCD xcd's items, for the whole workgroup
    if (tid == 0)
      *slot = __hip_atomic_fetch_add(deal + xcd * 16, 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int k = __builtin_amdgcn_readfirstlane(wg_xcd + *slot);
    __syncthreads();  // every wave has it before the slot is written again
    return k;
  };

  for (int k = blockIdx.x / 8;;) {
    // item k of XCD xcd: its routed items first (L = xcd * per_xcd + k), then the extra
    // expert's (Lx = xcd * per_xcd_x + k - n_r)
    const int n_r = max(0, min(per_xcd, items - xcd * per_xcd));
    const int n_local = n_r + max(0, min(per_xcd_x, items_x - xcd * per_xcd_x));
    if (k >= n_local) {  // that XCD's items are all taken: take the next XCD's
      if (tried == 8) break;
      ++tried;
      xcd = (xcd + 1) % 8;
      k = fetch_now();
      continue;
    }
    const bool xs = k >= n_r;
    int pid_n, row0, e;
    bool w_once;  // the W tile is streamed by this item only: non-temporal loads
    if (!xs) {
      const int L = xcd * per_xcd + k;
      // expert-aligned order (as moe_gemm_dma_kernel): column tile major, row block fastest
      const int b = L / num_n;
      const int eb = p.eids[b];
      int mb = b, me = b + 1;
      while (mb > 0 && p.eids[mb - 1] == eb) --mb;
      while (me < num_m && p.eids[me] == eb) ++me;
      const int cnt = me - mb;
      w_once = cnt == 1;
      const int local = L - mb * num_n;
      pid_n = local / cnt;
      const int pid_m = mb + local % cnt;
      row0 = pid_m * MT;
      if (p.sti[row0] >= p.num_valid) {  // a block with no real row: nothing to compute
        k = fetch_now();
        continue;
      }
      e = eb;  // the blocks mb .. me - 1 all hold expert eb
    } else {
      const int Lx = xcd * per_xcd_x + (k - n_r);
      pid_n = Lx / nbx;
      row0 = (Lx % nbx) * MT;
      e = 0;
      w_once = nbx == 1;
    }
    ++n_run;
    const int n0 = pid_n * NO;
    const int P = pid_n / SPLIT, sub = pid_n % SPLIT;  // the packed 512-row tile and half
    // The item's first stage (its stages run from there, wrapping), in the 512-row tiles of
    // the expert GEMMs (the 64- and 128-token tiles; o_proj's epilogues keep stage 0).  There most W tiles are streamed by
    // one item, the workgroups advance in step, and with every item at the same stage the
    // loads in flight sit a multiple of 2 MB apart; starting each expert's tiles 16 stages
    // apart spreads them over the HBM channels (T = 2048: w13 2275 -> 2164 us, w2 1340 ->
    // 1315 us).  The 256 x 256 tiles keep stage 0 first: there many row blocks share each
    // W tile through L2 and the same start ran w13 4058 -> 4127 us at T = 8192.  The start
    // depends on the expert and the 512-row tile only, so packed and in-place W, one launch
    // or separate ones, and the atomic merge (EPI 4) add an output's stages in one order.
    const int krot = (NTW == 512 && (EPI == 0 || EPI == 4))
                         ? (((xs ? 0 : e) * num_n512 + P) * 16) % nk
                         : 0;
    // the item's operands: the routed rows through the layout, the extra expert's directly
    const uint16_t* Ab = xs ? p.Ax : p.A;
    const int64_t sam = xs ? p.sax : p.sam;
    const int a_div = xs ? 1 : p.a_div;
    const int nvalid = xs ? p.x_rows : p.num_valid;
    auto tok_of = [&](int r) {  // the flat token of row r of the item (>= nvalid: padding)
      return xs ? (row0 + r < p.x_rows ? row0 + r : p.x_rows) : p.sti[row0 + r];
    };

    // The lane index through an opaque copy: the lane's offsets below are computed here, per
    // item, rather than hoisted out of the item loop to stay live (and be spilled) across it.
    int il = lane;
    asm volatile("" : "+v"(il));
    // load slots: lane -> row il / 4 of the instruction's 16-row slab, physical chunk il % 4
    const int dr = il >> 2;
    const int dc = (il & 3) ^ ((dr >> 2) & 3);  // the logical chunk that lands in that slot
    // the ring's address likewise: the prologue's LDS addresses (m0) are then formed per
    // item, not precomputed once and held across the item loop
    uint32_t rb = ring_base;
    asm volatile("" : "+s"(rb));

    // the tokens of the lane's staged rows, loaded beside the real-row count below (a row
    // past the real ones then re-reads the block's first row)
    int trl[AI];
#pragma unroll
    for (int i = 0; i < AI; ++i) trl[i] = tok_of(wv * (MT / 4) + i * RPI + dr);
    const int tr0 = tok_of(0);
    // real tokens fill a prefix of the block: every wave counts them (no LDS, no barrier)
    int nv_rows = 0;
#pragma unroll
    for (int q = 0; q < MT; q += kWave)
      nv_rows += __popcll(__ballot(q + il < MT && tok_of(q + il) < nvalid));
    nv_rows = __builtin_amdgcn_readfirstlane(nv_rows);
    const int nvf = __builtin_amdgcn_readfirstlane(max(0, min(TF, (nv_rows - wm * TPW + 31) / 32)));

    // W load instruction i of the wave fills slab rows (wv * WI + i) * 16 .. +15 of the
    // tile: packed, 1 KB of contiguous memory; in place, W rows wrow + phi32(lane / 4), 16
    // bytes at logical chunk dc each (the lane's byte offsets inside W[e], < 2^32)
    const uint16_t* wexp = PACKED ? (xs ? p.Wx : p.Wp) +
                                        (int64_t)(e * num_n512 + P) * packed_tile_elems(nk)
                                  : p.W + (int64_t)e * p.swe;
    uint32_t wvoff[WI];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      if (PACKED) {
        // load slot sub * 32 / SPLIT + wv * WI + i of the 512-row tile: nk KB per slot
        wvoff[i] = (uint32_t)(packed_slot_off(nk, sub * (32 / SPLIT) + wv * WI + i) * 2 +
                              il * 16);
      } else {
        const int slab = sub * (NTW / RPI) + wv * WI + i;  // 1 KB slab of the 512-row tile
        const int row = P * NO512 + w512_row(GATED, p.gu_off, slab / 8, slab % 8, il);
        wvoff[i] = (uint32_t)(((int64_t)row * p.swn + dc * 8) * 2);
      }
    }
    uint32_t avoff[AI];  // byte offsets of the lane's token rows in A (< 2^31, checked)
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const int rl = wv * (MT / 4) + i * RPI + dr;
      avoff[i] = (uint32_t)(((rl < nv_rows ? trl[i] : tr0) / a_div) * (int)sam + dc * 8) * 2u;
    }

    // the previous item's output stores and loads are done before this item's are counted
    GLM52_WAIT_VMCNT(0);
    // Past the last stage the loads keep their count (the waits stay constant) but every
    // lane reads the same 16 bytes, one cache line per instruction, into the free buffer.
    auto issue_one = [&](int i, int kt) {  // load instruction i of stage kt (clamped)
      const bool past = kt >= nk;  // wave-uniform
      int kr = min(kt, nk - 1) + krot;  // the stage loaded, from the item's first
      if (kr >= nk) kr -= nk;
      const int kc = kr * BKS;
      const uint32_t sb = rb + (uint32_t)((kt % NSTAGE) * SELEM * 2);
      if (i < WI) {
        const uint16_t* src = PACKED ? wexp + (int64_t)kr * kPackStride : wexp + kc;
        const uint32_t vo = past ? 0u : wvoff[i];
        if (w_once)
          dma16s_nt(src, vo, sb + (uint32_t)((wvu * WI + i) * RPI * BKS * 2));
        else
          dma16s(src, vo, sb + (uint32_t)((wvu * WI + i) * RPI * BKS * 2));
      } else {
        const int j = i - WI;
        dma16s(Ab + kc, past ? 0u : avoff[j], sb + (uint32_t)((NTW + wvu * (MT / 4) + j * RPI) * BKS * 2));
      }
    };

    auto run = [&](auto nv_tag) {
      constexpr int NV = decltype(nv_tag)::value;
      if constexpr (NV == 0) {
        // no real token in this wave's rows: it still stages its share of every stage
#pragma unroll
        for (int st = 0; st < NSTAGE - 1; ++st)
#pragma unroll
          for (int i = 0; i < IPS; ++i) issue_one(i, st);
        GLM52_WAIT_VMCNT((NSTAGE - 2) * IPS);
        __syncthreads();
#pragma unroll 1
        for (int kt = 0; kt < nk; ++kt) {
          GLM52_WAIT_VMCNT((NSTAGE - 3) * IPS);
          __syncthreads();
#pragma unroll
          for (int i = 0; i < IPS; ++i) issue_one(i, kt + NSTAGE - 1);
        }
        return;
      } else {
      constexpr int NMF = 8 * NV;           // MFMAs per stage
      constexpr int NRD = 8 + 2 * NV;       // fragment reads per stage
      constexpr int NOPS = NRD + IPS;       // reads and loads spread over the MFMAs
      floatx16_t acc[4][NV];
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int t = 0; t < NV; ++t)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[f][t][i] = 0.f;
      // fragments of two stages: [parity][k step][block]
      uint4 fw[2][2][4], fa[2][2][NV];

      auto read_op = [&](int q, const uint16_t* sb, uint4 (&dw)[2][4], uint4 (&da)[2][NV]) {
        if (q < 8) {
          const int ks = q / 4, f = q % 4;
          dw[ks][f] = *reinterpret_cast<const uint4*>(sb + (wn * 128 + f * 32) * BKS + (ks ? rd1 : rd0));
        } else {
          const int ks = (q - 8) / NV, t = (q - 8) % NV;
          da[ks][t] = *reinterpret_cast<const uint4*>(sb + (NTW + wm * TPW + t * 32) * BKS + (ks ? rd1 : rd0));
        }
      };

      // one stage: the MFMAs of stage kt on fragments [P], interleaved with the reads of
      // stage kt+1 into fragments [1-P] and the loads of stage kt+NSTAGE-1
      auto stage = [&](int kt, auto par_tag) {
        constexpr int PAR = decltype(par_tag)::value;
        // stage kt+1 landed for this wave (later stages may still be in flight) and for
        // every wave; every wave is done with the buffer refilled in this stage
        GLM52_WAIT_VMCNT((NSTAGE - 3) * IPS);
        __syncthreads();
        const uint16_t* sbn = ring + ((kt + 1) % NSTAGE) * SELEM;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < NMF; ++m) {
          const int ks = m / (4 * NV), f = (m / NV) % 4, t = m % NV;
          acc[f][t] = mfma32(fw[PAR][ks][f], fa[PAR][ks][t], acc[f][t]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int o = 0; o < NOPS; ++o) {
            if ((o * NMF) / NOPS == m) {  // op o goes after MFMA m
              // alternate loads and reads while both remain
              constexpr int both = 2 * (IPS < NRD ? IPS : NRD);
              const bool is_load = o < both ? (o % 2) == 0 : IPS > NRD;
              const int idx = o < both ? o / 2 : both / 2 + (o - both);
              if (is_load) issue_one(idx, kt + NSTAGE - 1);
              else read_op(idx, sbn, fw[1 - PAR], fa[1 - PAR]);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
      };

      // prologue: stages 0 .. NSTAGE-2 in flight; stage 0 landed everywhere; its fragments read
#pragma unroll
      for (int st = 0; st < NSTAGE - 1; ++st)
#pragma unroll
        for (int i = 0; i < IPS; ++i) issue_one(i, st);
      GLM52_WAIT_VMCNT((NSTAGE - 2) * IPS);
      __syncthreads();
#pragma unroll
      for (int q = 0; q < NRD; ++q) read_op(q, ring, fw[0], fa[0]);

#pragma unroll 1
      for (int kt = 0; kt < nk; kt += 2) {  // nk is even (the launcher checks K % 64)
        stage(kt, std::integral_constant<int, 0>{});
        stage(kt + 1, std::integral_constant<int, 1>{});
      }

      if constexpr (EPI == 0) {
        // The lane index through an opaque copy, as in the item's set-up; the tokens and
        // routing weights of the wave's rows are loaded together, before any store, into the
        // ring buffer of stage nk - 1 (free here: every wave has read its fragments, no load
        // past the last stage lands in it) and read back per 32-row block.  vmcnt also
        // counts stores, so a token loaded after a block's stores would wait for them.
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int el32 = ln % 32, eh = ln / 32;
        int* const etok =
            reinterpret_cast<int*>(ring + ((nk - 1) % NSTAGE) * SELEM) + wvu * 2 * TPW;
        float* const ewgt = reinterpret_cast<float*>(etok + TPW);
        static_assert(TPW % 64 == 0 && 4 * 2 * TPW * 4 <= SELEM * 2, "epilogue rows");
        {
          int qt[TPW / 64];
#pragma unroll
          for (int j = 0; j < TPW / 64; ++j) qt[j] = tok_of(wm * TPW + j * 64 + ln);
#pragma unroll
          for (int j = 0; j < TPW / 64; ++j) {
            etok[j * 64 + ln] = qt[j];
            if (WEIGHTED) ewgt[j * 64 + ln] = (!xs && qt[j] < nvalid) ? p.topw[qt[j]] : 1.f;
          }
        }
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          const int tok = etok[t * 32 + el32];
          if (tok >= nvalid) continue;
          uint16_t* const crow = xs ? p.Cx + (int64_t)tok * p.scx : p.C + (int64_t)tok * p.scm;
          if (GATED) {
#pragma unroll
            for (int fp = 0; fp < 2; ++fp) {
              float v[16];
#pragma unroll
              for (int i = 0; i < 16; ++i) v[i] = silu_mul(acc[fp][t][i], acc[fp + 2][t][i]);
              uint16_t* dst = crow + n0 + wn * 64 + fp * 32 + eh * 16;
              *reinterpret_cast<uint4*>(dst) = pack8(v);
              *reinterpret_cast<uint4*>(dst + 8) = pack8(v + 8);
            }
          } else {
            const float wgt = WEIGHTED ? ewgt[t * 32 + el32] : 1.f;
#pragma unroll
            for (int f = 0; f < 4; ++f) {
              float v[16];
#pragma unroll
              for (int i = 0; i < 16; ++i) v[i] = WEIGHTED ? acc[f][t][i] * wgt : acc[f][t][i];
              uint16_t* dst = crow + n0 + wn * 128 + f * 32 + eh * 16;
              *reinterpret_cast<uint4*>(dst) = pack8(v);
              *reinterpret_cast<uint4*>(dst + 8) = pack8(v + 8);
            }
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < NV; ++t) {  // o_proj epilogues and the atomic merge (plain only)
          const int tok = tok_of(wm * TPW + t * 32 + l32);
          if (tok >= nvalid) continue;
          uint16_t* crow = EPI >= 2 ? nullptr : p.C + (int64_t)tok * p.scm;
          float wgt = 1.f;
          if (WEIGHTED && !xs) wgt = p.topw[tok];
#pragma unroll
          for (int f = 0; f < 4; ++f) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = WEIGHTED ? acc[f][t][i] * wgt : acc[f][t][i];
            const int col = n0 + wn * 128 + f * 32 + h * 16;
            if (EPI == 1 || (EPI == 2 && p.R)) {  // + the residual row, in fp32 (epilogue 3: none)
              const uint16_t* rr = p.R + (int64_t)tok * p.srm + col;
              float rf[16];
              unpack8(*reinterpret_cast<const uint4*>(rr), rf);
              unpack8(*reinterpret_cast<const uint4*>(rr + 8), rf + 8);
#pragma unroll
              for (int i = 0; i < 16; ++i) v[i] = v[i] + rf[i];
            }
            if (EPI == 2) {  // accumulate into the fp32 output
              float4* dst = reinterpret_cast<float4*>(p.C32 + (int64_t)tok * p.scm + col);
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                float4 o = dst[q];
                o.x += v[4 * q];
                o.y += v[4 * q + 1];
                o.z += v[4 * q + 2];
                o.w += v[4 * q + 3];
                dst[q] = o;
              }
            } else if (EPI == 3) {  // fp32 partial sums, stored
              float4* dst = reinterpret_cast<float4*>(p.C32 + (int64_t)tok * p.scm + col);
#pragma unroll
              for (int q = 0; q < 4; ++q)
                dst[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
            } else if (EPI == 4) {  // atomic merge into row tok / top_k, two outputs a word
              uint16_t* dst = p.C + (int64_t)(tok / p.merge_topk) * p.scm + col;
#pragma unroll
              for (int q = 0; q < 8; ++q) atomic_add_bf16x2(dst + 2 * q, v[2 * q], v[2 * q + 1]);
            } else {  // EPI 1: bf16(acc + R)
              uint16_t* dst = crow + col;
              *reinterpret_cast<uint4*>(dst) = pack8(v);
              *reinterpret_cast<uint4*>(dst + 8) = pack8(v + 8);
            }
          }
        }
      }
      }
    };
    // the next item's index, fetched while this one runs.  The token-row offsets are
    // complete first: a load the compiler still counts as pending where the branch joins
    // would make it wait for the fetch there.  The address goes through a register the
    // compiler cannot prove uniform, or the atomic becomes a wave reduction that waits for
    // its result at once.  The first wait of the ring (an explicit vmcnt) covers it.
#pragma unroll
    for (int i = 0; i < AI; ++i) asm volatile("" : : "v"(avoff[i]) : "memory");
    int fetched = 0;
    if (tid == 0) {
      int z;
      asm volatile("v_mov_b32 %0, 0" : "=v"(z));
      fetched = __hip_atomic_fetch_add(deal + xcd * 16 + z, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    }
    switch (nvf) {
      case 0: run(std::integral_constant<int, 0>{}); break;
      case 1: run(std::integral_constant<int, 1>{}); break;
      case 2: run(std::integral_constant<int, (TF >= 2 ? 2 : 1)>{}); break;
      case 3: run(std::integral_constant<int, (TF >= 3 ? 3 : 1)>{}); break;
      default: run(std::integral_constant<int, (TF >= 4 ? 4 : 1)>{}); break;
    }
    if (tid == 0) *slot = fetched;
    __syncthreads();  // the ring is refilled by the next item
    k = __builtin_amdgcn_readfirstlane(wg_xcd + *slot);
    __syncthreads();  // every wave has the index before the next prologue refills the ring
  }
  if (p.wg_trace && tid == 0) {  // start, end, items, XCD (hardware register XCC_ID)
    unsigned long long* rec = p.wg_trace + (int64_t)blockIdx.x * 4;
    rec[0] = t_start;
    rec[1] = __builtin_amdgcn_s_memrealtime();
    rec[2] = (unsigned long long)n_run;
    rec[3] = (unsigned long long)(__builtin_amdgcn_s_getreg(20 | (3 << 11)) & 15);
  }
  // the last workgroup out clears the set for the next launch that uses it
  if (tid == 0 && __hip_atomic_fetch_add(deal + 128, 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1) {
    for (int x = 0; x < 8; ++x)
      __hip_atomic_store(deal + x * 16, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(deal + 128, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int MT, int NTW, bool GATED, bool WEIGHTED>
int launch_w512(const GemmArgs& a_in, int capacity, hipStream_t st) {
  constexpr int NO = GATED ? NTW / 2 : NTW;
  static std::atomic<unsigned> next_set{0};
  GemmArgs a = a_in;
  a.deal_set = (int)(next_set.fetch_add(1, std::memory_order_relaxed) % kDealSets);
  a.wg_trace = g_item_trace.load(std::memory_order_relaxed);
  if ((a.n_out % (GATED ? 256 : 512)) || (a.K % 64)) return GLM52_EUNSUPPORTED;
  const int x_blocks = (a.Wp && a.Wx && a.x_rows > 0) ? (a.x_rows + MT - 1) / MT : 0;
  const int items_max = (capacity / MT + x_blocks) * (a.n_out / NO);
  int grid = items_max < 256 ? items_max : 256;
  grid = ((grid + 7) / 8) * 8;
  if constexpr (!GATED && !WEIGHTED) {
    if (a.epi != 0 && !a.Wp) return GLM52_EUNSUPPORTED;
    if (a.epi == 1) {
      moe_gemm_w512_kernel<MT, NTW, false, false, true, 1><<<grid, 256, 0, st>>>(a);
      GLM52_RETURN_LAUNCH();
    }
    if (a.epi == 2) {
      moe_gemm_w512_kernel<MT, NTW, false, false, true, 2><<<grid, 256, 0, st>>>(a);
      GLM52_RETURN_LAUNCH();
    }
    if (a.epi == 3) {
      moe_gemm_w512_kernel<MT, NTW, false, false, true, 3><<<grid, 256, 0, st>>>(a);
      GLM52_RETURN_LAUNCH();
    }
  } else {
    if (a.epi != 0) return GLM52_EUNSUPPORTED;
  }
  if (a.merge_topk > 0) {  // the atomic expert merge: weighted w2 only
    if constexpr (!GATED && WEIGHTED) {
      if (a.Wp)
        moe_gemm_w512_kernel<MT, NTW, false, true, true, 4><<<grid, 256, 0, st>>>(a);
      else
        moe_gemm_w512_kernel<MT, NTW, false, true, false, 4><<<grid, 256, 0, st>>>(a);
      GLM52_RETURN_LAUNCH();
    } else {
      return GLM52_EUNSUPPORTED;
    }
  }
  if (a.Wp)
    moe_gemm_w512_kernel<MT, NTW, GATED, WEIGHTED, true><<<grid, 256, 0, st>>>(a);
  else
    moe_gemm_w512_kernel<MT, NTW, GATED, WEIGHTED, false><<<grid, 256, 0, st>>>(a);
  GLM52_RETURN_LAUNCH();
}

template <bool GATED, bool WEIGHTED>
int launch_w512_bm(const GemmArgs& a, int capacity, hipStream_t st) {
  switch (a.BM) {
    case 64: return launch_w512<64, 512, GATED, WEIGHTED>(a, capacity, st);
    case 128: return launch_w512<128, 512, GATED, WEIGHTED>(a, capacity, st);
    case 256: return launch_w512<256, 256, GATED, WEIGHTED>(a, capacity, st);
    default: return GLM52_EUNSUPPORTED;
  }
}

// One 16-byte chunk of the packed layout per thread and step: chunk d is lane d % 64 of
// stage (d / 64) % nk of load slot (d / (64 nk)) % 32 of tile d / (2048 nk), written at
// packed_slot_off(nk, slot) + stage * kPackStride (+ 16 lane bytes) of its tile.
template <bool GATED>
__global__ __launch_bounds__(256) void pack_w512_kernel(const uint16_t* __restrict__ w,
                                                        int64_t swe, int64_t swn, int64_t swk,
                                                        int gu_off, int num_n, int nk,
                                                        int64_t chunks,
                                                        uint16_t* __restrict__ out) {
  constexpr int NO = GATED ? 256 : 512;
  for (int64_t d = (int64_t)blockIdx.x * 256 + threadIdx.x; d < chunks;
       d += (int64_t)gridDim.x * 256) {
    const int l = (int)(d % 64);
    const int64_t q = d / 64;
    const int kt = (int)(q % nk);
    const int64_t rest = q / nk;  // tile * 32 + slot
    const int slot = (int)(rest % 32);
    const int64_t tile = rest / 32;
    uint16_t* dst = out + tile * packed_tile_elems(nk) + packed_slot_off(nk, slot) +
                    (int64_t)kt * kPackStride + l * 8;
    const int pid_n = (int)(tile % num_n);
    const int64_t e = tile / num_n;
    const int row = pid_n * NO + w512_row(GATED, gu_off, slot / 8, slot % 8, l);
    const int64_t k0 = (int64_t)kt * 32 + w512_chunk(l) * 8;
    const uint16_t* src = w + e * swe + (int64_t)row * swn + k0 * swk;
    if (swk == 1) {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    } else {  // k strided (a [K, N] operand packed as its transpose): gather 8 values
      uint16_t v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = src[q * swk];
      uint4 o;
      o.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
      o.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
      o.z = (uint32_t)v[4] | ((uint32_t)v[5] << 16);
      o.w = (uint32_t)v[6] | ((uint32_t)v[7] << 16);
      *reinterpret_cast<uint4*>(dst) = o;
    }
  }
}

}  // namespace

namespace glm52 {
int launch_wide512(const GemmArgs& a, int capacity, bool gated, bool weighted, hipStream_t st) {
  if (gated) return weighted ? launch_w512_bm<true, true>(a, capacity, st) : launch_w512_bm<true, false>(a, capacity, st);
  return weighted ? launch_w512_bm<false, true>(a, capacity, st) : launch_w512_bm<false, false>(a, capacity, st);
}

}  // namespace glm52

extern "C" int glm52_debug_item_trace(void* buf, int64_t bytes) {
  if (buf && bytes < 256 * 4 * (int64_t)sizeof(unsigned long long)) return GLM52_EINVAL;
  g_item_trace.store(static_cast<unsigned long long*>(buf), std::memory_order_relaxed);
  return GLM52_OK;
}

namespace glm52 {
int64_t pack_wide512(const uint16_t* w, int64_t swe, int64_t swn, int E, int n_out, int k,
                     int gate_up_offset, bool gated, uint16_t* out, hipStream_t st,
                     int64_t swk) {
  const int NO = gated ? 256 : 512;
  if (E <= 0 || n_out <= 0 || (n_out % NO) || k <= 0 || (k % 64)) return GLM52_EUNSUPPORTED;
  const int num_n = n_out / NO, nk = k / 32;
  const int64_t chunks = (int64_t)E * num_n * nk * 2048;  // 16-byte chunks written
  const int64_t bytes = (int64_t)E * num_n * packed_tile_elems(nk) * 2;
  if (!out) return bytes;
  const int64_t blocks = (chunks + 255) / 256;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
  if (gated)
    pack_w512_kernel<true><<<grid, 256, 0, st>>>(w, swe, swn, swk, gate_up_offset, num_n, nk, chunks, out);
  else
    pack_w512_kernel<false><<<grid, 256, 0, st>>>(w, swe, swn, swk, 0, num_n, nk, chunks, out);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? bytes : -(int64_t)err;
}
}  // namespace glm52
