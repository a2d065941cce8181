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
// Item.  One 16-row slice (an expert's block of BM = 16 layout slots, or 16 tokens of the
// extra expert) times 16 W rows: gated, 8 `gate` rows and the matching 8 `up` rows (8
// outputs); plain, 16 rows (16 outputs).  The extra expert's slices come first.  The four
// waves split K: wave w multiplies k-steps w*4 .. +3 of every 512-k stage with
// `v_mfma_f32_16x16x32_bf16` (W rows x tokens) and the partial sums meet in LDS in a fixed
// order at the item's end.
//
// Paired slots (packed weights, K >= 1024; the gated launch from 1024 routed rows): an
// item is two packed slots against the same token rows -- plain: two adjacent slots, 32 W
// rows (32 outputs); gated: both halves of a `gate` slot and of its `up` slot (2 x 8
// outputs) -- so a stage carries 32 KB of W per 16 KB of token rows instead of 16 KB,
// through a ring of three buffers with two in flight.  At T = 256 the w2 launch runs 1168
// against 1310 us (T = 64: 903 against 1007 us) and the w13 launch 1985 against 2086 us,
// the same bits.
//
// Pipeline.  A stage is the 512-k run of the item's 16 W rows and its real token rows (up
// to 16; the rows of padding slots are not loaded, and whatever their LDS rows hold only
// reaches the discarded outputs of those slots).  Stages flow through a ring of four LDS
// buffers with three in flight, and the ring runs across item boundaries, so every
// workgroup streams continuously.  Each wave counts the loads it issued per stage, and a
// stage is waited for with the count of the two newer stages; stages past the workgroup's
// last one re-read its last stage into the free buffer.  The layout entries an item needs
// (expert, token ids, routing weights) are read with scalar loads, which do not share the
// vector-memory counter, so reading them never drains the weight loads in flight; the
// epilogue takes the token ids and weights from a small LDS ring.  The epilogue adds no
// barrier: the waves stash their partial sums at the item's last stage, and all four
// reduce and store them after the next stage's barrier, a quarter of the outputs each.  Staged row R keeps
// global 16-byte chunk c at chunk c ^ (R & 15): the 16 lanes of an operand read hit 16
// distinct bank groups.
//
// Routing mode (decode, T <= 4 tokens, gated, with the shared expert as the extra one).
// The layout is not read but derived: every workgroup computes the biased top-k of the T
// tokens from the router logits (the rule of `glm52/reference.py:62-79` as in select.h; an
// expert's slot is the number of experts that beat it, counted by its own thread) and the
// sglang layout of the selected ids (`glm52/reference.py:85-128`; with T <= 4 no expert gets
// more than 16 ids, so each selected expert owns one block, in ascending expert order, its
// ids in ascending flat order) into LDS: the logits and the bias are loaded straight into
// LDS ahead of the loads of its first item -- a shared-expert item, which needs no
// routing -- and the routing waits for them alone.  Workgroup 0 writes the ids and weights; all
// workgroups share writing the layout, so the kernels that follow read the same tensors as
// after glm52_router_topk_align.  Nothing here waits on another workgroup.
#include "moe_gemm.h"
#include "select.h"

using namespace glm52;

namespace {

constexpr int KS = 512;            // k per stage: one 1 KB run of every staged row
constexpr int NSTAGE = 4;
constexpr int SROWS = 32;          // 16 W rows + 16 token rows
constexpr int SELEM = SROWS * KS;  // elements per stage
constexpr int RT = 4;              // routing mode: at most 4 tokens
constexpr int RSLOT = RT * 8;      // ... and at most 32 routed ids
constexpr int NMETA = 8;           // items whose token ids / weights are kept for the epilogue


struct RouteLds {
  float logits[RT][kMaxE];  // the T tokens' logits and the bias, loaded straight into LDS
  float bias[kMaxE];
  uint64_t key[RT][kMaxE];  // selection keys as unique ordered integers, and the scores
  float score[RT][kMaxE];
  float sel_s[RT][8];
  int sel_i[RT][8];
  uint64_t cand[RT][32];  // each wave's top-k keys (slot wave * 8 + its rank), zero-padded
  int ids[RSLOT];
  int blk_e[RSLOT];      // expert of layout block b
  int blk_n[RSLOT];      // its id count (<= RT)
  int blk_f[RSLOT][RT];  // its flat ids, ascending
  int nblk;
};

// A wave-uniform 32-bit load through the scalar cache (lgkmcnt, not vmcnt).
GLM52_DEV int sload_i32(const void* base, int idx) {
  int v;
  asm volatile("s_load_dword %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=s"(v)
               : "s"(base), "s"(idx * 4)
               : "memory");
  return v;
}

// A wave-uniform pointer the compiler keeps in SGPRs (the base operand of dma16s).
GLM52_DEV const uint16_t* uniform_ptr(const uint16_t* q) {
  const uint64_t v = reinterpret_cast<uint64_t>(q);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint16_t*>(((uint64_t)hi << 32) | lo);
}

typedef int sint4_t __attribute__((ext_vector_type(4)));

// Expert id eids[b] and the four slot entries sti[s .. s+3] (s a multiple of 4) in one
// scalar round trip (b and s wave-uniform).  The loads and their wait are one asm statement, so no use of a
// result can be scheduled before the wait.
GLM52_DEV void sload_block(const int32_t* eids, int b, const int32_t* sti, int s, int& e,
                           int f[4]) {
  int ev;
  sint4_t fv;
  asm volatile("s_load_dword %0, %2, %3\n\ts_load_dwordx4 %1, %4, %5\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(ev), "=&s"(fv)
               : "s"(eids), "s"(__builtin_amdgcn_readfirstlane(b * 4)), "s"(sti),
                 "s"(__builtin_amdgcn_readfirstlane(s * 4))
               : "memory");
  e = ev;
  f[0] = fv.x;
  f[1] = fv.y;
  f[2] = fv.z;
  f[3] = fv.w;
}

// Four scattered fp32 entries base[idx[i]] in one scalar round trip (idx wave-uniform).
GLM52_DEV void sload_f32x4(const float* base, const int idx[4], float v[4]) {
  int a, b, c, d;
  asm volatile(
      "s_load_dword %0, %4, %5\n\ts_load_dword %1, %4, %6\n\ts_load_dword %2, %4, %7\n\t"
      "s_load_dword %3, %4, %8\n\ts_waitcnt lgkmcnt(0)"
      : "=&s"(a), "=&s"(b), "=&s"(c), "=&s"(d)
      : "s"(base), "s"(__builtin_amdgcn_readfirstlane(idx[0] * 4)),
        "s"(__builtin_amdgcn_readfirstlane(idx[1] * 4)),
        "s"(__builtin_amdgcn_readfirstlane(idx[2] * 4)),
        "s"(__builtin_amdgcn_readfirstlane(idx[3] * 4))
      : "memory");
  v[0] = __builtin_bit_cast(float, a);
  v[1] = __builtin_bit_cast(float, b);
  v[2] = __builtin_bit_cast(float, c);
  v[3] = __builtin_bit_cast(float, d);
}

// Wait until at most n (wave-uniform, 0..24) of this wave's vector-memory loads are in
// flight; the count is an immediate, so each value is one branch.
GLM52_DEV void wait_vmcnt_at_most(int n) {
  switch (n) {
    case 0: GLM52_WAIT_VMCNT(0); break;
    case 1: GLM52_WAIT_VMCNT(1); break;
    case 2: GLM52_WAIT_VMCNT(2); break;
    case 3: GLM52_WAIT_VMCNT(3); break;
    case 4: GLM52_WAIT_VMCNT(4); break;
    case 5: GLM52_WAIT_VMCNT(5); break;
    case 6: GLM52_WAIT_VMCNT(6); break;
    case 7: GLM52_WAIT_VMCNT(7); break;
    case 8: GLM52_WAIT_VMCNT(8); break;
    case 9: GLM52_WAIT_VMCNT(9); break;
    case 10: GLM52_WAIT_VMCNT(10); break;
    case 11: GLM52_WAIT_VMCNT(11); break;
    case 12: GLM52_WAIT_VMCNT(12); break;
    case 13: GLM52_WAIT_VMCNT(13); break;
    case 14: GLM52_WAIT_VMCNT(14); break;
    case 15: GLM52_WAIT_VMCNT(15); break;
    case 16: GLM52_WAIT_VMCNT(16); break;
    case 17: GLM52_WAIT_VMCNT(17); break;
    case 18: GLM52_WAIT_VMCNT(18); break;
    case 19: GLM52_WAIT_VMCNT(19); break;
    case 20: GLM52_WAIT_VMCNT(20); break;
    case 21: GLM52_WAIT_VMCNT(21); break;
    case 22: GLM52_WAIT_VMCNT(22); break;
    case 23: GLM52_WAIT_VMCNT(23); break;
    default: GLM52_WAIT_VMCNT(24); break;
  }
}

// PAIR (packed, not routing): an item is two packed slots against the same token rows --
// plain: two adjacent slots (32 W rows, 32 outputs); gated: a whole `gate` slot and its
// `up` slot (both halves, 2 x 8 outputs) -- so a stage carries twice the W bytes per token
// row; a ring of three 48 KB stages, two in flight.  At T = 256 the token-row loads are a
// sixth of the w2 launch (1314 against 1105 us without them, a timing-only copy).  One
// partial-sum buffer: an item's stash and the previous item's reduce are a barrier apart
// when an item has two or more stages (the launcher requires K >= 1024).
template <bool GATED, bool WEIGHTED, bool ROUTE, bool PACKED, bool PAIR = false>
__global__ __launch_bounds__(256) void moe_gemm_runs_kernel(GemmArgs p) {
  static_assert(!PAIR || (PACKED && !ROUTE), "paired slots: packed, not routing");
  constexpr int NSB = PAIR ? 3 : NSTAGE;  // ring buffers
  constexpr int WR = PAIR ? 32 : 16;      // W rows (1 KB slabs) of a stage; token rows follow
  constexpr int SE = (WR + 16) * KS;      // elements per stage
  constexpr int NB = PAIR ? 2 : 1;        // 16 x 16 output blocks per item
  __shared__ __attribute__((aligned(1024))) uint16_t ring[NSB * SE];
  __shared__ float red[PAIR ? 1 : 2][4][4 * NB][kWave];  // partial sums by wave
  __shared__ int meta_tok[NMETA][16];    // flat ids of an item's token rows
  __shared__ float meta_w[NMETA][16];    // their routing weights (weighted)
  __shared__ RouteLds rs;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  const int r16 = lane % 16, g = lane / 16;

  constexpr int NOC = (GATED ? 8 : 16) * NB;  // outputs per item
  const int xm = (p.x_rows + 15) / 16;
  const int num_n = p.n_out / NOC;
  const int x_items = xm * num_n;  // the extra expert's items come first
  const int nks = p.K / KS;
  // packed weights: the item's 512-row tile and its 32-k stages
  constexpr int NO512 = GATED ? 256 : 512;
  const int num_n512 = p.n_out / NO512;
  const int nk32 = p.K / 32;
  // read once here in the packed instances, whose register pressure otherwise keeps these
  // fields of p in scratch (every scratch load waits for all loads in flight)
  const uint16_t* const pw_r = p.Wp;
  const uint16_t* const pw_x = p.Wx;
  const int nvalid = PACKED ? __builtin_amdgcn_readfirstlane(p.num_valid) : p.num_valid;
  int num_m = ROUTE ? 0 : sload_i32(p.ntp, 0) / 16;
  int items = (xm + num_m) * num_n;
  const uint32_t ring_base = lds_addr(ring);
  // Where the workgroup's it-th item sits in the item order.  Outside the routing mode,
  // inside each full round of gridDim.x items the workgroups of one XCD (blockIdx % 8)
  // take runs of C consecutive items, so the outputs that share a 128-byte line --
  // consecutive items of a layout block -- are written through one L2 instead of several.
  // C = 32 (all of an XCD's share of the round) for the gated launches and 4 (one line of
  // 64 outputs) for the plain ones on weights in place: measured at T = 256, w13 2235 ->
  // 2080 us and the block 3614 -> 3406 us.  The plain launch on packed weights keeps the
  // issue order (C = 1: consecutive items on consecutive XCDs), each item one packed slot:
  // at T = 256 its w2 launch runs 1349 us against 1402 (C = 4), 1417 (C = 2) and 1407 us
  // (C = 8), interleaved in one process.  The paired gated launch takes runs of 8 (T = 256:
  // w13 1985 us against 2020 with 32 and 1997 with 16); the paired plain launch keeps C = 1
  // (w2 1170 us against 1329, 1175 and 1184 with 2, 4 and 8).  The last, partial round
  // keeps the issue order.
  constexpr int C = GATED ? (PAIR ? 8 : 32) : (PACKED ? 1 : 4);
  auto place = [&](int it) {
    if (ROUTE) return it;
    const int G = (int)gridDim.x;
    if ((G % (8 * C)) || it >= (items / G) * G) return it;
    const int b = it % G;
    const int x = b & 7, k = b >> 3;
    return it - b + (x + 8 * (k / C)) * C + k % C;
  };

  // ---- load side: the wave's 4 W rows and its real token rows (da_n of 4) of the item
  // being loaded; the item's token ids (and weights) go to the LDS ring for its epilogue
  const uint16_t* dw[4];
  uint32_t wvo = 0;  // packed: the lane's byte offset inside the item's load slot(s)
  const uint16_t* da[4];
  int da_n = 0;
  // The first 512-k stage of the item being loaded (its stages run from there, wrapping).
  // Plain launches: the workgroups advance in step, and with every item at the same stage
  // the loads in flight sit a power of two apart and fall on fewer HBM channels; so each
  // 512-row tile's 32 output slots start at their own stage (w2 at T = 4: 135.3 -> 127.3
  // us, T = 16: 433.5 -> 421.0 us, T = 256: 1166 -> 1114 us; groups of 8, 16, 64, 128 or
  // 256 slots measured slower).  The start depends on the output slots only, so every
  // mapping adds an output's stages in one order.  Gated launches keep stage 0 first:
  // there a rotation slowed w13 (T = 1: 74.4 -> 92.5 us).
  int d_rot = 0;
  auto dma_setup = [&](int it) {
    const int L = place(it);
    if constexpr (!GATED) d_rot = (((PAIR ? 2 : 1) * (L % num_n)) >> 5) % nks;
    const int m = L / num_n;
    const int n0 = (L % num_n) * NOC;
    const bool extra = m < xm;
    const int slot = (it / (int)gridDim.x) % NMETA;
    // the block's expert and the wave's four slot entries: from LDS in routing mode, else
    // in one scalar round trip
    int e = 0;
    const int nv = PACKED ? nvalid : p.num_valid;
    int fr[4] = {nv, nv, nv, nv};
    if (!extra) {
      if constexpr (ROUTE) {
        e = __builtin_amdgcn_readfirstlane(rs.blk_e[m - xm]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tr = wvu * 4 + i;
          fr[i] = __builtin_amdgcn_readfirstlane(tr < rs.blk_n[m - xm] ? rs.blk_f[m - xm][tr] : nv);
        }
      } else {
        sload_block(p.eids, m - xm, p.sti, (m - xm) * 16 + wvu * 4, e, fr);
      }
    }
    if constexpr (PACKED) {
      // item n of the layout block: load slot ps of packed tile P (gated: half hs of the
      // `gate` slot and the same half of its `up` slot, four slots on, 512 B each); wave
      // instruction i loads 32-k stage 16 s + 4 wv + i of the slot(s) for 512-k stage s: an
      // item streams its slot's K / 32 pieces of 1 KB, kPackStride apart
      const int n = PAIR ? 2 * (L % num_n) : L % num_n;  // paired: the first slot's item
      const int P = n >> 5, q5 = n & 31;
      const int ps = GATED ? (q5 >> 3) * 8 + ((q5 >> 1) & 3) : q5;
      const uint16_t* tb = uniform_ptr(extra ? pw_x : pw_r) +
                           ((int64_t)e * num_n512 + P) * packed_tile_elems(nk32) +
                           packed_slot_off(nk32, ps);
      dw[0] = tb + (int64_t)(wvu * 4) * kPackStride;  // the slot's 32-k stages
      if (PAIR)  // the second slot's stages (gated: the `up` slot, four slots on)
        dw[1] = dw[0] + (packed_slot_off(nk32, ps + (GATED ? 4 : 1)) - packed_slot_off(nk32, ps));
      if (GATED && !PAIR) {
        const int hs = q5 & 1;
        wvo = (uint32_t)(lane < 32 ? (hs * 32 + lane) * 16
                                   : (packed_slot_off(nk32, ps + 4) - packed_slot_off(nk32, ps)) * 2 +
                                         (hs * 32 + lane - 32) * 16);
      } else {
        wvo = (uint32_t)(lane * 16);
      }
    } else {
      const uint16_t* wbase = extra ? p.Wx : p.W + (int64_t)e * p.swe;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wvu * 4 + i;  // W tile row
        const int grow = GATED ? (row < 8 ? n0 + row : p.gu_off + n0 + row - 8) : n0 + row;
        dw[i] = wbase + (int64_t)grow * p.swn;
      }
    }
    da_n = 0;
    int fs[4];
    bool oks[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tr = wvu * 4 + i;  // token row of the slice; real rows fill a prefix
      int f;
      bool ok;
      if (extra) {
        f = m * 16 + tr;
        ok = f < p.x_rows;
        da[i] = p.Ax + (int64_t)(ok ? f : 0) * p.sax;
      } else {
        f = fr[i];
        ok = f < nv;
        da[i] = p.A + (int64_t)(ok ? f / p.a_div : 0) * p.sam;
      }
      da_n += ok ? 1 : 0;
      fs[i] = f;
      oks[i] = ok;
    }
    float w[4] = {1.f, 1.f, 1.f, 1.f};
    if (WEIGHTED && !extra) {
      int wi[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) wi[i] = oks[i] ? fs[i] : 0;  // padding slots read entry 0
      sload_f32x4(p.topw, wi, w);
    }
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        meta_tok[slot][wvu * 4 + i] = oks[i] ? fs[i] : -1;
        meta_w[slot][wvu * 4 + i] = w[i];
      }
    }
  };
  auto issue = [&](int s0, int buf) {  // stage s0 (512-k run) of the item being loaded
    int s = s0;
    if constexpr (!GATED) s = s0 + d_rot < nks ? s0 + d_rot : s0 + d_rot - nks;
    const uint32_t sb = ring_base + (uint32_t)(buf * SE * 2);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int R = b * 16 + wvu * 4 + i;
        if constexpr (PACKED)
          dma16s_nt(uniform_ptr(dw[b] + (int64_t)(s * 16 + i) * kPackStride), wvo,
                    sb + (uint32_t)(R * KS * 2));
        else
          dma16s_nt(dw[i] + s * KS, (uint32_t)((lane ^ (R & 15)) * 16), sb + (uint32_t)(R * KS * 2));
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int R = WR + wvu * 4 + i;
      if (i < da_n) {
        if constexpr (PACKED)  // a per-lane address: SGPRs are short in these instances
          dma16(da[i] + s * KS + (lane ^ (R & 15)) * 8, sb + (uint32_t)(R * KS * 2));
        else
          dma16s(da[i] + s * KS, (uint32_t)((lane ^ (R & 15)) * 16), sb + (uint32_t)(R * KS * 2));
      }
    }
    return 4 * NB + da_n;  // loads issued
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

  // ---- routing mode: the top-k of every token and the layout, into LDS ------------------
  // Loads of the logits (wave t: token t) and the bias (wave 0) straight into LDS, issued
  // before the first item's stages so that they land first; returns the loads issued.
  auto route_load = [&]() {
    int n = 0;
    if (wvu < p.r_T) {
      if (4 * lane < p.r_E)
        dma16s(p.r_logits + (int64_t)wvu * p.r_sl, (uint32_t)(lane * 16),
               lds_addr(reinterpret_cast<const uint16_t*>(&rs.logits[wvu][0])));
      ++n;
    }
    if (wvu == 0 && p.r_bias) {
      if (4 * lane < p.r_E)
        dma16s(p.r_bias, (uint32_t)(lane * 16), lds_addr(reinterpret_cast<const uint16_t*>(&rs.bias[0])));
      ++n;
    }
    return n;
  };
  auto route = [&]() {
    const int T = p.r_T, E = p.r_E, topk = p.r_topk;
    const bool active = wv < T;
    // thread tid owns expert tid: its score and key for every token (the rule of topk_keys).
    // The key goes to LDS as one integer that orders like the selection order: the float
    // key mapped to an unsigned integer of the same order (-0 taken as +0, so that equal
    // keys stay equal) above the complement of the expert index, so that a larger key, or
    // an equal key at a lower index, is a larger integer.  A comparison is then a single
    // vector compare: boolean combinations of compares would run on the scalar unit, each
    // waiting on the vector unit's result.
    for (int t = 0; t < T; ++t) {
      if (tid < E) {
        const float sc = (float)(1.0 / (1.0 + exp(-(double)rs.logits[t][tid])));
        float k = p.r_bias ? sc + rs.bias[tid] : sc;
        k = (k != k) ? -INFINITY : (k == 0.f ? 0.f : k);
        const uint32_t b = __builtin_bit_cast(uint32_t, k);
        const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
        rs.key[t][tid] = ((uint64_t)ord << 32) | (uint32_t)(~tid);
        rs.score[t][tid] = sc;
      }
    }
    __syncthreads();
    // slot of expert tid = the number of experts whose key integer is larger.  First the
    // rank inside the wave's 64 experts; the wave's top k go to cand.  A key outside its
    // wave's top k has at least k larger keys, and for a key inside the global top k every
    // larger key is in its own wave's top k: so the global slots are the ranks among the
    // (at most 32) listed keys, and every other key ranks k or more there.
    int wrank[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      wrank[t] = kMaxE;
      if (t < T) {
        if (lane < 8) rs.cand[t][wv * 8 + lane] = 0ull;  // below every key
        if (tid < E) {
          const uint64_t k = rs.key[t][tid];
          const int e1 = min(E, (wv + 1) * kWave);
          int rank = 0;
#pragma unroll 8
          for (int e2 = wv * kWave; e2 < e1; e2 += 2) {
            const ulonglong2 q = *reinterpret_cast<const ulonglong2*>(&rs.key[t][e2]);
            rank += q.x > k ? 1 : 0;
            rank += q.y > k ? 1 : 0;
          }
          wrank[t] = rank;
          if (rank < topk) rs.cand[t][wv * 8 + rank] = k;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      if (t < T && wrank[t] < topk) {
        const uint64_t k = rs.key[t][tid];
        int rank = 0;
#pragma unroll
        for (int c = 0; c < 32; c += 2) {
          const ulonglong2 q = *reinterpret_cast<const ulonglong2*>(&rs.cand[t][c]);
          rank += q.x > k ? 1 : 0;
          rank += q.y > k ? 1 : 0;
        }
        if (rank < topk) {
          rs.sel_i[t][rank] = tid;
          rs.sel_s[t][rank] = rs.score[t][tid];
        }
      }
    }
    __syncthreads();
    if (active && lane < topk) {
      float w;
      int id;
      topk_weight(rs.sel_s[wv], rs.sel_i[wv], topk, p.r_scale, p.r_norm_prob, &w, &id);
      rs.ids[wv * topk + lane] = id;
      if (blockIdx.x == 0) {
        p.r_topw[(int64_t)wv * p.r_stw + lane] = w;
        p.r_topi[(int64_t)wv * p.r_sti + lane] = id;
      }
    }
    __syncthreads();
    const int numel = T * topk;
    if (wv == 0) {
      // one block per distinct expert, in expert order; ids of one expert in flat order.
      // Lane f (flat id f) counts with single compares: ids of a smaller expert (below),
      // ids before it in (expert, flat) order (pos), and ids of its expert (same); then the
      // distinct experts below its own, counting only the first id of each expert.
      const int e = lane < numel ? rs.ids[lane] : kMaxE;
      const int c = e * 64 + lane;
      int below = 0, pos = 0, upto = 0;
      for (int j = 0; j < numel; ++j) {
        const int ej = rs.ids[j];
        below += ej < e ? 1 : 0;
        upto += ej <= e ? 1 : 0;
        pos += ej * 64 + j < c ? 1 : 0;
      }
      const int earlier_same = pos - below;
      const uint64_t firsts = __ballot(lane < numel && earlier_same == 0);
      int distinct_below = 0;
      for (int j = 0; j < numel; ++j) {
        const int ej = rs.ids[j];
        const int fk = ((firsts >> j) & 1ull) ? ej : kMaxE;  // wave-uniform select
        distinct_below += fk < e ? 1 : 0;
      }
      if (lane < numel) {
        rs.blk_f[distinct_below][earlier_same] = lane;
        if (earlier_same == 0) {
          rs.blk_e[distinct_below] = e;
          rs.blk_n[distinct_below] = upto - below;
        }
      }
      if (lane == 0) rs.nblk = __popcll(firsts);
    }
    __syncthreads();
    // the layout tensors, split over the workgroups: slot s of sorted_token_ids holds the
    // flat id of slot s % 16 of block s / 16, or the sentinel numel; expert_ids[b] the
    // expert of block b, or -1 past the last block
    const int nblk = rs.nblk;
    const int cap = p.r_capacity;
    const int nent = cap + cap / 16;
    const int per = (nent + (int)gridDim.x - 1) / (int)gridDim.x;
    const int q1 = min(nent, ((int)blockIdx.x + 1) * per);
    for (int q = (int)blockIdx.x * per + tid; q < q1; q += 256) {
      if (q < cap) {
        const int b = q / 16, j = q % 16;
        p.r_sorted[q] = (b < nblk && j < rs.blk_n[b]) ? rs.blk_f[b][j] : numel;
      } else {
        const int b = q - cap;
        p.r_eids[b] = b < nblk ? rs.blk_e[b] : -1;
      }
    }
    if (blockIdx.x == 0 && tid == 0) p.r_ntp[0] = nblk * 16;
    num_m = __builtin_amdgcn_readfirstlane(nblk);
    items = (xm + num_m) * num_n;
  };

  // ---- multiply side ------------------------------------------------------------------
  // Packed: the W part of a stage holds 16 slabs of 1 KB, slab j the 32-k stage j as the
  // load wrote it; MFMA row r16 is packed row p = r16 (gated: rows 0-7 the `gate` half,
  // 8-15 the `up` half, p = 8 hs + r16 % 8 of each slot), and its 8-k chunk g sits in the
  // lane slot 4 p + (g ^ (p / 4 % 4)).  The element offset of lane (r16, g) in a slab:
  // Paired, block b reads slot b's slab (plain: slab 16 b + k; gated: rows 0-7 from the
  // `gate` slab k, 8-15 from the `up` slab 16 + k, both of half hs = b), so the offset
  // below includes the slab.
  auto w_ofs = [&](int it, int b) {
    if constexpr (!PACKED) {
      return 0;
    } else if constexpr (GATED) {
      const int hs = PAIR ? b : place(it) & 1;  // num_n is even
      const int pp = r16 & 7;
      if constexpr (PAIR) {
        const int pr = 8 * hs + pp;  // row of the whole slot
        return (r16 >> 3) * 16 * 512 + (4 * pr + (g ^ ((pr >> 2) & 3))) * 8;
      }
      return (r16 >> 3) * 256 + (4 * pp + (g ^ (2 * hs + (pp >> 2)))) * 8;
    } else {
      return b * 16 * 512 + (4 * r16 + (g ^ ((r16 >> 2) & 3))) * 8;
    }
  };
  auto compute = [&](int buf, floatx4_t (&acc)[NB], const int (&wofs)[NB]) {
    const uint16_t* sb = ring + buf * SE;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = (wv * 4 + q) * 4 + g;  // logical 16-byte chunk of the 512-k run
      const uint4 af = *reinterpret_cast<const uint4*>(sb + (WR + r16) * KS + ((c ^ r16) * 8));
#pragma unroll
      for (int b = 0; b < NB; ++b) {  // block b: the item's slot b (paired) or its only one
        const uint4 wf =
            PACKED ? *reinterpret_cast<const uint4*>(sb + (wv * 4 + q) * 512 + wofs[b])
                   : *reinterpret_cast<const uint4*>(sb + r16 * KS + ((c ^ r16) * 8));
        acc[b] = mfma16(wf, af, acc[b]);  // C[W row 4 g + i][token r16]
      }
    }
  };
  // Epilogue, in two halves.  At an item's last stage every wave stashes its partial sums
  // (no barrier).  After the next stage's barrier all four waves finish it together: wave
  // w takes token columns 4 w .. 4 w + 3, a lane one (token, output) pair, adds the four
  // waves' partials in a fixed order and stores; the 16 lanes of a token write 16
  // consecutive outputs.  A partial for W row r and token c sits in register r % 4 of
  // lane (r / 4) * 16 + c.
  auto stash = [&](int par, const floatx4_t (&acc)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[PAIR ? 0 : par][wv][b * 4 + i][lane] = acc[b][i];
  };
  auto rsum = [&](int par, int b, int row, int c) {
    const int i = b * 4 + row % 4, l = (row / 4) * 16 + c;
    const auto& rd = red[PAIR ? 0 : par];
    return ((rd[0][i][l] + rd[1][i][l]) + rd[2][i][l]) + rd[3][i][l];
  };
  // output column of output j of item L: n0 + j, or packed, row phi32(p) of the slot's
  // 32-row group (gated p = 8 hs + j)
  auto out_col = [&](int L, int b, int j) {
    const int n = PAIR ? 2 * (L % num_n) + b : L % num_n;
    if constexpr (!PACKED) {
      return n * NOC + j;
    } else if constexpr (GATED) {
      const int P = n >> 5, q5 = n & 31;
      const int i = (q5 >> 1) & 3;
      return P * 256 + (q5 >> 3) * 64 + (i >> 1) * 32 + (i & 1) * 8 + phi32(8 * (q5 & 1) + j);
    } else {
      const int P = n >> 5, q5 = n & 31;
      const int i = q5 & 7;
      return P * 512 + (q5 >> 3) * 128 + (i >> 1) * 32 + (i & 1) * 8 + phi32(j);
    }
  };
  auto finish = [&](int it, int par) {
    const int L = place(it);
    const int m = L / num_n;
    const bool extra = m < xm;
    const int slot = (it / (int)gridDim.x) % NMETA;
    const int c = wv * 4 + lane / 16;  // token column of the slice
    const int j = lane % 16;           // output of the item's block
    if (!GATED && p.merge_topk > 0) {  // atomic merge: lane pairs (j, j + 1) add as one word
      const int tok = meta_tok[slot][c];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float v = rsum(par, b, j, c);
        if (WEIGHTED && !extra) v = v * meta_w[slot][c];
        const float v1 = __shfl_down(v, 1, 16);  // every lane is active here
        if (tok >= 0 && !(j & 1) && !extra)
          atomic_add_bf16x2(p.C + (int64_t)(tok / p.merge_topk) * p.scm + out_col(L, b, j), v,
                            v1);
      }
      return;
    }
    if (GATED && j >= 8) return;
    const int tok = meta_tok[slot][c];
    if (tok < 0) return;
    uint16_t* dst = extra ? p.Cx + (int64_t)tok * p.scx : p.C + (int64_t)tok * p.scm;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float v;
      if (GATED) {
        v = silu_mul(rsum(par, b, j, c), rsum(par, b, 8 + j, c));  // `gate` row j, `up` 8 + j
      } else {
        v = rsum(par, b, j, c);
        if (WEIGHTED && !extra) v = v * meta_w[slot][c];
      }
      dst[out_col(L, b, j)] = f32_to_bf16(v);
    }
  };

  // prologue: the first three stages.  In routing mode the logits are loaded first and a
  // first item of the extra expert has its stages issued before the routing (which waits
  // only for the logits); the item count is known only after the routing, so the prologue
  // stops at the end of that item (K of fewer than three stages) and goes on after it.  A
  // routed first item is set up after the routing.
  int nst[3] = {0, 0, 0};  // loads issued for prologue stages 0..2
  int npro = 0;
  auto prologue_to = [&](int upto) {  // issue prologue stages npro .. upto-1
    while (npro < upto) {
      nst[npro] = issue(d_s, npro);
      if (++npro < upto) dma_advance();
    }
  };
  const bool first_extra = (int)blockIdx.x < x_items;
  if (!ROUTE) {
    if ((int)blockIdx.x >= items) return;
    dma_setup(d_item);
    prologue_to(NSB - 1);
    dma_advance();
  } else {
    route_load();
    if (first_extra) {
      dma_setup(d_item);
      prologue_to(nks < 3 ? nks : 3);
      // the logits landed (this wave's; every wave's after the routing's first barrier):
      // at most the prologue's loads are still in flight
      wait_vmcnt_at_most(nst[0] + nst[1] + nst[2]);
    } else {
      GLM52_WAIT_VMCNT(0);
    }
    __syncthreads();
    route();
    if (first_extra) {
      dma_advance();
      if (npro < 3) {
        prologue_to(3);
        dma_advance();
      }
    } else {
      if ((int)blockIdx.x >= items) return;
      dma_setup(d_item);
      prologue_to(3);
      dma_advance();
    }
  }
  int n1 = nst[1], n2 = nst[2];
  const int total = ((items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x) * nks;

  floatx4_t acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  int c_item = blockIdx.x, c_s = 0;
  int wofs[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) wofs[b] = w_ofs(c_item, b);
  int pend = -1, par = 0;  // the item whose partial sums wait in red[par ^ 1], if any
#pragma unroll 1
  for (int j = 0; j < total; ++j) {
    // stage j landed for this wave (the newer stages may be in flight) and for every wave;
    // every wave is done with the buffer refilled next, and the stashed partials are visible
    if constexpr (PAIR) {
      wait_vmcnt_at_most(n1);  // stage j + 1 in flight
      __syncthreads();
      n1 = issue(d_s, (j + NSB - 1) % NSB);
    } else {
      wait_vmcnt_at_most(n1 + n2);  // stages j + 1, j + 2 in flight
      __syncthreads();
      n1 = n2;
      n2 = issue(d_s, (j + NSB - 1) % NSB);
    }
    dma_advance();
    if (pend >= 0) {
      finish(pend, par ^ 1);
      pend = -1;
    }
    compute(j % NSB, acc, wofs);
    if (++c_s == nks) {
      stash(par, acc);
      pend = c_item;
      par ^= 1;
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[b] = floatx4_t{0.f, 0.f, 0.f, 0.f};
      c_s = 0;
      c_item += gridDim.x;
#pragma unroll
      for (int b = 0; b < NB; ++b) wofs[b] = w_ofs(c_item, b);
    }
  }
  if (pend >= 0) {
    __syncthreads();
    finish(pend, par ^ 1);
  }
  GLM52_WAIT_VMCNT(0);  // the re-reads past the last stage land before the workgroup ends
}

template <bool GATED, bool WEIGHTED, bool ROUTE, bool PACKED, bool PAIR = false>
int launch_runs_t(const GemmArgs& a, int capacity, hipStream_t st) {
  constexpr int NOC = (GATED ? 8 : 16) * (PAIR ? 2 : 1);
  if (a.BM != 16 || (a.n_out % NOC) || (a.K % KS) || a.K / KS < (PAIR ? 2 : 1))
    return GLM52_EUNSUPPORTED;
  // packed: whole 512-row tiles (256 outputs gated), no atomic merge
  if (PACKED && ((a.n_out % (GATED ? 256 : 512)) || a.merge_topk > 0 ||
                 (a.x_rows > 0 && !a.Wx)))
    return GLM52_EUNSUPPORTED;
  if (ROUTE && (a.x_rows < 1 || a.r_T < 1 || a.r_T > RT || a.r_topk < 1 || a.r_topk > 8 ||
                a.r_E < a.r_topk || a.r_E > kMaxE || (a.r_E % 4) ||
                a.r_capacity < a.r_T * a.r_topk + a.r_E * 15 || (a.r_capacity % 16)))
    return GLM52_EINVAL;
  const int items_max = (capacity / 16 + (a.x_rows + 15) / 16) * (a.n_out / NOC);
  int grid = items_max < 256 ? items_max : 256;
  if (grid < 1) grid = 1;
  moe_gemm_runs_kernel<GATED, WEIGHTED, ROUTE, PACKED, PAIR><<<grid, 256, 0, st>>>(a);
  GLM52_RETURN_LAUNCH();
}

}  // namespace

namespace glm52 {
int launch_runs(const GemmArgs& a, int capacity, bool gated, bool weighted, bool route,
                hipStream_t st) {
  if (a.Wp) {  // packed weights (glm52_pack_w512)
    if (route) {
      if (!gated || weighted) return GLM52_EUNSUPPORTED;
      return launch_runs_t<true, false, true, true>(a, capacity, st);
    }
    // paired slots from two 512-k stages on (K >= 1024); gated from 1024 routed rows (at
    // 512 the blocks hold about two real rows and the unpaired launch is 12 us faster)
    if (gated && a.K >= 2 * KS && a.num_valid >= 1024)
      return weighted ? launch_runs_t<true, true, false, true, true>(a, capacity, st)
                      : launch_runs_t<true, false, false, true, true>(a, capacity, st);
    if (gated) return weighted ? launch_runs_t<true, true, false, true>(a, capacity, st) : launch_runs_t<true, false, false, true>(a, capacity, st);
    if (a.K >= 2 * KS)
      return weighted ? launch_runs_t<false, true, false, true, true>(a, capacity, st)
                      : launch_runs_t<false, false, false, true, true>(a, capacity, st);
    return weighted ? launch_runs_t<false, true, false, true>(a, capacity, st) : launch_runs_t<false, false, false, true>(a, capacity, st);
  }
  if (route) {
    if (!gated || weighted) return GLM52_EUNSUPPORTED;
    return launch_runs_t<true, false, true, false>(a, capacity, st);
  }
  if (gated) return weighted ? launch_runs_t<true, true, false, false>(a, capacity, st) : launch_runs_t<true, false, false, false>(a, capacity, st);
  return weighted ? launch_runs_t<false, true, false, false>(a, capacity, st) : launch_runs_t<false, false, false, false>(a, capacity, st);
}
}  // namespace glm52
