// Pieces shared by the grouped expert GEMM kernels (moe_gemm.hip, moe_gemm_wide.hip).
#pragma once

#include "common.h"

namespace glm52 {

// C(16 x 16, fp32) += A(16 x 32) . B(32 x 16) on bf16 MFMA.  Lane l supplies row l % 16 of
// A and column l % 16 of B, each as the 8 consecutive k starting at 8 (l / 16); the result
// register i of lane l is row 4 (l / 16) + i, column l % 16.
GLM52_DEV floatx4_t mfma16(const uint4& a, const uint4& b, floatx4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

typedef float floatx16_t __attribute__((ext_vector_type(16)));

// C(32 x 32, fp32) += A(32 x 16) . B(16 x 32) on bf16 MFMA.  Lane l supplies row l % 32 of A
// and column l % 32 of B, each as the 8 consecutive k starting at 8 (l / 32); the result
// register i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.
GLM52_DEV floatx16_t mfma32(const uint4& a, const uint4& b, floatx16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

GLM52_DEV uint4 ldg_nt(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

GLM52_DEV uint4 ldg(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// 16-byte store with the non-temporal hint: for outputs no kernel of this launch reads.
GLM52_DEV void stg_nt(uint16_t* p, const uint4& v) {
  u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

// Raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3 for raw,
// range-checked 32-bit loads): a load whose offset is out of range returns zero without
// touching memory.
GLM52_DEV __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

GLM52_DEV uint4 ldb(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

typedef __attribute__((address_space(3))) uint16_t lds_u16_t;

// One direct 16-byte-per-lane load into LDS: lane l's 16 bytes land at byte `lds_base`
// + 16 l (lds_base wave-uniform).  Issued from inline assembly so that the compiler's
// wait-count pass, which loses track of these loads across the K loop's back edge and
// would then drain every stage, leaves them alone: the kernel orders them with explicit
// vmcnt waits before the barrier that publishes a stage.  m0 is set inside the statement
// and nothing else in these kernels keeps a value in it.
GLM52_DEV void dma16(const uint16_t* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(gptr)
               : "memory");
}

// The same load with a wave-uniform 64-bit base (SGPRs) and a 32-bit per-lane byte offset:
// lane l's 16 bytes at base + voff land at byte `lds_base` + 16 l.
GLM52_DEV void dma16s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(sbase)
               : "memory");
}

// dma16s with the non-temporal hint: for streams read once (decode weights), so that they
// do not displace cached data.
GLM52_DEV void dma16s_nt(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(voff), "s"(sbase)
               : "memory");
}

GLM52_DEV uint32_t lds_addr(const uint16_t* p) {
  return (uint32_t)(uintptr_t)(const lds_u16_t*)p;
}

// s_waitcnt vmcnt(n): every older vector-memory load of this wave has completed.
#define GLM52_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(%0)" : : "n"(n) : "memory")

// The packed weight layout (glm52_pack_w512).  W row (inside its 32-row group) held at
// LDS row p of the 512-row tile; load slot w * 8 + i of a tile holds 16 rows of one 32-row
// group (rows phi32(p) + 8 (i % 2) for p = 0 .. 15), each 32-k stage of them as 1 KB, lane
// l's 16 bytes being row p = l / 4, 8-k chunk (l % 4) ^ ((p / 4) % 4).  A tile's 32 slots
// (nk = K / 32 stages each) are interleaved 1 KB at a time in groups of kPackG = 8: stage j
// of slot s sits at KB (s / 8) * 8 nk + 8 j + s % 8 of the tile.  A slot's stages are 8 KB
// apart, as a row-major W's 1 KB row runs are a row stride apart, which the decode weight
// stream reads faster than one contiguous run (T = 256: w13 2224 -> 2081 us, w2 1380 ->
// 1319 us; interleaving 16 slots measured the same); a 512-row tile's stage is four 8 KB
// runs.
GLM52_DEV int phi32(int p) { return ((p >> 2) & 1) * 16 + (p >> 3) * 4 + (p & 3); }
// elements of one packed slot and of one packed 512-row tile, for nk 32-k stages
__host__ __device__ inline int64_t packed_slot_elems(int nk) { return (int64_t)nk * 512; }
__host__ __device__ inline int64_t packed_tile_elems(int nk) { return 32 * packed_slot_elems(nk); }
// stage j of slot s sits at element packed_slot_off(nk, s) + j * kPackStride of its tile
constexpr int kPackG = 8;
constexpr int kPackStride = kPackG * 512;  // elements between a slot's successive stages
__host__ __device__ inline int64_t packed_slot_off(int nk, int s) {
  return ((int64_t)(s / kPackG) * nk * kPackG + s % kPackG) * 512;
}

struct GemmArgs {
  const uint16_t* A;
  int64_t sam;
  int a_div;
  const uint16_t* W;
  int64_t swe;
  int64_t swn;
  int gu_off;  // row offset of the `up` half inside W[e] (gated only)
  uint16_t* C;
  int64_t scm;
  const float* topw;  // per flat token (weighted only)
  const int32_t* sti;
  const int32_t* eids;
  const int32_t* ntp;
  int BM;  // block size of the layout
  int n_out;
  int K;
  int num_valid;
  int group_m;  // tiled mapping: row blocks per swizzle group
  int stage_k;  // wide mapping: k per LDS stage (64: a three-buffer ring)
  // stream mapping: an extra expert (the shared one) whose rows are tokens 0 .. x_rows - 1
  // of its own input Ax, with weights Wx ([N, K] like W[e]) and its own output Cx;
  // x_rows = 0: none
  const uint16_t* Ax;
  int64_t sax;
  const uint16_t* Wx;
  uint16_t* Cx;
  int64_t scx;
  int x_rows;
  int a_bytes;   // stream mapping: bytes of A (and of Ax) its token rows span
  int ax_bytes;
  // contiguous-run mapping in routing mode (decode, T <= 4 tokens): the layout is not read
  // from sti / eids / ntp but derived in every workgroup from the router logits; the
  // routing (ids, weights) and the layout are written out for the kernels that follow
  const float* r_logits;
  int64_t r_sl;
  const float* r_bias;
  int r_T, r_E, r_topk, r_norm_prob;
  float r_scale;
  float* r_topw;
  int64_t r_stw;
  int32_t* r_topi;
  int64_t r_sti;
  int32_t* r_sorted;
  int32_t* r_eids;
  int32_t* r_ntp;
  int r_capacity;
  // 512-row tile mapping: W packed per (expert, tile, 32-k stage) in the order the tile's
  // loads fill LDS (glm52_pack_w512); null: W is read in place
  const uint16_t* Wp;
  // 512-row tile mapping, plain and unweighted only: epilogue 0 = bf16(acc); 1 =
  // bf16(acc + R); 2 = C32 += acc (+ R if R); 3 = C32 = acc (fp32 partial sums): the
  // dense GEMM + residual of o_proj
  int epi;
  const uint16_t* R;
  int64_t srm;
  float* C32;
  // > 0: the atomic expert merge (FUSE_MERGE): the bf16 result of flat token f is added
  // with packed bf16 atomics into row f / merge_topk of C (non-gated only; the 512-row
  // tile and contiguous-run mappings); 0: the result is stored into row f
  int merge_topk;
  // 512-row tile mapping: the set of per-XCD item counters this launch deals its items
  // from (set by the launcher)
  int deal_set;
  // 512-row tile mapping: null, or a record of 4 words per workgroup (start and end on the
  // 100 MHz wall clock, items run, XCD) written at the workgroup's end (glm52_debug_item_trace)
  unsigned long long* wg_trace;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// C[0..1] += (lo, hi) as one packed bf16 atomic (global_atomic_pk_add_bf16); p 4-byte
// aligned.  Each element's add rounds to bf16, in whatever order the adds land.
GLM52_DEV void atomic_add_bf16x2(uint16_t* p, float lo, float hi) {
  __builtin_amdgcn_global_atomic_fadd_v2bf16(reinterpret_cast<bf16x2_t*>(p),
                                             __builtin_bit_cast(bf16x2_t, pack_bf16x2(lo, hi)));
}

// The wide LDS-tiled mapping fed by direct global -> LDS loads (moe_gemm_wide.hip):
// returns GLM52_EUNSUPPORTED for a block size or shape it has no instance for.
int launch_wide(const GemmArgs& a, int capacity, bool gated, bool weighted, hipStream_t st);

// The 512-row W tile mapping (moe_gemm_wide.hip): GLM52_EUNSUPPORTED for a block size or
// shape it has no instance for.
int launch_wide512(const GemmArgs& a, int capacity, bool gated, bool weighted, hipStream_t st);

// Packs W for launch_wide512 (GemmArgs::Wp): E experts, n_out outputs (gated: the `gate`
// rows n and the `up` rows gate_up_offset + n), K = k.  Returns the bytes written, or a
// negative error for a shape the 512-row mapping has no instance for (out = null: size only).
int64_t pack_wide512(const uint16_t* w, int64_t swe, int64_t swn, int E, int n_out, int k,
                     int gate_up_offset, bool gated, uint16_t* out, hipStream_t st,
                     int64_t swk = 1);

// The decode mapping that streams W as contiguous 1 KB row runs (moe_gemm_runs.hip): block
// size 16; an optional extra expert (x_rows > 0) as in the stream mapping; `route`: the
// routing mode (gated, unweighted, with the extra expert).
int launch_runs(const GemmArgs& a, int capacity, bool gated, bool weighted, bool route,
                hipStream_t st);

}  // namespace glm52
