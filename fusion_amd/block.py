"""The GLM-5.2 MoE FFN block on one MI355X, composed from the drop-in launchers.

Chain (`glm52/bench/bench_layer.py:395-481`, configuration `H_f3_f10` without o_proj, with
the routing computed live instead of frozen, and the tail fused):

    1. ResAdd+RMSNorm           h = bf16(x + r), y = RMSNorm(h)           add_rmsnorm
    2. router logits            fp64-exact; decode: a wave per gate row   router (launch 1)
    3. sigmoid + biased top-8   ids, weights                              router (launch 2)
    4. dispatch/align           sglang layout, count kept on the device  moe_align
                                (T <= 16: 3 and 4 are one launch, router_topk_align;
                                 T <= 4: 1-2 are one launch, decode_norm_logits, and
                                 3-6 are one launch, moe_gemm_route_shared, which
                                 derives the routing from the logits in every workgroup)
    5. routed w13 + SwiGLU      act[8T, I]                                moe_gemm (gated)
    6. shared w13 + SwiGLU      act_s[T, I]                               moe_gemm (gated, E=1)
    7. routed w2 (weighted)     Y[8T, H] = w * (act . w2^T)               moe_gemm
    8. shared w2                s[T, H]                                   moe_gemm (E=1)
                                (5+6 and 7+8 are one launch each: moe_gemm_shared when
                                 streaming weights, moe_gemm_packed_shared at prefill)
    9. merge + ResAdd           out = bf16(sum_k Y[t, k] + h + s)         block_merge
                                (T = 1: 7-9 are one launch, down_token_major:
                                 out = bf16(sum_k w * (act . w2^T) + shared + h), fp32
                                 over all experts, one rounding -- the reference's
                                 token-major strategy #9(b))

The expert weights are held in one resident layout, packed once at load (`PackedExperts`,
`pack_w512`: every 32-k stage of a 512-row W tile as 32 KB of contiguous memory), which
every block size reads: the prefill tiles stage whole 32 KB stages, the decode weight
stream reads each load slot's 1 KB of 16 rows x 32 k.  The GEMMs compute the same bits as
on the row-major weights (the token-major tail sums in another order).  `pack=False` (or
a `variant`) reads the row-major weights in place instead.

Every buffer is allocated once in the constructor (destination passing, as the
reference's `LayerProblem` does, `glm52/bench/bench_layer.py:316-346`); `forward` only
launches kernels on torch's current stream and never syncs, so it can be captured in a
HIP graph (`capture()`), which is how decode is meant to run.
"""

from __future__ import annotations

import torch

from . import config as C
from . import _lib
from .dispatch import (DECODE_FRONT_MAX_T, capacity, decode_norm_logits_into,
                       align_workspace, moe_align_block_size_into, route_gateup_shared_into,
                       route_gateup_shared_packed_into, topk_align_into)
from .kernels import add_rmsnorm as KN
from .kernels import moe_down_merge as KD
from .kernels import norm_router as KR
from .kernels.moe_gateup import moe_gemm, moe_gemm_packed_shared, moe_gemm_shared, pack_w512

BF16 = torch.bfloat16

# token count from which the router runs the bounded bf16 logits on the gate rows
BOUNDED_ROUTER_MIN_T = 1024


def default_block_m(T: int) -> int:
    """Layout block size per regime: 16-row slices stream weights while each expert sees
    a handful of rows; 64- or 128-row blocks of the wide LDS-tiled mapping once rows per
    expert reach the tens, and 256-row blocks (256 x 256 tiles) once they pass a hundred,
    so that most experts' rows fit one block and each W tile is streamed by one workgroup."""
    rows_per_expert = T * C.TOPK / C.E
    if rows_per_expert <= 12:
        return 16
    if rows_per_expert <= 48:
        return 64
    if rows_per_expert <= 100:
        return 128
    return 256


def default_shared_block_m(T: int) -> int:
    """Block size of the shared expert's one-expert layout over T rows."""
    if T <= 12:
        return 16
    return 64 if T <= 512 else 128


def shared_layout(T: int, block_m: int, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Layout of the single shared expert over T tokens: what
    `moe_align_block_size(zeros(T, 1), BM, 1)` returns (`glm52/bench/bench_layer.py:384-388`),
    padded to the worst-case capacity like the routed layout."""
    cap = capacity(T, block_m, 1)
    sti = torch.full((cap,), T, dtype=torch.int32)
    sti[:T] = torch.arange(T, dtype=torch.int32)
    total = ((T + block_m - 1) // block_m) * block_m
    eids = torch.full((cap // block_m,), -1, dtype=torch.int32)
    eids[: total // block_m] = 0
    ntp = torch.tensor([total], dtype=torch.int32)
    return sti.to(device), eids.to(device), ntp.to(device)


def packed_shapes_ok(T: int, H: int, I: int, block_m: int | None = None,
                     shared_block_m: int | None = None) -> bool:
    """Whether the packed mappings cover this block: whole 512-row tiles (I % 256 gated,
    H % 512 plain); the weight stream (block size 16) reads 512-k stages (H, I % 512); the
    prefill tiles 64-k pairs of stages; the token-major tail K = I of 1024 or 2048."""
    bm = block_m or default_block_m(T)
    sbm = shared_block_m or default_shared_block_m(T)
    if I % 256 or H % 512:
        return False
    if bm == 16:
        return I % 512 == 0 and (T > DECODE_FRONT_MAX_T or I in (1024, 2048))
    return bm in (64, 128, 256) and sbm in (64, 128, 256) and I % 64 == 0


class PackedExperts:
    """The routed experts' and the shared expert's w13 and w2 in the one resident layout
    (`pack_w512`), packed once at load; the row-major tensors may be freed afterwards.
    w13 [E, 2I, H] (`gate` rows 0 .. I-1, `up` rows I .. 2I-1), w2 [E, H, I]; the shared
    ones [1, 2I, H] / [2I, H] and [1, H, I] / [H, I]."""

    def __init__(self, w13, w2, w13s, w2s):
        _lib.require_gpu(w13, w2, w13s, w2s)
        self.E, I2, self.H = w13.shape
        self.I = I2 // 2
        w13s = w13s if w13s.dim() == 3 else w13s.unsqueeze(0)
        w2s = w2s if w2s.dim() == 3 else w2s.unsqueeze(0)
        if tuple(w2.shape) != (self.E, self.H, self.I) or tuple(w13s.shape) != (1, I2, self.H) \
                or tuple(w2s.shape) != (1, self.H, self.I):
            raise ValueError("expert weight shapes must be [E, 2I, H], [E, H, I], "
                             "[1, 2I, H], [1, H, I]")
        self.device = w13.device
        self.w13 = pack_w512(w13, self.I, self.I, True)
        self.w2 = pack_w512(w2, self.H, 0, False)
        self.w13s = pack_w512(w13s, self.I, self.I, True)
        self.w2s = pack_w512(w2s, self.H, 0, False)

    def nbytes(self) -> int:
        return sum(t.numel() * 2 for t in (self.w13, self.w2, self.w13s, self.w2s))


class MoEBlock:
    def __init__(self, T: int, w_norm, wgt, bias, w13, w2=None, w13s=None, w2s=None,
                 block_m: int | None = None, shared_block_m: int | None = None,
                 variant: str | None = None, eps: float = C.RMS_NORM_EPS,
                 scale: float = C.ROUTED_SCALING_FACTOR, pack: bool = True,
                 token_major: bool | None = None):
        """w13 is either the row-major [E, 2I, H] tensor (with w2, w13s, w2s) or a
        `PackedExperts` (w2, w13s, w2s None).  Row-major weights are packed here unless
        `pack=False` or a `variant` asks for the in-place mappings; the block keeps one
        layout only, never both."""
        _lib.require_gpu(w_norm, wgt, bias)
        self.experts = None
        if isinstance(w13, PackedExperts):
            if w2 is not None or w13s is not None or w2s is not None or variant is not None:
                raise ValueError("with PackedExperts pass no other weights and no variant")
            self.experts = w13
        elif pack and variant is None and packed_shapes_ok(T, w13.shape[2], w13.shape[1] // 2,
                                                           block_m, shared_block_m):
            self.experts = PackedExperts(w13, w2, w13s, w2s)
        if self.experts is not None:
            P = self.experts
            dev = P.device
            self.E, self.H, self.I = P.E, P.H, P.I
            self.w13 = self.w2 = self.w13s = self.w2s = None  # not held
        else:
            _lib.require_gpu(w13, w2, w13s, w2s)
            dev = w13.device
            self.E, I2, self.H = w13.shape
            self.I = I2 // 2
            self.w13, self.w2 = w13, w2
            self.w13s = w13s if w13s.dim() == 3 else w13s.unsqueeze(0)
            self.w2s = w2s if w2s.dim() == 3 else w2s.unsqueeze(0)
        self.T = T
        self.topk = C.TOPK
        self.w_norm, self.wgt, self.bias = w_norm, wgt, bias
        self.eps, self.scale = eps, scale
        self.bm = block_m or default_block_m(T)
        self.sbm = shared_block_m or default_shared_block_m(T)
        self.variant = variant

        H, I, E, R = self.H, self.I, self.E, T * self.topk
        self.h = torch.empty(T, H, dtype=BF16, device=dev)
        self.y = torch.empty(T, H, dtype=BF16, device=dev)
        self.logits = torch.empty(T, E, dtype=torch.float32, device=dev)
        self.topw = torch.empty(T, self.topk, dtype=torch.float32, device=dev)
        self.topi = torch.empty(T, self.topk, dtype=torch.int32, device=dev)
        cap = capacity(R, self.bm, E)
        self.sti = torch.empty(cap, dtype=torch.int32, device=dev)
        self.eids = torch.empty(cap // self.bm, dtype=torch.int32, device=dev)
        self.ntp = torch.empty(1, dtype=torch.int32, device=dev)
        self.align_ws = align_workspace(R, E, dev)
        self.act = torch.empty(R, I, dtype=BF16, device=dev)
        self.ybuf = torch.empty(R, H, dtype=BF16, device=dev)
        self.act_s = torch.empty(T, I, dtype=BF16, device=dev)
        self.s_out = torch.empty(T, H, dtype=BF16, device=dev)
        self.out = torch.empty(T, H, dtype=BF16, device=dev)
        self.ssti, self.seids, self.sntp = shared_layout(T, self.sbm, dev)
        self.cfg_r = {"BLOCK_M": self.bm, "variant": variant}
        self.cfg_s = {"BLOCK_M": self.sbm, "variant": variant}
        # decode: the [E, H] gate rows feed the one-row-per-wave router, and top-k plus
        # the dispatch layout run as one single-workgroup launch; at T <= 4 norm and
        # logits are one launch and the routing is derived inside the w13 launch
        self.decode = T <= 16 and T * self.topk <= 256
        # weight-streaming decode runs the shared expert inside the routed launches
        self.shared_fused = self.bm == 16
        self.front_fused = T <= DECODE_FRONT_MAX_T and self.shared_fused
        # decode tail at T = 1: the token-major down GEMV sums the token's experts, the
        # shared expert and h in one launch (no Y rows, no merge launch); from T = 2 the
        # weight stream with paired slots + the merge is faster (whole blocks: T = 2 221.2
        # against 228.7 us, T = 3 305.7 against 321.6 us; T = 1 128.2 against 125.3 us)
        self.token_major = (self.front_fused and variant is None and T == 1) \
            if token_major is None else bool(token_major)
        if self.token_major and not self.shared_fused:
            # the token-major tail reads the shared expert's activations, which only the
            # weight-streaming w13 launch (block size 16) writes before the tail
            raise ValueError("token_major needs the weight-streaming layout (block size 16, "
                             f"T <= 384); T={T} runs block size {self.bm}")
        # the gate as rows [E, H]: decode streams a wave per row; above, the router runs
        # the bounded bf16 logits with the exact rule on each token's candidates
        self.gate_rows = wgt.t().contiguous()
        self.wgt_rows = self.gate_rows.t()  # its [H, E] view
        need = max(KR.workspace_bytes(T, H, E), KR.select_workspace_bytes(T, H, E))
        self.router_ws = torch.empty(max(need, 8), dtype=torch.uint8, device=dev)
        self.cfg_topk = {"correction_bias": bias, "scale": scale, "workspace": self.router_ws}
        self.graph = None
        # the GEMMs read the packed layout at every block size (16: the weight stream over
        # load slots; 64, 128, 256: the 512-row and 256-row tiles)
        self.packed = self.experts is not None
        if self.packed and not (self.shared_fused or (self.bm in (64, 128, 256)
                                                      and self.sbm in (64, 128, 256))):
            raise ValueError(f"no packed mapping for block sizes {self.bm} / {self.sbm}")

    # ---- the chain -------------------------------------------------------------------
    def front_end(self, x, r):
        T = self.T
        if self.front_fused:
            # norm + logits here; the routing is derived inside the w13 launch (experts())
            decode_norm_logits_into(x, r, self.w_norm, self.h, self.y, self.gate_rows,
                                    self.logits, self.eps)
            return
        KN.fused_add_rmsnorm(x, r, self.w_norm, self.h, self.y, {"eps": self.eps})
        if self.decode:
            # gate rows streamed once by 64 workgroups; top-k and layout in one launch
            KR.router_gemm(self.y, self.wgt_rows, self.logits, self.cfg_topk)
            topk_align_into(self.logits, self.topw, self.topi, self.cfg_topk, self.bm, self.E,
                            self.sti, self.eids, self.ntp)
        else:
            # from ~1k tokens the bounded bf16 router on the gate rows; below, the fp64
            # MFMA router on the [H, E] gate is the faster of the two (same ids, weights)
            gw = self.wgt_rows if T >= BOUNDED_ROUTER_MIN_T else self.wgt
            KR.router(self.y, gw, self.logits, self.topw, self.topi, self.cfg_topk)
            moe_align_block_size_into(self.topi, self.bm, self.E, self.sti, self.eids, self.ntp,
                                      self.align_ws)

    def w13_step(self):
        """Steps 5 and 6 (at T <= 4 also 3 and 4): the routed and the shared expert in one
        launch (weight streaming and packed prefill), else the routed launch (the shared one
        is in w2_step)."""
        T, I, R = self.T, self.I, self.T * self.topk
        P = self.experts
        if self.front_fused and self.packed:
            route_gateup_shared_packed_into(self.logits, self.cfg_topk, self.topw, self.topi,
                                            self.sti, self.eids, self.ntp, self.y, P.w13,
                                            self.act, self.y, P.w13s, self.act_s)
        elif self.front_fused:
            route_gateup_shared_into(self.logits, self.cfg_topk, self.topw, self.topi, self.sti,
                                     self.eids, self.ntp, self.y, self.w13, self.act, self.y,
                                     self.w13s, self.act_s)
        elif self.packed:
            # routed and shared w13 in one launch: the weight stream at block size 16, the
            # tiles above (the shared expert's items after each XCD's routed ones)
            moe_gemm_packed_shared(self.y, self.topk, P.w13, self.act, None, self.sti,
                                   self.eids, self.ntp, R, I, True, self.cfg_r, self.y,
                                   P.w13s, self.act_s)
        elif self.shared_fused:
            moe_gemm_shared(self.y, self.topk, self.w13, self.act, None, self.sti, self.eids,
                            self.ntp, R, I, I, True, self.cfg_r, self.y, self.w13s, self.act_s)
        else:
            moe_gemm(self.y, self.topk, self.w13, self.act, None, self.sti, self.eids, self.ntp,
                     R, I, I, True, self.cfg_r)

    def w2_step(self):
        T, H, I, R = self.T, self.H, self.I, self.T * self.topk
        if self.packed:
            P = self.experts
            moe_gemm_packed_shared(self.act, 1, P.w2, self.ybuf, self.topw.view(-1), self.sti,
                                   self.eids, self.ntp, R, H, False, self.cfg_r, self.act_s,
                                   P.w2s, self.s_out)
            return
        if self.shared_fused:
            moe_gemm_shared(self.act, 1, self.w2, self.ybuf, self.topw.view(-1), self.sti,
                            self.eids, self.ntp, R, H, 0, False, self.cfg_r, self.act_s, self.w2s,
                            self.s_out)
            return
        moe_gemm(self.y, 1, self.w13s, self.act_s, None, self.ssti, self.seids, self.sntp,
                 T, I, I, True, self.cfg_s)
        moe_gemm(self.act, 1, self.w2, self.ybuf, self.topw.view(-1), self.sti, self.eids,
                 self.ntp, R, H, 0, False, self.cfg_r)
        moe_gemm(self.act_s, 1, self.w2s, self.s_out, None, self.ssti, self.seids, self.sntp,
                 T, H, 0, False, self.cfg_s)

    def experts(self):
        self.w13_step()
        self.w2_step()

    def tail(self):
        """Steps 7-9: the token-major GEMV at decode sizes, else w2 then the merge."""
        if self.token_major and self.packed:
            P = self.experts
            KD.launch_down_token_major_packed(self.act, P.w2, self.out, self.topw, self.topi,
                                              self.h, self.topk, True, self.act_s, P.w2s)
            return
        if self.token_major:
            KD.launch_down_token_major(self.act, self.w2, self.out, self.topw, self.topi, self.h,
                                       self.topk, {}, True, self.act_s, self.w2s)
            return
        self.w2_step()
        self.merge()

    def merge(self):
        y3 = self.ybuf.view(self.T, self.topk, self.H)
        _lib.call("glm52_block_merge", _lib.ptr(y3), y3.stride(0), y3.stride(1),
                  _lib.ptr(self.h), self.h.stride(0), _lib.ptr(self.s_out), self.s_out.stride(0),
                  _lib.ptr(self.out), self.out.stride(0), self.T, self.H, _lib.stream())

    def forward(self, x: torch.Tensor, r: torch.Tensor) -> torch.Tensor:
        if x.shape != (self.T, self.H) or r.shape != (self.T, self.H):
            raise ValueError(f"expected x, r of shape {(self.T, self.H)}")
        self.front_end(x, r)
        self.w13_step()
        self.tail()
        return self.out

    __call__ = forward

    # ---- HIP graph -----------------------------------------------------------------
    def capture(self, x: torch.Tensor, r: torch.Tensor) -> None:
        """Capture `forward(x, r)` (x and r are read in place on every replay)."""
        self._gx, self._gr = x, r
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.forward(x, r)  # warm the launch path outside capture
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.forward(x, r)
        self.graph = g

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.out
