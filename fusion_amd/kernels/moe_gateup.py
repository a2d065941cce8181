"""Fusion #6 -- grouped w13 GEMM (+ SwiGLU), drop-in for `glm52/kernels/moe_gateup.py:199-266`.

`launch_gateup(a, w13, c, sorted_token_ids, expert_ids, num_tokens_post_padded,
num_valid_tokens, top_k, I, cfg, fused)` keeps the reference's arguments and layout
conventions (`glm52/kernels/REFERENCES.md:41-51`): A rows are gathered with
`sorted_token_ids // top_k`, `expert_ids[b]` owns BM-block b, padded slots hold
`num_valid_tokens` and are skipped, and the grid stops at `num_tokens_post_padded`
(read on the device).  `c` rows are indexed by the flat token id.

  fused=True : c[f, n] = bf16(silu(a . w13[e, n]) * (a . w13[e, I + n]))   ([R, I])
  fused=False: c[f, n] = bf16(a . w13[e, n])                                ([R, 2I])

`cfg["BLOCK_M"]` must equal the layout's block size (checked).  `cfg["variant"]` may
force "stream" (weight-streaming decode mapping), "tiled" (register-staged LDS tiles),
"wide" (256-row W tiles fed by direct global -> LDS loads through 64-k stages), "w512"
(512-row W tiles on the 32x32x16 MFMA, 32-k stages; 256 x 256 tiles at BM = 256) or
"runs" (the decode weight stream read as contiguous 1 KB row runs through LDS).  By
default BM = 16 runs "runs", and "stream" for the shapes it does not cover (K % 512 != 0,
output rows not 8-byte aligned); BM in {64, 128, 256} runs "w512", and at 64 and 128
"wide" for the shapes it does not cover (gated N % 256 != 0, plain N % 512 != 0); any
other BM (32) runs "tiled".
"""

from __future__ import annotations

import torch

from .. import _lib

VARIANTS = {None: 0, "auto": 0, "stream": 1, "tiled": 2, "wide": 3, "w512": 5, "runs": 6}


def check_layout(sorted_token_ids, expert_ids, num_tokens_post_padded, block_m: int) -> int:
    for t, n in ((sorted_token_ids, "sorted_token_ids"), (expert_ids, "expert_ids"),
                 (num_tokens_post_padded, "num_tokens_post_padded")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous int32 tensor")
    cap = sorted_token_ids.numel()
    if block_m <= 0 or cap % block_m or expert_ids.numel() * block_m != cap:
        raise ValueError(
            f"cfg BLOCK_M={block_m} does not match the layout "
            f"({cap} slots, {expert_ids.numel()} blocks)"
        )
    return cap


def moe_gemm(a, a_row_div, w, c, topk_weights, sorted_token_ids, expert_ids,
             num_tokens_post_padded, num_valid_tokens, n_out, gate_up_offset, gated, cfg):
    """Common launcher of the grouped GEMM (both expert GEMMs and the shared expert)."""
    _lib.require_gpu(a, w, c, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights)
    if a.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or c.dtype != torch.bfloat16:
        raise ValueError("grouped GEMM operands are bf16")
    if a.stride(1) != 1 or w.stride(2) != 1 or c.stride(1) != 1:
        raise ValueError("A rows, W rows and C rows must be contiguous")
    if topk_weights is not None and (topk_weights.dtype != torch.float32
                                     or not topk_weights.is_contiguous()):
        raise ValueError("topk weights must be a contiguous fp32 tensor")
    bm = int(cfg["BLOCK_M"])
    cap = check_layout(sorted_token_ids, expert_ids, num_tokens_post_padded, bm)
    K = a.shape[1]
    if w.shape[2] != K:
        raise ValueError(f"K mismatch: A has {K}, W has {w.shape[2]}")
    if num_valid_tokens == 0:
        return  # no routed row: nothing to compute
    variant = VARIANTS[cfg.get("variant")]
    _lib.call(
        "glm52_moe_gemm", _lib.ptr(a), a.stride(0), int(a_row_div), _lib.ptr(w), w.stride(0),
        w.stride(1), int(gate_up_offset), _lib.ptr(c), c.stride(0), _lib.ptr(topk_weights),
        _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded),
        cap, bm, int(num_valid_tokens), int(n_out), int(K), int(gated), variant, _lib.stream(),
    )


def pack_w512(w, n_out: int, gate_up_offset: int, gated: bool) -> torch.Tensor:
    """The packed copy of `w` ([E, N, K] bf16, K contiguous) read by `moe_gemm_packed`: every
    32-k stage of a 512-row W tile as 32 KB of contiguous memory (same values).  Returns a
    flat bf16 device tensor."""
    _lib.require_gpu(w)
    if w.dtype != torch.bfloat16 or w.dim() != 3 or w.stride(2) != 1:
        raise ValueError("w must be a [E, N, K] bf16 tensor with K contiguous")
    E, _, K = w.shape
    nbytes = _lib.query("glm52_packed_w512_bytes", E, int(n_out), K, int(gated))
    if nbytes < 0:
        raise ValueError(f"no 512-row tile instance for n_out={n_out}, K={K}")
    out = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=w.device)
    _lib.call("glm52_pack_w512", _lib.ptr(w), w.stride(0), w.stride(1), E, int(n_out), K,
              int(gate_up_offset), int(gated), _lib.ptr(out), _lib.stream())
    out.glm52_pack = (E, int(n_out), K, bool(gated))  # checked by moe_gemm_packed
    return out


def check_packed(w_packed, n_out: int, K: int, gated: bool) -> None:
    """Reject a packed buffer made for another shape: one from `pack_w512` must carry the
    same (n_out, K, gated); a bare buffer must hold a whole number of experts' packed W."""
    tag = getattr(w_packed, "glm52_pack", None)
    if tag is not None:
        if tag[1:] != (int(n_out), int(K), bool(gated)):
            raise ValueError(f"w_packed was packed for (n_out, K, gated) = {tag[1:]}, "
                             f"not {(int(n_out), int(K), bool(gated))}")
        return
    per = _lib.query("glm52_packed_w512_bytes", 1, int(n_out), int(K), int(gated))
    have = w_packed.numel() * 2
    if per <= 0 or have == 0 or have % per:
        raise ValueError(f"w_packed ({have} bytes) is not a whole number of experts packed "
                         f"for n_out={n_out}, K={K}, gated={bool(gated)}")


def moe_gemm_packed(a, a_row_div, w_packed, c, topk_weights, sorted_token_ids, expert_ids,
                    num_tokens_post_padded, num_valid_tokens, n_out, gated, cfg):
    """`moe_gemm` (BLOCK_M 64 or 128) on weights packed by `pack_w512`: the same bits."""
    _lib.require_gpu(a, w_packed, c, sorted_token_ids, expert_ids, num_tokens_post_padded,
                     topk_weights)
    if a.dtype != torch.bfloat16 or w_packed.dtype != torch.bfloat16 or c.dtype != torch.bfloat16:
        raise ValueError("grouped GEMM operands are bf16")
    if a.stride(1) != 1 or c.stride(1) != 1:
        raise ValueError("A rows and C rows must be contiguous")
    if topk_weights is not None and (topk_weights.dtype != torch.float32
                                     or not topk_weights.is_contiguous()):
        raise ValueError("topk weights must be a contiguous fp32 tensor")
    if not w_packed.is_contiguous():
        raise ValueError("w_packed must be contiguous")
    check_packed(w_packed, n_out, a.shape[1], gated)
    bm = int(cfg["BLOCK_M"])
    cap = check_layout(sorted_token_ids, expert_ids, num_tokens_post_padded, bm)
    if num_valid_tokens == 0:
        return
    _lib.call(
        "glm52_moe_gemm_packed", _lib.ptr(a), a.stride(0), int(a_row_div), _lib.ptr(w_packed),
        _lib.ptr(c), c.stride(0), _lib.ptr(topk_weights), _lib.ptr(sorted_token_ids),
        _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded), cap, bm, int(num_valid_tokens),
        int(n_out), a.shape[1], int(gated), _lib.stream(),
    )


def moe_gemm_packed_shared(a, a_row_div, w_packed, c, topk_weights, sorted_token_ids,
                           expert_ids, num_tokens_post_padded, num_valid_tokens, n_out, gated,
                           cfg, a_shared, w_shared_packed, c_shared):
    """`moe_gemm_packed` with the shared expert in the same launch: `w_shared_packed`
    (`pack_w512` of the [1, N, K] shared weight) applied to every row of `a_shared` (one
    row per token, no routing weight), written to `c_shared`."""
    _lib.require_gpu(a, w_packed, c, sorted_token_ids, expert_ids, num_tokens_post_padded,
                     topk_weights, a_shared, w_shared_packed, c_shared)
    for t, n in ((a, "a"), (w_packed, "w_packed"), (c, "c"), (a_shared, "a_shared"),
                 (w_shared_packed, "w_shared_packed"), (c_shared, "c_shared")):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError(f"{n} must be bf16 and contiguous along its last dim")
    if topk_weights is not None and (topk_weights.dtype != torch.float32
                                     or not topk_weights.is_contiguous()):
        raise ValueError("topk weights must be a contiguous fp32 tensor")
    if a_shared.shape[1] != a.shape[1] or c_shared.shape[0] != a_shared.shape[0]:
        raise ValueError("a_shared / c_shared rows must match (one per token)")
    check_packed(w_packed, n_out, a.shape[1], gated)
    check_packed(w_shared_packed, n_out, a.shape[1], gated)
    if getattr(w_shared_packed, "glm52_pack", (1,))[0] != 1:
        raise ValueError("w_shared_packed must hold one expert")
    bm = int(cfg["BLOCK_M"])
    cap = check_layout(sorted_token_ids, expert_ids, num_tokens_post_padded, bm)
    if num_valid_tokens == 0 and a_shared.shape[0] == 0:
        return
    _lib.call(
        "glm52_moe_gemm_packed_shared", _lib.ptr(a), a.stride(0), int(a_row_div),
        _lib.ptr(w_packed), _lib.ptr(c), c.stride(0), _lib.ptr(topk_weights),
        _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded), cap,
        bm, int(num_valid_tokens), _lib.ptr(a_shared), a_shared.stride(0),
        _lib.ptr(w_shared_packed), _lib.ptr(c_shared), c_shared.stride(0), a_shared.shape[0],
        int(n_out), a.shape[1], int(gated), _lib.stream(),
    )


def moe_gemm_shared(a, a_row_div, w, c, topk_weights, sorted_token_ids, expert_ids,
                    num_tokens_post_padded, num_valid_tokens, n_out, gate_up_offset, gated, cfg,
                    a_shared, w_shared, c_shared):
    """`moe_gemm` on the weight-streaming mapping with the shared expert in the same
    launch: `w_shared` ([1, N, K] or [N, K]) is applied to every row of `a_shared`
    (one row per token, no routing weight) and written to `c_shared`."""
    _lib.require_gpu(a, w, c, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
                     a_shared, w_shared, c_shared)
    for t, n in ((a, "a"), (w, "w"), (c, "c"), (a_shared, "a_shared"), (w_shared, "w_shared"),
                 (c_shared, "c_shared")):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError(f"{n} must be bf16 and contiguous along its last dim")
    ws = w_shared[0] if w_shared.dim() == 3 else w_shared
    if ws.shape[1:] != w.shape[2:] or ws.stride(0) != w.stride(1) or ws.shape[0] != w.shape[1]:
        raise ValueError("w_shared must have the routed experts' [N, K] shape and row stride")
    if a_shared.shape[1] != a.shape[1] or c_shared.shape[0] != a_shared.shape[0]:
        raise ValueError("a_shared / c_shared rows must match (one per token)")
    bm = int(cfg["BLOCK_M"])
    if bm != 16:
        raise ValueError("the fused shared-expert launch streams weights: BLOCK_M must be 16")
    cap = check_layout(sorted_token_ids, expert_ids, num_tokens_post_padded, bm)
    K = a.shape[1]
    if num_valid_tokens == 0 and a_shared.shape[0] == 0:
        return
    _lib.call(
        "glm52_moe_gemm_shared", _lib.ptr(a), a.stride(0), int(a_row_div), _lib.ptr(w), w.stride(0),
        w.stride(1), int(gate_up_offset), _lib.ptr(c), c.stride(0), _lib.ptr(topk_weights),
        _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded), cap,
        bm, int(num_valid_tokens), _lib.ptr(a_shared), a_shared.stride(0), _lib.ptr(ws),
        _lib.ptr(c_shared), c_shared.stride(0), a_shared.shape[0], int(n_out), int(K), int(gated),
        _lib.stream(),
    )


def smem_bytes(cfg: dict, fused: bool) -> int:
    """LDS bytes of the mapping this cfg selects (`moe_gateup.smem_bytes`'s question)."""
    bm = cfg["BLOCK_M"]
    variant = cfg.get("variant")
    if variant == "runs" or (variant is None and bm == 16):
        return 4 * 32 * 512 * 2 + 4 * 4 * 64 * 4
    if variant == "stream":
        return 8192
    if variant == "w512" or (variant is None and bm in (64, 128, 256)):
        return 5 * (256 + bm) * 32 * 2 if bm == 256 else 4 * (512 + bm) * 32 * 2
    if variant == "wide":
        return 3 * (256 + bm) * 64 * 2 + 4 * bm
    nb = 128
    return 2 * (bm + nb) * (64 + 8) * 2 + 4 * bm


def launch_gateup(a, w13, c, sorted_token_ids, expert_ids, num_tokens_post_padded,
                  num_valid_tokens, top_k, I, cfg, fused: bool):
    """`a`: [T, H] bf16.  `w13`: [E, 2I, H] bf16.  `c`: [T*top_k, I or 2I] bf16."""
    N = c.shape[1]
    if fused and N != I:
        raise ValueError(f"fused output width must be I={I}, got {N}")
    if not fused and N != 2 * I:
        raise ValueError(f"unfused output width must be 2I={2 * I}, got {N}")
    moe_gemm(a, top_k, w13, c, None, sorted_token_ids, expert_ids, num_tokens_post_padded,
             num_valid_tokens, N, I if fused else 0, fused, cfg)


def launch_silu_and_mul(x, y, cfg):
    _lib.require_gpu(x, y)
    M, two_i = x.shape
    if x.stride(1) != 1 or y.stride(1) != 1:
        raise ValueError("silu_and_mul operands must be row-contiguous")
    if M == 0:
        return
    _lib.call("glm52_silu_and_mul", _lib.ptr(x), x.stride(0), _lib.ptr(y), y.stride(0), M,
              two_i // 2, _lib.stream())
