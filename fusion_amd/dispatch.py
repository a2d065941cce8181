"""Token -> expert dispatch layout on the device, drop-in for
`glm52/reference.py::moe_align_block_size` (`glm52/reference.py:85-128`).

Returns the same three tensors (sorted_token_ids, expert_ids, num_tokens_post_padded)
with the same values in their first `num_tokens_post_padded` slots / blocks.  The
difference is the buffer size: the reference syncs to the host and allocates exactly
`num_tokens_post_padded` slots, while this version keeps the count on the device and
returns worst-case buffers (`capacity(numel, BM, E)` slots; the tail holds the sentinel
`numel` and the trailing blocks hold expert id -1).  The grouped GEMMs stop at the
device-side count, so nothing here syncs and the block can be captured in a graph.
`exact=True` trims to the reference's exact sizes (one device->host sync).
"""

from __future__ import annotations

import torch

from . import _lib


def capacity(numel: int, block_m: int, num_experts: int) -> int:
    """Worst-case padded slot count, rounded up to a whole block."""
    need = numel + num_experts * (block_m - 1)
    return ((need + block_m - 1) // block_m) * block_m


def align_workspace(numel: int, num_experts: int, device) -> torch.Tensor | None:
    """The chunk histograms of the multi-workgroup layout (None below 16384 ids, where one
    workgroup builds it as fast)."""
    n = _lib.query("glm52_moe_align_workspace_bytes", int(numel), int(num_experts))
    return torch.empty(n // 4, dtype=torch.int32, device=device) if n else None


def moe_align_block_size_into(topk_ids, block_m, num_experts, sorted_token_ids, expert_ids,
                              num_tokens_post_padded, workspace="auto"):
    """Destination-passing form (the caller owns the three buffers).  `workspace`: an int32
    buffer from `align_workspace`, "auto" (allocated here when the input is large), or
    None (the single-workgroup build, same result)."""
    _lib.require_gpu(topk_ids, sorted_token_ids, expert_ids, num_tokens_post_padded)
    if topk_ids.dtype != torch.int32 or not topk_ids.is_contiguous():
        raise ValueError("topk_ids must be a contiguous int32 tensor")
    cap = sorted_token_ids.numel()
    if expert_ids.numel() * block_m != cap:
        raise ValueError("expert_ids must hold capacity / block_m entries")
    if isinstance(workspace, str):
        workspace = align_workspace(topk_ids.numel(), num_experts, topk_ids.device)
    if workspace is not None:
        _lib.require_gpu(workspace)
        if workspace.dtype != torch.int32 or not workspace.is_contiguous():
            raise ValueError("the workspace is a contiguous int32 tensor")
    _lib.call(
        "glm52_moe_align_ws", _lib.ptr(topk_ids), topk_ids.numel(), int(block_m),
        int(num_experts), cap, _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids),
        _lib.ptr(num_tokens_post_padded), _lib.ptr(workspace),
        0 if workspace is None else workspace.numel() * 4, _lib.stream(),
    )


def moe_align_block_size(topk_ids: torch.Tensor, block_m: int, num_experts: int,
                         exact: bool = False):
    dev = topk_ids.device
    ids = topk_ids.to(torch.int32).contiguous()
    cap = capacity(ids.numel(), block_m, num_experts)
    sti = torch.empty(cap, dtype=torch.int32, device=dev)
    eids = torch.empty(cap // block_m, dtype=torch.int32, device=dev)
    ntp = torch.empty(1, dtype=torch.int32, device=dev)
    moe_align_block_size_into(ids, block_m, num_experts, sti, eids, ntp)
    if exact:
        total = int(ntp.item())
        return sti[:total].clone(), eids[: total // block_m].clone(), ntp
    return sti, eids, ntp


def topk_align_into(logits, topw, topi, cfg, block_m, num_experts, sorted_token_ids, expert_ids,
                    num_tokens_post_padded):
    """Decode fast path: the router's sigmoid + biased top-k (as `topk_only`) and the
    dispatch layout in one single-workgroup launch.  Needs T * top_k <= 256."""
    bias = cfg.get("correction_bias")
    _lib.require_gpu(logits, topw, topi, bias, sorted_token_ids, expert_ids,
                     num_tokens_post_padded)
    T, E = logits.shape
    cap = sorted_token_ids.numel()
    if expert_ids.numel() * block_m != cap:
        raise ValueError("expert_ids must hold capacity / block_m entries")
    _lib.call(
        "glm52_router_topk_align", _lib.ptr(logits), logits.stride(0), _lib.ptr(bias),
        _lib.ptr(topw), topw.stride(0), _lib.ptr(topi), topi.stride(0), T, E, topi.shape[1],
        float(cfg.get("scale", 2.5)), int(bool(cfg.get("NORM_PROB", True))), int(block_m), cap,
        _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded),
        _lib.stream(),
    )


DECODE_FRONT_MAX_T = 4


def decode_front_into(x, r, w_norm, h1, y, gate_rows, cfg, logits, topw, topi, block_m,
                      sorted_token_ids, expert_ids, num_tokens_post_padded, counter):
    """Decode front end in one launch (T <= 4): ResAdd + RMSNorm, router logits from the
    contiguous [E, H] gate rows, biased top-k and the dispatch layout -- the chain
    `fused_add_rmsnorm` -> `router_gemm` -> `topk_only` -> `moe_align_block_size`, with
    bit-identical outputs.  `counter` is an int32 device tensor that is zero before the
    first call and is left zero by every call."""
    bias = cfg.get("correction_bias")
    _lib.require_gpu(x, r, w_norm, h1, y, gate_rows, logits, topw, topi, bias,
                     sorted_token_ids, expert_ids, num_tokens_post_padded, counter)
    T, H = x.shape
    E = gate_rows.shape[0]
    if gate_rows.shape[1] != H or gate_rows.stride(1) != 1 or gate_rows.dtype != torch.bfloat16:
        raise ValueError("gate_rows must be the contiguous [E, H] bf16 gate")
    if counter.dtype != torch.int32:
        raise ValueError("counter must be an int32 device tensor")
    cap = sorted_token_ids.numel()
    if expert_ids.numel() * block_m != cap:
        raise ValueError("expert_ids must hold capacity / block_m entries")
    _lib.call(
        "glm52_decode_front", _lib.ptr(x), x.stride(0), _lib.ptr(r), r.stride(0),
        _lib.ptr(w_norm), _lib.ptr(h1), h1.stride(0), _lib.ptr(y), y.stride(0),
        _lib.ptr(gate_rows), gate_rows.stride(0), _lib.ptr(bias), _lib.ptr(logits),
        logits.stride(0), _lib.ptr(topw), topw.stride(0), _lib.ptr(topi), topi.stride(0), T, H,
        E, topi.shape[1], float(cfg.get("eps", 1e-5)), float(cfg.get("scale", 2.5)),
        int(bool(cfg.get("NORM_PROB", True))), int(block_m), cap, _lib.ptr(sorted_token_ids),
        _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded), _lib.ptr(counter),
        _lib.stream(),
    )


def decode_norm_logits_into(x, r, w_norm, h1, y, gate_rows, logits, eps: float = 1e-5):
    """ResAdd + RMSNorm and the router logits of T <= 4 tokens in one launch (the first
    part of `decode_front_into`): `fused_add_rmsnorm` -> `router_gemm`, bit-identical."""
    _lib.require_gpu(x, r, w_norm, h1, y, gate_rows, logits)
    T, H = x.shape
    E = gate_rows.shape[0]
    if gate_rows.shape[1] != H or gate_rows.stride(1) != 1 or gate_rows.dtype != torch.bfloat16:
        raise ValueError("gate_rows must be the contiguous [E, H] bf16 gate")
    _lib.call(
        "glm52_decode_norm_logits", _lib.ptr(x), x.stride(0), _lib.ptr(r), r.stride(0),
        _lib.ptr(w_norm), _lib.ptr(h1), h1.stride(0), _lib.ptr(y), y.stride(0),
        _lib.ptr(gate_rows), gate_rows.stride(0), _lib.ptr(logits), logits.stride(0), T, H, E,
        float(eps), _lib.stream(),
    )


def route_gateup_shared_into(logits, cfg, topw, topi, sorted_token_ids, expert_ids,
                             num_tokens_post_padded, a, w13, act, a_shared, w13_shared, act_shared):
    """Decode (T <= 4): `topk_only` -> `moe_align_block_size` (block size 16) ->
    `launch_gateup(fused=True)` for the routed experts and the shared expert, in one launch
    that derives the routing from the logits (no grid-wide wait).  Writes topw, topi and the
    three layout tensors like `topk_align_into`, act[f] for the routed slots and act_shared."""
    bias = cfg.get("correction_bias")
    _lib.require_gpu(logits, topw, topi, bias, sorted_token_ids, expert_ids,
                     num_tokens_post_padded, a, w13, act, a_shared, w13_shared, act_shared)
    T, E = logits.shape
    k = topi.shape[1]
    ws = w13_shared[0] if w13_shared.dim() == 3 else w13_shared
    for t, n in ((a, "a"), (w13, "w13"), (act, "act"), (a_shared, "a_shared"), (ws, "w13_shared"),
                 (act_shared, "act_shared")):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError(f"{n} must be bf16 and contiguous along its last dim")
    if ws.shape != w13.shape[1:] or ws.stride(0) != w13.stride(1):
        raise ValueError("w13_shared must have the routed experts' [2I, H] shape and row stride")
    I = act.shape[1]
    _lib.call(
        "glm52_moe_gemm_route_shared", _lib.ptr(logits), logits.stride(0), _lib.ptr(bias), T, E,
        k, float(cfg.get("scale", 2.5)), int(bool(cfg.get("NORM_PROB", True))), _lib.ptr(topw),
        topw.stride(0), _lib.ptr(topi), topi.stride(0), _lib.ptr(sorted_token_ids),
        _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded), sorted_token_ids.numel(),
        _lib.ptr(a), a.stride(0), _lib.ptr(w13), w13.stride(0), w13.stride(1), I, _lib.ptr(act),
        act.stride(0), _lib.ptr(a_shared), a_shared.stride(0), _lib.ptr(ws), _lib.ptr(act_shared),
        act_shared.stride(0), I, a.shape[1], _lib.stream(),
    )


def route_gateup_shared_packed_into(logits, cfg, topw, topi, sorted_token_ids, expert_ids,
                                    num_tokens_post_padded, a, w13_packed, act, a_shared,
                                    w13_shared_packed, act_shared):
    """`route_gateup_shared_into` on packed weights (`pack_w512(w13, I, I, True)` and the
    same of the [1, 2I, H] shared w13): the same routing, layout and bits."""
    from .kernels.moe_gateup import check_packed
    bias = cfg.get("correction_bias")
    _lib.require_gpu(logits, topw, topi, bias, sorted_token_ids, expert_ids,
                     num_tokens_post_padded, a, w13_packed, act, a_shared, w13_shared_packed,
                     act_shared)
    T, E = logits.shape
    k = topi.shape[1]
    for t, n in ((a, "a"), (w13_packed, "w13_packed"), (act, "act"), (a_shared, "a_shared"),
                 (w13_shared_packed, "w13_shared_packed"), (act_shared, "act_shared")):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError(f"{n} must be bf16 and contiguous along its last dim")
    I, H = act.shape[1], a.shape[1]
    check_packed(w13_packed, I, H, True)
    check_packed(w13_shared_packed, I, H, True)
    if w13_packed.numel() * 2 < E * _lib.query("glm52_packed_w512_bytes", 1, I, H, 1):
        raise ValueError(f"w13_packed holds fewer than the router's {E} experts")
    _lib.call(
        "glm52_moe_gemm_route_shared_packed", _lib.ptr(logits), logits.stride(0), _lib.ptr(bias),
        T, E, k, float(cfg.get("scale", 2.5)), int(bool(cfg.get("NORM_PROB", True))),
        _lib.ptr(topw), topw.stride(0), _lib.ptr(topi), topi.stride(0),
        _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded),
        sorted_token_ids.numel(), _lib.ptr(a), a.stride(0), _lib.ptr(w13_packed), _lib.ptr(act),
        act.stride(0), _lib.ptr(a_shared), a_shared.stride(0), _lib.ptr(w13_shared_packed),
        _lib.ptr(act_shared), act_shared.stride(0), I, H, _lib.stream(),
    )
