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


def moe_align_block_size_into(topk_ids, block_m, num_experts, sorted_token_ids, expert_ids,
                              num_tokens_post_padded):
    """Destination-passing form (the caller owns the three buffers)."""
    _lib.require_gpu(topk_ids, sorted_token_ids, expert_ids, num_tokens_post_padded)
    if topk_ids.dtype != torch.int32 or not topk_ids.is_contiguous():
        raise ValueError("topk_ids must be a contiguous int32 tensor")
    cap = sorted_token_ids.numel()
    if expert_ids.numel() * block_m != cap:
        raise ValueError("expert_ids must hold capacity / block_m entries")
    _lib.call(
        "glm52_moe_align", _lib.ptr(topk_ids), topk_ids.numel(), int(block_m), int(num_experts),
        cap, _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids),
        _lib.ptr(num_tokens_post_padded), _lib.stream(),
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
