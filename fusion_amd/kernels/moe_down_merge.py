"""Fusions #8/#9 -- grouped w2 GEMM + expert merge (+ residual add), drop-in for
`glm52/kernels/moe_down_merge.py:427-577`.

  launch_down(..., fuse_merge=False): c[f, :] = bf16(topk_w[f] * (a[f] . w2[e]^T))
      (`MUL_ROUTED_WEIGHT=True`, `moe_down_merge.py:155-158`); a rows by flat token f
  launch_moe_sum(c3, out, residual, topk, cfg, add_residual):
      out = bf16(sum_k fp32 c3[t, k] (+ fp32 residual))
  launch_resadd(x, r, o, cfg): o = bf16(fp32 x + fp32 r)
  launch_seed(o, r, cfg, from_residual): o = r, or zeros

  launch_down(..., fuse_merge=True): c[f // top_k, :] += bf16(topk_w[f] * (a[f] . w2[e]^T))
      with packed bf16 atomics into the pre-seeded [T, H] output (strategy (a))
  launch_down_token_major(a, w2, out, topk_weights, topk_ids, residual, top_k, cfg,
                          add_residual): out = bf16(sum_k w * (a . w2^T) (+ residual)),
      one token per workgroup column slice, fp32 over all experts, one rounding
      (strategy (b))
"""

from __future__ import annotations

import torch

from .. import _lib
from .moe_gateup import check_layout, moe_gemm


def smem_bytes(cfg: dict) -> int:
    bm = cfg["BLOCK_M"]
    if bm == 16 or cfg.get("variant") == "stream":
        return 4096
    return 2 * (bm + 128) * (64 + 8) * 2 + 4 * bm


def launch_down(a, w2, c, topk_weights_flat, sorted_token_ids, expert_ids,
                num_tokens_post_padded, num_valid_tokens, top_k, cfg, fuse_merge: bool):
    """a: [rows, I] bf16.  w2: [E, H, I] bf16.
    c: [rows, H] when fuse_merge=False, else the pre-seeded [T, H] output, to which every
    routed row's bf16 result is added with packed bf16 atomics (`moe_down_merge.py:
    160-169`); `cfg["w2_packed"]` (`moe_gateup.pack_w512(w2, H, 0, False)`) may supply
    the packed weights the 64/128-row mapping reads."""
    if not fuse_merge:
        moe_gemm(a, 1, w2, c, topk_weights_flat, sorted_token_ids, expert_ids,
                 num_tokens_post_padded, num_valid_tokens, w2.shape[1], 0, False, cfg)
        return
    wp = cfg.get("w2_packed")
    _lib.require_gpu(a, w2, c, topk_weights_flat, sorted_token_ids, expert_ids,
                     num_tokens_post_padded, wp)
    if a.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16 or c.dtype != torch.bfloat16:
        raise ValueError("down GEMM operands are bf16")
    if a.stride(1) != 1 or w2.stride(2) != 1 or c.stride(1) != 1:
        raise ValueError("a rows, w2 rows and c rows must be contiguous")
    if topk_weights_flat.dtype != torch.float32 or not topk_weights_flat.is_contiguous():
        raise ValueError("topk weights must be a contiguous fp32 tensor")
    H, K = w2.shape[1], w2.shape[2]
    if a.shape[1] != K or c.shape[1] != H or c.shape[0] * top_k < num_valid_tokens:
        raise ValueError(f"shape mismatch: a {tuple(a.shape)}, w2 {tuple(w2.shape)}, "
                         f"c {tuple(c.shape)} (the merged [T, H] output), top_k={top_k}")
    bm = int(cfg["BLOCK_M"])
    cap = check_layout(sorted_token_ids, expert_ids, num_tokens_post_padded, bm)
    if num_valid_tokens == 0:
        return
    _lib.call(
        "glm52_moe_down_merge", _lib.ptr(a), a.stride(0), _lib.ptr(w2), w2.stride(0),
        w2.stride(1), _lib.ptr(wp), _lib.ptr(c), c.stride(0), _lib.ptr(topk_weights_flat),
        _lib.ptr(sorted_token_ids), _lib.ptr(expert_ids), _lib.ptr(num_tokens_post_padded),
        cap, bm, int(num_valid_tokens), int(top_k), H, K, _lib.stream(),
    )


def smem_bytes_tokmaj(cfg: dict) -> int:
    """LDS of the token-major down GEMV (`glm52/kernels/moe_down_merge.py:421-424`): none,
    every lane keeps its rows and activation chunks in registers."""
    return 0


def launch_down_token_major(a, w2, out, topk_weights, topk_ids, residual, top_k, cfg,
                            add_residual: bool, a_shared=None, w2_shared=None):
    """a: [T*top_k, I].  out: [T, H].  topk_ids/topk_weights: [T, top_k].

    out[t] = bf16(sum_k w[t, k] * (a[t*top_k + k] @ w2[ids[t, k]]^T) (+ residual[t])), one
    fp32 accumulation, one rounding (`moe_down_merge.py:479-516`).  `a_shared` [T, I] and
    `w2_shared` [H, I] (this build's extension) add a shared expert with weight 1."""
    _lib.require_gpu(a, w2, out, topk_weights, topk_ids, residual if add_residual else None,
                     a_shared, w2_shared)
    T = topk_ids.shape[0]
    E, H, K = w2.shape
    if a.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise ValueError("token-major operands are bf16")
    if a.shape[0] < T * top_k or a.shape[1] != K or tuple(out.shape) != (T, H):
        raise ValueError(f"shape mismatch: a {tuple(a.shape)}, w2 {tuple(w2.shape)}, "
                         f"out {tuple(out.shape)}, T={T}, top_k={top_k}")
    if a.stride(1) != 1 or w2.stride(2) != 1 or out.stride(1) != 1:
        raise ValueError("a rows, w2 rows and out rows must be contiguous")
    if topk_ids.dtype != torch.int32:
        topk_ids = topk_ids.to(torch.int32)
    if topk_weights.dtype != torch.float32 or topk_weights.stride(1) != 1 \
            or topk_ids.stride(1) != 1 or topk_ids.stride(0) != topk_weights.stride(0):
        raise ValueError("topk weights (fp32) and ids (int32) must share a row stride")
    res = residual if add_residual else None
    if res is not None and (tuple(res.shape) != (T, H) or res.stride(1) != 1):
        raise ValueError("residual must be [T, H] with H contiguous")
    if (a_shared is None) != (w2_shared is None):
        raise ValueError("a_shared and w2_shared go together")
    if w2_shared is not None and (tuple(w2_shared.shape[-2:]) != (H, K)
                                  or a_shared.shape[-1] != K):
        raise ValueError("shared expert shapes must be [T, I] and [H, I]")
    ws = w2_shared.reshape(H, K) if w2_shared is not None else None
    _lib.call(
        "glm52_down_token_major", _lib.ptr(a), a.stride(0), _lib.ptr(w2), w2.stride(0),
        w2.stride(1), _lib.ptr(topk_weights), _lib.ptr(topk_ids), topk_ids.stride(0),
        int(top_k), E, _lib.ptr(a_shared), a_shared.stride(0) if a_shared is not None else 0,
        _lib.ptr(ws), ws.stride(0) if ws is not None else 0, _lib.ptr(res),
        res.stride(0) if res is not None else 0, _lib.ptr(out), out.stride(0), T, H, K,
        _lib.stream(),
    )


def launch_down_token_major_packed(a, w2_packed, out, topk_weights, topk_ids, residual, top_k,
                                   add_residual: bool, a_shared=None, w2_shared_packed=None):
    """`launch_down_token_major` on packed weights (`pack_w512(w2, H, 0, False)` and, for the
    shared expert, the same of its [1, H, I] w2): the same sum, one fp32 accumulation and
    one rounding, with the adds in another order.  out: [T, H]; a: [T*top_k, I]."""
    from .moe_gateup import check_packed
    _lib.require_gpu(a, w2_packed, out, topk_weights, topk_ids,
                     residual if add_residual else None, a_shared, w2_shared_packed)
    T = topk_ids.shape[0]
    H, K = out.shape[1], a.shape[1]
    for t, n in ((a, "a"), (w2_packed, "w2_packed"), (out, "out")):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError(f"{n} must be bf16 and contiguous along its last dim")
    if a.shape[0] < T * top_k or out.shape[0] != T:
        raise ValueError(f"shape mismatch: a {tuple(a.shape)}, out {tuple(out.shape)}, "
                         f"T={T}, top_k={top_k}")
    check_packed(w2_packed, H, K, False)
    E = w2_packed.numel() * 2 // _lib.query("glm52_packed_w512_bytes", 1, H, K, 0)
    if topk_ids.dtype != torch.int32:
        topk_ids = topk_ids.to(torch.int32)
    if topk_weights.dtype != torch.float32 or topk_weights.stride(1) != 1 \
            or topk_ids.stride(1) != 1 or topk_ids.stride(0) != topk_weights.stride(0):
        raise ValueError("topk weights (fp32) and ids (int32) must share a row stride")
    res = residual if add_residual else None
    if res is not None and (tuple(res.shape) != (T, H) or res.stride(1) != 1):
        raise ValueError("residual must be [T, H] with H contiguous")
    if (a_shared is None) != (w2_shared_packed is None):
        raise ValueError("a_shared and w2_shared_packed go together")
    if w2_shared_packed is not None:
        check_packed(w2_shared_packed, H, K, False)
        if w2_shared_packed.numel() * 2 != _lib.query("glm52_packed_w512_bytes", 1, H, K, 0):
            raise ValueError("w2_shared_packed must hold one expert")
        if a_shared.shape[-1] != K or a_shared.stride(-1) != 1:
            raise ValueError("a_shared must be [T, I] with I contiguous")
    _lib.call(
        "glm52_down_token_major_packed", _lib.ptr(a), a.stride(0), _lib.ptr(w2_packed),
        _lib.ptr(topk_weights), _lib.ptr(topk_ids), topk_ids.stride(0), int(top_k), E,
        _lib.ptr(a_shared), a_shared.stride(0) if a_shared is not None else 0,
        _lib.ptr(w2_shared_packed), _lib.ptr(res), res.stride(0) if res is not None else 0,
        _lib.ptr(out), out.stride(0), T, H, K, _lib.stream(),
    )


def launch_moe_sum(c3, out, residual, topk, cfg, add_residual: bool):
    """c3: [T, topk, H] (or a [rows, H] view).  out: [T, H]."""
    _lib.require_gpu(c3, out, residual if add_residual else None)
    T, Hd = out.shape
    if c3.dim() == 2:
        c3 = c3.view(T, topk, Hd)
    if c3.stride(2) != 1 or out.stride(1) != 1:
        raise ValueError("moe_sum operands must be contiguous along H")
    if T == 0:
        return
    _lib.call(
        "glm52_moe_sum", _lib.ptr(c3), c3.stride(0), c3.stride(1), _lib.ptr(out), out.stride(0),
        _lib.ptr(residual) if add_residual else None,
        residual.stride(0) if (add_residual and residual is not None) else 0,
        T, Hd, int(topk), int(bool(add_residual)), _lib.stream(),
    )


def launch_resadd(x, r, o, cfg):
    _lib.require_gpu(x, r, o)
    M, Nd = x.shape
    if M == 0:
        return
    _lib.call("glm52_resadd", _lib.ptr(x), x.stride(0), _lib.ptr(r), r.stride(0), _lib.ptr(o),
              o.stride(0), M, Nd, _lib.stream())


def launch_seed(o, r, cfg, from_residual: bool):
    """Seeding of the atomic strategy's output (`moe_down_merge.py:387-410`)."""
    _lib.require_gpu(o, r)
    if from_residual:
        o.copy_(r)
    else:
        o.zero_()
