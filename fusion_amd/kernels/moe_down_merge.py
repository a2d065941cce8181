"""Fusions #8/#9 -- grouped w2 GEMM + expert merge (+ residual add), drop-in for
`glm52/kernels/moe_down_merge.py:427-577`.

  launch_down(..., fuse_merge=False): c[f, :] = bf16(topk_w[f] * (a[f] . w2[e]^T))
      (`MUL_ROUTED_WEIGHT=True`, `moe_down_merge.py:155-158`); a rows by flat token f
  launch_moe_sum(c3, out, residual, topk, cfg, add_residual):
      out = bf16(sum_k fp32 c3[t, k] (+ fp32 residual))
  launch_resadd(x, r, o, cfg): o = bf16(fp32 x + fp32 r)
  launch_seed(o, r, cfg, from_residual): o = r, or zeros

The atomic-merge epilogue (`fuse_merge=True`) and the token-major GEMV are the ranked
"next" items of this build; they raise NotImplementedError rather than run something
else.
"""

from __future__ import annotations

import torch

from .. import _lib
from .moe_gateup import moe_gemm


def smem_bytes(cfg: dict) -> int:
    bm = cfg["BLOCK_M"]
    if bm == 16 or cfg.get("variant") == "stream":
        return 4096
    return 2 * (bm + 128) * (64 + 8) * 2 + 4 * bm


def launch_down(a, w2, c, topk_weights_flat, sorted_token_ids, expert_ids,
                num_tokens_post_padded, num_valid_tokens, top_k, cfg, fuse_merge: bool):
    """a: [rows, I] bf16.  w2: [E, H, I] bf16.  c: [rows, H] (fuse_merge=False)."""
    if fuse_merge:
        raise NotImplementedError("atomic FUSE_MERGE epilogue is not part of this build yet")
    moe_gemm(a, 1, w2, c, topk_weights_flat, sorted_token_ids, expert_ids,
             num_tokens_post_padded, num_valid_tokens, w2.shape[1], 0, False, cfg)


def smem_bytes_tokmaj(cfg: dict) -> int:
    """LDS of the token-major down GEMV (`glm52/kernels/moe_down_merge.py:421-424`), which
    this build does not implement (see `launch_down_token_major`)."""
    raise NotImplementedError("token-major down GEMV is not part of this build yet")


def launch_down_token_major(a, w2, out, topk_weights, topk_ids, residual, top_k, cfg,
                            add_residual: bool):
    raise NotImplementedError("token-major down GEMV is not part of this build yet")


def launch_moe_sum(c3, out, residual, topk, cfg, add_residual: bool):
    """c3: [T, topk, H] (or a [rows, H] view).  out: [T, H]."""
    _lib.require_gpu(c3, out, residual if add_residual else None)
    T, Hd = out.shape
    if c3.dim() == 2:
        c3 = c3.view(T, topk, Hd)
    if c3.stride(2) != 1 or out.stride(1) != 1:
        raise ValueError("moe_sum operands must be contiguous along H")
    _lib.call(
        "glm52_moe_sum", _lib.ptr(c3), c3.stride(0), c3.stride(1), _lib.ptr(out), out.stride(0),
        _lib.ptr(residual) if add_residual else None,
        residual.stride(0) if (add_residual and residual is not None) else 0,
        T, Hd, int(topk), int(bool(add_residual)), _lib.stream(),
    )


def launch_resadd(x, r, o, cfg):
    _lib.require_gpu(x, r, o)
    M, Nd = x.shape
    _lib.call("glm52_resadd", _lib.ptr(x), x.stride(0), _lib.ptr(r), r.stride(0), _lib.ptr(o),
              o.stride(0), M, Nd, _lib.stream())


def launch_seed(o, r, cfg, from_residual: bool):
    """Seeding of the atomic strategy's output (`moe_down_merge.py:387-410`)."""
    _lib.require_gpu(o, r)
    if from_residual:
        o.copy_(r)
    else:
        o.zero_()
