"""Half-fused pre-norm (fusion #11b'): drop-in for `glm52/kernels/lazy_prenorm.py`.

The RMSNorm of the block's input h is not materialised for a consumer GEMM: its weight w
is folded into the consumer's weight once (`fold_weight_rowmajor` / `fold_weight_nk`, the
reference's load-time transforms, `lazy_prenorm.py:75-85`), and the per-row scale rstd is
applied to the consumer's accumulator:

    ((h * rstd) * w) @ B  ==  (h @ (w[:, None] * B)) * rstd

Launchers, with the reference's names and arguments:

    launch_rstd(x, rstd, cfg, eps)                         (`lazy_prenorm.py:371-390`)
    launch_router(a, b, c, cfg, fuse_norm, eps, sq_mode, rstd)        (`:457-489`)
        c [M, N] fp32 = (a @ b) * rstd   (rstd given, or computed here when fuse_norm);
        the logits rounded to fp32 under the router's exact rule, then one fp32 product;
        with cfg["topw"] / cfg["topi"] also their top-k (the bounded router on gate rows
        from 17 tokens: `glm52_router_rstd`)
    launch_moe_gateup(a, b, c, sorted_token_ids, expert_ids, num_tokens_post_padded,
                      num_valid_tokens, top_k, cfg, fuse_norm, eps, sq_mode, rstd)
        c [T * top_k, N] bf16 = bf16((a[f / top_k] @ b[e]^T) * rstd[f / top_k])

`fuse_norm=True` (the fully fused #11, the sum of squares inside the GEMM's k-loop) runs
fully fused for the router at T <= 4 on a gate read as rows (one launch: the statistic and
the dot in the same pass over h); elsewhere it is computed as the half-fused form, the
rstd pass first, then the consumer with the rstd epilogue -- the same values.  `sq_mode` selects among Triton reduction
strategies and is ignored.  rstd's statistic is this build's RMSNorm rule (exact squares
summed in fp64, one rounding), so it equals the rstd inside `fused_add_rmsnorm`.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import moe_gateup as _mg
from . import norm_router as _nr


def fold_weight_rowmajor(b: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """B is [K, N] (contraction dim first): scale ROW k by w[k] (one rounding)."""
    return (b.float() * w.float()[:, None]).to(b.dtype)


def fold_weight_nk(bt: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """B^T is [..., N, K] (nn.Linear / sglang w13 layout): scale COLUMN k by w[k]."""
    return (bt.float() * w.float()).to(bt.dtype)


def smem_bytes(cfg: dict) -> int:
    """LDS of the consumers that run: the router's token tile (74752 B) and the grouped
    GEMM's 512-row ring (163840 B); the rstd pass uses none."""
    return 163840


def launch_rstd(x, rstd, cfg, eps: float = 1e-5, rstd_flat=None, repeat: int = 1):
    """rstd[t] = 1 / sqrt(mean(x[t]^2) + eps) (fp32); `rstd_flat`, if given, receives each
    value `repeat` times (the per-slot scale of a grouped GEMM with top_k = repeat)."""
    _lib.require_gpu(x, rstd, rstd_flat)
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1:
        raise ValueError("x must be bf16 with its last dim contiguous")
    for t in (rstd, rstd_flat):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError("rstd buffers are contiguous fp32")
    T, N = x.shape
    _lib.call("glm52_rstd", _lib.ptr(x), x.stride(0), T, N, float(eps), _lib.ptr(rstd),
              _lib.ptr(rstd_flat), int(repeat), _lib.stream())


def launch_router(a, b, c, cfg, fuse_norm: bool, eps: float = 1e-5, sq_mode: int = 0,
                  rstd=None):
    """`a`: [M,K] bf16.  `b`: [K,N] bf16.  `c`: [M,N] fp32.

    With `cfg["topw"]` and `cfg["topi"]` ([M, k] fp32 / int32 outputs) the launch also takes
    the router's top-k of these logits (`topk_only`, with cfg's `correction_bias`, `scale`
    and `NORM_PROB`).  On a gate read as rows (`b` the transposed view of [N, K]) from 17
    tokens that runs the bounded router: ids and weights are the exact rule's bit for bit,
    and `c` is exact for each token's candidate experts (every selected one among them) and
    within the proven bound, times rstd, elsewhere."""
    M = a.shape[0]
    if M == 0:
        return  # an empty batch: nothing to launch
    if cfg.get("topw") is not None or cfg.get("topi") is not None:
        _router_topk(a, b, c, cfg, fuse_norm, eps, rstd)
        return
    if (fuse_norm or rstd is not None) and M <= 4 and b.stride(0) == 1:
        _rows_router(a, b, c, rstd, eps)
        return
    if fuse_norm and rstd is None:
        rstd = torch.empty(M, dtype=torch.float32, device=a.device)
        launch_rstd(a, rstd, cfg, eps)
    if rstd is None:
        _nr.router_gemm(a, b, c, cfg)
        return
    _nr._check_router_operands(a, b, c)
    _lib.require_gpu(rstd)
    if rstd.dtype != torch.float32 or not rstd.is_contiguous() or rstd.numel() < M:
        raise ValueError("rstd must be a contiguous fp32 tensor of M values")
    K, N = a.shape[1], b.shape[1]
    ws, need = _nr._workspace(M, K, N, a.device, cfg, b)
    _lib.call("glm52_router_logits_rstd", _lib.ptr(a), a.stride(0), _lib.ptr(b), b.stride(0),
              b.stride(1), int(b.dtype == torch.float32), _lib.ptr(rstd), _lib.ptr(c),
              c.stride(0), _lib.ptr(ws), need, M, K, N, _lib.stream())


def _router_topk(a, b, c, cfg, fuse_norm, eps, rstd):
    """Logits (times rstd when given or when `fuse_norm` asks for the statistic) and their
    top-k: `glm52_router_rstd`, or the block's router when there is no epilogue."""
    topw, topi = cfg.get("topw"), cfg.get("topi")
    if topw is None or topi is None:
        raise ValueError("cfg needs both topw and topi for the router's top-k")
    if rstd is None and not fuse_norm:
        _nr.router(a, b, c, topw, topi, cfg)
        return
    M, K = a.shape
    if rstd is None:
        rstd = torch.empty(M, dtype=torch.float32, device=a.device)
        launch_rstd(a, rstd, cfg, eps)
    _nr._check_router_operands(a, b, c)
    _lib.require_gpu(rstd, topw, topi)
    if rstd.dtype != torch.float32 or not rstd.is_contiguous() or rstd.numel() < M:
        raise ValueError("rstd must be a contiguous fp32 tensor of M values")
    bias = cfg.get("correction_bias")
    if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous()):
        raise ValueError("correction_bias must be a contiguous fp32 tensor")
    N = b.shape[1]
    ws, need = _nr._workspace(M, K, N, a.device, cfg, b, select=True)
    _lib.call("glm52_router_rstd", _lib.ptr(a), a.stride(0), _lib.ptr(b), b.stride(0),
              b.stride(1), int(b.dtype == torch.float32), _lib.ptr(rstd), _lib.ptr(c),
              c.stride(0), _lib.ptr(ws), need, _lib.ptr(bias), _lib.ptr(topw), topw.stride(0),
              _lib.ptr(topi), topi.stride(0), M, K, N, topi.shape[1],
              float(cfg.get("scale", 2.5)), int(bool(cfg.get("NORM_PROB", True))),
              _lib.stream())


def _rows_router(a, b, c, rstd, eps):
    """T <= 4 on a gate read as rows (b = the transposed view of a [N, K] gate): one launch,
    the statistic computed in the same pass when rstd is None."""
    _nr._check_router_operands(a, b, c)
    _lib.require_gpu(rstd)
    if b.dtype != torch.bfloat16:
        raise ValueError("the decode pre-norm router reads a bf16 gate")
    if rstd is not None and (rstd.dtype != torch.float32 or not rstd.is_contiguous()):
        raise ValueError("rstd must be a contiguous fp32 tensor")
    M, K = a.shape
    _lib.call("glm52_prenorm_router_rows", _lib.ptr(a), a.stride(0), _lib.ptr(b), b.stride(1),
              _lib.ptr(rstd), float(eps), _lib.ptr(c), c.stride(0), 0, M, K, b.shape[1],
              _lib.stream())


def launch_moe_gateup(a, b, c, sorted_token_ids, expert_ids, num_tokens_post_padded,
                      num_valid_tokens, top_k, cfg, fuse_norm: bool, eps: float = 1e-5,
                      sq_mode: int = 0, rstd=None):
    """`a`: [T,K] bf16.  `b`: [E,N,K] bf16.  `c`: [T*top_k, N] bf16 (gate and up, unfused)."""
    T = a.shape[0]
    N = c.shape[1]
    if T == 0:
        return
    scale = None
    if fuse_norm or rstd is not None:
        # the per-slot scale rstd[f / top_k]; from the given rstd or computed here
        scale = torch.empty(T * top_k, dtype=torch.float32, device=a.device)
        if rstd is None:
            launch_rstd(a, None, cfg, eps, rstd_flat=scale, repeat=top_k)
        else:
            scale.view(T, top_k).copy_(rstd.view(T, 1).expand(T, top_k))
    _mg.moe_gemm(a, top_k, b, c, scale, sorted_token_ids, expert_ids, num_tokens_post_padded,
                 num_valid_tokens, N, 0, False, cfg)
