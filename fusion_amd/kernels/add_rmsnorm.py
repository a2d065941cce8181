"""Fusion #3 -- ResAdd + RMSNorm, drop-in for `glm52/kernels/add_rmsnorm.py:234-246`.

Same entry points, same destination-passing contract (the caller allocates h1 / out),
same semantics (`glm52/reference.py:22-33`):

    h1  = bf16(fp32 x + fp32 res)
    out = bf16(fp32(bf16(h1 * rsqrt(mean(h1^2) + eps))) * fp32 w)

`cfg` may carry `eps` (default 1e-5) and `WAVE_PER_ROW` (1: a wave per row, 0: a
workgroup per row, absent: chosen from T).  The Triton mapping keys (ROWS, BLOCK_N,
num_warps, ...) are accepted and ignored.
"""

from __future__ import annotations

from .. import _lib

HIDDEN = 6144


def _check(name, t, dtype_bf16=True):
    if t is None:
        raise ValueError(f"{name} is required")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous along the hidden dim")


def _launch(x, res, w, h1, out, cfg, do_add: bool, do_norm: bool):
    _lib.require_gpu(x, res, w, h1, out)
    T, N = x.shape
    _check("x", x)
    if do_add:
        _check("res", res)
        _check("h1", h1)
    if do_norm:
        _check("w", w)
        _check("out", out)
    if T == 0:
        return  # an empty batch: nothing to launch
    mode = cfg.get("WAVE_PER_ROW")
    mode = -1 if mode is None else int(bool(mode))
    _lib.call(
        "glm52_add_rmsnorm",
        _lib.ptr(x), _lib.ptr(res), _lib.ptr(w), _lib.ptr(h1), _lib.ptr(out),
        x.stride(0), res.stride(0) if res is not None else 0,
        h1.stride(0) if h1 is not None else 0, out.stride(0) if out is not None else 0,
        T, N, float(cfg.get("eps", 1e-5)), int(do_add), int(do_norm), mode, _lib.stream(),
    )


def fused_add_rmsnorm(x, res, w, h1, out, cfg):
    """FUSED: 2 reads + 2 writes."""
    _launch(x, res, w, h1, out, cfg, do_add=True, do_norm=True)


def add_only(x, res, h1, cfg):
    """unfused kernel #1: h1 = x + res (2 reads + 1 write)."""
    _launch(x, res, None, h1, None, cfg, do_add=True, do_norm=False)


def norm_only(h1, w, out, cfg):
    """unfused kernel #2: out = rmsnorm(h1) * w (1 read + 1 write)."""
    _launch(h1, None, w, None, out, cfg, do_add=False, do_norm=True)
