"""Router GEMM + sigmoid top-8, drop-in for `glm52/kernels/norm_router.py:251-389`.

Entry points and destination-passing contract are the reference's.  Semantics follow
`glm52/reference.py:46-79` (not the Triton `topk_only`, which never applied the
correction bias, `glm52/kernels/norm_router.py:221-238`):

    logits = x2 . Wg          (fp64-accumulated, rounded once to fp32 -- order independent)
    s      = sigmoid(logits)  (fp64, rounded once to fp32)
    ids    = top-k of s + correction_bias, descending, lower index first on ties
    w      = s[ids] / max(sum s[ids], 1e-20) * scale

`cfg` keys read: `scale` (2.5, as `norm_router.py:307`), `NORM_PROB` (True), and the one
addition this path needs, `correction_bias` (an fp32 [E] device tensor, or None).  The
fused norm+router variants measured 0.21-0.68x in the reference and are provided as the
composition of the two kernels they fuse, so callers keep working.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import add_rmsnorm as _an

HIDDEN = 6144
NUM_EXPERTS = 256
TOP_K = 8


def wgt_from_gate(gate_w: torch.Tensor) -> torch.Tensor:
    """[E, H] (nn.Linear) -> [H, E], the layout the router kernel reads."""
    return gate_w.t().contiguous()


def workspace_bytes(T: int, H: int = HIDDEN, E: int = NUM_EXPERTS) -> int:
    """Bytes of fp64 split-K partials the [H, E]-contiguous mapping needs at T tokens
    (0 when K is not split; the transposed-gate mapping needs none)."""
    return int(_lib.query("glm52_router_workspace_bytes", T, H, E))


def select_workspace_bytes(T: int, H: int = HIDDEN, E: int = NUM_EXPERTS) -> int:
    """Bytes the router (logits + top-k) on the transposed gate view needs at T tokens: the
    sums of squares behind its error bound, and its K-split partials (0 at T <= 16)."""
    return int(_lib.query("glm52_router_select_workspace_bytes", T, H, E))


def _workspace(T, H, E, device, cfg, wgt=None, select=False):
    rows = wgt is not None and wgt.stride(0) == 1
    if rows:
        need = select_workspace_bytes(T, H, E) if select and wgt.dtype == torch.bfloat16 else 0
    else:
        need = workspace_bytes(T, H, E)
    ws = cfg.get("workspace")
    if need and (ws is None or ws.numel() * ws.element_size() < need):
        ws = torch.empty(need, dtype=torch.uint8, device=device)
    return ws, need


def _check_router_operands(x2, wgt, logits):
    """`wgt` is [H, E]: either contiguous (the reference's kernel layout, read by the fp64
    MFMA mapping) or the transposed view of a contiguous [E, H] gate (`gate.t()`, read
    one expert row per wave -- the fast mapping at decode)."""
    _lib.require_gpu(x2, wgt, logits)
    if wgt.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("router weight must be bf16 or fp32")
    if x2.stride(-1) != 1 or logits.stride(-1) != 1:
        raise ValueError("router operands must be contiguous along their last dim")
    if wgt.stride(1) != 1 and wgt.stride(0) != 1:
        raise ValueError("router weight must be [H, E] contiguous or a transposed [E, H] gate")


def router_gemm(x2, wgt, logits, cfg):
    """logits[T, E] fp32 = x2 . wgt; `cfg["workspace"]` may hold the split-K scratch."""
    _check_router_operands(x2, wgt, logits)
    T, H = x2.shape
    if T == 0:
        return  # an empty batch: nothing to launch
    E = wgt.shape[1]
    ws, need = _workspace(T, H, E, x2.device, cfg, wgt)
    _lib.call(
        "glm52_router_logits", _lib.ptr(x2), x2.stride(0), _lib.ptr(wgt), wgt.stride(0),
        wgt.stride(1), int(wgt.dtype == torch.float32), _lib.ptr(logits), logits.stride(0),
        _lib.ptr(ws), need, T, H, E, _lib.stream(),
    )


def router(x2, wgt, logits, topw, topi, cfg):
    """router_gemm + topk_only in two launches (split-K partials reduced inside top-k).

    With the transposed gate view (`gate.t()`, bf16) and T > 16 the logits run on bf16
    MFMA with a proven error bound and only each token's candidate experts (those the
    bound cannot exclude from the top k) get the exact fp64 logit: ids and weights equal
    the exact rule's bit for bit; `logits` is exact for the candidates (every selected
    expert among them) and within the bound elsewhere."""
    _check_router_operands(x2, wgt, logits)
    _lib.require_gpu(topw, topi)
    bias = cfg.get("correction_bias")
    if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous()):
        raise ValueError("correction_bias must be a contiguous fp32 tensor")
    T, H = x2.shape
    if T == 0:
        return
    E = wgt.shape[1]
    ws, need = _workspace(T, H, E, x2.device, cfg, wgt, select=True)
    _lib.call(
        "glm52_router", _lib.ptr(x2), x2.stride(0), _lib.ptr(wgt), wgt.stride(0), wgt.stride(1),
        int(wgt.dtype == torch.float32), _lib.ptr(logits), logits.stride(0), _lib.ptr(ws), need,
        _lib.ptr(bias), _lib.ptr(topw), topw.stride(0), _lib.ptr(topi), topi.stride(0), T, H, E,
        topi.shape[1], float(cfg.get("scale", 2.5)), int(bool(cfg.get("NORM_PROB", True))),
        _lib.stream(),
    )


def topk_only(logits, topw, topi, cfg):
    _lib.require_gpu(logits, topw, topi)
    bias = cfg.get("correction_bias")
    if bias is not None:
        _lib.require_gpu(bias)
        if bias.dtype != torch.float32 or not bias.is_contiguous():
            raise ValueError("correction_bias must be a contiguous fp32 tensor")
    T, E = logits.shape
    if T == 0:
        return
    k = topi.shape[1]
    _lib.call(
        "glm52_router_topk", _lib.ptr(logits), logits.stride(0), _lib.ptr(bias), _lib.ptr(topw),
        topw.stride(0), _lib.ptr(topi), topi.stride(0), T, E, k, float(cfg.get("scale", 2.5)),
        int(bool(cfg.get("NORM_PROB", True))), _lib.stream(),
    )


# ---- unfused pieces (norm kernels of fusion #4/#5) -----------------------------------
def rmsnorm_only(x, w, x2, cfg):
    _an.norm_only(x, w, x2, cfg)


def add_rmsnorm_only(x, res, w, h1, x2, cfg):
    _an.fused_add_rmsnorm(x, res, w, h1, x2, cfg)


# ---- "fused" names, composed from the two kernels ------------------------------------
def fused_norm_router(x, w, x2, wgt, logits, cfg):
    _an.norm_only(x, w, x2, cfg)
    router_gemm(x2, wgt, logits, cfg)


def fused_norm_router_no_x2(x, w, x2, wgt, logits, cfg):
    """The reference's attribution-only variant (`glm52/kernels/norm_router.py:376-383`):
    the router logits of norm(x) without storing x2.  The normalised rows go to a scratch
    buffer (`cfg["x2_scratch"]`, else a temporary); `x2` is left untouched."""
    scratch = cfg.get("x2_scratch")
    if scratch is None:
        scratch = torch.empty_like(x)
    _an.norm_only(x, w, scratch, cfg)
    router_gemm(scratch, wgt, logits, cfg)


def fused_add_norm_router(x, res, w, h1, x2, wgt, logits, cfg):
    _an.fused_add_rmsnorm(x, res, w, h1, x2, cfg)
    router_gemm(x2, wgt, logits, cfg)


def _logits_scratch(T, wgt, cfg):
    lg = cfg.get("logits_buf")
    if lg is None:
        lg = torch.empty(T, wgt.shape[1], device=wgt.device, dtype=torch.float32)
    return lg


def fused_norm_router_topk(x, w, x2, wgt, topw, topi, cfg):
    _an.norm_only(x, w, x2, cfg)
    lg = _logits_scratch(x.shape[0], wgt, cfg)
    router_gemm(x2, wgt, lg, cfg)
    topk_only(lg, topw, topi, cfg)


def fused_add_norm_router_topk(x, res, w, h1, x2, wgt, topw, topi, cfg):
    _an.fused_add_rmsnorm(x, res, w, h1, x2, cfg)
    lg = _logits_scratch(x.shape[0], wgt, cfg)
    router_gemm(x2, wgt, lg, cfg)
    topk_only(lg, topw, topi, cfg)
