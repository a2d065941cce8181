"""o_proj GEMM + residual add (ResAdd1): drop-in for `glm52/kernels/oproj_resadd.py`.

Same launchers and chain builders as the reference module:

    gemm_launch(a, b, c, r, cfg, fuse_resadd, atomic_out)   (`oproj_resadd.py:144-178`)
        c = A @ B            fuse_resadd off
        c = A @ B + r        fuse_resadd on (beta = 1, one bf16 rounding)
        c += A @ B (+ r)     atomic_out: c is an fp32 accumulator, as after the reference's
                             split-K atomics; here each element has one writer
    epilogue_launch(c, r, o, cfg, has_res)                  (`oproj_resadd.py:181-196`)
        o = bf16(c + r) or bf16(c), c bf16 or fp32
    make_fused_chain / make_unfused_chain                   (`oproj_resadd.py:199-228`)

A is [M, K] bf16, B is [K, N] bf16 with any strides (the reference passes the nn.Linear
weight transposed and made contiguous).  Decode (M <= 16, B N-contiguous) streams B
through a split-K kernel with a fixed-order reduction; every other case runs the MoE
block's 512-row tile GEMM on a packed copy of B, made on first use and cached on the
tensor's address, shape, strides and version counter while that tensor lives (an in-place
update of B re-packs; a new B at a freed B's address re-packs).
When M gives too few 512-row tiles to fill the GPU (M up to a few hundred), the K range
is cut into slices run as separate experts into fp32 partials, summed in slice order.
Triton mapping keys in `cfg` (BLOCK_M/N/K, GROUP_M, SPLIT_K, num_warps, num_stages) are
accepted and ignored, except that SPLIT_K > 1 selects the fp32-accumulator chain in the
chain builders, as in the reference.
"""

from __future__ import annotations

import weakref
from collections import OrderedDict

import torch

from .. import _lib

# key -> (weak reference to the B that was packed, packed copy)
_PACKED: "OrderedDict[tuple, tuple]" = OrderedDict()
_PACK_CACHE_SIZE = 4
# (device, stream) -> workspace; outgrown ones are kept (a captured graph may still use
# them), and each new one at least doubles, so few are ever kept
_WORKSPACE: dict = {}
_RETIRED: list = []


def smem_bytes(cfg: dict) -> int:
    """LDS bytes per workgroup of the mapping that runs: the prefill tile ring (160 KB),
    or the decode split-K kernel's staged A slice (at most 16 rows x 512 k x 4 B)."""
    return 163840 if cfg.get("BLOCK_M", 64) > 16 else 32768


def _workspace(dev, nbytes: int, cfg: dict) -> torch.Tensor:
    ws = cfg.get("workspace")
    if ws is not None:
        if ws.numel() * ws.element_size() < nbytes:
            raise ValueError(f"cfg workspace holds fewer than the {nbytes} bytes needed")
        return ws
    key = (dev.type, dev.index, _lib.stream())
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)
        grown = max(nbytes, 1 << 20, 2 * (ws.numel() if ws is not None else 0))
        ws = torch.empty(grown, dtype=torch.uint8, device=dev)
        _WORKSPACE[key] = ws
    return ws


def packed_weight(b: torch.Tensor, splits: int = 1) -> torch.Tensor:
    """The packed copy of B ([K, N] bf16, cut into `splits` K slices) the prefill mapping
    reads, cached.

    A hit needs the tensor that owns B's storage (B itself, or the tensor B is a view of)
    to be alive: while it lives its memory cannot be handed to another tensor, so an equal
    address, shape, strides and version counter mean equal contents.  A caller that passes
    a fresh view of the same weight every call (`w.t()`) keeps hitting, since the owner
    stays alive.  Once the owner is freed the entry is dead, even if a new weight later
    lands at the same address with the same version."""
    key = (b.device.index, b.data_ptr(), tuple(b.shape), tuple(b.stride()), b._version, splits)
    hit = _PACKED.get(key)
    if hit is not None:
        src = hit[0]()
        if src is not None and src.untyped_storage().data_ptr() == b.untyped_storage().data_ptr():
            _PACKED.move_to_end(key)
            return hit[1]
        del _PACKED[key]
    K, N = b.shape
    nbytes = _lib.query("glm52_oproj_packed_bytes", K, N)
    if nbytes < 0:
        raise ValueError(f"no packed layout for K={K}, N={N} (N % 512, K % 64)")
    out = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=b.device)
    _lib.call("glm52_oproj_pack", _lib.ptr(b), b.stride(0), b.stride(1), K, N, int(splits),
              _lib.ptr(out), _lib.stream())
    owner = b._base if b._base is not None else b
    _PACKED[key] = (weakref.ref(owner), out)
    while len(_PACKED) > _PACK_CACHE_SIZE:
        _PACKED.popitem(last=False)
    return out


def gemm_launch(a, b, c, r, cfg, fuse_resadd: bool, atomic_out: bool):
    """a:[M,K] b:[K,N] (strided, any layout) c:[M,N] r:[M,N] or None."""
    _lib.require_gpu(a, b, c, r if fuse_resadd else None)
    M, K = a.shape
    N = c.shape[1]
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or a.stride(1) != 1:
        raise ValueError("a must be bf16 with K contiguous and b bf16")
    if tuple(b.shape) != (K, N) or c.shape[0] != M or c.stride(1) != 1:
        raise ValueError(f"shape mismatch: a {tuple(a.shape)}, b {tuple(b.shape)}, c {tuple(c.shape)}")
    want = torch.float32 if atomic_out else torch.bfloat16
    if c.dtype != want:
        raise ValueError(f"c must be {want} (atomic_out={atomic_out})")
    res = r if fuse_resadd else None
    if res is not None and (res.dtype != torch.bfloat16 or tuple(res.shape) != (M, N)
                            or res.stride(1) != 1):
        raise ValueError("r must be a [M, N] bf16 tensor with N contiguous")
    if M == 0:
        return  # an empty batch: nothing to launch
    decode = M <= 16 and b.stride(1) == 1
    splits = 1
    if not decode and a.stride(0) == K:
        splits = _lib.query("glm52_oproj_splits", M, N, K)
    packed = None if decode else packed_weight(b, splits)
    nbytes = _lib.query("glm52_oproj_workspace_bytes", M, N, K)
    ws = _workspace(a.device, nbytes, cfg)
    _lib.call("glm52_oproj_gemm", _lib.ptr(a), a.stride(0), _lib.ptr(b), b.stride(0),
              b.stride(1), _lib.ptr(packed), int(splits), _lib.ptr(res),
              res.stride(0) if res is not None else 0, _lib.ptr(c), c.stride(0), int(atomic_out),
              M, N, K, _lib.ptr(ws), ws.numel() * ws.element_size(), _lib.stream())


def epilogue_launch(c, r, o, cfg, has_res: bool):
    """o = bf16(c + r) (has_res) or bf16(c); c is bf16 or an fp32 accumulator."""
    rr = r if has_res else None
    _lib.require_gpu(c, o, rr)
    if c.dtype not in (torch.bfloat16, torch.float32) or o.dtype != torch.bfloat16:
        raise ValueError("c must be bf16 or fp32 and o bf16")
    M, N = o.shape
    if M == 0:
        return
    cv, ov = c.view(-1, N) if c.dim() != 2 else c, o
    _lib.call("glm52_cast_add", _lib.ptr(cv), int(c.dtype == torch.float32), cv.stride(0),
              _lib.ptr(rr), rr.stride(0) if rr is not None else 0, _lib.ptr(ov), ov.stride(0),
              M, N, _lib.stream())


def make_fused_chain(a, b, r, out, acc32, cfg):
    """FUSED: h1 = A@B + residual, written straight to `out` (`oproj_resadd.py:199-213`)."""
    sk = cfg.get("SPLIT_K", 1)
    if sk == 1:
        return [lambda: gemm_launch(a, b, out, r, cfg, True, False)]
    ecfg = cfg.get("EPI", {})
    return [
        lambda: acc32.zero_(),
        lambda: gemm_launch(a, b, acc32, r, cfg, True, True),
        lambda: epilogue_launch(acc32, None, out, ecfg, False),
    ]


def make_unfused_chain(a, b, r, out, cmat, acc32, gcfg, ecfg):
    """UNFUSED: the GEMM materializes C, then the elementwise kernel writes h1 = C + r
    (`oproj_resadd.py:216-228`)."""
    sk = gcfg.get("SPLIT_K", 1)
    if sk == 1:
        return [
            lambda: gemm_launch(a, b, cmat, None, gcfg, False, False),
            lambda: epilogue_launch(cmat, r, out, ecfg, True),
        ]
    return [
        lambda: acc32.zero_(),
        lambda: gemm_launch(a, b, acc32, None, gcfg, False, True),
        lambda: epilogue_launch(acc32, r, out, ecfg, True),
    ]
