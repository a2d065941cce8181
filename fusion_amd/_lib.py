"""ctypes binding of `libglm52_hip.so` (the C-ABI declared in `include/glm52_hip.h`).

The library is loaded after torch, so it binds to the HIP runtime torch loaded (same
SONAME) and shares torch's device pointers and streams.  There is no fallback: if the
library is missing, every launcher raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libglm52_hip.so"

_P = c_void_p
_I = c_int
_L = c_int64
_F = c_float

# name -> argument types (every entry point returns int: 0 on success)
SIGNATURES: dict[str, list] = {
    "glm52_add_rmsnorm": [_P, _P, _P, _P, _P, _L, _L, _L, _L, _I, _I, _F, _I, _I, _I, _P],
    "glm52_router_logits": [_P, _L, _P, _L, _L, _I, _P, _L, _P, _L, _I, _I, _I, _P],
    "glm52_router": [_P, _L, _P, _L, _L, _I, _P, _L, _P, _L, _P, _P, _L, _P, _L, _I, _I, _I, _I,
                     _F, _I, _P],
    "glm52_router_topk_align": [_P, _L, _P, _P, _L, _P, _L, _I, _I, _I, _F, _I, _I, _I, _P, _P,
                                _P, _P],
    "glm52_router_topk": [_P, _L, _P, _P, _L, _P, _L, _I, _I, _I, _F, _I, _P],
    "glm52_moe_align": [_P, _I, _I, _I, _I, _P, _P, _P, _P],
    "glm52_moe_align_ws": [_P, _I, _I, _I, _I, _P, _P, _P, _P, _L, _P],
    "glm52_moe_align_noalloc": [_P, _I, _I, _I, _I, _P, _P, _P, _P],
    "glm52_decode_front": [_P, _L, _P, _L, _P, _P, _L, _P, _L, _P, _L, _P, _P, _L, _P, _L, _P, _L,
                           _I, _I, _I, _I, _F, _F, _I, _I, _I, _P, _P, _P, _P, _P],
    "glm52_decode_norm_logits": [_P, _L, _P, _L, _P, _P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I,
                                 _F, _P],
    "glm52_moe_gemm_route_shared": [_P, _L, _P, _I, _I, _I, _F, _I, _P, _L, _P, _L, _P, _P, _P,
                                    _I, _P, _L, _P, _L, _L, _I, _P, _L, _P, _L, _P, _P, _L, _I,
                                    _I, _P],
    "glm52_moe_gemm_route_shared_packed": [_P, _L, _P, _I, _I, _I, _F, _I, _P, _L, _P, _L, _P,
                                           _P, _P, _I, _P, _L, _P, _P, _L, _P, _L, _P, _P, _L,
                                           _I, _I, _P],
    "glm52_moe_gemm": [_P, _L, _I, _P, _L, _L, _I, _P, _L, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                       _I, _I, _P],
    "glm52_moe_gemm_shared": [_P, _L, _I, _P, _L, _L, _I, _P, _L, _P, _P, _P, _P, _I, _I, _I,
                              _P, _L, _P, _P, _L, _I, _I, _I, _I, _P],
    "glm52_pack_w512": [_P, _L, _L, _I, _I, _I, _I, _I, _P, _P],
    "glm52_moe_gemm_packed": [_P, _L, _I, _P, _P, _L, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                              _P],
    "glm52_moe_gemm_packed_shared": [_P, _L, _I, _P, _P, _L, _P, _P, _P, _P, _I, _I, _I, _P, _L,
                                     _P, _P, _L, _I, _I, _I, _I, _P],
    "glm52_oproj_pack": [_P, _L, _L, _I, _I, _I, _P, _P],
    "glm52_oproj_gemm": [_P, _L, _P, _L, _L, _P, _I, _P, _L, _P, _L, _I, _I, _I, _I, _P, _L,
                         _P],
    "glm52_cast_add": [_P, _I, _L, _P, _L, _P, _L, _I, _I, _P],
    "glm52_rstd": [_P, _L, _I, _I, _F, _P, _P, _I, _P],
    "glm52_prenorm_router_rows": [_P, _L, _P, _L, _P, _F, _P, _L, _P, _I, _I, _I, _P],
    "glm52_router_logits_rstd": [_P, _L, _P, _L, _L, _I, _P, _P, _L, _P, _L, _I, _I, _I, _P],
    "glm52_router_rstd": [_P, _L, _P, _L, _L, _I, _P, _P, _L, _P, _L, _P, _P, _L, _P, _L, _I, _I,
                          _I, _I, _F, _I, _P],
    "glm52_moe_down_merge": [_P, _L, _P, _L, _L, _P, _P, _L, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                             _I, _P],
    "glm52_down_token_major": [_P, _L, _P, _L, _L, _P, _P, _L, _I, _I, _P, _L, _P, _L, _P, _L, _P,
                               _L, _I, _I, _I, _P],
    "glm52_down_token_major_packed": [_P, _L, _P, _P, _P, _L, _I, _I, _P, _L, _P, _P, _L, _P,
                                      _L, _I, _I, _I, _P],
    "glm52_silu_and_mul": [_P, _L, _P, _L, _I, _I, _P],
    "glm52_moe_sum": [_P, _L, _L, _P, _L, _P, _L, _I, _I, _I, _I, _P],
    "glm52_resadd": [_P, _L, _P, _L, _P, _L, _I, _I, _P],
    "glm52_merge_resadd": [_P, _L, _L, _P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I,
                           _P],
    "glm52_block_merge": [_P, _L, _L, _P, _L, _P, _L, _P, _L, _I, _I, _P],
    "glm52_selftest_mfma_layout": [_P, _P],
    "glm52_stream_read": [_P, _L, _I, _I, _P, _P],
    "glm52_debug_item_trace": [_P, _L],
}

# name -> (argument types, return type) for entry points that do not return a status
QUERIES: dict[str, tuple[list, type]] = {
    "glm52_router_workspace_bytes": ([_I, _I, _I], c_int64),
    "glm52_router_select_workspace_bytes": ([_I, _I, _I], c_int64),
    "glm52_moe_align_workspace_bytes": ([_I, _I], c_int64),
    "glm52_packed_w512_bytes": ([_I, _I, _I, _I], c_int64),
    "glm52_oproj_workspace_bytes": ([_I, _I, _I], c_int64),
    "glm52_oproj_packed_bytes": ([_I, _I], c_int64),
    "glm52_oproj_splits": ([_I, _I, _I], c_int),
}

ERRORS = {-1: "invalid argument", -2: "unsupported argument combination"}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -m fusion_amd.build` "
                "(the MI355X path has no CPU fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = c_int
        for name, (argtypes, restype) in QUERIES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        why = ERRORS.get(rc, f"hipError {rc}")
        raise RuntimeError(f"{name} failed: {why}")


def query(name: str, *args):
    return getattr(lib(), name)(*args)


def stream() -> int:
    """The HIP stream torch is issuing on (launches are ordered after torch's work)."""
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the MI355X kernels take device tensors only (no CPU fallback)")
