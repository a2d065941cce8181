"""CPU checks of the C-ABI library and the host-side logic (no GPU calls)."""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest
import torch

from fusion_amd import _lib, block, dispatch

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols() -> list[str]:
    hdr = (ROOT / "include" / "glm52_hip.h").read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t) (glm52_\w+)\(", hdr, flags=re.M)))


def test_header_declares_every_binding():
    assert declared_symbols() == sorted(list(_lib.SIGNATURES) + list(_lib.QUERIES))


def test_router_workspace_query():
    from fusion_amd.kernels import norm_router as KR

    # K is split until 512 workgroups (two per CU) run, at most 32 ways
    assert KR.workspace_bytes(1) > 0  # decode splits K
    assert KR.workspace_bytes(8192) == 2 * 8192 * 256 * 8  # 256 token blocks x 2 K slices
    assert KR.workspace_bytes(16384) == 0  # 512 token blocks: no split
    assert KR.workspace_bytes(256) == 32 * 256 * 256 * 8  # 8 token blocks x 32 K slices


def test_align_workspace_query():
    q = lambda n, e: _lib.query("glm52_moe_align_workspace_bytes", n, e)  # noqa: E731
    # one int32 histogram of E experts per chunk of 2048 ids, from 16384 ids up
    assert q(65536, 256) == 32 * 256 * 4
    assert q(16384, 256) == 8 * 256 * 4
    assert q(16385, 160) == 9 * 160 * 4
    assert q(16383, 256) == 0 and q(2048, 256) == 0
    assert q(65536, 257) == 0 and q(65536, 0) == 0
    assert q(1 << 21, 256) == 0  # past 512 chunks: the single-workgroup build


def test_library_exports_every_declared_symbol():
    handle = _lib.lib()
    for name in declared_symbols():
        assert hasattr(handle, name), name


def test_library_binds_torch_hip_runtime():
    _lib.lib()
    maps = Path("/proc/self/maps").read_text()
    hips = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    assert len(hips) == 1, hips


def test_argument_errors_are_reported_without_a_gpu():
    # invalid sizes are rejected on the host before any launch
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.call("glm52_add_rmsnorm", None, None, None, None, None, 0, 0, 0, 0, 4, 7, 1e-5, 1,
                  1, -1, None)
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.call("glm52_moe_align", None, 8, 16, 256, 16, None, None, None, None)


def test_launchers_refuse_cpu_tensors():
    from fusion_amd.kernels import add_rmsnorm as KN

    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        KN.fused_add_rmsnorm(x, x, x[0], x, x, {})


def test_capacity_bounds_every_layout():
    from oracle import glm52_oracle as O

    rng = np.random.default_rng(2)
    for T, bm in ((1, 16), (32, 16), (256, 64), (999, 128)):
        ids = np.stack([rng.choice(256, 8, replace=False) for _ in range(T)])
        _, _, ntp = O.moe_align_block_size(ids, bm, 256)
        cap = dispatch.capacity(T * 8, bm, 256)
        assert ntp[0] <= cap and cap % bm == 0
        # worst case: every expert holds count = 1 (mod bm)
        assert dispatch.capacity(T * 8, bm, 256) >= T * 8 + 256 * (bm - 1)


def test_shared_layout_matches_reference_rule():
    from oracle import glm52_oracle as O

    for T, bm in ((1, 16), (37, 16), (300, 64)):
        sti, eids, ntp = block.shared_layout(T, bm, "cpu")
        rs, re_, rn = O.moe_align_block_size(np.zeros((T, 1), dtype=np.int32), bm, 1)
        n = int(rn[0])
        assert int(ntp[0]) == n
        assert np.array_equal(sti[:n].numpy(), rs) and np.array_equal(eids[: n // bm].numpy(), re_)
        assert (sti[n:] == T).all() and (eids[n // bm:] == -1).all()


def test_default_block_m_regimes():
    # decode streams 16-row slices; prefill uses the wide tiles' 64-, 128- and 256-row blocks
    assert block.default_block_m(1) == 16
    assert block.default_block_m(256) == 16
    assert block.default_block_m(1024) == 64
    assert block.default_block_m(2048) == 128
    assert block.default_block_m(3200) == 128
    assert block.default_block_m(4096) == 256
    assert block.default_block_m(8192) == 256
    assert [block.default_shared_block_m(T) for T in (1, 32, 256, 2048, 8192)] == [16, 64, 64,
                                                                                    128, 128]


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No CPU fallback: with the library absent every entry point raises."""
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libglm52_hip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.call("glm52_moe_align", None, 0, 16, 256, 16, None, None, None, None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.query("glm52_moe_align_workspace_bytes", 65536, 256)


def test_router_select_workspace_query():
    q = lambda t: _lib.query("glm52_router_select_workspace_bytes", t, 6144, 256)  # noqa: E731
    assert q(16) == 0  # decode keeps the exact rows mapping
    # per K slice: the gate rows' and the token rows' sums of squares; with a K split also
    # the fp32 partial logits.  32768 tokens: 256 blocks of 128 tokens, no K split
    assert q(32768) == (256 + 32768) * 4 + 256
    # 8192 tokens: 64 blocks of 128 tokens x 4 K slices
    assert q(8192) == 4 * (256 + 8192) * 4 + 256 + 4 * 8192 * 256 * 4
    # 2048 tokens: 32 blocks of 64 tokens x 8 K slices
    assert q(2048) == 8 * (256 + 2048) * 4 + 256 + 8 * 2048 * 256 * 4


def test_item_trace_hook_checks_its_buffer():
    # the record needs 256 workgroups x 4 words; null turns it off (no GPU call either way)
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.call("glm52_debug_item_trace", 4096, 8)
    _lib.call("glm52_debug_item_trace", None, 0)
