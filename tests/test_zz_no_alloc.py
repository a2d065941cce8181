"""The allocation-free dispatch layout (`glm52_moe_align_noalloc`) through the C-ABI: its
sorted_token_ids, expert_ids and padded count must equal `glm52_moe_align_ws`'s (the same
layout with a caller-owned workspace) bit for bit, over the whole worst-case buffers, on
two calls in a row whose second input is smaller -- the scratch keeps the first call's
histograms, which the second must not see.  Sizes past the scratch are refused before any
launch."""

from __future__ import annotations

import pytest
import torch

from fusion_amd import _lib
from fusion_amd.dispatch import align_workspace, capacity

pytestmark = pytest.mark.gpu

E = 256


def skewed_ids(T: int, k: int, seed: int, dev) -> torch.Tensor:
    """T x k distinct expert ids per row, drawn with a Zipf-like skew (hot low experts)."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.arange(E, dtype=torch.float64) + 1.0) ** -1.1
    ids = torch.multinomial(w.expand(T, E).float(), k, replacement=False, generator=g)
    return ids.to(torch.int32).to(dev)


def layout(entry: str, ids, bm: int, ws=None):
    n = ids.numel()
    cap = capacity(n, bm, E)
    sti = torch.full((cap,), -7, dtype=torch.int32, device=ids.device)  # garbage to overwrite
    eids = torch.full((cap // bm,), -7, dtype=torch.int32, device=ids.device)
    ntp = torch.full((1,), -7, dtype=torch.int32, device=ids.device)
    args = [_lib.ptr(ids), n, bm, E, cap, _lib.ptr(sti), _lib.ptr(eids), _lib.ptr(ntp)]
    if entry == "glm52_moe_align_ws":
        args += [_lib.ptr(ws), 0 if ws is None else ws.numel() * 4]
    _lib.call(entry, *args, _lib.stream())
    return sti, eids, ntp


@pytest.mark.parametrize("bm", [16, 128])
def test_noalloc_layout_equals_workspace_layout(gpu, bm):
    for T, seed in ((8192, 1), (2048, 2), (100, 3)):  # the second and third are smaller
        print(f"noalloc layout T={T} BM={bm}", flush=True)
        ids = skewed_ids(T, 8, seed, gpu)
        got = layout("glm52_moe_align_noalloc", ids, bm)
        ws = align_workspace(ids.numel(), E, gpu)
        want = layout("glm52_moe_align_ws", ids, bm, ws)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        assert int(got[2].item()) > 0


def test_noalloc_refuses_sizes_past_its_scratch(gpu):
    n = (1 << 20) + 1
    cap = capacity(n, 16, E)
    ids = torch.zeros(8, dtype=torch.int32, device=gpu)  # never read: the call is refused
    out = torch.empty(16, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.call("glm52_moe_align_noalloc", _lib.ptr(ids), n, 16, E, cap, _lib.ptr(out),
                  _lib.ptr(out), _lib.ptr(out), _lib.stream())
    with pytest.raises(RuntimeError, match="invalid argument"):
        _lib.call("glm52_moe_align_noalloc", _lib.ptr(ids), 8, 16, E + 1, capacity(8, 16, E + 1),
                  _lib.ptr(out), _lib.ptr(out), _lib.ptr(out), _lib.stream())
