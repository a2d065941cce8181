"""CPU tests of the routing fixtures written by the reference's own chain
(`glm52/reference.py:28-33` add_rmsnorm -> `:46-79` router -> `:85-128`
moe_align_block_size, run by tests/golden/make_golden.py) at every token count the
block's GPU parity test runs: the oracle's device rule (order-independent statistic and
logits) must give the reference's ids and layouts bit for bit, and its weights within
the fp32 rounding of the reference's torch arithmetic.  The GPU block test checks the
device against the same fixtures.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from fusion_amd.problem import front_end
from oracle import glm52_oracle as O

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
from make_golden import BLOCK_MS, ROUTING_CASES, i32_sha, routing_path  # noqa: E402


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def load_routing(T: int, bias: str) -> dict:
    """The fixture of one case as plain numpy values (ids widened to int32)."""
    g = np.load(routing_path(T, bias))
    d = {k: g[k] for k in g.files}
    d["topk_ids"] = d["topk_ids"].astype(np.int32)
    return d


@pytest.mark.parametrize("T,bias", ROUTING_CASES)
def test_device_rule_reproduces_reference_routing(T, bias):
    g = load_routing(T, bias)
    fe = front_end(T, bias=bias)
    assert list(g["in_sha"]) == [sha(fe.x), sha(fe.r), sha(fe.w_norm), sha(fe.gate), sha(fe.bias)]

    y, h = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    assert sha(h) == str(g["h_sha"])
    # the reference's y is the exact-statistic y with a few elements one bf16 ulp away
    yu = u16(y).reshape(-1).copy()
    pos, val = g["y_patch_pos"], g["y_patch_val"]
    assert (np.abs(yu[pos].astype(np.int32) - val.astype(np.int32)) == 1).all()
    # a row's rstd differs by an fp32 ulp between the two summation orders in a few rows;
    # every other row is identical
    assert np.unique(pos // fe.x.shape[1]).size <= max(1, T // 50)
    yu[pos] = val
    assert hashlib.sha256(yu.view(np.int16).tobytes()).hexdigest() == str(g["y_sha"])

    # ids bit for bit from the device rule's own y; weights within the fp32 rounding of
    # the reference's torch arithmetic when fed the reference's y, and within the effect
    # of the one-ulp y differences otherwise
    _, w, ids = O.router_exact(y, fe.wgt, fe.bias.numpy())
    assert np.array_equal(ids, g["topk_ids"])
    ref_w = g["topk_weights"]
    y_ref = torch.from_numpy(yu.view(np.int16).reshape(y.shape)).view(torch.bfloat16)
    _, w_r, ids_r = O.router_exact(y_ref, fe.wgt, fe.bias.numpy())
    assert np.array_equal(ids_r, g["topk_ids"])
    assert (np.abs(w_r - ref_w) <= 2e-6 * np.abs(ref_w)).all()
    assert (np.abs(w - ref_w) <= 5e-4 * np.abs(ref_w)).all()

    # the three layouts, bit for bit (digests of the reference's exact-size tensors)
    for bm in BLOCK_MS:
        sti, eids, ntp = O.moe_align_block_size(ids, bm, 256)
        assert int(ntp[0]) == int(g[f"ntp_{bm}"])
        assert i32_sha(sti) == str(g[f"sti_sha_{bm}"])
        assert i32_sha(eids) == str(g[f"eids_sha_{bm}"])
        if f"sti_{bm}" in g:
            assert np.array_equal(sti, g[f"sti_{bm}"])
            assert np.array_equal(eids, g[f"eids_{bm}"])


def test_zipf_fixture_skew():
    """Configuration 4's routing, as the reference computes it: the literal
    0.5 * (e + 1)^-1.1 bias gives a top-20 % expert share near 0.37 (not the ~0.6 of
    the configuration's prose), so the load statistics the bench reports are pinned."""
    g = load_routing(8192, "zipf")
    counts = np.bincount(g["topk_ids"].reshape(-1), minlength=256)
    top = np.sort(counts)[::-1][: 256 // 5].sum() / counts.sum()
    assert counts.sum() == 8192 * 8
    assert 0.30 < top < 0.45
    assert counts.max() > 20 * counts.min()
