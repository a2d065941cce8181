"""o_proj + ResAdd1 (`glm52/kernels/oproj_resadd.py`) on the GPU, through the C-ABI.

Inputs follow the reference's own benchmark (`glm52/bench/bench_f01_oproj_resadd.py:224-236`):
a ~ N(0, 0.05) [M, K], the nn.Linear weight ~ N(0, 0.02) [N, K] passed as B = W^T made
contiguous, r ~ N(0, 0.5), all bf16; its reference is torch.addmm in fp32, computed here
on the GPU.  Outputs are bf16, so each must sit within rounding of that fp32 result
(rtol 1e-2, atol 1e-2; the north-star bar is 2e-2); the fused chain and its fp32
accumulator form (SPLIT_K > 1) must agree bit for bit, and repeat launches too.
"""

from __future__ import annotations

import pytest
import torch

from fusion_amd.kernels import oproj_resadd as KO
from oracle import glm52_oracle as O

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
N_OUT = 6144


def say(*a):
    print(*a, flush=True)


def _problem(M, K, gpu, N=N_OUT):
    g = torch.Generator(device=gpu).manual_seed(1234 + M)
    a = (torch.randn(M, K, device=gpu, generator=g) * 0.05).to(BF16)
    w_nk = (torch.randn(N, K, device=gpu, generator=g) * 0.02).to(BF16)
    b = w_nk.t().contiguous()
    r = (torch.randn(M, N, device=gpu, generator=g) * 0.5).to(BF16)
    return a, w_nk, b, r


def _run(chain):
    for fn in chain:
        fn()


@pytest.mark.parametrize("M,K", [(1, 32768), (4, 32768), (16, 32768), (32, 32768),
                                 (256, 16384), (300, 16384), (2048, 16384), (2600, 16384)])
def test_oproj_chains(gpu, M, K):
    say(f"oproj M={M} K={K}")
    a, w_nk, b, r = _problem(M, K, gpu)
    N = N_OUT
    prod = a.float() @ b.float()
    ref = prod + r.float()
    out = torch.full((M, N), float("nan"), dtype=BF16, device=gpu)
    cmat = torch.empty(M, N, dtype=BF16, device=gpu)
    acc32 = torch.zeros(M, N, dtype=torch.float32, device=gpu)
    fused = {"SPLIT_K": 1}
    split = {"SPLIT_K": 2, "EPI": {}}
    _run(KO.make_fused_chain(a, b, r, out, acc32, fused))
    torch.cuda.synchronize()
    f1 = out.clone()
    torch.testing.assert_close(f1.float(), ref, rtol=1e-2, atol=1e-2)
    _run(KO.make_fused_chain(a, b, r, out, acc32, split))
    torch.cuda.synchronize()
    assert torch.equal(out, f1), "fused chain and its fp32-accumulator form differ"
    _run(KO.make_fused_chain(a, b, r, out, acc32, fused))
    torch.cuda.synchronize()
    assert torch.equal(out, f1), "repeat launch differs"
    # unfused: the product rounded to bf16 first, then the split-out add
    _run(KO.make_unfused_chain(a, b, r, out, cmat, acc32, {"SPLIT_K": 1}, {}))
    torch.cuda.synchronize()
    u1 = out.clone()
    torch.testing.assert_close(cmat.float(), prod, rtol=1e-2, atol=1e-2)
    assert torch.equal(u1, O.oproj_cast(cmat.cpu(), r.cpu()).to(gpu))
    _run(KO.make_unfused_chain(a, b, r, out, cmat, acc32, {"SPLIT_K": 2}, {}))
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float(), ref, rtol=1e-2, atol=1e-2)
    err = O.rel_err(f1.cpu(), ref.cpu())
    say(f"  rel_err fused vs fp32 {err:.2e}")
    assert err <= 2e-2


@pytest.mark.parametrize("M", [1, 64])
def test_oproj_k_major_weight_view(gpu, M):
    """B passed as the transposed view of the nn.Linear weight (K contiguous) runs on the
    packed mapping, for decode and prefill sizes."""
    K = 4096
    a, w_nk, _, r = _problem(M, K, gpu)
    b = w_nk.t()
    assert b.stride(0) == 1
    out = torch.empty(M, N_OUT, dtype=BF16, device=gpu)
    KO.gemm_launch(a, b, out, r, {}, True, False)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float(), a.float() @ b.float() + r.float(), rtol=1e-2, atol=1e-2)


def test_oproj_pack_cache_follows_in_place_updates(gpu):
    M, K = 64, 2048
    a, _, b, r = _problem(M, K, gpu)
    out = torch.empty(M, N_OUT, dtype=BF16, device=gpu)
    KO.gemm_launch(a, b, out, None, {}, False, False)
    torch.cuda.synchronize()
    first = out.clone()
    b.mul_(2.0)  # exact in bf16: the packed copy must be rebuilt
    KO.gemm_launch(a, b, out, None, {}, False, False)
    torch.cuda.synchronize()
    assert torch.equal(out, (first.float() * 2).to(BF16))


def test_oproj_rejects_wrong_output_dtype(gpu):
    a, _, b, r = _problem(1, 1024, gpu)
    with pytest.raises(ValueError, match="must be"):
        KO.gemm_launch(a, b, torch.empty(1, N_OUT, dtype=BF16, device=gpu), r, {}, True, True)


def test_oproj_pack_cache_misses_a_new_weight_at_a_freed_address(gpu):
    """A new B tensor at the address of a B that is gone, with the same shape, strides and
    version counter but other values, must be packed again: the cache holds only a weak
    reference to the tensor it packed.  (`.data` gives tensors over one memory block with
    version counters of their own, so the address and version collide by construction.)"""
    M, K, N = 64, 2048, N_OUT
    a, _, b0, _ = _problem(M, K, gpu)
    b = torch.empty(K, N, dtype=BF16, device=gpu)
    b.data.copy_(b0)  # b._version stays 0
    out = torch.empty(M, N, dtype=BF16, device=gpu)
    KO.gemm_launch(a, b, out, None, {}, False, False)
    torch.cuda.synchronize()
    first = out.clone()
    ptr, ver = b.data_ptr(), b._version
    keep = b.data  # the memory block lives on under another tensor
    del b
    b2 = keep.view(K, N)
    b2.data.copy_((torch.randn(K, N, device=gpu) * 0.02).to(BF16))
    assert b2.data_ptr() == ptr and b2._version == ver
    KO.gemm_launch(a, b2, out, None, {}, False, False)
    torch.cuda.synchronize()
    assert not torch.equal(out, first)
    torch.testing.assert_close(out.float(), a.float() @ b2.float(), rtol=1e-2, atol=1e-2)


def test_oproj_pack_cache_hits_fresh_views(gpu):
    """A caller passing a fresh view of one weight each call (`w.t()`) reuses the packed
    copy: the cache keeps the view's base alive-checked, not the short-lived view."""
    K, N = 2048, N_OUT
    bt = (torch.randn(N, K, device=gpu) * 0.02).to(BF16)
    p1 = KO.packed_weight(bt.t())
    p2 = KO.packed_weight(bt.t())
    assert p1 is p2
    bt.mul_(2.0)  # an in-place update bumps the shared version counter: repacked
    assert KO.packed_weight(bt.t()) is not p1
