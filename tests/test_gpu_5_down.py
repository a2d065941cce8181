"""The down GEMM's merge strategies (`glm52/kernels/moe_down_merge.py`) on the GPU.

Atomic merge (fusion #8(a) / #9(a), `launch_down(fuse_merge=True)` into a seeded [T, H]
output with packed bf16 atomics): bit for bit against the oracle where the result cannot
depend on the add order (integer-valued sums; top_k = 1, where it must also equal the
unfused GEMM's row plus the seed in one rounding), and within the rel_err gate and
rtol/atol 2e-2 of the fp64 one-rounding value for random inputs, at BLOCK_M 16, 64, 128
(64 and 128 also on packed weights); eight bf16 roundings per output put the random
case on the block tolerance (2e-2) rather than the GEMMs' 1e-2.

Token-major (fusion #8(b) / #9(b)): out = bf16(sum_k w * (a . w2^T) (+ r)), fp32 over all
experts and one rounding.  Checked on sampled tokens against the fp64 oracle
(`down_token_major`) within bf16 output rounding (rtol/atol 1e-2) and the reference's
rel_err gate (2e-2, `glm52/common.py:186-200`), against the unfused chain (grouped GEMM
into [T, top_k, H], then moe_sum) within the same gate, bit for bit on a repeat launch,
with the shared-expert extension, and with ids outside [0, E) contributing nothing.
Inputs follow the reference's bench (`glm52/bench/bench_f08f09_down_merge_resadd.py`):
a ~ N(0, 1) bf16, w2 ~ N(0, 0.02), residual ~ N(0, 0.1).
"""

from __future__ import annotations

import pytest
import torch

from fusion_amd.dispatch import moe_align_block_size
from fusion_amd.kernels import moe_down_merge as KD
from fusion_amd.kernels import moe_gateup as KG
from oracle import glm52_oracle as O

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
H = 6144


def say(*a):
    print(*a, flush=True)


def _problem(T, E, K, k, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    a = torch.randn(T * k, K, device=gpu, generator=g).to(BF16)
    w2 = (torch.randn(E, H, K, device=gpu, generator=g) * 0.02).to(BF16)
    ids = torch.stack([torch.randperm(E, device=gpu, generator=g)[:k] for _ in range(T)])
    tw = torch.rand(T, k, device=gpu, generator=g) * 0.5
    r = (torch.randn(T, H, device=gpu, generator=g) * 0.1).to(BF16)
    return a, w2, ids.to(torch.int32).contiguous(), tw.contiguous(), r


def _check(got, want, what, tol=1e-2):
    torch.testing.assert_close(got.float().cpu(), want.float(), rtol=tol, atol=tol,
                               msg=lambda m: f"{what}: {m}")
    assert O.rel_err(got.cpu(), want) <= 2e-2


@pytest.mark.parametrize("T,E,K", [(1, 16, 2048), (4, 16, 2048), (16, 32, 2048),
                                   (33, 16, 1024)])
def test_token_major_vs_oracle(gpu, T, E, K):
    say(f"token-major T={T} E={E} K={K}")
    k = 8
    a, w2, ids, tw, r = _problem(T, E, K, k, gpu, 500 + T)
    out = torch.full((T, H), float("nan"), dtype=BF16, device=gpu)
    KD.launch_down_token_major(a, w2, out, tw, ids, r, k, {}, True)
    out_nr = torch.full_like(out, float("nan"))
    KD.launch_down_token_major(a, w2, out_nr, tw, ids, r, k, {}, False)
    again = torch.full_like(out, float("nan"))
    KD.launch_down_token_major(a, w2, again, tw, ids, r, k, {}, True)
    torch.cuda.synchronize()
    assert torch.equal(again, out), "repeat launch differs"
    w_cpu, a_cpu = w2.cpu(), a.cpu()
    for t in sorted({0, T // 2, T - 1}):
        sl = slice(t * k, (t + 1) * k)
        want = O.down_token_major(a_cpu[sl], w_cpu, tw[t:t + 1].cpu(), ids[t:t + 1].cpu(),
                                  r[t:t + 1].cpu())
        _check(out[t:t + 1], want, f"t={t}")
        want0 = O.down_token_major(a_cpu[sl], w_cpu, tw[t:t + 1].cpu(), ids[t:t + 1].cpu())
        _check(out_nr[t:t + 1], want0, f"t={t} no residual")
    # the unfused chain: grouped GEMM (weighted) into [T * k, H], then moe_sum + residual
    bm = 16
    sti, eids, ntp = moe_align_block_size(ids, bm, E)
    c3 = torch.empty(T * k, H, dtype=BF16, device=gpu)
    KD.launch_down(a, w2, c3, tw.reshape(-1), sti, eids, ntp, T * k, k, {"BLOCK_M": bm}, False)
    un = torch.empty(T, H, dtype=BF16, device=gpu)
    KD.launch_moe_sum(c3, un, r, k, {}, True)
    torch.cuda.synchronize()
    err = O.rel_err(out, un)
    say(f"  rel_err token-major vs unfused chain {err:.2e}")
    assert err <= 2e-2


def test_token_major_shared_expert_and_invalid_ids(gpu):
    T, E, K, k = 3, 16, 2048, 8
    a, w2, ids, tw, r = _problem(T, E, K, k, gpu, 77)
    g = torch.Generator(device=gpu).manual_seed(78)
    a_s = torch.randn(T, K, device=gpu, generator=g).to(BF16)
    w2_s = (torch.randn(1, H, K, device=gpu, generator=g) * 0.02).to(BF16)
    out = torch.empty(T, H, dtype=BF16, device=gpu)
    KD.launch_down_token_major(a, w2, out, tw, ids, r, k, {}, True, a_s, w2_s)
    # ids outside [0, E): those slots contribute nothing, as a zero weight does
    bad = ids.clone()
    bad[:, 3] = -1
    bad[:, 5] = E
    out_bad = torch.empty_like(out)
    KD.launch_down_token_major(a, w2, out_bad, tw, bad, r, k, {}, True)
    tw0 = tw.clone()
    tw0[:, 3] = 0
    tw0[:, 5] = 0
    out_zero = torch.empty_like(out)
    KD.launch_down_token_major(a, w2, out_zero, tw0, ids, r, k, {}, True)
    torch.cuda.synchronize()
    want = O.down_token_major(a.cpu(), w2.cpu(), tw.cpu(), ids.cpu(), r.cpu(), a_s.cpu(),
                              w2_s.cpu())
    _check(out, want, "shared expert")
    assert torch.equal(out_bad, out_zero)


def test_token_major_rejects_unsupported_k(gpu):
    a, w2, ids, tw, r = _problem(1, 4, 512, 2, gpu, 5)
    out = torch.empty(1, H, dtype=BF16, device=gpu)
    with pytest.raises(RuntimeError, match="unsupported"):
        KD.launch_down_token_major(a, w2, out, tw, ids, r, 2, {}, True)


def _merge(a, w2, out, tw, ids, k, bm, packed):
    E = w2.shape[0]
    sti, eids, ntp = moe_align_block_size(ids, bm, E)
    cfg = {"BLOCK_M": bm}
    if packed:
        cfg["w2_packed"] = KG.pack_w512(w2, w2.shape[1], 0, False)
    KD.launch_down(a, w2, out, tw.reshape(-1).contiguous(), sti, eids, ntp, ids.numel(), k,
                   cfg, True)


MERGE_CASES = [(16, False), (64, False), (64, True), (128, True)]


@pytest.mark.parametrize("bm,packed", MERGE_CASES)
def test_atomic_merge_exact_sums(gpu, bm, packed):
    """Integer-valued rows: every partial sum is exact in bf16, so the atomics' order
    cannot show and the result is the oracle's bit for bit."""
    say(f"atomic merge exact bm={bm} packed={packed}")
    T, E, K, k = 40, 16, 2048, 8
    g = torch.Generator(device=gpu).manual_seed(900 + bm)
    a = torch.zeros(T * k, K, dtype=BF16, device=gpu)
    a[:, :3] = 1.0
    w2 = torch.randint(-2, 3, (E, H, K), device=gpu, generator=g).to(BF16)
    ids = torch.stack([torch.randperm(E, device=gpu, generator=g)[:k] for _ in range(T)])
    ids = ids.to(torch.int32).contiguous()
    tw = torch.full((T, k), 0.5, device=gpu)
    seed = torch.randint(-5, 6, (T, H), device=gpu, generator=g).to(BF16)
    out = seed.clone()
    _merge(a, w2, out, tw, ids, k, bm, packed)
    torch.cuda.synchronize()
    want = O.down_merge_atomic(a.cpu(), w2.cpu(), tw.cpu(), ids.cpu(), seed.cpu())
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("bm,packed", MERGE_CASES)
def test_atomic_merge_top1_equals_unfused(gpu, bm, packed):
    """top_k = 1: one add per output row, so out = bf16(seed + y) with y the unfused GEMM's
    bf16 row -- bit for bit."""
    T, E, K, k = 200, 8, 2048, 1
    a, w2, ids, tw, r = _problem(T, E, K, k, gpu, 950 + bm)
    out = r.clone()
    _merge(a, w2, out, tw, ids, k, bm, packed)
    sti, eids, ntp = moe_align_block_size(ids, bm, E)
    c3 = torch.empty(T, H, dtype=BF16, device=gpu)
    KD.launch_down(a, w2, c3, tw.reshape(-1).contiguous(), sti, eids, ntp, T, k,
                   {"BLOCK_M": bm}, False)
    torch.cuda.synchronize()
    assert torch.equal(out, (r.float() + c3.float()).to(BF16))


@pytest.mark.parametrize("bm,packed", MERGE_CASES)
@pytest.mark.parametrize("T", [4, 300])
def test_atomic_merge_random(gpu, T, bm, packed):
    say(f"atomic merge random T={T} bm={bm} packed={packed}")
    E, K, k = 32, 2048, 8
    a, w2, ids, tw, r = _problem(T, E, K, k, gpu, 1000 + T + bm)
    out = r.clone()
    _merge(a, w2, out, tw, ids, k, bm, packed)
    zero = torch.zeros_like(r)
    _merge(a, w2, zero, tw, ids, k, bm, packed)
    torch.cuda.synchronize()
    w_cpu, a_cpu = w2.cpu(), a.cpu()
    for t in sorted({0, T // 2, T - 1}):
        sl = slice(t * k, (t + 1) * k)
        exact = O.down_token_major(a_cpu[sl], w_cpu, tw[t:t + 1].cpu(), ids[t:t + 1].cpu(),
                                   r[t:t + 1].cpu())
        # eight bf16 roundings per output (one per atomic add): the block tolerance
        _check(out[t:t + 1], exact, f"t={t}", tol=2e-2)
        exact0 = O.down_token_major(a_cpu[sl], w_cpu, tw[t:t + 1].cpu(), ids[t:t + 1].cpu())
        _check(zero[t:t + 1], exact0, f"t={t} zero seed", tol=2e-2)


def test_atomic_merge_rejects_bad_block(gpu):
    a, w2, ids, tw, r = _problem(4, 8, 2048, 2, gpu, 3)
    sti, eids, ntp = moe_align_block_size(ids, 32, 8)
    with pytest.raises(RuntimeError, match="unsupported"):
        KD.launch_down(a, w2, r.clone(), tw.reshape(-1).contiguous(), sti, eids, ntp, 8, 2,
                       {"BLOCK_M": 32}, True)
