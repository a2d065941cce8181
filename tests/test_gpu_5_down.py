"""The down GEMM's merge strategies (`glm52/kernels/moe_down_merge.py`) on the GPU.

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


def _check(got, want, what):
    torch.testing.assert_close(got.float().cpu(), want.float(), rtol=1e-2, atol=1e-2,
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
