"""Half-fused pre-norm (`glm52/kernels/lazy_prenorm.py`) on the GPU, through the C-ABI.

Inputs follow the reference's own #11 benchmark (`glm52/bench/bench_f11_lazy_prenorm.py:
238-330`): h ~ N(0, 0.5) [T, 6144], the norm weight w ~ 1 + N(0, 0.1), the router weight
[6144, 256] and w13 [E, 4096, 6144] ~ N(0, 0.02), each folded with w once.

  rstd                    bit for bit against the oracle's statistic
  router (rstd given, or  bit for bit against the oracle: exact-rule logits of h @ b_fold,
  fuse_norm)              one fp32 multiply by rstd; within the reference's 5e-2 bar of
                          the unfused norm -> router on the raw weight
  gate/up GEMM            rstd given and fuse_norm give the same bits; sampled slots within
                          bf16 output rounding (rtol/atol 1e-2) of the fp64 oracle; within
                          5e-2 of the unfused norm -> GEMM on the raw weight
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from fusion_amd.dispatch import moe_align_block_size
from fusion_amd.kernels import add_rmsnorm as KN
from fusion_amd.kernels import lazy_prenorm as KL
from fusion_amd.kernels import moe_gateup as KG
from fusion_amd.kernels import norm_router as KR
from oracle import glm52_oracle as O

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
H, ER, EPS = 6144, 256, 1e-5


def say(*a):
    print(*a, flush=True)


def _h(T, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    h = (torch.randn(T, H, device=gpu, generator=g) * 0.5).to(BF16)
    w = (torch.randn(H, device=gpu, generator=g) * 0.1 + 1).to(BF16)
    return h, w, g


@pytest.mark.parametrize("T", [1, 5, 300])
def test_rstd_bitwise(gpu, T):
    say(f"rstd T={T}")
    h, _, _ = _h(T, gpu, 70 + T)
    rstd = torch.full((T,), float("nan"), device=gpu)
    flat = torch.full((T * 8,), float("nan"), device=gpu)
    KL.launch_rstd(h, rstd, {}, EPS)
    KL.launch_rstd(h, None, {}, EPS, rstd_flat=flat, repeat=8)
    torch.cuda.synchronize()
    want = O.rstd_exact(h.cpu(), EPS)
    assert np.array_equal(rstd.cpu().numpy(), want)
    assert np.array_equal(flat.cpu().numpy(), np.repeat(want, 8))


def test_rstd_strided_rows_and_empty(gpu):
    h, _, _ = _h(6, gpu, 77)
    view = h[:, : H // 2]  # rows of a wider tensor
    rstd = torch.empty(6, device=gpu)
    KL.launch_rstd(view, rstd, {}, EPS)
    KL.launch_rstd(h[:0], torch.empty(0, device=gpu), {}, EPS)
    torch.cuda.synchronize()
    assert np.array_equal(rstd.cpu().numpy(), O.rstd_exact(view.cpu(), EPS))


@pytest.mark.parametrize("layout", ["kn", "rows"])
@pytest.mark.parametrize("T", [1, 3, 4, 7, 64, 1000])
def test_prenorm_router_bitwise(gpu, T, layout):
    """`kn`: B [K, N] contiguous, as the reference passes it; `rows`: B the transposed view
    of the [N, K] gate (the one-launch fully fused mapping at T <= 4)."""
    say(f"prenorm router T={T} {layout}")
    h, w, g = _h(T, gpu, 80 + T)
    if layout == "kn":
        b_raw = (torch.randn(H, ER, device=gpu, generator=g) * 0.02).to(BF16)
        b_fold = KL.fold_weight_rowmajor(b_raw, w)
        assert torch.equal(b_fold.cpu(), O.fold_weight(b_raw.cpu(), w.cpu(), 0))
    else:
        gate = (torch.randn(ER, H, device=gpu, generator=g) * 0.02).to(BF16)
        gate_f = KL.fold_weight_nk(gate, w)
        assert torch.equal(gate_f.cpu(), O.fold_weight(gate.cpu(), w.cpu(), 1))
        b_raw, b_fold = gate.t(), gate_f.t()
    rstd = torch.empty(T, device=gpu)
    KL.launch_rstd(h, rstd, {}, EPS)
    half = torch.full((T, ER), float("nan"), device=gpu)
    KL.launch_router(h, b_fold, half, {}, False, EPS, 0, rstd)
    fused = torch.full((T, ER), float("nan"), device=gpu)
    KL.launch_router(h, b_fold, fused, {}, True, EPS)
    # unfused: materialised norm, then the router on the raw weight
    x2 = torch.empty_like(h)
    KN.norm_only(h, w, x2, {})
    un = torch.empty(T, ER, device=gpu)
    KL.launch_router(x2, b_raw, un, {}, False, EPS)
    torch.cuda.synchronize()
    want = O.prenorm_router(h.cpu(), b_fold.cpu(), O.rstd_exact(h.cpu(), EPS))
    assert np.array_equal(half.cpu().numpy(), want)
    assert torch.equal(fused, half)
    assert np.array_equal(un.cpu().numpy(), O.router_logits_exact(x2.cpu(), b_raw.cpu()))
    ref = x2.float() @ b_raw.float()
    err = O.rel_err(half, ref)
    say(f"  rel_err half vs unfused fp32 {err:.2e}")
    assert err < 5e-2


@pytest.mark.parametrize("bm", [16, 64])
@pytest.mark.parametrize("T", [3, 200])
def test_prenorm_gateup(gpu, bm, T):
    say(f"prenorm gate/up bm={bm} T={T}")
    E, N, k = 8, 4096, 8
    h, w, g = _h(T, gpu, 90 + T + bm)
    w13 = (torch.randn(E, N, H, device=gpu, generator=g) * 0.02).to(BF16)
    w13f = KL.fold_weight_nk(w13, w)
    ids = torch.stack([torch.randperm(E, device=gpu, generator=g)[:k] for _ in range(T)])
    ids = ids.to(torch.int32)
    sti, eids, ntp = moe_align_block_size(ids, bm, E)
    cfg = {"BLOCK_M": bm}
    R = T * k
    rstd = torch.empty(T, device=gpu)
    KL.launch_rstd(h, rstd, {}, EPS)
    c_half = torch.full((R, N), float("nan"), dtype=BF16, device=gpu)
    KL.launch_moe_gateup(h, w13f, c_half, sti, eids, ntp, R, k, cfg, False, EPS, 0, rstd)
    c_fused = torch.full((R, N), float("nan"), dtype=BF16, device=gpu)
    KL.launch_moe_gateup(h, w13f, c_fused, sti, eids, ntp, R, k, cfg, True, EPS)
    x2 = torch.empty_like(h)
    KN.norm_only(h, w, x2, {})
    c_un = torch.full((R, N), float("nan"), dtype=BF16, device=gpu)
    KL.launch_moe_gateup(x2, w13, c_un, sti, eids, ntp, R, k, cfg, False, EPS)
    torch.cuda.synchronize()
    assert torch.equal(c_fused, c_half)
    # sampled tokens against the fp64 oracle
    r_cpu, w_cpu = rstd.cpu().numpy(), w13f.cpu()
    for t in sorted({0, T // 2, T - 1}):
        want = O.prenorm_gateup_rows(h[t:t + 1].cpu(), w_cpu, r_cpu[t:t + 1],
                                     ids[t:t + 1].cpu())
        got = c_half[t * k:(t + 1) * k].cpu()
        torch.testing.assert_close(got.float(), want.float(), rtol=1e-2, atol=1e-2)
    err = O.rel_err(c_half, c_un)
    say(f"  rel_err half vs unfused {err:.2e}")
    assert err < 5e-2


def test_norm_router_no_x2_leaves_x2(gpu):
    T = 33
    h, w, g = _h(T, gpu, 99)
    gate = (torch.randn(ER, H, device=gpu, generator=g) * 0.02).to(BF16)
    wgt = KR.wgt_from_gate(gate)
    x2 = torch.empty_like(h)
    lg = torch.empty(T, ER, device=gpu)
    KR.fused_norm_router(h, w, x2, wgt, lg, {})
    sentinel = torch.full_like(h, 3.0)
    lg2 = torch.full_like(lg, float("nan"))
    KR.fused_norm_router_no_x2(h, w, sentinel, wgt, lg2, {})
    torch.cuda.synchronize()
    assert torch.equal(lg2, lg)
    assert bool((sentinel == 3.0).all())


@pytest.mark.parametrize("T", [5, 17, 1000, 2048, 4100])
def test_prenorm_router_topk(gpu, T):
    """The router with the rstd epilogue and its top-k (`glm52_router_rstd`) on a gate read
    as rows: from 17 tokens the bounded router, below it the exact logits (T = 5).  Ids and weights bit for bit against the
    exact rule on the oracle's pre-norm logits (exact logit, one fp32 multiply by rstd);
    the selected logits exact; every other logit within rstd times the bounded router's
    bound.  fuse_norm (the statistic computed here) gives the same bits as rstd given."""
    say(f"prenorm router + top-k T={T}")
    h, w, g = _h(T, gpu, 300 + T)
    gate = (torch.randn(ER, H, device=gpu, generator=g) * 0.02).to(BF16)
    gate_f = KL.fold_weight_nk(gate, w)
    bias = torch.randn(ER, device=gpu, generator=g) * 0.01
    rstd = torch.empty(T, device=gpu)
    KL.launch_rstd(h, rstd, {}, EPS)
    out = {}
    for name, fuse in (("half", False), ("fused", True)):
        lg = torch.full((T, ER), float("nan"), device=gpu)
        tw = torch.empty(T, 8, device=gpu)
        ti = torch.empty(T, 8, dtype=torch.int32, device=gpu)
        cfg = {"topw": tw, "topi": ti, "correction_bias": bias}
        KL.launch_router(h, gate_f.t(), lg, cfg, fuse, EPS, 0, None if fuse else rstd)
        out[name] = (lg, tw, ti)
    torch.cuda.synchronize()
    for a, b in zip(out["half"], out["fused"]):
        assert torch.equal(a, b)
    lg, tw, ti = (t.cpu().numpy() for t in out["half"])
    r_o = O.rstd_exact(h.cpu(), EPS)
    want = O.prenorm_router(h.cpu(), gate_f.t().contiguous().cpu(), r_o)
    w_o, ids_o, _ = O.router_select(want, bias.cpu().numpy())
    assert np.array_equal(ti, ids_o)
    assert np.array_equal(tw, w_o)
    sel = np.take_along_axis(lg, ids_o.astype(np.int64), 1)
    assert np.array_equal(sel, np.take_along_axis(want, ids_o.astype(np.int64), 1))
    hn = np.sqrt((h.cpu().double().numpy() ** 2).sum(1))[:, None]
    gn = np.sqrt((gate_f.cpu().double().numpy() ** 2).sum(1))[None, :]
    bound = (r_o.astype(np.float64)[:, None] * 1.375 * 2.0 ** -16 * hn * gn
             + 2.0 ** -19 * np.abs(want) + 1e-30)
    ratio = np.abs(lg.astype(np.float64) - want) / bound
    say(f"  max |error| / bound = {ratio.max():.3e}, exact fraction {(lg == want).mean():.3f}")
    assert ratio.max() <= 1.0
