"""CPU tests that pin the oracle (oracle/glm52_oracle.py) before anything is checked
against it: golden vectors written by the reference's own `glm52/reference.py`
(tests/golden/make_golden.py), closed forms, brute force on small inputs and invariants.
Each check is chosen so that a plausible slip (a dropped bias, a reversed tie rule, a
missing bf16 round, an off-by-one in the layout) fails it.
"""

from __future__ import annotations

import hashlib
import itertools
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

from fusion_amd.problem import front_end, zipf_bias
from oracle import glm52_oracle as O

BF16 = torch.bfloat16

GOLD = Path(__file__).resolve().parent / "golden"


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_from_u16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


@pytest.fixture(scope="module")
def cfg0():
    g = np.load(GOLD / "config0_t32.npz")
    fe = front_end(32)
    return g, fe


# ---------------------------------------------------------------------- golden vectors
def test_config0_inputs_regenerate(cfg0):
    g, fe = cfg0
    assert list(g["in_sha"]) == [sha(fe.x), sha(fe.r), sha(fe.w_norm), sha(fe.gate), sha(fe.bias)]


def test_add_rmsnorm_matches_reference_bitwise(cfg0):
    g, fe = cfg0
    y, h = O.add_rmsnorm(fe.x, fe.r, fe.w_norm)
    assert np.array_equal(u16(h), g["h"])
    assert np.array_equal(u16(y), g["y"])


def ulp_diff_bf16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in bf16 ulps for same-sign values (bit patterns as uint16)."""
    ai, bi = a.astype(np.int32), b.astype(np.int32)
    return np.abs(ai - bi)


def test_add_rmsnorm_exact_within_one_ulp_of_reference(cfg0):
    g, fe = cfg0
    y, h = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    assert np.array_equal(u16(h), g["h"])
    d = ulp_diff_bf16(u16(y), g["y"])
    assert d.max() <= 1
    # and it is not a copy of the torch path: the statistic differs in some row
    ss_torch = fe.x.float().add(fe.r.float()).to(torch.bfloat16).float().pow(2).mean(-1)
    ss_exact = (h.float().double() ** 2).mean(-1)
    assert (ss_torch.double() != ss_exact).any()


def test_rmsnorm_exact_statistic_closed_form():
    """rstd from an exact rational sum of squares, rounded once."""
    g = torch.Generator().manual_seed(12)
    h = torch.randn(3, 256, generator=g).to(torch.bfloat16)
    w = torch.ones(256, dtype=torch.bfloat16)
    y = O.rmsnorm_exact(h, w)
    for t in range(3):
        ss = sum(Fraction(float(v)) ** 2 for v in h[t].float().tolist())
        ms = float(ss) / 256 + float(np.float32(1e-5))
        rstd = np.float32(1.0 / np.sqrt(ms))
        want = (torch.from_numpy(h[t].float().numpy() * rstd).to(torch.bfloat16).float()
                ).to(torch.bfloat16)
        assert torch.equal(y[t], want)


def test_router_exact_on_exact_norm_matches_reference_ids(cfg0):
    """The full device rule (exact norm, exact logits, exact sigmoid) picks the
    reference's ids at configuration 0."""
    g, fe = cfg0
    y, _ = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    _, w, ids = O.router_exact(y, fe.wgt, fe.bias.numpy())
    assert np.array_equal(ids, g["topk_ids"])
    np.testing.assert_allclose(w, g["topk_weights"], rtol=2e-6, atol=1e-7)


def test_router_exact_matches_reference_ids(cfg0):
    g, fe = cfg0
    y = bf16_from_u16(g["y"]).reshape(32, -1)
    lg, w, ids = O.router_exact(y, fe.wgt, fe.bias.numpy())
    assert np.array_equal(ids, g["topk_ids"])
    np.testing.assert_allclose(w, g["topk_weights"], rtol=2e-6, atol=1e-7)
    # logits: reference's fp32 F.linear vs the exact rule, against the dynamic range
    assert np.abs(lg - g["logits"]).max() / np.abs(g["logits"]).max() < 1e-5
    lg0, w0, ids0 = O.router_exact(y, fe.wgt, None)
    assert np.array_equal(ids0, g["topk_ids_nobias"])
    np.testing.assert_allclose(w0, g["topk_weights_nobias"], rtol=2e-6, atol=1e-7)


def test_bias_golden_is_discriminative(cfg0):
    """The biased and unbiased golden ids differ, so dropping the bias fails above."""
    g, _ = cfg0
    assert not np.array_equal(g["topk_ids"], g["topk_ids_nobias"])


def test_router_reference_restatement_matches_golden(cfg0):
    g, fe = cfg0
    y = bf16_from_u16(g["y"]).reshape(32, -1)
    lg, w, ids = O.router_reference(y, fe.gate, fe.bias)
    assert np.array_equal(ids.numpy(), g["topk_ids"])
    assert np.array_equal(lg.numpy(), g["logits"])
    assert np.array_equal(w.numpy(), g["topk_weights"])


def _tiny():
    import sys
    sys.path.insert(0, str(GOLD))
    from make_golden import tiny_inputs  # the same generator that wrote the fixture

    return tiny_inputs()


def test_tiny_moe_matches_reference():
    g = np.load(GOLD / "tiny_moe.npz")
    d = _tiny()
    assert list(g["in_sha"]) == [sha(v) for v in d.values()]
    lg, tw, ti = O.router_reference(d["x"], d["gate"], None, topk=4)
    assert np.array_equal(ti.numpy(), g["topk_ids"])
    routed = O.moe_mlp(d["x"], d["w13"], d["w2"], tw, ti)
    assert np.array_equal(u16(routed), g["routed"])
    assert np.array_equal(u16(O.silu_and_mul(d["act_in"])), g["silu"])
    assert np.array_equal(u16(O.expert_merge(d["y3"], d["wt"])), g["merged"])


# ---------------------------------------------------------------------- closed forms
def test_rmsnorm_special_cases():
    H = 64
    w = (1.0 + 0.1 * torch.randn(H)).to(torch.bfloat16)
    z = torch.zeros(3, H, dtype=torch.bfloat16)
    y, h = O.add_rmsnorm(z, z, w)
    assert torch.count_nonzero(y.float()) == 0 and torch.count_nonzero(h.float()) == 0
    for c in (0.5, -3.0, 7.25):
        x = torch.full((1, H), c, dtype=torch.bfloat16)
        y = O.rmsnorm(x, w)
        rn = np.float32(c) / np.sqrt(np.float32(c) * np.float32(c) + np.float32(1e-5))
        want = (torch.tensor(rn).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16)
        assert torch.equal(y[0], want)


def test_add_is_single_rounding():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 128, generator=g).to(torch.bfloat16)
    r = torch.randn(4, 128, generator=g).to(torch.bfloat16)
    _, h = O.add_rmsnorm(x, r, torch.ones(128, dtype=torch.bfloat16))
    exact = x.double() + r.double()  # exact: two bf16 fit in fp64 without rounding
    assert torch.equal(h, exact.float().to(torch.bfloat16))


def test_silu_and_mul_closed_form():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    got = O.silu_and_mul(x).float().numpy()
    gd, ud = x[:, :32].double().numpy(), x[:, 32:].double().numpy()
    want = gd / (1 + np.exp(-gd)) * ud
    ulp = np.abs(want) * 2.0 ** -8 + 1e-30
    assert (np.abs(got - want) <= ulp).all()


# ---------------------------------------------------------------------- router
def _exact_fp32_round(fr: Fraction) -> np.float32:
    """Correctly rounded Fraction -> fp32 (brute force via the two neighbours)."""
    f = np.float32(float(fr))
    cands = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    return min(cands, key=lambda c: (abs(Fraction(float(c)) - fr), int(np.float32(c).view(np.int32)) & 1))


def test_router_logits_exact_vs_rational_sum():
    g = torch.Generator().manual_seed(3)
    T, H, E = 3, 128, 5
    y = torch.randn(T, H, generator=g).to(torch.bfloat16)
    wg = (torch.randn(H, E, generator=g) * 0.1).to(torch.bfloat16)
    got = O.router_logits_exact(y, wg)
    yf, wf = y.float().numpy(), wg.float().numpy()
    for t, e in itertools.product(range(T), range(E)):
        s = sum(Fraction(float(yf[t, k])) * Fraction(float(wf[k, e])) for k in range(H))
        assert got[t, e] == _exact_fp32_round(s)


def _brute_select(logits, bias, k, scale=2.5):
    s = O.sigmoid_exact(logits)
    ids, ws = [], []
    for t in range(s.shape[0]):
        key = [(-(np.float32(s[t, e] + (0 if bias is None else bias[e]))), e) for e in range(s.shape[1])]
        sel = [e for _, e in sorted(key)[:k]]
        sv = [s[t, e] for e in sel]
        tot = np.float32(0)
        for v in sv:
            tot = np.float32(tot + v)
        ids.append(sel)
        ws.append([np.float32(np.float32(v / max(tot, np.float32(1e-20))) * np.float32(scale)) for v in sv])
    return np.array(ws, dtype=np.float32), np.array(ids, dtype=np.int32)


def test_router_select_vs_brute_force():
    rng = np.random.default_rng(5)
    for E, k in ((16, 8), (256, 8), (9, 3)):
        lg = rng.normal(size=(20, E)).astype(np.float32)
        bias = (0.01 * rng.normal(size=E)).astype(np.float32)
        w, ids, _ = O.router_select(lg, bias, k)
        bw, bids = _brute_select(lg, bias, k)
        assert np.array_equal(ids, bids)
        assert np.array_equal(w, bw)


def test_router_ties_lower_index_first():
    lg = np.zeros((2, 16), dtype=np.float32)  # every score 0.5: a 16-way tie
    _, ids, _ = O.router_select(lg, None, 8)
    assert ids.tolist() == [list(range(8))] * 2
    lg[1, 12] = lg[1, 13] = 1.0  # two tied winners, then the lowest-index ties
    _, ids, _ = O.router_select(lg, None, 8)
    assert ids[1].tolist() == [12, 13, 0, 1, 2, 3, 4, 5]


def test_router_large_bias_picks_biased_experts_in_bias_order():
    rng = np.random.default_rng(6)
    lg = rng.normal(size=(4, 256)).astype(np.float32)
    bias = np.zeros(256, dtype=np.float32)
    chosen = [200, 3, 17, 99, 5, 250, 64, 128]
    for rank, e in enumerate(chosen):
        bias[e] = 100.0 - rank
    w, ids, s = O.router_select(lg, bias, 8)
    assert (ids == np.array(chosen)).all()
    # weights are the UNBIASED scores renormalised: sum to 2.5, ratios = score ratios
    np.testing.assert_allclose(w.sum(1), 2.5, rtol=1e-6)
    np.testing.assert_allclose(w[:, 0] / w[:, 1], s[:, 200] / s[:, 3], rtol=1e-6)


def test_router_invariants_zipf():
    fe = front_end(64, bias="zipf")
    y, _ = O.add_rmsnorm(fe.x, fe.r, fe.w_norm)
    lg, w, ids = O.router_exact(y, fe.wgt, zipf_bias().numpy())
    assert all(len(set(r)) == 8 for r in ids.tolist())
    np.testing.assert_allclose(w.sum(1), 2.5, rtol=8 * 2 ** -23)
    # the skewed bias concentrates load on the low experts
    counts = np.bincount(ids.reshape(-1), minlength=256)
    assert counts[:51].sum() > counts[51:].sum() / 4


# ---------------------------------------------------------------------- dispatch layout
def _brute_align(flat, bm, E):
    """Independent restatement: walk experts, collect indices in order, pad."""
    sorted_ids, expert_ids = [], []
    numel = len(flat)
    for e in range(E):
        mine = [i for i, v in enumerate(flat) if v == e]
        if not mine:
            continue
        nblk = -(-len(mine) // bm)
        sorted_ids += mine + [numel] * (nblk * bm - len(mine))
        expert_ids += [e] * nblk
    return np.array(sorted_ids, dtype=np.int32), np.array(expert_ids, dtype=np.int32), len(sorted_ids)


@pytest.mark.parametrize("T,k,E,bm", [(1, 8, 256, 16), (5, 8, 16, 4), (32, 8, 256, 16),
                                      (33, 8, 256, 64), (7, 1, 1, 16), (40, 2, 3, 128)])
def test_align_vs_brute_force(T, k, E, bm):
    rng = np.random.default_rng(T * 1000 + bm)
    ids = np.stack([rng.choice(E, size=k, replace=(k > E)) for _ in range(T)]).astype(np.int32)
    sti, eids, ntp = O.moe_align_block_size(ids, bm, E)
    bs, be, bn = _brute_align(ids.reshape(-1).tolist(), bm, E)
    assert ntp[0] == bn
    assert np.array_equal(sti, bs) and np.array_equal(eids, be)


def test_align_invariants_large():
    rng = np.random.default_rng(11)
    T, k, E, bm = 2048, 8, 256, 64
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    sti, eids, ntp = O.moe_align_block_size(ids, bm, E)
    numel = T * k
    real = sti[sti < numel]
    assert np.array_equal(np.sort(real), np.arange(numel))  # a permutation
    flat = ids.reshape(-1)
    for b, e in enumerate(eids):
        blk = sti[b * bm:(b + 1) * bm]
        blk = blk[blk < numel]
        assert (flat[blk] == e).all() and (np.diff(blk) > 0).all()
    counts = np.bincount(flat, minlength=E)
    assert ntp[0] == (((counts + bm - 1) // bm) * bm).sum()
    assert set(eids.tolist()) == set(np.nonzero(counts)[0].tolist())


# ---------------------------------------------------------------------- experts / merges
def test_tiny_moe_vs_fp64_textbook():
    d = _tiny()
    lg, tw, ti = O.router_reference(d["x"], d["gate"], None, topk=4)
    got = O.moe_mlp(d["x"], d["w13"], d["w2"], tw, ti).float().numpy()
    x = d["x"].double().numpy()
    w13, w2 = d["w13"].double().numpy(), d["w2"].double().numpy()
    want = np.zeros_like(x)
    I = w2.shape[2]
    for t in range(x.shape[0]):
        for j in range(4):
            e = int(ti[t, j])
            hh = w13[e] @ x[t]
            a = hh[:I] / (1 + np.exp(-hh[:I])) * hh[I:]
            want[t] += float(tw[t, j]) * (w2[e] @ a)
    assert np.abs(got - want).max() / np.abs(want).max() < 2e-2


def test_shared_expert_vs_fp64():
    d = _tiny()
    got = O.shared_expert(d["x"], d["w13s"], d["w2s"]).numpy()
    x = d["x"].double().numpy()
    w13, w2 = d["w13s"][0].double().numpy(), d["w2s"][0].double().numpy()
    hh = x @ w13.T
    I = w2.shape[1]
    want = (hh[:, :I] / (1 + np.exp(-hh[:, :I])) * hh[:, I:]) @ w2.T
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-2


def test_merges_closed_form():
    g = torch.Generator().manual_seed(8)
    y3 = torch.randn(5, 8, 64, generator=g).to(torch.bfloat16)
    res = torch.randn(5, 64, generator=g).to(torch.bfloat16)
    wt = torch.rand(5, 8, generator=g)
    s = O.moe_sum(y3, res).float().numpy()
    want = y3.double().sum(1).numpy() + res.double().numpy()
    assert (np.abs(s - want) <= np.abs(want) * 2 ** -8 + 1e-6).all()
    m = O.merge_resadd(y3, wt, res, round_mid=False).float().numpy()
    want = (y3.double() * wt.double().unsqueeze(-1)).sum(1).numpy() + res.double().numpy()
    assert (np.abs(m - want) <= np.abs(want) * 2 ** -8 + 1e-5).all()
    # expert_merge is the round_mid merge without the residual
    assert torch.equal(O.expert_merge(y3, wt),
                       O.merge_resadd(y3, wt, torch.zeros_like(res), round_mid=True))


# ------------------------------------------------------------------ o_proj + ResAdd1
def test_oproj_one_hot_rows_are_exact():
    """A row with a single 1 at k selects row k of B exactly; with the residual the one
    fp32 add rounds once to bf16 (closed form)."""
    g = torch.Generator().manual_seed(3)
    K, N = 64, 48
    b = (torch.randn(K, N, generator=g) * 0.3).to(BF16)
    r = torch.randn(5, N, generator=g).to(BF16)
    ks = [0, 7, 31, 32, 63]
    a = torch.zeros(5, K, dtype=BF16)
    for i, k in enumerate(ks):
        a[i, k] = 1.0
    assert torch.equal(O.oproj_gemm(a, b), b[ks])
    want = (b[ks].float() + r.float()).to(BF16)
    assert torch.equal(O.oproj_gemm(a, b, r), want)
    # a scaled one-hot: exact powers of two keep the rows exact
    assert torch.equal(O.oproj_gemm(a * 4, b), (b[ks].float() * 4).to(BF16))


def test_oproj_vs_fp64_textbook_and_cast():
    g = torch.Generator().manual_seed(4)
    M, K, N = 6, 96, 40
    a = (torch.randn(M, K, generator=g) * 0.05).to(BF16)
    b = (torch.randn(K, N, generator=g) * 0.02).to(BF16)
    r = (torch.randn(M, N, generator=g) * 0.5).to(BF16)
    an, bn = a.double().numpy(), b.double().numpy()
    ref = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            ref[m, n] = sum(an[m, k] * bn[k, n] for k in range(K))
    got = O.oproj_gemm(a, b, out_dtype=torch.float32).double().numpy()
    assert np.abs(got - ref).max() <= 1e-7 * np.abs(ref).max()
    # fused = cast(unrounded product + r); unfused = cast(bf16 product + r)
    fused = O.oproj_gemm(a, b, r)
    assert torch.equal(fused, O.oproj_cast(O.oproj_gemm(a, b, out_dtype=torch.float32), r))
    unfused = O.oproj_cast(O.oproj_gemm(a, b), r)
    d = (unfused.float() - fused.float()).abs()
    assert (d <= fused.float().abs() * 2 ** -7 + 1e-6).all()  # within one extra rounding


# ------------------------------------------------------------------ half-fused pre-norm
def test_rstd_exact_rational_sum_and_closed_forms():
    g = torch.Generator().manual_seed(21)
    h = torch.randn(4, 192, generator=g).to(BF16)
    r = O.rstd_exact(h)
    for t in range(4):
        ss = sum(Fraction(float(v)) ** 2 for v in h[t].float().tolist())
        want = np.float32(1.0 / np.sqrt(float(ss / 192) + float(np.float32(1e-5))))
        assert r[t] == want
    # constant rows: rstd = 1 / sqrt(c^2 + eps)
    for c in (0.5, -3.0, 7.25):
        x = torch.full((1, 64), c, dtype=BF16)
        assert O.rstd_exact(x)[0] == np.float32(1.0 / np.sqrt(c * c + float(np.float32(1e-5))))
    # eps = 0: doubling the row halves rstd exactly
    assert np.array_equal(O.rstd_exact(h * 2, eps=0.0), O.rstd_exact(h, eps=0.0) / 2)
    # the statistic inside rmsnorm_exact (w = 1: y = bf16(h * rstd))
    y = O.rmsnorm_exact(h, torch.ones(192, dtype=BF16))
    assert torch.equal(y, (h.float() * torch.from_numpy(r)[:, None]).to(BF16))


def test_fold_weight_axes_and_exact_cases():
    g = torch.Generator().manual_seed(22)
    b = torch.randn(64, 24, generator=g).to(BF16)
    w = torch.full((64,), 2.0, dtype=BF16)
    assert torch.equal(O.fold_weight(b, w, 0), (b.float() * 2).to(BF16))
    assert torch.equal(O.fold_weight(b, torch.ones(64, dtype=BF16), 0), b)
    w = (1 + 0.1 * torch.randn(64, generator=g)).to(BF16)
    bt = b.t().contiguous()
    assert torch.equal(O.fold_weight(b, w, 0).t(), O.fold_weight(bt, w, 1))
    assert torch.equal(O.fold_weight(b, w, 0)[5], (b[5].float() * w[5].float()).to(BF16))


def test_prenorm_router_one_hot_and_identity():
    g = torch.Generator().manual_seed(23)
    K, N = 128, 32
    b = (torch.randn(K, N, generator=g) * 0.02).to(BF16)
    w = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16)
    bf = O.fold_weight(b, w, 0)
    # one-hot rows: the logits are fp32(bf[k] * c) * rstd, rstd = 1 / sqrt(c^2 / K + eps)
    ks, c = [0, 17, 127], 3.0
    h = torch.zeros(3, K, dtype=BF16)
    for i, k in enumerate(ks):
        h[i, k] = c
    rstd = O.rstd_exact(h)
    assert np.all(rstd == np.float32(1.0 / np.sqrt(c * c / K + float(np.float32(1e-5)))))
    got = O.prenorm_router(h, bf, rstd)
    want = (bf[ks].float().numpy() * np.float32(c)) * rstd[:, None]
    assert np.array_equal(got, want.astype(np.float32))
    # w = 1 folds to the plain weight: the logits times rstd
    hr = (torch.randn(5, K, generator=g) * 0.5).to(BF16)
    rr = O.rstd_exact(hr)
    plain = O.router_logits_exact(hr, b)
    assert np.array_equal(O.prenorm_router(hr, O.fold_weight(b, torch.ones(K, dtype=BF16), 0), rr),
                          (plain * rr[:, None]).astype(np.float32))
    # the folding identity against norm -> router (`bench_f11_lazy_prenorm.py:996-1014`)
    un = O.router_logits_exact(O.rmsnorm_exact(hr, w), b)
    assert O.rel_err(torch.from_numpy(O.prenorm_router(hr, bf, rr)), torch.from_numpy(un)) < 5e-2


def test_prenorm_gateup_rows_one_hot_and_identity():
    g = torch.Generator().manual_seed(24)
    T, K, N, E, k = 3, 64, 32, 4, 2
    w13 = (torch.randn(E, N, K, generator=g) * 0.02).to(BF16)
    wn = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16)
    wf = O.fold_weight(w13, wn, 2)
    ids = torch.tensor([[0, 3], [2, 1], [3, 0]])
    h = (torch.randn(T, K, generator=g) * 0.5).to(BF16)
    r = O.rstd_exact(h)
    got = O.prenorm_gateup_rows(h, wf, r, ids)
    # textbook per slot: an exact rational dot product, rounded to fp32, times rstd
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            for n_ in (0, 13, N - 1):
                dot = sum(Fraction(float(wf[e, n_, q])) * Fraction(float(h[t, q]))
                          for q in range(K))
                want = torch.tensor(np.float32(np.float32(float(dot)) * r[t])).to(BF16)
                assert torch.equal(got[t * k + j, n_], want)
    # one-hot h: slot rows are bf16(fp32(wf[e, :, kk] * c) * rstd)
    c, kk = 2.0, 9
    h1 = torch.zeros(1, K, dtype=BF16)
    h1[0, kk] = c
    r1 = O.rstd_exact(h1)
    got1 = O.prenorm_gateup_rows(h1, wf, r1, ids[:1])
    for j in range(k):
        e = int(ids[0, j])
        want = ((wf[e, :, kk].float() * c) * float(r1[0])).to(BF16)
        assert torch.equal(got1[j], want)
    # the folding identity against norm -> gate/up GEMM on the raw weight
    x2 = O.rmsnorm_exact(h, wn)
    un = O.prenorm_gateup_rows(x2, w13, np.ones(T, dtype=np.float32), ids)
    assert O.rel_err(got, un) < 5e-2


# ------------------------------------------------------------------ token-major down GEMV
def _tokmaj_problem(T=3, k=2, E=4, H=24, K=32, seed=31):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(T * k, K, generator=g) * 0.5).to(BF16)
    w2 = (torch.randn(E, H, K, generator=g) * 0.1).to(BF16)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    tw = torch.rand(T, k, generator=g) + 0.25
    return a, w2, ids, tw


def test_down_token_major_rational_and_closed_forms():
    a, w2, ids, tw = _tokmaj_problem()
    T, k = ids.shape
    out = O.down_token_major(a, w2, tw, ids)
    # exact rational sums of the weighted products, rounded once (fp32, then bf16)
    for t in range(T):
        for n in (0, 7, 23):
            s = sum(Fraction(float(tw[t, j])) * sum(Fraction(float(a[t * k + j, q])) *
                                                    Fraction(float(w2[int(ids[t, j]), n, q]))
                                                    for q in range(a.shape[1]))
                    for j in range(k))
            want = torch.tensor(np.float32(float(s))).to(BF16)
            assert torch.equal(out[t, n], want)
    # one-hot rows with weight 1: the output row is the sum of the selected W columns
    a1 = torch.zeros_like(a)
    a1[:, 5] = 1.0
    ones = torch.ones_like(tw)
    got = O.down_token_major(a1, w2, ones, ids)
    for t in range(T):
        col = sum(w2[int(ids[t, j]), :, 5].double() for j in range(k))
        assert torch.equal(got[t], col.float().to(BF16))
    # linearity: doubling the weights doubles the output exactly (no residual)
    assert torch.equal(O.down_token_major(a, w2, tw * 2, ids).float(), out.float() * 2)


def test_down_token_major_shared_and_residual_and_unfused():
    a, w2, ids, tw = _tokmaj_problem(seed=32)
    T, k = ids.shape
    H, K = w2.shape[1:]
    g = torch.Generator().manual_seed(33)
    a_s = (torch.randn(T, K, generator=g) * 0.5).to(BF16)
    w2_s = (torch.randn(1, H, K, generator=g) * 0.1).to(BF16)
    r = torch.randn(T, H, generator=g).to(BF16)
    got = O.down_token_major(a, w2, tw, ids, r, a_s, w2_s)
    routed = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            routed[t] += float(tw[t, j]) * (w2[int(ids[t, j])].double() @ a[t * k + j].double())
    shared = a_s.double() @ w2_s[0].double().t()
    want = ((routed + shared).float() + r.float()).to(BF16)
    assert torch.equal(got, want)
    # the unfused chain rounds every expert's row to bf16 first (moe_sum over Y)
    y3 = torch.empty(T, k, H, dtype=BF16)
    for t in range(T):
        for j in range(k):
            acc = (w2[int(ids[t, j])].double() @ a[t * k + j].double()).float()
            y3[t, j] = (acc * float(tw[t, j])).to(BF16)
    un = O.moe_sum(y3, None)
    fused = O.down_token_major(a, w2, tw, ids)
    bound = (k + 1) * 2.0 ** -8 * y3.float().abs().sum(dim=1) + 1e-6
    assert ((un.float() - fused.float()).abs() <= bound).all()


# ------------------------------------------------------------------ atomic expert merge
def test_down_merge_atomic_closed_forms():
    a, w2, ids, tw = _tokmaj_problem(T=4, k=1, seed=41)
    g = torch.Generator().manual_seed(42)
    seed = torch.randn(4, w2.shape[1], generator=g).to(BF16)
    got = O.down_merge_atomic(a, w2, tw, ids, seed)
    for t in range(4):  # top_k = 1: one rounding of seed + bf16(y)
        y = ((w2[int(ids[t, 0])].double() @ a[t].double()).float() * float(tw[t, 0])).to(BF16)
        assert torch.equal(got[t], (seed[t].float() + y.float()).to(BF16))
    # integer-valued rows: every partial sum is exact, so any add order gives the sum
    T, k, E, H, K = 3, 4, 6, 16, 64
    a_i = torch.zeros(T * k, K, dtype=BF16)
    a_i[:, :3] = 1.0
    w_i = torch.randint(-2, 3, (E, H, K), generator=g).to(BF16)
    ids_i = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    tw_i = torch.full((T, k), 2.0)
    seed_i = torch.randint(-5, 6, (T, H), generator=g).to(BF16)
    got_i = O.down_merge_atomic(a_i, w_i, tw_i, ids_i, seed_i)
    want = seed_i.double().clone()
    for t in range(T):
        for j in range(k):
            want[t] += 2.0 * w_i[int(ids_i[t, j]), :, :3].double().sum(-1)
    assert torch.equal(got_i.double(), want)
    # against the one-rounding token-major result: within one rounding per add
    a, w2, ids, tw = _tokmaj_problem(T=3, k=4, seed=43)
    r = torch.randn(3, w2.shape[1], generator=g).to(BF16)
    at = O.down_merge_atomic(a, w2, tw, ids, r)
    tm = O.down_token_major(a, w2, tw, ids, r)
    bound = 5 * 2.0 ** -8 * (at.float().abs() + 4 * r.float().abs().max()) + 1e-3
    assert ((at.float() - tm.float()).abs() <= bound).all()


def test_moe_mlp_rows_equals_moe_mlp():
    """`moe_mlp_rows` over every row is `moe_mlp` before its bf16 round, bit for bit (and so
    the reference's golden routed output); over a subset it gives the same rows."""
    g = np.load(GOLD / "tiny_moe.npz")
    d = _tiny()
    _, tw, ti = O.router_reference(d["x"], d["gate"], None, topk=4)
    T = d["x"].shape[0]
    full = O.moe_mlp_rows(d["x"], d["w13"], d["w2"], tw, ti, list(range(T)))
    assert full.dtype == torch.float32
    assert np.array_equal(u16(full.to(BF16)), g["routed"])
    assert torch.equal(full.to(BF16), O.moe_mlp(d["x"], d["w13"], d["w2"], tw, ti))
    rows = [0, 3, 7, 15]
    sub = O.moe_mlp_rows(d["x"], d["w13"], d["w2"], tw, ti, rows)
    torch.testing.assert_close(sub, full[rows], rtol=1e-6, atol=1e-6)


def test_block_reference_vs_fp64_composition():
    """`block_reference` = bf16(routed + h + shared) against the same composition in
    fp64 (textbook GEMMs, exact SwiGLU, no intermediate rounding); with the shared
    weights zeroed it drops to bf16(moe_mlp + h), so a dropped or doubled term fails."""
    d = _tiny()
    _, tw, ti = O.router_reference(d["x"], d["gate"], None, topk=4)
    x, h = d["x"], d["act_in"][:, : d["x"].shape[1]].contiguous()
    got = O.block_reference(h, x, d["w13"], d["w2"], d["w13s"], d["w2s"], tw, ti)
    xd, hd = x.double().numpy(), h.double().numpy()
    w13, w2 = d["w13"].double().numpy(), d["w2"].double().numpy()
    w13s, w2s = d["w13s"][0].double().numpy(), d["w2s"][0].double().numpy()
    I = w2.shape[2]
    silu = lambda v: v / (1 + np.exp(-v))
    want = hd.copy()
    for t in range(xd.shape[0]):
        for j in range(ti.shape[1]):
            e = int(ti[t, j])
            g_ = w13[e] @ xd[t]
            want[t] += float(tw[t, j]) * (w2[e] @ (silu(g_[:I]) * g_[I:]))
        gs = w13s @ xd[t]
        want[t] += w2s @ (silu(gs[:I]) * gs[I:])
    err = np.abs(got.double().numpy() - want).max() / np.abs(want).max()
    assert err < 1e-2
    # the shared term is not negligible here, and zeroing it gives bf16(routed + h)
    shared_only = want - hd
    assert np.abs(shared_only).max() > 0.05 * np.abs(want).max()
    z13, z2 = torch.zeros_like(d["w13s"]), torch.zeros_like(d["w2s"])
    no_sh = O.block_reference(h, x, d["w13"], d["w2"], z13, z2, tw, ti)
    routed = O.moe_mlp(x, d["w13"], d["w2"], tw, ti)
    assert torch.equal(no_sh, (routed.float() + h.float()).to(BF16))
