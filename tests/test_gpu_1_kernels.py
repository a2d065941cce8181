"""GPU parity of each kernel against the CPU oracle, through the C-ABI library.

Integer and index outputs (ids, dispatch layout) and everything the exact front-end rule
fixes (h, y, logits, top-k weights) must match bit for bit; the grouped GEMMs are
checked against fp32 references of the same op within bf16 output rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from fusion_amd import _lib
from fusion_amd.dispatch import (align_workspace, capacity, decode_front_into,
                                 decode_norm_logits_into, moe_align_block_size,
                                 moe_align_block_size_into, route_gateup_shared_into,
                                 topk_align_into)
from fusion_amd.kernels import add_rmsnorm as KN
from fusion_amd.kernels import merge_resadd as KM
from fusion_amd.kernels import moe_down_merge as KD
from fusion_amd.kernels import moe_gateup as KG
from fusion_amd.kernels import norm_router as KR
from fusion_amd.problem import front_end, zipf_bias
from oracle import glm52_oracle as O

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def say(*a):
    print(*a, flush=True)


# ------------------------------------------------------------------ MFMA layout
def test_mfma_layout_selftest(gpu):
    out = torch.zeros(1536, dtype=torch.float32, device=gpu)
    _lib.call("glm52_selftest_mfma_layout", _lib.ptr(out), _lib.stream())
    m = out[:512].view(2, 16, 16).cpu()
    want = torch.arange(1, 17, dtype=torch.float32).unsqueeze(1).expand(16, 16)
    assert torch.equal(m[0], want), m[0]
    assert torch.equal(m[1], want), m[1]
    # 32x32x16: register i of lane l holds C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32] = 32 row + col
    got = out[512:].view(64, 16).cpu()
    lane = torch.arange(64).unsqueeze(1)
    i = torch.arange(16).unsqueeze(0)
    row = 8 * (i // 4) + 4 * (lane // 32) + i % 4
    col = (lane % 32).expand(64, 16)
    assert torch.equal(got, (32 * row + col).float()), got


# ------------------------------------------------------------------ ResAdd + RMSNorm
@pytest.mark.parametrize("T", [1, 7, 32, 600])
@pytest.mark.parametrize("mode", [None, 0, 1])
def test_add_rmsnorm_bitwise(gpu, T, mode):
    say(f"add_rmsnorm T={T} mode={mode}")
    fe = front_end(T)
    x, r, w = fe.x.to(gpu), fe.r.to(gpu), fe.w_norm.to(gpu)
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    cfg = {} if mode is None else {"WAVE_PER_ROW": mode}
    KN.fused_add_rmsnorm(x, r, w, h, y, cfg)
    y_o, h_o = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    assert np.array_equal(u16(h), u16(h_o))
    assert np.array_equal(u16(y), u16(y_o))
    # split kernels give the same bits
    h2, y2 = torch.empty_like(x), torch.empty_like(x)
    KN.add_only(x, r, h2, cfg)
    KN.norm_only(h2, w, y2, cfg)
    assert torch.equal(h2, h) and torch.equal(y2, y)


def test_add_rmsnorm_golden_config0(gpu):
    g = np.load("tests/golden/config0_t32.npz")
    fe = front_end(32)
    x, r, w = fe.x.to(gpu), fe.r.to(gpu), fe.w_norm.to(gpu)
    h, y = torch.empty_like(x), torch.empty_like(x)
    KN.fused_add_rmsnorm(x, r, w, h, y, {})
    assert np.array_equal(u16(h), g["h"])
    assert np.abs(u16(y).astype(np.int32) - g["y"].astype(np.int32)).max() <= 1


def test_add_rmsnorm_strided_rows(gpu):
    fe = front_end(16)
    big = torch.zeros(16, 6144 + 64, dtype=BF16, device=gpu)
    big[:, :6144] = fe.x.to(gpu)
    x = big[:, :6144]
    r, w = fe.r.to(gpu), fe.w_norm.to(gpu)
    h, y = torch.empty_like(r), torch.empty_like(r)
    KN.fused_add_rmsnorm(x, r, w, h, y, {})
    y_o, h_o = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    assert np.array_equal(u16(y), u16(y_o))


# ------------------------------------------------------------------ router
@pytest.mark.parametrize("T,bias", [(1, "normal"), (3, "normal"), (8, "zipf"), (13, "zipf"),
                                    (32, "normal"), (100, "zero"), (256, "normal"),
                                    (2048, "normal"), (2048, "zipf")])
def test_router_bitwise(gpu, T, bias):
    say(f"router T={T} bias={bias}")
    fe = front_end(T, bias=bias)
    y_o, _ = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    y = y_o.to(gpu)
    wgt = fe.wgt.to(gpu)
    logits = torch.empty(T, 256, dtype=torch.float32, device=gpu)
    KR.router_gemm(y, wgt, logits, {})
    lg_o = O.router_logits_exact(y_o, fe.wgt)
    lg = logits.cpu().numpy()
    assert (lg != lg_o).sum() == 0, f"{(lg != lg_o).sum()} logits differ"
    topw = torch.empty(T, 8, dtype=torch.float32, device=gpu)
    topi = torch.empty(T, 8, dtype=torch.int32, device=gpu)
    b = None if bias == "zero" else fe.bias
    KR.topk_only(logits, topw, topi, {"correction_bias": None if b is None else b.to(gpu)})
    w_o, ids_o, _ = O.router_select(lg_o, None if b is None else b.numpy(), 8)
    assert np.array_equal(topi.cpu().numpy(), ids_o)
    assert np.array_equal(topw.cpu().numpy(), w_o)
    # the two-launch router (split-K partials reduced inside top-k) gives the same bits
    cfg = {"correction_bias": None if b is None else b.to(gpu)}
    lg2 = torch.full_like(logits, float("nan"))
    topw2, topi2 = torch.empty_like(topw), torch.empty_like(topi)
    KR.router(y, wgt, lg2, topw2, topi2, cfg)
    assert torch.equal(lg2, logits) and torch.equal(topw2, topw) and torch.equal(topi2, topi)
    # the transposed-gate mapping (a wave per gate row) gives the same bits
    rows = fe.gate.to(gpu).t()  # [H, E] view of the contiguous [E, H] gate
    lg3 = torch.full_like(logits, float("nan"))
    KR.router_gemm(y, rows, lg3, {})
    assert torch.equal(lg3, logits)
    if T * 8 <= 256:  # the fused top-k + layout launch
        for bm in (16, 64):
            cap = capacity(T * 8, bm, 256)
            sti = torch.empty(cap, dtype=torch.int32, device=gpu)
            eids = torch.empty(cap // bm, dtype=torch.int32, device=gpu)
            ntp = torch.empty(1, dtype=torch.int32, device=gpu)
            topw4, topi4 = torch.empty_like(topw), torch.empty_like(topi)
            topk_align_into(logits, topw4, topi4, cfg, bm, 256, sti, eids, ntp)
            assert torch.equal(topw4, topw) and torch.equal(topi4, topi)
            rs, re_, rn = O.moe_align_block_size(ids_o, bm, 256)
            n = int(rn[0])
            assert int(ntp.item()) == n
            assert np.array_equal(sti.cpu().numpy()[:n], rs)
            assert np.array_equal(eids.cpu().numpy()[: n // bm], re_)
            assert (sti.cpu().numpy()[n:] == T * 8).all() and (eids.cpu().numpy()[n // bm:] == -1).all()


def test_router_golden_config0(gpu):
    g = np.load("tests/golden/config0_t32.npz")
    fe = front_end(32)
    x, r, w = fe.x.to(gpu), fe.r.to(gpu), fe.w_norm.to(gpu)
    h, y = torch.empty_like(x), torch.empty_like(x)
    KN.fused_add_rmsnorm(x, r, w, h, y, {})
    topw = torch.empty(32, 8, dtype=torch.float32, device=gpu)
    topi = torch.empty(32, 8, dtype=torch.int32, device=gpu)
    KR.fused_norm_router_topk(h, w, y, fe.wgt.to(gpu), topw, topi,
                              {"correction_bias": fe.bias.to(gpu)})
    assert np.array_equal(topi.cpu().numpy(), g["topk_ids"])
    np.testing.assert_allclose(topw.cpu().numpy(), g["topk_weights"], rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T", [1, 2, 3, 4])
@pytest.mark.parametrize("bias", ["normal", "zipf", "zero"])
def test_decode_front_bitwise(gpu, T, bias):
    """The one-launch decode front end against the oracle's exact rule, on three
    launches in a row (the arrival counter must come back to zero after each)."""
    say(f"decode front T={T} bias={bias}")
    fe = front_end(T, bias=bias)
    x, r, w = fe.x.to(gpu), fe.r.to(gpu), fe.w_norm.to(gpu)
    gate_rows = fe.gate.to(gpu).contiguous()
    b = None if bias == "zero" else fe.bias.to(gpu)
    cfg = {"correction_bias": b}
    y_o, h_o = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    lg_o, w_o, ids_o = O.router_exact(y_o, fe.wgt, None if b is None else fe.bias.numpy())
    bm = 16
    rs, re_, rn = O.moe_align_block_size(ids_o, bm, 256)
    n = int(rn[0])
    cap = capacity(T * 8, bm, 256)
    counter = torch.zeros(1, dtype=torch.int32, device=gpu)
    for rep in range(3):
        h, y = torch.full_like(x, float("nan")), torch.full_like(x, float("nan"))
        logits = torch.full((T, 256), float("nan"), device=gpu)
        topw = torch.empty(T, 8, dtype=torch.float32, device=gpu)
        topi = torch.empty(T, 8, dtype=torch.int32, device=gpu)
        sti = torch.empty(cap, dtype=torch.int32, device=gpu)
        eids = torch.empty(cap // bm, dtype=torch.int32, device=gpu)
        ntp = torch.empty(1, dtype=torch.int32, device=gpu)
        decode_front_into(x, r, w, h, y, gate_rows, cfg, logits, topw, topi, bm, sti, eids, ntp,
                          counter)
        torch.cuda.synchronize()
        assert int(counter.item()) == 0, "arrival counter not reset"
        assert np.array_equal(u16(h), u16(h_o)) and np.array_equal(u16(y), u16(y_o))
        assert np.array_equal(logits.cpu().numpy(), lg_o)
        assert np.array_equal(topi.cpu().numpy(), ids_o)
        assert np.array_equal(topw.cpu().numpy(), w_o)
        assert int(ntp.item()) == n
        assert np.array_equal(sti.cpu().numpy()[:n], rs)
        assert np.array_equal(eids.cpu().numpy()[: n // bm], re_)
        assert (sti.cpu().numpy()[n:] == T * 8).all() and (eids.cpu().numpy()[n // bm:] == -1).all()


def test_decode_front_rejects_large_T(gpu):
    T = 5
    fe = front_end(T)
    x = fe.x.to(gpu)
    gate_rows = fe.gate.to(gpu).contiguous()
    cap = capacity(T * 8, 16, 256)
    bufs = [torch.empty(cap, dtype=torch.int32, device=gpu),
            torch.empty(cap // 16, dtype=torch.int32, device=gpu),
            torch.empty(1, dtype=torch.int32, device=gpu)]
    with pytest.raises(RuntimeError, match="invalid argument"):
        decode_front_into(x, x, fe.w_norm.to(gpu), x.clone(), x.clone(), gate_rows,
                          {"correction_bias": fe.bias.to(gpu)},
                          torch.empty(T, 256, device=gpu), torch.empty(T, 8, device=gpu),
                          torch.empty(T, 8, dtype=torch.int32, device=gpu), 16, *bufs,
                          torch.zeros(1, dtype=torch.int32, device=gpu))


@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_decode_norm_logits_bitwise(gpu, T):
    """ResAdd + RMSNorm and the router logits in one launch: the oracle's exact rule."""
    say(f"decode norm+logits T={T}")
    fe = front_end(T, seed=900 + T)
    x, r, w = fe.x.to(gpu), fe.r.to(gpu), fe.w_norm.to(gpu)
    gate_rows = fe.gate.to(gpu).contiguous()
    y_o, h_o = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    lg_o = O.router_logits_exact(y_o, fe.wgt)
    for rep in range(2):
        h, y = torch.full_like(x, float("nan")), torch.full_like(x, float("nan"))
        logits = torch.full((T, 256), float("nan"), device=gpu)
        decode_norm_logits_into(x, r, w, h, y, gate_rows, logits)
        torch.cuda.synchronize()
        assert np.array_equal(u16(h), u16(h_o)) and np.array_equal(u16(y), u16(y_o))
        assert np.array_equal(logits.cpu().numpy(), lg_o)


def _route_logits(T, kind, rng):
    """Router logits for the routing-launch test: random, or drawn from a few values so
    that many keys tie, or with NaNs (their key counts as -inf)."""
    if kind == "ties":
        lg = rng.choice(np.array([-1.0, 0.0, 0.5, 2.0], dtype=np.float32), size=(T, 256))
        lg[:, 200:] = 2.0  # more tied maxima than slots: lower index first
    else:
        lg = rng.standard_normal((T, 256)).astype(np.float32)
    if kind == "nan":
        lg[:, rng.choice(256, 40, replace=False)] = np.nan
        lg[0, 3:] = np.nan  # token 0: only 3 finite keys, so NaN experts fill the top-8
    return lg.astype(np.float32)


ROUTE_CASES = [(1, "normal", "normal", 8, True), (2, "zero", "normal", 8, True),
               (3, "normal", "ties", 8, True), (4, "zipf", "normal", 8, True),
               (4, "none", "ties", 8, True), (2, "normal", "nan", 8, True),
               (3, "normal", "normal", 6, False), (4, "zipf", "normal", 8, False)]


@pytest.mark.parametrize("T,bias,kind,topk,norm", ROUTE_CASES)
def test_route_gateup_shared_bitwise(gpu, T, bias, kind, topk, norm):
    """The decode w13 launch that derives the routing itself: ids, weights and dispatch
    layout bit for bit against the oracle's rule, and the activations bit for bit against
    the launch that reads the oracle's layout (`moe_gemm_shared`), on two launches in a row
    over buffers filled with garbage."""
    say(f"route+gateup T={T} bias={bias} kind={kind} topk={topk} norm={norm}")
    rng = np.random.default_rng(1000 * T + topk + len(kind))
    E, H, I = 256, 1024, 256
    lg = _route_logits(T, kind, rng)
    if bias == "none":
        b = None
    elif bias == "zero":
        b = np.zeros(E, dtype=np.float32)
    elif bias == "zipf":
        b = zipf_bias(E).numpy()
    else:
        b = (0.01 * rng.standard_normal(E)).astype(np.float32)
    if kind == "ties" and b is not None:
        b = rng.choice(np.array([0.0, 0.25], dtype=np.float32), size=E)
    scale = 2.5
    w_o, ids_o, _ = O.router_select(lg, b, topk, scale, norm)
    rs, re_, rn = O.moe_align_block_size(ids_o, 16, E)
    n = int(rn[0])
    R = T * topk
    cap = capacity(R, 16, E)

    torch.manual_seed(T)
    a = torch.randn(T, H, device=gpu).to(BF16)
    w13 = (torch.randn(E, 2 * I, H, device=gpu) * 0.05).to(BF16)
    w13s = (torch.randn(1, 2 * I, H, device=gpu) * 0.05).to(BF16)
    cfg = {"correction_bias": None if b is None else torch.from_numpy(b).to(gpu),
           "scale": scale, "NORM_PROB": norm}
    # the same activations from the launch that reads the oracle's layout
    sti_o = torch.full((cap,), R, dtype=torch.int32)
    sti_o[:n] = torch.from_numpy(rs)
    eids_o = torch.full((cap // 16,), -1, dtype=torch.int32)
    eids_o[: n // 16] = torch.from_numpy(re_)
    sti_o, eids_o, ntp_o = sti_o.to(gpu), eids_o.to(gpu), torch.from_numpy(rn).to(gpu)
    act_ref = torch.empty(R, I, dtype=BF16, device=gpu)
    act_s_ref = torch.empty(T, I, dtype=BF16, device=gpu)
    KG.moe_gemm_shared(a, topk, w13, act_ref, None, sti_o, eids_o, ntp_o, R, I, I, True,
                       {"BLOCK_M": 16}, a, w13s, act_s_ref)
    logits = torch.from_numpy(lg).to(gpu)
    for rep in range(2):
        topw = torch.full((T, topk), float("nan"), device=gpu)
        topi = torch.full((T, topk), -7, dtype=torch.int32, device=gpu)
        sti = torch.full((cap,), -7, dtype=torch.int32, device=gpu)
        eids = torch.full((cap // 16,), -7, dtype=torch.int32, device=gpu)
        ntp = torch.full((1,), -7, dtype=torch.int32, device=gpu)
        act = torch.full((R, I), float("nan"), dtype=BF16, device=gpu)
        act_s = torch.full((T, I), float("nan"), dtype=BF16, device=gpu)
        route_gateup_shared_into(logits, cfg, topw, topi, sti, eids, ntp, a, w13, act, a, w13s,
                                 act_s)
        torch.cuda.synchronize()
        assert np.array_equal(topi.cpu().numpy(), ids_o)
        np.testing.assert_array_equal(topw.cpu().numpy(), w_o)  # NaN where the oracle has NaN
        assert int(ntp.item()) == n
        s_, e_ = sti.cpu().numpy(), eids.cpu().numpy()
        assert np.array_equal(s_[:n], rs) and np.array_equal(e_[: n // 16], re_)
        assert (s_[n:] == R).all() and (e_[n // 16:] == -1).all()
        assert torch.equal(act, act_ref) and torch.equal(act_s, act_s_ref)


def test_route_gateup_shared_rejects_bad_shapes(gpu):
    T, E, H, I = 5, 256, 512, 64
    z = lambda *s, dt=torch.float32: torch.zeros(*s, dtype=dt, device=gpu)  # noqa: E731
    a, w13 = z(T, H, dt=BF16), z(E, 2 * I, H, dt=BF16)
    cap = capacity(T * 8, 16, E)
    with pytest.raises(RuntimeError, match="invalid argument"):
        route_gateup_shared_into(z(T, E), {"correction_bias": z(E)}, z(T, 8),
                                 z(T, 8, dt=torch.int32), z(cap, dt=torch.int32),
                                 z(cap // 16, dt=torch.int32), z(1, dt=torch.int32), a, w13,
                                 z(T * 8, I, dt=BF16), a, w13[:1], z(T, I, dt=BF16))


# ------------------------------------------------------------------ dispatch layout
@pytest.mark.parametrize("T,E,k,bm", [(1, 256, 8, 16), (32, 256, 8, 16), (256, 256, 8, 16),
                                      (2048, 256, 8, 64), (8192, 256, 8, 128), (300, 1, 1, 16),
                                      (8192, 1, 1, 128), (77, 256, 8, 32)])
def test_moe_align_bitwise(gpu, T, E, k, bm):
    say(f"align T={T} E={E} bm={bm}")
    rng = np.random.default_rng(T + bm)
    if E == 1:
        ids = np.zeros((T, 1), dtype=np.int32)
    else:
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    sti, eids, ntp = moe_align_block_size(torch.from_numpy(ids).to(gpu), bm, E)
    rs, re_, rn = O.moe_align_block_size(ids, bm, E)
    n = int(rn[0])
    assert int(ntp.item()) == n
    s, e = sti.cpu().numpy(), eids.cpu().numpy()
    assert np.array_equal(s[:n], rs)
    assert np.array_equal(e[: n // bm], re_)
    assert (s[n:] == ids.size).all() and (e[n // bm:] == -1).all()
    assert s.size == capacity(ids.size, bm, E)


def test_moe_align_skewed_routing(gpu):
    """Configuration 4's Zipf bias concentrates thousands of slots on a few experts."""
    T = 8192
    fe = front_end(T, bias="zipf")
    y_o, _ = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    _, _, ids = O.router_exact(y_o, fe.wgt, zipf_bias().numpy())
    for bm in (16, 128):
        sti, eids, ntp = moe_align_block_size(torch.from_numpy(ids).to(gpu), bm, 256)
        rs, re_, rn = O.moe_align_block_size(ids, bm, 256)
        n = int(rn[0])
        assert int(ntp.item()) == n
        assert np.array_equal(sti.cpu().numpy()[:n], rs)
        assert np.array_equal(eids.cpu().numpy()[: n // bm], re_)


@pytest.mark.parametrize("numel,E,bm", [(2049, 256, 16), (4096, 7, 64), (30000, 160, 32),
                                         (65536 + 13, 256, 128)])
def test_moe_align_chunked_matches_single(gpu, numel, E, bm):
    """The multi-workgroup layout (two launches over chunks of 2048 ids) against the
    single-workgroup one, bit for bit, on ragged sizes with ids outside [0, E) mixed in
    (both skip them), and against the oracle on the valid ids alone."""
    say(f"align chunked numel={numel} E={E} bm={bm}")
    rng = np.random.default_rng(numel + E)
    ids = rng.integers(-2, E + 2, size=numel).astype(np.int32)
    t = torch.from_numpy(ids).to(gpu)
    cap = capacity(numel, bm, E)
    # a workspace of ceil(numel / 2048) * E histograms selects the chunked build at any size
    ws = torch.empty(-(-numel // 2048) * E, dtype=torch.int32, device=gpu)
    want = align_workspace(numel, E, gpu)
    assert (want is None) == (numel < 16384)
    assert want is None or want.numel() == ws.numel()
    got = []
    for w in (None, ws):
        sti = torch.full((cap,), -7, dtype=torch.int32, device=gpu)
        eids = torch.full((cap // bm,), -7, dtype=torch.int32, device=gpu)
        ntp = torch.full((1,), -7, dtype=torch.int32, device=gpu)
        moe_align_block_size_into(t, bm, E, sti, eids, ntp, w)
        got.append((sti.cpu(), eids.cpu(), ntp.cpu()))
    for a, b in zip(*got):
        assert torch.equal(a, b)
    valid = np.where((ids >= 0) & (ids < E), ids, E)  # an extra expert E collects the rest
    rs, re_, rn = O.moe_align_block_size(valid, bm, E + 1)
    n = int(got[1][2][0])
    keep = re_ < E  # drop the extra expert's blocks, which come last
    assert n == int(keep.sum()) * bm
    assert np.array_equal(got[1][0].numpy()[:n], rs[:n])
    assert np.array_equal(got[1][1].numpy()[: n // bm], re_[keep])


# ------------------------------------------------------------------ grouped GEMMs
def _gemm_problem(T, E, H, I, k, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(T, H, generator=g).to(BF16)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(BF16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.05).to(BF16)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    tw = torch.rand(T, k, generator=g)
    return a, w13, w2, ids, tw


def _gateup_ref(a, w13, ids, k, I, fused):
    """fp32 reference of the gated GEMM: rows by flat token f = t * k + j."""
    T = a.shape[0]
    out = torch.zeros(T * k, I if fused else 2 * I)
    af = a.float()
    flat = ids.reshape(-1)
    for e in torch.unique(flat).tolist():
        f = (flat == e).nonzero().view(-1)
        hh = af[f // k] @ w13[e].float().t()
        out[f] = (torch.nn.functional.silu(hh[:, :I]) * hh[:, I:]) if fused else hh
    return out


def _down_ref(act, w2, ids, tw):
    actf = act.float().cpu()
    flat = ids.reshape(-1)
    twf = tw.reshape(-1)
    out = torch.zeros(actf.shape[0], w2.shape[1])
    for e in torch.unique(flat).tolist():
        f = (flat == e).nonzero().view(-1)
        out[f] = twf[f].unsqueeze(1) * (actf[f] @ w2[e].float().t())
    return out


def _close(got: torch.Tensor, ref: torch.Tensor, what: str):
    got = got.float().cpu()
    tol = ref.abs() * 2 ** -7 + 1e-2 * ref.abs().max() * 2 ** -7
    bad = ((got - ref).abs() > tol).sum().item()
    assert bad == 0, f"{what}: {bad} elements outside bf16 rounding of the fp32 reference"


@pytest.mark.parametrize("bm,variant", [(16, "stream"), (32, "tiled"), (64, "tiled"),
                                        (128, "tiled"), (64, "stream"), (64, "wide"),
                                        (128, "wide"),
                                        (64, "w512"), (128, "w512"), (128, None)])
def test_grouped_gemms_small(gpu, bm, variant):
    say(f"grouped gemm small bm={bm} {variant}")
    T, E, H, I, k = 40, 16, 512, 256, 8
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 21 + bm, gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), bm, E)
    cfg = {"BLOCK_M": bm, "variant": variant}
    ag, w13g, w2g = a.to(gpu), w13.to(gpu), w2.to(gpu)
    act = torch.full((T * k, I), float("nan"), dtype=BF16, device=gpu)
    KG.launch_gateup(ag, w13g, act, sti, eids, ntp, T * k, k, I, cfg, True)
    act_ref = _gateup_ref(a, w13, ids, k, I, True)
    _close(act, act_ref, "w13+SwiGLU")
    # unfused: [R, 2I] then the split-out SwiGLU
    inter = torch.empty(T * k, 2 * I, dtype=BF16, device=gpu)
    KG.launch_gateup(ag, w13g, inter, sti, eids, ntp, T * k, k, I, cfg, False)
    _close(inter, _gateup_ref(a, w13, ids, k, I, False), "w13 unfused")
    act2 = torch.empty(T * k, I, dtype=BF16, device=gpu)
    KG.launch_silu_and_mul(inter, act2, {})
    d = u16(act2).astype(np.int32) - u16(O.silu_and_mul(inter.cpu())).astype(np.int32)
    assert np.abs(d).max() <= 1  # device exp vs torch's silu: at most one bf16 ulp
    # down GEMM, routing weight applied in the epilogue
    y = torch.full((T * k, H), float("nan"), dtype=BF16, device=gpu)
    twf = tw.reshape(-1).contiguous()
    KD.launch_down(act, w2g, y, twf.to(gpu), sti, eids, ntp, T * k, k, cfg, False)
    _close(y, _down_ref(act, w2, ids, tw), "w2 weighted")


def test_grouped_gemm_full_width(gpu):
    """Real GLM-5.2 widths (H = 6144, I = 2048) on a few experts, both mappings."""
    T, E, H, I, k = 24, 4, 6144, 2048, 2
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 5, gpu)
    ag, w13g, w2g = a.to(gpu), w13.to(gpu), w2.to(gpu)
    act_ref = _gateup_ref(a, w13, ids, k, I, True)
    for bm, variant in ((16, "stream"), (16, "runs"), (32, "tiled"), (64, "wide"), (128, "wide"),
                        (64, "w512"), (128, "w512")):
        say(f"grouped gemm full width bm={bm} {variant}")
        sti, eids, ntp = moe_align_block_size(ids.to(gpu), bm, E)
        cfg = {"BLOCK_M": bm, "variant": variant}
        act = torch.empty(T * k, I, dtype=BF16, device=gpu)
        KG.launch_gateup(ag, w13g, act, sti, eids, ntp, T * k, k, I, cfg, True)
        _close(act, act_ref, f"w13 {variant}")
        y = torch.empty(T * k, H, dtype=BF16, device=gpu)
        twf = tw.reshape(-1).contiguous()
        KD.launch_down(act, w2g, y, twf.to(gpu), sti, eids, ntp, T * k, k, cfg, False)
        _close(y, _down_ref(act, w2, ids, tw), f"w2 {variant}")


@pytest.mark.parametrize("bm", [64, 128, 256])
@pytest.mark.parametrize("T,E,H,I", [(300, 8, 512, 256), (200, 8, 6144, 2048)])
def test_packed_w512_matches_unpacked(gpu, bm, T, E, H, I):
    """The prefill GEMM on packed weights: the same bits as on the weights in place, for the
    gated w13 + SwiGLU, the weighted w2 and the plain (shared-expert) w2.  At block size 256
    (the 256 x 256 tiles) T = 300 gives each expert a second block of 44 real rows, so the
    waves whose 128 token rows are all padding take the path that only stages loads."""
    say(f"packed w512 bm={bm} T={T} E={E} H={H} I={I}")
    k = 8  # every slot of the layout is routed (E >= k distinct ids per token)
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 60 + bm, gpu)
    ag, w13g, w2g = a.to(gpu), w13.to(gpu), w2.to(gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), bm, E)
    cfg = {"BLOCK_M": bm, "variant": "w512"}
    R = T * k
    w13p = KG.pack_w512(w13g, I, I, True)
    w2p = KG.pack_w512(w2g, H, 0, False)
    assert w13p.numel() == w13g.numel() and w2p.numel() == w2g.numel()
    act = torch.empty(R, I, dtype=BF16, device=gpu)
    KG.moe_gemm(ag, k, w13g, act, None, sti, eids, ntp, R, I, I, True, cfg)
    act_p = torch.full_like(act, float("nan"))
    KG.moe_gemm_packed(ag, k, w13p, act_p, None, sti, eids, ntp, R, I, True, cfg)
    twf = tw.reshape(-1).contiguous().to(gpu)
    y = torch.empty(R, H, dtype=BF16, device=gpu)
    KG.moe_gemm(act, 1, w2g, y, twf, sti, eids, ntp, R, H, 0, False, cfg)
    y_p = torch.full_like(y, float("nan"))
    KG.moe_gemm_packed(act, 1, w2p, y_p, twf, sti, eids, ntp, R, H, False, cfg)
    y0 = torch.empty(R, H, dtype=BF16, device=gpu)
    KG.moe_gemm(act, 1, w2g, y0, None, sti, eids, ntp, R, H, 0, False, cfg)
    y0_p = torch.full_like(y0, float("nan"))
    KG.moe_gemm_packed(act, 1, w2p, y0_p, None, sti, eids, ntp, R, H, False, cfg)
    torch.cuda.synchronize()
    assert torch.equal(act_p, act)
    assert torch.equal(y_p, y)
    assert torch.equal(y0_p, y0)
    _close(act, _gateup_ref(a, w13, ids, k, I, True), "w13 (packed path reference)")
    _close(y, _down_ref(act, w2, ids, tw), "w2 weighted (packed path reference)")


@pytest.mark.parametrize("bm", [64, 128, 256])
@pytest.mark.parametrize("T", [77, 300])
def test_moe_gemm_packed_shared_matches_separate_launches(gpu, bm, T):
    """Routed + shared expert in one prefill launch (`moe_gemm_packed_shared`, the shared
    expert's row blocks after each XCD's routed items): the same bits as the routed launch
    and a separate launch over the shared expert's one-expert layout, with T rows not a
    multiple of the block size (the last shared block partly padding)."""
    from fusion_amd.block import shared_layout

    say(f"moe_gemm_packed_shared bm={bm} T={T}")
    E, H, I, k = 8, 512, 256, 8
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 500 + T + bm, gpu)
    g = torch.Generator().manual_seed(900 + T)
    w13s = (torch.randn(1, 2 * I, H, generator=g) * 0.05).to(BF16).to(gpu)
    w2s = (torch.randn(1, H, I, generator=g) * 0.05).to(BF16).to(gpu)
    ag = a.to(gpu)
    w13p, w2p = KG.pack_w512(w13.to(gpu), I, I, True), KG.pack_w512(w2.to(gpu), H, 0, False)
    w13sp, w2sp = KG.pack_w512(w13s, I, I, True), KG.pack_w512(w2s, H, 0, False)
    twf = tw.reshape(-1).contiguous().to(gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), bm, E)
    ssti, seids, sntp = shared_layout(T, bm, gpu)
    cfg = {"BLOCK_M": bm}
    R = T * k
    act, act_s = torch.empty(R, I, dtype=BF16, device=gpu), torch.empty(T, I, dtype=BF16, device=gpu)
    KG.moe_gemm_packed(ag, k, w13p, act, None, sti, eids, ntp, R, I, True, cfg)
    KG.moe_gemm_packed(ag, 1, w13sp, act_s, None, ssti, seids, sntp, T, I, True, cfg)
    y, s_out = torch.empty(R, H, dtype=BF16, device=gpu), torch.empty(T, H, dtype=BF16, device=gpu)
    KG.moe_gemm_packed(act, 1, w2p, y, twf, sti, eids, ntp, R, H, False, cfg)
    KG.moe_gemm_packed(act_s, 1, w2sp, s_out, None, ssti, seids, sntp, T, H, False, cfg)
    act2, act_s2 = torch.full_like(act, float("nan")), torch.full_like(act_s, float("nan"))
    KG.moe_gemm_packed_shared(ag, k, w13p, act2, None, sti, eids, ntp, R, I, True, cfg, ag, w13sp,
                              act_s2)
    y2, s_out2 = torch.full_like(y, float("nan")), torch.full_like(s_out, float("nan"))
    KG.moe_gemm_packed_shared(act2, 1, w2p, y2, twf, sti, eids, ntp, R, H, False, cfg, act_s2,
                              w2sp, s_out2)
    torch.cuda.synchronize()
    assert torch.equal(act2, act) and torch.equal(act_s2, act_s)
    assert torch.equal(y2, y) and torch.equal(s_out2, s_out)
    _close(act_s, _gateup_ref(a, w13s.cpu(), torch.zeros(T, 1, dtype=torch.int32), 1, I, True),
           "shared w13 (fp32 reference)")


@pytest.mark.parametrize("bm", [64, 128, 256])
def test_w512_item_dealing(gpu, bm):
    """The prefill tile deals its items from per-XCD counters that the last workgroup out
    clears, one counter set per launch out of 64 in turn.  (1) A layout block with no real
    row (the workgroup fetches the next item at once) leaves the results as they are
    without it.  (2) 70 launches in a row (more than the 64 sets, so every set is reused
    after it was cleared) all give the first launch's bits.  (3) Two launches issued on two
    streams at once give the bits of the same launches in order."""
    say(f"w512 item dealing bm={bm}")
    T, E, H, I, k = 300, 8, 512, 256, 8
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 700 + bm, gpu)
    ag = a.to(gpu)
    w13p, w2p = KG.pack_w512(w13.to(gpu), I, I, True), KG.pack_w512(w2.to(gpu), H, 0, False)
    twf = tw.reshape(-1).contiguous().to(gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), bm, E)
    cfg = {"BLOCK_M": bm}
    R = T * k
    nan = float("nan")

    def gateup(layout, out):
        KG.moe_gemm_packed(ag, k, w13p, out, None, *layout, R, I, True, cfg)

    def down(layout, x, out):
        KG.moe_gemm_packed(x, 1, w2p, out, twf, *layout, R, H, False, cfg)

    act = torch.full((R, I), nan, dtype=BF16, device=gpu)
    gateup((sti, eids, ntp), act)
    y = torch.full((R, H), nan, dtype=BF16, device=gpu)
    down((sti, eids, ntp), act, y)
    torch.cuda.synchronize()
    _close(y, _down_ref(act, w2, ids, tw), "w2 weighted")

    # (1) an all-padding block (sentinel rows) inside the run of the middle block's expert
    n = int(ntp.item())
    nb, b = n // bm, n // bm // 2
    s, e_ = sti.cpu(), eids.cpu()
    sti2 = torch.cat([s[: b * bm], torch.full((bm,), R, dtype=torch.int32), s[b * bm: n]])
    eids2 = torch.cat([e_[:b], e_[b: b + 1], e_[b:nb]])
    lay2 = (sti2.to(gpu), eids2.to(gpu), torch.tensor([n + bm], dtype=torch.int32, device=gpu))
    act2 = torch.full_like(act, nan)
    gateup(lay2, act2)
    y2 = torch.full_like(y, nan)
    down(lay2, act2, y2)
    torch.cuda.synchronize()
    assert torch.equal(act2, act) and torch.equal(y2, y)

    # (2) launches in a row, every output refilled first
    y3 = torch.empty_like(y)
    for i in range(70):
        y3.fill_(nan)
        down((sti, eids, ntp), act, y3)
        assert torch.equal(y3, y), f"launch {i}"

    # (3) two streams at once (default priority)
    act4, y4 = torch.full_like(act, nan), torch.full_like(y, nan)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        gateup((sti, eids, ntp), act4)
    with torch.cuda.stream(s2):
        down((sti, eids, ntp), act, y4)
    torch.cuda.synchronize()
    assert torch.equal(act4, act) and torch.equal(y4, y)


def test_w512_item_trace_record(gpu):
    """The prefill tile's measurement hook: every workgroup's record has its start before
    its end, an XCD below 8, and the records' item counts add up to the launch's items (one
    item per 256-token block and 256-output tile, T = 1000 on 8 experts); with the hook off
    again nothing more is written."""
    T, E, H, I, k = 1000, 8, 512, 256, 8
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 811, gpu)
    w2p = KG.pack_w512(w2.to(gpu), H, 0, False)
    act = (torch.randn(T * k, I, generator=torch.Generator().manual_seed(3)) * 0.5).to(BF16).to(gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), 256, E)
    y = torch.empty(T * k, H, dtype=BF16, device=gpu)
    rec = torch.zeros(256 * 4, dtype=torch.int64, device=gpu)
    _lib.call("glm52_debug_item_trace", _lib.ptr(rec), rec.numel() * 8)
    try:
        KG.moe_gemm_packed(act, 1, w2p, y, None, sti, eids, ntp, T * k, H, False, {"BLOCK_M": 256})
        torch.cuda.synchronize()
    finally:
        _lib.call("glm52_debug_item_trace", None, 0)
    r = rec.view(256, 4).cpu()
    used = r[:, 0] > 0
    assert bool((r[used, 1] >= r[used, 0]).all()) and bool((r[used, 3] < 8).all())
    blocks = int(ntp.item()) // 256
    assert int(r[used, 2].sum()) == blocks * (H // 256)
    rec.zero_()
    KG.moe_gemm_packed(act, 1, w2p, y, None, sti, eids, ntp, T * k, H, False, {"BLOCK_M": 256})
    torch.cuda.synchronize()
    assert int(rec.abs().sum()) == 0


@pytest.mark.parametrize("T", [1, 3, 16, 40, 160])
def test_packed_weight_stream_matches_in_place(gpu, T):
    """The decode weight stream (block size 16) on packed weights, routed and shared expert
    in one launch: the same bits as on the weights in place -- gated w13 + SwiGLU, weighted
    w2, both with two packed slots per item (K = 1024; the gated launch from 1024 routed
    rows, T = 160) -- and the packed token-major tail within one bf16 rounding step of the in-place one
    (it adds in another order; 1e-3 absolute where the sum cancels) and both within bf16
    rounding of the fp32 reference."""
    E, H, I, k = 8, 1024, 1024, 8
    say(f"packed weight stream T={T} E={E} H={H} I={I}")
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 90 + T, gpu)
    ag, w13g, w2g = a.to(gpu), w13.to(gpu), w2.to(gpu)
    g = torch.Generator().manual_seed(5)
    w13s = (torch.randn(1, 2 * I, H, generator=g) * 0.02).to(BF16).to(gpu)
    w2s = (torch.randn(1, H, I, generator=g) * 0.02).to(BF16).to(gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), 16, E)
    cfg = {"BLOCK_M": 16}
    R = T * k
    w13p, w2p = KG.pack_w512(w13g, I, I, True), KG.pack_w512(w2g, H, 0, False)
    w13sp, w2sp = KG.pack_w512(w13s, I, I, True), KG.pack_w512(w2s, H, 0, False)
    act = torch.empty(R, I, dtype=BF16, device=gpu)
    act_s = torch.empty(T, I, dtype=BF16, device=gpu)
    KG.moe_gemm_shared(ag, k, w13g, act, None, sti, eids, ntp, R, I, I, True, cfg, ag, w13s,
                       act_s)
    act_p, act_sp = torch.full_like(act, float("nan")), torch.full_like(act_s, float("nan"))
    KG.moe_gemm_packed_shared(ag, k, w13p, act_p, None, sti, eids, ntp, R, I, True, cfg, ag,
                              w13sp, act_sp)
    twf = tw.reshape(-1).contiguous().to(gpu)
    y = torch.empty(R, H, dtype=BF16, device=gpu)
    s_out = torch.empty(T, H, dtype=BF16, device=gpu)
    KG.moe_gemm_shared(act, 1, w2g, y, twf, sti, eids, ntp, R, H, 0, False, cfg, act_s, w2s,
                       s_out)
    y_p, s_p = torch.full_like(y, float("nan")), torch.full_like(s_out, float("nan"))
    KG.moe_gemm_packed_shared(act, 1, w2p, y_p, twf, sti, eids, ntp, R, H, False, cfg, act_s,
                              w2sp, s_p)
    # the token-major tail, both layouts, + a residual
    h = (torch.randn(T, H, generator=g) * 0.5).to(BF16).to(gpu)
    twg, idg = tw.to(gpu).float().contiguous(), ids.to(gpu).int().contiguous()
    out = torch.empty(T, H, dtype=BF16, device=gpu)
    KD.launch_down_token_major(act, w2g, out, twg, idg, h, k, {}, True, act_s, w2s)
    out_p = torch.full_like(out, float("nan"))
    KD.launch_down_token_major_packed(act, w2p, out_p, twg, idg, h, k, True, act_s, w2sp)
    torch.cuda.synchronize()
    assert torch.equal(act_p, act)
    assert torch.equal(act_sp, act_s)
    assert torch.equal(y_p, y)
    assert torch.equal(s_p, s_out)
    # one bf16 rounding step apart, plus the fp32 reordering where the sum cancels
    d = (out_p.float() - out.float()).abs()
    assert (d <= torch.maximum(out_p.float().abs(), out.float().abs()) * 2.0 ** -7 + 1e-3).all()
    ref = h.float() + act_s.float() @ w2s[0].float().t()
    for t in range(T):
        for j in range(k):
            ref[t] += twg[t, j] * (act[t * k + j].float() @ w2g[idg[t, j]].float().t())
    _close(out_p, ref.cpu(), "token-major tail on packed weights")
    _close(out, ref.cpu(), "token-major tail in place")
    _close(act, _gateup_ref(a, w13, ids, k, I, True), "w13 (weight stream reference)")


def test_pack_w512_rejects_unsupported_shape(gpu):
    w = torch.zeros(2, 384, 512, dtype=BF16, device=gpu)
    with pytest.raises(ValueError, match="no 512-row tile instance"):
        KG.pack_w512(w, 384, 0, False)


@pytest.mark.parametrize("T", [1, 3, 16])
def test_moe_gemm_shared_matches_separate_launches(gpu, T):
    """Routed + shared expert in one weight-streaming launch: the same bits as the two
    separate launches (routed layout, and the shared expert's one-expert layout)."""
    from fusion_amd.block import shared_layout

    say(f"moe_gemm_shared T={T}")
    E, H, I, k = 16, 6144, 2048, 8
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 40 + T, gpu)
    g = torch.Generator().manual_seed(77)
    w13s = (torch.randn(1, 2 * I, H, generator=g) * 0.05).to(BF16).to(gpu)
    w2s = (torch.randn(1, H, I, generator=g) * 0.05).to(BF16).to(gpu)
    ag, w13g, w2g = a.to(gpu), w13.to(gpu), w2.to(gpu)
    twf = tw.reshape(-1).contiguous().to(gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), 16, E)
    ssti, seids, sntp = shared_layout(T, 16, gpu)
    cfg = {"BLOCK_M": 16}
    R = T * k
    act, act_s = torch.empty(R, I, dtype=BF16, device=gpu), torch.empty(T, I, dtype=BF16, device=gpu)
    KG.moe_gemm(ag, k, w13g, act, None, sti, eids, ntp, R, I, I, True, cfg)
    KG.moe_gemm(ag, 1, w13s, act_s, None, ssti, seids, sntp, T, I, I, True, cfg)
    y, s_out = torch.empty(R, H, dtype=BF16, device=gpu), torch.empty(T, H, dtype=BF16, device=gpu)
    KG.moe_gemm(act, 1, w2g, y, twf, sti, eids, ntp, R, H, 0, False, cfg)
    KG.moe_gemm(act_s, 1, w2s, s_out, None, ssti, seids, sntp, T, H, 0, False, cfg)
    act2, act_s2 = torch.full_like(act, float("nan")), torch.full_like(act_s, float("nan"))
    KG.moe_gemm_shared(ag, k, w13g, act2, None, sti, eids, ntp, R, I, I, True, cfg, ag, w13s,
                       act_s2)
    y2, s_out2 = torch.full_like(y, float("nan")), torch.full_like(s_out, float("nan"))
    KG.moe_gemm_shared(act2, 1, w2g, y2, twf, sti, eids, ntp, R, H, 0, False, cfg, act_s2, w2s,
                       s_out2)
    torch.cuda.synchronize()
    assert torch.equal(act2, act) and torch.equal(act_s2, act_s)
    assert torch.equal(y2, y) and torch.equal(s_out2, s_out)


def test_layout_mismatch_is_rejected(gpu):
    T, E, H, I, k = 8, 16, 512, 256, 8
    a, w13, w2, ids, tw = _gemm_problem(T, E, H, I, k, 1, gpu)
    sti, eids, ntp = moe_align_block_size(ids.to(gpu), 16, E)
    act = torch.empty(T * k, I, dtype=BF16, device=gpu)
    with pytest.raises(ValueError, match="BLOCK_M"):
        KG.launch_gateup(a.to(gpu), w13.to(gpu), act, sti, eids, ntp, T * k, k, I,
                         {"BLOCK_M": 64}, True)


# ------------------------------------------------------------------ merges
def test_merges_bitwise(gpu):
    g = torch.Generator().manual_seed(4)
    T, H = 37, 6144
    y3 = torch.randn(T, 8, H, generator=g).to(BF16)
    res = torch.randn(T, H, generator=g).to(BF16)
    s = torch.randn(T, H, generator=g).to(BF16)
    wt = torch.rand(T, 8, generator=g)
    y3g, resg, sg, wtg = y3.to(gpu), res.to(gpu), s.to(gpu), wt.to(gpu)
    out = torch.empty(T, H, dtype=BF16, device=gpu)
    KD.launch_moe_sum(y3g, out, resg, 8, {}, True)
    assert torch.equal(out.cpu(), O.moe_sum(y3, res))
    KD.launch_moe_sum(y3g, out, resg, 8, {}, False)
    assert torch.equal(out.cpu(), O.moe_sum(y3))
    KD.launch_resadd(sg, resg, out, {})
    assert torch.equal(out.cpu(), (s.float() + res.float()).to(BF16))
    # block tail: bf16((sum_k Y + h) + s)
    _lib.call("glm52_block_merge", _lib.ptr(y3g), y3g.stride(0), y3g.stride(1), _lib.ptr(resg),
              resg.stride(0), _lib.ptr(sg), sg.stride(0), _lib.ptr(out), out.stride(0), T, H,
              _lib.stream())
    acc = torch.zeros(T, H)
    for k in range(8):
        acc = acc + y3[:, k].float()
    want = ((acc + res.float()) + s.float()).to(BF16)
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("round_mid", [1, 0])
def test_merge_resadd(gpu, round_mid):
    g = torch.Generator().manual_seed(5)
    T, H = 19, 6144
    y3 = torch.randn(T, 8, H, generator=g).to(BF16)
    res = torch.randn(T, H, generator=g).to(BF16)
    wt = torch.rand(T, 8, generator=g)
    out = torch.empty(T, H, dtype=BF16, device=gpu)
    KM.fused_merge_resadd(y3.to(gpu), wt.to(gpu), res.to(gpu), out, {"ROUND_MID": round_mid})
    want = O.merge_resadd(y3, wt, res, round_mid=bool(round_mid))
    assert torch.equal(out.cpu(), want)
    m = torch.empty(T, H, dtype=BF16, device=gpu)
    KM.merge_only(y3.to(gpu), wt.to(gpu), m, {})
    out2 = torch.empty(T, H, dtype=BF16, device=gpu)
    KM.resadd_only(m, res.to(gpu), out2, {})
    if round_mid:
        assert torch.equal(out2, out)


# ------------------------------------------------------------------ router, bounded path
def select_bound(y_o, gate, logits_exact):
    """The error bound the bounded router promises for every logit it does not recompute:
    1.375 * 2^-16 * ||y_t|| ||w_e|| + 2^-24 |L~| (chains of eight MFMAs, at most 64 chain
    sums per K slice in fp32, one rounding of L~), taken here with 2^-20 |L| for the last
    term."""
    yn = np.sqrt((y_o.double().numpy() ** 2).sum(1))[:, None]
    wn = np.sqrt((gate.double().numpy() ** 2).sum(1))[None, :]
    return 1.375 * 2.0 ** -16 * yn * wn + 2.0 ** -20 * np.abs(logits_exact) + 1e-30


def run_router_rows(gpu, y, gate, bias, topk=8):
    T = y.shape[0]
    E = gate.shape[0]
    logits = torch.full((T, E), float("nan"), device=gpu)
    topw = torch.empty(T, topk, dtype=torch.float32, device=gpu)
    topi = torch.empty(T, topk, dtype=torch.int32, device=gpu)
    cfg = {"correction_bias": None if bias is None else bias.to(gpu)}
    KR.router(y.to(gpu), gate.to(gpu).t(), logits, topw, topi, cfg)
    torch.cuda.synchronize()
    return logits.cpu().numpy(), topw.cpu().numpy(), topi.cpu().numpy()


@pytest.mark.parametrize("T,bias", [(17, "normal"), (100, "zero"), (512, "zipf"),
                                    (2048, "normal"), (8192, "zipf")])
def test_router_bounded_path_bitwise(gpu, T, bias):
    """The gate-rows router above 16 tokens: ids and weights bit for bit against the exact
    rule; logits exact on every selected expert and within the proven bound elsewhere."""
    say(f"bounded router T={T} bias={bias}")
    fe = front_end(T, bias=bias)
    y_o, _ = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    b = None if bias == "zero" else fe.bias
    lg, w, ids = run_router_rows(gpu, y_o, fe.gate, b)
    lg_o, w_o, ids_o = O.router_exact(y_o, fe.wgt, None if b is None else b.numpy())
    assert np.array_equal(ids, ids_o)
    assert np.array_equal(w, w_o)
    sel = np.take_along_axis(lg, ids_o.astype(np.int64), 1)
    assert np.array_equal(sel, np.take_along_axis(lg_o, ids_o.astype(np.int64), 1))
    bound = select_bound(y_o, fe.gate, lg_o)
    ratio = np.abs(lg.astype(np.float64) - lg_o) / bound
    say(f"  approximate logits: max |error| / bound = {ratio.max():.3e}, "
        f"exact (recomputed) fraction {(lg == lg_o).mean():.3f}")
    assert ratio.max() <= 1.0


@pytest.mark.parametrize("T,H", [(4133, 6144), (300, 4096), (1100, 4096), (300, 8192),
                                 (4100, 8192)])
def test_router_bounded_path_shapes(gpu, T, H):
    """The bounded router at the other hidden sizes it serves (H = 4096, 8192: 8 and 16
    chunks of 512 k per lane) and at ragged token counts on both token tiles (64 below
    4096 tokens, 128 from there; K split 8 or 4 ways): ids and weights bit for bit against
    the exact rule, selected logits exact, the others within the proven bound."""
    say(f"bounded router T={T} H={H}")
    g = torch.Generator().manual_seed(7000 + T + H)
    y = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gate = (torch.randn(256, H, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(256, generator=g) * 0.01
    lg, w, ids = run_router_rows(gpu, y, gate, bias)
    lg_o, w_o, ids_o = O.router_exact(y, gate.t().contiguous(), bias.numpy())
    assert np.array_equal(ids, ids_o)
    assert np.array_equal(w, w_o)
    sel = np.take_along_axis(lg, ids_o.astype(np.int64), 1)
    assert np.array_equal(sel, np.take_along_axis(lg_o, ids_o.astype(np.int64), 1))
    ratio = np.abs(lg.astype(np.float64) - lg_o) / select_bound(y, gate, lg_o)
    assert ratio.max() <= 1.0


def test_router_bounded_path_ties_and_nan(gpu):
    """Exact ties above the cut (16 identical gate rows lifted by the bias: the lower
    indices win), a token of NaN (every key -inf: ids 0..7, NaN weights, as the exact
    rule) and top-k 6 without normalisation."""
    T, H, E = 40, 6144, 256
    fe = front_end(T)
    y_o, _ = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    gate = fe.gate.clone()
    gate[3:19] = gate[3]  # experts 3..18 identical
    bias = torch.zeros(E, dtype=torch.float32)
    bias[3:19] = 1.0
    y = y_o.clone()
    y[5] = float("nan")
    lg, w, ids = run_router_rows(gpu, y, gate, bias)
    lg_o, w_o, ids_o = O.router_exact(y, gate.t().contiguous(), bias.numpy())
    assert np.array_equal(ids, ids_o)
    assert (ids[:5] == np.arange(3, 11)).all() and (ids[5] == np.arange(8)).all()
    assert np.array_equal(np.isnan(w), np.isnan(w_o))
    ok = ~np.isnan(w_o)
    assert np.array_equal(w[ok], w_o[ok])
    # top-k 6, unnormalised weights
    logits = torch.empty(T, E, device=gpu)
    topw = torch.empty(T, 6, dtype=torch.float32, device=gpu)
    topi = torch.empty(T, 6, dtype=torch.int32, device=gpu)
    KR.router(y_o.to(gpu), fe.gate.to(gpu).t(), logits, topw, topi,
              {"correction_bias": fe.bias.to(gpu), "NORM_PROB": False})
    lg6 = O.router_logits_exact(y_o, fe.wgt)
    w6, ids6, _ = O.router_select(lg6, fe.bias.numpy(), 6, norm_prob=False)
    assert np.array_equal(topi.cpu().numpy(), ids6)
    assert np.array_equal(topw.cpu().numpy(), w6)
