"""The configuration harness on the CPU: the configuration table against the reference's,
the launches each configuration builds (with recording stand-ins for the launchers), the
result schema and device fence, and the interleaved-protocol verdict."""

from __future__ import annotations

import json
from types import SimpleNamespace

import pytest

from fusion_amd.harness import layer as L
from fusion_amd.harness import protocol as P

# `glm52/bench/bench_layer.py:531-545`
REFERENCE_CONFIGS = {
    "A_all_unfused": ("separate", "split", "split", "split"),
    "B_f3": ("separate", "fused3", "split", "split"),
    "C_f1": ("in_oproj", "split", "split", "split"),
    "D_f6": ("separate", "split", "fused6", "split"),
    "E_f10": ("separate", "split", "split", "merge_f10"),
    "F_f8": ("separate", "split", "split", "atomic8"),
    "G_f9": ("separate", "split", "split", "atomic9"),
    "H_f3_f10": ("separate", "fused3", "split", "merge_f10"),
    "I_f3_f9": ("separate", "fused3", "split", "atomic9"),
    "J_greedy_all": ("in_oproj", "split", "fused6", "atomic9"),
    "K_f3_f8": ("separate", "fused3", "split", "atomic8"),
}


def test_configs_match_the_reference():
    for name, axes in REFERENCE_CONFIGS.items():
        sel = L.CONFIGS[name]
        assert (sel["resadd1"], sel["norm"], sel["gateup"], sel["down"]) == axes
    assert set(L.CONFIGS) == set(REFERENCE_CONFIGS) | {"Z_mi355x_block"}
    assert L.REGIMES["decode_bs1"] == (1, 32768) and L.REGIMES["prefill_t8192"] == (8192, 16384)


class _Rec:
    """Stands in for a launcher module: records (module.function, buffer names)."""

    def __init__(self, mod, log):
        self.mod, self.log = mod, log

    def __getattr__(self, fn):
        def call(*args, **kw):
            names = [a for a in args if isinstance(a, str)]
            self.log.append((f"{self.mod}.{fn}", tuple(names)))
        return call


class _Buf(str):
    def zero_(self):
        _Buf.log.append(("zero_", (str(self),)))


def _fake_problem(log):
    _Buf.log = log
    p = SimpleNamespace()
    for n in ("a_attn", "w_o", "h_in", "c", "h1", "acc32", "w_norm", "x2", "wg_t", "logits",
              "topw_scratch", "topi_scratch", "w13", "w2", "inter", "act", "y3", "y3v",
              "routed", "out", "w13s", "w2s", "s_inter", "s_act", "s_out", "ones", "tw_flat"):
        setattr(p, n, _Buf(n))
    p.rows, p.T, p.bm, p.sbm, p.cfg_topk = 8, 1, 16, 16, {}
    p.layout = lambda bm: ("sti", "eid", "ntp")
    p.shared_layout = lambda bm: ("ssti", "seid", "sntp")
    return p


EXPECTED_TAIL = [("KG.launch_gateup", ("x2", "w13s", "s_inter", "ssti", "seid", "sntp")),
                 ("KG.launch_silu_and_mul", ("s_inter", "s_act")),
                 ("KD.launch_down", ("s_act", "w2s", "s_out", "ones", "ssti", "seid", "sntp")),
                 ("KD.launch_resadd", ("s_out", "out", "out"))]


@pytest.mark.parametrize("name", sorted(REFERENCE_CONFIGS))
def test_build_chain_follows_the_reference(monkeypatch, name):
    log: list = []
    for mod in ("KO", "KN", "KR", "KG", "KD"):
        monkeypatch.setattr(L, mod, _Rec(mod, log))
    p = _fake_problem(log)
    fns, out = L.build_chain(p, L.CONFIGS[name])
    for fn in fns:
        fn()
    assert out == "out"
    r1, norm, gateup, down = REFERENCE_CONFIGS[name]
    calls = [c[0] for c in log]
    if r1 == "in_oproj":
        assert log[0] == ("KO.gemm_launch", ("a_attn", "w_o", "h1", "h_in"))
        assert calls[1] == "KN.norm_only"
    elif norm == "fused3":
        assert calls[:2] == ["KO.gemm_launch", "KN.fused_add_rmsnorm"]
    else:
        assert calls[:3] == ["KO.gemm_launch", "KN.add_only", "KN.norm_only"]
    assert ("KR.topk_only", ("logits", "topw_scratch", "topi_scratch")) in log
    gu = [c for c in log if c[0] == "KG.launch_gateup" and "w13" in c[1]]
    assert len(gu) == 1 and (("act" in gu[0][1]) == (gateup == "fused6"))
    assert ("KG.launch_silu_and_mul" in calls) is True  # the shared expert always has one
    downs = [c for c in log if c[0] == "KD.launch_down" and "w2" in c[1]]
    assert len(downs) == 1
    if down in ("atomic8", "atomic9"):
        assert downs[0][1][2] == ("routed" if down == "atomic8" else "out")
    else:
        assert downs[0][1][2] == "y3"
    assert log[-4:] == EXPECTED_TAIL
    n = {"split": 14, "merge_f10": 13, "atomic8": 14, "atomic9": 13}[down]
    n -= (1 if norm == "fused3" else 0) + (1 if r1 == "in_oproj" else 0)
    n -= 1 if gateup == "fused6" else 0
    assert len(fns) == n


def test_record_meta_and_device_fence(tmp_path):
    path = P.record("x", {"id": "x", "v": 1}, tmp_path, device="AMD Instinct MI355X")
    meta = json.loads(path.read_text())["_meta"]
    assert meta["device"] == "AMD Instinct MI355X" and "recorded_at" in meta
    P.record("sub/y", {"id": "y"}, tmp_path, device="NVIDIA H200")
    (tmp_path / "broken.json").write_text("{not json")
    warnings: list = []
    moved = P.quarantine_foreign_results(tmp_path, "AMD  Instinct MI355X", True, warnings)
    assert [m["file"] for m in moved] == ["sub/y.json"]
    assert (tmp_path / "x.json").exists() and not (tmp_path / "sub" / "y.json").exists()
    assert (tmp_path / "broken.json").exists()
    assert len(list(tmp_path.glob("_quarantine_foreign_*/sub/y.json"))) == 1
    # a second pass leaves the quarantine alone
    assert P.quarantine_foreign_results(tmp_path, "AMD Instinct MI355X") == []
    w2: list = []
    assert P.quarantine_foreign_results(tmp_path, "", True, w2) == [] and w2
    w3: list = []
    assert P.quarantine_foreign_results(tmp_path, "other", False, w3) == [] and w3


def test_ab_verdict_separated_and_tied():
    stats, v = P.ab_verdict({"a": [1.00, 1.01, 1.02], "b": [1.20, 1.21, 1.19],
                             "c": [1.5, 1.6, 1.4]})
    assert v["best"] == "a" and v["runner_up"] == "b" and v["separated"]
    assert v["tied_set"] == ["a"]
    assert stats["c"]["median"] == 1.5 and stats["c"]["min"] == 1.4
    _, v = P.ab_verdict({"a": [1.00, 1.10], "b": [1.04, 1.05]})
    assert not v["separated"] and set(v["tied_set"]) == {"a", "b"}
    _, v = P.ab_verdict({"only": [2.0]})
    assert v == {"best": "only"}
