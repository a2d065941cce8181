"""The whole-layer configuration harness (`glm52/bench/bench_layer.py`) on the GPU, with 16
routed experts at the real widths: every configuration A-K and the composed block must
pass the reference's layer gate (rel_err <= 5e-2) against the independent fp32 reference
rows, agree with one another, and time through the reference's protocol."""

from __future__ import annotations

import pytest
import torch

from fusion_amd.harness import layer as L
from fusion_amd.harness import protocol as P

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("regime", ["decode_bs1", "decode_bs32"])
def test_every_configuration_passes_the_layer_gate(gpu, regime):
    say(f"layer harness {regime}")
    p = L.LayerProblem(regime, E=16)
    outs = {}
    for name in L.CONFIGS:
        r = L.run_once(p, name)
        ck = r["check"]
        say(f"  {name}: rel_err {ck['rel_err']:.2e}")
        assert ck["ok"], f"{name}: rel_err {ck['rel_err']}"
        out = p.block().out if name == "Z_mi355x_block" else p.out
        outs[name] = out.clone()
    base = outs["A_all_unfused"]
    for name, o in outs.items():
        assert P.rel_err(o, base) <= L.LAYER_TOL, name
    p.release_block()


def test_regime_and_interleaved_protocol(gpu, tmp_path):
    p = L.LayerProblem("decode_bs1", E=16)
    names = ["A_all_unfused", "H_f3_f10", "Z_mi355x_block"]
    res = L.run_regime(p, names, rep=3, warmup=1, log=say)
    assert set(res["rows"]) == set(names) and res["best"] in names
    assert all(res["rows"][n]["correct"] for n in names)
    ab = L.run_ab(p, names, rounds=2, rep=3, log=say)
    assert ab["verdict"]["best"] in names and len(ab["stats"]["H_f3_f10"]["rounds"]) == 2
    path = P.record("layer_configurations", {"regimes": {"decode_bs1": res}}, tmp_path)
    assert path.exists()
