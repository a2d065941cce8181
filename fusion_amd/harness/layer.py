"""Whole-layer configuration harness: which combination of fusions minimises the layer
subgraph's time, per regime, on MI355X.

Restates `glm52/bench/bench_layer.py` (regimes `:60-72`, `LayerProblem` `:292-389`,
`build_chain` `:395-481`, `CONFIGS` A-K `:531-545`, the run loop `:548-611`) and the
interleaved re-measurement of `glm52/bench/bench_layer_ab.py`, over this build's drop-in
launchers.  The subgraph is the reference's:

    o_proj -> ResAdd1 -> post-attention RMSNorm -> router + top-8
           -> w13 grouped GEMM -> SwiGLU -> w2 grouped GEMM -> expert merge -> ResAdd2
           -> shared expert (w13_s -> SwiGLU -> w2_s) -> add

The routing is frozen (computed once from the value the pipeline produces, as in the
reference); every configuration still pays for the router GEMM and the top-k, written to
scratch buffers.  The dispatch layouts are built outside the timed region.  Each
configuration's output is checked, on sampled token rows, against an fp32 reference
computed independently with torch (fp32 GEMMs and SwiGLU, one bf16 rounding), with the
reference's layer gate rel_err <= 5e-2.

One configuration is this build's own: `Z_mi355x_block` = o_proj with ResAdd1 fused,
then the composed `MoEBlock` (norm, live routing, fused decode/prefill GEMMs, merged
tail) on h1 with a zero residual.  Its routing is live, but computed from the same h1 by
the same kernels as the frozen routing, so it selects the same experts (an h1 rounded
differently -- the unfused o_proj's -- could flip near-tied experts and is not used).

Run: python -m fusion_amd.harness.layer --regimes decode_bs1,prefill_t8192 \\
         --results-dir results [--ab]
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

import torch

from .. import config as C
from ..block import MoEBlock, default_block_m, default_shared_block_m
from ..dispatch import moe_align_block_size
from ..kernels import add_rmsnorm as KN
from ..kernels import moe_down_merge as KD
from ..kernels import moe_gateup as KG
from ..kernels import norm_router as KR
from ..kernels import oproj_resadd as KO
from . import protocol as P

H, I, TOPK = C.H, C.I, C.TOPK
OPROJ_K_DECODE = 32768   # absorbed MLA: 64 heads x 512 (`glm52/config.py:58-59`)
OPROJ_K_PREFILL = 16384  # 64 heads x 256 (`glm52/config.py:55-56`)

REGIMES = {
    "decode_bs1": (1, OPROJ_K_DECODE),
    "decode_bs32": (32, OPROJ_K_DECODE),
    "decode_bs256": (256, OPROJ_K_DECODE),
    "decode_bs512": (512, OPROJ_K_DECODE),
    "decode_bs1024": (1024, OPROJ_K_DECODE),
    "prefill_t2048": (2048, OPROJ_K_PREFILL),
    "prefill_t8192": (8192, OPROJ_K_PREFILL),
}

# The reference's curated set (`glm52/bench/bench_layer.py:531-545`): a baseline, one axis
# at a time, and the combinations; plus this build's composed block.
CONFIGS = {
    "A_all_unfused": dict(resadd1="separate", norm="split", gateup="split", down="split"),
    "B_f3": dict(resadd1="separate", norm="fused3", gateup="split", down="split"),
    "C_f1": dict(resadd1="in_oproj", norm="split", gateup="split", down="split"),
    "D_f6": dict(resadd1="separate", norm="split", gateup="fused6", down="split"),
    "E_f10": dict(resadd1="separate", norm="split", gateup="split", down="merge_f10"),
    "F_f8": dict(resadd1="separate", norm="split", gateup="split", down="atomic8"),
    "G_f9": dict(resadd1="separate", norm="split", gateup="split", down="atomic9"),
    "H_f3_f10": dict(resadd1="separate", norm="fused3", gateup="split", down="merge_f10"),
    "I_f3_f9": dict(resadd1="separate", norm="fused3", gateup="split", down="atomic9"),
    "J_greedy_all": dict(resadd1="in_oproj", norm="split", gateup="fused6", down="atomic9"),
    "K_f3_f8": dict(resadd1="separate", norm="fused3", gateup="split", down="atomic8"),
    "Z_mi355x_block": dict(block=True),
}

LAYER_TOL = 5e-2  # `glm52/bench/bench_layer.py:573`


class LayerProblem:
    """Inputs, weights and buffers of one regime (the reference's `LayerProblem`), with
    `E` routed experts (256 in GLM-5.2; fewer for quick checks)."""

    def __init__(self, regime: str, seed: int = 0, E: int = C.E, ref_rows: int = 32,
                 device="cuda"):
        T, Kq = REGIMES[regime]
        self.regime, self.T, self.Kq, self.E = regime, T, Kq, E
        self.rows = T * TOPK
        dev, dt = torch.device(device), torch.bfloat16
        self.dev = dev
        g = torch.Generator(device=dev).manual_seed(seed)

        def rnd(*shape, scale=0.05):
            t = torch.empty(*shape, device=dev, dtype=dt)
            if t.numel() > 2 ** 28:  # big expert stacks are filled slice by slice
                for i in range(t.shape[0]):
                    t[i].normal_(0.0, scale, generator=g)
            else:
                t.normal_(0.0, scale, generator=g)
            return t

        self.a_attn = rnd(T, Kq)
        self.w_o = rnd(Kq, H, scale=0.02)
        self.h_in = rnd(T, H)
        self.c = torch.empty(T, H, device=dev, dtype=dt)
        self.h1 = torch.empty(T, H, device=dev, dtype=dt)
        self.acc32 = torch.zeros(T, H, device=dev, dtype=torch.float32)
        self.w_norm = (torch.randn(H, generator=g, device=dev) * 0.1 + 1).to(dt)
        self.x2 = torch.empty(T, H, device=dev, dtype=dt)
        self.wg_t = rnd(H, E, scale=0.02)
        self.logits = torch.empty(T, E, device=dev, dtype=torch.float32)
        self.topw = torch.empty(T, TOPK, device=dev, dtype=torch.float32)
        self.topi = torch.empty(T, TOPK, device=dev, dtype=torch.int32)
        self.w13 = rnd(E, 2 * I, H, scale=0.02)
        self.w2 = rnd(E, H, I, scale=0.02)
        self.inter = torch.empty(self.rows, 2 * I, device=dev, dtype=dt)
        self.act = torch.empty(self.rows, I, device=dev, dtype=dt)
        self.y3 = torch.zeros(self.rows, H, device=dev, dtype=dt)
        self.y3v = self.y3.view(T, TOPK, H)
        self.routed = torch.zeros(T, H, device=dev, dtype=dt)
        self.out = torch.zeros(T, H, device=dev, dtype=dt)
        self.w13s = rnd(1, 2 * I, H, scale=0.02)
        self.w2s = rnd(1, H, I, scale=0.02)
        self.s_inter = torch.empty(T, 2 * I, device=dev, dtype=dt)
        self.s_act = torch.empty(T, I, device=dev, dtype=dt)
        self.s_out = torch.empty(T, H, device=dev, dtype=dt)
        self.ones = torch.ones(T, device=dev, dtype=torch.float32)
        self.zero_bias = torch.zeros(E, device=dev, dtype=torch.float32)
        self.zero_res = torch.zeros(T, H, device=dev, dtype=dt)
        self.bm = default_block_m(T)
        self.sbm = default_shared_block_m(T)
        self.cfg_topk = {"scale": C.ROUTED_SCALING_FACTOR}

        # frozen routing, from the value the pipeline produces (h1 = o_proj + h_in)
        KO.gemm_launch(self.a_attn, self.w_o, self.h1, self.h_in, {}, True, False)
        KN.norm_only(self.h1, self.w_norm, self.x2, {})
        KR.router_gemm(self.x2, self.wg_t, self.logits, {})
        KR.topk_only(self.logits, self.topw, self.topi, self.cfg_topk)
        self.tw_flat = self.topw.reshape(-1).contiguous()
        self.topw_scratch = torch.empty_like(self.topw)
        self.topi_scratch = torch.empty_like(self.topi)
        self._layouts: dict = {}
        self._shared_layouts: dict = {}
        self._block = None

        # independent fp32 reference on sampled token rows
        if T <= ref_rows:
            self.ref_idx = torch.arange(T, device=dev)
        else:
            gg = torch.Generator(device=dev).manual_seed(1234)
            self.ref_idx = torch.randperm(T, device=dev, generator=gg)[:ref_rows].sort().values
        self.ref_out = self._reference()

    def _reference(self) -> torch.Tensor:
        idx = self.ref_idx
        silu = torch.nn.functional.silu
        h1 = (self.a_attn[idx].float() @ self.w_o.float() + self.h_in[idx].float()).to(
            torch.bfloat16)
        hf = h1.float()
        rstd = torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + C.RMS_NORM_EPS)
        x2 = ((hf * rstd).to(torch.bfloat16).float() * self.w_norm.float()).to(torch.bfloat16)
        out = torch.empty(len(idx), H, device=self.dev, dtype=torch.float32)
        ids, tw = self.topi[idx], self.topw[idx]
        for r in range(len(idx)):
            xr = x2[r].float()
            acc = h1[r].float().clone()
            for k in range(TOPK):
                e = int(ids[r, k])
                gu = self.w13[e].float() @ xr
                acc += float(tw[r, k]) * (self.w2[e].float() @ (silu(gu[:I]) * gu[I:]))
            gu = self.w13s[0].float() @ xr
            acc += self.w2s[0].float() @ (silu(gu[:I]) * gu[I:])
            out[r] = acc
        return out.to(torch.bfloat16)

    def layout(self, block_m: int):
        if block_m not in self._layouts:
            self._layouts[block_m] = moe_align_block_size(self.topi, block_m, self.E)
        return self._layouts[block_m]

    def shared_layout(self, block_m: int):
        if block_m not in self._shared_layouts:
            ids = torch.zeros(self.T, 1, dtype=torch.int32, device=self.dev)
            self._shared_layouts[block_m] = moe_align_block_size(ids, block_m, 1)
        return self._shared_layouts[block_m]

    def block(self) -> MoEBlock:
        if self._block is None:
            self._block = MoEBlock(self.T, self.w_norm, self.wg_t, self.zero_bias, self.w13,
                                   self.w2, self.w13s, self.w2s)
        return self._block

    def release_block(self) -> None:
        self._block = None


def build_chain(p: LayerProblem, sel: dict) -> tuple[list, torch.Tensor]:
    """The launches of one configuration (`glm52/bench/bench_layer.py:395-481`), and the
    tensor holding its output."""
    if sel.get("block"):
        # o_proj with ResAdd1 fused (#1) gives h1; the block adds a zero residual (exact),
        # so its live routing is computed from the same h1 as the frozen routing
        blk = p.block()
        return [lambda: KO.gemm_launch(p.a_attn, p.w_o, p.h1, p.h_in, {}, True, False),
                lambda: blk(p.h1, p.zero_res)], blk.out

    fns = []
    # o_proj (+ ResAdd1)
    if sel["resadd1"] == "in_oproj":
        fns.append(lambda: KO.gemm_launch(p.a_attn, p.w_o, p.h1, p.h_in, {}, True, False))
        fns.append(lambda: KN.norm_only(p.h1, p.w_norm, p.x2, {}))
    else:
        fns.append(lambda: KO.gemm_launch(p.a_attn, p.w_o, p.c, None, {}, False, False))
        if sel["norm"] == "fused3":
            fns.append(lambda: KN.fused_add_rmsnorm(p.c, p.h_in, p.w_norm, p.h1, p.x2, {}))
        else:
            fns.append(lambda: KN.add_only(p.c, p.h_in, p.h1, {}))
            fns.append(lambda: KN.norm_only(p.h1, p.w_norm, p.x2, {}))
    # router + top-k into scratch (the routing stays frozen)
    fns.append(lambda: KR.router_gemm(p.x2, p.wg_t, p.logits, {}))
    fns.append(lambda: KR.topk_only(p.logits, p.topw_scratch, p.topi_scratch, p.cfg_topk))
    # w13 (+ SwiGLU)
    gc = {"BLOCK_M": p.bm}
    sti, eid, ntp = p.layout(p.bm)
    if sel["gateup"] == "fused6":
        fns.append(lambda: KG.launch_gateup(p.x2, p.w13, p.act, sti, eid, ntp, p.rows, TOPK, I,
                                            gc, True))
    else:
        fns.append(lambda: KG.launch_gateup(p.x2, p.w13, p.inter, sti, eid, ntp, p.rows, TOPK,
                                            I, gc, False))
        fns.append(lambda: KG.launch_silu_and_mul(p.inter, p.act, {}))
    # w2 + merge + ResAdd2 (launch_down applies the routing weight: the merge is a plain sum)
    d = sel["down"]
    if d == "atomic8":
        fns += [lambda: p.routed.zero_(),
                lambda: KD.launch_down(p.act, p.w2, p.routed, p.tw_flat, sti, eid, ntp, p.rows,
                                       TOPK, gc, True),
                lambda: KD.launch_resadd(p.routed, p.h1, p.out, {})]
    elif d == "atomic9":
        fns += [lambda: KD.launch_seed(p.out, p.h1, {}, True),
                lambda: KD.launch_down(p.act, p.w2, p.out, p.tw_flat, sti, eid, ntp, p.rows,
                                       TOPK, gc, True)]
    else:
        fns.append(lambda: KD.launch_down(p.act, p.w2, p.y3, p.tw_flat, sti, eid, ntp, p.rows,
                                          TOPK, gc, False))
        if d == "merge_f10":
            fns.append(lambda: KD.launch_moe_sum(p.y3v, p.out, p.h1, TOPK, {}, True))
        else:
            fns += [lambda: KD.launch_moe_sum(p.y3v, p.routed, p.h1, TOPK, {}, False),
                    lambda: KD.launch_resadd(p.routed, p.h1, p.out, {})]
    # shared expert, identical in every configuration
    sc = {"BLOCK_M": p.sbm}
    ssti, seid, sntp = p.shared_layout(p.sbm)
    fns += [
        lambda: KG.launch_gateup(p.x2, p.w13s, p.s_inter, ssti, seid, sntp, p.T, 1, I, sc,
                                 False),
        lambda: KG.launch_silu_and_mul(p.s_inter, p.s_act, {}),
        lambda: KD.launch_down(p.s_act, p.w2s, p.s_out, p.ones, ssti, seid, sntp, p.T, 1, sc,
                               False),
        lambda: KD.launch_resadd(p.s_out, p.out, p.out, {}),
    ]
    return fns, p.out


def run_once(p: LayerProblem, name: str) -> dict:
    """Build and run one configuration once; check it against the fp32 reference rows."""
    chain, out = build_chain(p, CONFIGS[name])
    p.out.zero_()
    p.routed.zero_()
    p.y3.zero_()
    for fn in chain:
        fn()
    torch.cuda.synchronize()
    ck = P.check(out[p.ref_idx], p.ref_out, tol=LAYER_TOL, label=name)
    return {"chain": chain, "check": ck}


def run_regime(p: LayerProblem, names, rep: int = 40, warmup: int = 15, log=print) -> dict:
    rows = {}
    for name in names:
        try:
            r = run_once(p, name)
            ck = r["check"]
            if not ck["ok"]:
                log(f"  {name:<18} !! FAILS CORRECTNESS rel_err={ck['rel_err']:.3e}")
            t = P.bench_chain(r["chain"], warmup=warmup, rep=rep)
            rows[name] = {"ms": t.p50_ms, "p10_p90": [t.p10_ms, t.p90_ms],
                          "noflush_ms": t.noflush_p50_ms, "n_kernels": len(r["chain"]),
                          "sel": CONFIGS[name], "rel_err_vs_fp32_ref": ck["rel_err"],
                          "correct": ck["ok"]}
            log(f"  {name:<18} {t.p50_ms:9.4f} ms  ({len(r['chain'])} launches)  "
                f"rel_err {ck['rel_err']:.2e}")
        except (RuntimeError, ValueError) as exc:
            rows[name] = {"error": f"{type(exc).__name__}: {exc}"[:300]}
            log(f"  {name:<18} FAILED {type(exc).__name__}: {exc}")
    ok = {k: v for k, v in rows.items() if "ms" in v and v.get("correct")}
    if not ok:
        raise RuntimeError(f"{p.regime}: no configuration passed correctness")
    best = min(ok, key=lambda k: ok[k]["ms"])
    base = ok.get("A_all_unfused", {}).get("ms")
    log(f"  --> BEST {best} = {ok[best]['ms']:.4f} ms"
        + (f"  ({base / ok[best]['ms']:.3f}x vs all-unfused)" if base else ""))
    return {"rows": rows, "best": best,
            "speedup_vs_unfused": (base / ok[best]["ms"]) if base else None,
            "T": p.T, "oproj_K": p.Kq, "moe_rows": p.rows, "experts": p.E}


def run_ab(p: LayerProblem, names, rounds: int = 8, rep: int = 15, log=print) -> dict:
    """Interleaved rounds: every candidate once per round, in the same order."""
    chains = {}
    for name in names:
        r = run_once(p, name)
        if not r["check"]["ok"]:
            log(f"  {name} FAILS CORRECTNESS ({r['check']['rel_err']:.2e}) -- dropped")
            continue
        chains[name] = r["chain"]
    per: dict[str, list[float]] = {k: [] for k in chains}
    for i in range(rounds):
        for name, chain in chains.items():
            per[name].append(P.bench_chain(chain, warmup=5, rep=rep).p50_ms)
        log(f"  round {i}: " + "  ".join(f"{n}={per[n][-1]:.4f}" for n in chains))
    stats, verdict = P.ab_verdict(per)
    base = stats.get("A_all_unfused", {}).get("median")
    best = verdict.get("best")
    return {"stats": stats, "verdict": verdict,
            "speedup_vs_unfused": (base / stats[best]["median"]) if base and best else None}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--regimes", default=",".join(REGIMES))
    ap.add_argument("--configs", default=",".join(CONFIGS))
    ap.add_argument("--rep", type=int, default=40)
    ap.add_argument("--experts", type=int, default=C.E)
    ap.add_argument("--results-dir", default="results")
    ap.add_argument("--no-device-fence", action="store_true")
    ap.add_argument("--ab", action="store_true", help="also run the interleaved re-measurement")
    ap.add_argument("--rounds", type=int, default=8)
    ap.add_argument("--ab-rep", type=int, default=15)
    ap.add_argument("--top", type=int, default=6)
    args = ap.parse_args(argv)

    def log(*a):
        print(*a, flush=True)

    dev = P.device_name()
    warnings: list = []
    moved = P.quarantine_foreign_results(args.results_dir, dev, not args.no_device_fence,
                                         warnings)
    for w in warnings:
        log(f"!! {w}")
    names = [n.strip() for n in args.configs.split(",") if n.strip()]
    out_all, ab_all = {}, {}
    for regime in [r.strip() for r in args.regimes.split(",") if r.strip()]:
        log(f"\n===== {regime} =====")
        p = LayerProblem(regime, E=args.experts)
        out_all[regime] = run_regime(p, names, rep=args.rep, log=log)
        if args.ab:
            rows = out_all[regime]["rows"]
            good = sorted((k for k, v in rows.items() if "ms" in v and v.get("correct")),
                          key=lambda k: rows[k]["ms"])
            cands = good[: args.top]
            if "A_all_unfused" in good and "A_all_unfused" not in cands:
                cands.append("A_all_unfused")
            log(f"  interleaved: {', '.join(cands)}")
            ab_all[regime] = run_ab(p, cands, rounds=args.rounds, rep=args.ab_rep, log=log)
        p.release_block()
        del p
        torch.cuda.empty_cache()
    scope = ("o_proj + ResAdd1 + RMSNorm + router/top-8 + w13/SwiGLU + w2 + merge + ResAdd2 "
             "+ shared expert; dispatch layouts built outside the timed region; routing "
             "frozen (router and top-k still run, into scratch)")
    P.record("layer_configurations", {"id": "layer_configurations", "scope": scope,
                                      "configs": CONFIGS, "regimes": out_all,
                                      "quarantined": moved, "warnings": warnings},
             args.results_dir, dev)
    if args.ab:
        P.record("layer_configurations_ab", {
            "id": "layer_configurations_ab",
            "protocol": f"{args.rounds} interleaved rounds, rep={args.ab_rep} per round; "
                        "per-config median across rounds; a winner only if its gap to the "
                        "runner-up exceeds the round-to-round spread of both",
            "regimes": ab_all}, args.results_dir, dev)
    log(f"\nwrote {Path(args.results_dir) / 'layer_configurations.json'}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
