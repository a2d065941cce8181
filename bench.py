"""Benchmark of the GLM-5.2 MoE FFN block on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 25] [--tokens 1,256,2048,8192]

A step is one pass of the whole block (ResAdd+RMSNorm -> router -> top-8 -> dispatch ->
routed w13+SwiGLU / shared w13+SwiGLU -> routed w2 / shared w2 -> merge+ResAdd) over one
batch of T synthetic tokens, with the real 256-expert weight set (19.3 GB) resident.
The headline `value` is microseconds per block at T = 1 (configuration 1); T = 256, 2048
and 8192 (configurations 2-4, the last with the skewed router bias, whose expert loads
are reported with it) are under `per_T`.  Timing follows the reference's `bench_chain`
(`glm52/common.py:73-122`): one cache flush (1 GiB, larger than the 256 MB Infinity
Cache) before every step, never inside it, HIP events around the step, eager launches;
each size first runs untimed blocks for 50 ms (the GPU's clocks settle over ~30 ms of load
after an idle gap) and then the W warm-up steps before its K timed steps;
decode sizes also report the replay of a captured HIP graph (`graph_us`).  Each size
reports the reference's timing record: median, p10, p90, mean and min over the timed
steps and the median of the same steps without the flush; the headline size also lists
every step.  The dominant kernel -- the block's w13 + SwiGLU launch, which at T <= 4 also
derives the routing and runs the shared expert -- is timed with events on its stream
around it inside whole blocks (after the flush and the front end, before the tail): that
mean is the `roofline` object's `avg_us`; the same launch timed alone is `solo_us`.  HIP
events around one launch read 4-6 us more than a kernel trace's begin-to-end of the same
dispatch (their marker packets and the dispatch's own set-up and completion), so `avg_us`
is the conservative figure.  Its
HBM traffic comes
from two `rocprofv3 --pmc` runs of a child process (`--pmc-child`), scaled by a plain
copy of known size.  The CPU baseline is the oracle's restatement of
`glm52/reference.py`'s path (fp32 router, per-expert bf16 `moe_mlp`, fp32 shared expert)
on all of this host's cores at every T of `--tokens` (median of 5 blocks at T <= 256, 3 at
2048, 1 at 8192), with the CPU model recorded.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE-layer µs at T=1/256/8192 + % of roofline (HBM GB/s or MFMA util)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 25 untimed steps, as the reference's bench_chain (after the 50 ms clock settle)
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--tokens", default="1,256,2048,8192",
                    help="token counts; the first is the headline (configuration 1 is T=1)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--json-out", default="")
    ap.add_argument("--calibrate", action="store_true",
                    help="only measure the read-bandwidth ceiling (glm52_stream_read) and exit")
    ap.add_argument("--no-oproj", action="store_true",
                    help="skip the o_proj + ResAdd1 and pre-norm router timings reported beside each T")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc child runs behind roofline.traffic")
    ap.add_argument("--pmc-child", action="store_true",
                    help="(internal) the process profiled for roofline.traffic: three 256 MiB "
                         "copies, then the block's w13 launch at the first --tokens value")
    ap.add_argument("--pmc-step", default="w13",
                    choices=("w13", "w2", "block", "tail", "tail-rowmajor", "oproj"),
                    help="(with --pmc-child) the launch profiled: the block's w13 launch, its "
                         "w2 launch, the whole block, its token-major tail (T = 1, packed "
                         "weights), or the same tail on the row-major weights")
    ap.add_argument("--item-trace", action="store_true",
                    help="only record, per workgroup, when each prefill tile launch (w13, w2) of "
                         "the block at the first --tokens value starts and ends, its items and "
                         "XCD (glm52_debug_item_trace), print the per-XCD finish spread and exit")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first run a plain 256 MiB device copy three times: the known-size "
                         "dispatch that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the block's sharding is a design note only); run with --gpus 1", flush=True)
        return 2

    import torch

    from fusion_amd import roofline as RL
    from fusion_amd.block import MoEBlock, PackedExperts
    from fusion_amd.problem import expert_weights, front_end

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate:
        print(json.dumps({"calibration": calibrate(dev)}), flush=True)
        return 0
    if args.copy_probe or args.pmc_child:
        src = torch.ones(2 ** 26, dtype=torch.int32, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy probe: 3 x 256 MiB device copies")
        del src, dst
    if args.pmc_child and args.pmc_step == "oproj":  # o_proj + ResAdd1 alone, no expert weights
        T = int(args.tokens.split(",")[0])
        flush_buf = torch.empty(2 ** 28, dtype=torch.int32, device=dev)  # 1 GiB
        step, _ = oproj_inputs(T, dev)
        for _ in range(PMC_LAUNCHES):
            flush_buf.zero_()
            step()
        torch.cuda.synchronize()
        log(f"pmc child: T={T}, {PMC_LAUNCHES} oproj launches")
        return 0
    t0 = time.time()
    W = expert_weights(device=dev)
    # the blocks read one resident layout, packed once here; the row-major set stays for
    # the reference-API strategies of down_merge_bench and the CPU baseline
    PW = PackedExperts(W.w13, W.w2, W.w13s, W.w2s)
    torch.cuda.synchronize()
    log(f"weights ready in {time.time() - t0:.1f}s ({PW.nbytes() / 1e9:.1f} GB packed)")
    flush_buf = torch.empty(2 ** 28, dtype=torch.int32, device=dev)  # 1 GiB
    if args.item_trace:
        T = int(args.tokens.split(",")[0])
        print(json.dumps({"item_trace": item_trace(T, PW, flush_buf, dev)}), flush=True)
        return 0
    if args.pmc_child:
        T = int(args.tokens.split(",")[0])
        fe = front_end(T, bias="zipf" if T == 8192 else "normal")
        x, r = fe.x.to(dev), fe.r.to(dev)
        blk = MoEBlock(T, fe.w_norm.to(dev), fe.wgt.to(dev), fe.bias.to(dev), PW)
        blk(x, r)
        torch.cuda.synchronize()
        from fusion_amd.kernels import moe_down_merge as KD

        out_rm = torch.empty_like(blk.out)

        def tail_rowmajor():  # the same sum on the row-major weights (the layout comparison)
            KD.launch_down_token_major(blk.act, W.w2, out_rm, blk.topw, blk.topi, blk.h,
                                       blk.topk, {}, True, blk.act_s, W.w2s)

        step = {"w13": blk.w13_step, "w2": blk.w2_step, "block": lambda: blk(x, r),
                "tail": blk.tail, "tail-rowmajor": tail_rowmajor}[args.pmc_step]
        if args.pmc_step.startswith("tail") and not blk.token_major:
            raise SystemExit("--pmc-step tail needs the token-major tail (--tokens 1)")
        for _ in range(PMC_LAUNCHES):
            flush_buf.zero_()
            step()
        torch.cuda.synchronize()
        log(f"pmc child: T={T}, {PMC_LAUNCHES} {args.pmc_step} launches")
        return 0

    def flush():
        flush_buf.zero_()

    def settle(fn, ms=SETTLE_MS):
        """Untimed steps (each after the flush) until `ms` of them have run: after an idle
        gap the GPU's clocks take ~30 ms of load to settle (the T = 1 w13 launch runs 78 us
        after 76 ms idle, 70-72 us 30 ms later), which W steps of decode alone do not
        cover."""
        t_end = time.perf_counter() + ms * 1e-3
        n = 0
        while time.perf_counter() < t_end or n == 0:
            for _ in range(8):
                flush()
                fn()
            torch.cuda.synchronize()
            n += 8
        return n

    def timed(fn, steps, warmup, do_flush=True):
        for _ in range(warmup):
            flush()
            fn()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        w0 = time.perf_counter()
        for s, e in ev:
            if do_flush:
                flush()
            s.record()
            fn()
            e.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
        ms = [s.elapsed_time(e) for s, e in ev]
        return ms, wall

    def timed_inside(before, fn, after, steps, warmup):
        """Events around `fn` only, inside whole blocks: flush, before(), [fn], after()."""
        for _ in range(warmup):
            flush()
            before()
            fn()
            after()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        for s, e in ev:
            flush()
            before()
            s.record()
            fn()
            e.record()
            after()
        torch.cuda.synchronize()
        return [s.elapsed_time(e) for s, e in ev]

    tokens = [int(t) for t in args.tokens.split(",") if t]
    per_T = {}
    headline = None
    for T in tokens:
        bias = "zipf" if T == 8192 else "normal"
        fe = front_end(T, bias=bias)
        x, r = fe.x.to(dev), fe.r.to(dev)
        blk = MoEBlock(T, fe.w_norm.to(dev), fe.wgt.to(dev), fe.bias.to(dev), PW)
        blk(x, r)
        torch.cuda.synchronize()
        loads = torch.bincount(blk.topi.reshape(-1).long(), minlength=blk.E).cpu()
        n_e = int((loads > 0).sum())
        top20 = float(loads.sort(descending=True).values[: blk.E // 5].sum() / loads.sum())
        # the headline times eager launches, as the reference's bench_chain does; decode
        # sizes also time a captured HIP graph of the same chain (reported, not headline:
        # on this ROCm its replay adds launch gaps between the nodes)
        n_settle = settle(lambda: blk(x, r))
        ms, wall = timed(lambda: blk(x, r), args.steps, args.warmup)
        # the reference's no-flush median (`glm52/common.py:95-110`), same steps
        nf_ms, _ = timed(lambda: blk(x, r), args.steps, 2, do_flush=False)
        graph_ms = None
        if (not args.no_graph) and T <= 256:
            blk.capture(x, r)
            graph_ms, _ = timed(blk.replay, args.steps, args.warmup)

        # dominant kernel: the block's w13 + SwiGLU launch, events on its stream around it
        # inside whole blocks (the figure the roofline uses), and the same launch alone
        k_ms = timed_inside(lambda: blk.front_end(x, r), blk.w13_step, blk.tail, args.steps, 2)
        solo_ms, _ = timed(blk.w13_step, args.steps, 2)
        kc = RL.w13_launch(T, n_e, blk.shared_fused or blk.packed, blk.front_fused)
        k_us = statistics.mean(k_ms) * 1e3
        roof_us = RL.block_roofline_us(T, n_e)
        st = step_stats(ms)
        med_us = st["p50_us"]
        rec = {
            "us_per_block": med_us,
            "settle_steps": n_settle,
            "p10_us": st["p10_us"],
            "p90_us": st["p90_us"],
            "us_mean": st["mean_us"],
            "us_min": st["min_us"],
            "noflush_p50_us": step_stats(nf_ms)["p50_us"],
            "graph_us": round(statistics.median(graph_ms) * 1e3, 2) if graph_ms else None,
            "wall_us_per_step_incl_flush": round(wall / args.steps * 1e6, 1),
            "distinct_experts": n_e,
            "block_roofline_us": round(roof_us, 1),
            "block_roofline_frac": round(roof_us / med_us, 4),
            "w13_us": round(k_us, 2),
            "w13_p50_us": step_stats(k_ms)["p50_us"],
            "w13_solo_us": round(statistics.mean(solo_ms) * 1e3, 2),
            "w13_GBps": round(kc.bytes / (k_us * 1e-6) / 1e9, 1),
            "w13_TFLOPs": round(kc.flops / (k_us * 1e-6) / 1e12, 1),
            "w13_launch": w13_kernel_name(blk),
            "block_m": blk.bm,
            "bias": bias,
            # expert loads (slots per expert): the share the busiest 20 % of experts take,
            # and the largest and smallest load among the experts hit
            "top20_share": round(top20, 4),
            "max_load": int(loads.max()),
            "min_load": int(loads[loads > 0].min()),
        }
        if not args.no_oproj:
            rec["down_merge"] = down_merge_bench(blk, W, T, n_e, timed, args.steps, args.warmup)
            rec["oproj"] = oproj_bench(T, timed, args.steps, args.warmup, dev)
            rec["prenorm_router"] = prenorm_bench(T, timed, args.steps, args.warmup, dev)
        if headline is None:
            # every timed step of the headline size, in order (µs)
            rec["step_us"] = [round(v * 1e3, 2) for v in ms]
        per_T[str(T)] = rec
        log(f"T={T}: {rec}")
        if headline is None:
            headline = (T, rec, kc, k_us, n_e, w13_kernel_name(blk))
        del blk, x, r
        torch.cuda.empty_cache()

    T, rec, kc, k_us, n_e, kname = headline
    achieved = kc.bytes / (k_us * 1e-6) / 1e9
    # avg_us: the launch's mean duration inside the timed blocks (events around it); the
    # launch timed alone after a flush is kept beside it as solo_us
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
            "frac": round(achieved / 8000.0, 4), "traffic": None, "kernel": kname,
            "algorithmic_bytes": int(kc.bytes), "avg_us": round(k_us, 2),
            "solo_us": rec["w13_solo_us"]}
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(W, tokens, args.cpu_seconds)
    del W, flush_buf
    torch.cuda.empty_cache()
    if not args.no_traffic:
        tr = hbm_traffic(T)
        if tr is not None:
            roof["traffic"] = tr["bytes"]
            roof["traffic_over_algorithmic"] = round(tr["bytes"] / kc.bytes, 4)
            roof["traffic_detail"] = tr


    line = {
        "metric": METRIC, "value": rec["us_per_block"], "unit": "us", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(rec["us_per_block"] / 1e3, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, random init)",
        "config": {"workload": f"config1: full GLM-5.2 MoE FFN block, decode T={T}", "T": T,
                   "experts": 256, "shared_experts": 1, "topk": 8, "H": 6144, "I": 2048,
                   "weights_GB": 19.33, "launch": "eager (torch current stream)"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "per_T": per_T,
    }
    s = json.dumps(line)
    print(s, flush=True)
    if args.json_out:
        Path(args.json_out).write_text(s + "\n")
    return 0


def step_stats(ms: list) -> dict:
    """p10 / p50 / p90 / mean / min (µs) of per-step times in ms, with the reference's
    index rule for the percentiles (`glm52/common.py:112-121`)."""
    ts = sorted(ms)
    n = len(ts)
    return {"p50_us": round(ts[n // 2] * 1e3, 2), "p10_us": round(ts[max(0, int(0.1 * n))] * 1e3, 2),
            "p90_us": round(ts[min(n - 1, int(0.9 * n))] * 1e3, 2),
            "mean_us": round(statistics.fmean(ts) * 1e3, 2), "min_us": round(ts[0] * 1e3, 2)}


# untimed blocks before each size's W warm-up steps, in ms of wall time (clock settle)
SETTLE_MS = 50.0
PMC_LAUNCHES = 3
COPY_KIB = 262144  # the child's plain copies: 256 MiB read and 256 MiB written each


def w13_kernel_name(blk) -> str:
    """The kernel behind `MoEBlock.w13_step` (as the profiler names it)."""
    pk = "true" if blk.packed else "false"
    if blk.front_fused:
        return (f"moe_gemm_runs_kernel<true, false, true, {pk}> (routing + routed and shared "
                "w13 + SwiGLU)")
    if blk.shared_fused:
        return (f"moe_gemm_runs_kernel<true, false, false, {pk}> (routed and shared w13 + "
                "SwiGLU)")
    ntw = 256 if blk.bm == 256 else 512
    return (f"moe_gemm_w512_kernel<{blk.bm}, {ntw}, true, false, true, 0> (routed and shared "
            f"w13 + SwiGLU)")


def hbm_traffic(T: int, timeout_s: float = 240.0) -> dict | None:
    """HBM bytes per launch of the block's w13 launch at T tokens: two `rocprofv3 --pmc`
    runs of a child process (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each counter
    scaled by what it reads for the child's plain 256 MiB device copies.  None if the
    profiler is missing or a run fails."""
    import csv
    import shutil
    import signal
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        log("traffic: rocprofv3 not found")
        return None
    got = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="pmc_")
        cmd = [exe, "--pmc", ctr, "--output-format", "csv", "-d", d, "-o", "run", "--",
               sys.executable, str(ROOT / "bench.py"), "--pmc-child", "--tokens", str(T)]
        log(f"traffic: {ctr} pass")
        proc = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE,
                                start_new_session=True, cwd=str(ROOT))
        try:
            _, err = proc.communicate(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.wait()
            log(f"traffic: {ctr} pass timed out")
            return None
        files = list(Path(d).rglob("*counter_collection.csv"))
        if not files:
            log(f"traffic: {ctr} pass gave no counters (rc {proc.returncode}): "
                f"{err.decode(errors='replace')[-400:]}")
            return None
        rows = sorted(csv.DictReader(open(files[0])), key=lambda r: int(r["Dispatch_Id"]))
        rows = [r for r in rows if r["Counter_Name"] == ctr]
        copies = sorted((float(r["Counter_Value"]) for r in rows
                         if "copyBuffer" in r["Kernel_Name"]), reverse=True)[:3]
        if len(copies) < 3 or not rows:
            log(f"traffic: {ctr} pass: copy dispatches not found")
            return None
        name = rows[-1]["Kernel_Name"]
        vals = [float(r["Counter_Value"]) for r in rows if r["Kernel_Name"] == name][-PMC_LAUNCHES:]
        scale = COPY_KIB / statistics.mean(copies)
        got[ctr] = {"kib_raw": round(statistics.mean(vals), 1), "scale": round(scale, 4),
                    "kernel": name.replace("void ", "").replace("(anonymous namespace)::", "")
                    .split("(")[0]}
        shutil.rmtree(d, ignore_errors=True)
    f, w = got["FETCH_SIZE"], got["WRITE_SIZE"]
    nbytes = (f["kib_raw"] * f["scale"] + w["kib_raw"] * w["scale"]) * 1024
    return {"bytes": int(nbytes), "fetch_kib": f["kib_raw"], "fetch_scale": f["scale"],
            "write_kib": w["kib_raw"], "write_scale": w["scale"], "kernel": f["kernel"]}


def oproj_inputs(T: int, dev):
    """The fused o_proj + ResAdd1 chain of `fusion_amd.kernels.oproj_resadd` on the
    reference's inputs for this T (`glm52/bench/bench_f01_oproj_resadd.py:224-236`): the
    step that runs it, and K."""
    import torch

    from fusion_amd import roofline as RL
    from fusion_amd.kernels import oproj_resadd as KO

    K, N = RL.oproj_k(T), 6144
    g = torch.Generator(device=dev).manual_seed(1234)
    a = (torch.randn(T, K, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    b = (torch.randn(K, N, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    r = (torch.randn(T, N, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    out = torch.empty(T, N, device=dev, dtype=torch.bfloat16)
    acc32 = torch.zeros(T, N, device=dev, dtype=torch.float32)
    chain = KO.make_fused_chain(a, b, r, out, acc32, {"SPLIT_K": 1})

    def step():
        for fn in chain:
            fn()

    return step, K


def oproj_bench(T: int, timed, steps: int, warmup: int, dev) -> dict:
    """o_proj + ResAdd1 (upstream of the block, not part of `value`): `oproj_inputs`'s
    chain, timed like the block."""
    from fusion_amd import roofline as RL

    N = 6144
    step, K = oproj_inputs(T, dev)
    ms, _ = timed(step, steps, warmup)
    us = statistics.median(ms) * 1e3
    kc = RL.oproj_cost(T, K, N)
    roof = kc.seconds() * 1e6
    del step
    return {"K": K, "us": round(us, 2), "roofline_us": round(roof, 1),
            "roofline_frac": round(roof / us, 4), "bound": kc.bound(),
            "GBps": round(kc.bytes / (us * 1e-6) / 1e9, 1),
            "TFLOPs": round(kc.flops / (us * 1e-6) / 1e12, 1)}


def down_merge_bench(blk, W, T: int, n_e: int, timed, steps: int, warmup: int) -> dict:
    """The reference's three accumulation strategies for the routed down GEMM + merge +
    residual (fusions #8 / #9, `glm52/bench/bench_f08f09_down_merge_resadd.py:1-30`), on
    the block's own activations and routing at this T with the real w2 (routed experts
    only, residual = h): unfused = down GEMM into [T, 8, H] then moe_sum with the residual;
    atomic = seed out with the residual, then the GEMM adding into it (`fuse_merge=True`);
    token-major = one launch summing each token's experts (T <= 256 only: above, every
    token re-streams its experts).  The roofline counts w2 once per distinct expert, the
    activation rows, the residual and the output (the unfused chain's [T, 8, H] round trip
    is its own cost, not the roofline's)."""
    import torch

    from fusion_amd import roofline as RL
    from fusion_amd.kernels import moe_down_merge as KD

    H, I, k = blk.H, blk.I, blk.topk
    R = T * k
    cfg = {"BLOCK_M": blk.bm}
    if blk.packed and blk.bm != 16:  # the 512-row mapping of the atomic merge reads it
        cfg["w2_packed"] = blk.experts.w2
    tw = blk.topw.reshape(-1)
    c3 = torch.empty(R, H, dtype=torch.bfloat16, device=blk.h.device)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=blk.h.device)

    def unfused():
        KD.launch_down(blk.act, W.w2, c3, tw, blk.sti, blk.eids, blk.ntp, R, k, cfg, False)
        KD.launch_moe_sum(c3, out, blk.h, k, {}, True)

    def atomic():
        KD.launch_seed(out, blk.h, {}, True)
        KD.launch_down(blk.act, W.w2, out, tw, blk.sti, blk.eids, blk.ntp, R, k, cfg, True)

    def token_major():
        KD.launch_down_token_major(blk.act, W.w2, out, blk.topw, blk.topi, blk.h, k, {}, True)

    res = {}
    for name, fn in (("unfused_us", unfused), ("atomic_us", atomic),
                     ("token_major_us", token_major if T <= 256 else None)):
        if fn is None:
            res[name] = None
            continue
        ms, _ = timed(fn, steps, warmup)
        res[name] = round(statistics.median(ms) * 1e3, 2)
    kc = RL.KernelCost("down_merge", 2.0 * R * I * H,
                       n_e * H * I * 2 + R * I * 2 + 2 * T * H * 2)
    roof = kc.seconds() * 1e6
    best = min(v for v in res.values() if v is not None)
    res.update({"roofline_us": round(roof, 2), "roofline_frac": round(roof / best, 4),
                "bound": kc.bound()})
    del c3, out
    return res


def prenorm_bench(T: int, timed, steps: int, warmup: int, dev) -> dict:
    """The half-fused pre-norm router beside the unfused one (upstream of the block's own
    front end, not part of `value`), on the reference's #11b problem
    (`glm52/prof/prof_f11b.py:27-46`): unfused = RMSNorm into x2, then the router on the
    raw gate; half-fused = the rstd pass, then the router on the folded gate with the rstd
    epilogue; fused = `fuse_norm=True` (one launch at T <= 4).  The gate is read as [E, H]
    rows at T <= 16 and from BOUNDED_ROUTER_MIN_T tokens, as [H, E] in between, as in the
    block; from BOUNDED_ROUTER_MIN_T tokens every arm also takes the top-8 (`with_topk`),
    which is what lets the router run its bounded path there.  The roofline counts bytes
    only (the bf16 MFMA bound of the router's flops is below them at every T)."""
    import torch

    from fusion_amd import roofline as RL
    from fusion_amd.block import BOUNDED_ROUTER_MIN_T
    from fusion_amd.kernels import add_rmsnorm as KN
    from fusion_amd.kernels import lazy_prenorm as KL

    H, E = 6144, 256
    g = torch.Generator(device=dev).manual_seed(0)
    h1 = (torch.randn(T, H, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    w = (torch.randn(H, device=dev, generator=g) * 0.1 + 1).to(torch.bfloat16)
    gate = (torch.randn(E, H, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    gate_f = KL.fold_weight_nk(gate, w)
    # as the block: the gate's rows at decode and from BOUNDED_ROUTER_MIN_T tokens (there
    # with the top-k, the bounded router's consumer), the [H, E] copy in between
    topk = T >= BOUNDED_ROUTER_MIN_T
    if T <= 16 or topk:
        b_raw, b_fold = gate.t(), gate_f.t()
    else:
        b_raw, b_fold = gate.t().contiguous(), gate_f.t().contiguous()
    x2 = torch.empty_like(h1)
    rstd = torch.empty(T, device=dev, dtype=torch.float32)
    lg = torch.empty(T, E, device=dev, dtype=torch.float32)
    cfg = {}
    if topk:
        bias = torch.randn(E, device=dev, generator=g) * 0.01
        cfg = {"topw": torch.empty(T, 8, device=dev), "correction_bias": bias,
               "topi": torch.empty(T, 8, dtype=torch.int32, device=dev)}

    def unfused():
        KN.norm_only(h1, w, x2, {})
        KL.launch_router(x2, b_raw, lg, cfg, False)

    def half():
        KL.launch_rstd(h1, rstd, {})
        KL.launch_router(h1, b_fold, lg, cfg, False, 1e-5, 0, rstd)

    def fused():  # one launch at T <= 4 (gate rows); the half-fused pair above that
        KL.launch_router(h1, b_fold, lg, cfg, True)

    u_ms, _ = timed(unfused, steps, warmup)
    h_ms, _ = timed(half, steps, warmup)
    f_ms, _ = timed(fused, steps, warmup)
    u_us, h_us = statistics.median(u_ms) * 1e3, statistics.median(h_ms) * 1e3
    f_us = statistics.median(f_ms) * 1e3
    act = T * H * 2
    # half-fused: the rstd pass reads act; the router reads act and the gate, writes logits
    kc = RL.KernelCost("prenorm_router", 2.0 * T * H * E, 2 * act + H * E * 2 + T * E * 4)
    roof = kc.seconds() * 1e6
    del h1, x2, gate, gate_f, b_raw, b_fold, lg
    return {"unfused_us": round(u_us, 2), "half_fused_us": round(h_us, 2),
            "fused_us": round(f_us, 2), "with_topk": topk,
            "gain": round(u_us / min(h_us, f_us), 3),
            "roofline_us": round(roof, 2), "roofline_frac": round(roof / min(h_us, f_us), 4),
            "bound": kc.bound()}


def item_trace(T: int, PW, flush_buf, dev) -> dict:
    """The block at T (Zipf routing at 8192): after 50 ms of blocks, its w13 and its w2
    launch once each (after the flush) with the per-workgroup record on; per launch, each
    workgroup's finish time from the launch's first start, summarised per XCD."""
    import torch

    from fusion_amd import _lib
    from fusion_amd.block import MoEBlock
    from fusion_amd.problem import front_end

    fe = front_end(T, bias="zipf" if T == 8192 else "normal")
    x, r = fe.x.to(dev), fe.r.to(dev)
    blk = MoEBlock(T, fe.w_norm.to(dev), fe.wgt.to(dev), fe.bias.to(dev), PW)
    t_end = time.perf_counter() + SETTLE_MS * 1e-3
    while time.perf_counter() < t_end:
        flush_buf.zero_()
        blk(x, r)
        torch.cuda.synchronize()
    rec = torch.zeros(256 * 4, dtype=torch.int64, device=dev)
    out = {"T": T, "block_m": blk.bm, "clock": "s_memrealtime, 100 MHz"}
    for name, step in (("w13", blk.w13_step), ("w2", blk.w2_step)):
        rec.zero_()
        flush_buf.zero_()
        torch.cuda.synchronize()
        _lib.call("glm52_debug_item_trace", _lib.ptr(rec), rec.numel() * 8)
        try:
            step()
            torch.cuda.synchronize()
        finally:
            _lib.call("glm52_debug_item_trace", None, 0)
        v = rec.view(256, 4).cpu().tolist()
        rows = [w for w in v if w[0] > 0]
        t0 = min(w[0] for w in rows)
        ends = [(w[1] - t0) / 100.0 for w in rows]
        xcd = {}
        for w, e in zip(rows, ends):
            xcd.setdefault(int(w[3]), []).append((e, int(w[2])))
        per = {str(k): {"workgroups": len(l), "end_min_us": round(min(e for e, _ in l), 1),
                        "end_max_us": round(max(e for e, _ in l), 1),
                        "spread_us": round(max(e for e, _ in l) - min(e for e, _ in l), 1),
                        "items": sum(n for _, n in l)}
               for k, l in sorted(xcd.items())}
        items = [int(w[2]) for w in rows]
        out[name] = {"workgroups": len(rows), "span_us": round(max(ends), 1),
                     "end_min_us": round(min(ends), 1),
                     "spread_us": round(max(ends) - min(ends), 1),
                     "xcd_end_max_spread_us": round(max(p["end_max_us"] for p in per.values())
                                                    - min(p["end_max_us"] for p in per.values()), 1),
                     "max_spread_in_xcd_us": max(p["spread_us"] for p in per.values()),
                     "items_per_wg_min": min(items), "items_per_wg_max": max(items),
                     "items": sum(items), "per_xcd": per}
        log(f"item trace {name}: span {out[name]['span_us']} us, finish spread "
            f"{out[name]['spread_us']} us")
    return out


def calibrate(dev) -> list:
    """Read-bandwidth ceiling: median of 5 runs of `glm52_stream_read` per (size, load
    kind, grid), each after a 1 GiB flush, timed with events on torch's stream."""
    import torch

    from fusion_amd import _lib

    buf = torch.ones(4_000_000_000 // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    flush_buf = torch.empty(2 ** 28, dtype=torch.int32, device=dev)
    out = []
    for nbytes in (400_000_000, 4_000_000_000):
        for nt in (0, 1):
            for grid in (2048, 8192, 16384):
                ms = []
                for _ in range(6):
                    flush_buf.zero_()
                    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    s.record()
                    _lib.call("glm52_stream_read", _lib.ptr(buf), nbytes, nt, grid, _lib.ptr(sink),
                              _lib.stream())
                    e.record()
                    torch.cuda.synchronize()
                    ms.append(s.elapsed_time(e))
                med = statistics.median(ms[1:])
                rec = {"bytes": nbytes, "nontemporal": bool(nt), "grid": grid,
                       "us": round(med * 1e3, 2), "GBps": round(nbytes / (med * 1e-3) / 1e9, 1)}
                log(rec)
                out.append(rec)
    del buf
    out.extend(copy_ceiling(dev, flush_buf))
    return out


def copy_ceiling(dev, flush_buf) -> list:
    """Read + write ceiling for the vector kernels at T = 8192: two plain device copies of a
    [8192, 6144] bf16 tensor (403 MB moved, the bytes of ResAdd + RMSNorm) against this
    build's ResAdd + RMSNorm on the same sizes, median of 20 runs after the benchmark's
    zeroing flush (which leaves the Infinity Cache full of dirty lines) and after a flush
    followed by a read of the flush buffer (clean lines)."""
    import torch

    from fusion_amd.kernels import add_rmsnorm as KN

    T, H = 8192, 6144
    a, b = (torch.randn(T, H, device=dev).to(torch.bfloat16) for _ in range(2))
    c, d = torch.empty_like(a), torch.empty_like(a)
    w = torch.ones(H, dtype=torch.bfloat16, device=dev)
    nbytes = 4 * T * H * 2
    kinds = {"copy x2": lambda: (c.copy_(a), d.copy_(b)),
             "add_rmsnorm": lambda: KN.fused_add_rmsnorm(a, b, w, c, d, {"eps": 1e-5})}
    out = []
    for flush_kind in ("zero", "zero+read"):
        for name, fn in kinds.items():
            ms = []
            for _ in range(21):
                flush_buf.zero_()
                if flush_kind == "zero+read":
                    flush_buf.sum()
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                fn()
                e.record()
                torch.cuda.synchronize()
                ms.append(s.elapsed_time(e))
            med = statistics.median(ms[1:])
            rec = {"read_write": name, "bytes": nbytes, "flush": flush_kind,
                   "us": round(med * 1e3, 2), "GBps": round(nbytes / (med * 1e-3) / 1e9, 1)}
            log(rec)
            out.append(rec)
    return out


def cpu_model() -> str:
    """The host CPU's model name (as `lscpu` prints it), from /proc/cpuinfo."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


# repetitions per T (median reported), the plan of the reference's CPU baseline; T = 1
# runs for `--cpu-seconds` instead
CPU_REPS = {256: 5, 2048: 3, 8192: 1}
CPU_BUDGET_S = 150.0  # whole CPU leg; a T whose one block is predicted past it is skipped


def cpu_baseline(W, tokens: list, seconds: float) -> dict:
    """The oracle's restatement of the reference path on all of the host's cores, at every
    T of `tokens`: add_rmsnorm, the fp32 router with the correction bias, the per-expert
    bf16 `moe_mlp` and the fp32 shared expert, composed as `glm52/bench/bench_layer.py:365-374`.
    `value` is the first T (configuration 1); the others are under `per_T`."""
    import torch

    from fusion_amd.problem import front_end
    from oracle import glm52_oracle as O

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    w13s, w2s = W.w13s.cpu(), W.w2s.cpu()
    full = None  # the whole expert stack on the host, copied once for T > 1
    per_T = {}
    t_leg = time.perf_counter()
    last = None  # (T, seconds per block) of the previous T, to predict the next
    for T in tokens:
        fe = front_end(T, bias="zipf" if T == 8192 else "normal")
        if T == 1:
            y, _ = O.add_rmsnorm(fe.x, fe.r, fe.w_norm)
            _, _, ti = O.router_reference(y, fe.gate, fe.bias)
            experts = sorted(set(ti.view(-1).tolist()))
            w13 = {e: W.w13[e].cpu() for e in experts}
            w2 = {e: W.w2[e].cpu() for e in experts}

            def block():
                y, h = O.add_rmsnorm(fe.x, fe.r, fe.w_norm)
                _, tw, ti = O.router_reference(y, fe.gate, fe.bias)
                routed = O.moe_mlp_rows(y, w13, w2, tw, ti, [0]).to(torch.bfloat16).float()
                return (routed + h.float() + O.shared_expert(y, w13s, w2s)).to(torch.bfloat16)
        else:
            if full is None:
                full = (W.w13.cpu(), W.w2.cpu())

            def block():
                y, h = O.add_rmsnorm(fe.x, fe.r, fe.w_norm)
                _, tw, ti = O.router_reference(y, fe.gate, fe.bias)
                routed = O.moe_mlp(y, full[0], full[1], tw, ti).float()
                return (routed + h.float() + O.shared_expert(y, w13s, w2s)).to(torch.bfloat16)
        left = CPU_BUDGET_S - (time.perf_counter() - t_leg)
        if last is not None:
            predicted = last[1] * T / last[0]
            if predicted > left:
                per_T[str(T)] = {"us": None, "reps": 0,
                                 "note": f"skipped: one block predicted {predicted:.0f}s, "
                                         f"{max(left, 0):.0f}s of the CPU leg left"}
                log(f"cpu baseline T={T}: {per_T[str(T)]['note']}")
                continue
        times = []
        if T == 1:
            block()  # warm
            t_end = time.perf_counter() + seconds
            while time.perf_counter() < t_end or len(times) < 3:
                t0 = time.perf_counter()
                block()
                times.append(time.perf_counter() - t0)
        else:
            for _ in range(CPU_REPS.get(T, 1)):
                t0 = time.perf_counter()
                block()
                times.append(time.perf_counter() - t0)
                if time.perf_counter() - t_leg > CPU_BUDGET_S:
                    break
        med = statistics.median(times)
        last = (T, med)
        per_T[str(T)] = {"us": round(med * 1e6, 1), "reps": len(times)}
        log(f"cpu baseline T={T}: {per_T[str(T)]}")
    del full
    T0 = tokens[0]
    return {"value": per_T[str(T0)]["us"], "unit": "us", "cores": ncores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"full blocks at T={T0} (configuration 1), median of "
                      f"{per_T[str(T0)]['reps']} over ~{seconds:.0f}s; torch-CPU fp32 router + "
                      f"per-expert bf16 moe_mlp + fp32 shared expert on {ncores} threads; "
                      f"other T under per_T (median of 5 at T<=256, 3 at 2048, 1 at 8192)",
            "per_T": per_T}


if __name__ == "__main__":
    sys.exit(main())
