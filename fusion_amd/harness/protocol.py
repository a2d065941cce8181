"""Measurement protocol and result schema of the whole-layer harness.

Restates, for MI355X, the parts of the reference's benchmark methodology that make its
tables comparable:

  bench_chain    `glm52/common.py:73-122`: a chain of launches timed as one operation,
                 one cache flush before every timed repetition, median / p10 / p90 over
                 the repetitions plus a no-flush median.  The flush zeroes a 1 GiB buffer,
                 four times MI355X's 256 MB Infinity Cache (the reference flushes an L2).
  rel_err/check  `glm52/common.py:186-200`: max-abs error over the reference's max-abs,
                 and the acceptance gate on it.
  record         `glm52/common.py:206-220`: one JSON file per result with a `_meta` block
                 (time, device, visible devices, torch and HIP versions).
  quarantine_foreign_results
                 `run_h200.py:972-1023`: result files whose `_meta.device` is not the
                 present GPU are moved aside (never deleted) before a resumable run, so a
                 result from another device is never reported as a fresh measurement.
  ab_verdict     `glm52/bench/bench_layer_ab.py:77-113`: interleaved rounds; a winner only
                 when its median beats the runner-up's by more than the larger round-to-
                 round spread of the two, else the tied set.
"""

from __future__ import annotations

import json
import os
import shutil
import statistics
import time
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Callable, Sequence

FLUSH_BYTES = 1 << 30


@dataclass
class Timing:
    p50_ms: float
    p10_ms: float
    p90_ms: float
    mean_ms: float
    n: int
    noflush_p50_ms: float = float("nan")

    def as_dict(self) -> dict:
        return asdict(self)


_FLUSH: dict = {}


def flush_cache(device=None) -> None:
    """Evict the caches between repetitions: zero a 1 GiB device buffer."""
    import torch

    dev = torch.device(device or "cuda")
    key = (dev.type, dev.index)
    buf = _FLUSH.get(key)
    if buf is None:
        buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)
        _FLUSH[key] = buf
    buf.zero_()


def _summary(times: list[float], noflush: float) -> Timing:
    ts = sorted(times)
    n = len(ts)
    return Timing(p50_ms=ts[n // 2], p10_ms=ts[max(0, int(0.1 * n))],
                  p90_ms=ts[min(n - 1, int(0.9 * n))], mean_ms=statistics.fmean(ts), n=n,
                  noflush_p50_ms=noflush)


def bench_chain(fns: Sequence[Callable[[], object]] | Callable[[], object], warmup: int = 25,
                rep: int = 100, flush: bool = True) -> Timing:
    """Time `fns` run back to back as one operation (events on torch's current stream)."""
    import torch

    if callable(fns):
        fns = [fns]
    for _ in range(warmup):
        for fn in fns:
            fn()
    torch.cuda.synchronize()

    def measure(do_flush: bool) -> list[float]:
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(rep)]
        for s, e in ev:
            if do_flush:
                flush_cache()
            s.record()
            for fn in fns:
                fn()
            e.record()
        torch.cuda.synchronize()
        return [s.elapsed_time(e) for s, e in ev]

    times = measure(flush)
    nf = sorted(measure(False))
    return _summary(times, nf[len(nf) // 2])


def rel_err(got, ref) -> float:
    """Max-abs error over the reference's max-abs (floored at 1e-6)."""
    got32, ref32 = got.float(), ref.float()
    denom = ref32.abs().max().clamp_min(1e-6)
    return ((got32 - ref32).abs().max() / denom).item()


def check(got, ref, tol: float = 2e-2, label: str = "") -> dict:
    import torch

    err = rel_err(got, ref)
    ok = err <= tol and bool(torch.isfinite(got.float()).all().item())
    return {"label": label, "rel_err": err, "tol": tol, "ok": bool(ok)}


def device_name() -> str:
    import torch

    try:
        return torch.cuda.get_device_name(0) if torch.cuda.is_available() else ""
    except Exception:  # noqa: BLE001 -- no device: the fence is skipped, and says so
        return ""


def _norm_dev(name) -> str:
    return " ".join(str(name or "").split()).lower()


def record(name: str, payload: dict, results_dir: str | os.PathLike,
           device: str | None = None) -> Path:
    """Write `payload` to `<results_dir>/<name>.json` with a `_meta` block."""
    import torch

    path = Path(results_dir) / f"{name}.json"
    path.parent.mkdir(parents=True, exist_ok=True)
    payload = dict(payload)
    meta = dict(payload.get("_meta") or {})
    meta.update({
        "recorded_at": time.strftime("%Y-%m-%d %H:%M:%S"),
        "device": device if device is not None else device_name(),
        "visible_devices": os.environ.get("HIP_VISIBLE_DEVICES",
                                          os.environ.get("CUDA_VISIBLE_DEVICES", "all")),
        "torch": torch.__version__,
        "hip": getattr(torch.version, "hip", None),
    })
    payload["_meta"] = meta
    path.write_text(json.dumps(payload, indent=2, default=str))
    return path


def quarantine_foreign_results(results_dir: str | os.PathLike, device: str,
                               enabled: bool = True, warnings: list | None = None) -> list[dict]:
    """Move every result JSON under `results_dir` whose `_meta.device` differs from
    `device` into `_quarantine_foreign_<time>/` (same relative path).  Returns what moved."""
    warnings = warnings if warnings is not None else []
    results = Path(results_dir)
    moved: list[dict] = []
    if not results.exists():
        return moved
    if not device:
        warnings.append("device name unknown -- result files were not device-fenced")
        return moved
    if not enabled:
        warnings.append("device fence disabled: pre-existing results were reused unchecked")
        return moved
    present = _norm_dev(device)
    qdir = results / f"_quarantine_foreign_{time.strftime('%Y%m%d_%H%M%S')}"
    for p in sorted(results.rglob("*.json")):
        rel = p.relative_to(results)
        if any(part.startswith("_quarantine_foreign_") for part in rel.parts):
            continue
        try:
            payload = json.loads(p.read_text())
        except (OSError, ValueError):
            continue  # unreadable: left for the resume logic to report
        got = _norm_dev((payload.get("_meta") or {}).get("device")) \
            if isinstance(payload, dict) else ""
        if got == present:
            continue
        dst = qdir / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.move(str(p), str(dst))
        moved.append({"file": str(rel), "recorded_device": got or None,
                      "present_device": present, "moved_to": str(dst)})
    if moved:
        warnings.append(f"{len(moved)} result file(s) from another device were quarantined "
                        f"under {qdir.name}")
    return moved


def ab_verdict(rounds: dict[str, list[float]]) -> tuple[dict, dict]:
    """Per-candidate statistics over interleaved rounds, and the verdict: the best median
    wins only if its gap to the runner-up exceeds the larger max - min spread of the two;
    otherwise every candidate within that spread of the best is reported tied."""
    stats = {}
    for name, xs in rounds.items():
        xs_s = sorted(xs)
        med = statistics.median(xs)
        stats[name] = {"median": med, "min": xs_s[0], "max": xs_s[-1],
                       "spread_pct": (xs_s[-1] - xs_s[0]) / med * 100 if med else 0.0,
                       "rounds": list(xs)}
    order = sorted(stats, key=lambda k: stats[k]["median"])
    if len(order) < 2:
        return stats, ({"best": order[0]} if order else {})
    best, runner = order[0], order[1]
    gap = stats[runner]["median"] - stats[best]["median"]
    noise = max(stats[best]["max"] - stats[best]["min"],
                stats[runner]["max"] - stats[runner]["min"])
    tied = [n for n in order if stats[n]["median"] - stats[best]["median"] <= noise]
    return stats, {"best": best, "runner_up": runner, "gap_ms": gap, "noise_ms": noise,
                   "separated": gap > noise, "tied_set": tied}
