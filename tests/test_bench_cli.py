"""bench.py's command-line contract, on the CPU: a multi-GPU request exits with a message
(this build measures one MI355X) before anything touches a device."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args, env_extra=None):
    import os

    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, env=env,
                          capture_output=True, text=True, timeout=120)


def test_bench_refuses_more_than_one_gpu():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one MI355X" in r.stdout and "--gpus 1" in r.stdout


def test_bench_refuses_a_multi_rank_launch():
    r = _run("--gpus", "1", env_extra={"WORLD_SIZE": "4"})
    assert r.returncode == 2
    assert "one MI355X" in r.stdout


def test_bench_help_names_the_contract_flags():
    r = _run("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--tokens"):
        assert flag in r.stdout
