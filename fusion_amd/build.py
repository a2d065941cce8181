"""Build `fusion_amd/libglm52_hip.so` from `fusion_amd/csrc/*.hip` for gfx950.

    python -m fusion_amd.build            # build in place (always recompiles)

The library is a plain C-ABI shared object (`include/glm52_hip.h`).  It links the HIP
runtime by SONAME (`libamdhip64.so.7`), so inside a process that imported torch first it
binds to the runtime torch already loaded and shares its device pointers and streams.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libglm52_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-mcode-object-version=5",
    # packed fp32 VALU forms are disabled for every kernel of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source (one hipcc per file, in parallel) and link them into one
    shared library; raises on failure.  The sources share no device code, so each object
    carries its own gfx950 code object."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = max(1, min(len(srcs), len(os.sched_getaffinity(0)), 16))
    with tempfile.TemporaryDirectory(prefix="glm52_build_") as tmpdir:
        objs = [Path(tmpdir) / (src.stem + ".o") for src in srcs]
        with ThreadPoolExecutor(jobs) as pool:
            list(pool.map(lambda so: _run([hipcc(), *compile_flags, "-c", "-I", str(CSRC),
                                           "-o", str(so[1]), str(so[0])], verbose),
                          zip(srcs, objs)))
        tmp = LIB.with_suffix(".so.tmp")
        _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
              *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
