"""Bind this build under the reference package's own module paths.

The reference's callers import the launchers as `glm52.kernels.<module>` and the dispatch
layout as `glm52.reference.moe_align_block_size` (`glm52/bench/bench_layer.py:45-52`,
`:379-388`).  `install()` makes those names resolve to this build:

* `glm52.kernels.{add_rmsnorm, norm_router, moe_gateup, moe_down_merge, merge_resadd,
  oproj_resadd, lazy_prenorm}` become the modules of `fusion_amd.kernels` (entered in
  `sys.modules` and set as attributes of the `glm52.kernels` package);
* `glm52.reference.moe_align_block_size` becomes the device layout with the reference's
  exact-size return (`exact=True`: one device-to-host read of the padded count, as the
  reference's own `.item()` at `glm52/reference.py:103`), same three tensors, same values.

When the reference package is importable (a maintainer's checkout), its `glm52` and
`glm52.reference` modules are kept and only those names are replaced, so the rest of
`glm52.reference` (the CPU ground truth) stays the reference's own.  When it is not (a
machine that has only this build), `install()` creates the `glm52`, `glm52.kernels` and
`glm52.reference` packages with just these names.  A maintainer binds the reference by
calling `install()` from the reference's `glm52/kernels/__init__.py`.
"""

from __future__ import annotations

import importlib
import sys
import types

KERNEL_MODULES = ("add_rmsnorm", "norm_router", "moe_gateup", "moe_down_merge", "merge_resadd",
                  "oproj_resadd", "lazy_prenorm")


def moe_align_block_size(topk_ids, block_m: int, num_experts: int):
    """`glm52/reference.py:85-128` on the device: exact-size (sorted_token_ids,
    expert_ids, num_tokens_post_padded), as the reference returns them."""
    from .dispatch import moe_align_block_size as device_layout

    return device_layout(topk_ids, block_m, num_experts, exact=True)


def _package(name: str) -> types.ModuleType:
    mod = sys.modules.get(name)
    if mod is None:
        try:
            mod = importlib.import_module(name)
        except ImportError:
            mod = types.ModuleType(name)
            mod.__path__ = []  # a package, so submodule imports resolve through sys.modules
            sys.modules[name] = mod
    return mod


def install() -> list[str]:
    """Point the reference's module names at this build; returns the names bound."""
    root = _package("glm52")
    kern = sys.modules.get("glm52.kernels")
    if kern is None:
        # the reference's kernels/__init__.py may be what is calling install(): only
        # create the package when it is not being (or has not been) imported
        kern = types.ModuleType("glm52.kernels")
        kern.__path__ = []
        sys.modules["glm52.kernels"] = kern
    root.kernels = kern
    bound = []
    for name in KERNEL_MODULES:
        mod = importlib.import_module(f"fusion_amd.kernels.{name}")
        sys.modules[f"glm52.kernels.{name}"] = mod
        setattr(kern, name, mod)
        bound.append(f"glm52.kernels.{name}")
    ref = _package("glm52.reference")
    ref.moe_align_block_size = moe_align_block_size
    root.reference = ref
    bound.append("glm52.reference.moe_align_block_size")
    return bound


def uninstall() -> None:
    """Remove what `install()` created when no reference package was importable (tests)."""
    for name in [n for n in sys.modules if n == "glm52" or n.startswith("glm52.")]:
        mod = sys.modules[name]
        if getattr(mod, "__file__", None) is None or name.startswith("glm52.kernels."):
            del sys.modules[name]
