"""CPU test of the reference-name binding: after `fusion_amd.binding.install()` the
reference's import paths (`glm52.kernels.<module>`, `glm52.reference.moe_align_block_size`,
as `glm52/bench/bench_layer.py:45-52` imports them) resolve to this build's modules; no
launch is made."""

from __future__ import annotations

import importlib
import sys

from fusion_amd import binding


def test_install_binds_the_reference_names():
    try:
        bound = binding.install()
        assert "glm52.reference.moe_align_block_size" in bound
        for name in binding.KERNEL_MODULES:
            mine = importlib.import_module(f"fusion_amd.kernels.{name}")
            assert sys.modules[f"glm52.kernels.{name}"] is mine
            assert importlib.import_module(f"glm52.kernels.{name}") is mine
        from glm52.kernels import moe_gateup, norm_router  # noqa: F401  (the callers' form)
        from glm52.reference import moe_align_block_size

        assert moe_gateup.launch_gateup.__module__ == "fusion_amd.kernels.moe_gateup"
        assert norm_router.topk_only.__module__ == "fusion_amd.kernels.norm_router"
        assert moe_align_block_size is binding.moe_align_block_size
    finally:
        binding.uninstall()
    assert "glm52.kernels.moe_gateup" not in sys.modules
