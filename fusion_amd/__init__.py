"""MI355X-native GLM-5.2 MoE FFN block (gfx950 HIP kernels behind a C-ABI library).

`fusion_amd.kernels.*` keeps the launcher names and signatures of the reference package's
`glm52/kernels/*.py`; `fusion_amd.dispatch.moe_align_block_size` replaces
`glm52/reference.py::moe_align_block_size`; `fusion_amd.block.MoEBlock` composes the block.
"""

__all__ = ["config", "kernels", "dispatch", "block", "problem"]
