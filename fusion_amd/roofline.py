"""Algorithmic flops and HBM bytes of the MoE block's kernels, and the MI355X roofline.

Follows the reference's traffic model (`glm52/traffic.py:171-227`): every kernel costs
max(flops / P, bytes / BW), a chain costs the sum, and expert weights are counted once
per distinct expert touched (`glm52/traffic.py:8-10`).  Peaks are MI355X's published
dense figures (bf16 MFMA 2.5 PFLOP/s, HBM3E 8 TB/s).

Per-kernel bytes (T tokens, R = 8T routed rows, act = T * H * 2, n_e distinct experts):
    addnorm   4 act
    router    act + H * E * 2 (gate) + T * E * 4 (logits)
    w13       act + n_e * 2I * H * 2 + R * I * 2
    w2        R * I * 2 + n_e * H * I * 2 + R * H * 2
    shared    act + 3 * I * H * 2 + T * I * 2 + act
    merge     8 act + 3 act
"""

from __future__ import annotations

from dataclasses import dataclass

from . import config as C

PEAK_BF16_FLOPS = 2.5e15
PEAK_HBM_BYTES = 8.0e12


@dataclass
class KernelCost:
    name: str
    flops: float
    bytes: float

    def seconds(self, peak_flops: float = PEAK_BF16_FLOPS, peak_bw: float = PEAK_HBM_BYTES) -> float:
        return max(self.flops / peak_flops, self.bytes / peak_bw)

    def bound(self, peak_flops: float = PEAK_BF16_FLOPS, peak_bw: float = PEAK_HBM_BYTES) -> str:
        return "mfma" if self.flops / peak_flops > self.bytes / peak_bw else "hbm"


def expected_distinct_experts(T: int, topk: int = C.TOPK, E: int = C.E) -> float:
    """Uniform-routing expectation E * (1 - (1 - 1/E)^(T * topk)) (`glm52/traffic.py:29-38`)."""
    return E * (1.0 - (1.0 - 1.0 / E) ** (T * topk))


def block_kernels(T: int, n_e: float, H: int = C.H, I: int = C.I, E: int = C.E,
                  topk: int = C.TOPK) -> list[KernelCost]:
    R = T * topk
    act = T * H * 2
    return [
        KernelCost("addnorm", 0.0, 4 * act),
        KernelCost("router", 2.0 * T * H * E, act + H * E * 2 + T * E * 4),
        KernelCost("w13", 2.0 * R * H * 2 * I, act + n_e * 2 * I * H * 2 + R * I * 2),
        KernelCost("w2", 2.0 * R * I * H, R * I * 2 + n_e * H * I * 2 + R * H * 2),
        KernelCost("shared", 2.0 * T * H * 2 * I + 2.0 * T * I * H,
                   act + 3 * I * H * 2 + T * I * 2 + act),
        KernelCost("merge", 0.0, 11 * act),
    ]


def block_roofline_us(T: int, n_e: float, **kw) -> float:
    return sum(k.seconds() for k in block_kernels(T, n_e, **kw)) * 1e6


def kernel(name: str, T: int, n_e: float) -> KernelCost:
    return next(k for k in block_kernels(T, n_e) if k.name == name)


def w13_launch(T: int, n_e: float, shared: bool, route: bool, H: int = C.H, I: int = C.I,
               E: int = C.E, topk: int = C.TOPK) -> KernelCost:
    """One w13 + SwiGLU launch as the block issues it: the routed experts, plus the shared
    expert when it runs in the same launch (weight streaming), plus, when the launch derives
    the routing itself (T <= 4), the logits and bias it reads and the ids, weights and
    dispatch layout it writes.  Weights count once per distinct expert; the activation rows
    are read once."""
    R = T * topk
    s = 1 if shared else 0
    rows = R + s * T
    nbytes = T * H * 2 + (n_e + s) * 2 * I * H * 2 + rows * I * 2
    if route:
        cap = -(-(R + E * 15) // 16) * 16
        nbytes += T * E * 4 + E * 4 + R * 8 + 4 * (cap + cap // 16 + 1)
    return KernelCost("w13", 2.0 * rows * H * 2 * I, nbytes)


OPROJ_K_DECODE = 32768   # absorbed MLA: 64 heads x 512 (`glm52/config.py:58-59`)
OPROJ_K_PREFILL = 16384  # 64 heads x 256 (`glm52/config.py:55-56`)


def oproj_k(T: int) -> int:
    """K of o_proj in the reference's regimes: decode batches use the absorbed-MLA width,
    prefill (T >= 2048) the non-absorbed one (`glm52/config.py:83-88`)."""
    return OPROJ_K_PREFILL if T >= 2048 else OPROJ_K_DECODE


def oproj_cost(T: int, K: int, N: int = C.H) -> KernelCost:
    """o_proj + ResAdd1, fused: read A [T, K], B [K, N] and r, write h1 [T, N]."""
    return KernelCost("oproj", 2.0 * T * K * N, K * N * 2 + T * K * 2 + 2 * T * N * 2)
