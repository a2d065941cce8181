"""Synthetic inputs of the benchmark configurations, generated deterministically.

The reference draws everything from seeded torch generators; there is no checkpoint or
dataset (`glm52/bench/bench_layer.py:292-346`).  The same is done here:

* front end (x, r, RMSNorm weight, router gate, correction bias): a CPU
  `torch.Generator` seeded with 1234 + T, so the CPU oracle and the GPU see the same
  bytes;  x, r ~ N(0, 1); w = 1 + N(0, 0.02); gate [E, H] ~ N(0, 1/H)
  (`glm52/bench/bench_f04f05_norm_router.py:292-300`); bias ~ N(0, 0.01), or the skewed
  0.5 * (e + 1)^-1.1 of configuration 4.
* expert weights: w13 [E, 2I, H] and w2 [E, H, I] ~ N(0, 0.02), filled one expert at a
  time in bf16 on the target device (no fp32 temporary of the 19.3 GB stack), from a
  generator on that device seeded per tensor.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import config as C

BF16 = torch.bfloat16


@dataclass
class FrontEnd:
    x: torch.Tensor  # [T, H] bf16
    r: torch.Tensor  # [T, H] bf16
    w_norm: torch.Tensor  # [H] bf16
    gate: torch.Tensor  # [E, H] bf16 (nn.Linear layout)
    bias: torch.Tensor  # [E] fp32

    @property
    def wgt(self) -> torch.Tensor:
        """[H, E] layout the router kernel consumes (`wgt_from_gate`)."""
        return self.gate.t().contiguous()

    def to(self, device) -> "FrontEnd":
        return FrontEnd(*(t.to(device) for t in (self.x, self.r, self.w_norm, self.gate, self.bias)))


def zipf_bias(E: int = C.E, s: float = 1.1, scale: float = 0.5) -> torch.Tensor:
    """Configuration 4's skewed correction bias: scale * (e + 1)^-s."""
    e = torch.arange(E, dtype=torch.float64)
    return (scale * (e + 1.0) ** (-s)).to(torch.float32)


def front_end(T: int, seed: int | None = None, H: int = C.H, E: int = C.E,
              bias: str = "normal") -> FrontEnd:
    g = torch.Generator().manual_seed(C.seed_for(T) if seed is None else seed)
    x = torch.randn(T, H, generator=g).to(BF16)
    r = torch.randn(T, H, generator=g).to(BF16)
    w = (1.0 + 0.02 * torch.randn(H, generator=g)).to(BF16)
    gate = (torch.randn(E, H, generator=g) * H ** -0.5).to(BF16)
    nb = (0.01 * torch.randn(E, generator=g)).to(torch.float32)
    if bias == "normal":
        b = nb
    elif bias == "zipf":
        b = zipf_bias(E)
    elif bias == "zero":
        b = torch.zeros(E, dtype=torch.float32)
    else:
        raise ValueError(f"unknown bias kind {bias!r}")
    return FrontEnd(x, r, w, gate, b)


@dataclass
class ExpertWeights:
    w13: torch.Tensor  # [E, 2I, H] bf16
    w2: torch.Tensor  # [E, H, I] bf16
    w13s: torch.Tensor  # [1, 2I, H] bf16
    w2s: torch.Tensor  # [1, H, I] bf16


def _fill(t: torch.Tensor, std: float, g: torch.Generator) -> torch.Tensor:
    for e in range(t.shape[0]):
        t[e].normal_(0.0, std, generator=g)
    return t


def expert_weights(E: int = C.E, H: int = C.H, I: int = C.I, device="cuda", seed: int = 7,
                   std: float = 0.02) -> ExpertWeights:
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    w13 = _fill(torch.empty(E, 2 * I, H, dtype=BF16, device=dev), std, g)
    w2 = _fill(torch.empty(E, H, I, dtype=BF16, device=dev), std, g)
    w13s = _fill(torch.empty(1, 2 * I, H, dtype=BF16, device=dev), std, g)
    w2s = _fill(torch.empty(1, H, I, dtype=BF16, device=dev), std, g)
    return ExpertWeights(w13, w2, w13s, w2s)
