"""Empty batches (T = 0 tokens) through every launcher: each returns without error and
without touching its outputs, as the reference's destination-passing launchers do when
their grid is empty."""

from __future__ import annotations

import pytest
import torch

from fusion_amd.dispatch import moe_align_block_size
from fusion_amd.kernels import add_rmsnorm as KN
from fusion_amd.kernels import lazy_prenorm as KL
from fusion_amd.kernels import moe_down_merge as KD
from fusion_amd.kernels import moe_gateup as KG
from fusion_amd.kernels import norm_router as KR
from fusion_amd.kernels import oproj_resadd as KO

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
H, E, I, K = 6144, 16, 2048, 8


def test_empty_batches(gpu):
    z = lambda *s, dt=BF16: torch.empty(*s, dtype=dt, device=gpu)  # noqa: E731
    x, r, h, y = z(0, H), z(0, H), z(0, H), z(0, H)
    w = torch.ones(H, dtype=BF16, device=gpu)
    KN.fused_add_rmsnorm(x, r, w, h, y, {})
    KN.add_only(x, r, h, {})
    KN.norm_only(h, w, y, {})
    gate = torch.zeros(E, H, dtype=BF16, device=gpu)
    logits = z(0, E, dt=torch.float32)
    KR.router_gemm(y, gate.t(), logits, {})
    KR.router_gemm(y, gate.t().contiguous(), logits, {})
    topw, topi = z(0, K, dt=torch.float32), z(0, K, dt=torch.int32)
    KR.topk_only(logits, topw, topi, {})
    sti, eids, ntp = moe_align_block_size(topi, 16, E)
    torch.cuda.synchronize()
    assert int(ntp.item()) == 0
    w13 = torch.zeros(E, 2 * I, H, dtype=BF16, device=gpu)
    w2 = torch.zeros(E, H, I, dtype=BF16, device=gpu)
    act = z(0, I)
    KG.launch_gateup(y, w13, act, sti, eids, ntp, 0, K, I, {"BLOCK_M": 16}, True)
    y3 = z(0, H)
    KD.launch_down(act, w2, y3, z(0, dt=torch.float32), sti, eids, ntp, 0, K, {"BLOCK_M": 16},
                   False)
    out = z(0, H)
    KD.launch_down(act, w2, out, z(0, dt=torch.float32), sti, eids, ntp, 0, K, {"BLOCK_M": 16},
                   True)
    KD.launch_moe_sum(y3.view(0, K, H), out, r, K, {}, True)
    KD.launch_down_token_major(act, w2, out, topw, topi, r, K, {}, True)
    a = z(0, 32768)
    b = torch.zeros(32768, H, dtype=BF16, device=gpu)
    KO.gemm_launch(a, b, out, r, {}, True, False)
    KO.epilogue_launch(out, r, out, {}, True)
    rstd = z(0, dt=torch.float32)
    KL.launch_rstd(h, rstd, {})
    KL.launch_router(h, gate.t(), logits, {}, True)
    torch.cuda.synchronize()
