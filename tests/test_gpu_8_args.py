"""Argument checks on the host that keep a kernel from reading what it was not given: a
forced token-major tail where its shared-expert input is never written, and a packed
weight buffer made for another shape.  Each raises ValueError before any launch."""

from __future__ import annotations

import pytest
import torch

from fusion_amd.block import MoEBlock
from fusion_amd.dispatch import moe_align_block_size
from fusion_amd.kernels import moe_gateup as KG

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def test_token_major_override_needs_the_streaming_layout(gpu):
    E, H, I, T = 16, 512, 256, 512
    w13 = torch.zeros(E, 2 * I, H, dtype=BF16, device=gpu)
    w2 = torch.zeros(E, H, I, dtype=BF16, device=gpu)
    w13s, w2s = w13[:1].clone(), w2[:1].clone()
    wn = torch.ones(H, dtype=BF16, device=gpu)
    wgt = torch.zeros(H, E, dtype=BF16, device=gpu)
    bias = torch.zeros(E, dtype=torch.float32, device=gpu)
    with pytest.raises(ValueError, match="token_major"):
        MoEBlock(T, wn, wgt, bias, w13, w2, w13s, w2s, token_major=True)
    blk = MoEBlock(T, wn, wgt, bias, w13, w2, w13s, w2s)  # the default is accepted
    assert not blk.token_major


def test_packed_weight_shape_is_checked(gpu):
    E, H, I, T, K = 4, 256, 256, 64, 8
    w13 = (torch.randn(E, 2 * I, H, device=gpu) * 0.02).to(BF16)
    packed = KG.pack_w512(w13, I, I, True)
    ids = torch.randint(0, E, (T, K), dtype=torch.int32, device=gpu)
    sti, eids, ntp = moe_align_block_size(ids, 64, E)
    a = torch.randn(T, H, device=gpu).to(BF16)
    c = torch.empty(T * K, I, dtype=BF16, device=gpu)
    cfg = {"BLOCK_M": 64}
    KG.moe_gemm_packed(a, K, packed, c, None, sti, eids, ntp, T * K, I, True, cfg)
    with pytest.raises(ValueError, match="packed for"):
        KG.moe_gemm_packed(a, K, packed, c[:, :256], None, sti, eids, ntp, T * K, 256, False,
                           cfg)
    bare = torch.empty(packed.numel() - 8, dtype=BF16, device=gpu)
    with pytest.raises(ValueError, match="whole number"):
        KG.moe_gemm_packed(a, K, bare, c, None, sti, eids, ntp, T * K, I, True, cfg)
    torch.cuda.synchronize()
