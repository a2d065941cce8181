"""The whole MoE block on one MI355X with the real 256-expert weight set (19.3 GB)
resident, at the token counts of the benchmark configurations.

* front end (h, y, logits, ids, weights) and the dispatch layout: bit for bit against
  the CPU oracle's exact rule;
* block output: against the framework-faithful fp32 ground truth of
  `glm52/bench/bench_layer.py:365-374` on sampled tokens, computed in fp32 with torch on
  the GPU (a floating-point reference of the same op), within rtol 2e-2 / atol 2e-2 and
  the reference's own `rel_err <= 2e-2` gate (`glm52/common.py:186-200`);
* HIP-graph replay and repeat launches: bitwise identical to the eager result.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from fusion_amd.block import MoEBlock
from fusion_amd.problem import expert_weights, front_end
from oracle import glm52_oracle as O

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def weights(gpu):
    say("allocating the 256-expert weight set")
    w = expert_weights(device=gpu)
    torch.cuda.synchronize()
    yield w
    del w
    torch.cuda.empty_cache()


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rows_reference(y, h, ids, tw, W, rows):
    """Framework-faithful block output for token rows `rows` in fp32 on the GPU:
    bf16 w13 linear -> bf16 SwiGLU -> bf16 w2 linear -> fp32 weighted sum
    (`glm52/reference.py:134-156`), + h, + fp32 shared expert (`bench_layer.py:369-372`)."""
    out = []
    for t in rows:
        acc = torch.zeros(y.shape[1], dtype=torch.float32, device=y.device)
        yt = y[t].float()
        for k in range(ids.shape[1]):
            e = int(ids[t, k])
            hh = (W.w13[e].float() @ yt).to(BF16)
            a = O.silu_and_mul(hh.cpu().unsqueeze(0)).to(y.device)[0]
            yo = (W.w2[e].float() @ a.float()).to(BF16).float()
            acc += yo * float(tw[t, k])
        routed = acc.to(BF16).float()
        sh = W.w13s[0].float() @ yt
        sa = O.silu_and_mul(sh.to(BF16).cpu().unsqueeze(0)).to(y.device)[0]
        sy = W.w2s[0].float() @ sa.float()
        out.append((routed + h[t].float() + sy).to(BF16))
    return torch.stack(out)


CONFIGS = [(1, "normal"), (32, "normal"), (256, "normal"), (2048, "normal"), (8192, "zipf")]


@pytest.mark.parametrize("T,bias", CONFIGS)
def test_block_parity(gpu, weights, T, bias):
    say(f"block T={T} bias={bias}")
    fe = front_end(T, bias=bias)
    x, r = fe.x.to(gpu), fe.r.to(gpu)
    blk = MoEBlock(T, fe.w_norm.to(gpu), fe.wgt.to(gpu), fe.bias.to(gpu), weights.w13,
                   weights.w2, weights.w13s, weights.w2s)
    out = blk(x, r).clone()
    torch.cuda.synchronize()

    # front end and layout: bitwise against the oracle's exact rule
    y_o, h_o = O.add_rmsnorm_exact(fe.x, fe.r, fe.w_norm)
    assert np.array_equal(u16(blk.h), u16(h_o))
    assert np.array_equal(u16(blk.y), u16(y_o))
    lg_o, w_o, ids_o = O.router_exact(y_o, fe.wgt, fe.bias.numpy())
    assert np.array_equal(blk.logits.cpu().numpy(), lg_o)
    assert np.array_equal(blk.topi.cpu().numpy(), ids_o)
    assert np.array_equal(blk.topw.cpu().numpy(), w_o)
    rs, re_, rn = O.moe_align_block_size(ids_o, blk.bm, 256)
    n = int(rn[0])
    assert int(blk.ntp.item()) == n
    assert np.array_equal(blk.sti.cpu().numpy()[:n], rs)
    assert np.array_equal(blk.eids.cpu().numpy()[: n // blk.bm], re_)

    # block output on sampled tokens vs the fp32 ground truth
    g = torch.Generator().manual_seed(T)
    rows = sorted(set([0, T - 1] + torch.randint(0, T, (6,), generator=g).tolist()))
    ref = rows_reference(blk.y, blk.h, blk.topi.cpu(), blk.topw.cpu(), weights, rows)
    got = out[rows]
    assert torch.isfinite(got.float()).all()
    err = O.rel_err(got.cpu(), ref.cpu())
    say(f"  rel_err {err:.3e} over rows {rows}")
    assert err <= 2e-2
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-2, atol=2e-2)

    # determinism: a second launch gives the same bits
    out2 = blk(x, r)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)


@pytest.mark.parametrize("T", [1, 256])
def test_block_graph_replay(gpu, weights, T):
    say(f"graph replay T={T}")
    fe = front_end(T)
    x, r = fe.x.to(gpu), fe.r.to(gpu)
    blk = MoEBlock(T, fe.w_norm.to(gpu), fe.wgt.to(gpu), fe.bias.to(gpu), weights.w13,
                   weights.w2, weights.w13s, weights.w2s)
    eager = blk(x, r).clone()
    blk.capture(x, r)
    for i in range(3):
        blk.out.zero_()
        blk.ybuf.zero_()
        torch.cuda.synchronize()
        got = blk.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {i} differs from eager"
        _ = (x.float() * 2).sum().item()  # eager work between replays
