"""The whole MoE block on one MI355X with the real 256-expert weight set (19.3 GB)
resident, at the token counts of the benchmark configurations.

* front end (h, y, logits, ids, weights) and the dispatch layout: bit for bit against
  the CPU oracle's exact rule;
* block output on sampled tokens, against references computed in fp32 with torch on the
  GPU (floating-point references of the same op): within rtol 2e-2 / atol 2e-2 of the
  fp32 ground truth, and within the reference's own `rel_err <= 2e-2` gate
  (`glm52/common.py:186-200`) of its framework-faithful path
  (`glm52/bench/bench_layer.py:365-374`);
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
    """Two references for token rows `rows`, computed in fp32 on the GPU.

    exact:    the fp32 ground truth -- fp32 GEMMs, fp32 SwiGLU, fp32 weighted sum and
              fp32 shared expert, one bf16 rounding at the end (`moe_mlp_exact_fp32`,
              `glm52_h200/reference.py:262-291`, with the shared expert likewise unrounded);
    faithful: the framework path the reference gates on -- bf16 w13 linear, bf16 SwiGLU,
              bf16 w2 linear, bf16 routed sum (`glm52/reference.py:134-156`), + h, + the
              shared expert of `glm52/bench/bench_layer.py:369-372`.
    """
    exact, faithful = [], []
    silu = torch.nn.functional.silu
    I = W.w2.shape[2]
    for t in rows:
        yt = y[t].float()
        acc_x = torch.zeros(y.shape[1], dtype=torch.float32, device=y.device)
        acc_f = torch.zeros_like(acc_x)
        for k in range(ids.shape[1]):
            e, wk = int(ids[t, k]), float(tw[t, k])
            hh = W.w13[e].float() @ yt
            acc_x += wk * (W.w2[e].float() @ (silu(hh[:I]) * hh[I:]))
            hb = hh.to(BF16).float()
            a = (silu(hb[:I]) * hb[I:]).to(BF16).float()
            acc_f += (W.w2[e].float() @ a).to(BF16).float() * wk
        sh = W.w13s[0].float() @ yt
        sy_x = W.w2s[0].float() @ (silu(sh[:I]) * sh[I:])
        shb = sh.to(BF16).float()
        sy_f = W.w2s[0].float() @ (silu(shb[:I]) * shb[I:]).to(BF16).float()
        exact.append((acc_x + h[t].float() + sy_x).to(BF16))
        faithful.append((acc_f.to(BF16).float() + h[t].float() + sy_f).to(BF16))
    return torch.stack(exact), torch.stack(faithful)


CONFIGS = [(1, "normal"), (4, "zipf"), (16, "normal"), (32, "normal"), (256, "normal"),
           (2048, "normal"), (8192, "zipf")]


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
    exact, faithful = rows_reference(blk.y, blk.h, blk.topi.cpu(), blk.topw.cpu(), weights,
                                     rows)
    got = out[rows]
    assert torch.isfinite(got.float()).all()
    err_x = O.rel_err(got.cpu(), exact.cpu())
    err_f = O.rel_err(got.cpu(), faithful.cpu())
    say(f"  rel_err vs fp32 ground truth {err_x:.3e}, vs framework path {err_f:.3e}")
    # north-star tolerance against the fp32 ground truth
    torch.testing.assert_close(got.float(), exact.float(), rtol=2e-2, atol=2e-2)
    # the reference's own gate against its framework path (`glm52/common.py:186-200`)
    assert err_f <= 2e-2

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
