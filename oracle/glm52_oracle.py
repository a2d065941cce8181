"""CPU oracle for the GLM-5.2 MoE block -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import
this module, and only as the checker (or the timed CPU baseline); the product path in
`fusion_amd/` never calls it and has no CPU fallback.

It restates the reference's fp32/bf16 path, `glm52/reference.py:22-188` (plus the shared
expert of `glm52_h200/reference.py:294-311` and the block composition of
`glm52/bench/bench_layer.py:354-374`), on the CPU with torch and numpy, keeping the
reference's op order and every bf16 rounding point.

One deliberate refinement, applied identically on the device: routing.  The reference's
`F.linear` sums 6144 fp32 products in an order set by the BLAS, so the 8th/9th expert of
a near-tied token depends on that order.  `router_logits_exact` fixes the logits to an
order-independent rule (exact bf16 products, fp64 sum, one rounding to fp32) and
`router_select` evaluates the sigmoid in fp64 with one rounding, then selects with a
lower-index-first tie rule (the `tl.argmax` rule of `glm52/kernels/norm_router.py:232-238`).
`router_reference` keeps the reference's own torch arithmetic for pinning.

Parity status of each function (how it is pinned, see tests/test_oracle.py):
  rmsnorm / add_rmsnorm      golden vectors from glm52/reference.py at T=32; closed forms
  add_rmsnorm_exact          h bitwise and y within 1 bf16 ulp of the golden vectors; fp64
                             closed form of the statistic; special cases
  silu_and_mul               golden vectors; closed form
  router_logits_exact        fp64 matmul with float128-free brute force on small shapes;
                             golden logits within 2 fp32 ulp
  router_select              golden ids/weights at T=32; brute-force sort; invariants
  moe_align_block_size       golden layouts (BM=16, 64); brute force; invariants
  moe_mlp / shared_expert    golden tiny-shape outputs; fp64 textbook GEMM
  block_reference            composition of the above (bench_layer.py:365-374)
  moe_sum / merge_resadd     closed forms (weighted sums) on small shapes
  oproj_gemm / oproj_cast    one-hot A (exact rows of B, with and without the residual);
                             fp64 textbook GEMM on small shapes
  down_token_major           single expert with w = 1 equals the fp64 GEMM row; linearity
                             in the weights; closed forms on one-hot rows; within one
                             bf16 rounding per expert of moe_sum over the unfused rows
  down_merge_atomic          top_k = 1 is one rounding of seed + bf16(y) (closed form);
                             integer-valued sums are exact in any order; within one
                             rounding per add of down_token_major
  rstd_exact                 exact rational sum of squares; constant rows (closed form);
                             exact halving under h -> 2h at eps = 0; rmsnorm_exact's y
  fold_weight                power-of-two w (exact), w = 1 (identity), axis choice
  prenorm_router /           one-hot h (closed form w[k] * b[k] * c * rstd); w = 1 reduces
  prenorm_gateup_rows        to the plain logits / rows times rstd; the folding identity
                             against norm -> consumer within the reference's 5e-2 bar
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
EPS = 1e-5
SCALE = 2.5
TOPK = 8


# --------------------------------------------------------------------------------------
# norms / activations
# --------------------------------------------------------------------------------------
def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """`glm52/reference.py:22-25`: bf16(fp32(bf16(x * rstd)) * w)."""
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * rstd).to(x.dtype) * w


def add_rmsnorm(x, residual, w, eps: float = EPS):
    """`glm52/reference.py:28-33`: returns (normed, new_residual)."""
    h = (x.float() + residual.float()).to(x.dtype)
    return rmsnorm(h, w, eps), h


def _bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 -> fp32, round to nearest even (NaN not expected here)."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def add_rmsnorm_exact(x, residual, w, eps: float = EPS):
    """`add_rmsnorm` under the order-independent statistic the device uses.

    h is the same (one fp32 add, RNE to bf16).  The sum of squares is exact per term
    (a bf16 square fits fp32) and summed in fp64; rstd = fp32(1 / sqrt(ss / N + eps)) in
    fp64 with one rounding, eps taken as the fp32 value the kernels receive; then
    y = bf16(fp32(bf16(h * rstd)) * w) with fp32 products, as `glm52/reference.py:25`.
    Returns (y, h) as bf16 torch tensors; `y` equals `add_rmsnorm`'s within 1 bf16 ulp.
    """
    h = (x.float() + residual.float()).to(torch.bfloat16)
    return rmsnorm_exact(h, w, eps), h


def rstd_exact(h, eps: float = EPS) -> np.ndarray:
    """The RMSNorm statistic alone, [T] fp32: fp32(1 / sqrt(sum_k h[t, k]^2 / N + eps)), the
    exact squares summed in fp64 and rounded once.  The reference's rstd-only kernel
    (`glm52/kernels/lazy_prenorm.py:347-368`) evaluates the same formula in fp32; the two
    differ by at most an fp32 ulp or so."""
    hf = h.float().numpy().astype(np.float64)
    ss = (hf ** 2).sum(-1)
    return (1.0 / np.sqrt(ss / hf.shape[-1] + np.float64(np.float32(eps)))).astype(np.float32)


def rmsnorm_exact(h, w, eps: float = EPS):
    hf = h.float().numpy()
    rstd = rstd_exact(h, eps)[..., None]
    y = _bf16_round((hf * rstd).astype(np.float32)) * w.float().numpy()
    return torch.from_numpy(y.astype(np.float32)).to(torch.bfloat16)


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """`glm52/reference.py:36-40`; x = [gate | up] along the last axis."""
    d = x.shape[-1] // 2
    gate, up = x[..., :d], x[..., d:]
    return (F.silu(gate.float()) * up.float()).to(x.dtype)


# --------------------------------------------------------------------------------------
# router
# --------------------------------------------------------------------------------------
def router_logits_exact(y: torch.Tensor, wgt_he: torch.Tensor) -> np.ndarray:
    """Logits under the order-independent rule: fp64(y) @ fp64(Wg), rounded once to fp32.

    `y` is [T, H] bf16, `wgt_he` is the kernel layout [H, E] (`wgt_from_gate`,
    `glm52/kernels/norm_router.py:251-255`).  bf16 x bf16 products are exact in fp64 and
    the fp64 sum's error is far below half an fp32 ulp, so any summation order rounds to
    the same fp32 value (up to ties at the 2^-29 level).
    """
    yd = y.float().numpy().astype(np.float64)
    wd = wgt_he.float().numpy().astype(np.float64)
    return (yd @ wd).astype(np.float32)


def sigmoid_exact(logits: np.ndarray) -> np.ndarray:
    """fp32(1 / (1 + exp(-x))) evaluated in fp64, one rounding."""
    lg = np.asarray(logits, dtype=np.float32).astype(np.float64)
    return (1.0 / (1.0 + np.exp(-lg))).astype(np.float32)


def router_select(logits: np.ndarray, bias: np.ndarray | None, topk: int = TOPK,
                  scale: float = SCALE, norm_prob: bool = True):
    """Top-k selection of `glm52/reference.py:62-79` under the exact rule.

    choice = fp32(s + bias); ids sorted by descending choice, lower index first on ties;
    weights = fp32(fp32(s[ids] / max(sum, 1e-20)) * scale) with the 8 scores summed in
    selection order.  Returns (topk_weights fp32 [T, k], topk_ids int32 [T, k], scores).
    """
    s = sigmoid_exact(logits)
    choice = s if bias is None else (s + np.asarray(bias, dtype=np.float32)).astype(np.float32)
    T, E = choice.shape
    # lexsort: last key is primary -> descending choice, then ascending index
    idx = np.broadcast_to(np.arange(E), (T, E))
    order = np.lexsort((idx, -choice.astype(np.float64)), axis=-1)
    ids = order[:, :topk].astype(np.int32)
    sv = np.take_along_axis(s, ids, axis=1)
    tot = np.zeros(T, dtype=np.float32)
    for k in range(topk):
        tot = (tot + sv[:, k]).astype(np.float32)
    if norm_prob:
        denom = np.maximum(tot, np.float32(1e-20)).astype(np.float32)
        w = (sv / denom[:, None]).astype(np.float32)
        w = (w * np.float32(scale)).astype(np.float32)
    else:
        w = (sv * np.float32(scale)).astype(np.float32)
    return w, ids, s


def router_exact(y: torch.Tensor, wgt_he: torch.Tensor, bias=None, topk: int = TOPK,
                 scale: float = SCALE):
    """Router under the device rule. Returns (logits, weights, ids) as numpy."""
    lg = router_logits_exact(y, wgt_he)
    w, ids, _ = router_select(lg, None if bias is None else np.asarray(bias), topk, scale)
    return lg, w, ids


def router_reference(x: torch.Tensor, gate_w: torch.Tensor, correction_bias=None,
                     topk: int = TOPK, routed_scaling_factor: float = SCALE):
    """`glm52/reference.py:46-79` with n_group = 1 (torch arithmetic, as the reference)."""
    logits = F.linear(x.float(), gate_w.float())
    scores = logits.sigmoid()
    choice = scores if correction_bias is None else scores + correction_bias
    topk_ids = choice.topk(topk, dim=-1).indices
    topk_weights = scores.gather(1, topk_ids)
    topk_weights = topk_weights / topk_weights.sum(-1, keepdim=True).clamp_min(1e-20)
    topk_weights = topk_weights * routed_scaling_factor
    return logits, topk_weights.float(), topk_ids.int()


# --------------------------------------------------------------------------------------
# dispatch layout
# --------------------------------------------------------------------------------------
def moe_align_block_size(topk_ids, block_m: int, num_experts: int):
    """`glm52/reference.py:85-128` in numpy: (sorted_token_ids, expert_ids, ntp)."""
    flat = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    numel = flat.size
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=num_experts)
    padded = ((counts + block_m - 1) // block_m) * block_m
    total = int(padded.sum())
    sorted_ids = np.full(total, numel, dtype=np.int32)
    expert_ids = np.zeros(total // block_m, dtype=np.int32)
    starts = np.concatenate([[0], np.cumsum(padded)[:-1]])
    src = 0
    for e in range(num_experts):
        c, s = int(counts[e]), int(starts[e])
        if c:
            sorted_ids[s:s + c] = order[src:src + c]
            src += c
        nblk = int(padded[e]) // block_m
        if nblk:
            expert_ids[s // block_m: s // block_m + nblk] = e
    return sorted_ids, expert_ids, np.array([total], dtype=np.int32)


# --------------------------------------------------------------------------------------
# experts
# --------------------------------------------------------------------------------------
def moe_mlp(x, w13, w2, topk_weights, topk_ids) -> torch.Tensor:
    """`glm52/reference.py:134-156`: per expert bf16 linear, bf16 SwiGLU, bf16 linear,
    fp32 weighted index_add_, bf16 result."""
    T, H = x.shape
    out = torch.zeros(T, H, dtype=torch.float32)
    for e in range(w13.shape[0]):
        sel = (topk_ids == e).nonzero(as_tuple=False)
        if sel.numel() == 0:
            continue
        rows, ks = sel[:, 0], sel[:, 1]
        h = F.linear(x[rows], w13[e])
        a = silu_and_mul(h)
        y = F.linear(a, w2[e]).float()
        out.index_add_(0, rows, y * topk_weights[rows, ks].unsqueeze(1))
    return out.to(x.dtype)


def moe_mlp_rows(x, w13, w2, topk_weights, topk_ids, rows) -> torch.Tensor:
    """`moe_mlp` restricted to the token rows `rows` (fp32 [len(rows), H] before the
    final bf16 round), for sampled checks at full size; same per-row arithmetic."""
    rows = torch.as_tensor(rows)
    xs, ids, ws = x[rows], topk_ids[rows], topk_weights[rows]
    out = torch.zeros(len(rows), x.shape[1], dtype=torch.float32)
    for e in torch.unique(ids).tolist():
        sel = (ids == e).nonzero(as_tuple=False)
        r, ks = sel[:, 0], sel[:, 1]
        h = F.linear(xs[r], w13[e])
        a = silu_and_mul(h)
        y = F.linear(a, w2[e]).float()
        out.index_add_(0, r, y * ws[r, ks].unsqueeze(1))
    return out


def shared_expert(x, w13s, w2s) -> torch.Tensor:
    """`glm52_h200/reference.py:294-311` / `glm52/bench/bench_layer.py:369-372`: fp32
    linears around a bf16-rounded SwiGLU; returns fp32."""
    w13s = w13s[0] if w13s.dim() == 3 else w13s
    w2s = w2s[0] if w2s.dim() == 3 else w2s
    h = F.linear(x.float(), w13s.float())
    a = silu_and_mul(h.to(x.dtype))
    return F.linear(a.float(), w2s.float())


def block_reference(h1, x2, w13, w2, w13s, w2s, topk_weights, topk_ids) -> torch.Tensor:
    """`glm52/bench/bench_layer.py:365-374`: bf16(fp32 routed + fp32 h1 + fp32 shared)."""
    routed = moe_mlp(x2, w13, w2, topk_weights, topk_ids).float()
    s_y = shared_expert(x2, w13s, w2s)
    return (routed + h1.float() + s_y).to(BF16)


# --------------------------------------------------------------------------------------
# merges
# --------------------------------------------------------------------------------------
def expert_merge(per_expert_out, topk_weights) -> torch.Tensor:
    """`glm52/reference.py:159-188` (one-shot form; bit-identical to the chunked one)."""
    return (per_expert_out.float() * topk_weights.unsqueeze(-1)).sum(1).to(per_expert_out.dtype)


def moe_sum(y3, residual=None) -> torch.Tensor:
    """`glm52/kernels/moe_down_merge.py:300-349`: bf16(sum_k fp32 Y[:, k] (+ fp32 res)),
    summed in k order."""
    acc = torch.zeros(y3.shape[0], y3.shape[2], dtype=torch.float32)
    for k in range(y3.shape[1]):
        acc = acc + y3[:, k].float()
    if residual is not None:
        acc = acc + residual.float()
    return acc.to(y3.dtype)


def merge_resadd(y3, wt, res, round_mid: bool = True) -> torch.Tensor:
    """`glm52/kernels/merge_resadd.py:3-29`: m = sum_k w_k * Y_k in fp32 (k order),
    optionally rounded to bf16, then bf16(m + res)."""
    acc = torch.zeros(y3.shape[0], y3.shape[2], dtype=torch.float32)
    for k in range(y3.shape[1]):
        acc = acc + y3[:, k].float() * wt[:, k:k + 1].float()
    if round_mid:
        acc = acc.to(y3.dtype).float()
    return (acc + res.float()).to(y3.dtype)


# --------------------------------------------------------------------------------------
# token-major down GEMV (fusion #8(b) / #9(b))
# --------------------------------------------------------------------------------------
def down_token_major(a, w2, topk_weights, topk_ids, residual=None, a_shared=None,
                     w2_shared=None) -> torch.Tensor:
    """`moe_down_token_major_kernel` (`glm52/kernels/moe_down_merge.py:165-293`): for each
    token t, sum_k w[t, k] * (a[t * top_k + k] @ w2[ids[t, k]]^T) accumulated without
    rounding (here fp64, rounded once to fp32), plus the shared expert's product with
    weight 1 if given, then + fp32 residual and one rounding to bf16.  [T, H] bf16."""
    T, k = topk_ids.shape
    acc = torch.zeros(T, w2.shape[1], dtype=torch.float64)
    ad = a.double()
    for t in range(T):
        for j in range(k):
            e = int(topk_ids[t, j])
            acc[t] += float(topk_weights[t, j]) * (w2[e].double() @ ad[t * k + j])
        if w2_shared is not None:
            acc[t] += w2_shared.reshape(w2.shape[1], -1).double() @ a_shared[t].double()
    v = acc.float()
    if residual is not None:
        v = v + residual.float()
    return v.to(BF16)


def down_merge_atomic(a, w2, topk_weights, topk_ids, seed) -> torch.Tensor:
    """`moe_down_kernel` with FUSE_MERGE (`glm52/kernels/moe_down_merge.py:154-166`): each
    routed row's result y = bf16(w * fp32(a[f] @ w2[e]^T)) is added to the seeded output
    row f // top_k, every add rounded to bf16 (the bf16 `tl.atomic_add`).  The device adds
    in whatever order the atomics land; this restatement adds in k order, which fixes the
    value whenever the sums are exact (or top_k = 1).  [T, H] bf16."""
    T, k = topk_ids.shape
    out = seed.clone().to(BF16)
    for t in range(T):
        for j in range(k):
            e = int(topk_ids[t, j])
            acc = (w2[e].double() @ a[t * k + j].double()).float()
            y = (acc * float(topk_weights[t, j])).to(BF16)
            out[t] = (out[t].float() + y.float()).to(BF16)
    return out


# --------------------------------------------------------------------------------------
# o_proj + ResAdd1 (upstream of the block)
# --------------------------------------------------------------------------------------
def oproj_gemm(a, b, r=None, out_dtype=BF16) -> torch.Tensor:
    """`oproj_gemm_kernel` (`glm52/kernels/oproj_resadd.py:32-116`): A [M, K] @ B [K, N]
    accumulated in fp32 (here: fp64, rounded once to fp32), + fp32 r when the residual is
    fused, one rounding to the output dtype."""
    acc = (a.double() @ b.double()).float()
    if r is not None:
        acc = acc + r.float()
    return acc.to(out_dtype)


def oproj_cast(c, r=None) -> torch.Tensor:
    """`epilogue_kernel` (`glm52/kernels/oproj_resadd.py:119-136`): bf16(fp32 c (+ fp32 r))."""
    v = c.float()
    if r is not None:
        v = v + r.float()
    return v.to(BF16)


# --------------------------------------------------------------------------------------
# half-fused pre-norm (lazy_prenorm): the norm weight folded into the consumer weight
# --------------------------------------------------------------------------------------
def fold_weight(b, w, k_axis: int) -> torch.Tensor:
    """`fold_weight_rowmajor` / `fold_weight_nk` (`glm52/kernels/lazy_prenorm.py:75-85`):
    bf16(fp32 b * fp32 w[k]) along the contraction axis `k_axis` of b."""
    shape = [1] * b.dim()
    shape[k_axis] = -1
    return (b.float() * w.float().reshape(shape)).to(b.dtype)


def prenorm_router(h, b_fold, rstd) -> np.ndarray:
    """`router_gemm_kernel` with USE_RSTD (`lazy_prenorm.py:229-330`): fp32 logits of
    h @ b_fold under the order-independent rule, then one fp32 multiply by rstd[t]."""
    lg = router_logits_exact(h, b_fold)
    return (lg * np.asarray(rstd, dtype=np.float32)[:, None]).astype(np.float32)


def prenorm_gateup_rows(h, w_fold, rstd, topk_ids) -> torch.Tensor:
    """`moe_gateup_prenorm_kernel` with USE_RSTD (`lazy_prenorm.py:89-226`), no activation:
    slot f = t * top_k + j holds bf16(fp32(h[t] @ w_fold[topk_ids[t, j]]^T) * rstd[t]),
    the accumulator in fp64 rounded once to fp32.  Returns [T * top_k, N] bf16."""
    T, k = topk_ids.shape
    hd = h.double()
    out = torch.empty(T * k, w_fold.shape[1], dtype=torch.float32)
    r = torch.from_numpy(np.asarray(rstd, dtype=np.float32))
    for t in range(T):
        for j in range(k):
            acc = (w_fold[int(topk_ids[t, j])].double() @ hd[t]).float()
            out[t * k + j] = acc * r[t]
    return out.to(BF16)


def rel_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    """`glm52/common.py:186-190`: max-abs error over the reference's max-abs."""
    got32, ref32 = got.float(), ref.float()
    denom = ref32.abs().max().clamp_min(1e-6)
    return ((got32 - ref32).abs().max() / denom).item()
