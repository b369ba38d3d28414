"""MoE blocks of the path, restated on the CPU in float32 (test infrastructure only).

* ``toy_moe``: BASELINE config 1, a plain bf16 softmax top-2 SwiGLU MoE block, the
  CPU-runnable plumbing case.
* ``fp8_moe_block``: BASELINE config 2, the reference's post-attention half of the
  decoder layer in its W8A8 mode (glm53/gfx950/kernel.py:4199-5187): RMSNorm, bf16
  router GEMV, sigmoid, top-8 + shared expert, per-128 FP8 activation quant, FP8 x FP8
  up/gate with 128 x 128 weight block scales, SiLU, per-128 FP8 quant of the mid
  activation, FP8 down, route weighting, residual add.
* ``mxfp4_moe_block``: BASELINE config 4, the A16W4 expert path (MXFP4 weights,
  bf16 activations; glm53/gfx950/kernel.py:966-970,1068-1085 and
  minimax_m31/a16w4.py:26-92) behind a softmax top-8 router.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import codecs, topk
# one RMSNorm for every phase (glm53/gfx950/kernel.py:1367-1415): the projections'
from .layer import rmsnorm  # noqa: F401


# ---------------------------------------------------------------- config 1
def toy_moe(x, w_router, w_gate, w_up, w_down, top_k: int = 2):
    """Config 1: logits = x W_r^T (bf16 weights, f32 accumulation); softmax top-k
    renormalised (``topk.softmax_topk``); y = sum_k w_k * down(silu(gate x) * up x).
    Shapes: x [S, H] bf16, w_router [E, H], w_gate / w_up [E, I, H], w_down [E, H, I].
    Returns (ids [S, k], weights [S, k], y f32 [S, H])."""
    xf = x.float()
    logits = xf @ w_router.float().T
    ids, wts = topk.softmax_topk(logits, top_k)
    y = torch.zeros(x.shape[0], w_down.shape[1])
    for s in range(x.shape[0]):
        for j in range(top_k):
            e = int(ids[s, j])
            g = w_gate[e].float() @ xf[s]
            u = w_up[e].float() @ xf[s]
            y[s] += wts[s, j] * (w_down[e].float() @ (F.silu(g) * u))
    return ids, wts, y


# ---------------------------------------------------------------- config 2
def fp8_gemv_blocks(xq, xs, wq, ws):
    """Block-scaled FP8 x FP8 GEMV of rows ``xq`` [R, K] (per-128 scales ``xs`` [R, K/128])
    against weight ``wq`` [N, K] (scales ``ws`` [N/128, K/128]): per 128-k block the exact
    FP8 products are summed in f32, then scaled by act scale x weight scale and
    accumulated (glm53/gfx950/kernel.py:847-875 ``unit_f8f8``, :4396-4416)."""
    R, K = xq.shape
    N = wq.shape[0]
    xv = codecs.e4m3_decode(xq).reshape(R, K // 128, 128)
    wv = codecs.e4m3_decode(wq).reshape(N, K // 128, 128)
    part = torch.einsum("rbk,nbk->rnb", xv, wv)  # [R, N, K/128]
    sw = ws.float().repeat_interleave(128, 0)  # [N, K/128]
    return (part * xs.float()[:, None, :] * sw[None]).sum(-1)


def fp8_expert(xq, xs, w13q, s13, w2q, s2, inter: int):
    """One FP8 expert on FP8 rows: (mid f32 [R, I], mid codes, mid scales, down f32 [R, H]
    before route weighting). Gate rows are w13[:I], up rows w13[I:] (SGLang's fused
    w13); mid = silu(gate) * up in f32 (kernel.py:4396-4416), quantised per 128
    (kernel.py:5118-5125) before the down GEMV."""
    gu = fp8_gemv_blocks(xq, xs, w13q, s13)
    g, u = gu[:, :inter], gu[:, inter:]
    mid = g * torch.sigmoid(g) * u
    mq, ms = codecs.fp8_block_quant(mid)
    down = fp8_gemv_blocks(mq, ms, w2q, s2)
    return mid, mq, ms, down


def fp8_router(a, g_post, w_router, eps: float):
    """Post-attention RMSNorm + router GEMV + sigmoid (kernel.py:4199-4330): the router
    reads the normed rows rounded to bf16 (the LDS staging of ``stage_x_rmsnorm``),
    bf16 weights, f32 accumulation. Returns (x f32 normed rows, scores f32 [S, E])."""
    x = rmsnorm(a, g_post, eps)
    logits = codecs.bf16_round(x) @ w_router.float().T
    return x, torch.sigmoid(logits)


def fp8_moe_block(a, g_post, w_router, bias, w13, s13, w2, s2, *, eps=1e-6,
                  top_k=8, inter=512, shared=None, ids=None, weights=None):
    """Config 2. ``a`` [S, H] bf16 residual stream; ``w13`` [E+1, 2I, H] uint8 E4M3,
    ``s13`` [E+1, 2I/128, H/128] f32, ``w2`` [E+1, H, I], ``s2`` [E+1, H/128, I/128];
    the shared expert is id E (SGLang's fused shared-expert id, glm53/check.py:36).

    ``ids`` / ``weights`` override the router's picks (used to evaluate the experts on
    the device's routing when comparing outputs). Returns a dict with scores, ids,
    weights, y (f32 MoE sum) and out (bf16 a + y, kernel.py:5176-5185 without the
    TP reduce)."""
    S = a.shape[0]
    E = w_router.shape[0]
    shared = E if shared is None else shared
    x, scores = fp8_router(a, g_post, w_router, eps)
    r_ids, r_w = topk.router_top8(scores, bias, top_k)
    if ids is None:
        ids, weights = r_ids, r_w
    xq, xs = codecs.fp8_block_quant(x)
    y = torch.zeros(S, a.shape[1])
    # the shared expert (weight 1) and every picked expert once (kernel.py:4345-4350)
    experts = sorted(set(ids.flatten().tolist()) | {shared})
    for e in experts:
        if e == shared:
            rows = torch.arange(S)
            w_rows = torch.ones(S)
        else:
            hit = ids == e
            rows = hit.any(1).nonzero().flatten()
            w_rows = (weights * hit).sum(1)[rows]
        _, _, _, down = fp8_expert(xq[rows], xs[rows], w13[e], s13[e], w2[e], s2[e], inter)
        y[rows] += w_rows[:, None] * down
    out = (a.float() + y).to(torch.bfloat16)
    return dict(scores=scores, ids=r_ids, weights=r_w, y=y, out=out, xq=xq, xs=xs, x=x)


# ---------------------------------------------------------------- config 4
def a16w4_gemv(x_bf16, wq, ws):
    """bf16 rows [R, K] x MXFP4 weight [N, K/2] + E8M0 [N, K/32]: the weight widened
    exactly to bf16 (``cvt_scalef32_pk_bf16_fp4``, common/ops.py:349-363), f32
    accumulation."""
    w = codecs.mxfp4_dequant(wq, ws)
    return x_bf16.float() @ w.T


def mxfp4_moe_block(x, logits, w13, s13, w2, s2, *, top_k=8, inter=384, shared=None,
                    ids=None, weights=None):
    """Config 4. ``x`` [S, H] bf16 activations, ``logits`` [S, E] f32 gate logits;
    ``w13`` [E+1, 2I, H/2] packed E2M1, ``s13`` [E+1, 2I, H/32] E8M0, ``w2`` [E+1, H, I/2],
    ``s2`` [E+1, H, I/32]; shared expert id E, weight 1. mid = bf16(silu(gate) * up)
    (the A16W4 down stage stages mid as bf16, glm53/gfx950/kernel.py:5111-5117);
    y = sum of route weight * down; out = bf16(y)."""
    S = x.shape[0]
    E = logits.shape[1]
    shared = E if shared is None else shared
    r_ids, r_w = topk.softmax_topk(logits, top_k)
    if ids is None:
        ids, weights = r_ids, r_w
    y = torch.zeros(S, x.shape[1])
    experts = sorted(set(ids.flatten().tolist()) | {shared})
    for e in experts:
        if e == shared:
            rows = torch.arange(S)
            w_rows = torch.ones(S)
        else:
            hit = ids == e
            rows = hit.any(1).nonzero().flatten()
            w_rows = (weights * hit).sum(1)[rows]
        gu = a16w4_gemv(x[rows], w13[e], s13[e])
        g, u = gu[:, :inter], gu[:, inter:]
        mid = codecs.bf16_round(g * torch.sigmoid(g) * u)
        down = a16w4_gemv(mid, w2[e], s2[e])
        y[rows] += w_rows[:, None] * down
    return dict(ids=r_ids, weights=r_w, y=y, out=y.to(torch.bfloat16))
