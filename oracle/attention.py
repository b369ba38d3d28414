"""Sparse-attention phase of the path, restated on the CPU (test infrastructure only).

the FP4 indexer's scores over every cached key of a row, the exact
top-2048 of those scores, and sparse MLA decode attention over the selected tokens.

Cache layouts (64-token pages; a slot is ``page * 64 + offset``):

* FP4 index keys, SGLang's DSA index plane (deepseek_v41/gfx950/indexer/score_fp4.py:8-12,
  deepseek_v4/gfx950/runner.py:336-347): ``payload`` uint8 [pages, 4 (32-dim chunk),
  64 (key), 16] two E2M1 codes a byte (low nibble = even dim), ``kscale`` uint8
  [pages, 4, 64] E8M0 with key ``t``'s byte at ``(t % 16) * 4 + t // 16``.
* MLA latent cache: ``kv`` uint8 [slots, 576] E4M3 (512 latent dims then 64 RoPE
  dims, the 576-B row of glm53/gfx950/runner.py:90-96) and ``kv_scale`` f32 [slots],
  one dequantisation scale a token.
"""

from __future__ import annotations

import numpy as np
import torch

from . import codecs, topk

PAGE = 64
KV_LORA, PE_DIM = 512, 64
KV_ROW = KV_LORA + PE_DIM
TOPK = 2048
SOFTMAX_SCALE = (128 + 64) ** -0.5  # (nope_dim + pe_dim)^-1/2, glm53/gfx950/config.py:171-173


def scale_byte(t):
    """Position of key ``t``'s E8M0 byte in a chunk's 64 scale bytes
    (test/kernels/test_deepseek_v41_k2i.py:158, ``(slot % 16) * 4 + slot // 16``)."""
    return (t % 16) * 4 + t // 16


def index_keys(payload, kscale, page_table_row, n):
    """The first ``n`` keys of one request as f32 [n, 128] (E2M1 x E8M0 per 32 dims)."""
    pos = torch.arange(n)
    page = page_table_row[pos // PAGE].long()
    t = pos % PAGE
    raw = payload[page, :, t, :]  # [n, 4, 16]
    vals = codecs.e2m1_decode(raw)  # [n, 4, 32]
    sc = kscale[page[:, None], torch.arange(4)[None], scale_byte(t)[:, None]]  # [n, 4]
    return (vals * codecs.e8m0_decode(sc)[..., None]).reshape(n, 128)


def index_query(iq, iqs):
    """One row's FP4 index query: ``iq`` uint8 [heads, 64] packed E2M1, ``iqs`` uint8
    [heads, 4] E8M0 (one a 32-dim chunk) -> f32 [heads, 128]."""
    v = codecs.e2m1_decode(iq).reshape(iq.shape[0], 4, 32)
    return (v * codecs.e8m0_decode(iqs)[..., None]).reshape(iq.shape[0], 128)


def index_scores(iq, iqs, iw, payload, kscale, page_table, seq_lens, max_keys):
    """Scores [S, max_keys] f32 (0 past a row's keys):
    score[t] = sum_h w_h * relu(q_h . k_t) over the 128-dim FP4 vectors
    (test/kernels/test_deepseek_v41_k2i.py:149-167 ``ref_logits``;
    deepseek_v4/gfx950/kernels/stages/indexer.py:460-602 ``i_score``)."""
    S = iq.shape[0]
    out = torch.zeros(S, max_keys)
    for s in range(S):
        n = int(seq_lens[s])
        k = index_keys(payload, kscale, page_table[s], n)
        q = index_query(iq[s], iqs[s])
        dots = q @ k.T  # [heads, n]
        out[s, :n] = (iw[s].float()[:, None] * dots.clamp_min(0)).sum(0)
    return out


def index_scores_fp64(iq, iqs, iw, payload, kscale, page_table_row, n):
    """One row's scores in float64 (the closed form the f32 path is pinned to)."""
    k = index_keys(payload, kscale, page_table_row, n).double()
    q = index_query(iq, iqs).double()
    return (iw.double()[:, None] * (q @ k.T).clamp_min(0)).sum(0)


def select_topk(scores, seq_lens, page_table, k=TOPK):
    """Exact top-k slots of every row: positions by (score desc, position asc), each
    mapped to its slot ``page_table[p // 64] * 64 + p % 64`` (glm53/gfx950/kernel.py:
    3341-3346), in ascending position order, -1 past the row's count
    (glm53/check.py:100-117). Returns int32 [S, k]."""
    S = scores.shape[0]
    out = np.full((S, k), -1, dtype=np.int32)
    for s in range(S):
        n = int(seq_lens[s])
        pos = topk.exact_topk(scores[s, :n], k)
        pt = page_table[s].numpy().astype(np.int64)
        out[s, : pos.shape[0]] = pt[pos // PAGE] * PAGE + pos % PAGE
    return torch.from_numpy(out)


def kv_rows(kv, kv_scale, slots):
    """Dequantised f32 [n, 576] cache rows at ``slots`` (``kv_scale`` None: raw E4M3
    rows, scale 1)."""
    rows = codecs.e4m3_decode(kv[slots.long()])
    return rows if kv_scale is None else rows * kv_scale[slots.long()].float()[:, None]


def sparse_mla(q, kv, kv_scale, sel, scale=SOFTMAX_SCALE):
    """Sparse MLA decode over the selected slots (glm53/gfx950/kernel.py:3638-4123):
    s_j = (q_lat . c_j + q_pe . k_pe_j) * scale, p = softmax_j(s), o_lat = sum_j p_j c_j.
    ``q`` [S, heads, 576] bf16 (absorbed latent query then RoPE query), ``sel`` int32
    [S, k] slots (-1 = unused). Returns o_lat f32 [S, heads, 512]."""
    S, H, _ = q.shape
    out = torch.zeros(S, H, KV_LORA)
    for s in range(S):
        slots = sel[s][sel[s] >= 0]
        if slots.numel() == 0:
            continue
        rows = kv_rows(kv, kv_scale, slots)  # [n, 576]
        logits = (q[s].float() @ rows.T) * scale  # [H, n]
        p = torch.softmax(logits, -1)
        out[s] = p @ rows[:, :KV_LORA]
    return out


def sparse_mla_fp64(q, rows, scale=SOFTMAX_SCALE):
    """Dense softmax attention in float64 over explicit rows [n, 576] (the brute-force
    closed form ``sparse_mla`` is pinned to)."""
    lg = (q.double() @ rows.double().T) * scale
    return torch.softmax(lg, -1) @ rows.double()[:, :KV_LORA]
