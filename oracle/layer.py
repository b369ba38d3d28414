"""Projection phases of the decoder layer, restated on the CPU in float32 (test
infrastructure only: imported by tests/, smoke() and bench.py's cpu_baseline leg).

BASELINE config 5 around the attention (oracle.attention) and MoE (oracle.moe)
phases, one GPU's TP=4 share of a DeepSeek-V3.2-shaped layer with an FP4 indexer:

* ``front``: input RMSNorm, the fused q_a | kv_a projection and the indexer's key and
  head-weight projections off the normed rows, q_a RMSNorm, q_b (+RoPE on the 64 pe
  dims of each head), the absorbed query q_lat = W_UK^T q_nope, the KV RMSNorm +
  k_pe RoPE + per-token FP8 row written to the MLA cache, the index key
  (LayerNorm + RoPE + Hadamard + FP4) written to the index plane, and the index query
  (W_iq q_an + RoPE + Hadamard + FP4) and head weights handed to the attention phase.
* ``back``: o = W_UV o_lat per head, then a = h + W_o o (the TP all-reduce becomes a
  local residual add).

Weights are 128 x 128 block-scaled E4M3 unless noted; GEMVs widen FP8 exactly and
accumulate in f32 against bf16 activations (glm53/gfx950/kernel.py:30-37, "FP8 is
widened exactly to bf16 ... the math is exact block-scaled FP8 on bf16 activations").
"""

from __future__ import annotations

import torch

from . import codecs
from .attention import PAGE, scale_byte

HIDDEN, Q_LORA, KV_LORA, PE_DIM = 7168, 1536, 512, 64
HEADS, NOPE_DIM, V_DIM = 32, 128, 128
QK_DIM = NOPE_DIM + PE_DIM
INDEX_HEADS, INDEX_DIM = 64, 128
EPS = 1e-6  # RMSNorm eps (DeepSeek-V3.2's; glm53/gfx950/config.py:276 uses 1e-5 for GLM)
INDEX_LN_EPS = 1e-6  # glm53/gfx950/kernel.py:2125-2127
FP8_MAX = 448.0
# index head-weight scale IHD^-1/2 * IH^-1/2 (deepseek_v4/gfx950/kernels/stages/indexer.py:403-405)
INDEX_W_SCALE = float(INDEX_DIM) ** -0.5 * float(INDEX_HEADS) ** -0.5


def block_dequant(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """[N, K] E4M3 with f32 [ceil(N/128), K/128] block scales -> f32 [N, K]; the last
    row block may be partial (q_a | kv_a has 2112 rows under 17 scale rows,
    with a ``[17, 56]`` scale grid; glm53/gfx950/kernel.py:5-45)."""
    n, k = codes.shape
    s = scales.float().repeat_interleave(128, 0)[:n].repeat_interleave(128, 1)[:, :k]
    return codecs.e4m3_decode(codes) * s


def gemv(x_bf16: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Rows [R, K] (bf16 values) times a block-scaled FP8 weight [N, K] -> f32 [R, N]."""
    return x_bf16.float() @ block_dequant(codes, scales).T


def rmsnorm(x: torch.Tensor, gamma: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """f32 x * rsqrt(mean(x^2) + eps) * gamma (glm53/gfx950/kernel.py:1367-1398)."""
    x = x.float()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * gamma.float()


def layernorm(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = INDEX_LN_EPS):
    """(x - mean) * rsqrt(var + eps) * gamma + beta, biased variance
    (glm53/gfx950/kernel.py:2121-2133)."""
    x = x.float()
    mean = x.mean(-1, keepdim=True)
    c = x - mean
    return c * torch.rsqrt(c.pow(2).mean(-1, keepdim=True) + eps) * gamma.float() + beta.float()


def rope_tables(max_pos: int, dim: int = PE_DIM, theta: float = 10000.0):
    """cos / sin f32 [max_pos, dim/2]: angle = pos * theta^(-2i/dim)."""
    inv = theta ** (-torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None]
    return torch.cos(ang).float(), torch.sin(ang).float()


def rope_pairs(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved RoPE over the last dim: pair (2i, 2i+1) -> (x0 c - x1 s, x0 s + x1 c)
    with c, s = cos[i], sin[i] (glm53/gfx950/kernel.py:2072, 2254-2257). ``cos`` /
    ``sin`` broadcast against x[..., ::2]."""
    x0, x1 = x[..., 0::2].float(), x[..., 1::2].float()
    out = torch.empty(x.shape, dtype=torch.float32)
    out[..., 0::2] = x0 * cos - x1 * sin
    out[..., 1::2] = x0 * sin + x1 * cos
    return out


def fwht(x: torch.Tensor) -> torch.Tensor:
    """Walsh-Hadamard transform over the last dim (a power of two) by butterflies in
    Sylvester order, scaled by n^-1/2 (deepseek_v4/gfx950/kernels/stages/indexer.py:127-141
    ``had_pair``: at stride 2^h the element with bit h clear becomes a + b, its partner
    a - b)."""
    y = x.float().clone()
    n = y.shape[-1]
    h = 1
    while h < n:
        v = y.reshape(*y.shape[:-1], n // (2 * h), 2, h)
        a, b = v[..., 0, :].clone(), v[..., 1, :].clone()
        v[..., 0, :], v[..., 1, :] = a + b, a - b
        y = v.reshape(y.shape)
        h *= 2
    return y * (float(n) ** -0.5)


def fp8_row_quant_pow2(row: torch.Tensor, scaled: bool = True):
    """Per-token E4M3 with a power-of-two scale: scale = 2^ceil(log2(max(amax, 1e-4)/448))
    (the index cache's UE8M0 rule, glm53/gfx950/kernel.py:2137-2151), codes =
    E4M3(v / scale) (exact division by a power of two). Returns (codes uint8 [..., n],
    scale f32 [...]). ``scaled=False``: SGLang's raw E4M3 row (the reference's
    scale-less 576-B row, glm53/gfx950/runner.py:90-96): scale 1, values clamped to
    [-448, 448]."""
    if not scaled:
        codes = codecs.e4m3_encode(row.float().clamp(-FP8_MAX, FP8_MAX))
        return codes, torch.ones(row.shape[:-1], dtype=torch.float32)
    amax = row.float().abs().amax(-1)
    e = codecs.code_ceil(torch.clamp(amax, min=1e-4) / FP8_MAX)
    scale = torch.exp2(e.double() - 127).float()
    codes = codecs.e4m3_encode(row.float() / scale[..., None])
    return codes, scale


def slot_of(page_table: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """Cache slot of position ``pos`` of each row: page_table[s, pos / 64] * 64 + pos % 64."""
    s = torch.arange(pos.shape[0])
    return page_table[s, (pos // PAGE).long()].long() * PAGE + (pos % PAGE).long()


def index_fp4(v: torch.Tensor):
    """An index vector [..., 128] after its projection, norm and RoPE: bf16, Hadamard,
    bf16, FP4 over 32-dim blocks with power-of-two scales
    (deepseek_v4/gfx950/kernels/stages/indexer.py:240-246, 335-340 ``had_pair`` +
    ``fp4_block``). Returns (codes uint8 [..., 128], e8m0 uint8 [..., 4], dequantised
    f32, the rotated bf16 vector before FP4)."""
    h = codecs.bf16_round(fwht(codecs.bf16_round(v)))
    codes, e8, deq = codecs.fp4_block_quant(h)
    return codes, e8, deq, h


def index_key(ik: torch.Tensor, g_ik, b_ik, c, s):
    """The indexer's key of rows ``ik`` [S, 128] (the f32 projection) at RoPE angles
    ``c``/``s`` [S, 32]: LayerNorm, RoPE on dims [0, 64), then ``index_fp4``
    (glm53/gfx950/kernel.py:2103-2133)."""
    kn = layernorm(ik, g_ik, b_ik)
    kn = torch.cat([rope_pairs(kn[:, :PE_DIM], c, s), kn[:, PE_DIM:]], -1)
    return index_fp4(kn)


def index_query(q_an: torch.Tensor, w_iq, s_iq, c, s):
    """The indexer's query of rows ``q_an`` [S, 1536] (bf16 values) at RoPE angles
    ``c``/``s`` [S, 32]: W_iq q_an (row h*128 + d is head h's dim d) rounded to bf16,
    RoPE on each head's dims [0, 64) (the dims the key rotates), then ``index_fp4``
    (deepseek_v4/gfx950/kernels/stages/indexer.py:271-338; glm53/gfx950/kernel.py:2121-2133).
    Returns ``index_fp4``'s tuple over [S, 64 heads, 128]."""
    S = q_an.shape[0]
    raw = codecs.bf16_round(gemv(q_an, w_iq, s_iq)).reshape(S, INDEX_HEADS, INDEX_DIM)
    rot = torch.cat([rope_pairs(raw[..., :PE_DIM], c[:, None], s[:, None]), raw[..., PE_DIM:]], -1)
    return index_fp4(rot)


def front(h, pos, page_table, w, cos, sin, kv_scaled: bool = True):
    """The front of the layer for rows ``h`` [S, 7168] bf16 at positions ``pos`` [S]
    (each row's new token; its slot from ``page_table``). ``w``: dict of row-major
    weights (see ``sgl_amd_mono_amd.layer.LayerWeights``). Returns a dict:

    q [S, 32, 576] bf16 (q_lat | q_pe), iq [S, 64, 64] uint8 (packed E2M1),
    iqs [S, 64, 4] uint8, iw [S, 64] bf16, and the cache rows this step writes:
    slot [S], kv [S, 576] uint8 E4M3 + kv_scale [S] f32, ikv [S, 4, 16] uint8 + iks
    [S, 4] uint8; plus intermediates (x, q_a, kv_a, ik, q_an, q_nope, q_pe, q_lat, and
    the index query / key before FP4, iq_h [S, 64, 128] and ik_h [S, 128]).
    ``kv_scaled=False`` writes raw E4M3 MLA rows (scale 1)."""
    S = h.shape[0]
    pos = pos.long()
    c, s_ = cos[pos], sin[pos]  # [S, 32]
    x = codecs.bf16_round(rmsnorm(h, w["g_in"]))  # LDS bf16 staging, kernel.py:1367-1398
    qkv = gemv(x, w["w_qkv"], w["s_qkv"])
    q_a, kv_a = qkv[:, :Q_LORA], qkv[:, Q_LORA:]
    ik = gemv(x, w["w_ik"], w["s_ik"])
    iw_raw = x @ w["w_iw"].float().T

    # q path: q_a RMSNorm -> q_b -> nope / RoPE'd pe (kernel.py:1978-2003, 2183-2260)
    q_an = codecs.bf16_round(rmsnorm(q_a, w["g_q"]))
    qb = gemv(q_an, w["w_qb"], w["s_qb"]).reshape(S, HEADS, QK_DIM)
    q_nope = codecs.bf16_round(qb[..., :NOPE_DIM])
    q_pe = codecs.bf16_round(rope_pairs(qb[..., NOPE_DIM:], c[:, None], s_[:, None]))
    # absorbed query q_lat[h] = W_UK[h] q_nope[h]; W_UK rows h*512 + c (kernel.py:2355-2443)
    wuk = block_dequant(w["w_uk"], w["s_uk"]).reshape(HEADS, KV_LORA, NOPE_DIM)
    q_lat = codecs.bf16_round(torch.einsum("hcd,shd->shc", wuk, q_nope))
    q = torch.cat([q_lat, q_pe], -1).to(torch.bfloat16)

    # KV row: RMSNorm(latent) and RoPE(k_pe), each rounded to bf16 (kernel.py:2005-2101),
    # then one power-of-two E4M3 scale a token
    kvn = codecs.bf16_round(rmsnorm(kv_a[:, :KV_LORA], w["g_kv"]))
    kpe = codecs.bf16_round(rope_pairs(kv_a[:, KV_LORA:], c, s_))
    kv_codes, kv_scale = fp8_row_quant_pow2(torch.cat([kvn, kpe], -1), scaled=kv_scaled)

    # index key and query (LayerNorm / W_iq, RoPE on dims [0, 64), Hadamard, FP4)
    k_codes, k_e8, _, ik_h = index_key(ik, w["g_ik"], w["b_ik"], c, s_)
    q_codes, q_e8, _, iq_h = index_query(q_an, w["w_iq"], w["s_iq"], c, s_)

    # head weights: bf16(W_iw x) * IHD^-1/2 * IH^-1/2, stored bf16 (indexer.py:340-408)
    iw = (codecs.bf16_round(iw_raw) * INDEX_W_SCALE).to(torch.bfloat16)

    return dict(
        q=q, iq=codecs.e2m1_pack(q_codes), iqs=q_e8, iw=iw,
        slot=slot_of(page_table, pos), kv=kv_codes, kv_scale=kv_scale,
        ikv=codecs.e2m1_pack(k_codes).reshape(S, 4, 16), iks=k_e8,
        x=x, q_a=q_a, kv_a=kv_a, ik=ik, q_an=q_an, q_nope=q_nope, q_pe=q_pe, q_lat=q_lat,
        iq_h=iq_h, ik_h=ik_h,
    )  # fmt: skip


def write_caches(f, caches_ikv, caches_iks, caches_kv, caches_kv_scale):
    """Apply ``front``'s cache rows to CPU copies of the caches in place (the index
    plane ``[pages, 4, 64, 16]`` + scales ``[pages, 4, 64]`` with key t's byte at
    ``(t % 16) * 4 + t // 16``; the MLA cache ``[slots, 576]`` + ``[slots]``)."""
    for i, slot in enumerate(f["slot"].tolist()):
        page, t = slot // PAGE, slot % PAGE
        caches_kv[slot] = f["kv"][i]
        if caches_kv_scale is not None:
            caches_kv_scale[slot] = f["kv_scale"][i]
        caches_ikv[page, :, t, :] = f["ikv"][i]
        caches_iks[page, :, scale_byte(t)] = f["iks"][i]


def back(o_lat, h, w):
    """o[s, h] = bf16(W_UV[h] o_lat[s, h]) (W_UV rows h*128 + v,
    glm53/gfx950/kernel.py:4040-4112), then a = bf16(h + W_o o) with the TP reduce as a
    local add (kernel.py:4125-4197). Returns dict(o [S, 4096] f32 (bf16 values),
    y [S, 7168] f32, a [S, 7168] bf16)."""
    S = o_lat.shape[0]
    wuv = block_dequant(w["w_uv"], w["s_uv"]).reshape(HEADS, V_DIM, KV_LORA)
    o = codecs.bf16_round(torch.einsum("hvc,shc->shv", wuv, o_lat.float())).reshape(S, HEADS * V_DIM)
    y = gemv(o, w["w_o"], w["s_o"])
    return dict(o=o, y=y, a=(h.float() + y).to(torch.bfloat16))
