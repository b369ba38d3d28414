"""SGLang's loaded tensors as the launches' arguments: one covered layer's weights, its
caches and the rotary table, read in place wherever SGLang's layout is the kernels'.

The layout rules follow the reference's binder (sgl_amd_mono/glm53/gfx950/weights.py:
``_need`` :74-80, ``_fp8`` :83-91, ``_shuffled`` :94-100, ``_linear`` :103-108,
``_uk_uv`` :145-177, ``_indexer`` :180-205, ``layer_weights`` :208-311,
``rope_tables`` :321-345) and SGLang's DeepSeek-V2 module names
(``self_attn.fused_qkv_a_proj_with_mqa``, ``q_b_proj``, ``o_proj``, ``w_kc`` /
``w_vc`` / ``w_scale``, ``indexer.{wk, wq_b, weights_proj, k_norm}``,
``mlp.{gate, experts}`` with the shared expert appended as expert 256).

In place: every block-FP8 projection and expert tensor (viewed as bytes, never
copied), the norms, the router and its bias. Copied once at build, and recorded in
``copies`` with what they came from: W_UK / W_UV (SGLang keeps them as per-tensor FP8
``w_kc`` / ``w_vc`` per head; the kernels read [heads * 512, 128] / [heads * 128, 512]
in the (16, 16) layout with a block-scale plane), the indexer's ``weights_proj``
(bf16, read by the MFMA tiles in the (16, 16) byte layout), the indexer's k LayerNorm
in f32 and the rotary table in f32 [positions, 32].
"""

from __future__ import annotations

import torch

from .attn import AttnCaches
from .layer import (HEADS, HIDDEN, INDEX_DIM, INDEX_HEADS, KV_LORA, N_QKV, NOPE_DIM, PE_DIM, Q_LORA, QK_DIM,
                    V_DIM, LayerWeights, ProjWeights)
from .layouts import shuffle_16x16
from .moe import FP8_MOE, Fp8MoeWeights

N_EXPERTS = FP8_MOE.n_experts
# SGLang appends the shared expert to the routed ones (num_fused_shared_experts = 1)
PHYSICAL_EXPERTS = N_EXPERTS + 1
INTER = FP8_MOE.inter
KV_ROW = KV_LORA + PE_DIM
PAGE = 64


class BindError(ValueError):
    """A tensor SGLang loaded does not have the layout the kernels read."""


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _need(name: str, t, shape: tuple, dtypes: tuple) -> torch.Tensor:
    if t is None:
        raise BindError(f"needs {name}; the module has none")
    if tuple(t.shape) != tuple(shape) or t.dtype not in dtypes or not t.is_contiguous():
        raise BindError(
            f"needs {name} as contiguous {'/'.join(str(d) for d in dtypes)} {tuple(shape)}, "
            f"got {t.dtype} {tuple(t.shape)} strides {tuple(t.stride())}"
        )
    return t


def is_shuffled(linear) -> bool:
    """SGLang marks a linear whose FP8 weight it rewrote into AITER's (16, 16) layout."""
    return bool(getattr(linear, "aiter_bpreshuffled", False) or getattr(linear.weight, "is_shuffled", False))


def _fp8_linear(name: str, linear, rows: int, cols: int):
    """A block-FP8 linear in SGLang's (16, 16) layout: (weight bytes, f32 block scales)."""
    w = _need(f"{name}.weight", linear.weight, (rows, cols), (torch.float8_e4m3fn,))
    s = _need(f"{name}.weight_scale_inv", getattr(linear, "weight_scale_inv", None),
              (_cdiv(rows, 128), _cdiv(cols, 128)), (torch.float32,))
    if not is_shuffled(linear):
        raise BindError(f"needs {name} in AITER's (16, 16) FP8 layout; SGLang left it row-major")
    return w.view(torch.uint8), s


def _packed_per_tensor(w: torch.Tensor, scale: torch.Tensor, cols: int):
    """A per-tensor-scaled FP8 matrix as the kernels read it: bytes in the (16, 16)
    layout and an f32 block-scale plane [rows / 128, ceil(cols / 128)] holding the
    one scale."""
    rows = w.shape[0]
    bytes_ = shuffle_16x16(w.contiguous().view(torch.uint8))
    s = scale.reshape(1, 1).float().expand(rows // 128, _cdiv(cols, 128)).contiguous()
    return bytes_, s


def uk_uv(attn, copies: dict, idx: int):
    """W_UK [heads * 512, 128] and W_UV [heads * 128, 512] from SGLang's per-head
    ``w_kc`` [heads, 128, 512] and ``w_vc`` [heads, 512, 128] (per-tensor E4M3 with a
    scalar ``w_scale``): W_UK[(h, c), d] = w_kc[h, d, c], W_UV[(h, v), c] = w_vc[h, c, v]
    (glm53/gfx950/weights.py:145-177)."""
    w_kc, w_vc, w_scale = getattr(attn, "w_kc", None), getattr(attn, "w_vc", None), getattr(attn, "w_scale", None)
    if w_kc is None or w_vc is None:
        raise BindError("needs the absorbed w_kc / w_vc SGLang splits out of kv_b_proj")
    if w_kc.dtype != torch.float8_e4m3fn or w_vc.dtype != torch.float8_e4m3fn or w_scale is None \
            or w_scale.numel() != 1:
        raise BindError(
            f"needs w_kc / w_vc as per-tensor FP8 E4M3 with a scalar w_scale, got {w_kc.dtype} / {w_vc.dtype} "
            f"and {None if w_scale is None else tuple(w_scale.shape)}"
        )
    if tuple(w_kc.shape) != (HEADS, NOPE_DIM, KV_LORA) or tuple(w_vc.shape) != (HEADS, KV_LORA, V_DIM):
        raise BindError(
            f"needs w_kc [{HEADS}, {NOPE_DIM}, {KV_LORA}] and w_vc [{HEADS}, {KV_LORA}, {V_DIM}] (one GPU's TP=4 "
            f"share), got {tuple(w_kc.shape)} and {tuple(w_vc.shape)}"
        )
    uk = w_kc.transpose(1, 2).reshape(HEADS * KV_LORA, NOPE_DIM)
    uv = w_vc.transpose(1, 2).reshape(HEADS * V_DIM, KV_LORA)
    w_uk, s_uk = _packed_per_tensor(uk, w_scale, NOPE_DIM)
    w_uv, s_uv = _packed_per_tensor(uv, w_scale, KV_LORA)
    for name, t in (("w_uk", w_uk), ("s_uk", s_uk), ("w_uv", w_uv), ("s_uv", s_uv)):
        copies[idx, name] = t
    return w_uk, s_uk, w_uv, s_uv


def experts_reason(mlp) -> str | None:
    """Why a layer's MoE cannot run on the kernels (None: it can)."""
    experts = getattr(mlp, "experts", None)
    if experts is None or getattr(mlp, "gate", None) is None:
        return "needs a routed MoE (gate + experts)"
    w13 = getattr(experts, "w13_weight", None)
    if w13 is None or w13.dtype != torch.float8_e4m3fn:
        return f"needs block-FP8 experts, got {None if w13 is None else w13.dtype}"
    if w13.shape[0] != PHYSICAL_EXPERTS:
        return (f"needs the shared expert fused into the routed ones ({PHYSICAL_EXPERTS} physical experts, "
                f"SGLang's num_fused_shared_experts = 1), got {w13.shape[0]}")
    if not bool(getattr(experts, "is_shuffled", False) or getattr(w13, "is_shuffled", False)):
        return "needs the experts in AITER's (16, 16) FP8 layout (SGLang's AITER MoE runner shuffles them)"
    return None


def moe_weights(layer) -> Fp8MoeWeights:
    mlp = layer.mlp
    why = experts_reason(mlp)
    if why is not None:
        raise BindError(why)
    ex, gate = mlp.experts, mlp.gate
    f8, f32, bf16 = (torch.float8_e4m3fn,), (torch.float32,), (torch.bfloat16,)
    H, E1, I = HIDDEN, PHYSICAL_EXPERTS, INTER
    w13 = _need("experts.w13_weight", ex.w13_weight, (E1, 2 * I, H), f8)
    s13 = _need("experts.w13_weight_scale_inv", getattr(ex, "w13_weight_scale_inv", None), (E1, 2 * I // 128, H // 128), f32)
    w2 = _need("experts.w2_weight", ex.w2_weight, (E1, H, I), f8)
    s2 = _need("experts.w2_weight_scale_inv", getattr(ex, "w2_weight_scale_inv", None), (E1, H // 128, I // 128), f32)
    w_router = _need("gate.weight", gate.weight, (N_EXPERTS, H), bf16)
    bias = _need("gate.e_score_correction_bias", getattr(gate, "e_score_correction_bias", None), (N_EXPERTS,), f32)
    g_post = _need("post_attention_layernorm.weight", layer.post_attention_layernorm.weight, (H,), bf16)
    return Fp8MoeWeights(g_post=g_post, w_router=w_router, bias=bias, w13=w13.view(torch.uint8), s13=s13,
                         w2=w2.view(torch.uint8), s2=s2)


def proj_weights(layer, idx: int, copies: dict) -> ProjWeights:
    attn = layer.self_attn
    bf16 = (torch.bfloat16,)
    ind = getattr(attn, "indexer", None)
    if ind is None:
        raise BindError("needs the layer's own indexer (every covered layer scores and selects its keys)")
    w_qkv, s_qkv = _fp8_linear("fused_qkv_a_proj_with_mqa", attn.fused_qkv_a_proj_with_mqa, N_QKV, HIDDEN)
    w_qb, s_qb = _fp8_linear("q_b_proj", attn.q_b_proj, HEADS * QK_DIM, Q_LORA)
    w_o, s_o = _fp8_linear("o_proj", attn.o_proj, HIDDEN, HEADS * V_DIM)
    w_ik, s_ik = _fp8_linear("indexer.wk", ind.wk, INDEX_DIM, HIDDEN)
    w_iq, s_iq = _fp8_linear("indexer.wq_b", ind.wq_b, INDEX_HEADS * INDEX_DIM, Q_LORA)
    iw = _need("indexer.weights_proj.weight", ind.weights_proj.weight, (INDEX_HEADS, HIDDEN), bf16)
    w_iw = shuffle_16x16(iw.view(torch.uint8)).view(torch.bfloat16)
    g_ik = ind.k_norm.weight.detach().float().contiguous()
    b_ik = ind.k_norm.bias.detach().float().contiguous()
    _need("indexer.k_norm.weight", g_ik, (INDEX_DIM,), (torch.float32,))
    _need("indexer.k_norm.bias", b_ik, (INDEX_DIM,), (torch.float32,))
    copies[idx, "w_iw"], copies[idx, "g_ik"], copies[idx, "b_ik"] = w_iw, g_ik, b_ik
    w_uk, s_uk, w_uv, s_uv = uk_uv(attn, copies, idx)
    return ProjWeights(
        g_in=_need("input_layernorm.weight", layer.input_layernorm.weight, (HIDDEN,), bf16),
        w_qkv=w_qkv, s_qkv=s_qkv, w_ik=w_ik, s_ik=s_ik, w_iw=w_iw,
        g_q=_need("q_a_layernorm.weight", attn.q_a_layernorm.weight, (Q_LORA,), bf16),
        g_kv=_need("kv_a_layernorm.weight", attn.kv_a_layernorm.weight, (KV_LORA,), bf16),
        g_ik=g_ik, b_ik=b_ik, w_qb=w_qb, s_qb=s_qb, w_iq=w_iq, s_iq=s_iq,
        w_uk=w_uk, s_uk=s_uk, w_uv=w_uv, s_uv=s_uv, w_o=w_o, s_o=s_o,
    )  # fmt: skip


def layer_weights(layer, idx: int, copies: dict) -> LayerWeights:
    """A covered layer's tensors; raises ``BindError`` naming the first tensor whose
    layout the kernels cannot read."""
    try:
        return LayerWeights(proj=proj_weights(layer, idx, copies), moe=moe_weights(layer))
    except BindError as e:
        raise BindError(f"layer {idx}: {e}") from None


def unshuffled(layer) -> list[str]:
    """The layer's block-FP8 projections SGLang left row-major."""
    attn = layer.self_attn
    names = {"fused_qkv_a_proj_with_mqa": attn.fused_qkv_a_proj_with_mqa, "q_b_proj": attn.q_b_proj,
             "o_proj": attn.o_proj}
    ind = getattr(attn, "indexer", None)
    if ind is not None:
        names["indexer.wk"], names["indexer.wq_b"] = ind.wk, ind.wq_b
    return [n for n, lin in names.items() if not is_shuffled(lin)]


def _cos_sin(rotary):
    """(cos, sin) [positions, 32] of a rotary: SGLang's f32 ``cos_sin_cache``
    [positions, 64] (cos, then sin) or separate ``cos_cache`` / ``sin_cache``."""
    cache = getattr(rotary, "cos_sin_cache", None)
    if cache is not None:
        return cache[:, : PE_DIM // 2], cache[:, PE_DIM // 2:]
    cos, sin = rotary.cos_cache, rotary.sin_cache
    return cos.reshape(cos.shape[0], -1), sin.reshape(sin.shape[0], -1)


def rope_tables(layers: list, copies: dict):
    """The f32 cos / sin [positions, 32] every covered layer's MLA and indexer rotaries
    read (both must hold the first layer's MLA table)."""
    cos, sin = _cos_sin(layers[0].self_attn.rotary_emb)
    if cos.dim() != 2 or cos.shape[1] != PE_DIM // 2:
        raise BindError(f"needs rotary tables [positions, {PE_DIM // 2}], got {tuple(cos.shape)}")
    for layer in layers:
        for rot in (layer.self_attn.rotary_emb, getattr(layer.self_attn.indexer, "rotary_emb", None)):
            if rot is None:
                continue
            c, s = _cos_sin(rot)
            if c.shape != cos.shape or not (torch.equal(c, cos) and torch.equal(s, sin)):
                raise BindError("needs every rotary table (MLA and indexer, all layers) to be the first layer's")
    cos, sin = cos.float().contiguous(), sin.float().contiguous()
    copies["rope", "cos"], copies["rope", "sin"] = cos, sin
    return cos, sin


def caches(pool, idx: int) -> AttnCaches:
    """Layer ``idx``'s caches from SGLang's DSA pool, in place: the MLA cache
    [slots, 1, 576] of raw E4M3 rows (SGLang's HIP DSA layout, no scale: the launches
    run with ``kv_scale=None``) and the FP4 index plane (payload [pages, 1, 4, 64, 16],
    E8M0 scales [pages, 1, 4, 64]; deepseek_v4/gfx950/runner.py:336-347)."""
    kv = pool.get_key_buffer(idx)
    if kv.dtype not in (torch.float8_e4m3fn, torch.uint8) or kv.shape[-1] != KV_ROW or not kv.is_contiguous():
        raise BindError(f"layer {idx}: MLA cache {kv.dtype} {tuple(kv.shape)}; needs contiguous E4M3 [slots, 1, {KV_ROW}]")
    slots = kv.numel() // KV_ROW
    if slots % PAGE:
        raise BindError(f"layer {idx}: MLA cache of {slots} slots is not whole {PAGE}-token pages")
    pay = pool.get_index_k_fp4_payload_buffer(idx)
    sc = pool.get_index_k_fp4_scale_buffer(idx)
    pages = slots // PAGE
    if tuple(pay.shape[1:]) != (1, 4, PAGE, 16) or tuple(sc.shape[1:]) != (1, 4, PAGE) or pay.dtype != torch.uint8 \
            or sc.dtype != torch.uint8 or pay.shape[0] < pages or sc.shape[0] < pages:
        raise BindError(
            f"layer {idx}: FP4 index pages {pay.dtype} {tuple(pay.shape)} / {sc.dtype} {tuple(sc.shape)}; needs "
            f"uint8 [>= {pages}, 1, 4, {PAGE}, 16] / [>= {pages}, 1, 4, {PAGE}]"
        )
    return AttnCaches(ikv=pay.view(pay.shape[0], 4, PAGE, 16), iks=sc.view(sc.shape[0], 4, PAGE),
                      kv=kv.view(torch.uint8).view(slots, KV_ROW), kv_scale=None)
