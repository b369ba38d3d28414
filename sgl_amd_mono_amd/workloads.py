"""Seeded synthetic inputs of the BASELINE configs (random-init weights of the real
shapes; there is no checkpoint or dataset offline).

Distributions follow the reference's own test generators where they exist
(test/kernels/glm53/check_layer.py:52-146 for the FP8 layer,
test/kernels/test_minimax_m31_ffn.py:40-60 for MXFP4 codes and scales,
test/kernels/test_deepseek_v41_k2i.py:103-130 for FP4 index keys). Generators run
on whatever device they are given; the GPU's and the CPU's random streams differ,
so a parity test generates once and copies.
"""

from __future__ import annotations

import torch

from .layouts import shuffle_16x16
from .moe import Fp8MoeWeights, MoeGeometry, Mxfp4MoeWeights


def _gen(device, seed: int) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


def fp8_codes(shape, g: torch.Generator, device) -> torch.Tensor:
    """E4M3 codes of N(0, 1) samples rounded through bf16 (check_layer.py:56-59)."""
    x = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    return x.to(torch.bfloat16).to(torch.float8_e4m3fn).view(torch.uint8)


def fp8_moe_weights(geo: MoeGeometry, device, seed: int = 0) -> Fp8MoeWeights:
    """One layer's FP8 MoE weights: router ~N(0,1)*2/sqrt(H) bf16 (check_layer.py:96-98),
    bias ~N(0, 0.1) f32 (:99), post-norm weight 1 + 0.1*N(0,1) bf16, experts E4M3 from
    N(0,1) with 128x128 f32 block scales ~U(0.5, 2)/448, stored in AITER's (16, 16)
    shuffled layout as SGLang's ROCm MoE leaves them. Expert E is the shared one."""
    H, E, I = geo.hidden, geo.n_experts, geo.inter
    g = _gen(device, seed)
    w_router = (torch.randn(E, H, generator=g, device=device) * (2.0 / H**0.5)).to(torch.bfloat16)
    bias = torch.randn(E, generator=g, device=device) * 0.1
    g_post = (1.0 + 0.1 * torch.randn(H, generator=g, device=device)).to(torch.bfloat16)
    w13 = torch.empty(E + 1, 2 * I, H, dtype=torch.uint8, device=device)
    w2 = torch.empty(E + 1, H, I, dtype=torch.uint8, device=device)
    for e0 in range(0, E + 1, 32):  # 32 experts at a time bound the f32 temporaries
        e1 = min(e0 + 32, E + 1)
        w13[e0:e1] = shuffle_16x16(fp8_codes((e1 - e0, 2 * I, H), g, device))
        w2[e0:e1] = shuffle_16x16(fp8_codes((e1 - e0, H, I), g, device))
    s13 = (torch.rand(E + 1, 2 * I // 128, H // 128, generator=g, device=device) * 1.5 + 0.5) / 448.0
    s2 = (torch.rand(E + 1, H // 128, I // 128, generator=g, device=device) * 1.5 + 0.5) / 448.0
    return Fp8MoeWeights(g_post=g_post, w_router=w_router, bias=bias, w13=w13, s13=s13, w2=w2, s2=s2)


def rows_bf16(rows: int, hidden: int, device, seed: int) -> torch.Tensor:
    """Activation rows ~N(0, 1) in bf16."""
    g = _gen(device, seed)
    return torch.randn(rows, hidden, generator=g, device=device).to(torch.bfloat16)


def mxfp4_moe_weights(geo: MoeGeometry, device, seed: int = 0) -> Mxfp4MoeWeights:
    """MXFP4 experts: uniform random E2M1 code bytes in AITER's (16, 16) layout, E8M0
    scales uniform in [119, 123) (test_minimax_m31_ffn.py:47-51: 'e8m0 codes around
    2^-7')."""
    H, E, I = geo.hidden, geo.n_experts, geo.inter
    g = _gen(device, seed)
    u8 = dict(generator=g, device=device, dtype=torch.uint8)
    return Mxfp4MoeWeights(
        w13=shuffle_16x16(torch.randint(0, 256, (E + 1, 2 * I, H // 2), **u8)),
        s13=torch.randint(119, 123, (E + 1, 2 * I, H // 32), **u8),
        w2=shuffle_16x16(torch.randint(0, 256, (E + 1, H, I // 2), **u8)),
        s2=torch.randint(119, 123, (E + 1, H, I // 32), **u8),
    )


def gate_logits(rows: int, n_experts: int, device, seed: int) -> torch.Tensor:
    """f32 gate logits ~N(0, 1)."""
    return torch.randn(rows, n_experts, generator=_gen(device, seed), device=device)


def toy_moe(seed: int = 0, rows: int = 4, hidden: int = 1024, n_experts: int = 8, inter: int = 512):
    """BASELINE config 1 on the CPU: bf16 weights ~N(0, 0.02), rows ~N(0, 1),
    ``torch.manual_seed(seed)``."""
    torch.manual_seed(seed)
    return dict(
        x=torch.randn(rows, hidden).to(torch.bfloat16),
        w_router=(torch.randn(n_experts, hidden) * 0.02).to(torch.bfloat16),
        w_gate=(torch.randn(n_experts, inter, hidden) * 0.02).to(torch.bfloat16),
        w_up=(torch.randn(n_experts, inter, hidden) * 0.02).to(torch.bfloat16),
        w_down=(torch.randn(n_experts, hidden, inter) * 0.02).to(torch.bfloat16),
    )


def attn_case(ctx_lens, device, seed: int = 0, max_ctx: int = 32768, spare_pages: int = 3):
    """BASELINE config 3 inputs: ``len(ctx_lens)`` rows, each an independent request of
    ``ctx_lens[s]`` keys whose pages are scattered over SGLang-layout caches
    (test/kernels/test_deepseek_v41_k2i.py:103-130 ``fp4_case``): index keys are uniform
    random E2M1 bytes with E8M0 scales in [123, 130), index queries likewise, head
    weights ~N(0, 0.05) bf16, the MLA cache E4M3 of N(0, 1) samples with per-token
    scales ~U(0.5, 2), q ~N(0, 1) bf16. Returns (AttnStep, AttnCaches)."""
    from .attn import DQK, IH, ID, NH, PAGE, AttnCaches, AttnStep

    g = _gen(device, seed)
    S = len(ctx_lens)
    ppr = max_ctx // PAGE
    used = [-(-int(n) // PAGE) for n in ctx_lens]
    pages = sum(used) + spare_pages
    u8 = dict(generator=g, device=device, dtype=torch.uint8)
    ikv = torch.randint(0, 256, (pages, 4, PAGE, 16), **u8)
    iks = torch.randint(123, 130, (pages, 4, PAGE), **u8)
    kv = fp8_codes((pages * PAGE, DQK), g, device)
    kv_scale = torch.rand(pages * PAGE, generator=g, device=device) * 1.5 + 0.5
    perm = torch.randperm(pages, generator=g, device=device).to(torch.int32)
    table = torch.zeros(S, ppr, dtype=torch.int32, device=device)
    at = 0
    for s, u in enumerate(used):
        table[s, :u] = perm[at:at + u]
        at += u
    step = AttnStep(
        iq=torch.randint(0, 256, (S, IH, ID // 2), **u8),
        iqs=torch.randint(123, 130, (S, IH, ID // 32), **u8),
        iw=(torch.randn(S, IH, generator=g, device=device) * 0.05).to(torch.bfloat16),
        q=torch.randn(S, NH, DQK, generator=g, device=device).to(torch.bfloat16),
        page_table=table,
        seq_lens=torch.tensor([int(n) for n in ctx_lens], dtype=torch.int32, device=device),
    )
    return step, AttnCaches(ikv=ikv, iks=iks, kv=kv, kv_scale=kv_scale)


def _fp8_matrix(n: int, k: int, g: torch.Generator, device):
    """E4M3 codes of N(0, 1) samples in the (16, 16) layout and f32 128 x 128 block
    scales ~U(0.5, 2) / (1.25 sqrt(K)), so a GEMV of unit-variance rows gives outputs
    of about unit variance."""
    codes = shuffle_16x16(fp8_codes((n, k), g, device))
    s = (torch.rand(-(-n // 128), k // 128, generator=g, device=device) * 1.5 + 0.5) / (1.25 * k**0.5)
    return codes, s


def proj_weights(device, seed: int = 0):
    """One layer's attention-block projection weights (sgl_amd_mono_amd.layer.WEIGHT_SPECS):
    FP8 matrices as ``_fp8_matrix``, RMSNorm weights 1 + 0.1 N(0, 1) bf16, the index
    key LayerNorm weight 1 + 0.1 N(0, 1) and bias 0.1 N(0, 1) f32, the index head-weight
    matrix N(0, 1/7168) bf16 (its bytes (16, 16)-shuffled)."""
    from .layer import HEADS, HIDDEN, INDEX_DIM, INDEX_HEADS, KV_LORA, N_QKV, NOPE_DIM, Q_LORA, QK_DIM, V_DIM
    from .layer import ProjWeights

    g = _gen(device, seed)

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)

    w = {}
    w["g_in"] = norm(HIDDEN)
    w["w_qkv"], w["s_qkv"] = _fp8_matrix(N_QKV, HIDDEN, g, device)
    w["w_ik"], w["s_ik"] = _fp8_matrix(INDEX_DIM, HIDDEN, g, device)
    iw = (torch.randn(INDEX_HEADS, HIDDEN, generator=g, device=device) * HIDDEN**-0.5).to(torch.bfloat16)
    w["w_iw"] = shuffle_16x16(iw.view(torch.uint8)).view(torch.bfloat16)
    w["g_q"] = norm(Q_LORA)
    w["g_kv"] = norm(KV_LORA)
    w["g_ik"] = 1.0 + 0.1 * torch.randn(INDEX_DIM, generator=g, device=device)
    w["b_ik"] = 0.1 * torch.randn(INDEX_DIM, generator=g, device=device)
    w["w_qb"], w["s_qb"] = _fp8_matrix(HEADS * QK_DIM, Q_LORA, g, device)
    w["w_iq"], w["s_iq"] = _fp8_matrix(INDEX_HEADS * INDEX_DIM, Q_LORA, g, device)
    w["w_uk"], w["s_uk"] = _fp8_matrix(HEADS * KV_LORA, NOPE_DIM, g, device)
    w["w_uv"], w["s_uv"] = _fp8_matrix(HEADS * V_DIM, KV_LORA, g, device)
    w["w_o"], w["s_o"] = _fp8_matrix(HIDDEN, HEADS * V_DIM, g, device)
    return ProjWeights(**w)


def rope_tables(max_pos: int, device, dim: int = 64, theta: float = 10000.0):
    """RoPE cos / sin f32 [max_pos, dim / 2]: angle = pos * theta^(-2i / dim), formed
    in f64."""
    inv = theta ** (-torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None]
    return torch.cos(ang).float().to(device), torch.sin(ang).float().to(device)
