"""Number formats of the path, restated on the CPU (test infrastructure only).

E4M3 (OCP ``float8_e4m3fn``), E2M1 (MXFP4 element), E8M0 (MX block scale), the
per-128 FP8 block quantisation the reference applies to activations, and the
per-32 FP4 quantisation of the indexer's query.
"""

from __future__ import annotations

import torch

FP8_MAX = 448.0  # glm53/gfx950/config.py:278 (FP8_MAX = 448.0)
FP4_MAX = 6.0  # the largest E2M1 magnitude
# E2M1 code -> value, code 8..15 the negatives (test/kernels/test_deepseek_v41_k2i.py:95-96)
E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
E2M1 = E2M1 + [-v for v in E2M1]


def e4m3_decode(codes: torch.Tensor) -> torch.Tensor:
    """uint8 E4M3 codes -> float32 (exact; 0x7F / 0xFF are NaN). The reference
    widens FP8 to bf16 exactly before its MFMA (common/ops.py:333-346)."""
    return codes.contiguous().view(torch.float8_e4m3fn).float()


def e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    """float32 already clamped to [-448, 448] -> uint8 E4M3 codes, round to nearest
    even (the hardware ``v_cvt_pk_fp8_f32`` the reference uses, common/ops.py:259-263)."""
    if bool((x.abs() > FP8_MAX).any()):
        raise ValueError("e4m3_encode: input outside [-448, 448]; clamp first")
    return x.float().to(torch.float8_e4m3fn).view(torch.uint8)


def e2m1_decode(packed: torch.Tensor) -> torch.Tensor:
    """uint8 [..., K/2] two E2M1 codes a byte, element 2i in the low nibble
    (test/kernels/test_deepseek_v41_k2i.py:144-146) -> float32 [..., K]."""
    lut = torch.tensor(E2M1, dtype=torch.float32)
    p = packed.long()
    return torch.stack([lut[p & 15], lut[p >> 4]], -1).flatten(-2)


def e2m1_encode(x: torch.Tensor) -> torch.Tensor:
    """float32 in [-6, 6] -> uint8 E2M1 codes (one a byte), round to nearest with
    ties to the even code, as the hardware FP4 convert does."""
    a = x.abs().float()
    mag = torch.tensor(E2M1[:8], dtype=torch.float32)
    # distance to each representable magnitude; ties go to the even code
    d = (a[..., None] - mag).abs()
    best = d.min(-1, keepdim=True).values
    cand = d == best
    codes = torch.arange(8)
    # among tied candidates prefer the even code
    score = torch.where(cand, codes % 2, torch.full_like(codes, 99))
    code = score.argmin(-1)
    neg = (x < 0) & (code != 0)
    return (code + 8 * neg.long()).to(torch.uint8)


def e2m1_pack(codes: torch.Tensor) -> torch.Tensor:
    """uint8 codes [..., K] -> packed bytes [..., K/2] (element 2i low nibble)."""
    c = codes.to(torch.int64).reshape(*codes.shape[:-1], -1, 2)
    return (c[..., 0] | (c[..., 1] << 4)).to(torch.uint8)


def e8m0_decode(codes: torch.Tensor) -> torch.Tensor:
    """uint8 E8M0 codes -> float32 2^(code - 127) (code 255 = NaN)."""
    c = codes.to(torch.float64)
    v = torch.exp2(c - 127.0)
    v[codes == 255] = float("nan")
    return v.float()


def code_ceil(v: torch.Tensor) -> torch.Tensor:
    """Biased exponent of the smallest power of two >= v, clamped to [1, 254]
    (common/mx.py:26-32)."""
    bits = v.float().contiguous().view(torch.int32)
    e = ((bits >> 23) & 0xFF) + ((bits & 0x7FFFFF) != 0).int()
    return e.clamp(1, 254)


def fp8_block_quant(x: torch.Tensor, block: int = 128):
    """Per-``block`` FP8 quantisation along the last dim: (codes uint8, scales f32).

    glm53/gfx950/kernel.py:1440-1450 (``quant_scaled``): amax over the block,
    scale = amax * (1/448), values x * (448 / amax) clamped to +-448 and rounded to
    E4M3; an all-zero block has scale 1 and zero values. The reference forms the
    reciprocal with the hardware ``v_rcp_f32``; this restatement divides exactly,
    which can move a value across an E4M3 rounding boundary by one code.
    """
    g = x.float().reshape(*x.shape[:-1], -1, block)
    amax = g.abs().amax(-1, keepdim=True)
    nz = amax > 0
    scale = torch.where(nz, amax * (1.0 / FP8_MAX), torch.ones_like(amax))
    inv = torch.where(nz, FP8_MAX / amax.clamp_min(1e-38), torch.ones_like(amax))
    q = (g * inv).clamp(-FP8_MAX, FP8_MAX)
    codes = e4m3_encode(q).reshape(x.shape)
    return codes, scale.squeeze(-1)


def fp8_block_dequant(codes: torch.Tensor, scales: torch.Tensor, block: int = 128):
    """Inverse of ``fp8_block_quant`` along the last dim."""
    v = e4m3_decode(codes).reshape(*codes.shape[:-1], -1, block)
    return (v * scales[..., None]).reshape(codes.shape)


def mxfp4_dequant(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """[N, K/2] packed E2M1 + [N, K/32] E8M0 -> f32 [N, K]
    (test/kernels/deepseek_v41/check_ffn.py:107-114, ``deq_fp4``)."""
    v = e2m1_decode(packed)
    return v * e8m0_decode(scales).repeat_interleave(32, -1)


def fp4_block_quant(v: torch.Tensor):
    """FP4 quantisation over 32-element blocks with a power-of-two scale
    (deepseek_v4/gfx950/kernels/stages/indexer.py:143-151, ``fp4_block``):
    scale = pow2_ceil(max(amax, 6 * 2^-126) / 6), codes = E2M1(clamp(v / scale, +-6)).
    Returns (codes uint8 [..., K], e8m0 uint8 [..., K/32], dequantised f32)."""
    g = v.float().reshape(*v.shape[:-1], -1, 32)
    amax = g.abs().amax(-1, keepdim=True)
    code = code_ceil(torch.maximum(amax, torch.tensor(FP4_MAX * 2.0**-126)) * (1.0 / FP4_MAX))
    sc = torch.exp2(code.double() - 127).float()
    q = (g / sc).clamp(-FP4_MAX, FP4_MAX)
    codes = e2m1_encode(q)
    deq = e2m1_decode_codes(codes) * sc
    return codes.reshape(v.shape), code.squeeze(-1).to(torch.uint8), deq.reshape(v.shape)


def e2m1_decode_codes(codes: torch.Tensor) -> torch.Tensor:
    """uint8 E2M1 codes (one a byte) -> float32."""
    lut = torch.tensor(E2M1, dtype=torch.float32)
    return lut[codes.long()]


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    """float32 -> bf16 (round to nearest even) -> float32."""
    return x.float().to(torch.bfloat16).float()


def aiter_unshuffle(ws: torch.Tensor) -> torch.Tensor:
    """AITER (16, 16)-shuffled ``[..., N, K]`` bytes -> row-major ``[..., N, K]`` uint8.

    Byte (n, k) of the row-major matrix sits at flat offset
    ``((n // 16 * K / 32 + k // 32) * 2 + (k % 32) // 16) * 256 + (n % 16) * 16 + k % 16``
    of the shuffled one: the ``[N/16, K/32, 2, 16 rows, 16 B]`` order that
    glm53/gfx950/kernel.py:787-808 (``ld_fp8_chunk``) reads and
    test/kernels/glm53_flash/check_layer.py:932-939 (``_dequant``) undoes. Computed as
    a gather from that formula."""
    *lead, n, k = ws.shape
    flat = ws.contiguous().view(torch.uint8).reshape(*lead, n * k)
    ni = torch.arange(n)[:, None]
    ki = torch.arange(k)[None, :]
    src = ((ni // 16 * (k // 32) + ki // 32) * 2 + (ki % 32) // 16) * 256 + (ni % 16) * 16 + ki % 16
    return flat[..., src.reshape(-1)].reshape(*lead, n, k)
