"""Independent pins of three oracle functions the rest of the suite builds on.

* ``codecs.aiter_unshuffle`` against the reference's two statements of AITER's (16, 16)
  layout: the inverse reshape/permute of test/kernels/glm53_flash/check_layer.py:932-939
  and the per-lane chunk addresses of ``ld_fp8_chunk`` (glm53/gfx950/kernel.py:787-808),
  on a hand-numbered matrix (every byte carries its own shuffled offset).
* ``moe.fp8_router`` (post-attention RMSNorm, bf16 staging, bf16 router GEMV, sigmoid;
  kernel.py:4199-4330) against a constant-row closed form and a float64 loop.
* ``moe.fp8_expert`` (gate = the first I rows of w13, up = the next I, silu(gate) * up,
  per-128 FP8 mid, block-scaled down; the structure of
  test/kernels/deepseek_v41/check_ffn.py:208-219) against a float64 loop.

Each checker is also run on a copy of the function with a plausible mistake planted
(halves swapped, gate and up swapped, gamma dropped, ...) and must reject it.
"""

import math

import pytest
import torch

from oracle import codecs, layer, moe


# ---------------------------------------------------------------- AITER (16, 16) layout
def _numbered(n: int, k: int):
    """A shuffled [n, k] byte matrix whose bytes spell their own flat offset, as two
    byte planes (offset // 256, offset % 256)."""
    off = torch.arange(n * k, dtype=torch.int64).reshape(n, k)
    return (off // 256).to(torch.uint8), (off % 256).to(torch.uint8)


def _offsets(unshuffle, n: int, k: int) -> torch.Tensor:
    """[n, k]: the shuffled offset `unshuffle` reads element (n, k) from."""
    hi, lo = _numbered(n, k)
    return unshuffle(hi).long() * 256 + unshuffle(lo).long()


def _check_against_permute(unshuffle, n: int, k: int) -> None:
    """check_layer.py:932-939: w.reshape(n // 16, k // 32, 2, 16, 16).permute(0, 3, 1, 2, 4)."""
    want = torch.arange(n * k).reshape(n // 16, k // 32, 2, 16, 16).permute(0, 3, 1, 2, 4).reshape(n, k)
    got = _offsets(unshuffle, n, k)
    assert torch.equal(got, want), "unshuffle disagrees with the reference's inverse permute"


def _check_against_lane_addresses(unshuffle, n: int, k: int) -> None:
    """kernel.py:787-808: lane ln = 16 b + r of 64-k chunk kc of row group rg loads 8
    bytes at word ((rg K/32 + 2 kc) 512 + (b / 2) 256 + r 16 + (b % 2) 8) / 4 and 8 more
    128 words on: row 16 rg + r, k = 64 kc + 8 b + [0, 8) and 64 kc + 32 + 8 b + [0, 8)
    (the bf16 MFMA operand a lane holds)."""
    got = _offsets(unshuffle, n, k)
    for rg in range(n // 16):
        for kc in range(k // 64):
            for ln in range(64):
                b, r = ln // 16, ln % 16
                byte = (rg * (k // 32) + 2 * kc) * 512 + (b // 2) * 256 + r * 16 + (b % 2) * 8
                row = 16 * rg + r
                for j in range(8):
                    assert int(got[row, 64 * kc + 8 * b + j]) == byte + j, (rg, kc, ln, j)
                    assert int(got[row, 64 * kc + 32 + 8 * b + j]) == byte + 512 + j, (rg, kc, ln, j)


def test_aiter_unshuffle_matches_the_reference_permute():
    for n, k in ((16, 32), (32, 128), (64, 256)):
        _check_against_permute(codecs.aiter_unshuffle, n, k)


def test_aiter_unshuffle_matches_the_kernel_lane_addresses():
    _check_against_lane_addresses(codecs.aiter_unshuffle, 32, 128)


def _mutant_unshuffle(kind: str):
    """aiter_unshuffle with one plausible misreading of the layout."""

    def f(ws):
        n, k = ws.shape
        flat = ws.contiguous().reshape(-1)
        ni = torch.arange(n)[:, None]
        ki = torch.arange(k)[None, :]
        half = (ki % 32) // 16
        if kind == "halves_swapped":
            half = 1 - half
        if kind == "row_major_tiles":  # [N/16, K/32, 16 rows, 32 B]
            src = (ni // 16 * (k // 32) + ki // 32) * 512 + (ni % 16) * 32 + ki % 32
        elif kind == "kblocks_outer":  # [K/32, N/16, 2, 16, 16]
            src = ((ki // 32 * (n // 16) + ni // 16) * 2 + half) * 256 + (ni % 16) * 16 + ki % 16
        else:
            src = ((ni // 16 * (k // 32) + ki // 32) * 2 + half) * 256 + (ni % 16) * 16 + ki % 16
        return flat[src.reshape(-1)].reshape(n, k)

    return f


@pytest.mark.parametrize("kind", ["halves_swapped", "row_major_tiles", "kblocks_outer"])
def test_layout_pins_reject_planted_mistakes(kind):
    with pytest.raises(AssertionError):
        _check_against_permute(_mutant_unshuffle(kind), 32, 128)
    with pytest.raises(AssertionError):
        _check_against_lane_addresses(_mutant_unshuffle(kind), 32, 128)


# ---------------------------------------------------------------- router
def _router_case(seed: int, S=3, H=256, E=24):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(S, H, generator=g) * 3).to(torch.bfloat16)
    g_post = (1 + 0.5 * torch.randn(H, generator=g)).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.2).to(torch.bfloat16)
    return a, g_post, w


def _router_fp64(a, g_post, w, eps):
    """float64 loops: rstd = 1 / sqrt(sum(a^2) / H + eps), the normed value bf16-rounded
    as the kernel stages it, the dot with the bf16 weight row, sigmoid."""
    S, H = a.shape
    E = w.shape[0]
    av, gv, wv = a.double(), g_post.double(), w.double()
    x = torch.zeros(S, H, dtype=torch.float64)
    scores = torch.zeros(S, E, dtype=torch.float64)
    for s in range(S):
        rstd = 1.0 / math.sqrt(sum(float(v) ** 2 for v in av[s]) / H + eps)
        x[s] = av[s] * rstd * gv
        xb = x[s].float().to(torch.bfloat16).double()
        for e in range(E):
            z = float((xb * wv[e]).sum())
            scores[s, e] = 1.0 / (1.0 + math.exp(-z))
    return x, scores


def _check_router(router, seed: int, eps: float) -> None:
    a, g_post, w = _router_case(seed)
    x, scores = router(a, g_post, w, eps)
    x64, s64 = _router_fp64(a, g_post, w, eps)
    assert torch.allclose(x.double(), x64, rtol=1e-5, atol=1e-6), "normed rows"
    assert torch.allclose(scores.double(), s64, rtol=0, atol=2e-6), "sigmoid scores"


@pytest.mark.parametrize("eps", [1e-6, 0.5, 4.0])
def test_fp8_router_equals_fp64_loops(eps):
    _check_router(moe.fp8_router, 11, eps)


def test_fp8_router_constant_rows_closed_form():
    """a row of constant c: mean(a^2) = c^2, so x_j = c gamma_j / sqrt(c^2 + eps); a
    one-hot router row e picks x_e: score = sigmoid(bf16(x_e) w)."""
    H, E, eps = 256, 4, 0.25
    c = 1.5
    a = torch.full((1, H), c).to(torch.bfloat16)
    g_post = torch.linspace(0.5, 2.0, H).to(torch.bfloat16)
    w = torch.zeros(E, H)
    picks = [0, 17, 128, 255]
    for e, j in enumerate(picks):
        w[e, j] = 0.75 * (e + 1)
    w = w.to(torch.bfloat16)
    _, scores = moe.fp8_router(a, g_post, w, eps)
    for e, j in enumerate(picks):
        xj = c * float(g_post[j]) / math.sqrt(c * c + eps)
        z = float(torch.tensor(xj).to(torch.bfloat16)) * float(w[e, j])
        assert abs(float(scores[0, e]) - 1.0 / (1.0 + math.exp(-z))) < 1e-6, (e, j)


def _router_mutant(kind: str):
    def f(a, g_post, w, eps):
        x = a.float()
        if kind == "sum_not_mean":
            rstd = torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + eps)
        elif kind == "eps_dropped":
            rstd = torch.rsqrt(x.pow(2).mean(-1, keepdim=True))
        else:
            rstd = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
        x = x * rstd if kind == "gamma_dropped" else x * rstd * g_post.float()
        logits = codecs.bf16_round(x) @ w.float().T
        return x, (torch.softmax(logits, -1) if kind == "softmax" else torch.sigmoid(logits))

    return f


@pytest.mark.parametrize("kind", ["gamma_dropped", "eps_dropped", "sum_not_mean", "softmax"])
def test_router_pin_rejects_planted_mistakes(kind):
    with pytest.raises(AssertionError):
        _check_router(_router_mutant(kind), 11, 0.5)


# ---------------------------------------------------------------- expert
def _expert_case(seed: int, R=3, H=256, I=128):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(R, H, generator=g) * 2
    xq, xs = codecs.fp8_block_quant(x)
    w13 = codecs.e4m3_encode(torch.randn(2 * I, H, generator=g).clamp(-448, 448))
    w2 = codecs.e4m3_encode(torch.randn(H, I, generator=g).clamp(-448, 448))
    s13 = (torch.rand(2 * I // 128, H // 128, generator=g) + 0.5) / 16
    s2 = (torch.rand(H // 128, I // 128, generator=g) + 0.5) / 16
    return xq, xs, w13, s13, w2, s2, I


def _block_gemv_fp64(xq, xs, wq, ws):
    """row r, output n: sum over 128-k blocks of (sum_k x w) x act scale x weight scale."""
    xv, wv = codecs.e4m3_decode(xq).double(), codecs.e4m3_decode(wq).double()
    R, K = xv.shape
    N = wv.shape[0]
    out = torch.zeros(R, N, dtype=torch.float64)
    for kb in range(K // 128):
        ks = slice(128 * kb, 128 * kb + 128)
        part = xv[:, ks] @ wv[:, ks].T  # [R, N], exact products
        out += part * xs[:, kb:kb + 1].double() * ws[:, kb].double().repeat_interleave(128)[None, :N]
    return out


def _check_expert(expert, seed: int) -> None:
    xq, xs, w13, s13, w2, s2, I = _expert_case(seed)
    mid, mq, ms, down = expert(xq, xs, w13, s13, w2, s2, I)
    gu = _block_gemv_fp64(xq, xs, w13, s13)
    gate, up = gu[:, :I], gu[:, I:]  # SGLang's fused w13: gate rows first (check_ffn.py:213)
    mid64 = gate / (1.0 + torch.exp(-gate)) * up
    assert torch.allclose(mid.double(), mid64, rtol=1e-5, atol=1e-5 * float(mid64.abs().max())), "mid"
    # the mid's per-128 FP8: scale amax / 448, every value within half an E4M3 step
    blocks = mid64.reshape(mid64.shape[0], -1, 128)
    amax = blocks.abs().amax(-1)
    assert torch.allclose(ms.double(), amax / 448.0, rtol=1e-6), "mid block scales"
    deq = (codecs.e4m3_decode(mq).double().reshape_as(blocks) * ms.double()[..., None]).reshape_as(mid64)
    assert bool(((deq - mid64).abs() <= mid64.abs() * 2.0**-4 + amax.repeat_interleave(128, 1) * 2.0**-9).all()), "mid codes"
    # down on the quantised mid, block by block
    want = _block_gemv_fp64(mq, ms, w2, s2)
    assert torch.allclose(down.double(), want, rtol=1e-5, atol=1e-5 * float(want.abs().max())), "down"


def test_fp8_expert_equals_fp64_loops():
    for seed in (21, 22):
        _check_expert(moe.fp8_expert, seed)


def _expert_mutant(kind: str):
    def f(xq, xs, w13q, s13, w2q, s2, inter):
        gu = moe.fp8_gemv_blocks(xq, xs, w13q, s13)
        g, u = gu[:, :inter], gu[:, inter:]
        if kind == "gate_up_swapped":
            g, u = u, g
        mid = g * torch.sigmoid(g) * u if kind != "silu_on_up" else g * u * torch.sigmoid(u)
        mq, ms = codecs.fp8_block_quant(mid)
        if kind == "mid_scale_dropped":
            ms = torch.ones_like(ms)
        down = moe.fp8_gemv_blocks(mq, ms, w2q, s2)
        return mid, mq, ms, down

    return f


@pytest.mark.parametrize("kind", ["gate_up_swapped", "silu_on_up", "mid_scale_dropped"])
def test_expert_pin_rejects_planted_mistakes(kind):
    with pytest.raises(AssertionError):
        _check_expert(_expert_mutant(kind), 21)


def test_moe_rmsnorm_is_the_pinned_layer_rmsnorm():
    assert moe.rmsnorm is layer.rmsnorm
