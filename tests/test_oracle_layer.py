"""Pins of the projection phases' CPU restatement (oracle/layer.py) against what the
mathematics fixes, each chosen so a plausible slip (a transposed operand, a swapped
RoPE sign, a wrong Hadamard order, a misplaced scale row, a wrong cache index) fails:

* Walsh-Hadamard against scipy's Sylvester matrix, and its involution;
* RoPE against complex multiplication by e^{i theta}, angle additivity and norm;
* RMSNorm / LayerNorm against fp64 textbook forms;
* the power-of-two FP8 row scale on known answers;
* block dequantisation with a partial last row block;
* the absorbed query against the unabsorbed q_nope . (W_UK^T c) it replaces;
* the cache writer against the attention phase's reader (oracle.attention.index_keys);
* the whole front on tiny shapes against an fp64 re-derivation of each output;
* the index query (W_iq rows h*128 + d, RoPE on dims [0, 64), Hadamard, FP4) against
  an fp64 re-derivation, and the index score's dependence on the position difference
  alone (query and key rotated on the same dims), each shown to reject a planted slip
  (the query rotated on [64, 128), the Hadamard dropped, heads and dims transposed).
"""

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import attention as oattn
from oracle import codecs
from oracle import layer as ol


def test_fwht_matches_sylvester_matrix_and_is_an_involution():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 128, generator=g)
    H = torch.from_numpy(scipy.linalg.hadamard(128).astype(np.float64))
    ref = (x.double() @ H.T) / np.sqrt(128.0)
    assert torch.allclose(ol.fwht(x).double(), ref, atol=1e-5)
    assert torch.allclose(ol.fwht(ol.fwht(x)), x, atol=1e-5)
    # a single impulse at index j spreads as row j of H / sqrt(n)
    e = torch.zeros(128)
    e[37] = 1.0
    assert torch.allclose(ol.fwht(e).double(), H[37] / np.sqrt(128.0), atol=1e-7)


def test_rope_pairs_is_complex_rotation():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 64, generator=g)
    cos, sin = ol.rope_tables(4096)
    pos = torch.tensor([0, 17, 4095])
    y = ol.rope_pairs(x, cos[pos], sin[pos])
    z = torch.complex(x[:, 0::2].double(), x[:, 1::2].double())
    inv = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    rot = torch.polar(torch.ones(3, 32, dtype=torch.float64), pos[:, None].double() * inv[None])
    want = z * rot
    assert torch.allclose(y[:, 0::2].double(), want.real, atol=1e-5)
    assert torch.allclose(y[:, 1::2].double(), want.imag, atol=1e-5)
    # position 0 is the identity; every pair keeps its norm
    assert torch.allclose(y[0], x[0], atol=0)
    assert torch.allclose(y.reshape(3, 32, 2).norm(dim=-1), x.reshape(3, 32, 2).norm(dim=-1), atol=1e-5)
    # angle additivity: rotating by a then b equals rotating by a + b
    a, b = 100, 23
    yab = ol.rope_pairs(ol.rope_pairs(x, cos[a], sin[a]), cos[b], sin[b])
    assert torch.allclose(yab, ol.rope_pairs(x, cos[a + b], sin[a + b]), atol=1e-4)


def test_norms_match_fp64_textbook():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 512, generator=g) * 3 + 0.5
    gamma = torch.rand(512, generator=g) + 0.5
    beta = torch.randn(512, generator=g)
    xd = x.double()
    rms = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + ol.EPS) * gamma.double()
    assert torch.allclose(ol.rmsnorm(x, gamma).double(), rms, rtol=1e-5, atol=1e-6)
    mu = xd.mean(-1, keepdim=True)
    ln = (xd - mu) / torch.sqrt(((xd - mu) ** 2).mean(-1, keepdim=True) + ol.INDEX_LN_EPS) * gamma.double() + beta.double()
    assert torch.allclose(ol.layernorm(x, gamma, beta).double(), ln, rtol=1e-5, atol=1e-5)
    # with unit weight and zero bias: zero mean and unit variance
    y = ol.layernorm(x, torch.ones(512), torch.zeros(512)).double()
    assert torch.allclose(y.mean(-1), torch.zeros(4, dtype=torch.float64), atol=1e-5)
    assert torch.allclose(y.var(-1, unbiased=False), torch.ones(4, dtype=torch.float64), atol=1e-4)


def test_fp8_row_quant_pow2_known_answers():
    rows = torch.tensor([
        [448.0, -1.0, 0.5],      # amax 448 -> scale 1, codes exact
        [449.0, 0.0, 0.0],       # just above -> scale 2
        [0.0, 0.0, 0.0],         # all zero -> amax clamps to 1e-4 -> 2^-22
        [3.5, -7.0, 1.75],       # amax 7: 7/448 = 2^-6 exactly -> scale 2^-6
    ])  # fmt: skip
    codes, scale = ol.fp8_row_quant_pow2(rows)
    assert scale.tolist() == [1.0, 2.0, 2.0**-22, 2.0**-6]
    dec = codecs.e4m3_decode(codes) * scale[:, None]
    assert dec[0].tolist() == [448.0, -1.0, 0.5]
    assert dec[1].tolist() == [448.0, 0.0, 0.0]  # 449 / 2 = 224.5 rounds to 224 (even)
    assert dec[3].tolist() == [3.5, -7.0, 1.75]
    # no code exceeds 448 in magnitude and the relative error stays within E4M3's half ulp
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 576, generator=g) * torch.rand(64, 1, generator=g) * 50
    c, s = ol.fp8_row_quant_pow2(x)
    d = codecs.e4m3_decode(c) * s[:, None]
    assert float(codecs.e4m3_decode(c).abs().max()) <= 448.0
    big = x.abs() > s[:, None] * 2.0**-6 * 8  # normal range of the scaled E4M3
    assert float(((d - x).abs() / x.abs())[big].max()) <= 2.0**-4 + 1e-6


def test_block_dequant_partial_last_block():
    codes = torch.full((200, 256), 0x38, dtype=torch.uint8)  # E4M3 0x38 = 1.0
    scales = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    w = ol.block_dequant(codes, scales)
    assert w.shape == (200, 256)
    assert w[0, 0] == 1.0 and w[127, 255] == 2.0 and w[128, 0] == 3.0 and w[199, 200] == 4.0


def _layer_weights():
    """Projection weights of the real shapes (the oracle hard-codes them), unshuffled."""
    from sgl_amd_mono_amd import workloads

    w = workloads.proj_weights("cpu", seed=5)
    out = {}
    for name in ol_weight_names():
        t = getattr(w, name)
        if name.startswith("w_") and name != "w_iw":
            t = codecs.aiter_unshuffle(t)
        elif name == "w_iw":
            t = codecs.aiter_unshuffle(t.view(torch.uint8)).view(torch.bfloat16)
        out[name] = t
    return out


def ol_weight_names():
    from sgl_amd_mono_amd.layer import WEIGHT_SPECS

    return list(WEIGHT_SPECS)


@pytest.fixture(scope="module")
def front_case():
    g = torch.Generator().manual_seed(7)
    w = _layer_weights()
    S, pages = 3, 6
    h = torch.randn(S, ol.HIDDEN, generator=g).to(torch.bfloat16)
    page_table = torch.tensor([[4, 1, 0], [2, 5, 0], [3, 0, 0]], dtype=torch.int32)
    pos = torch.tensor([70, 5, 63])
    cos, sin = ol.rope_tables(256)
    return w, h, pos, page_table, cos, sin, pages


def test_absorbed_query_equals_unabsorbed_scores(front_case):
    """q_lat . c == q_nope . (W_UK^T c) for a latent row c: the absorption identity
    fixes which operand of W_UK is contracted (a transposed W_UK fails it)."""
    w, h, pos, pt, cos, sin, _ = front_case
    f = ol.front(h, pos, pt, w, cos, sin)
    wuk = ol.block_dequant(w["w_uk"], w["s_uk"]).double().reshape(ol.HEADS, ol.KV_LORA, ol.NOPE_DIM)
    c = torch.randn(ol.KV_LORA, generator=torch.Generator().manual_seed(9)).double()
    k_nope = torch.einsum("hcd,c->hd", wuk, c)  # the un-absorbed key of latent c, per head
    direct = (f["q_nope"].double() * k_nope[None]).sum(-1)  # [S, heads]
    absorbed = f["q_lat"].double() @ c
    assert torch.allclose(absorbed, direct, rtol=2e-2, atol=2e-2 * float(direct.abs().mean()))


def test_front_outputs_against_fp64_rederivation(front_case):
    """Each front output re-derived in fp64 from the same weights (the bf16 roundings
    the restatement applies are the only difference)."""
    w, h, pos, pt, cos, sin, _ = front_case
    f = ol.front(h, pos, pt, w, cos, sin)
    hd = h.double()
    x = hd / torch.sqrt((hd * hd).mean(-1, keepdim=True) + ol.EPS) * w["g_in"].double()
    qkv = x @ ol.block_dequant(w["w_qkv"], w["s_qkv"]).double().T
    assert torch.allclose(f["q_a"].double(), qkv[:, : ol.Q_LORA], rtol=2e-2, atol=2e-2)
    qa = qkv[:, : ol.Q_LORA]
    qan = qa / torch.sqrt((qa * qa).mean(-1, keepdim=True) + ol.EPS) * w["g_q"].double()
    qb = (qan @ ol.block_dequant(w["w_qb"], w["s_qb"]).double().T).reshape(-1, ol.HEADS, ol.QK_DIM)
    assert torch.allclose(f["q_nope"].double(), qb[..., : ol.NOPE_DIM], rtol=3e-2, atol=3e-2)
    # q_pe: rotate the fp64 pe dims by the row's position, as complex numbers
    pe = qb[..., ol.NOPE_DIM:]
    z = torch.complex(pe[..., 0::2], pe[..., 1::2])
    inv = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    rot = torch.polar(torch.ones(len(pos), 1, 32, dtype=torch.float64), pos[:, None, None].double() * inv)
    zr = z * rot
    assert torch.allclose(f["q_pe"][..., 0::2].double(), zr.real, rtol=3e-2, atol=3e-2)
    assert torch.allclose(f["q_pe"][..., 1::2].double(), zr.imag, rtol=3e-2, atol=3e-2)
    # the q output is q_lat | q_pe
    assert torch.equal(f["q"][..., : ol.KV_LORA].float(), f["q_lat"])
    assert torch.equal(f["q"][..., ol.KV_LORA:].float(), f["q_pe"])
    # index head weights
    iw = (x @ w["w_iw"].double().T) * (128.0**-0.5 * 64.0**-0.5)
    assert torch.allclose(f["iw"].double(), iw, rtol=2e-2, atol=1e-4)


def test_cache_rows_read_back_through_the_attention_reader(front_case):
    """The rows front writes, read back by oracle.attention's cache readers, are the
    FP4 / FP8 round trips of the fp64 key and KV row at the row's position."""
    w, h, pos, pt, cos, sin, pages = front_case
    f = ol.front(h, pos, pt, w, cos, sin)
    ikv = torch.zeros(pages, 4, 64, 16, dtype=torch.uint8)
    iks = torch.zeros(pages, 4, 64, dtype=torch.uint8)
    kv = torch.zeros(pages * 64, 576, dtype=torch.uint8)
    kvs = torch.zeros(pages * 64)
    ol.write_caches(f, ikv, iks, kv, kvs)
    assert f["slot"].tolist() == [1 * 64 + 6, 2 * 64 + 5, 3 * 64 + 63]
    for s in range(len(pos)):
        n = int(pos[s]) + 1
        keys = oattn.index_keys(ikv, iks, pt[s], n)  # [n, 128]
        got = keys[n - 1]
        # fp64 index key: LayerNorm, RoPE on [0, 64), Hadamard
        k = f["ik"][s].double()
        kn = (k - k.mean()) / torch.sqrt(((k - k.mean()) ** 2).mean() + 1e-6) * w["g_ik"].double() + w["b_ik"].double()
        z = torch.complex(kn[0:64:2], kn[1:64:2])
        inv = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
        zr = z * torch.polar(torch.ones(32, dtype=torch.float64), pos[s].double() * inv)
        kr = kn.clone()
        kr[0:64:2], kr[1:64:2] = zr.real, zr.imag
        H = torch.from_numpy(scipy.linalg.hadamard(128).astype(np.float64)) / np.sqrt(128.0)
        want = H @ kr
        # FP4 keeps a value within half a code step (at most 1 x the block scale, between
        # the codes 4 and 6), plus the two bf16 roundings of values up to 6 x the scale
        blk_scale = codecs.e8m0_decode(f["iks"][s]).double().repeat_interleave(32)
        assert float(((got.double() - want).abs() / blk_scale).max()) < 1.0 + 12 * 2.0**-9
        rows = oattn.kv_rows(kv, kvs, torch.tensor([int(f["slot"][s])]))[0]
        kvn = f["kv_a"][s, :512].double()
        kvn = kvn / torch.sqrt((kvn * kvn).mean() + ol.EPS) * w["g_kv"].double()
        assert torch.allclose(rows[:512].double(), kvn, rtol=0.07, atol=float(kvs[f["slot"][s]]) * 2)
    # nothing else was written
    written = set(f["slot"].tolist())
    for sl in range(pages * 64):
        if sl not in written:
            assert int(kv[sl].abs().sum()) == 0 and float(kvs[sl]) == 0.0


def test_back_is_residual_plus_two_projections():
    g = torch.Generator().manual_seed(11)
    w = _layer_weights()
    S = 2
    o_lat = torch.randn(S, ol.HEADS, ol.KV_LORA, generator=g).to(torch.bfloat16)
    h = torch.randn(S, ol.HIDDEN, generator=g).to(torch.bfloat16)
    b = ol.back(o_lat, h, w)
    wuv = ol.block_dequant(w["w_uv"], w["s_uv"]).double().reshape(ol.HEADS, ol.V_DIM, ol.KV_LORA)
    o = torch.einsum("hvc,shc->shv", wuv, o_lat.double()).reshape(S, -1)
    assert torch.allclose(b["o"].double(), o, rtol=1e-2, atol=1e-2)
    y = o @ ol.block_dequant(w["w_o"], w["s_o"]).double().T
    assert torch.allclose(b["a"].double(), h.double() + y, rtol=2e-2, atol=5e-2)
    # zero attention output leaves the residual stream unchanged
    z = ol.back(torch.zeros_like(o_lat), h, w)
    assert torch.equal(z["a"], h)


def test_raw_e4m3_mla_row_is_unscaled_and_clamped():
    """SGLang's scale-less MLA row: every E4M3 value codes itself (scale 1) and values
    past the format's range clamp to +-448 (the largest finite E4M3)."""
    from oracle import codecs

    row = torch.tensor([[0.0, 1.0, -2.5, 448.0, 1000.0, -3000.0, 0.0625, 2.0**-9]])
    codes, scale = ol.fp8_row_quant_pow2(row, scaled=False)
    assert scale.tolist() == [1.0]
    assert codecs.e4m3_decode(codes).tolist() == [[0.0, 1.0, -2.5, 448.0, 448.0, -448.0, 0.0625, 2.0**-9]]
    # the scaled row of the same values is a power of two times codes within range
    codes2, scale2 = ol.fp8_row_quant_pow2(row)
    assert float(scale2) == 8.0 and bool((codecs.e4m3_decode(codes2).abs() <= 448).all())


# ---------------------------------------------------------------- index query / key
def _bf16_64(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).double()


def _iq_fp64(q_an, w_iq, s_iq, pos):
    """The index query re-derived in fp64 with the restatement's bf16 rounding points:
    rows h*128 + d of W_iq (row-major, read by explicit row slices) on q_an, bf16; the
    complex rotation of each head's dims [0, 64) by the row's position, bf16; the
    Sylvester Hadamard matrix / sqrt(128), bf16. Returns [S, 64, 128] float64."""
    W = ol.block_dequant(w_iq, s_iq).double()
    S = q_an.shape[0]
    out = torch.zeros(S, ol.INDEX_HEADS, ol.INDEX_DIM, dtype=torch.float64)
    H = torch.from_numpy(scipy.linalg.hadamard(128).astype(np.float64)) / np.sqrt(128.0)
    inv = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    for s in range(S):
        for h in range(ol.INDEX_HEADS):
            v = _bf16_64(W[h * 128 : (h + 1) * 128] @ q_an[s].double())
            z = torch.complex(v[0:64:2], v[1:64:2]) * torch.polar(torch.ones(32, dtype=torch.float64), float(pos[s]) * inv)
            r = v.clone()
            r[0:64:2], r[1:64:2] = z.real, z.imag
            out[s, h] = _bf16_64(H @ _bf16_64(r))
    return out


def _check_iq_against_fp64(codes, e8, q_an, w, pos):
    """FP4 codes / E8M0 scales of an index query against the fp64 re-derivation: each
    block's scale byte is pow2_ceil(max(amax, 6 * 2^-126) / 6) of the fp64 block (one
    step off only where amax / 6 sits within 1e-3 of a power of two), and every decoded
    value lies within one scale unit of the fp64 value (the widest half gap of E2M1,
    between 4 and 6, plus the bf16 roundings)."""
    want = _iq_fp64(q_an, w["w_iq"], w["s_iq"], pos)
    blocks = want.reshape(*want.shape[:-1], 4, 32)
    amax = blocks.abs().amax(-1).clamp_min(6.0 * 2.0**-126) / 6.0
    code = torch.ceil(torch.log2(amax)) + 127
    frac = torch.log2(amax) - torch.round(torch.log2(amax))
    e8 = e8.reshape(code.shape).double()
    near = frac.abs() < 1e-3
    assert bool(((e8 == code) | (near & ((e8 - code).abs() <= 1))).all()), "index-query scale bytes"
    dec = codecs.e2m1_decode_codes(codes.reshape(want.shape)).double()
    scale = torch.exp2(e8 - 127).repeat_interleave(32, -1)
    assert float(((dec * scale - want).abs() / scale).max()) < 1.0 + 12 * 2.0**-9, "index-query values"


def _check_relative_position(index_query, index_key, w, seed=21):
    """RoPE on the same dims of query and key plus one orthogonal Hadamard on both make
    the index score q . k (before FP4) a function of the position difference alone:
    shifting the query's and the key's positions by the same delta keeps every
    head's q . k to within the bf16 roundings, while moving the query alone does not."""
    g = torch.Generator().manual_seed(seed)
    q_an = torch.randn(2, ol.Q_LORA, generator=g).to(torch.bfloat16)
    ik = torch.randn(3, ol.INDEX_DIM, generator=g) * 2
    cos, sin = ol.rope_tables(4096)
    m, n = torch.tensor([70, 900]), torch.tensor([5, 2000, 640])

    def dots(dm, dn):
        qh = index_query(q_an, w["w_iq"], w["s_iq"], cos[m + dm], sin[m + dm])[3].double()
        kh = index_key(ik, w["g_ik"], w["b_ik"], cos[n + dn], sin[n + dn])[3].double()
        d = torch.einsum("shd,td->sht", qh, kh)
        return d / (qh.norm(dim=-1)[..., None] * kh.norm(dim=-1)[None, None])

    # cosines of random 128-dim vectors are ~0.09 rms; the bf16 roundings move them by
    # ~1.5e-3 at most, a query rotated on other dims than the key by ~0.09 and more
    base = dots(0, 0)
    for delta in (1, 37, 1000):
        assert float((dots(delta, delta) - base).abs().max()) < 0.01, f"shift {delta}"
    assert float((dots(37, 0) - base).abs().max()) > 0.1  # the check can see a rotation


def test_index_query_against_fp64_rederivation(front_case):
    w, h, pos, pt, cos, sin, _ = front_case
    f = ol.front(h, pos, pt, w, cos, sin)
    codes = torch.stack([f["iq"] & 15, f["iq"] >> 4], -1).flatten(-2)
    _check_iq_against_fp64(codes, f["iqs"], f["q_an"], w, pos)


def test_index_score_depends_on_position_difference_only():
    _check_relative_position(ol.index_query, ol.index_key, _layer_weights())


def _mutant_index_query(kind: str):
    """``layer.index_query`` with one plausible slip planted."""

    def f(q_an, w_iq, s_iq, c, s):
        S = q_an.shape[0]
        raw = codecs.bf16_round(ol.gemv(q_an, w_iq, s_iq))
        if kind == "heads_dims_transposed":
            raw = raw.reshape(S, ol.INDEX_DIM, ol.INDEX_HEADS).transpose(1, 2)
        raw = raw.reshape(S, ol.INDEX_HEADS, ol.INDEX_DIM)
        lo, hi = raw[..., : ol.PE_DIM], raw[..., ol.PE_DIM :]
        if kind == "rope_high_dims":
            rot = torch.cat([lo, ol.rope_pairs(hi, c[:, None], s[:, None])], -1)
        else:
            rot = torch.cat([ol.rope_pairs(lo, c[:, None], s[:, None]), hi], -1)
        hv = codecs.bf16_round(rot)
        if kind != "no_hadamard":
            hv = codecs.bf16_round(ol.fwht(hv))
        codes, e8, deq = codecs.fp4_block_quant(hv)
        return codes, e8, deq, hv

    return f


@pytest.mark.parametrize("kind", ["rope_high_dims", "no_hadamard", "heads_dims_transposed"])
def test_index_query_pins_reject_planted_mistakes(front_case, kind):
    w, h, pos, pt, cos, sin, _ = front_case
    mutant = _mutant_index_query(kind)
    f = ol.front(h, pos, pt, w, cos, sin)
    codes, e8, _, _ = mutant(f["q_an"], w["w_iq"], w["s_iq"], cos[pos], sin[pos])
    with pytest.raises(AssertionError):
        _check_iq_against_fp64(codes, e8, f["q_an"], w, pos)
    if kind != "heads_dims_transposed":  # a transposed reshape still rotates matching dims
        with pytest.raises(AssertionError):
            _check_relative_position(mutant, ol.index_key, w)
    # the unmutated restatement passes the same checks
    codes, e8, _, _ = ol.index_query(f["q_an"], w["w_iq"], w["s_iq"], cos[pos], sin[pos])
    _check_iq_against_fp64(codes, e8, f["q_an"], w, pos)
