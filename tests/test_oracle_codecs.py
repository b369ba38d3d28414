"""Pins of the oracle's number formats against closed forms and known answers."""

import math

import numpy as np
import pytest
import torch

from oracle import codecs


def e4m3_closed_form(c: int) -> float:
    """OCP E4M3FN: bias 7, no infinities, S.1111.111 is NaN."""
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    if e == 15 and m == 7:
        return float("nan")
    v = (m / 8.0) * 2.0**-6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
    return -v if s else v


def test_e4m3_decode_all_codes():
    got = codecs.e4m3_decode(torch.arange(256, dtype=torch.uint8)).double().numpy()
    want = np.array([e4m3_closed_form(c) for c in range(256)])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])


def test_e4m3_known_answers():
    vals = codecs.e4m3_decode(torch.tensor([0x38, 0x7E, 0x01, 0xB8, 0x08], dtype=torch.uint8))
    assert vals.tolist() == [1.0, 448.0, 2.0**-9, -1.0, 2.0**-6]


def test_e4m3_encode_round_trip_and_ties_to_even():
    codes = torch.tensor([c for c in range(256) if not math.isnan(e4m3_closed_form(c))], dtype=torch.uint8)
    back = codecs.e4m3_encode(codecs.e4m3_decode(codes))
    # -0 may come back as +0's code; every other code is its own round trip
    same = (back == codes) | ((codes == 0x80) & (back == 0x00))
    assert bool(same.all())
    # 1 + 1/16 sits halfway between 1 (mantissa 0, even) and 1.125 (mantissa 1)
    assert codecs.e4m3_decode(codecs.e4m3_encode(torch.tensor([1.0625]))).item() == 1.0
    # 1.1875 is halfway between 1.125 (odd) and 1.25 (even)
    assert codecs.e4m3_decode(codecs.e4m3_encode(torch.tensor([1.1875]))).item() == 1.25
    with pytest.raises(ValueError):
        codecs.e4m3_encode(torch.tensor([500.0]))


def e2m1_closed_form(c: int) -> float:
    s, e, m = c >> 3, (c >> 1) & 3, c & 1
    v = m * 0.5 if e == 0 else (1 + m / 2.0) * 2.0 ** (e - 1)
    return -v if s else v


def test_e2m1_table_is_the_closed_form():
    assert codecs.E2M1 == [e2m1_closed_form(c) for c in range(16)]
    packed = torch.tensor([0x21, 0xF7], dtype=torch.uint8)  # (1: 0.5, 2: 1.0), (7: 6.0, 15: -6.0)
    assert codecs.e2m1_decode(packed).tolist() == [0.5, 1.0, 6.0, -6.0]


def test_e2m1_encode_nearest_ties_even():
    grid = torch.tensor(codecs.E2M1[:8])
    assert codecs.e2m1_decode_codes(codecs.e2m1_encode(grid)).tolist() == grid.tolist()
    # midpoints: 0.25 -> 0 (code 0), 0.75 -> 1.0 (code 2), 1.25 -> 1.0, 1.75 -> 2.0,
    # 2.5 -> 2.0 (code 4), 3.5 -> 4.0 (code 6), 5.0 -> 4.0
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -5.0, 0.3])
    want = [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0, -4.0, 0.5]
    assert codecs.e2m1_decode_codes(codecs.e2m1_encode(mids)).tolist() == want
    c = torch.randint(0, 16, (64,), dtype=torch.uint8)
    assert torch.equal(codecs.e2m1_decode(codecs.e2m1_pack(c)), codecs.e2m1_decode_codes(c))


def test_e8m0_and_code_ceil():
    assert codecs.e8m0_decode(torch.tensor([127, 128, 120, 0], dtype=torch.uint8)).tolist() == [
        1.0, 2.0, 2.0**-7, 2.0**-127]
    assert math.isnan(codecs.e8m0_decode(torch.tensor([255], dtype=torch.uint8)).item())
    rng = np.random.default_rng(0)
    v = torch.from_numpy(rng.uniform(1e-6, 1e6, 500).astype(np.float32))
    # x = m * 2^e, m in [0.5, 1): the smallest power of two >= x is 2^(e-1) if m == 0.5
    # else 2^e; biased by 127
    want = [min(max(math.frexp(float(x))[1] - (1 if math.frexp(float(x))[0] == 0.5 else 0) + 127, 1), 254)
            for x in v]
    assert codecs.code_ceil(v).tolist() == want
    # exact powers of two map to themselves
    p = torch.tensor([1.0, 2.0, 0.5, 2.0**-100])
    assert codecs.code_ceil(p).tolist() == [127, 128, 126, 27]


def test_fp8_block_quant_properties():
    torch.manual_seed(0)
    x = torch.randn(3, 512) * torch.tensor([1.0, 1e-3, 50.0])[:, None]
    x[1, 128:256] = 0.0
    q, s = codecs.fp8_block_quant(x)
    assert q.dtype == torch.uint8 and s.shape == (3, 4)
    deq = codecs.fp8_block_dequant(q, s)
    g = x.reshape(3, 4, 128)
    amax = g.abs().amax(-1)
    # zero block: scale 1, zero values; otherwise scale = amax / 448
    assert s[1, 1].item() == 1.0 and bool((deq[1, 128:256] == 0).all())
    nz = amax > 0
    torch.testing.assert_close(s[nz], amax[nz] / 448.0, rtol=1e-6, atol=0)
    # the block's largest magnitude maps to +-448 exactly; every value within half an E4M3 step
    rel = ((deq - x).abs() / (s.repeat_interleave(128, -1) * 448.0)).max().item()
    assert rel <= 2.0**-4 + 1e-6


def test_fp4_block_quant_properties():
    torch.manual_seed(1)
    v = torch.randn(4, 128) * 3.0
    codes, e8, deq = codecs.fp4_block_quant(v)
    sc = codecs.e8m0_decode(e8)
    amax = v.reshape(4, 4, 32).abs().amax(-1)
    # power-of-two scale, the smallest with amax / scale <= 6
    assert bool(((amax / sc) <= 6.0).all()) and bool(((amax / (sc / 2)) > 6.0).all())
    # values already on the scaled grid survive exactly
    grid = codecs.e2m1_decode_codes(torch.randint(0, 16, (2, 64), dtype=torch.uint8))
    grid[:, 0] = 6.0
    grid[:, 32] = -6.0
    _, _, back = codecs.fp4_block_quant(grid * 0.25)
    assert torch.equal(back, grid * 0.25)
    del codes, deq
