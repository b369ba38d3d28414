"""Pins of the oracle's selection rules (oracle/topk.py) against brute force.

Each rule is checked against an independent restatement: Python's sort of
(value, position) pairs, with -0 below +0 and NaN-free inputs, and against the
oracle's second (radix-digit) implementation. The tie-heavy inputs draw values from a
handful of levels, so a wrong tie rule (highest index first, unstable order) fails.
"""

import math
import struct

import numpy as np
import pytest
import torch

from oracle import topk


def _order_key(v: float):
    """Brute-force total order of the reference's radix key: by value, -0 below +0."""
    return (v, math.copysign(1.0, v))


def brute_topk(vals, k):
    """Positions of the top k by (value desc, position asc), ascending positions."""
    n = len(vals)
    if n <= k:
        return list(range(n))
    order = sorted(range(n), key=lambda i: (tuple(-x for x in _order_key(vals[i])), i))
    return sorted(order[:k])


def test_radix_key_orders_like_the_floats():
    vals = [0.0, -0.0, 1.0, -1.0, 1e-40, -1e-40, float("inf"), float("-inf"), 3.5, -3.5, 1e30, -1e30]
    keys = topk.radix_key(np.array(vals, dtype=np.float32))
    by_key = [vals[i] for i in np.argsort(keys, kind="stable")]
    by_val = sorted(vals, key=_order_key)
    assert [struct.pack("f", v) for v in by_key] == [struct.pack("f", v) for v in by_val]
    # known answers: +0 -> 0x80000000, -0 -> 0x7fffffff, 1.0 -> 0xbf800000
    assert topk.radix_key(np.array([0.0, -0.0, 1.0], dtype=np.float32)).tolist() == [
        0x80000000, 0x7FFFFFFF, 0xBF800000]


@pytest.mark.parametrize("n,k,levels,seed", [
    (300, 64, 5, 0), (300, 64, 300, 1), (64, 64, 3, 2), (10, 64, 3, 3), (65, 64, 2, 4),
    (5000, 2048, 7, 5), (5000, 2048, 5000, 6), (2049, 2048, 1, 7),
])
def test_exact_topk_equals_brute_force_and_radix_select(n, k, levels, seed):
    rng = np.random.default_rng(seed)
    pool = rng.standard_normal(levels).astype(np.float32)
    pool[0] = 0.0
    if levels > 2:
        pool[1] = -0.0
    vals = pool[rng.integers(0, levels, n)]
    want = brute_topk([float(v) for v in vals], k)
    got = topk.exact_topk(vals, k)
    assert got.tolist() == want
    assert topk.radix_select(vals, k).tolist() == want
    assert len(got) == min(n, k)


def test_exact_topk_ties_go_to_lowest_positions():
    vals = np.zeros(10, dtype=np.float32)
    vals[7] = 1.0
    assert topk.exact_topk(vals, 4).tolist() == [0, 1, 2, 7]
    vals = np.full(3000, 2.5, dtype=np.float32)
    assert topk.exact_topk(vals, 2048).tolist() == list(range(2048))


def test_router_top8_rule_and_weights():
    torch.manual_seed(0)
    scores = torch.sigmoid(torch.randn(3, 256))
    bias = torch.randn(256) * 0.1
    # row 1: ten experts tie exactly on score + bias
    scores[1, 40:50] = 0.9
    bias[40:50] = 0.25
    ids, w = topk.router_top8(scores, bias, 8, 2.5)
    for s in range(3):
        key = (scores[s] + bias).tolist()  # f32 addition, as the device does it
        want = sorted(range(256), key=lambda e: (-key[e], e))[:8]
        assert ids[s].tolist() == want
        raw = scores[s, ids[s]].double()
        torch.testing.assert_close(w[s].double(), raw / raw.sum() * 2.5, rtol=1e-6, atol=0)
    assert ids[1].tolist() == list(range(40, 48))
    torch.testing.assert_close(w.sum(-1), torch.full((3,), 2.5), rtol=1e-6, atol=0)


def test_softmax_topk_is_renormalised_softmax():
    torch.manual_seed(1)
    logits = torch.randn(4, 256)
    logits[2, 10:20] = 10.0  # exact ties, above every N(0, 1) logit
    ids, w = topk.softmax_topk(logits, 8)
    assert ids[2].tolist() == list(range(10, 18))
    full = torch.softmax(logits.double(), -1)
    for s in range(4):
        want = sorted(range(256), key=lambda e: (-float(logits[s, e]), e))[:8]
        assert ids[s].tolist() == want
        p = full[s, ids[s]]
        torch.testing.assert_close(w[s].double(), p / p.sum(), rtol=1e-6, atol=1e-7)
