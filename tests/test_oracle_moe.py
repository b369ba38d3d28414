"""Pins of the oracle's MoE blocks (oracle/moe.py) against closed forms.

* The block-scaled FP8 GEMV against a float64 matmul of weights and rows expanded
  block by block in an explicit loop (a transposed or shifted scale index fails).
* The toy MoE against a dense restatement: every expert on every
  row, combined through a dense [rows, experts] routing matrix.
* The FP8 and MXFP4 blocks with every expert identical: the output must be
  (sum of route weights + 1 for the shared expert) x one expert's output.
"""

import numpy as np
import torch

from oracle import codecs, moe, topk


def _rand_fp8(shape, g):
    return codecs.e4m3_encode(torch.randn(*shape, generator=g).clamp(-448, 448))


def test_fp8_gemv_blocks_equals_fp64_blockwise_expansion():
    g = torch.Generator().manual_seed(0)
    R, N, K = 3, 256, 384
    xq, wq = _rand_fp8((R, K), g), _rand_fp8((N, K), g)
    xs = torch.rand(R, K // 128, generator=g) + 0.5
    ws = torch.rand(N // 128, K // 128, generator=g) + 0.5
    got = moe.fp8_gemv_blocks(xq, xs, wq, ws).double()
    xv, wv = codecs.e4m3_decode(xq).double(), codecs.e4m3_decode(wq).double()
    want = torch.zeros(R, N, dtype=torch.float64)
    for nb in range(N // 128):
        for kb in range(K // 128):
            ks, ns = slice(kb * 128, kb * 128 + 128), slice(nb * 128, nb * 128 + 128)
            want[:, ns] += (xv[:, ks] * xs[:, kb:kb + 1].double()) @ (wv[ns, ks] * float(ws[nb, kb])).T
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_toy_moe_equals_dense_restatement():
    from sgl_amd_mono_amd import workloads

    t = workloads.toy_moe(seed=0)
    ids, w, y = moe.toy_moe(t["x"], t["w_router"], t["w_gate"], t["w_up"], t["w_down"], top_k=2)
    x = t["x"].double()
    logits = x @ t["w_router"].double().T
    E = logits.shape[1]
    dense = torch.zeros(x.shape[0], E, dtype=torch.float64)
    for s in range(x.shape[0]):
        order = sorted(range(E), key=lambda e: (-float(logits[s, e]), e))[:2]
        p = torch.softmax(logits[s, order], -1)
        dense[s, order] = p
    out = torch.zeros(x.shape[0], t["w_down"].shape[1], dtype=torch.float64)
    for e in range(E):
        gt = x @ t["w_gate"][e].double().T
        up = x @ t["w_up"][e].double().T
        out += dense[:, e:e + 1] * ((gt * torch.sigmoid(gt) * up) @ t["w_down"][e].double().T)
    torch.testing.assert_close(w.double().sum(-1), torch.ones(x.shape[0], dtype=torch.float64), rtol=1e-6, atol=0)
    torch.testing.assert_close(y.double(), out, rtol=2e-4, atol=2e-5)


def test_fp8_moe_block_identical_experts_closed_form():
    g = torch.Generator().manual_seed(2)
    S, H, E, I = 3, 256, 16, 128
    a = torch.randn(S, H, generator=g).to(torch.bfloat16)
    g_post = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    w_router = (torch.randn(E, H, generator=g) * 0.1).to(torch.bfloat16)
    bias = torch.randn(E, generator=g) * 0.1
    w13_1, w2_1 = _rand_fp8((2 * I, H), g), _rand_fp8((H, I), g)
    s13_1 = (torch.rand(2 * I // 128, H // 128, generator=g) + 0.5) / 448
    s2_1 = (torch.rand(H // 128, I // 128, generator=g) + 0.5) / 448
    rep = lambda t: t.unsqueeze(0).repeat(E + 1, *[1] * t.dim())  # noqa: E731
    r = moe.fp8_moe_block(a, g_post, w_router, bias, rep(w13_1), rep(s13_1), rep(w2_1), rep(s2_1),
                          eps=1e-6, top_k=4, inter=I)
    _, _, _, down = moe.fp8_expert(r["xq"], r["xs"], w13_1, s13_1, w2_1, s2_1, I)
    want = (r["weights"].sum(-1, keepdim=True) + 1.0) * down
    torch.testing.assert_close(r["y"], want, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(r["weights"].sum(-1), torch.full((S,), 2.5), rtol=1e-6, atol=0)
    # the router's picks follow the rule on its own scores
    ids, _ = topk.router_top8(r["scores"], bias, 4)
    assert torch.equal(ids, r["ids"])


def test_mxfp4_dequant_closed_form():
    g = torch.Generator().manual_seed(3)
    packed = torch.randint(0, 256, (4, 32), dtype=torch.uint8, generator=g)
    scales = torch.randint(115, 135, (4, 2), dtype=torch.uint8, generator=g)
    got = codecs.mxfp4_dequant(packed, scales)
    p, sc = packed.numpy(), scales.numpy()
    for n in range(4):
        for k in range(64):
            code = (p[n, k // 2] >> (4 * (k % 2))) & 15
            mag = [0, 0.5, 1, 1.5, 2, 3, 4, 6][code & 7] * (-1 if code & 8 else 1)
            assert float(got[n, k]) == mag * 2.0 ** (int(sc[n, k // 32]) - 127)


def test_mxfp4_moe_block_identical_experts_closed_form():
    g = torch.Generator().manual_seed(4)
    S, H, E, I = 2, 256, 16, 128
    x = torch.randn(S, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(S, E, generator=g)
    u8 = dict(dtype=torch.uint8, generator=g)
    w13 = torch.randint(0, 256, (2 * I, H // 2), **u8)
    s13 = torch.randint(119, 123, (2 * I, H // 32), **u8)
    w2 = torch.randint(0, 256, (H, I // 2), **u8)
    s2 = torch.randint(119, 123, (H, I // 32), **u8)
    rep = lambda t: t.unsqueeze(0).repeat(E + 1, 1, 1)  # noqa: E731
    r = moe.mxfp4_moe_block(x, logits, rep(w13), rep(s13), rep(w2), rep(s2), top_k=4, inter=I)
    # one expert in float64 from the closed-form dequantisation
    w13d = codecs.mxfp4_dequant(w13, s13).double()
    w2d = codecs.mxfp4_dequant(w2, s2).double()
    gu = x.double() @ w13d.T
    mid = codecs.bf16_round((gu[:, :I] * torch.sigmoid(gu[:, :I]) * gu[:, I:]).float()).double()
    want = 2.0 * (mid @ w2d.T)  # softmax weights sum to 1, plus the shared expert
    torch.testing.assert_close(r["y"].double(), want, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(r["weights"].sum(-1).numpy(), 1.0, rtol=1e-6)
