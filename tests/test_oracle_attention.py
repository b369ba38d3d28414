"""Pins of the oracle's sparse-attention phase (oracle/attention.py).

* The FP4 index-plane layout by known answer: a key written at a chosen slot must
  decode to its values, with its E8M0 byte at (slot % 16) * 4 + slot // 16
  (test/kernels/test_deepseek_v41_k2i.py:158).
* Index scores against the reference's own fp64 closed form, restated here from
  test/kernels/test_deepseek_v41_k2i.py:149-167 (``ref_logits``): per 32-dim chunk
  scaled dot products, relu of their sum, weighted sum over heads.
* Exact top-k slots through a scattered page table by brute force.
* Sparse MLA against a float64 dense softmax over explicit rows.
"""

import torch

from oracle import attention as att
from oracle import codecs

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
E2M1 += [-v for v in E2M1]


def _unpack64(b):
    lut = torch.tensor(E2M1, dtype=torch.float64)
    return torch.stack([lut[(b & 15).long()], lut[(b >> 4).long()]], -1).flatten(-2)


def fp4_case(n_rows=2, ctx=(300, 150), pages=12, heads=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    u8 = dict(generator=g, dtype=torch.uint8)
    payload = torch.randint(0, 256, (pages, 4, 64, 16), **u8)
    kscale = torch.randint(123, 130, (pages, 4, 64), **u8)
    perm = torch.randperm(pages, generator=g).to(torch.int32)
    ppr = 5
    table = perm[: n_rows * ppr].view(n_rows, ppr).contiguous()
    iq = torch.randint(0, 256, (n_rows, heads, 64), **u8)
    iqs = torch.randint(123, 130, (n_rows, heads, 4), **u8)
    iw = (torch.randn(n_rows, heads, generator=g) * 0.05).to(torch.bfloat16)
    return dict(payload=payload, kscale=kscale, table=table, iq=iq, iqs=iqs, iw=iw,
                seq_lens=torch.tensor(ctx, dtype=torch.int32))


def ref_logits_fp64(c, t, n):
    """fp64 logits of row t over its first n positions, restated after ref_logits."""
    cols = torch.arange(n)
    page = c["table"][t][cols // 64].long()
    slot = cols % 64
    k = _unpack64(c["payload"][page, :, slot, :])  # [n, 4, 32]
    ke = c["kscale"][page[:, None], torch.arange(4)[None], ((slot % 16) * 4 + slot // 16)[:, None]]
    ks = torch.exp2(ke.double() - 127)  # [n, 4]
    q = _unpack64(c["iq"][t].view(-1, 4, 16))  # [h, 4, 32]
    qs = torch.exp2(c["iqs"][t].double() - 127)  # [h, 4]
    s = torch.einsum("hcd,ncd->hnc", q, k) * qs[:, None, :] * ks[None]
    return (c["iw"][t].double()[:, None] * s.sum(-1).clamp_min(0)).sum(0)


def test_index_plane_layout_known_answer():
    payload = torch.zeros(3, 4, 64, 16, dtype=torch.uint8)
    kscale = torch.full((3, 4, 64), 127, dtype=torch.uint8)
    # logical position 64 + 37 -> page table entry 1 -> physical page 2, slot 37
    table = torch.tensor([0, 2], dtype=torch.int32)
    codes = torch.arange(128) % 16
    payload[2, :, 37, :] = codecs.e2m1_pack(codes.to(torch.uint8)).view(4, 16)
    for c in range(4):
        kscale[2, c, (37 % 16) * 4 + 37 // 16] = 127 + c
    keys = att.index_keys(payload, kscale, table, 64 + 38)
    want = torch.tensor([E2M1[int(v)] for v in codes]).view(4, 32) * torch.tensor([1.0, 2, 4, 8])[:, None]
    assert torch.equal(keys[101], want.flatten())
    assert bool((keys[:64] == 0).all()) and bool((keys[64:101] == 0).all())


def test_index_scores_match_reference_closed_form():
    c = fp4_case()
    n_max = 320
    got = att.index_scores(c["iq"], c["iqs"], c["iw"], c["payload"], c["kscale"], c["table"],
                           c["seq_lens"], n_max)
    for t in range(2):
        n = int(c["seq_lens"][t])
        want = ref_logits_fp64(c, t, n)
        torch.testing.assert_close(got[t, :n].double(), want, rtol=1e-5, atol=1e-5)
        assert bool((got[t, n:] == 0).all())
        f64 = att.index_scores_fp64(c["iq"][t], c["iqs"][t], c["iw"][t], c["payload"], c["kscale"],
                                    c["table"][t], n)
        torch.testing.assert_close(f64, want, rtol=1e-12, atol=1e-12)


def test_select_topk_maps_positions_through_the_page_table():
    scores = torch.zeros(2, 200)
    scores[0, [5, 70, 199]] = torch.tensor([3.0, 2.0, 1.0])
    scores[1, :3] = torch.tensor([1.0, 1.0, 1.0])  # ties: lowest positions win
    table = torch.tensor([[7, 2, 9, 4], [1, 0, 3, 5]], dtype=torch.int32)
    sel = att.select_topk(scores, torch.tensor([200, 150]), table, k=3)
    assert sel[0].tolist() == [7 * 64 + 5, 2 * 64 + 6, 4 * 64 + 7]
    assert sel[1].tolist() == [64, 65, 66]
    short = att.select_topk(scores, torch.tensor([2, 1]), table, k=3)
    assert short.tolist() == [[7 * 64, 7 * 64 + 1, -1], [64, -1, -1]]


def test_sparse_mla_matches_fp64_dense_softmax():
    g = torch.Generator().manual_seed(5)
    slots = 300
    kv = codecs.e4m3_encode((torch.randn(slots, 576, generator=g) * 4).clamp(-448, 448))
    kv_scale = torch.rand(slots, generator=g) * 0.1 + 0.01
    q = torch.randn(2, 4, 576, generator=g).to(torch.bfloat16)
    sel = torch.full((2, 16), -1, dtype=torch.int32)
    sel[0] = torch.randperm(slots, generator=g)[:16].to(torch.int32)
    sel[1, :5] = torch.tensor([3, 1, 4, 159, 26], dtype=torch.int32)
    got = att.sparse_mla(q, kv, kv_scale, sel)
    for s in range(2):
        idx = sel[s][sel[s] >= 0].long()
        rows = codecs.e4m3_decode(kv[idx]).double() * kv_scale[idx].double()[:, None]
        want = att.sparse_mla_fp64(q[s], rows)
        # independent restatement: explicit logits, max-subtracted exponentials
        lg = (q[s].double() @ rows.T) * (192 ** -0.5)
        p = torch.exp(lg - lg.max(-1, keepdim=True).values)
        ref = (p / p.sum(-1, keepdim=True)) @ rows[:, :512]
        torch.testing.assert_close(want, ref, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(got[s].double(), ref, rtol=1e-5, atol=1e-6)

