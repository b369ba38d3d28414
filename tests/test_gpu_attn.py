"""Sparse-attention phase on the GPU against the CPU oracle.

* Index scores against the oracle's f32 restatement of the FP4 indexer (within f32
  summation-order error).
* The exact top-2048 bit-exact: the oracle's rule (score desc, position asc, mapped
  through the page table) applied to the device's own scores must give exactly the
  device's slots, in order.
* The attention output against the oracle's sparse MLA over the device's selection:
  bf16 within the (atol 2e-2, rtol 1e-2) pair elementwise and 1e-2 relative in norm.
Rows mirror the reference's decode positions (test/kernels/glm53/check_layer.py:45-47)
below and above 2048 keys, plus a full 32768-key context.
"""

import pytest
import torch

from oracle import attention as oatt
from sgl_amd_mono_amd import workloads
from sgl_amd_mono_amd.attn import AttnRuntime

pytestmark = pytest.mark.gpu

OUT_MAX_ABS, OUT_REL = 2e-2, 1e-2
SCORE_REL = 1e-4  # of the row's largest score magnitude: f32 summation order only

CTX_8 = [8447, 1500, 5000, 300, 32768, 2047, 2048, 9000]


@pytest.fixture(scope="module")
def rt(gpu_device):
    r = AttnRuntime(64, 32768, device=gpu_device)
    yield r
    r.close()


def _crowding(scores, ctx, bits=16):
    """For each row longer than 2048: how many of its keys share the 2048th largest
    key's upper ``bits`` bits (at 16, the device exchanges them when at most 512, else
    takes two more radix digits)."""
    out = []
    for s, n in enumerate(ctx):
        if n <= 2048:
            continue
        b = scores[s, :n].contiguous().view(torch.int32).long() & 0xFFFFFFFF
        key = torch.where(b >= 2**31, b ^ 0xFFFFFFFF, b | 2**31)
        t = key.sort(descending=True).values[2047]
        out.append(int(((key >> (32 - bits)) == (t >> (32 - bits))).sum()))
    return out


def _check(rt, ctx, seed, gpu_device, period=0, shape=None):
    print(f"[attn] rows={len(ctx)} seed={seed} period={period} ctx={ctx[:8]}...", flush=True)
    step, caches = workloads.attn_case(ctx, gpu_device, seed=seed)
    if period:  # every page of the index plane a copy of page p % period: repeated scores
        src = torch.arange(caches.ikv.shape[0], device=gpu_device) % period
        caches.ikv.copy_(caches.ikv[src].clone())
        caches.iks.copy_(caches.iks[src].clone())
    if shape is not None:
        shape(step, caches)
    out, dbg = rt.forward(step, caches, debug=True)
    torch.cuda.synchronize()
    rt.check_errors()
    c = {k: v.cpu() for k, v in vars(caches).items()}
    st = {k: v.cpu() for k, v in vars(step).items()}
    scores, sel = dbg["scores"].cpu(), dbg["topk"].cpu()
    ref_scores = oatt.index_scores(st["iq"], st["iqs"], st["iw"], c["ikv"], c["iks"], st["page_table"],
                                   st["seq_lens"], rt.max_ctx)
    for s, n in enumerate(ctx):
        d = (scores[s, :n] - ref_scores[s, :n]).abs().max().item()
        scale = ref_scores[s, :n].abs().max().item()
        assert d <= SCORE_REL * scale + 1e-6, (s, d, scale)
    want_sel = oatt.select_topk(scores, st["seq_lens"], st["page_table"])
    print(f"[attn] keys sharing the threshold's upper 16 bits: {_crowding(scores, ctx)}", flush=True)
    assert torch.equal(sel, want_sel), [s for s in range(len(ctx)) if not torch.equal(sel[s], want_sel[s])]
    if shape is not None:
        dbg["crowding"] = [_crowding(scores, ctx, b) for b in (16, 24, 32)]
    ref = oatt.sparse_mla(st["q"], c["kv"], c["kv_scale"], sel)
    got = out.cpu().float()
    err = (got - ref).abs()
    rel = ((got - ref).norm() / ref.norm()).item()
    print(f"[attn] out max-abs {err.max().item():.3e} (|ref| max {ref.abs().max().item():.2f}) "
          f"norm-rel {rel:.3e}", flush=True)
    # the bound as an (atol, rtol) pair, elementwise: |a - b| <= 2e-2 + 1e-2 |b|
    assert bool((err <= OUT_MAX_ABS + OUT_REL * ref.abs()).all()) and rel <= OUT_REL
    return out, sel, dbg


def test_attn_8_rows_matches_oracle(rt, gpu_device):
    _check(rt, CTX_8, 0, gpu_device)


def test_attn_1_row_full_context(rt, gpu_device):
    _check(rt, [32768], 1, gpu_device)


def test_attn_48_rows_mixed_contexts(rt, gpu_device):
    g = torch.Generator().manual_seed(2)
    ctx = torch.randint(1, 12000, (48,), generator=g).tolist()
    ctx[0], ctx[1], ctx[2] = 32768, 2048, 2049
    _check(rt, ctx, 2, gpu_device)


def test_attn_24_rows_long_splits(rt, gpu_device):
    """24 rows take 8 splits a row of 256 selected tokens (four sub-tiles each) and merges
    of 4 heads: the same selection and, within the bound, the same output."""
    g = torch.Generator().manual_seed(4)
    ctx = torch.randint(1, 32768, (24,), generator=g).tolist()
    ctx[0], ctx[1], ctx[2], ctx[3] = 32768, 2048, 2049, 300
    _check(rt, ctx, 9, gpu_device)


def test_attn_48_rows_full_contexts(rt, gpu_device):
    """BASELINE config 3 at its largest size: 48 rows of (nearly) 32768 keys each (5 splits
    a row of 6 or 7 sub-tiles, merges of 8 heads)."""
    ctx = [32768] * 44 + [32767, 32704, 30001, 16385]
    _check(rt, ctx, 7, gpu_device)


def test_attn_56_rows_wide_launch(rt, gpu_device):
    """Above 48 rows the launch takes 4 even splits a row (its own kernel build): the same
    selection and, within the bound, the same output."""
    g = torch.Generator().manual_seed(11)
    ctx = torch.randint(1, 32768, (56,), generator=g).tolist()
    ctx[0], ctx[1], ctx[2], ctx[3] = 32768, 2048, 2049, 300
    _check(rt, ctx, 13, gpu_device)


@pytest.mark.parametrize("period", [1, 6])
def test_attn_repeated_scores(rt, gpu_device, period):
    """Index planes whose pages repeat every `period` pages: each score recurs about
    n / (64 period) times in a row, so the keys sharing the threshold's upper 16 bits
    tie in whole groups (512 copies at period 1 and 32768 keys: exactly the largest
    candidate exchange), and the lowest positions of the threshold score are taken."""
    _check(rt, [32768, 20000, 9000, 4100, 2049], 5, gpu_device, period=period)


def _crowd_planes(group: int, fine_code: int):
    """An index plane that crowds the threshold: every page is one base page, whose
    ``group`` key slots ranked around the 2048th key are made identical (so about
    ``group`` x 512 keys of a 32768-key row share the threshold's upper 16 bits, more
    than the 512-word candidate exchange takes). Dims 96-99 of every key (in block 3,
    scaled down to E8M0 ``fine_code``) then carry codes that vary with the physical
    page, which moves each score by a small fraction below its upper 16 bits: radix
    digits 3 and 4 discriminate, and equal perturbations leave exact ties. Every row
    uses row 0's index query and head weights, so every row is crowded alike."""

    def shape(step, caches):
        for k in ("iq", "iqs", "iw"):
            getattr(step, k)[:] = getattr(step, k)[0:1].clone()
        B, Bs = caches.ikv[0].cpu(), caches.iks[0].cpu()  # [4, 64, 16], [4, 64]
        sb = oatt.scale_byte(torch.arange(64))
        Bs[3, sb] = fine_code
        B[3, :, 0:2] = 0
        base = oatt.index_scores(step.iq[:1].cpu(), step.iqs[:1].cpu(), step.iw[:1].cpu(), B[None], Bs[None],
                                 torch.zeros(1, 1, dtype=torch.int32), torch.tensor([64]), 64)[0]
        order = base.argsort(descending=True)
        r0 = 3 if group <= 2 else 1  # the group straddles rank 2048 (512 copies a slot)
        src = int(order[r0])
        for j in range(r0 + 1, r0 + group):
            d = int(order[j])
            B[:, d] = B[:, src]
            Bs[:, sb[d]] = Bs[:, sb[src]]
        caches.ikv[:] = B.to(caches.ikv.device)[None]
        caches.iks[:] = Bs.to(caches.iks.device)[None]
        p = torch.arange(caches.ikv.shape[0], device=caches.ikv.device)
        lo = (p % 8) | ((p // 8 % 8) << 4)
        hi = (p // 64 % 8) | ((p // 512 % 8) << 4)
        caches.ikv[:, 3, :, 0] = lo[:, None].to(torch.uint8)
        caches.ikv[:, 3, :, 1] = hi[:, None].to(torch.uint8)

    return shape


@pytest.mark.parametrize("rows,group,fine", [(1, 2, 118), (1, 8, 116), (8, 2, 116), (8, 8, 118)])
def test_attn_crowded_threshold_takes_digits_3_and_4(rt, gpu_device, rows, group, fine):
    """600-4000 keys share the threshold's upper 16 bits but differ below them: the
    top-k team's crowded path (digits 3 and 4 over the members' exchanged histograms,
    then the count exchange) must still give the oracle's exact selection, ties at the
    threshold going to the lowest positions (indexer.py:693-781 refines the same way)."""
    _, _, dbg = _check(rt, [32768] * rows, 8, gpu_device, shape=_crowd_planes(group, fine))
    c16, c24, c32 = dbg["crowding"]
    print(f"[attn crowd] upper-16 {c16} upper-24 {c24} equal {c32}", flush=True)
    assert min(c16) > 512  # every row takes the crowded path
    assert any(a > b for a, b in zip(c16, c24))  # digit 3 discriminates
    assert any(a > b for a, b in zip(c24, c32))  # digit 4 discriminates


def test_attn_ties_take_lowest_positions(rt, gpu_device):
    """An index query of all-zero codes makes every score 0: the selection must be the
    first 2048 positions of the row (lowest-position ties, glm53/check.py:100-117)."""
    step, caches = workloads.attn_case([5000, 3000], gpu_device, seed=3)
    step.iq.zero_()
    out, dbg = rt.forward(step, caches, debug=True)
    torch.cuda.synchronize()
    rt.check_errors()
    pt = step.page_table.cpu()
    pos = torch.arange(2048)
    for s in range(2):
        want = (pt[s, pos // 64].long() * 64 + pos % 64).to(torch.int32)
        assert torch.equal(dbg["topk"][s].cpu(), want)


def test_attn_repeat_is_bitwise(rt, gpu_device):
    step, caches = workloads.attn_case(CTX_8, gpu_device, seed=4)
    a, da = rt.forward(step, caches, debug=True)
    b, db = rt.forward(step, caches, debug=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(da["topk"], db["topk"]) and torch.equal(da["scores"], db["scores"])


def test_attn_fail_stop_each_site(rt, gpu_device):
    step, caches = workloads.attn_case([5000, 1000, 3000], gpu_device, seed=5)
    good = rt.forward(step, caches)
    torch.cuda.synchronize()
    for site in (0, 1, 2, 3):
        print(f"[attn fault] site {site}", flush=True)
        rt.set_fault(site)
        rt.forward(step, caches)
        assert rt.error_words()[1] == site + 1
        rt.set_fault(-1)
        rt.clear_errors()
        again = rt.forward(step, caches)
        torch.cuda.synchronize()
        rt.check_errors()
        assert torch.equal(again, good)


def test_attn_rejects_bad_arguments(rt, gpu_device):
    step, caches = workloads.attn_case([100], gpu_device, seed=6)
    step.q = step.q.float()
    with pytest.raises(ValueError, match="q"):
        rt.forward(step, caches)
