"""Projection launches (mono_front_forward / mono_back_forward) on the GPU against the
CPU oracle (oracle/layer.py) on the same seeded weights, rows and caches.

Tolerances: bf16 outputs elementwise within |a - b| <= 2e-2 + 1e-2 |b| and 1e-2
relative in norm (the north star's bound). Quantised outputs (the FP4 index query and
key, the FP8 MLA cache row) are compared code by code: f32 accumulation order differs
between the GPU and the CPU, so a value on a rounding boundary may take the
neighbouring code. At least 98% of the codes (95% for the few index-key bytes) must
match exactly, every other one must be a single code step away, and the decoded
vectors must agree within 1e-2 (FP8) / 5e-2 (FP4, where one step is up to a third of
a value) relative in norm. Cache slots the step does not write must keep their bytes.
"""

import pytest
import torch

from oracle import attention as oattn
from oracle import codecs as ocodecs
from oracle import layer as ol
from sgl_amd_mono_amd import workloads
from sgl_amd_mono_amd.layer import WEIGHT_SPECS, ProjRuntime

pytestmark = pytest.mark.gpu

CTX = [1500, 70, 4097, 64, 2048, 2049, 300, 1]  # new tokens at ctx - 1: page starts, ends, middles
MAX_POS = 8192


def _cpu_weights(w):
    out = {}
    for name in WEIGHT_SPECS:
        t = getattr(w, name).cpu()
        if name == "w_iw":
            t = ocodecs.aiter_unshuffle(t.view(torch.uint8)).view(torch.bfloat16)
        elif name.startswith("w_"):
            t = ocodecs.aiter_unshuffle(t)
        out[name] = t
    return out


@pytest.fixture(scope="module")
def setup(gpu_device):
    print("[setup] projection weights", flush=True)
    w = workloads.proj_weights(gpu_device, seed=3)
    rt = ProjRuntime(16, gpu_device)
    cos, sin = workloads.rope_tables(MAX_POS, gpu_device)
    torch.cuda.synchronize()
    yield w, rt, cos, sin, _cpu_weights(w)
    rt.close()


def _close(got, want, what):
    got, want = got.float(), want.float()
    err = (got - want).abs()
    bound = 2e-2 + 1e-2 * want.abs()
    rel = float((got - want).norm() / want.norm().clamp_min(1e-30))
    print(f"  {what}: max err {float(err.max()):.3e}, rel {rel:.3e}", flush=True)
    assert bool((err <= bound).all()), f"{what}: {int((err > bound).sum())} elements out of bound"
    assert rel <= 1e-2, f"{what}: rel {rel}"


def _codes_close(got, want, dec_got, dec_want, step, what, min_exact=0.98, max_rel=1e-2):
    """Quantised outputs: >= min_exact of the codes equal, every other one a single code
    step away (|difference| <= step, the largest gap between neighbouring codes at that
    scale), and the decoded vectors within max_rel in norm."""
    exact = float((got == want).float().mean())
    diff = (dec_got - dec_want).abs()
    rel = float((dec_got - dec_want).norm() / dec_want.norm().clamp_min(1e-30))
    print(f"  {what}: {exact:.4f} codes exact, decoded rel {rel:.3e}, max step {float((diff / step).max()):.3f}",
          flush=True)
    assert exact >= min_exact, what
    assert bool((diff <= step * (1 + 1e-6)).all()), what
    assert rel <= max_rel, what


def _fp4_step(scales_e8m0):
    """Largest E2M1 code gap (4 -> 6) times each 32-block's scale, per element."""
    return 2.0 * ocodecs.e8m0_decode(scales_e8m0).repeat_interleave(32, -1)


@pytest.mark.parametrize("rows", [1, 8, 16])
def test_front_matches_oracle(setup, gpu_device, rows):
    w, rt, cos, sin, wc = setup
    rows_ctx = (CTX * 2)[:rows]
    print(f"[front] rows={rows}", flush=True)
    step, caches = workloads.attn_case(rows_ctx, gpu_device, seed=40 + rows, max_ctx=8192)
    h = workloads.rows_bf16(rows, ol.HIDDEN, gpu_device, seed=50 + rows)
    before = {k: getattr(caches, k).cpu().clone() for k in ("ikv", "iks", "kv", "kv_scale")}
    out = rt.front(h, step.seq_lens, step.page_table, caches, w, cos, sin)
    torch.cuda.synchronize()
    rt.check_errors()
    pos = step.seq_lens.cpu().long() - 1
    pt = step.page_table.cpu()
    f = ol.front(h.cpu(), pos, pt, wc, cos.cpu(), sin.cpu())

    _close(out.q.cpu()[..., ol.KV_LORA:], f["q_pe"], "q_pe")
    _close(out.q.cpu()[..., : ol.KV_LORA], f["q_lat"], "q_lat")
    _close(out.iw.cpu(), f["iw"], "iw")
    dq = oattn.index_query
    # FP4: one flipped code moves its value by a whole step (up to a third of it)
    assert float((out.iqs.cpu() == f["iqs"]).float().mean()) >= 0.99
    scl = torch.maximum(out.iqs.cpu(), f["iqs"])
    _codes_close(out.iq.cpu(), f["iq"], torch.stack([dq(out.iq[s].cpu(), out.iqs[s].cpu()) for s in range(rows)]),
                 torch.stack([dq(f["iq"][s], f["iqs"][s]) for s in range(rows)]), _fp4_step(scl), "index query",
                 max_rel=5e-2)

    # the caches: this step's rows match, everything else is untouched
    exp = {k: v.clone() for k, v in before.items()}
    ol.write_caches(f, exp["ikv"], exp["iks"], exp["kv"], exp["kv_scale"])
    got = {k: getattr(caches, k).cpu() for k in exp}
    slots = f["slot"]
    pages, offs = slots // 64, slots % 64
    kv_got = ocodecs.e4m3_decode(got["kv"][slots]) * got["kv_scale"][slots, None]
    kv_want = ocodecs.e4m3_decode(exp["kv"][slots]) * exp["kv_scale"][slots, None]
    kv_step = torch.maximum(kv_got.abs(), kv_want.abs()) * 2.0**-3 + got["kv_scale"][slots, None] * 2.0**-9
    _codes_close(got["kv"][slots], exp["kv"][slots], kv_got, kv_want, kv_step, "MLA cache rows")
    k_got = torch.stack([oattn.index_keys(got["ikv"], got["iks"], pt[s], int(pos[s]) + 1)[-1] for s in range(rows)])
    k_want = torch.stack([oattn.index_keys(exp["ikv"], exp["iks"], pt[s], int(pos[s]) + 1)[-1] for s in range(rows)])
    ks_got = got["iks"][pages[:, None], torch.arange(4)[None], oattn.scale_byte(offs)[:, None]]
    ks_want = exp["iks"][pages[:, None], torch.arange(4)[None], oattn.scale_byte(offs)[:, None]]
    assert float((ks_got == ks_want).float().mean()) >= 0.95
    _codes_close(got["ikv"][pages, :, offs], exp["ikv"][pages, :, offs], k_got, k_want,
                 _fp4_step(torch.maximum(ks_got, ks_want)), "index keys", min_exact=0.95, max_rel=5e-2)
    keep_kv = torch.ones(got["kv"].shape[0], dtype=torch.bool)
    keep_kv[slots] = False
    assert torch.equal(got["kv"][keep_kv], before["kv"][keep_kv])
    assert torch.equal(got["kv_scale"][keep_kv], before["kv_scale"][keep_kv])
    keep_ik = torch.ones(got["ikv"].shape[0], 4, 64, dtype=torch.bool)
    keep_ik[pages, :, offs] = False
    assert torch.equal(got["ikv"][keep_ik], before["ikv"][keep_ik])
    keep_s = torch.ones(got["iks"].shape, dtype=torch.bool)
    for p, t in zip(pages.tolist(), offs.tolist()):
        keep_s[p, :, oattn.scale_byte(t)] = False
    assert torch.equal(got["iks"][keep_s], before["iks"][keep_s])


def test_front_pad_rows_write_nothing(setup, gpu_device):
    """A row at position -1 (seq_len 0) or past the page table writes no cache row."""
    w, rt, cos, sin, _ = setup
    step, caches = workloads.attn_case([100, 200, 300], gpu_device, seed=61, max_ctx=8192)
    step.seq_lens[0] = 0
    step.seq_lens[2] = 8192 + 5  # past the table's 128 pages
    h = workloads.rows_bf16(3, ol.HIDDEN, gpu_device, seed=62)
    before = {k: getattr(caches, k).clone() for k in ("ikv", "iks", "kv", "kv_scale")}
    rt.front(h, step.seq_lens, step.page_table, caches, w, cos, sin)
    torch.cuda.synchronize()
    rt.check_errors()
    pt = step.page_table.cpu()
    slot = int(pt[1, 199 // 64]) * 64 + 199 % 64
    changed = (caches.kv != before["kv"]).any(1).nonzero().flatten().tolist()
    assert changed == [slot], changed
    assert torch.equal(caches.kv_scale[torch.arange(caches.kv_scale.numel(), device=gpu_device) != slot],
                       before["kv_scale"][torch.arange(caches.kv_scale.numel(), device=gpu_device) != slot])


@pytest.mark.parametrize("rows", [1, 8, 16])
def test_back_matches_oracle(setup, gpu_device, rows):
    w, rt, _, _, wc = setup
    print(f"[back] rows={rows}", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(70 + rows)
    o_lat = (torch.randn(rows, ol.HEADS, ol.KV_LORA, generator=g, device=gpu_device) * 0.5).to(torch.bfloat16)
    h = workloads.rows_bf16(rows, ol.HIDDEN, gpu_device, seed=80 + rows)
    o = torch.empty(rows, ol.HEADS * ol.V_DIM, dtype=torch.bfloat16, device=gpu_device)
    a = rt.back(o_lat, h, w, o=o)
    torch.cuda.synchronize()
    rt.check_errors()
    b = ol.back(o_lat.cpu(), h.cpu(), wc)
    _close(o.cpu(), b["o"], "o")
    _close(a.cpu(), b["a"], "a")


def test_proj_repeat_is_bitwise(setup, gpu_device):
    w, rt, cos, sin, _ = setup
    step, caches = workloads.attn_case(CTX, gpu_device, seed=90, max_ctx=8192)
    h = workloads.rows_bf16(8, ol.HIDDEN, gpu_device, seed=91)
    o1 = rt.front(h, step.seq_lens, step.page_table, caches, w, cos, sin)
    kv1 = caches.kv.clone()
    o2 = rt.front(h, step.seq_lens, step.page_table, caches, w, cos, sin)
    torch.cuda.synchronize()
    for name in ("q", "iq", "iqs", "iw"):
        assert torch.equal(getattr(o1, name), getattr(o2, name)), name
    assert torch.equal(kv1, caches.kv)
    o_lat = o1.q[..., :512].contiguous()
    a1 = rt.back(o_lat, h, w)
    a2 = rt.back(o_lat, h, w)
    torch.cuda.synchronize()
    assert torch.equal(a1, a2)


def test_proj_fail_stop_on_forced_wait(setup, gpu_device):
    w, rt, cos, sin, _ = setup
    step, caches = workloads.attn_case(CTX, gpu_device, seed=95, max_ctx=8192)
    h = workloads.rows_bf16(8, ol.HIDDEN, gpu_device, seed=96)
    good = rt.front(h, step.seq_lens, step.page_table, caches, w, cos, sin).q.clone()
    o_lat = good[..., :512].contiguous()
    a_good = rt.back(o_lat, h, w).clone()
    torch.cuda.synchronize()
    rt.check_errors()
    for site in (0, 1, 2, 3, 4):
        print(f"[fault] forcing wait site {site}", flush=True)
        rt.set_deadline(0.02)
        rt.set_fault(site)
        if site < 4:
            rt.front(h, step.seq_lens, step.page_table, caches, w, cos, sin)
        else:
            rt.back(o_lat, h, w)
        torch.cuda.synchronize()
        assert rt.error_words()[1] == site + 1, rt.error_words()
        with pytest.raises(Exception, match="stopped"):
            rt.check_errors()
        rt.set_fault(-1)
        rt.set_deadline(2.0)
        rt.clear_errors()
    again = rt.front(h, step.seq_lens, step.page_table, caches, w, cos, sin).q
    a_again = rt.back(o_lat, h, w)
    torch.cuda.synchronize()
    rt.check_errors()
    assert torch.equal(again, good) and torch.equal(a_again, a_good)


def test_proj_rejects_bad_args(setup, gpu_device):
    w, rt, cos, sin, _ = setup
    step, caches = workloads.attn_case([10, 20], gpu_device, seed=97, max_ctx=8192)
    h = workloads.rows_bf16(2, ol.HIDDEN, gpu_device, seed=98)
    with pytest.raises(ValueError, match="h"):
        rt.front(h.float(), step.seq_lens, step.page_table, caches, w, cos, sin)
    with pytest.raises(ValueError, match="seq_lens"):
        rt.front(h, step.seq_lens.long(), step.page_table, caches, w, cos, sin)
    with pytest.raises(ValueError, match="rows"):
        rt.front(workloads.rows_bf16(17, ol.HIDDEN, gpu_device, seed=1), step.seq_lens, step.page_table, caches,
                 w, cos, sin)
