"""The whole decoder layer on the GPU: two stacked, independently
seeded layers at 8 rows over 32768-key contexts, each phase checked against the CPU
oracle on the inputs the device handed it (the same teacher-forced comparison the
phase tests make), so the test pins how the layer runtime wires the phases together:

* front: q (q_lat | q_pe) and the index head weights against oracle.layer.front;
* attention: the exact top-2048 of the device's index scores bit-exact, o_lat against
  oracle.attention.sparse_mla over that selection and the caches front wrote;
* back: a against oracle.layer.back on the device's o_lat;
* MoE: routing bit-exact on the device's scores, x_out against oracle.moe.fp8_moe_block.
"""

import pytest
import torch

from oracle import attention as oatt
from oracle import codecs as ocodecs
from oracle import layer as ol
from oracle import moe as omoe
from oracle import topk as otopk
from sgl_amd_mono_amd import workloads
from sgl_amd_mono_amd.layer import WEIGHT_SPECS, LayerRuntime, LayerWeights
from sgl_amd_mono_amd.moe import FP8_MOE

pytestmark = pytest.mark.gpu

ROWS, CTX, LAYERS = 8, 32768, 2


class CpuExperts:
    def __init__(self, t, shuffled=False):
        self.t, self.shuffled, self.cache = t, shuffled, {}

    def __getitem__(self, e):
        if e not in self.cache:
            x = self.t[e].cpu()
            self.cache[e] = ocodecs.aiter_unshuffle(x) if self.shuffled else x
        return self.cache[e]


def _cpu_proj(w):
    out = {}
    for name in WEIGHT_SPECS:
        t = getattr(w, name).cpu()
        if name == "w_iw":
            t = ocodecs.aiter_unshuffle(t.view(torch.uint8)).view(torch.bfloat16)
        elif name.startswith("w_"):
            t = ocodecs.aiter_unshuffle(t)
        out[name] = t
    return out


def _close(got, want, what):
    got, want = got.float(), want.float()
    err = (got - want).abs()
    rel = float((got - want).norm() / want.norm().clamp_min(1e-30))
    print(f"  {what}: max err {float(err.max()):.3e}, rel {rel:.3e}", flush=True)
    assert bool((err <= 2e-2 + 1e-2 * want.abs()).all()), what
    assert rel <= 1e-2, what


def test_two_layers_phase_by_phase(gpu_device):
    rt = LayerRuntime(ROWS, CTX, gpu_device)
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    lens = [CTX, 9000, 2049, 300, CTX - 5, 2048, 16000, 64]  # new tokens at len - 1
    x = workloads.rows_bf16(ROWS, ol.HIDDEN, gpu_device, seed=5)
    try:
        for layer in range(LAYERS):
            seed = 1000 * layer + 7  # per-layer seeds (test/kernels/glm53/check_layer.py:84)
            print(f"[layer {layer}] weights", flush=True)
            w = LayerWeights(proj=workloads.proj_weights(gpu_device, seed=seed),
                             moe=workloads.fp8_moe_weights(FP8_MOE, gpu_device, seed=seed + 1))
            step, caches = workloads.attn_case(lens, gpu_device, seed=seed + 2, max_ctx=CTX)
            x_out, it = rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin, keep=True)
            torch.cuda.synchronize()
            rt.check_errors()
            h = x.cpu()
            pos = step.seq_lens.cpu().long() - 1
            pt = step.page_table.cpu()

            f = ol.front(h, pos, pt, _cpu_proj(w.proj), cos.cpu(), sin.cpu())
            _close(it["q"].cpu(), f["q"], "front q")
            _close(it["iw"].cpu(), f["iw"], "front iw")

            c = {k: v.cpu() for k, v in vars(caches).items()}
            scores, sel = it["index_scores"].cpu(), it["topk_slots"].cpu()
            ref_scores = oatt.index_scores(it["iq"].cpu(), it["iqs"].cpu(), it["iw"].cpu(), c["ikv"], c["iks"], pt,
                                           step.seq_lens.cpu(), CTX)
            for s, n in enumerate(lens):
                d = float((scores[s, :n] - ref_scores[s, :n]).abs().max())
                assert d <= 1e-4 * float(ref_scores[s, :n].abs().max()) + 1e-6, (s, d)
            assert torch.equal(sel, oatt.select_topk(scores, step.seq_lens.cpu(), pt))
            o_ref = oatt.sparse_mla(it["q"].cpu(), c["kv"], c["kv_scale"], sel)
            _close(it["o_lat"].cpu(), o_ref, "attention o_lat")

            b = ol.back(it["o_lat"].cpu(), h, _cpu_proj(w.proj))
            _close(it["a"].cpu(), b["a"], "back a")

            m = w.moe
            ids_ref, w_ref = otopk.router_top8(it["scores"].cpu(), m.bias.cpu(), FP8_MOE.top_k, FP8_MOE.route_scale)
            assert torch.equal(it["topk_ids"].cpu().long(), ids_ref)
            ref = omoe.fp8_moe_block(
                it["a"].cpu(), m.g_post.cpu(), m.w_router.cpu(), m.bias.cpu(), CpuExperts(m.w13, True),
                CpuExperts(m.s13), CpuExperts(m.w2, True), CpuExperts(m.s2), eps=FP8_MOE.eps, top_k=FP8_MOE.top_k,
                inter=FP8_MOE.inter, ids=ids_ref, weights=w_ref,
            )  # fmt: skip
            _close(x_out.cpu(), ref["out"], "moe x_out")
            x = x_out.clone()
            del w, caches
    finally:
        rt.close()


@pytest.mark.parametrize("rows", [1, 8])
def test_fused_attention_back_equals_two_launches(gpu_device, rows):
    """mono_attn_back_forward (one launch) gives bit for bit what mono_attn_forward then
    mono_back_forward give, launch after launch (the launch-parity mailboxes alternate)."""
    from sgl_amd_mono_amd.attn import AttnRuntime
    from sgl_amd_mono_amd.layer import ProjRuntime, attn_back

    lens = [CTX, 9000, 2049, 300, CTX - 5, 2048, 16000, 64][:rows]
    ra, rp = AttnRuntime(8, CTX, device=gpu_device), ProjRuntime(8, gpu_device)
    try:
        w = workloads.proj_weights(gpu_device, seed=11)
        for it in range(3):
            print(f"[rows {rows}] launch pair {it}", flush=True)
            step, caches = workloads.attn_case(lens, gpu_device, seed=12 + it, max_ctx=CTX)
            h = workloads.rows_bf16(rows, ol.HIDDEN, gpu_device, seed=20 + it)
            o1 = ra.forward(step, caches)
            a1 = rp.back(o1, h, w)
            o2, a2 = attn_back(ra, step, caches, w, h)
            torch.cuda.synchronize()
            ra.check_errors()
            rp.check_errors()
            assert torch.equal(o1, o2), "o_lat"
            assert torch.equal(a1, a2), "a"
    finally:
        ra.close()
        rp.close()


def test_layer_raw_e4m3_mla_rows(gpu_device):
    """A layer over an MLA cache without a scale plane (``kv_scale=None``: raw E4M3
    rows, SGLang's HIP DSA layout): the front writes each new row as E4M3 of the
    values themselves (scale 1) and the attention reads every row unscaled."""
    ctx, rows = 4096, 4
    rt = LayerRuntime(rows, ctx, gpu_device)
    cos, sin = workloads.rope_tables(ctx, gpu_device)
    lens = [4096, 1500, 65, 2049]
    print("[raw e4m3] weights", flush=True)
    w = LayerWeights(proj=workloads.proj_weights(gpu_device, seed=21),
                     moe=workloads.fp8_moe_weights(FP8_MOE, gpu_device, seed=22))
    step, caches = workloads.attn_case(lens, gpu_device, seed=23, max_ctx=ctx)
    caches.kv_scale = None
    x = workloads.rows_bf16(rows, ol.HIDDEN, gpu_device, seed=24)
    kv_before = caches.kv.cpu().clone()
    try:
        _, it = rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin, keep=True)
        torch.cuda.synchronize()
        rt.check_errors()
    finally:
        rt.close()
    pos = step.seq_lens.cpu().long() - 1
    pt = step.page_table.cpu()
    f = ol.front(x.cpu(), pos, pt, _cpu_proj(w.proj), cos.cpu(), sin.cpu(), kv_scaled=False)
    _close(it["q"].cpu(), f["q"], "front q")
    kv = caches.kv.cpu()
    slots = f["slot"]
    got, want = ocodecs.e4m3_decode(kv[slots]), ocodecs.e4m3_decode(f["kv"])
    exact = float((kv[slots] == f["kv"]).float().mean())
    step_ = torch.maximum(got.abs(), want.abs()) * 2.0**-3 + 2.0**-9
    print(f"  raw rows: {exact:.4f} codes exact", flush=True)
    assert exact >= 0.98 and bool(((got - want).abs() <= step_ * (1 + 1e-6)).all())
    keep = torch.ones(kv.shape[0], dtype=torch.bool)
    keep[slots] = False
    assert torch.equal(kv[keep], kv_before[keep])
    sel = it["topk_slots"].cpu()
    c = {k: v.cpu() for k, v in vars(caches).items() if v is not None}
    assert torch.equal(sel, oatt.select_topk(it["index_scores"].cpu(), step.seq_lens.cpu(), pt))
    o_ref = oatt.sparse_mla(it["q"].cpu(), c["kv"], None, sel)
    _close(it["o_lat"].cpu(), o_ref, "attention o_lat (unscaled rows)")
    b = ol.back(it["o_lat"].cpu(), x.cpu(), _cpu_proj(w.proj))
    _close(it["a"].cpu(), b["a"], "back a")


@pytest.mark.parametrize("rows", [1, 8, 16])
def test_layer_launch_modes_agree_bitwise(gpu_device, rows):
    """The fused layer launch (mono_layer_forward: front, then attention + back + MoE as
    one launch) gives bit for bit what the three- and four-launch splits give, its
    intermediates included, over two steps in a row (fresh tags on the second)."""
    ctx = 8192
    cos, sin = workloads.rope_tables(ctx, gpu_device)
    lens = ([8192, 1500, 65, 2049, 4000, 64, 7000, 300] * 2)[:rows]
    print(f"[modes] rows={rows}", flush=True)
    w = LayerWeights(proj=workloads.proj_weights(gpu_device, seed=31),
                     moe=workloads.fp8_moe_weights(FP8_MOE, gpu_device, seed=32))
    x = workloads.rows_bf16(rows, ol.HIDDEN, gpu_device, seed=34)
    got = {}
    for mode in ("layer", "attn_back", "split"):
        step, caches = workloads.attn_case(lens, gpu_device, seed=33, max_ctx=ctx)
        rt = LayerRuntime(rows, ctx, gpu_device, mode=mode)
        try:
            outs = []
            for _ in range(2):
                outs.append(rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin, keep=True))
            torch.cuda.synchronize()
            rt.check_errors()
        finally:
            rt.close()
        got[mode] = (outs, caches.kv.clone(), caches.ikv.clone())
    ref_outs, ref_kv, ref_ikv = got["split"]
    for mode in ("layer", "attn_back"):
        outs, kv, ikv = got[mode]
        assert torch.equal(kv, ref_kv) and torch.equal(ikv, ref_ikv), mode
        for (xo, it), (xr, ir) in zip(outs, ref_outs):
            assert torch.equal(xo, xr), (mode, float((xo.float() - xr.float()).abs().max()))
            for k in ("q", "o_lat", "a", "topk_slots", "topk_ids", "topk_w", "y"):
                assert torch.equal(it[k], ir[k]), (mode, k)


@pytest.mark.parametrize("site,what", [(10, "attention block output rows"), (11, "front: stage-A partial sums"),
                                       (17, "front index query and keys"), (18, "front q")])
def test_layer_launch_fail_stop(gpu_device, site, what):
    """A forced wait failure in the one-launch layer (the MoE's wait on the attention
    block's output rows, the front's stage-A wait, the attention's waits on the front)
    stops it without a fault: the error names the site, the host word reports it
    without a synchronisation, the failed launch's output is NaN, later launches are
    refused (their output NaN too) until the errors are cleared, then the layer runs
    again."""
    ctx, rows = 4096, 2
    cos, sin = workloads.rope_tables(ctx, gpu_device)
    w = LayerWeights(proj=workloads.proj_weights(gpu_device, seed=41),
                     moe=workloads.fp8_moe_weights(FP8_MOE, gpu_device, seed=42))
    step, caches = workloads.attn_case([4096, 100], gpu_device, seed=43, max_ctx=ctx)
    x = workloads.rows_bf16(rows, ol.HIDDEN, gpu_device, seed=44)
    rt = LayerRuntime(rows, ctx, gpu_device)
    try:
        good = rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin).clone()
        torch.cuda.synchronize()
        rt.check_errors()
        assert rt.handle.pending_error() == 0
        rt.handle.set_fault(site)
        bad = rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin).clone()
        torch.cuda.synchronize()
        assert rt.handle.pending_error() == site + 1
        with pytest.raises(Exception, match=what):
            rt.raise_pending()
        with pytest.raises(Exception, match=what):
            rt.check_errors()
        assert bool(bad.isnan().all()), "a failed launch's output is NaN"
        rt.handle.set_fault(-1)
        refused = rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin).clone()
        torch.cuda.synchronize()
        assert bool(refused.isnan().all()), "a refused launch's output is NaN"
        rt.clear_errors()
        assert rt.handle.pending_error() == 0
        again = rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin)
        torch.cuda.synchronize()
        rt.check_errors()
        rt.raise_pending()
        assert torch.equal(again, good)
    finally:
        rt.close()


def test_layer_verify_chain_sees_its_own_draft_keys(gpu_device):
    """MTP verify rows: four rows of one request at consecutive positions (sharing its
    page table) in one step, the chain crossing a 1024-key chunk boundary. Each row
    must score the keys the earlier rows write in the same step: the one-launch layer
    gives bit for bit what the split launches give (where the front's launch ends
    before the attention's starts), and every row selects the chain's earlier keys."""
    ctx = 4096
    cos, sin = workloads.rope_tables(ctx, gpu_device)
    w = LayerWeights(proj=workloads.proj_weights(gpu_device, seed=51),
                     moe=workloads.fp8_moe_weights(FP8_MOE, gpu_device, seed=52))
    x = workloads.rows_bf16(4, ol.HIDDEN, gpu_device, seed=54)
    lens = [1023, 1024, 1025, 1026]  # new keys at 1022 .. 1025
    got = {}
    for mode in ("layer", "split"):
        step, caches = workloads.attn_case([ctx], gpu_device, seed=53, max_ctx=ctx)
        pt = step.page_table[:1].repeat(4, 1).contiguous()
        seq = torch.tensor(lens, dtype=torch.int32, device=gpu_device)
        rt = LayerRuntime(4, ctx, gpu_device, mode=mode)
        try:
            got[mode] = rt.forward(x, seq, pt, caches, w, cos, sin, keep=True)
            torch.cuda.synchronize()
            rt.check_errors()
        finally:
            rt.close()
    (xl, il), (xs, is_) = got["layer"], got["split"]
    assert torch.equal(il["index_scores"], is_["index_scores"])
    assert torch.equal(il["topk_slots"], is_["topk_slots"])
    assert torch.equal(xl, xs)
    # rows of at most 2048 keys select all of them, the chain's earlier keys included
    pt0 = step.page_table[0].cpu().long()
    for j, n in enumerate(lens):
        want = (pt0[torch.arange(n) // 64] * 64 + torch.arange(n) % 64).to(torch.int32)
        assert torch.equal(il["topk_slots"][j, :n].cpu(), want), j


def test_layer_verify_chain_matches_oracle(gpu_device):
    """MTP verify rows past 2048 keys against the oracle (glm53/check.py:100-146):
    four rows of one request at positions 5118 .. 5121 (the chain crosses the 5120-key
    chunk boundary), one launch. The oracle runs each row's front and writes its cache
    rows in order into CPU copies of the caches; then, per row over those caches:

    * the device's chain rows match the oracle's cache rows code by code;
    * index scores over the device's caches within 1e-4 of the row's largest score,
      the chain keys included (a stale read of a draft key would miss by far more);
    * the selection bit-exact against the exact top-2048 of the row's own scores, and
      it holds every chain key that the oracle's own scores select (``topk_own``);
    * o_lat against sparse MLA over the oracle-written caches, then ``a`` and x_out
      on the device's intermediates as in the phase-by-phase test."""
    ctx, rows = 8192, 4
    lens = [5119, 5120, 5121, 5122]  # new keys at 5118 .. 5121
    cos, sin = workloads.rope_tables(ctx, gpu_device)
    print("[verify chain] weights", flush=True)
    w = LayerWeights(proj=workloads.proj_weights(gpu_device, seed=61),
                     moe=workloads.fp8_moe_weights(FP8_MOE, gpu_device, seed=62))
    step, caches = workloads.attn_case([ctx], gpu_device, seed=63, max_ctx=ctx)
    pt_dev = step.page_table[:1].repeat(rows, 1).contiguous()
    seq = torch.tensor(lens, dtype=torch.int32, device=gpu_device)
    x = workloads.rows_bf16(rows, ol.HIDDEN, gpu_device, seed=64)
    before = {k: getattr(caches, k).cpu().clone() for k in ("ikv", "iks", "kv", "kv_scale")}
    rt = LayerRuntime(rows, ctx, gpu_device)
    try:
        x_out, it = rt.forward(x, seq, pt_dev, caches, w, cos, sin, keep=True)
        torch.cuda.synchronize()
        rt.check_errors()
    finally:
        rt.close()
    h, pt, pos = x.cpu(), pt_dev.cpu(), seq.cpu().long() - 1
    proj = _cpu_proj(w.proj)
    exp = {k: v.clone() for k, v in before.items()}
    fronts = []
    for j in range(rows):  # each draft's front, its cache rows written before the next row's
        f = ol.front(h[j:j + 1], pos[j:j + 1], pt[j:j + 1], proj, cos.cpu(), sin.cpu())
        ol.write_caches(f, exp["ikv"], exp["iks"], exp["kv"], exp["kv_scale"])
        fronts.append(f)
    _close(it["q"].cpu(), torch.cat([f["q"] for f in fronts]), "front q")
    got = {k: getattr(caches, k).cpu() for k in exp}
    slots = torch.cat([f["slot"] for f in fronts])
    assert len(set(slots.tolist())) == rows
    exact = float((got["kv"][slots] == exp["kv"][slots]).float().mean())
    pages, offs = slots // 64, slots % 64
    ik_exact = float((got["ikv"][pages, :, offs] == exp["ikv"][pages, :, offs]).float().mean())
    print(f"  chain rows: MLA codes {exact:.4f} exact, index-key bytes {ik_exact:.4f} exact", flush=True)
    assert exact >= 0.98 and ik_exact >= 0.9

    scores, sel = it["index_scores"].cpu(), it["topk_slots"].cpu()
    ref_dev = oatt.index_scores(it["iq"].cpu(), it["iqs"].cpu(), it["iw"].cpu(), got["ikv"], got["iks"], pt,
                                seq.cpu(), ctx)
    ref_own = oatt.index_scores(it["iq"].cpu(), it["iqs"].cpu(), it["iw"].cpu(), exp["ikv"], exp["iks"], pt,
                                seq.cpu(), ctx)
    want_sel = oatt.select_topk(scores, seq.cpu(), pt)
    own_sel = oatt.select_topk(ref_own, seq.cpu(), pt)
    chain_total = 0
    for j, n in enumerate(lens):
        tol = 1e-4 * float(ref_dev[j, :n].abs().max()) + 1e-6
        assert float((scores[j, :n] - ref_dev[j, :n]).abs().max()) <= tol, j
        assert float((scores[j, n - j - 1:n] - ref_dev[j, n - j - 1:n]).abs().max()) <= tol, j  # chain keys
        chain = set(slots[:j + 1].tolist())
        picked, oracle_picked = set(sel[j, :2048].tolist()), set(own_sel[j, :2048].tolist())
        assert (oracle_picked & chain) <= picked, (j, oracle_picked & chain, picked & chain)
        chain_total += len(picked & chain)
    print(f"  chain keys selected over the four rows: {chain_total}", flush=True)
    assert torch.equal(sel, want_sel)
    assert chain_total > 0  # the seeds put draft keys in the selections
    o_ref = oatt.sparse_mla(it["q"].cpu(), exp["kv"], exp["kv_scale"], sel)
    _close(it["o_lat"].cpu(), o_ref, "attention o_lat")
    b = ol.back(it["o_lat"].cpu(), h, proj)
    _close(it["a"].cpu(), b["a"], "back a")
    m = w.moe
    ids_ref, w_ref = otopk.router_top8(it["scores"].cpu(), m.bias.cpu(), FP8_MOE.top_k, FP8_MOE.route_scale)
    assert torch.equal(it["topk_ids"].cpu().long(), ids_ref)
    ref = omoe.fp8_moe_block(
        it["a"].cpu(), m.g_post.cpu(), m.w_router.cpu(), m.bias.cpu(), CpuExperts(m.w13, True),
        CpuExperts(m.s13), CpuExperts(m.w2, True), CpuExperts(m.s2), eps=FP8_MOE.eps, top_k=FP8_MOE.top_k,
        inter=FP8_MOE.inter, ids=ids_ref, weights=w_ref,
    )  # fmt: skip
    _close(x_out.cpu(), ref["out"], "moe x_out")
