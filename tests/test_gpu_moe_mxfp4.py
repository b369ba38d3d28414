"""MXFP4 A16W4 MoE on the GPU against the CPU oracle.

Routing is checked bit-exact on the same f32 logits: the oracle's softmax top-8 (key
descending, lowest id on ties) must give the device's ids in the same order, and the
route weights (softmax over the picks) within 1e-5. The expert outputs are compared
on the oracle's routing: the f32 MoE sum within 1e-2 relative (norm) and the bf16
output within the (atol 2e-2, rtol 1e-2) pair elementwise and 1e-2 relative in norm.
The expert matrices are unshuffled for the oracle by its own gather formula.
"""

import pytest
import torch

from oracle import codecs as ocodecs
from oracle import moe as omoe
from oracle import topk as otopk
from sgl_amd_mono_amd import workloads
from sgl_amd_mono_amd.moe import MXFP4_MOE, MoeRuntime

pytestmark = pytest.mark.gpu

G = MXFP4_MOE
OUT_MAX_ABS, OUT_REL = 2e-2, 1e-2  # the north star's bf16 output bound
Y_REL = 1e-2  # the MoE sum itself (f32), relative to its norm


class CpuExperts:
    """Expert tensors fetched to the CPU on first use; shuffled byte matrices are
    unshuffled by the oracle's gather."""

    def __init__(self, t, shuffled=False):
        self.t, self.shuffled, self.cache = t, shuffled, {}

    def __getitem__(self, e):
        if e not in self.cache:
            x = self.t[e].cpu()
            self.cache[e] = ocodecs.aiter_unshuffle(x) if self.shuffled else x
        return self.cache[e]


@pytest.fixture(scope="module")
def setup(gpu_device):
    print(f"[setup] generating MXFP4 MoE weights {G}", flush=True)
    w = workloads.mxfp4_moe_weights(G, gpu_device, seed=0)
    rt = MoeRuntime(G, 16, gpu_device)
    torch.cuda.synchronize()
    cpu = dict(w13=CpuExperts(w.w13, True), s13=CpuExperts(w.s13), w2=CpuExperts(w.w2, True), s2=CpuExperts(w.s2))
    yield w, rt, cpu
    rt.close()


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30)).item()


def _run(rt, w, x, logits):
    out, dbg = rt.forward_mxfp4(x, logits, w, debug=True)
    torch.cuda.synchronize()
    return out.cpu(), {k: v.cpu() for k, v in dbg.items()}


def _check(out, dbg, x, logits, cpu):
    ids_ref, w_ref = otopk.softmax_topk(logits.cpu(), G.top_k)
    assert torch.equal(dbg["topk_ids"].long(), ids_ref), (dbg["topk_ids"], ids_ref)
    torch.testing.assert_close(dbg["topk_w"], w_ref, rtol=1e-5, atol=1e-6)
    ref = omoe.mxfp4_moe_block(
        x.cpu(), logits.cpu(), cpu["w13"], cpu["s13"], cpu["w2"], cpu["s2"], top_k=G.top_k, inter=G.inter,
    )  # fmt: skip
    y_rel = _rel(dbg["y"], ref["y"])
    print(f"[mxfp4 moe] rows={x.shape[0]} y rel={y_rel:.3e}", flush=True)
    assert y_rel < Y_REL
    err = (out.float() - ref["out"].float()).abs()
    # the bound as an (atol, rtol) pair, elementwise: |a - b| <= 2e-2 + 1e-2 |b|
    assert bool((err <= OUT_MAX_ABS + OUT_REL * ref["out"].float().abs()).all()), err.max().item()
    assert _rel(out, ref["out"]) <= OUT_REL


@pytest.mark.parametrize("rows", [1, 8, 16])
def test_mxfp4_moe_matches_oracle(setup, gpu_device, rows):
    w, rt, cpu = setup
    print(f"[mxfp4 moe] rows={rows}", flush=True)
    x = workloads.rows_bf16(rows, G.hidden, gpu_device, seed=300 + rows)
    logits = workloads.gate_logits(rows, G.n_experts, gpu_device, seed=400 + rows)
    out, dbg = _run(rt, w, x, logits)
    _check(out, dbg, x, logits, cpu)


def test_mxfp4_router_ties_take_lowest_ids(setup, gpu_device):
    """Ten experts share the top logit; the eight lowest ids win, each with weight 1/8
    of the softmax mass (glm53/gfx950/kernel.py:1575-1629)."""
    w, rt, cpu = setup
    logits = workloads.gate_logits(4, G.n_experts, gpu_device, seed=12)
    tied = list(range(90, 100))
    logits[:, tied] = 10.0
    x = workloads.rows_bf16(4, G.hidden, gpu_device, seed=13)
    out, dbg = _run(rt, w, x, logits)
    assert dbg["topk_ids"].tolist() == [tied[:8]] * 4
    assert torch.allclose(dbg["topk_w"], torch.full((4, 8), 0.125), atol=1e-6)
    _check(out, dbg, x, logits, cpu)


def test_mxfp4_moe_repeat_is_bitwise(setup, gpu_device):
    """Two launches in a row give identical bits; a narrower step after a wider one
    routes its rows as the wider step did."""
    w, rt, _ = setup
    x = workloads.rows_bf16(16, G.hidden, gpu_device, seed=17)
    logits = workloads.gate_logits(16, G.n_experts, gpu_device, seed=18)
    first, d1 = _run(rt, w, x, logits)
    second, d2 = _run(rt, w, x, logits)
    assert torch.equal(first, second) and torch.equal(d1["y"], d2["y"])
    small, ds = _run(rt, w, x[:5].contiguous(), logits[:5].contiguous())
    assert torch.equal(ds["topk_ids"], d1["topk_ids"][:5])


def test_mxfp4_moe_fail_stop_on_forced_wait(setup, gpu_device):
    """A wait the host forces to fail ends the launch with its site recorded; after
    the error is cleared the runtime computes the same bits as before. The launch waits
    at two sites (every workgroup routes the rows itself): the mid activations and
    the expert outputs."""
    w, rt, _ = setup
    x = workloads.rows_bf16(8, G.hidden, gpu_device, seed=21)
    logits = workloads.gate_logits(8, G.n_experts, gpu_device, seed=22)
    good, _ = _run(rt, w, x, logits)
    rt.check_errors()
    for site in (2, 3):
        print(f"[fault] forcing wait site {site}", flush=True)
        rt.set_deadline(0.02)
        rt.set_fault(site)
        _run(rt, w, x, logits)
        assert rt.error_words()[1] == site + 1, rt.error_words()
        with pytest.raises(Exception, match="stopped"):
            rt.check_errors()
        rt.set_fault(-1)
        rt.set_deadline(2.0)
        rt.clear_errors()
        again, _ = _run(rt, w, x, logits)
        rt.check_errors()
        assert torch.equal(again, good)


def test_mxfp4_moe_rejects_bad_args(setup, gpu_device):
    w, rt, _ = setup
    x = workloads.rows_bf16(2, G.hidden, gpu_device, seed=1)
    with pytest.raises(ValueError, match="logits"):
        rt.forward_mxfp4(x, workloads.gate_logits(2, G.n_experts - 1, gpu_device, seed=2), w)
    with pytest.raises(ValueError, match="dtype"):
        rt.forward_mxfp4(x.float(), workloads.gate_logits(2, G.n_experts, gpu_device, seed=2), w)
