"""FP8 routed MoE on the GPU against the CPU oracle.

Routing is checked bit-exact on identical inputs: the oracle's top-8 rule applied to
the device's own sigmoid scores must give the device's ids in the same order. The
expert outputs are then compared on that routing: the f32 MoE sum within 1e-2
relative (norm) and the bf16 output within the (atol 2e-2, rtol 1e-2) pair elementwise
and 1e-2 relative in norm.
"""

import pytest
import torch

from oracle import codecs as ocodecs
from oracle import moe as omoe
from oracle import topk as otopk
from sgl_amd_mono_amd import workloads
from sgl_amd_mono_amd.moe import FP8_MOE, MoeRuntime

pytestmark = pytest.mark.gpu

G = FP8_MOE
OUT_MAX_ABS, OUT_REL = 2e-2, 1e-2  # the north star's bf16 output bound
Y_REL = 1e-2  # the MoE sum itself (f32), relative to its norm
# Sigmoid scores. The f32 summation order of the RMSNorm's sum of squares can move rstd
# by an ulp, which flips the bf16 rounding of a normed element lying on a rounding
# boundary (about one row in five): that moves every logit of the row by |w_k| ulp(x_k)
# <= 0.08 * 2^-6 (|x_k| < 4, router weights within 3.4 sigma of 2 / sqrt(H)), a score by
# at most 0.25 of that, 3.1e-4. Without a flip the scores agree to ~1e-6 (GEMV order).
SCORE_ABS = 4e-4


class CpuExperts:
    """Expert tensors fetched to the CPU on first use (the oracle reads a few); the
    (16, 16)-shuffled FP8 matrices are unshuffled by the oracle's own gather."""

    def __init__(self, t, shuffled=False):
        self.t, self.shuffled, self.cache = t, shuffled, {}

    def __getitem__(self, e):
        if e not in self.cache:
            x = self.t[e].cpu()
            self.cache[e] = ocodecs.aiter_unshuffle(x) if self.shuffled else x
        return self.cache[e]


@pytest.fixture(scope="module")
def setup(gpu_device):
    print(f"[setup] generating FP8 MoE weights {G}", flush=True)
    w = workloads.fp8_moe_weights(G, gpu_device, seed=0)
    rt = MoeRuntime(G, 16, gpu_device)
    torch.cuda.synchronize()
    cpu = dict(
        g_post=w.g_post.cpu(), w_router=w.w_router.cpu(), bias=w.bias.cpu(),
        w13=CpuExperts(w.w13, True), s13=CpuExperts(w.s13), w2=CpuExperts(w.w2, True), s2=CpuExperts(w.s2),
    )  # fmt: skip
    yield w, rt, cpu
    rt.close()


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30)).item()


def _run(rt, w, a):
    out, dbg = rt.forward_fp8(a, w, debug=True)
    torch.cuda.synchronize()
    return out.cpu(), {k: v.cpu() for k, v in dbg.items()}


@pytest.mark.parametrize("rows", [1, 4, 8, 16])
def test_fp8_moe_matches_oracle(setup, gpu_device, rows):
    w, rt, cpu = setup
    print(f"[fp8 moe] rows={rows}", flush=True)
    a = workloads.rows_bf16(rows, G.hidden, gpu_device, seed=100 + rows)
    out, dbg = _run(rt, w, a)
    a_cpu = a.cpu()

    _, scores_ref = omoe.fp8_router(a_cpu, cpu["g_post"], cpu["w_router"], G.eps)
    assert (dbg["scores"] - scores_ref).abs().max().item() < SCORE_ABS

    ids_ref, w_ref = otopk.router_top8(dbg["scores"], cpu["bias"], G.top_k, G.route_scale)
    assert torch.equal(dbg["topk_ids"].long(), ids_ref), (dbg["topk_ids"], ids_ref)
    torch.testing.assert_close(dbg["topk_w"], w_ref, rtol=1e-5, atol=1e-6)

    ref = omoe.fp8_moe_block(
        a_cpu, cpu["g_post"], cpu["w_router"], cpu["bias"], cpu["w13"], cpu["s13"], cpu["w2"],
        cpu["s2"], eps=G.eps, top_k=G.top_k, inter=G.inter, ids=ids_ref, weights=w_ref,
    )  # fmt: skip
    y_rel = _rel(dbg["y"], ref["y"])
    print(f"[fp8 moe] rows={rows} y rel={y_rel:.3e}", flush=True)
    assert y_rel < Y_REL
    err = (out.float() - ref["out"].float()).abs()
    # the bound as an (atol, rtol) pair, elementwise: |a - b| <= 2e-2 + 1e-2 |b|
    assert bool((err <= OUT_MAX_ABS + OUT_REL * ref["out"].float().abs()).all()), err.max().item()
    assert _rel(out, ref["out"]) <= OUT_REL


def test_fp8_moe_repeat_is_bitwise_and_resets_counters(setup, gpu_device):
    """Two launches in a row give identical bits (the last-arrival counters return to
    zero and the plan order is deterministic); a narrower step after a wider one too."""
    w, rt, _ = setup
    a16 = workloads.rows_bf16(16, G.hidden, gpu_device, seed=7)
    first, d1 = _run(rt, w, a16)
    second, d2 = _run(rt, w, a16)
    assert torch.equal(first, second) and torch.equal(d1["y"], d2["y"])
    small, ds = _run(rt, w, a16[:3].contiguous())
    again, da = _run(rt, w, a16[:3].contiguous())
    assert torch.equal(small, again) and torch.equal(ds["topk_ids"], da["topk_ids"])
    # rows are independent: the 3-row step's routing equals the 16-row step's first rows
    assert torch.equal(ds["topk_ids"], d1["topk_ids"][:3])


def test_fp8_router_ties_take_lowest_ids(setup, gpu_device):
    """Ten experts with identical router rows and bias tie for the top; the eight lowest
    ids win (glm53/gfx950/kernel.py:1575-1629)."""
    w, rt, cpu = setup
    w_r = w.w_router.clone()
    bias = w.bias.clone()
    tied = list(range(40, 50))
    w_r[tied] = w_r[40].clone()
    bias[tied] = 5.0
    wt = type(w)(g_post=w.g_post, w_router=w_r, bias=bias, w13=w.w13, s13=w.s13, w2=w.w2, s2=w.s2)
    a = workloads.rows_bf16(4, G.hidden, gpu_device, seed=11)
    _, dbg = _run(rt, wt, a)
    assert dbg["topk_ids"].tolist() == [tied[:8]] * 4
    ids_ref, _ = otopk.router_top8(dbg["scores"], bias.cpu(), G.top_k, G.route_scale)
    assert torch.equal(dbg["topk_ids"].long(), ids_ref)


def test_fp8_moe_rejects_bad_shapes(setup, gpu_device):
    w, rt, _ = setup
    a = workloads.rows_bf16(17, G.hidden, gpu_device, seed=1)
    with pytest.raises(ValueError, match="rows"):
        rt.forward_fp8(a, w)
    a = workloads.rows_bf16(2, G.hidden, gpu_device, seed=1).float()
    with pytest.raises(ValueError, match="dtype"):
        rt.forward_fp8(a, w)


def test_fp8_moe_fail_stop_on_forced_wait(setup, gpu_device):
    """A wait the host forces to fail (guard.py:79-88) ends the launch with its site
    recorded; later launches refuse to run until the error is cleared, then the
    runtime computes the same bits as before."""
    w, rt, _ = setup
    a = workloads.rows_bf16(8, G.hidden, gpu_device, seed=21)
    good, _ = _run(rt, w, a)
    rt.check_errors()
    for site in (2, 3, 0):
        print(f"[fault] forcing wait site {site}", flush=True)
        rt.set_deadline(0.02)
        rt.set_fault(site)
        _run(rt, w, a)
        words = rt.error_words()
        assert words[1] == site + 1, words
        with pytest.raises(Exception, match="stopped"):
            rt.check_errors()
        rt.set_fault(-1)
        rt.set_deadline(2.0)
        _run(rt, w, a)  # sticky: exits at once, the error stays
        assert rt.error_words()[1] == site + 1
        rt.clear_errors()
        again, _ = _run(rt, w, a)
        rt.check_errors()
        assert torch.equal(again, good)


def test_fp8_moe_deadline_expiry_stops_the_launch(setup, gpu_device):
    """With a deadline of one 10 ns tick, a wait that has to spin passes its deadline:
    the launch stops with a valid site recorded instead of hanging, and the runtime
    recovers once the error is cleared and the deadline restored."""
    w, rt, _ = setup
    a = workloads.rows_bf16(8, G.hidden, gpu_device, seed=22)
    good, _ = _run(rt, w, a)
    rt.set_deadline(1e-8)
    _run(rt, w, a)
    words = rt.error_words()
    print(f"[deadline] guard words {words}", flush=True)
    assert 1 <= words[1] <= 4, words
    rt.set_deadline(2.0)
    rt.clear_errors()
    again, _ = _run(rt, w, a)
    rt.check_errors()
    assert torch.equal(again, good)
