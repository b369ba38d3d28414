"""The multi-layer launch (mono_layer_stack_forward: every layer of a step in ONE
persistent launch) against one launch a layer (mono_layer_forward) on the same
inputs: each layer's output rows and caches bit for bit, over steps in a row, mixed
with one-layer launches on the same runtime (the guard's ordinals and launch-parity
copies), across a tag epoch, replayed from a HIP graph, and its fail-stop path."""

import pytest
import torch

from oracle import layer as ol
from sgl_amd_mono_amd import _lib, workloads
from sgl_amd_mono_amd.layer import LayerRuntime, LayerWeights
from sgl_amd_mono_amd.moe import FP8_MOE

pytestmark = pytest.mark.gpu

CTX = 8192


def _weights(dev, n, seed0):
    """n layers' weights; the layers reuse two seeded sets (weights are read-only)."""
    sets = [LayerWeights(proj=workloads.proj_weights(dev, seed=seed0 + 10 * k),
                         moe=workloads.fp8_moe_weights(FP8_MOE, dev, seed=seed0 + 10 * k + 1)) for k in range(2)]
    return [sets[l % 2] for l in range(n)]


def _case(dev, n, rows, seed):
    """Each layer's own caches (one attn_case a layer) and the step's input rows."""
    lens = ([CTX, 1500, 65, 2049, 4000, 64, 7000, 300] * 2)[:rows]
    steps, caches = [], []
    for l in range(n):
        st, c = workloads.attn_case(lens, dev, seed=seed + l, max_ctx=CTX)
        steps.append(st)
        caches.append(c)
    x = workloads.rows_bf16(rows, ol.HIDDEN, dev, seed=seed + 100)
    return steps, caches, x


def _clone(c):
    return type(c)(**{k: (None if getattr(c, k) is None else getattr(c, k).clone())
                      for k in ("ikv", "iks", "kv", "kv_scale")})


def _one_by_one(rt, x, steps, caches, ws, cos, sin):
    outs = []
    for l in range(len(ws)):
        x = rt.forward(x, steps[l].seq_lens, steps[l].page_table, caches[l], ws[l], cos, sin).clone()
        outs.append(x)
    return outs


def _stack(rt, x, steps, caches, ws, cos, sin):
    n = len(ws)
    last = rt.forward_layers(x, [s.seq_lens for s in steps], [s.page_table for s in steps], caches, ws, cos, sin)
    return [rt._xs[l, :x.shape[0]].clone() for l in range(n - 1)] + [last.clone()]


def _same(got, want, what):
    for l, (g, w) in enumerate(zip(got, want)):
        assert torch.equal(g, w), (what, l, float((g.float() - w.float()).abs().max()))


@pytest.mark.parametrize("rows,n", [(1, 3), (8, 4), (16, 2), (8, 1)])
def test_stack_equals_one_launch_a_layer(gpu_device, rows, n):
    """Every layer's output and caches equal the one-launch-a-layer run's, over two
    steps in a row; then a one-layer launch on the same runtime and a third stacked
    step (the stack takes an even count of ordinals, so the one-layer launch finds its
    launch-parity copies as it left them)."""
    print(f"[stack] rows={rows} layers={n}", flush=True)
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    ws = _weights(gpu_device, n, 300)
    steps, caches, x = _case(gpu_device, n, rows, 310)
    ref_caches = [_clone(c) for c in caches]
    ref = LayerRuntime(rows, CTX, gpu_device)
    rt = LayerRuntime(rows, CTX, gpu_device, max_layers=4)
    try:
        want = _one_by_one(ref, x, steps, ref_caches, ws, cos, sin)
        torch.cuda.synchronize()
        ref.check_errors()
        for k in range(2):
            got = _stack(rt, x, steps, caches, ws, cos, sin)
            torch.cuda.synchronize()
            rt.check_errors()
            _same(got, want, f"stacked step {k}")
        for c, r in zip(caches, ref_caches):
            for f in ("kv", "ikv", "iks", "kv_scale"):
                assert torch.equal(getattr(c, f), getattr(r, f)), f
        one = rt.forward(x, steps[0].seq_lens, steps[0].page_table, caches[0], ws[0], cos, sin).clone()
        got = _stack(rt, x, steps, caches, ws, cos, sin)
        torch.cuda.synchronize()
        rt.check_errors()
        assert torch.equal(one, want[0])
        _same(got, want, "stacked after a one-layer launch")
        words = rt.handle.error_words()
        ordinal = (words[_lib.G_TICKET] & 0xFFFFFFFF) | (words[_lib.G_TICKET + 1] & 0xFFFFFFFF) << 32
        assert ordinal == 3 * (n + n % 2) + 1, ordinal
    finally:
        rt.close()
        ref.close()


def test_stack_across_a_tag_epoch(gpu_device):
    """A stacked step whose third layer starts a tag epoch (its ordinal is a multiple of
    the tag period): that layer meets the whole grid and scrubs every mailbox, the
    layers before's done words included, and still equals the one-launch-a-layer run."""
    n, rows = 4, 8
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    ws = _weights(gpu_device, n, 400)
    steps, caches, x = _case(gpu_device, n, rows, 410)
    ref_caches = [_clone(c) for c in caches]
    ref = LayerRuntime(rows, CTX, gpu_device)
    rt = LayerRuntime(rows, CTX, gpu_device, max_layers=n)
    try:
        want = _one_by_one(ref, x, steps, ref_caches, ws, cos, sin)
        got = _stack(rt, x, steps, caches, ws, cos, sin)  # plant words of the first tags
        torch.cuda.synchronize()
        rt.check_errors()
        _same(got, want, "before the epoch")
        rt.handle.set_launch_ordinal(_lib.TAG_PERIOD - 2)
        print("[stack epoch] layers at ordinals P-2 .. P+1", flush=True)
        for k in range(2):
            got = _stack(rt, x, steps, caches, ws, cos, sin)
            torch.cuda.synchronize()
            rt.check_errors()
            _same(got, want, f"across the epoch, step {k}")
        words = rt.handle.error_words()
        assert words[_lib.G_EPOCH] == 1, words
    finally:
        rt.close()
        ref.close()


def test_stack_replayed_from_a_graph(gpu_device):
    """A stacked step captured in a HIP graph once its arguments are set: three replays
    with eager work between them each equal the eager step."""
    n, rows = 3, 8
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    ws = _weights(gpu_device, n, 500)
    steps, caches, x = _case(gpu_device, n, rows, 510)
    rt = LayerRuntime(rows, CTX, gpu_device, max_layers=n)
    try:
        eager = _stack(rt, x, steps, caches, ws, cos, sin)
        torch.cuda.synchronize()
        rt.check_errors()
        lens, tables = [s.seq_lens for s in steps], [s.page_table for s in steps]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = rt.forward_layers(x, lens, tables, caches, ws, cos, sin)
        for k in range(3):
            g.replay()
            torch.cuda.synchronize()
            rt.check_errors()
            assert torch.equal(out, eager[-1]), k
            for l in range(n - 1):
                assert torch.equal(rt._xs[l, :rows], eager[l]), (k, l)
            _ = (x.float() * 2).sum().item()  # eager work between the replays
    finally:
        rt.close()


@pytest.mark.parametrize("site,after,what", [(19, 0, "the layer before's output rows"),
                                             (11, 2, "front: stage-A partial sums")])
def test_stack_fail_stop(gpu_device, site, after, what):
    """A forced wait failure in a later layer of a stacked step (the second layer's
    wait on the first's output rows; the third layer's front) stops the launch without
    a fault: the host word names the site, the last layer's output is NaN (workgroups
    still in an earlier layer stop at their next wait too), the next launch is refused,
    and after a clear the step equals the good one."""
    n, rows = 3, 2
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    ws = _weights(gpu_device, n, 600)
    steps, caches, x = _case(gpu_device, n, rows, 610)
    rt = LayerRuntime(rows, CTX, gpu_device, max_layers=n)
    try:
        rt.set_deadline(0.5)
        good = _stack(rt, x, steps, caches, ws, cos, sin)
        torch.cuda.synchronize()
        rt.check_errors()
        rt.handle.set_fault(site, after)
        bad = _stack(rt, x, steps, caches, ws, cos, sin)
        torch.cuda.synchronize()
        assert rt.handle.pending_error() == site + 1
        with pytest.raises(Exception, match=what):
            rt.raise_pending()
        assert bool(bad[-1].isnan().all()), "a failed launch's last output is NaN"
        rt.handle.set_fault(-1)
        refused = _stack(rt, x, steps, caches, ws, cos, sin)
        torch.cuda.synchronize()
        assert bool(refused[-1].isnan().all()), "a refused launch's last output is NaN"
        rt.clear_errors()
        again = _stack(rt, x, steps, caches, ws, cos, sin)
        torch.cuda.synchronize()
        rt.check_errors()
        _same(again, good, "after the clear")
    finally:
        rt.close()


def test_stack_refuses_shared_buffers(gpu_device):
    """The packer refuses layers whose caches (or outputs) share memory: a later layer
    would reread lines an earlier one cached."""
    n, rows = 2, 1
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    ws = _weights(gpu_device, n, 700)
    steps, caches, x = _case(gpu_device, n, rows, 710)
    rt = LayerRuntime(rows, CTX, gpu_device, max_layers=n)
    try:
        with pytest.raises(ValueError, match="overlaps"):  # MONO_EINVAL
            rt.forward_layers(x, steps[0].seq_lens, steps[0].page_table, [caches[0], caches[0]], ws, cos, sin)
        with pytest.raises(ValueError, match="max_layers"):
            rt.forward_layers(x, steps[0].seq_lens, steps[0].page_table, caches * 2, ws * 2, cos, sin)
    finally:
        rt.close()
