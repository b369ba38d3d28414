"""The layer runtime's guard on the GPU: one count of launches for every launch of a layer
(whichever launches a caller mixes), tag epochs (tags repeat every 2^32 - 2 launches,
and the first launch of an epoch scrubs every mailbox, the reference's reason for its
own scrub: deepseek_v4/gfx950/kernels/layer.py:837-849), and the host-forced fault
armed a number of launches ahead (the reference's SGLANG_AMD_MONO_FAULT_INJECT
rank:site:after, common/guard.py:79-88).

Every comparison is bit for bit: a layer's outputs depend only on its inputs and the
caches, never on the tags its launches carry.
"""

import time

import pytest
import torch

from sgl_amd_mono_amd import _lib, workloads
from sgl_amd_mono_amd.layer import HIDDEN, LayerRuntime, LayerWeights
from sgl_amd_mono_amd.moe import FP8_MOE

pytestmark = pytest.mark.gpu

CTX = 4096
LENS = [4096, 1500, 65, 2049, 4000, 64, 3000, 300, 1024, 1025, 2048, 2047, 100, 3500, 700, 4095]


def _weights(dev, seed):
    return LayerWeights(proj=workloads.proj_weights(dev, seed=seed),
                        moe=workloads.fp8_moe_weights(FP8_MOE, dev, seed=seed + 1))


def _step(rt, rows, seed, dev, cos, sin, w, on_phase=None):
    """One launch of `rt` on a fresh seeded case of `rows` rows: its output, the caches'
    written planes, and the attention's selection."""
    step, caches = workloads.attn_case(LENS[:rows], dev, seed=seed, max_ctx=CTX)
    x = workloads.rows_bf16(rows, HIDDEN, dev, seed=seed + 1)
    out, it = rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin, keep=True, on_phase=on_phase)
    return out.clone(), it["topk_slots"], caches.kv.clone(), caches.ikv.clone()


def _same(a, b, what):
    for k, (u, v) in enumerate(zip(a, b)):
        assert torch.equal(u, v), (what, k)


def test_layer_mixed_launches_share_one_guard(gpu_device):
    """forward, forward with on_phase (front and the rest as two launches), forward again
    on ONE runtime: every launch takes its tag from one counter, so the front's done
    words of one call are never taken for the next call's. Each result equals the
    four-launch split's on the same inputs."""
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    w = _weights(gpu_device, 61)
    marks = []
    plan = [(8, 63, None), (8, 65, marks.append), (3, 67, None), (16, 69, marks.append), (16, 71, None)]
    rt = LayerRuntime(16, CTX, gpu_device)
    ref = LayerRuntime(16, CTX, gpu_device, mode="split")
    try:
        for rows, seed, hook in plan:
            print(f"[mixed] rows {rows} seed {seed} {'two launches' if hook else 'one launch'}", flush=True)
            got = _step(rt, rows, seed, gpu_device, cos, sin, w, on_phase=hook)
            want = _step(ref, rows, seed, gpu_device, cos, sin, w)
            torch.cuda.synchronize()
            rt.check_errors()
            ref.check_errors()
            _same(got, want, f"rows {rows} seed {seed}")
        assert marks == [0, 1, 0, 1]
    finally:
        rt.close()
        ref.close()


def test_layer_tag_epoch_wrap(gpu_device):
    """Launches at tags 1..3 leave words of those tags in every mailbox (16 rows); the
    ordinal then jumps three launches short of the wrap and six launches cross it, rows
    changing between 8, 16 and 3. The launch that starts the new epoch (tag 1 again)
    must scrub the stale words of the old tags 1..3 before anything polls them: every
    result equals a fresh runtime's on the same inputs, and the guard counts one epoch."""
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    w = _weights(gpu_device, 81)
    rt = LayerRuntime(16, CTX, gpu_device)
    fresh = LayerRuntime(16, CTX, gpu_device)
    try:
        for k in range(3):  # plant words of tags 1..3 (other inputs)
            print(f"[wrap] planting tag {k + 1}", flush=True)
            _step(rt, 16, 83 + 10 * k, gpu_device, cos, sin, w)
        torch.cuda.synchronize()
        rt.check_errors()
        rt.handle.set_launch_ordinal(_lib.TAG_PERIOD - 3)
        crossing = [(8, 201), (16, 203), (3, 205), (16, 207), (8, 209), (3, 211)]
        fresh_runs = []
        for i, (rows, seed) in enumerate(crossing):
            words = rt.handle.error_words()
            # guard words 4-5: the launches begun (the ordinal of the next launch)
            ordinal = (words[_lib.G_TICKET] & 0xFFFFFFFF) | (words[_lib.G_TICKET + 1] & 0xFFFFFFFF) << 32
            assert ordinal == _lib.TAG_PERIOD - 3 + i, (i, ordinal)
            print(f"[wrap] launch {i}: ordinal {ordinal}, tag {ordinal % _lib.TAG_PERIOD + 1}, rows {rows}", flush=True)
            got = _step(rt, rows, seed, gpu_device, cos, sin, w)
            torch.cuda.synchronize()
            rt.check_errors()
            fresh_runs.append((got, rows, seed))
        # a fresh runtime (no scrub, never wrapped) on the same inputs
        for got, rows, seed in fresh_runs:
            want = _step(fresh, rows, seed, gpu_device, cos, sin, w)
            torch.cuda.synchronize()
            fresh.check_errors()
            _same(got, want, f"rows {rows} seed {seed}")
        words = rt.handle.error_words()
        assert words[_lib.G_EPOCH] == 1, words
        assert words[_lib.G_ERROR] == 0, words
    finally:
        rt.close()
        fresh.close()


def test_layer_fault_armed_launches_ahead(gpu_device):
    """A fault armed `after` launches ahead (the reference's rank:site:after) lets that
    many launches run, then stops the next one at the site; the pinned host word
    reports it without a synchronisation."""
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    w = _weights(gpu_device, 91)
    rt = LayerRuntime(4, CTX, gpu_device)
    site = 8  # expert mid activations
    try:
        first = _step(rt, 4, 93, gpu_device, cos, sin, w)
        torch.cuda.synchronize()
        rt.handle.set_fault(site, after=2)
        for k in range(2):
            got = _step(rt, 4, 93, gpu_device, cos, sin, w)
            torch.cuda.synchronize()
            assert rt.handle.pending_error() == 0, k
            rt.check_errors()
            _same(got, first, f"armed launch {k}")
        bad = _step(rt, 4, 93, gpu_device, cos, sin, w)
        torch.cuda.synchronize()
        assert rt.handle.pending_error() == site + 1
        assert bool(bad[0].isnan().all())
        with pytest.raises(_lib.MonoError, match=_lib.LAYER_SITES[site]):
            rt.check_errors()
        rt.handle.set_fault(-1)
        rt.clear_errors()
        again = _step(rt, 4, 93, gpu_device, cos, sin, w)
        torch.cuda.synchronize()
        rt.check_errors()
        _same(again, first, "after clear")
    finally:
        rt.close()


def test_layer_fault_in_a_replayed_graph_reaches_the_watcher(gpu_device):
    """A step replayed from a HIP graph runs none of the plugin's host code, so the
    per-step check of the spec never sees it. The fail-stop watcher (a host thread on
    the pinned error word) must: a fault armed two launches ahead (before the capture,
    as the served path arms it at build: a launch's fault is one of its kernel
    arguments, which the graph keeps) stops the third replay, the watcher reports the
    site once (its default ends the process; here it records), later replays are
    refused, and after a clear an eager launch gives the first result again."""
    cos, sin = workloads.rope_tables(CTX, gpu_device)
    w = _weights(gpu_device, 95)
    rt = LayerRuntime(4, CTX, gpu_device)
    site = 9  # expert outputs
    seen = []
    try:
        step, caches = workloads.attn_case(LENS[:4], gpu_device, seed=97, max_ctx=CTX)
        x = workloads.rows_bf16(4, HIDDEN, gpu_device, seed=98)
        out = torch.empty(4, HIDDEN, dtype=torch.bfloat16, device=gpu_device)

        def launch():
            rt.forward(x, step.seq_lens, step.page_table, caches, w, cos, sin, out=out, check_weights=False)

        launch()
        torch.cuda.synchronize()
        rt.check_errors()
        first = out.clone()
        rt.handle.set_fault(site, after=2)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            launch()
        torch.cuda.synchronize()
        rt.handle.set_fault(-1)  # later eager launches run unarmed; the graph keeps its arguments
        watch = rt.watch(on_fail=seen.append)
        for k in range(2):
            print(f"[replay fault] replay {k} (armed)", flush=True)
            graph.replay()
            torch.cuda.synchronize()
            assert rt.handle.pending_error() == 0 and seen == [], k
            assert torch.equal(out, first), k
        print("[replay fault] replay 2 (fails at the site)", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        until = time.monotonic() + 5.0
        while not seen and time.monotonic() < until:
            time.sleep(1e-3)
        assert seen == [site + 1]
        assert bool(out.isnan().any())
        print("[replay fault] replay 3 (refused)", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert rt.handle.pending_error() == site + 1 and seen == [site + 1] and watch.code == site + 1
        rt.unwatch()
        rt.clear_errors()
        print("[replay fault] eager launch after clear", flush=True)
        launch()
        torch.cuda.synchronize()
        rt.check_errors()
        assert torch.equal(out, first)
    finally:
        rt.unwatch()
        rt.close()
