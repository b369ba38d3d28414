"""Benchmark of the decoder-layer path on one MI355X (gfx950).

``python bench.py [--workload layer] [--steps K] [--warmup W] [--rows 8]`` prints one
JSON line. A step is one pass of the hot path over one batch of synthetic decode rows
whose inputs and weights are already resident in HBM:

* ``layer`` (default): 61 stacked, independently seeded decoder
  layers at 8 rows over 32768-key contexts. Each layer is one persistent pass (front,
  sparse attention, back and FP8 MoE); by default the 61 layers of a step run as ONE
  launch (``k_layers``, ``--launch stack``), or one launch a layer (``k_layer``,
  ``--launch layer``). The step is replayed from a HIP graph. ``value`` is
  microseconds per layer.
* ``moe_fp8`` (BASELINE config 2 at 8 rows): the FP8 routed + shared MoE half of the
  layer (RMSNorm, router, top-8, W8A8 experts, residual) through ``mono_moe_fp8_forward``.
* ``moe_mxfp4``: the MXFP4 A16W4 routed + shared MoE behind a
  softmax router through ``mono_moe_mxfp4_forward``.
* ``attn``: FP4 index scores over ``--ctx`` keys a row, the exact
  top-2048 and sparse MLA decode, through ``mono_attn_forward``.

Weights never repeat within ~1.5 GB of streamed bytes (rotating weight sets for the
single-phase workloads; 61 distinct layers for ``layer``), so every step streams from
HBM rather than from the 256 MB Infinity Cache. The timed region is K steps bracketed
by ``torch.cuda.synchronize()``; HIP events on the launch stream time each step.
``roofline`` prices the dominant kernel's algorithmic bytes (distinct experts read
once, the router once, activations in and out) against 8 TB/s. ``cpu_baseline`` times
the CPU oracle's restatement of the same work on this host (rank 0 only, a bounded
sample) as a reported baseline.

Only one GPU is used: ``--gpus`` above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "µs per decoder layer at 8 rows; MoE/attn achieved HBM TB/s vs 8 TB/s peak"
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_steps(args, dev, step, reps: int = 5):
    """``args.warmup`` untimed calls of ``step(i)``; then the next ``args.steps`` calls
    captured in one HIP graph (the launches run back to back, with no host work between
    them) and the graph replayed ``reps`` times, each replay bracketed by HIP events on
    the launch stream. Falls back to timing the calls eagerly (an event after each) when
    the capture fails. Returns (per-replay us a step, mean us a step, wall s a replay,
    how it was timed)."""
    import torch

    if args.pmc_pass:  # counter runs: eager launches (the profiler sees each) + calibration
        for i in range(args.warmup + args.steps):
            step(i)
        calibration_copy(dev)
        print(json.dumps({"pmc_pass": True, "workload": args.workload, "launches": args.warmup + args.steps,
                          "rows": args.rows, "calib_copy_bytes": CALIB_BYTES}), flush=True)
        raise PmcPassDone()
    log(f"warmup {args.warmup} steps")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    graph = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(graph):
            for i in range(args.steps):
                step(args.warmup + i)
        torch.cuda.synchronize()
        graph.replay()  # untimed
        torch.cuda.synchronize()
    except RuntimeError as e:  # pragma: no cover - a path that cannot be captured
        log(f"graph capture failed ({e}); timing eager launches")
        graph = None
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    log(f"timing {reps} x {args.steps} steps" + (" (graph replays)" if graph is not None else " (eager)"))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for k in range(reps):
        if graph is not None:
            graph.replay()
        else:
            for i in range(args.steps):
                step(args.warmup + i)
        ev[k + 1].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / reps
    per = [ev[k].elapsed_time(ev[k + 1]) * 1e3 / args.steps for k in range(reps)]
    return per, statistics.fmean(per), wall, ("graph" if graph is not None else "eager")


# ------------------------------------------------------------------ FP8 MoE (config 2)
def fp8_expert_bytes(geo) -> int:
    """Bytes of one FP8 expert: w13 [2I, H] + w2 [H, I] E4M3 and their f32 block scales."""
    H, I = geo.hidden, geo.inter
    return 2 * I * H + H * I + 4 * ((2 * I // 128) * (H // 128) + (H // 128) * (I // 128))


def bench_moe_fp8(args, dev):
    import torch

    from sgl_amd_mono_amd import workloads
    from sgl_amd_mono_amd.moe import FP8_MOE, MoeRuntime

    G = FP8_MOE
    H, E = G.hidden, G.n_experts
    S = args.rows
    log(f"generating {args.sets} FP8 MoE weight sets (H={H} E={E}+1 I={G.inter}) on {dev}")
    wsets = [workloads.fp8_moe_weights(G, dev, seed=1000 + i) for i in range(args.sets)]
    acts = [workloads.rows_bf16(S, H, dev, seed=2000 + i) for i in range(args.batches)]
    rt = MoeRuntime(G, max(S, 1), dev)
    out = torch.empty(S, H, dtype=torch.bfloat16, device=dev)
    n_combo = len(wsets) * len(acts)

    # distinct experts a (weight set, batch) pair touches: from the device's own routing
    distinct = {}
    for wi, w in enumerate(wsets):
        for ai, a in enumerate(acts):
            _, dbg = rt.forward_fp8(a, w, debug=True)
            distinct[(wi, ai)] = len(set(dbg["topk_ids"].flatten().tolist())) + 1  # + shared
    torch.cuda.synchronize()

    def pair(i):
        return i % len(wsets), (i // len(wsets)) % len(acts)

    def step(i):
        wi, ai = pair(i)
        rt.forward_fp8(acts[ai], wsets[wi], out=out)

    per, us, wall, how = time_steps(args, dev, step)
    rt.check_errors()

    exp_b = fp8_expert_bytes(G)
    fixed = E * H * 2 + E * 4 + H * 2 + 2 * S * H * 2  # router, bias, norm weight, a in + out
    step_bytes = [distinct[pair(args.warmup + i)] * exp_b + fixed for i in range(args.steps)]
    mean_bytes = statistics.fmean(step_bytes)
    achieved = mean_bytes / (us * 1e-6) / 1e9  # GB/s
    d_mean = statistics.fmean(distinct[pair(args.warmup + i)] for i in range(args.steps))
    log(f"{us:.2f} us/step (median {statistics.median(per):.2f}), {achieved:.0f} GB/s, "
        f"{d_mean:.1f} distinct experts, wall {wall:.3f} s")

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline_moe_fp8(args, wsets[0], acts, G)
    rt.close()
    return dict(
        value=us,
        unit="us",
        ms_per_step=us / 1e3,
        dtype="fp8_e4m3 (f32 accumulate)",
        config=dict(
            workload="BASELINE config 2: FP8 routed MoE decode, one GPU's TP=4 share",
            rows=S, hidden=H, experts=E, top_k=G.top_k, shared_experts=1, inter=G.inter,
            weight_sets=len(wsets), activation_batches=len(acts), combos=n_combo, timed=how,
        ),
        extra=dict(
            us_median=statistics.median(per), us_min=min(per), us_max=max(per),
            rows_per_s=S / (us * 1e-6), distinct_experts_mean=d_mean,
            algorithmic_bytes_mean=mean_bytes,
        ),
        roofline=dict(
            bound="hbm", achieved=achieved, peak=HBM_PEAK_GBS, unit="GB/s",
            frac=achieved / HBM_PEAK_GBS, traffic=None,
            kernel="k_moe_fp8 (one persistent launch: router, route, up, down, final)",
            bytes_per_launch=mean_bytes, avg_launch_us=statistics.fmean(per),
        ),
        cpu_baseline=cpu,
    )


def cpu_baseline_moe_fp8(args, w, acts, G):
    """The CPU oracle's FP8 MoE block (its own router and experts) on this host."""
    import torch

    from oracle import codecs as ocodecs
    from oracle import moe as omoe

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)

    class Lazy:
        """Experts fetched on first use; (16, 16)-shuffled FP8 matrices unshuffled."""

        def __init__(self, t, shuffled=False):
            self.t, self.shuffled, self.c = t, shuffled, {}

        def __getitem__(self, e):
            if e not in self.c:
                x = self.t[e].cpu()
                self.c[e] = ocodecs.aiter_unshuffle(x) if self.shuffled else x
            return self.c[e]

    cw = dict(g_post=w.g_post.cpu(), w_router=w.w_router.cpu(), bias=w.bias.cpu(),
              w13=Lazy(w.w13, True), s13=Lazy(w.s13), w2=Lazy(w.w2, True), s2=Lazy(w.s2))
    batches = [a.cpu() for a in acts]

    def one(a):
        return omoe.fp8_moe_block(a, cw["g_post"], cw["w_router"], cw["bias"], cw["w13"], cw["s13"],
                                  cw["w2"], cw["s2"], eps=G.eps, top_k=G.top_k, inter=G.inter)

    for a in batches[:2]:  # warm-up, and fetch the experts these batches touch
        one(a)
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    i = 0
    while (len(times) < 5 or time.perf_counter() < t_end) and len(times) < 50:
        a = batches[i % 2]
        t = time.perf_counter()
        one(a)
        times.append((time.perf_counter() - t) * 1e6)
        i += 1
    med = statistics.median(times)
    log(f"cpu oracle: {med:.0f} us/step median of {len(times)} on {threads} threads")
    return dict(
        value=med, unit="us", cores=torch.get_num_threads(), kind="port",
        sample=(f"oracle.moe.fp8_moe_block (f32 torch restatement) on {len(times)} steps of "
                f"{args.rows} rows, alternating 2 activation batches of weight set 0; median; "
                f"host '{cpu_model()}', os.cpu_count()={os.cpu_count()}"),
    )


# ------------------------------------------------------------------ MXFP4 MoE (config 4)
def mxfp4_expert_bytes(geo) -> int:
    """Bytes of one MXFP4 expert: w13 [2I, H] + w2 [H, I] E2M1 (two a byte) and their
    E8M0 scales (one a 32 values)."""
    H, I = geo.hidden, geo.inter
    return (3 * I * H) // 2 + (3 * I * H) // 32


def bench_moe_mxfp4(args, dev):
    import torch

    from sgl_amd_mono_amd import workloads
    from sgl_amd_mono_amd.moe import MXFP4_MOE, MoeRuntime

    G = MXFP4_MOE
    H, E = G.hidden, G.n_experts
    S = args.rows
    n_sets = max(args.sets, 8)  # 483 MB a set: 8 sets keep the experts out of the Infinity Cache
    log(f"generating {n_sets} MXFP4 MoE weight sets (H={H} E={E}+1 I={G.inter}) on {dev}")
    wsets = [workloads.mxfp4_moe_weights(G, dev, seed=1100 + i) for i in range(n_sets)]
    acts = [workloads.rows_bf16(S, H, dev, seed=2100 + i) for i in range(args.batches)]
    lgts = [workloads.gate_logits(S, E, dev, seed=2200 + i) for i in range(args.batches)]
    rt = MoeRuntime(G, max(S, 1), dev)
    out = torch.empty(S, H, dtype=torch.bfloat16, device=dev)

    def pair(i):
        return i % len(wsets), (i // len(wsets)) % len(acts)

    distinct = {}
    for ai in range(len(acts)):  # routing depends on the logits only
        _, dbg = rt.forward_mxfp4(acts[ai], lgts[ai], wsets[0], debug=True)
        distinct[ai] = len(set(dbg["topk_ids"].flatten().tolist())) + 1  # + shared
    torch.cuda.synchronize()

    def step(i):
        wi, ai = pair(i)
        rt.forward_mxfp4(acts[ai], lgts[ai], wsets[wi], out=out)

    per, us, wall, how = time_steps(args, dev, step)
    rt.check_errors()

    exp_b = mxfp4_expert_bytes(G)
    fixed = S * E * 4 + 2 * S * H * 2  # logits, x in + out
    step_bytes = [distinct[pair(args.warmup + i)[1]] * exp_b + fixed for i in range(args.steps)]
    mean_bytes = statistics.fmean(step_bytes)
    achieved = mean_bytes / (us * 1e-6) / 1e9
    d_mean = statistics.fmean(distinct[pair(args.warmup + i)[1]] for i in range(args.steps))
    log(f"{us:.2f} us/step (median {statistics.median(per):.2f}), {achieved:.0f} GB/s, "
        f"{d_mean:.1f} distinct experts, wall {wall:.3f} s")

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline_moe_mxfp4(args, wsets[0], acts, lgts, G)
    rt.close()
    return dict(
        value=us,
        unit="us",
        ms_per_step=us / 1e3,
        dtype="bf16 x mxfp4 (f32 accumulate)",
        config=dict(
            workload="BASELINE config 4: MXFP4 A16W4 routed MoE decode, one GPU's TP=4 share",
            rows=S, hidden=H, experts=E, top_k=G.top_k, shared_experts=1, inter=G.inter,
            weight_sets=len(wsets), activation_batches=len(acts), timed=how,
        ),
        extra=dict(
            us_median=statistics.median(per), us_min=min(per), us_max=max(per),
            rows_per_s=S / (us * 1e-6), distinct_experts_mean=d_mean,
            algorithmic_bytes_mean=mean_bytes,
        ),
        roofline=dict(
            bound="hbm", achieved=achieved, peak=HBM_PEAK_GBS, unit="GB/s",
            frac=achieved / HBM_PEAK_GBS, traffic=None,
            kernel="k_moe_mxfp4 (one persistent launch: route, up, down, final)",
            bytes_per_launch=mean_bytes, avg_launch_us=statistics.fmean(per),
        ),
        cpu_baseline=cpu,
    )


def cpu_baseline_moe_mxfp4(args, w, acts, lgts, G):
    """The CPU oracle's MXFP4 MoE block (its own router and experts) on this host."""
    import torch

    from oracle import codecs as ocodecs
    from oracle import moe as omoe

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)

    class Lazy:
        def __init__(self, t, shuffled=False):
            self.t, self.shuffled, self.c = t, shuffled, {}

        def __getitem__(self, e):
            if e not in self.c:
                x = self.t[e].cpu()
                self.c[e] = ocodecs.aiter_unshuffle(x) if self.shuffled else x
            return self.c[e]

    cw = [Lazy(w.w13, True), Lazy(w.s13), Lazy(w.w2, True), Lazy(w.s2)]
    batches = [(a.cpu(), lg.cpu()) for a, lg in zip(acts[:2], lgts[:2])]

    def one(b):
        return omoe.mxfp4_moe_block(b[0], b[1], *cw, top_k=G.top_k, inter=G.inter)

    for b in batches:
        one(b)
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    i = 0
    while (len(times) < 5 or time.perf_counter() < t_end) and len(times) < 50:
        t = time.perf_counter()
        one(batches[i % 2])
        times.append((time.perf_counter() - t) * 1e6)
        i += 1
    med = statistics.median(times)
    log(f"cpu oracle: {med:.0f} us/step median of {len(times)} on {threads} threads")
    return dict(
        value=med, unit="us", cores=torch.get_num_threads(), kind="port",
        sample=(f"oracle.moe.mxfp4_moe_block (f32 torch restatement) on {len(times)} steps of "
                f"{args.rows} rows, alternating 2 batches of weight set 0; median; "
                f"host '{cpu_model()}', os.cpu_count()={os.cpu_count()}"),
    )


# ------------------------------------------------------------------ sparse attention (config 3)
def attn_step_bytes(ctx_lens) -> int:
    """Algorithmic bytes of one attention step: every index key of every row (16 B of
    E2M1 + 1 E8M0 byte per 32 dims = 68 B a key), the selected cache rows (576 B of E4M3 +
    a 4-byte scale), the row's queries (FP4 index query + scales + weights, bf16 q), its
    page-table entries, and the bf16 output."""
    total = 0
    for n in ctx_lens:
        sel = min(n, 2048)
        total += n * 68 + sel * 580 + (64 * 64 + 64 * 4 + 64 * 2) + 32 * 576 * 2 + (-(-n // 64)) * 4 + 32 * 512 * 2
    return total


def bench_attn(args, dev):
    import torch

    from sgl_amd_mono_amd import workloads
    from sgl_amd_mono_amd.attn import AttnRuntime

    S, ctx = args.rows, args.ctx
    lens = [ctx] * S
    step_b = attn_step_bytes(lens)
    sets = max(args.sets, -(-1_500_000_000 // step_b))  # > 1.5 GB streamed before a set repeats
    log(f"generating {sets} attention cases of {S} rows x {ctx} keys ({step_b / 1e6:.1f} MB a step)")
    cases = [workloads.attn_case(lens, dev, seed=3000 + i) for i in range(sets)]
    rt = AttnRuntime(S, max(ctx, 1024), device=dev)
    out = torch.empty(S, 32, 512, dtype=torch.bfloat16, device=dev)

    def step(i):
        st, ca = cases[i % sets]
        rt.forward(st, ca, out=out)

    per, us, wall, how = time_steps(args, dev, step)
    rt.check_errors()
    achieved = step_b / (us * 1e-6) / 1e9
    log(f"{us:.2f} us/step (median {statistics.median(per):.2f}), {achieved:.0f} GB/s")
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline_attn(args, cases[0])
    rt.close()
    return dict(
        value=us, unit="us", ms_per_step=us / 1e3, dtype="fp4_e2m1 scores, fp8_e4m3 kv (bf16 MFMA, f32 accumulate)",
        config=dict(workload="BASELINE config 3: sparse MLA decode with FP4 indexer top-2048", rows=S,
                    context=ctx, heads=32, index_heads=64, topk=2048, cache_sets=sets, timed=how),
        extra=dict(us_median=statistics.median(per), us_min=min(per), us_max=max(per),
                   rows_per_s=S / (us * 1e-6), algorithmic_bytes=step_b),
        roofline=dict(bound="hbm", achieved=achieved, peak=HBM_PEAK_GBS, unit="GB/s", frac=achieved / HBM_PEAK_GBS,
                      traffic=None, kernel="k_attn (one persistent launch: score, top-k, split, merge)",
                      bytes_per_launch=step_b, avg_launch_us=statistics.fmean(per)),
        cpu_baseline=cpu,
    )


def cpu_baseline_attn(args, case):
    """The CPU oracle's attention step (index scores, exact top-2048, sparse MLA)."""
    import torch

    from oracle import attention as oatt

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    st, ca = case
    c = {k: v.cpu() for k, v in vars(ca).items()}
    s = {k: v.cpu() for k, v in vars(st).items()}

    def one():
        sc = oatt.index_scores(s["iq"], s["iqs"], s["iw"], c["ikv"], c["iks"], s["page_table"], s["seq_lens"],
                               args.ctx)
        sel = oatt.select_topk(sc, s["seq_lens"], s["page_table"])
        return oatt.sparse_mla(s["q"], c["kv"], c["kv_scale"], sel)

    one()
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    while (len(times) < 3 or time.perf_counter() < t_end) and len(times) < 20:
        t = time.perf_counter()
        one()
        times.append((time.perf_counter() - t) * 1e6)
    med = statistics.median(times)
    log(f"cpu oracle: {med:.0f} us/step median of {len(times)} on {threads} threads")
    return dict(value=med, unit="us", cores=torch.get_num_threads(), kind="port",
                sample=(f"oracle.attention index_scores + select_topk + sparse_mla (f32 torch restatement) on "
                        f"{len(times)} steps of {args.rows} rows x {args.ctx} keys, one cache set; median; "
                        f"host '{cpu_model()}', os.cpu_count()={os.cpu_count()}"))


# ------------------------------------------------------------------ full layer (config 5)
def proj_bytes(w, names) -> int:
    return sum(getattr(w, n).numel() * getattr(w, n).element_size() for n in names)


FRONT_W = ("g_in", "w_qkv", "s_qkv", "w_ik", "s_ik", "w_iw", "g_q", "g_kv", "g_ik", "b_ik", "w_qb", "s_qb",
           "w_iq", "s_iq", "w_uk", "s_uk")
BACK_W = ("w_uv", "s_uv", "w_o", "s_o")


def bench_layer(args, dev):
    """``--layers`` (61) stacked, independently seeded decoder layers
    at ``--rows`` (8) rows, every row a ``--ctx``-key (32768) request whose new token is
    its last. One step runs all layers once, as ONE persistent launch (``--launch
    stack``, the default) or one launch a layer (``--launch layer``); it is captured in a
    HIP graph and replayed, so host dispatch is off the timed path. The value is
    microseconds per layer. The stacked step's output is first checked bit for bit
    against the chained one-launch-a-layer step. A second region runs the step eagerly
    with HIP event pairs around the launches (the launch duration for ``roofline``);
    in-kernel ticks give the phase breakdown."""
    import torch

    from sgl_amd_mono_amd import workloads
    from sgl_amd_mono_amd.layer import LayerRuntime, LayerWeights
    from sgl_amd_mono_amd.moe import FP8_MOE

    L, S, ctx = args.layers, args.rows, args.ctx
    lens = [ctx] * S
    log(f"generating {L} layers (seeds 1000 l + 7) of weights and {S} x {ctx}-key caches on {dev}")
    t0 = time.perf_counter()
    layers = []
    for l in range(L):
        seed = 1000 * l + 7
        w = LayerWeights(proj=workloads.proj_weights(dev, seed=seed),
                         moe=workloads.fp8_moe_weights(FP8_MOE, dev, seed=seed + 1))
        step, caches = workloads.attn_case(lens, dev, seed=seed + 2, max_ctx=ctx)
        layers.append((w, step, caches))
    cos, sin = workloads.rope_tables(ctx, dev)
    torch.cuda.synchronize()
    log(f"generated in {time.perf_counter() - t0:.1f} s; {torch.cuda.memory_allocated(dev) / 1e9:.1f} GB allocated")
    rt = LayerRuntime(S, ctx, dev, mode=args.mode)
    x_in = workloads.rows_bf16(S, 7168, dev, seed=5)
    xb = [torch.empty_like(x_in), torch.empty_like(x_in)]
    # --routing uniform: every layer takes its own independent random rows instead of the
    # previous layer's output, and its router bias is zeroed (the synthetic bias, ~N(0,
    # 0.1), outweighs the spread of the top scores, which sit near 1, and sends every row
    # to the same experts), so the rows route independently: about 57.4 distinct experts
    # of 256 at 8 rows x top-8, the traffic of uniform routing
    own_rows = None
    if args.routing == "uniform":
        own_rows = [workloads.rows_bf16(S, 7168, dev, seed=5 + l) for l in range(L)]
        for w, _, _ in layers:
            w.moe.bias.zero_()

    def layer_in(l, x):
        return x if own_rows is None else own_rows[l]

    def run_step(marks=None):
        x = x_in
        for l, (w, step, caches) in enumerate(layers):
            hook = None if marks is None else (lambda i, l=l: marks(l, i))
            x = rt.forward(layer_in(l, x), step.seq_lens, step.page_table, caches, w, cos, sin, out=xb[l % 2],
                           check_weights=False, on_phase=hook)
        return x

    # validation pass: routing per layer (distinct experts), and the weights' shapes
    distinct = []
    x = x_in
    for l, (w, step, caches) in enumerate(layers):
        w.proj.check(rt.device)
        x, it = rt.forward(layer_in(l, x), step.seq_lens, step.page_table, caches, w, cos, sin, out=xb[l % 2],
                           keep=True)
        distinct.append(len(set(it["topk_ids"].flatten().tolist())) + 1)
    torch.cuda.synchronize()
    rt.check_errors()

    stacked = args.launch == "stack"
    stack_parity = None
    if stacked:
        # every layer of the step as ONE launch (mono_layer_stack_forward); its output
        # must equal the chained one-launch-a-layer step's bit for bit
        chained = x.clone()
        srt = LayerRuntime(S, ctx, dev, mode="layer", max_layers=L)
        ws_l = [w for w, _, _ in layers]
        caches_l = [c for _, _, c in layers]
        lens_l = [st.seq_lens for _, st, _ in layers]
        pts_l = [st.page_table for _, st, _ in layers]

        def run_step(marks=None, ticks=None):
            return srt.forward_layers(x_in, lens_l, pts_l, caches_l, ws_l, cos, sin, check_weights=False,
                                      ticks=ticks)

        got = run_step()
        torch.cuda.synchronize()
        srt.check_errors()
        stack_parity = bool(torch.equal(got, chained))
        log(f"stacked step (one launch, {L} layers) equals the chained one-launch-a-layer step: {stack_parity}")
        if not stack_parity:
            raise RuntimeError("the stacked step differs from the chained one-launch-a-layer step")
        rt.close()
        rt = srt

    if args.pmc_pass:
        return pmc_pass(args, dev, run_step, distinct)
    for _ in range(max(args.warmup, 1)):
        run_step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_step()
    torch.cuda.synchronize()
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    rt.check_errors()

    stream = torch.cuda.current_stream(dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    log(f"timing {args.steps} graph replays of {L} layers")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(args.steps):
        graph.replay()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    rt.check_errors()
    per = [ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(args.steps)]  # us a step
    step_us = ev[0].elapsed_time(ev[-1]) * 1e3 / args.steps
    us = step_us / L

    # eager pass with phase events: the breakdown and the MoE launch durations
    n_eager = max(1, min(3, args.steps))
    phases = ("layers",) if stacked else rt.phases  # front, then attention + back + MoE (one launch) by default
    ph = {p: [] for p in phases}
    if stacked:  # one launch a step: an event pair around it, each layer its mean share
        sev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_eager)]
        torch.cuda.synchronize()
        for k in range(n_eager):
            sev[k][0].record(stream)
            run_step()
            sev[k][1].record(stream)
        torch.cuda.synchronize()
        rt.check_errors()
        step_durs = [a.elapsed_time(b) * 1e3 for a, b in sev]
        ph["layers"] = [d / L for d in step_durs]
    else:
        pev = [[[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(L)]
               for _ in range(n_eager)]
        torch.cuda.synchronize()
        for k in range(n_eager):
            x = x_in
            for l, (w, step, caches) in enumerate(layers):
                pev[k][l][0].record(stream)
                x = rt.forward(layer_in(l, x), step.seq_lens, step.page_table, caches, w, cos, sin, out=xb[l % 2],
                               check_weights=False, on_phase=lambda i, l=l, k=k: pev[k][l][i + 1].record(stream))
        torch.cuda.synchronize()
        rt.check_errors()
        for k in range(n_eager):
            for l in range(L):
                for i, p in enumerate(phases):
                    ph[p].append(pev[k][l][i].elapsed_time(pev[k][l][i + 1]) * 1e3)
    ph_us = {p: statistics.fmean(v) for p, v in ph.items()}
    eager_layer_us = sum(ph_us.values())
    # one launch a layer: each layer's launch timed alone (an event pair around it, eager)
    one = rt.launches == 1 and not stacked
    layer_durs = []
    if one:
        lev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(L)]
               for _ in range(n_eager)]
        torch.cuda.synchronize()
        for k in range(n_eager):
            x = x_in
            for l, (w, step, caches) in enumerate(layers):
                lev[k][l][0].record(stream)
                x = rt.forward(layer_in(l, x), step.seq_lens, step.page_table, caches, w, cos, sin, out=xb[l % 2],
                               check_weights=False)
                lev[k][l][1].record(stream)
        torch.cuda.synchronize()
        rt.check_errors()
        layer_durs = [lev[k][l][0].elapsed_time(lev[k][l][1]) * 1e3 for k in range(n_eager) for l in range(L)]

    # eager pass with in-kernel phase ticks (one launch a layer): the critical path and
    # each phase's span inside the launch
    stamped = None
    if one or stacked:
        grid = torch.cuda.get_device_properties(dev).multi_processor_count
        ticks = torch.zeros(n_eager, L, grid, 16, dtype=torch.int64, device=dev)
        torch.cuda.synchronize()
        for k in range(n_eager):
            if stacked:
                run_step(ticks=ticks[k])
                continue
            x = x_in
            for l, (w, step, caches) in enumerate(layers):
                x = rt.forward(layer_in(l, x), step.seq_lens, step.page_table, caches, w, cos, sin, out=xb[l % 2],
                               check_weights=False, ticks=ticks[k, l])
        torch.cuda.synchronize()
        rt.check_errors()
        stamped = ticks.cpu()

    w0 = layers[0][0]
    moe_fixed = 256 * 7168 * 2 + 256 * 4 + 7168 * 2 + 2 * S * 7168 * 2
    moe_b = [d * fp8_expert_bytes(FP8_MOE) + moe_fixed for d in distinct]
    phase_bytes = {
        "front": proj_bytes(w0.proj, FRONT_W) + S * 7168 * 2 + S * (576 + 4 + 68) + S * (32 * 576 * 2 + 64 * 68 + 128),
        "attn": attn_step_bytes(lens),
        "back": proj_bytes(w0.proj, BACK_W) + S * (32 * 512 * 2 + 2 * 7168 * 2),
        "moe": statistics.fmean(moe_b),
    }
    if "attn_back" in phases:
        phase_bytes["attn_back"] = phase_bytes.pop("attn") + phase_bytes.pop("back")
    if "attn_back_moe" in phases:
        phase_bytes["attn_back_moe"] = phase_bytes.pop("attn") + phase_bytes.pop("back") + phase_bytes.pop("moe")
    if stacked:
        phase_bytes = {"layers": sum(phase_bytes.values())}
    # the dominant launch: the whole step's (one launch a step), the whole layer's (one
    # launch a layer), else the MoE's own
    dom = "stack" if stacked else "layer" if one else "moe"
    dom_kernel = {"moe": "k_moe_fp8", "layer": "k_layer", "stack": "k_layers"}[dom]
    dom_fixed = (sum(phase_bytes.values()) if dom != "moe" else phase_bytes["moe"]) - statistics.fmean(moe_b)
    dom_b = [b + dom_fixed for b in moe_b]  # per layer (each layer's own distinct experts)
    traffic = read_traffic(dom_kernel)
    if stacked:  # bytes of every layer over the step launch's duration
        bytes_launch = sum(dom_b)
        moe_durs = step_durs
        moe_achieved = statistics.fmean(bytes_launch / (t * 1e-6) for t in step_durs) / 1e9
    else:
        bytes_launch = statistics.fmean(dom_b)
        moe_durs = layer_durs if one else ph[dom]
        moe_achieved = statistics.fmean(
            b / (t * 1e-6) for b, t in zip([dom_b[l] for _ in range(n_eager) for l in range(L)], moe_durs)) / 1e9
    layer_bytes = sum(phase_bytes.values())
    phase_ticks = None
    if stamped is not None:
        pb = {"front": proj_bytes(w0.proj, FRONT_W) + S * 7168 * 2 + S * (576 + 4 + 68)
                       + S * (32 * 576 * 2 + 64 * 68 + 128),
              "attn": attn_step_bytes(lens), "back": proj_bytes(w0.proj, BACK_W) + S * (32 * 512 * 2 + 2 * 7168 * 2)}
        phase_ticks = layer_phase_breakdown(stamped, pb, [moe_b[l] for l in range(L)])
        log("phases (in-kernel ticks, us): " + ", ".join(f"{k} {v:.2f}" for k, v in phase_ticks.items()
                                                         if k.endswith("_us")))
    log(f"{us:.2f} us/layer ({step_us / 1e3:.3f} ms a {L}-layer step, median {statistics.median(per) / L:.2f}), "
        f"{layer_bytes / (us * 1e-6) / 1e9:.0f} GB/s over the layer; eager phases "
        + ", ".join(f"{p} {ph_us[p]:.1f}" for p in phases) + f" us; {dom_kernel} {moe_achieved:.0f} GB/s; "
        f"wall {wall:.2f} s")

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline_layer(args, layers[0], x_in, cos, sin)
    rt.close()
    return dict(
        value=us, unit="us",
        ms_per_step=step_us / 1e3,
        dtype="fp8_e4m3 weights (bf16 / fp8 MFMA, f32 accumulate), fp4 index, fp8 kv",
        config=dict(workload="BASELINE config 5: full fused decoder layer, one GPU's TP=4 share, 61 stacked layers",
                    rows=S, context=ctx, layers=L, hidden=7168, heads=32, experts=256, top_k=8, shared_experts=1,
                    inter=512, launches_per_step=1 if stacked else L * rt.launches, graph=True,
                    launch=("stack: every layer of the step in ONE persistent launch (k_layers)" if stacked
                            else "layer: one launch a layer" if one else f"{args.mode}: {rt.launches} a layer"),
                    routing=("uniform: each layer's own independent random rows, router bias 0" if own_rows is not None
                             else "chained: each layer's rows are the previous layer's output")),
        extra=dict(
            us_per_layer_median=statistics.median(per) / L, us_per_layer_min=min(per) / L,
            us_per_layer_max=max(per) / L, rows_per_s=S / (us * 1e-6), step_wall_s=wall / args.steps,
            layer_algorithmic_bytes=layer_bytes, layer_achieved_gbs=layer_bytes / (us * 1e-6) / 1e9,
            phases_us_eager=ph_us, eager_layer_us=eager_layer_us,
            layer_launch_us_eager=statistics.fmean(layer_durs) if one else None,
            step_launch_us_eager=statistics.fmean(step_durs) if stacked else None,
            stack_equals_chained_step=stack_parity,
            phases_algorithmic_bytes=phase_bytes,
            phases_achieved_gbs={p: phase_bytes[p] / (ph_us[p] * 1e-6) / 1e9 for p in phases},
            distinct_experts_mean=statistics.fmean(distinct),
        ),
        phases=phase_ticks,
        roofline=dict(
            bound="hbm", achieved=moe_achieved, peak=HBM_PEAK_GBS, unit="GB/s", frac=moe_achieved / HBM_PEAK_GBS,
            traffic=traffic,
            kernel=(f"{dom_kernel} (the MoE phase: 86% of the layer's bytes)" if dom == "moe" else
                    f"{dom_kernel} (every decoder layer of the step, one launch)" if dom == "stack" else
                    f"{dom_kernel} (the whole decoder layer, one launch)"),
            bytes_per_launch=bytes_launch, avg_launch_us=statistics.fmean(moe_durs),
        ),
        cpu_baseline=cpu,
    )


def layer_phase_breakdown(ticks, fixed_bytes: dict, moe_bytes: list) -> dict:
    """Phases of one-launch layers from their per-workgroup ticks ([steps, layers, grid, 8]:
    begin, front done, attention done, back done, MoE plan ready, end; 100 MHz).

    The critical path: the launch's begin (first workgroup), then the moment the last
    workgroup finished each phase (front, attention, back, MoE plan, end); the five
    differences add up to the launch. A phase's span runs from the first workgroup
    entering it (its previous phase done) to the last leaving it; its achieved GB/s is
    its algorithmic bytes over that span. Means over every stamped launch."""
    t = ticks.double() * 10e-3  # us
    begin = t[..., 0].min(-1).values
    last = [t[..., i].max(-1).values for i in range(1, 6)]  # front, attn, back, plan, end
    first = [t[..., i].min(-1).values for i in range(0, 4)]  # entering front, attn, back, MoE
    crit = {"front_us": last[0] - begin, "attn_us": last[1] - last[0], "back_us": last[2] - last[1],
            "moe_prologue_us": last[3] - last[2], "moe_stream_us": last[4] - last[3]}
    span = {"front_span_us": last[0] - first[0], "attn_span_us": last[1] - first[1],
            "back_span_us": last[2] - first[2], "moe_span_us": last[4] - first[3]}
    out = {k: float(v.mean()) for k, v in {**crit, **span}.items()}
    out["launch_us"] = float((last[4] - begin).mean())
    moe_b = torch_tensor(moe_bytes)[None, :].expand_as(span["moe_span_us"]).double()
    out["front_gbs"] = fixed_bytes["front"] / out["front_span_us"] / 1e3
    out["attn_gbs"] = fixed_bytes["attn"] / out["attn_span_us"] / 1e3
    out["back_gbs"] = fixed_bytes["back"] / out["back_span_us"] / 1e3
    out["moe_gbs"] = float((moe_b / span["moe_span_us"]).mean()) / 1e3
    out["attn_frac"] = out["attn_gbs"] / HBM_PEAK_GBS
    out["moe_frac"] = out["moe_gbs"] / HBM_PEAK_GBS
    out["note"] = ("critical path *_us add up to launch_us; *_span_us from the first workgroup entering a phase "
                   "to the last leaving it (phases overlap); *_gbs = algorithmic bytes / span")
    return out


def torch_tensor(v):
    import torch

    return torch.tensor(v, dtype=torch.float64)


CALIB_BYTES = 1 << 30  # the calibration copy of a PMC pass: 1 GiB read, 1 GiB written
TRAFFIC_FILE = ROOT / "profiles" / "traffic_layer_8rows.md"


class PmcPassDone(Exception):
    """A single-phase workload's counter pass ran and printed its own line."""


def calibration_copy(dev) -> None:
    """One device copy of CALIB_BYTES (read once, written once): what FETCH_SIZE and
    WRITE_SIZE read for it converts each counter to bytes."""
    import torch

    src = torch.empty(CALIB_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def pmc_pass(args, dev, run_step, distinct):
    """For ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE`` runs: ``--steps`` eager
    layer steps (every dispatch seen by the profiler; no graph) and then one device copy
    of CALIB_BYTES, whose counter reading calibrates the counter in bytes. Prints one
    JSON line naming what ran."""
    import torch

    from sgl_amd_mono_amd.moe import FP8_MOE

    for _ in range(args.steps):
        run_step()
    calibration_copy(dev)
    moe_fixed = 256 * 7168 * 2 + 256 * 4 + 7168 * 2 + 2 * args.rows * 7168 * 2
    print(json.dumps({"pmc_pass": True, "steps": args.steps, "layers": args.layers, "rows": args.rows,
                      "calib_copy_bytes": CALIB_BYTES,
                      "moe_algorithmic_bytes_mean": statistics.fmean(
                          d * fp8_expert_bytes(FP8_MOE) + moe_fixed for d in distinct)}), flush=True)
    return None


def read_traffic(kernel: str):
    """HBM bytes a launch of `kernel` (fetched + written) from the committed PMC summary,
    whose lines `traffic <kernel> <bytes>` come from two rocprofv3 --pmc runs calibrated
    by a copy of known size; None when the summary is absent."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            f = line.strip().strip("`").split()
            if len(f) == 3 and f[0] == "traffic" and f[1] == kernel:
                return float(f[2])
    except OSError:
        return None
    return None


def cpu_baseline_layer(args, layer, x_in, cos, sin):
    """One layer of the CPU oracle chain (oracle.layer.front, oracle.attention,
    oracle.layer.back, oracle.moe.fp8_moe_block) at the same rows, on this host."""
    import torch

    from oracle import attention as oatt
    from oracle import codecs as ocodecs
    from oracle import layer as ol
    from oracle import moe as omoe
    from sgl_amd_mono_amd.layer import WEIGHT_SPECS
    from sgl_amd_mono_amd.moe import FP8_MOE

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    w, step, caches = layer

    class Lazy:
        def __init__(self, t, shuffled=False):
            self.t, self.shuffled, self.c = t, shuffled, {}

        def __getitem__(self, e):
            if e not in self.c:
                x = self.t[e].cpu()
                self.c[e] = ocodecs.aiter_unshuffle(x) if self.shuffled else x
            return self.c[e]

    pw = {}
    for name in WEIGHT_SPECS:
        t = getattr(w.proj, name).cpu()
        if name == "w_iw":
            t = ocodecs.aiter_unshuffle(t.view(torch.uint8)).view(torch.bfloat16)
        elif name.startswith("w_"):
            t = ocodecs.aiter_unshuffle(t)
        pw[name] = t
    m = w.moe
    mw = dict(g_post=m.g_post.cpu(), w_router=m.w_router.cpu(), bias=m.bias.cpu(), w13=Lazy(m.w13, True),
              s13=Lazy(m.s13), w2=Lazy(m.w2, True), s2=Lazy(m.s2))
    c = {k: v.cpu() for k, v in vars(caches).items()}
    seq, pt = step.seq_lens.cpu(), step.page_table.cpu()
    h = x_in.cpu()
    cs, sn = cos.cpu(), sin.cpu()

    def one():
        f = ol.front(h, seq.long() - 1, pt, pw, cs, sn)
        ol.write_caches(f, c["ikv"], c["iks"], c["kv"], c["kv_scale"])
        sc = oatt.index_scores(f["iq"], f["iqs"], f["iw"], c["ikv"], c["iks"], pt, seq, args.ctx)
        sel = oatt.select_topk(sc, seq, pt)
        o_lat = oatt.sparse_mla(f["q"], c["kv"], c["kv_scale"], sel).to(torch.bfloat16)
        a = ol.back(o_lat, h, pw)["a"]
        return omoe.fp8_moe_block(a, mw["g_post"], mw["w_router"], mw["bias"], mw["w13"], mw["s13"], mw["w2"],
                                  mw["s2"], eps=FP8_MOE.eps, top_k=FP8_MOE.top_k, inter=FP8_MOE.inter)["out"]

    one()  # warm-up: fetches the experts this layer's routing touches
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    while (len(times) < 3 or time.perf_counter() < t_end) and len(times) < 20:
        t = time.perf_counter()
        one()
        times.append((time.perf_counter() - t) * 1e6)
    med = statistics.median(times)
    log(f"cpu oracle: {med:.0f} us a layer, median of {len(times)} on {threads} threads")
    return dict(value=med, unit="us", cores=torch.get_num_threads(), kind="port",
                sample=(f"one layer (layer 0) of the oracle chain front + index scores + top-2048 + sparse MLA + "
                        f"back + FP8 MoE (f32 torch restatement) at {args.rows} rows x {args.ctx} keys, "
                        f"{len(times)} runs, median; x {args.layers} layers would be {med * args.layers / 1e6:.1f} s "
                        f"a step; host '{cpu_model()}', os.cpu_count()={os.cpu_count()}"))


WORKLOADS = {"layer": bench_layer, "moe_fp8": bench_moe_fp8, "moe_mxfp4": bench_moe_mxfp4, "attn": bench_attn}
DEFAULT_STEPS = {"layer": 20, "moe_fp8": 200, "moe_mxfp4": 200, "attn": 200}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default: 20 for layer, else 200)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rows", type=int, default=8)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="layer")
    ap.add_argument("--layers", type=int, default=61, help="stacked layers (layer workload)")
    ap.add_argument("--routing", choices=("chained", "uniform"), default="chained",
                    help="layer workload: rows chained through the layers, or independent rows a layer")
    ap.add_argument("--mode", choices=("layer", "attn_back", "split"), default="layer",
                    help="layer workload: the launch split (layer: front + one fused launch of attention, back "
                         "and MoE; attn_back: three launches; split: four)")
    ap.add_argument("--launch", choices=("stack", "layer"), default=None,
                    help="layer workload: every layer of a step as ONE persistent launch (stack, the default with "
                         "--mode layer and chained routing) or one launch (set) a layer")
    ap.add_argument("--sets", type=int, default=2, help="weight sets rotated over the steps")
    ap.add_argument("--batches", type=int, default=16, help="activation batches rotated")
    ap.add_argument("--ctx", type=int, default=32768, help="keys a row (attn workload)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="wall budget of the CPU baseline sample (0 skips it)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="eager launches (warmup + steps; layer: steps) plus a 1 GiB calibration copy, for "
                         "rocprofv3 --pmc runs")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = DEFAULT_STEPS[args.workload]
    if args.launch is None:
        args.launch = "stack" if args.mode == "layer" and args.routing == "chained" else "layer"
    elif args.launch == "stack" and (args.mode != "layer" or args.routing != "chained"):
        ap.error("--launch stack runs --mode layer with chained routing")

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}): "
              "this build runs one GPU's TP=4 share of the layer with the cross-GPU reduces "
              "replaced by a local residual add; there is no multi-GPU path to time.",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_properties(dev).gcnArchName}, workload {args.workload}")
    try:
        r = WORKLOADS[args.workload](args, dev)
    except PmcPassDone:
        return 0
    if r is None:  # a PMC pass printed its own line
        return 0
    line = {
        "metric": METRIC,
        "value": round(r["value"], 3),
        "unit": r["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": r["dtype"],
        "data": "synthetic (seeded random-init weights of the real shapes, resident in HBM)",
        "config": r["config"],
        "roofline": r["roofline"],
        "cpu_baseline": r["cpu_baseline"],
        "phases": r.get("phases"),
        **r["extra"],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
