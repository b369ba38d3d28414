"""Host side of the attention block's projections (and, through them, the whole layer).

``ProjRuntime`` owns the projection launches' mailboxes and guard, as the reference's
``Glm53Runtime`` owns its scratch (sgl_amd_mono/glm53/gfx950/runner.py:133-215);
``front`` and ``back`` check SGLang-shaped tensors and dispatch raw pointers as
``Glm53LayerOp.launch`` does (runner.py:240-321):

* ``front``: rows h -> the attention phase's inputs (q, FP4 index query + scales,
  index head weights), writing this step's MLA cache row and FP4 index key in place.
* ``back``: the attention output o_lat -> a = h + W_o W_UV o_lat.
"""

from __future__ import annotations

import ctypes as C
import logging
import os
import sys
import threading
from dataclasses import dataclass, fields

import torch

from . import _lib
from .attn import AttnCaches
from .moe import Fp8MoeWeights
from .runtime import Runtime, need

HIDDEN, Q_LORA, KV_LORA, PE_DIM = 7168, 1536, 512, 64
HEADS, NOPE_DIM, V_DIM = 32, 128, 128
QK_DIM = NOPE_DIM + PE_DIM
INDEX_HEADS, INDEX_DIM = 64, 128
N_QKV = Q_LORA + KV_LORA + PE_DIM
MAX_ROWS = 16
FRONT_TASKS_FIXED = 224 + 32 + 16  # stage C, D and bf16 stage-A tasks; B and E add 1 + 8 a row


def front_tasks(rows: int) -> int:
    """Tasks of one front launch: 140 FP8 stage-A tiles whole (rows <= 8) or in K
    halves, 16 bf16 tile quarters, two row tasks (norm, stage B) and 8 index-query
    tasks a row, 224 + 32."""
    return 140 * (1 if rows <= 8 else 2) + FRONT_TASKS_FIXED + 10 * rows
BACK_TASKS = 32 + 224


def _blocks(n: int) -> int:
    return -(-n // 128)


# name -> (shape, dtype); FP8 matrices are E4M3 bytes in AITER's (16, 16) layout with
# f32 [ceil(N/128), K/128] block scales; w_iw is bf16 whose bytes are (16, 16)-shuffled
WEIGHT_SPECS = {
    "g_in": ((HIDDEN,), torch.bfloat16),
    "w_qkv": ((N_QKV, HIDDEN), torch.uint8),
    "s_qkv": ((_blocks(N_QKV), HIDDEN // 128), torch.float32),
    "w_ik": ((INDEX_DIM, HIDDEN), torch.uint8),
    "s_ik": ((1, HIDDEN // 128), torch.float32),
    "w_iw": ((INDEX_HEADS, HIDDEN), torch.bfloat16),
    "g_q": ((Q_LORA,), torch.bfloat16),
    "g_kv": ((KV_LORA,), torch.bfloat16),
    "g_ik": ((INDEX_DIM,), torch.float32),
    "b_ik": ((INDEX_DIM,), torch.float32),
    "w_qb": ((HEADS * QK_DIM, Q_LORA), torch.uint8),
    "s_qb": ((HEADS * QK_DIM // 128, Q_LORA // 128), torch.float32),
    "w_iq": ((INDEX_HEADS * INDEX_DIM, Q_LORA), torch.uint8),
    "s_iq": ((INDEX_HEADS * INDEX_DIM // 128, Q_LORA // 128), torch.float32),
    "w_uk": ((HEADS * KV_LORA, NOPE_DIM), torch.uint8),
    "s_uk": ((HEADS * KV_LORA // 128, 1), torch.float32),
    "w_uv": ((HEADS * V_DIM, KV_LORA), torch.uint8),
    "s_uv": ((HEADS * V_DIM // 128, KV_LORA // 128), torch.float32),
    "w_o": ((HIDDEN, HEADS * V_DIM), torch.uint8),
    "s_o": ((HIDDEN // 128, HEADS * V_DIM // 128), torch.float32),
}


@dataclass
class ProjWeights:
    """One layer's attention-block projection weights (device tensors, read in place)."""

    g_in: torch.Tensor
    w_qkv: torch.Tensor
    s_qkv: torch.Tensor
    w_ik: torch.Tensor
    s_ik: torch.Tensor
    w_iw: torch.Tensor
    g_q: torch.Tensor
    g_kv: torch.Tensor
    g_ik: torch.Tensor
    b_ik: torch.Tensor
    w_qb: torch.Tensor
    s_qb: torch.Tensor
    w_iq: torch.Tensor
    s_iq: torch.Tensor
    w_uk: torch.Tensor
    s_uk: torch.Tensor
    w_uv: torch.Tensor
    s_uv: torch.Tensor
    w_o: torch.Tensor
    s_o: torch.Tensor

    def check(self, device) -> None:
        for f in fields(self):
            shape, dtype = WEIGHT_SPECS[f.name]
            need(getattr(self, f.name), f.name, shape, dtype, device)

    def c_struct(self) -> _lib.ProjWeights:
        return _lib.ProjWeights(**{n: _lib.ptr(getattr(self, n)) for n in _lib.PROJ_WEIGHT_FIELDS})

    def nbytes(self) -> int:
        return sum(getattr(self, f.name).numel() * getattr(self, f.name).element_size() for f in fields(self))


@dataclass
class FrontOut:
    """The attention phase's inputs for one step."""

    q: torch.Tensor  # bf16 [rows, 32, 576]
    iq: torch.Tensor  # u8 [rows, 64, 64]
    iqs: torch.Tensor  # u8 [rows, 64, 4]
    iw: torch.Tensor  # bf16 [rows, 64]

    @staticmethod
    def empty(rows: int, device) -> "FrontOut":
        return FrontOut(
            q=torch.empty(rows, HEADS, KV_LORA + PE_DIM, dtype=torch.bfloat16, device=device),
            iq=torch.empty(rows, INDEX_HEADS, INDEX_DIM // 2, dtype=torch.uint8, device=device),
            iqs=torch.empty(rows, INDEX_HEADS, INDEX_DIM // 32, dtype=torch.uint8, device=device),
            iw=torch.empty(rows, INDEX_HEADS, dtype=torch.bfloat16, device=device),
        )


def _rows(t: torch.Tensor, name: str, max_rows: int) -> int:
    if t.dim() != 2 or not 1 <= t.shape[0] <= max_rows:
        raise ValueError(f"{name}: expected [rows <= {max_rows}, {HIDDEN}], got {tuple(t.shape)}")
    return t.shape[0]


def front_args(dev, max_rows: int, h: torch.Tensor, seq_lens: torch.Tensor, page_table: torch.Tensor,
               caches: AttnCaches, w: ProjWeights, rope_cos: torch.Tensor, rope_sin: torch.Tensor,
               out: "FrontOut | None", check_weights: bool, timeline: torch.Tensor | None):
    """Checked mono_front_args (and the weight table) for a runtime of ``max_rows`` on
    ``dev``: (args, out, weights)."""
    S = _rows(h, "h", max_rows)
    need(h, "h", (S, HIDDEN), torch.bfloat16, dev)
    need(seq_lens, "seq_lens", (S,), torch.int32, dev)
    if page_table.dim() != 2 or page_table.shape[0] < S:
        raise ValueError(f"page_table: expected [>= {S}, pages], got {tuple(page_table.shape)}")
    need(page_table, "page_table", tuple(page_table.shape), torch.int32, dev)
    pages = caches.ikv.shape[0]
    need(caches.ikv, "ikv", (pages, 4, 64, 16), torch.uint8, dev)
    need(caches.iks, "iks", (pages, 4, 64), torch.uint8, dev)
    need(caches.kv, "kv", (pages * 64, KV_LORA + PE_DIM), torch.uint8, dev)
    if caches.kv_scale is not None:  # None: raw E4M3 rows (scale 1)
        need(caches.kv_scale, "kv_scale", (pages * 64,), torch.float32, dev)
    if rope_cos.dim() != 2 or rope_cos.shape[1] != PE_DIM // 2:
        raise ValueError(f"rope_cos: expected [max_pos, {PE_DIM // 2}], got {tuple(rope_cos.shape)}")
    need(rope_cos, "rope_cos", tuple(rope_cos.shape), torch.float32, dev)
    need(rope_sin, "rope_sin", tuple(rope_cos.shape), torch.float32, dev)
    if check_weights:
        w.check(dev)
    out = FrontOut.empty(S, dev) if out is None else out
    need(out.q, "q", (S, HEADS, KV_LORA + PE_DIM), torch.bfloat16, dev)
    need(out.iq, "iq", (S, INDEX_HEADS, INDEX_DIM // 2), torch.uint8, dev)
    need(out.iqs, "iqs", (S, INDEX_HEADS, INDEX_DIM // 32), torch.uint8, dev)
    need(out.iw, "iw", (S, INDEX_HEADS), torch.bfloat16, dev)
    P = _lib.ptr
    args = _lib.FrontArgs(
        h=P(h), seq_lens=P(seq_lens), page_table=P(page_table), pt_stride=page_table.shape[1],
        n_pages=pages, rope_cos=P(rope_cos), rope_sin=P(rope_sin), max_pos=rope_cos.shape[0],
        ikv=P(caches.ikv), iks=P(caches.iks), kv=P(caches.kv), kv_scale=P(caches.kv_scale),
        q=P(out.q), iq=P(out.iq), iqs=P(out.iqs), iw=P(out.iw), rows=S, timeline=P(timeline),
    )  # fmt: skip
    if timeline is not None:
        need(timeline, "timeline", (front_tasks(S), 4), torch.int64, dev)
    ws = w.c_struct()
    return args, out, ws


class ProjRuntime(Runtime):
    """The C library's projection handle for a widest step ``max_rows`` (<= 16)."""

    PREFIX = "mono_proj"
    SITES = _lib.PROJ_SITES
    KIND = "projection"

    def __init__(self, max_rows: int, device=None):
        super().__init__(device)
        self.max_rows = max_rows
        self._create(_lib.ProjConfig(device=self.device.index, max_rows=max_rows))

    def _rows(self, t: torch.Tensor, name: str) -> int:
        if t.dim() != 2 or not 1 <= t.shape[0] <= self.max_rows:
            raise ValueError(f"{name}: expected [rows <= {self.max_rows}, {HIDDEN}], got {tuple(t.shape)}")
        return t.shape[0]

    def front(self, h: torch.Tensor, seq_lens: torch.Tensor, page_table: torch.Tensor, caches: AttnCaches,
              w: ProjWeights, rope_cos: torch.Tensor, rope_sin: torch.Tensor, out: FrontOut | None = None,
              check_weights: bool = True, timeline: torch.Tensor | None = None) -> FrontOut:
        """Rows ``h`` [rows, 7168] bf16 whose new tokens sit at ``seq_lens - 1`` ->
        FrontOut; writes each row's MLA cache row and FP4 index key in place.
        ``timeline`` (int64 [front_tasks(rows), 4]) receives each task's start,
        inputs-ready and end ticks and workgroup << 8 | stage."""
        args, out, ws = front_args(self.device, self.max_rows, h, seq_lens, page_table, caches, w, rope_cos,
                                   rope_sin, out, check_weights, timeline)
        _lib.check(_lib.lib().mono_front_forward(self._h, C.byref(ws), C.byref(args), self._stream()))
        return out

    def back(self, o_lat: torch.Tensor, h: torch.Tensor, w: ProjWeights, a: torch.Tensor | None = None,
             o: torch.Tensor | None = None, check_weights: bool = True,
             timeline: torch.Tensor | None = None) -> torch.Tensor:
        """a = h + W_o W_UV o_lat [rows, 7168] bf16 (``o``, if given, receives W_UV o_lat
        [rows, 4096] bf16)."""
        dev = self.device
        S = self._rows(h, "h")
        need(h, "h", (S, HIDDEN), torch.bfloat16, dev)
        need(o_lat, "o_lat", (S, HEADS, KV_LORA), torch.bfloat16, dev)
        if check_weights:
            w.check(dev)
        a = torch.empty_like(h) if a is None else a
        need(a, "a", (S, HIDDEN), torch.bfloat16, dev)
        if o is not None:
            need(o, "o", (S, HEADS * V_DIM), torch.bfloat16, dev)
        P = _lib.ptr
        if timeline is not None:
            need(timeline, "timeline", (BACK_TASKS, 4), torch.int64, dev)
        args = _lib.BackArgs(o_lat=P(o_lat), h=P(h), a=P(a), o=P(o), rows=S, timeline=P(timeline))
        ws = w.c_struct()
        _lib.check(_lib.lib().mono_back_forward(self._h, C.byref(ws), C.byref(args), self._stream()))
        return a


def attn_back(attn, step, caches, w: ProjWeights, h: torch.Tensor, o_lat: torch.Tensor | None = None,
              a: torch.Tensor | None = None, o: torch.Tensor | None = None, check_weights: bool = True,
              debug: bool = False, timeline: torch.Tensor | None = None,
              back_timeline: torch.Tensor | None = None):
    """The sparse attention (``attn``, an AttnRuntime) and the back of the attention
    block on its output as ONE launch (mono_attn_back_forward; the reference's layer
    launch runs both, kernel.py:2684-4197): returns (o_lat, a) and, with ``debug``, the
    attention's index scores and selected slots. Results equal AttnRuntime.forward
    followed by ProjRuntime.back."""
    dev = attn.device
    args, o_lat, dbg = attn.args(step, caches, o_lat, debug, timeline)
    S = args.rows
    need(h, "h", (S, HIDDEN), torch.bfloat16, dev)
    if check_weights:
        w.check(dev)
    a = torch.empty_like(h) if a is None else a
    need(a, "a", (S, HIDDEN), torch.bfloat16, dev)
    if o is not None:
        need(o, "o", (S, HEADS * V_DIM), torch.bfloat16, dev)
    if back_timeline is not None:
        need(back_timeline, "back_timeline", (BACK_TASKS, 4), torch.int64, dev)
    P = _lib.ptr
    bargs = _lib.BackArgs(o_lat=P(o_lat), h=P(h), a=P(a), o=P(o), rows=S, timeline=P(back_timeline))
    ws = w.c_struct()
    _lib.check(_lib.lib().mono_attn_back_forward(attn._h, C.byref(args), C.byref(ws), C.byref(bargs),
                                                 attn._stream()))
    return (o_lat, a, dbg) if debug else (o_lat, a)


@dataclass
class LayerWeights:
    """One decoder layer: the attention block's projections and the FP8 MoE."""

    proj: ProjWeights
    moe: Fp8MoeWeights


class LayerHandle(Runtime):
    """The C library's layer runtime (mono_layer): the front launch's and the fused
    attention + back + MoE launch's mailboxes and guards in one handle."""

    PREFIX = "mono_layer"
    KIND = "layer"

    def __init__(self, max_rows: int, max_ctx: int, device=None, max_layers: int = 0):
        from .attn import SOFTMAX_SCALE
        from .moe import FP8_MOE

        super().__init__(device)
        self._create(_lib.LayerConfig(device=self.device.index, max_rows=max_rows, max_ctx=max_ctx,
                                      softmax_scale=SOFTMAX_SCALE, route_scale=FP8_MOE.route_scale,
                                      eps=FP8_MOE.eps, max_layers=max_layers))

    SITES = _lib.LAYER_SITES

    def set_fault(self, site: int, after: int = 0) -> None:
        """Tests of the fail-stop path (the reference's fault injection): every wait at
        ``site`` (layer numbering, ``_lib.LAYER_SITES``) of every launch from the
        ``after``-th next one on fails at once (-1: off)."""
        _lib.check(self._fn("set_fault")(self._h, int(site), int(after)))

    def pending_error(self) -> int:
        """The pinned host error word, read without synchronising: 0, or 1 + the wait
        site of a launch that failed or was refused since the last clear."""
        return int(self._fn("pending_error")(self._h))

    def set_launch_ordinal(self, ordinal: int) -> None:
        """Tests of the tag epochs (synchronises): the next launch takes tag
        ``ordinal % TAG_PERIOD + 1``."""
        with torch.cuda.device(self.device):
            _lib.check(self._fn("set_launch_ordinal")(self._h, int(ordinal)))


FAIL_STOP_EXIT = 70  # the process's exit status when a layer launch stopped (EX_SOFTWARE)
FAIL_STOP_POLL_S = 5e-4

_log = logging.getLogger(__name__)


class FailStopWatch:
    """A host thread that sees a stopped layer launch within about a millisecond, also
    when the launch was replayed from a graph (a replayed step runs none of the
    plugin's host code). The reference ends the process at the failing wait itself, by
    a store to the null page (common/guard.py:91-97); here the kernel copies the wait
    site to a pinned host word (``pending()``, a plain memory read, no GPU call) and
    this thread, polling it every ``interval`` seconds, calls ``on_fail(code)`` once.
    The default ``on_fail`` logs the site and ends the process with exit status
    ``FAIL_STOP_EXIT`` (``os._exit``: nothing runs that could wait on the GPU), as
    the reference's stop does. The window left: a step's tokens can be sampled and
    handed on between the launch's failure and the thread's next poll (the interval
    plus the thread's wait for the interpreter lock, a few milliseconds at most)."""

    def __init__(self, pending, on_fail=None, interval: float = FAIL_STOP_POLL_S, name: str = "layer"):
        self._pending, self.interval = pending, float(interval)
        self._on_fail = on_fail if on_fail is not None else self._exit
        self._name = name
        self._stop = threading.Event()
        self.code = 0
        self._thread = threading.Thread(target=self._run, name=f"mono-fail-stop-{name}", daemon=True)
        self._thread.start()

    def _run(self) -> None:
        while not self._stop.wait(self.interval):
            code = int(self._pending())
            if code > 0:
                self.code = code
                self._on_fail(code)
                return

    def _exit(self, code: int) -> None:
        site = code - 1
        msg = (f"sgl_amd_mono_amd: a {self._name} launch stopped at wait "
               f"'{_lib.LAYER_SITES.get(site, site)}' (deadline passed or refused after an earlier "
               f"failure); ending the process (exit status {FAIL_STOP_EXIT}) before its output is served")
        _log.critical(msg)
        print(msg, file=sys.stderr, flush=True)
        os._exit(FAIL_STOP_EXIT)

    def stop(self) -> None:
        """End the thread (idempotent); the runtime calls it before it is destroyed."""
        self._stop.set()
        if self._thread.is_alive() and self._thread is not threading.current_thread():
            self._thread.join()


class LayerRuntime:
    """One GPU's TP=4 share of a DeepSeek-V3.2-shaped decoder layer with an FP4 indexer
    its launches on the caller's stream and each phase's outputs
    in scratch this runtime owns. The reference launches the whole layer as one grid
    (glm53/gfx950/kernel.py:6-45) with the TP all-reduces that are local residual adds
    here. ``mode`` picks the launch split; every mode gives the same results:

    * ``"layer"`` (default, mono_layer_forward): the whole layer as ONE persistent
      launch (front, sparse attention, back, FP8 MoE); with ``on_phase`` the front and
      the rest run as two launches so a caller can time them apart;
    * ``"attn_back"``: front; attention + back (mono_attn_back_forward); MoE;
    * ``"split"``: front; attention; back; MoE (four launches).

    No call synchronises with the host, so a caller may capture a step in a HIP graph.
    """

    # the launches of a layer, the names of forward's on_phase indices
    MODES = {"layer": ("front", "attn_back_moe"), "attn_back": ("front", "attn_back", "moe"),
             "split": ("front", "attn", "back", "moe")}

    def __init__(self, max_rows: int = 8, max_ctx: int = 32768, device=None, mode: str = "layer",
                 fused: bool | None = None, max_layers: int = 0):
        from .attn import AttnRuntime
        from .moe import FP8_MOE, MoeRuntime

        if fused is not None:  # the older switch: fused=False is the four-launch split
            mode = "attn_back" if fused else "split"
        if mode not in self.MODES:
            raise ValueError(f"mode must be one of {sorted(self.MODES)}, got {mode!r}")
        if not 1 <= max_rows <= MAX_ROWS:
            raise ValueError(f"max_rows must be in [1, {MAX_ROWS}], got {max_rows}")
        if max_layers and mode != "layer":
            raise ValueError("max_layers (the multi-layer launch) needs mode 'layer'")
        self.mode = mode
        self.max_rows, self.max_ctx = max_rows, max_ctx
        self.max_layers = max_layers
        self._stack_key = None
        if mode == "layer":
            self.handle = LayerHandle(max_rows, max_ctx, device, max_layers)
            self.device = self.handle.device
            self.parts = (self.handle,)
        else:
            self.proj = ProjRuntime(max_rows, device)
            self.device = self.proj.device
            self.attn = AttnRuntime(max_rows, max_ctx, device=self.device)
            self.moe = MoeRuntime(FP8_MOE, max_rows, self.device)
            self.parts = (self.proj, self.attn, self.moe)
        self.geo = FP8_MOE
        # the launches of a layer, the names of forward's on_phase indices
        self.phases = self.MODES[mode]
        # launches a step of one layer takes without on_phase
        self.launches = 1 if mode == "layer" else len(self.phases)
        self._front = FrontOut.empty(max_rows, self.device)
        self._o_lat = torch.empty(max_rows, HEADS, KV_LORA, dtype=torch.bfloat16, device=self.device)
        self._a = torch.empty(max_rows, HIDDEN, dtype=torch.bfloat16, device=self.device)
        if max_layers:  # the multi-layer launch's buffers: each layer's own
            self._fronts = [FrontOut.empty(max_rows, self.device) for _ in range(max_layers)]
            self._as = torch.empty(max_layers, max_rows, HIDDEN, dtype=torch.bfloat16, device=self.device)
            self._xs = torch.empty(max_layers, max_rows, HIDDEN, dtype=torch.bfloat16, device=self.device)

    def close(self) -> None:
        self.unwatch()
        for rt in self.parts:
            rt.close()

    def watch(self, on_fail=None, interval: float = FAIL_STOP_POLL_S) -> FailStopWatch:
        """Start the fail-stop watcher (one-launch mode): a host thread that polls the
        pinned error word and calls ``on_fail(code)`` (default: log and end the
        process) when a launch stops, also for steps replayed from a graph."""
        if self.mode != "layer":
            raise ValueError("the fail-stop watcher reads the one-launch layer's pinned host word (mode 'layer')")
        self.unwatch()
        self._watch = FailStopWatch(self.handle.pending_error, on_fail, interval)
        return self._watch

    def unwatch(self) -> None:
        w = getattr(self, "_watch", None)
        if w is not None:
            w.stop()
            self._watch = None

    def set_deadline(self, seconds: float) -> None:
        for rt in self.parts:
            rt.set_deadline(seconds)

    def clear_errors(self) -> None:
        for rt in self.parts:
            rt.clear_errors()

    def forward(self, h: torch.Tensor, seq_lens: torch.Tensor, page_table: torch.Tensor, caches: AttnCaches,
                w: LayerWeights, rope_cos: torch.Tensor, rope_sin: torch.Tensor, out: torch.Tensor | None = None,
                check_weights: bool = True, keep: bool = False, on_phase=None, ticks: torch.Tensor | None = None,
                timelines: dict | None = None):
        """x_out [rows, 7168] bf16 = the layer applied to rows ``h`` whose new tokens sit
        at ``seq_lens - 1`` (this step's cache rows are written in place). ``keep``
        also returns the intermediates (front outputs, the index scores and selected
        slots, o_lat, a, the MoE routing and sum) as copies. ``on_phase(i)`` (if given)
        is called after the launch of phase i (``self.phases[i]``) is enqueued, e.g. to
        record timing events between the phases. ``ticks`` (int64 [grid, 16], one-launch
        mode) receives each workgroup's phase ticks (``_lib.LAYER_TICKS``, 100 MHz);
        ``timelines`` (one-launch mode) maps "front" / "attn" / "back" to int64 per-task
        timelines of those phases (front_tasks(rows), attn.n_tasks(max_ctx, rows),
        BACK_TASKS rows of start, inputs-ready and end ticks, workgroup << 8 | stage)."""
        from .attn import AttnStep, attn_args
        from .moe import fp8_args

        S = h.shape[0] if h.dim() == 2 else -1
        if not 1 <= S <= self.max_rows:
            raise ValueError(f"h: expected [rows <= {self.max_rows}, {HIDDEN}], got {tuple(h.shape)}")
        fo = FrontOut(q=self._front.q[:S], iq=self._front.iq[:S], iqs=self._front.iqs[:S], iw=self._front.iw[:S])
        mark = on_phase if on_phase is not None else (lambda i: None)
        step = AttnStep(iq=fo.iq, iqs=fo.iqs, iw=fo.iw, q=fo.q, page_table=page_table, seq_lens=seq_lens)
        if self.mode == "layer":
            dev = self.device
            tl = timelines or {}
            fargs, _, ws = front_args(dev, self.max_rows, h, seq_lens, page_table, caches, w.proj, rope_cos,
                                      rope_sin, fo, check_weights, tl.get("front"))
            aargs, o_lat, adbg = attn_args(dev, self.max_rows, self.max_ctx, step, caches, self._o_lat[:S], keep,
                                           tl.get("attn"))
            a = self._a[:S]
            need(h, "h", (S, HIDDEN), torch.bfloat16, dev)
            if tl.get("back") is not None:
                need(tl["back"], "timelines['back']", (BACK_TASKS, 4), torch.int64, dev)
            bargs = _lib.BackArgs(o_lat=_lib.ptr(o_lat), h=_lib.ptr(h), a=_lib.ptr(a), o=None, rows=S,
                                  timeline=_lib.ptr(tl.get("back")))
            margs, x, mdbg = fp8_args(dev, self.max_rows, self.geo, a, w.moe, out, keep)
            if ticks is not None:
                grid = torch.cuda.get_device_properties(dev).multi_processor_count
                need(ticks, "ticks", (grid, _lib.LAYER_TICK_WORDS), torch.int64, dev)
            largs = _lib.LayerArgs(C.pointer(fargs), C.pointer(aargs), C.pointer(bargs), C.pointer(margs),
                                   _lib.ptr(ticks))
            lib, hd, st = _lib.lib(), self.handle._h, self.handle._stream()
            if on_phase is None:
                _lib.check(lib.mono_layer_forward(hd, C.byref(ws), C.byref(largs), st))
            else:  # the two launches one by one, marked in between
                _lib.check(lib.mono_layer_front_forward(hd, C.byref(ws), C.byref(largs), st))
                mark(0)
                _lib.check(lib.mono_layer_tail_forward(hd, C.byref(ws), C.byref(largs), st))
                mark(1)
        else:
            self.proj.front(h, seq_lens, page_table, caches, w.proj, rope_cos, rope_sin, out=fo,
                            check_weights=check_weights)
            mark(0)
            if self.mode == "attn_back":
                res = attn_back(self.attn, step, caches, w.proj, h, o_lat=self._o_lat[:S], a=self._a[:S],
                                check_weights=check_weights, debug=keep)
                o_lat, a = res[0], res[1]
                adbg = res[2] if keep else None
                mark(1)
            else:
                if keep:
                    o_lat, adbg = self.attn.forward(step, caches, out=self._o_lat[:S], debug=True)
                else:
                    o_lat = self.attn.forward(step, caches, out=self._o_lat[:S])
                mark(1)
                a = self.proj.back(o_lat, h, w.proj, a=self._a[:S], check_weights=check_weights)
                mark(2)
            if keep:
                x, mdbg = self.moe.forward_fp8(a, w.moe, out=out, debug=True)
            else:
                x = self.moe.forward_fp8(a, w.moe, out=out)
            mark(len(self.phases) - 1)
        if not keep:
            return x
        inter = dict(q=fo.q.clone(), iq=fo.iq.clone(), iqs=fo.iqs.clone(), iw=fo.iw.clone(), o_lat=o_lat.clone(),
                     a=a.clone(), index_scores=adbg["scores"], topk_slots=adbg["topk"], **mdbg)
        return x, inter

    def forward_layers(self, h: torch.Tensor, seq_lens, page_table, caches, ws, rope_cos: torch.Tensor,
                       rope_sin: torch.Tensor, out: torch.Tensor | None = None, check_weights: bool = True,
                       ticks: torch.Tensor | None = None) -> torch.Tensor:
        """x_out [rows, 7168] bf16 of ``len(ws)`` decoder layers applied in turn to rows
        ``h`` as ONE persistent launch (mono_layer_stack_forward): layer l runs as
        ``forward`` would with ``ws[l]`` and ``caches[l]`` (each layer's own caches) and
        takes layer l - 1's output rows, results equal layer by layer. ``seq_lens`` and
        ``page_table`` are one tensor for every layer or a sequence of one a layer.
        ``ticks`` (int64 [layers, grid, 16]) receives each layer's phase ticks.

        The layers' arguments are packed and uploaded (mono_layer_stack_set, which
        synchronises the device) only when the buffers change: the key is the objects
        passed (held here while they are the last set) and the data pointers of h, out
        and ticks, so a caller that swaps a tensor inside a weights or caches object it
        passed again calls ``reset_layers()`` first. No other call synchronises, so a
        step can be captured in a HIP graph once its arguments are set (a replay reads
        the arguments last set)."""
        from .attn import AttnStep, attn_args
        from .moe import fp8_args

        n = len(ws)
        if not 1 <= n <= self.max_layers:
            raise ValueError(f"{n} layers: the runtime takes 1 to max_layers = {self.max_layers} a launch")
        if len(caches) != n:
            raise ValueError(f"caches: expected {n} (one a layer), got {len(caches)}")
        lens = list(seq_lens) if isinstance(seq_lens, (list, tuple)) else [seq_lens] * n
        tables = list(page_table) if isinstance(page_table, (list, tuple)) else [page_table] * n
        if len(lens) != n or len(tables) != n:
            raise ValueError(f"seq_lens / page_table: one tensor or {n} (one a layer)")
        S = _rows(h, "h", self.max_rows)
        x_last = self._xs[n - 1, :S] if out is None else out
        P = _lib.ptr
        key = (n, S, P(h), P(x_last), P(ticks), P(rope_cos), P(rope_sin), tuple(map(id, ws)),
               tuple(map(id, caches)), tuple(map(id, lens)), tuple(map(id, tables)))
        if key != self._stack_key:
            dev = self.device
            if ticks is not None:
                grid = torch.cuda.get_device_properties(dev).multi_processor_count
                need(ticks, "ticks", (n, grid, _lib.LAYER_TICK_WORDS), torch.int64, dev)
            keep, wps, lps = [], [], []
            x = h
            for l in range(n):
                fr = self._fronts[l]
                fo = FrontOut(q=fr.q[:S], iq=fr.iq[:S], iqs=fr.iqs[:S], iw=fr.iw[:S])
                fargs, _, wst = front_args(dev, self.max_rows, x, lens[l], tables[l], caches[l], ws[l].proj,
                                           rope_cos, rope_sin, fo, check_weights, None)
                step = AttnStep(iq=fo.iq, iqs=fo.iqs, iw=fo.iw, q=fo.q, page_table=tables[l], seq_lens=lens[l])
                aargs, o_lat, _ = attn_args(dev, self.max_rows, self.max_ctx, step, caches[l], self._o_lat[:S],
                                            False, None)
                a = self._as[l, :S]
                bargs = _lib.BackArgs(o_lat=P(o_lat), h=P(x), a=P(a), o=None, rows=S, timeline=None)
                xo = x_last if l == n - 1 else self._xs[l, :S]
                margs, _, _ = fp8_args(dev, self.max_rows, self.geo, a, ws[l].moe, xo, False)
                largs = _lib.LayerArgs(C.pointer(fargs), C.pointer(aargs), C.pointer(bargs), C.pointer(margs),
                                       None if ticks is None else P(ticks[l]))
                keep.append((fargs, aargs, bargs, margs, largs, wst))
                wps.append(C.pointer(wst))
                lps.append(C.pointer(largs))
                x = xo
            warr = (C.POINTER(_lib.ProjWeights) * n)(*wps)
            larr = (C.POINTER(_lib.LayerArgs) * n)(*lps)
            self._stack_key = None
            with torch.cuda.device(self.device):
                _lib.check(_lib.lib().mono_layer_stack_set(self.handle._h, n, warr, larr))
            # the objects whose ids make the key stay alive while it is the last set
            self._stack_key, self._stack_refs = key, (ws, caches, lens, tables, keep)
        _lib.check(_lib.lib().mono_layer_stack_forward(self.handle._h, self.handle._stream()))
        return x_last

    def reset_layers(self) -> None:
        """Forget the multi-layer launch's packed arguments: the next forward_layers
        packs and uploads them again."""
        self._stack_key = None
        self._stack_refs = None

    def check_errors(self) -> None:
        for rt in self.parts:
            rt.check_errors()

    def raise_pending(self) -> None:
        """Raise MonoError if a launch failed or was refused since the last clear, read
        from the pinned host word without synchronising (a serving loop calls it once a
        step; the launch that failed wrote NaN over its output)."""
        if self.mode != "layer":
            return
        code = self.handle.pending_error()
        if code:
            site = code - 1
            raise _lib.MonoError(
                _lib.MONO_ESTATE,
                f"a layer launch stopped at wait '{_lib.LAYER_SITES.get(site, site)}' (deadline passed or refused "
                "after an earlier failure); its output is NaN and the runtime refuses launches until clear_errors()",
            )
