"""Host side of the sparse-attention phase: a runtime and its forward call.

Mirrors the reference's split between the runtime that owns scratch
(``Glm53Runtime``, sgl_amd_mono/glm53/gfx950/runner.py:133-215) and the launch that
checks SGLang's tensors and dispatches raw pointers (``Glm53LayerOp.launch``,
runner.py:240-321). The caches are SGLang's, read in place: the FP4 index plane
(payload ``[pages, 4, 64, 16]``, E8M0 scales ``[pages, 4, 64]``,
deepseek_v4/gfx950/runner.py:336-347) and the E4M3 MLA cache ``[pages * 64, 576]``
with one f32 scale a token.
"""

from __future__ import annotations

from dataclasses import dataclass

import ctypes as C

import torch

from . import _lib
from .runtime import Runtime, need

IH, ID, NH, DQK, DV, PAGE, TOPK = 64, 128, 32, 576, 512, 64, 2048


def splits_of(rows: int) -> int:
    """Attention splits a row: 32 up to 16 rows, then fewer and longer ones, so a step's
    splits fill one round of a 256-CU grid."""
    return 32 if rows <= 16 else 8 if rows <= 32 else 5 if rows <= 48 else 4


def merges_of(rows: int) -> int:
    """Merge tasks a row (32 / merges heads each): as many as splits, except 4 with 5."""
    return 4 if splits_of(rows) == 5 else splits_of(rows)
SOFTMAX_SCALE = (128 + 64) ** -0.5  # (qk_nope + qk_rope)^-1/2, glm53/gfx950/config.py:171-173


@dataclass
class AttnCaches:
    """One layer's caches (SGLang's pools, read in place)."""

    ikv: torch.Tensor  # u8 [pages, 4, 64, 16] E2M1 index keys
    iks: torch.Tensor  # u8 [pages, 4, 64] E8M0
    kv: torch.Tensor  # u8 [pages * 64, 576] E4M3
    kv_scale: torch.Tensor | None  # f32 [pages * 64]; None: raw E4M3 rows (scale 1)


@dataclass
class AttnStep:
    """One decode step's rows: queries, page tables and lengths."""

    iq: torch.Tensor  # u8 [rows, 64, 64] E2M1 index query
    iqs: torch.Tensor  # u8 [rows, 64, 4] E8M0
    iw: torch.Tensor  # bf16 [rows, 64] index head weights
    q: torch.Tensor  # bf16 [rows, 32, 576]
    page_table: torch.Tensor  # i32 [rows, >= max_ctx / 64]
    seq_lens: torch.Tensor  # i32 [rows]


class AttnRuntime(Runtime):
    """The C library's sparse-attention handle for a widest step ``max_rows`` and a
    longest row ``max_ctx`` keys."""

    PREFIX = "mono_attn"
    SITES = _lib.ATTN_SITES
    KIND = "attention"

    def __init__(self, max_rows: int, max_ctx: int = 32768, softmax_scale: float = SOFTMAX_SCALE,
                 device=None):
        super().__init__(device)
        self.max_rows, self.max_ctx = max_rows, max_ctx
        self._create(_lib.AttnConfig(device=self.device.index, max_rows=max_rows, max_ctx=max_ctx,
                                     softmax_scale=softmax_scale))

    def n_tasks(self, rows: int) -> int:
        """Tasks of one launch over ``rows`` rows (the timeline's length)."""
        return n_tasks(self.max_ctx, rows)

    def forward(self, step: AttnStep, caches: AttnCaches, out: torch.Tensor | None = None,
                debug: bool = False, timeline: torch.Tensor | None = None):
        """o_lat [rows, 32, 512] bf16 for one decode step. ``debug`` also returns the
        index scores [rows, max_ctx] and the selected slots [rows, 2048]. ``timeline``
        (int64 [n_tasks(rows), 4]) receives each task's start, inputs-ready and end
        s_memrealtime ticks (100 MHz) and workgroup << 8 | kind (0 score, 1 top-k,
        2 split, 3 merge)."""
        args, out, dbg = self.args(step, caches, out, debug, timeline)
        _lib.check(_lib.lib().mono_attn_forward(self._h, C.byref(args), self._stream()))
        return (out, dbg) if debug else out

    def args(self, step: AttnStep, caches: AttnCaches, out: torch.Tensor | None, debug: bool,
             timeline: torch.Tensor | None):
        """The checked launch arguments of ``forward`` (and of the fused attention + back
        launch): (mono_attn_args, out, debug outputs)."""
        return attn_args(self.device, self.max_rows, self.max_ctx, step, caches, out, debug, timeline)


def n_tasks(max_ctx: int, rows: int) -> int:
    """Tasks of one attention launch over ``rows`` rows (the timeline's length)."""
    team = 16 if rows <= 16 else 4  # top-k team members a row
    n_score = -(-rows * (max_ctx // 1024) // team) * team  # padded to whole top-k teams
    return n_score + rows * team + rows * (splits_of(rows) + merges_of(rows))


def attn_args(dev, max_rows: int, max_ctx: int, step: AttnStep, caches: AttnCaches, out: torch.Tensor | None,
              debug: bool, timeline: torch.Tensor | None):
    """Checked mono_attn_args for a runtime of ``max_rows`` x ``max_ctx`` on ``dev``:
    (args, out, debug outputs)."""
    S = step.q.shape[0] if step.q.dim() == 3 else -1
    if not 1 <= S <= max_rows:
        raise ValueError(f"q: expected [rows <= {max_rows}, {NH}, {DQK}], got {tuple(step.q.shape)}")
    pages = caches.ikv.shape[0]
    need(step.iq, "iq", (S, IH, ID // 2), torch.uint8, dev)
    need(step.iqs, "iqs", (S, IH, ID // 32), torch.uint8, dev)
    need(step.iw, "iw", (S, IH), torch.bfloat16, dev)
    need(step.q, "q", (S, NH, DQK), torch.bfloat16, dev)
    if step.page_table.dim() != 2 or step.page_table.shape[1] < max_ctx // PAGE:
        raise ValueError(f"page_table: expected [rows, >= {max_ctx // PAGE}], got {tuple(step.page_table.shape)}")
    need(step.page_table, "page_table", (S, step.page_table.shape[1]), torch.int32, dev)
    need(step.seq_lens, "seq_lens", (S,), torch.int32, dev)
    need(caches.ikv, "ikv", (pages, 4, PAGE, 16), torch.uint8, dev)
    need(caches.iks, "iks", (pages, 4, PAGE), torch.uint8, dev)
    need(caches.kv, "kv", (pages * PAGE, DQK), (torch.uint8, torch.float8_e4m3fn), dev)
    if caches.kv_scale is not None:  # None: raw E4M3 rows (scale 1)
        need(caches.kv_scale, "kv_scale", (pages * PAGE,), torch.float32, dev)
    if out is None:
        out = torch.empty(S, NH, DV, dtype=torch.bfloat16, device=dev)
    need(out, "out", (S, NH, DV), torch.bfloat16, dev)
    dbg = {}
    if debug:
        dbg = dict(scores=torch.zeros(S, max_ctx, dtype=torch.float32, device=dev),
                   topk=torch.empty(S, TOPK, dtype=torch.int32, device=dev))
    P = _lib.ptr
    args = _lib.AttnArgs(
        iq=P(step.iq), iqs=P(step.iqs), iw=P(step.iw), ikv=P(caches.ikv), iks=P(caches.iks),
        q=P(step.q), kv=P(caches.kv), kv_scale=P(caches.kv_scale), page_table=P(step.page_table),
        seq_lens=P(step.seq_lens), pt_stride=step.page_table.shape[1], n_pages=pages, out=P(out),
        rows=S, scores=P(dbg.get("scores")), topk=P(dbg.get("topk")), timeline=P(timeline),
    )  # fmt: skip
    if timeline is not None:
        need(timeline, "timeline", (n_tasks(max_ctx, S), 4), torch.int64, dev)
    return args, out, dbg

