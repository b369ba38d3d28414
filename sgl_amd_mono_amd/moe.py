"""Host side of the MoE phase: a runtime per (width, geometry) and its forward calls.

Mirrors the reference's runtime / launch split (sgl_amd_mono/glm53/gfx950/runner.py:
``Glm53Runtime`` :133-215 owns the scratch; ``Glm53LayerOp.launch`` :240-321 checks
every tensor's shape, dtype and stride and dispatches raw pointers). Here the
scratch lives in the C library's handle; this module checks the tensors, passes
their ``data_ptr()`` through the C-ABI and enqueues on the current stream.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from .runtime import Runtime, need


@dataclass(frozen=True)
class MoeGeometry:
    """One GPU's share of a MoE layer."""

    hidden: int
    n_experts: int
    top_k: int
    inter: int
    route_scale: float
    eps: float
    router: str  # "sigmoid_bias" | "softmax"
    weights: str  # "fp8_block128" | "mxfp4"


# DeepSeek-V3.2-shaped MoE at TP=4 (intermediate 2048 / 4)
FP8_MOE = MoeGeometry(7168, 256, 8, 512, 2.5, 1e-6, "sigmoid_bias", "fp8_block128")
# MXFP4 experts at TP=4 (intermediate 1536 / 4), softmax router
MXFP4_MOE = MoeGeometry(3072, 256, 8, 384, 1.0, 0.0, "softmax", "mxfp4")


@dataclass
class Fp8MoeWeights:
    """One layer's MoE tensors as SGLang loads them (read in place, never copied)."""

    g_post: torch.Tensor  # bf16 [H]
    w_router: torch.Tensor  # bf16 [E, H]
    bias: torch.Tensor  # f32 [E]
    w13: torch.Tensor  # float8_e4m3fn / uint8 [E+1, 2I, H], AITER (16, 16) layout
    s13: torch.Tensor  # f32 [E+1, 2I/128, H/128]
    w2: torch.Tensor  # float8_e4m3fn / uint8 [E+1, H, I], AITER (16, 16) layout
    s2: torch.Tensor  # f32 [E+1, H/128, I/128]


@dataclass
class Mxfp4MoeWeights:
    w13: torch.Tensor  # uint8 [E+1, 2I, H/2] packed E2M1, AITER (16, 16) layout
    s13: torch.Tensor  # uint8 [E+1, 2I, H/32] E8M0
    w2: torch.Tensor  # uint8 [E+1, H, I/2] packed E2M1, AITER (16, 16) layout
    s2: torch.Tensor  # uint8 [E+1, H, I/32] E8M0


FP8_TYPES = (torch.float8_e4m3fn, torch.uint8)


class MoeRuntime(Runtime):
    """The C library's MoE handle for one geometry and a widest step ``max_rows``."""

    PREFIX = "mono_moe"
    SITES = _lib.MOE_SITES
    KIND = "MoE"

    def __init__(self, geo: MoeGeometry, max_rows: int, device=None):
        super().__init__(device)
        self.geo = geo
        self.max_rows = max_rows
        cfg = _lib.MoeConfig(
            device=self.device.index, max_rows=max_rows, hidden=geo.hidden, n_experts=geo.n_experts,
            top_k=geo.top_k, inter=geo.inter,
            weight_format=_lib.WEIGHT_FP8_BLOCK128 if geo.weights == "fp8_block128" else _lib.WEIGHT_MXFP4,
            router=_lib.ROUTER_SIGMOID_BIAS if geo.router == "sigmoid_bias" else _lib.ROUTER_SOFTMAX,
            route_scale=geo.route_scale, eps=geo.eps,
        )  # fmt: skip
        self._create(cfg)

    def forward_fp8(self, a: torch.Tensor, w: Fp8MoeWeights, out: torch.Tensor | None = None,
                    debug: bool = False):
        """``a + MoE(a)`` for one decode step. ``debug`` also
        returns the routing (scores, top-k ids / weights) and the f32 MoE sum."""
        args, out, dbg = fp8_args(self.device, self.max_rows, self.geo, a, w, out, debug)
        _lib.check(_lib.lib().mono_moe_fp8_forward(self._h, C.byref(args), self._stream()))
        return (out, dbg) if debug else out

    def mxfp4_tasks(self) -> int:
        """Rows of an MXFP4 launch's timeline: the task list at most (every expert slot's
        24 up tiles and 12 down groups, then 96 final tasks)."""
        max_act = min(self.max_rows * self.geo.top_k, self.geo.n_experts) + 1
        return max_act * (self.geo.inter // 16 + self.geo.hidden // 256) + self.geo.hidden // 32

    def forward_mxfp4(self, x: torch.Tensor, logits: torch.Tensor, w: Mxfp4MoeWeights,
                      out: torch.Tensor | None = None, debug: bool = False, timeline: torch.Tensor | None = None):
        """``MoE(x)`` with MXFP4 experts behind a softmax router.
        ``timeline`` (int64 [mxfp4_tasks(), 4]) receives each task's start,
        inputs-ready and end ticks and workgroup << 8 | kind (1 up, 2 down, 3 final)."""
        g, dev = self.geo, self.device
        H, E, I, K = g.hidden, g.n_experts, g.inter, g.top_k
        if x.dim() != 2 or not 1 <= x.shape[0] <= self.max_rows:
            raise ValueError(f"x: expected [rows <= {self.max_rows}, {H}], got {tuple(x.shape)}")
        S = x.shape[0]
        need(x, "x", (S, H), torch.bfloat16, dev)
        need(logits, "logits", (S, E), torch.float32, dev)
        need(w.w13, "w13", (E + 1, 2 * I, H // 2), torch.uint8, dev)
        need(w.s13, "s13", (E + 1, 2 * I, H // 32), torch.uint8, dev)
        need(w.w2, "w2", (E + 1, H, I // 2), torch.uint8, dev)
        need(w.s2, "s2", (E + 1, H, I // 32), torch.uint8, dev)
        if out is None:
            out = torch.empty_like(x)
        need(out, "out", (S, H), torch.bfloat16, dev)
        if timeline is not None:
            need(timeline, "timeline", (self.mxfp4_tasks(), 4), torch.int64, dev)
        dbg = {}
        if debug:
            dbg = dict(
                y=torch.empty(S, H, dtype=torch.float32, device=dev),
                topk_ids=torch.empty(S, K, dtype=torch.int32, device=dev),
                topk_w=torch.empty(S, K, dtype=torch.float32, device=dev),
            )
        P = _lib.ptr
        args = _lib.MoeMxfp4Args(
            x=P(x), logits=P(logits), w13=P(w.w13), s13=P(w.s13), w2=P(w.w2), s2=P(w.s2),
            out=P(out), rows=S, y=P(dbg.get("y")), topk_ids=P(dbg.get("topk_ids")),
            topk_w=P(dbg.get("topk_w")), timeline=P(timeline),
        )  # fmt: skip
        _lib.check(_lib.lib().mono_moe_mxfp4_forward(self._h, C.byref(args), self._stream()))
        return (out, dbg) if debug else out

def fp8_args(dev, max_rows: int, geo: MoeGeometry, a: torch.Tensor, w: Fp8MoeWeights, out: torch.Tensor | None,
             debug: bool):
    """Checked mono_moe_fp8_args for a runtime of ``max_rows`` on ``dev``: (args, out,
    debug outputs)."""
    g = geo
    H, E, I, K = g.hidden, g.n_experts, g.inter, g.top_k
    if a.dim() != 2 or not 1 <= a.shape[0] <= max_rows:
        raise ValueError(f"a: expected [rows <= {max_rows}, {H}], got {tuple(a.shape)}")
    S = a.shape[0]
    need(a, "a", (S, H), torch.bfloat16, dev)
    need(w.g_post, "g_post", (H,), torch.bfloat16, dev)
    need(w.w_router, "w_router", (E, H), torch.bfloat16, dev)
    need(w.bias, "bias", (E,), torch.float32, dev)
    need(w.w13, "w13", (E + 1, 2 * I, H), FP8_TYPES, dev)
    need(w.s13, "s13", (E + 1, 2 * I // 128, H // 128), torch.float32, dev)
    need(w.w2, "w2", (E + 1, H, I), FP8_TYPES, dev)
    need(w.s2, "s2", (E + 1, H // 128, I // 128), torch.float32, dev)
    if out is None:
        out = torch.empty_like(a)
    need(out, "out", (S, H), torch.bfloat16, dev)
    dbg = {}
    if debug:
        dbg = dict(
            y=torch.empty(S, H, dtype=torch.float32, device=dev),
            scores=torch.empty(S, E, dtype=torch.float32, device=dev),
            topk_ids=torch.empty(S, K, dtype=torch.int32, device=dev),
            topk_w=torch.empty(S, K, dtype=torch.float32, device=dev),
        )
    P = _lib.ptr
    args = _lib.MoeFp8Args(
        a=P(a), g_post=P(w.g_post), w_router=P(w.w_router), bias=P(w.bias),
        w13=P(w.w13), s13=P(w.s13), w2=P(w.w2), s2=P(w.s2), out=P(out), rows=S,
        y=P(dbg.get("y")), scores=P(dbg.get("scores")),
        topk_ids=P(dbg.get("topk_ids")), topk_w=P(dbg.get("topk_w")),
    )  # fmt: skip
    return args, out, dbg
