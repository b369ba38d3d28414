"""Check mode (``SGLANG_AMD_MONO_CHECK=1``, eager steps only; the reference's
glm53/check.py:183-277 and its call site glm53/spec.py:394-413): every covered layer
also runs SGLang's own layer module on the same input and on the caches as they were,
and the launch's outputs are measured against it:

* ``streams``: the hidden stream the layer hands on (max_abs, rel, cosine);
* ``kv``: the MLA cache rows the step writes, decoded (E4M3, times the row scale when
  the cache has a scale plane);
* ``index``: the FP4 index keys the step writes, decoded (E2M1 times E8M0 per 32 dims);
* ``topk_exact``: over the rows past 2048 keys, the most keys of the exact top-2048 of
  the launch's own index scores (score descending, then position) a selection misses;
* ``topk_own`` / ``topk`` (when the layer's indexer module exposes its selection as
  KV slots, -1 past a row's keys): the most of the step's own new slots a row's
  selection misses among those SGLang selects, and the largest share of SGLang's
  selection a row misses.

Each value is logged; one past its bound in ``spec.NUMERICS`` is logged as a
violation. SGLang's module runs first and the cache rows it wrote are restored before
the launch writes its own, so both start from the same caches.
"""

from __future__ import annotations

import logging
import math

import torch

from .attn import PAGE, TOPK

logger = logging.getLogger(__name__)

CHECK_ENV = "SGLANG_AMD_MONO_CHECK"
# SGLang's id of the shared expert it fuses after the routed ones
SHARED_EXPERT = 256
# E2M1 code -> value (codes 8..15 the negatives), two codes a byte, element 2i low
_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def _distances(got: torch.Tensor, want: torch.Tensor) -> dict[str, float]:
    """How far ``got`` lies from ``want``, in float64 over the flattened values: the
    largest elementwise difference, the difference's norm relative to ``want``'s, and
    the cosine of the angle between them (1 when both are zero)."""
    g = got.detach().reshape(-1).double()
    w = want.detach().reshape(-1).double().to(g.device)
    if g.numel() == 0:
        return {}
    d = g - w
    gg, ww, gw = float(g @ g), float(w @ w), float(g @ w)
    tiny = 1e-60
    return {
        "max_abs": float(d.abs().max()),
        "rel": (float(d @ d) / max(ww, tiny)) ** 0.5,
        "cosine": 1.0 if gg == ww == 0.0 else gw / max((gg * ww) ** 0.5, tiny),
    }


def _scale_byte(t: torch.Tensor) -> torch.Tensor:
    """Where key ``t`` (0..63 in its page) keeps its E8M0 byte among a block's 64."""
    return (t % 16) * 4 + t // 16


def _index_values(payload: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Index keys [n, 4, 16] packed E2M1 with E8M0 scales [n, 4] -> f32 [n, 128]."""
    lut = torch.tensor(_E2M1, dtype=torch.float32, device=payload.device)
    p = payload.long()
    vals = torch.stack([lut[p & 15], lut[p >> 4]], -1).reshape(*p.shape[:-1], 32)
    return (vals * torch.exp2(scales.float() - 127.0)[..., None]).reshape(p.shape[0], 128)


def _kv_values(rows: torch.Tensor, scale: torch.Tensor | None) -> torch.Tensor:
    v = rows.contiguous().view(torch.float8_e4m3fn).float()
    return v if scale is None else v * scale[:, None].float()


class _Regions:
    """The cache entries a step writes: the MLA rows at its new slots and those keys'
    index bytes (payload and scale)."""

    def __init__(self, caches, slots: torch.Tensor):
        self.c = caches
        self.slots = slots[slots != 0].long()  # SGLang's padding slot 0 marks a pad row
        self.pages, self.offs = self.slots // PAGE, self.slots % PAGE
        self.blk = torch.arange(4, device=self.slots.device)

    def read(self) -> dict:
        c, p, t = self.c, self.pages, self.offs
        out = {"kv": c.kv[self.slots].clone(),
               "ikv": c.ikv[p, :, t].clone(),
               "iks": c.iks[p[:, None], self.blk[None], _scale_byte(t)[:, None]].clone()}
        if c.kv_scale is not None:
            out["kv_scale"] = c.kv_scale[self.slots].clone()
        return out

    def write(self, saved: dict) -> None:
        c, p, t = self.c, self.pages, self.offs
        c.kv[self.slots] = saved["kv"]
        c.ikv[p, :, t] = saved["ikv"]
        c.iks[p[:, None], self.blk[None], _scale_byte(t)[:, None]] = saved["iks"]
        if c.kv_scale is not None:
            c.kv_scale[self.slots] = saved["kv_scale"]


def launch_routing(x: torch.Tensor, gate_w: torch.Tensor, bias: torch.Tensor, top_k: int,
                   route_scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """The launch's routing rule on the host, in f32 (glm53/gfx950/kernel.py:4199-4330):
    logits of the MoE input against the router rows, sigmoid scores, the ``top_k``
    experts of the largest score + bias (f32, not bf16), each weighted by its score over
    the picked scores' sum times ``route_scale``. Returns (ids [S, top_k] int64,
    weights [S, top_k] f32)."""
    score = torch.sigmoid(x.float() @ gate_w.float().t())
    pick = torch.topk(score + bias.float(), top_k, dim=-1).indices
    chosen = torch.take_along_dim(score, pick, dim=-1)
    return pick, chosen * (route_scale / chosen.sum(-1, keepdim=True))


class _RouteAsTheLaunch:
    """While active, SGLang's MoE module routes as the launch does: a forward hook on
    its ``topk`` submodule (which receives the MoE input as its first argument) recomputes
    the routed columns with ``launch_routing`` and keeps the fused shared expert's
    trailing columns (id ``SHARED_EXPERT``) as SGLang made them. SGLang's own top-k adds
    the correction bias in bf16, which can pick other experts than the f32 rule. A
    module without ``gate`` / ``topk`` is left alone."""

    def __init__(self, mlp, top_k: int, route_scale: float):
        self.gate, self.topk = getattr(mlp, "gate", None), getattr(mlp, "topk", None)
        self.k, self.scale = top_k, route_scale
        self.handle = None

    def __enter__(self):
        if self.gate is not None and hasattr(self.topk, "register_forward_hook"):
            self.handle = self.topk.register_forward_hook(self._rewrite, with_kwargs=True)
        return self

    def __exit__(self, *exc) -> None:
        if self.handle is not None:
            self.handle.remove()
            self.handle = None

    def _rewrite(self, module, args, kwargs, out):
        x = args[0] if args else kwargs["hidden_states"]
        ids, weights = launch_routing(x, self.gate.weight, self.gate.e_score_correction_bias, self.k, self.scale)
        shared_ids, shared_w = out.topk_ids[:, self.k:], out.topk_weights[:, self.k:]
        if not bool((shared_ids == SHARED_EXPERT).all()):
            raise ValueError(f"check mode: SGLang's top-k output has {out.topk_ids.shape[1]} columns; the ones "
                             f"past {self.k} must be the fused shared expert {SHARED_EXPERT}")
        return out._replace(topk_ids=torch.cat([ids.to(out.topk_ids.dtype), shared_ids], 1),
                            topk_weights=torch.cat([weights.to(out.topk_weights.dtype), shared_w], 1))


def _selection_hook(module, seen: dict):
    """Record the indexer module's selection (its output, or the output's first item)."""
    indexer = getattr(getattr(module, "self_attn", None), "indexer", None)
    if not hasattr(indexer, "register_forward_hook"):
        return []

    def keep(mod, args, out):
        seen["topk"] = (out[0] if isinstance(out, (tuple, list)) else out).detach().clone()

    return [indexer.register_forward_hook(keep)]


def reference(L, positions: torch.Tensor, h: torch.Tensor, forward_batch, S: int, top_k: int,
              route_scale: float) -> dict:
    """SGLang's layer ``L.module`` on a copy of the stream ``h`` [S, 7168] bf16 (routed
    in f32): the stream it hands on, its selection when its indexer exposes one, and
    the cache rows it writes. The caches are restored afterwards."""
    regions = _Regions(L.caches, forward_batch.out_cache_loc[:S])
    saved = regions.read()
    seen = {}
    hooks = _selection_hook(L.module, seen)
    try:
        with _RouteAsTheLaunch(getattr(L.module, "mlp", None), top_k, route_scale):
            out, residual = L.module(positions[:S], h.clone(), forward_batch, None)
    finally:
        for hook in hooks:
            hook.remove()
    stream = out if residual is None else out + residual
    ref = {"streams": stream[:S].clone(), "topk": seen.get("topk"), "regions": regions.read(),
           "slots": forward_batch.out_cache_loc[:S].clone()}
    regions.write(saved)
    return ref


def _radix_keys(scores: torch.Tensor) -> torch.Tensor:
    """f32 scores -> int64 keys of the same order (larger score, larger key)."""
    b = scores.contiguous().view(torch.int32).to(torch.int64)
    return torch.where(b >= 0, b + (1 << 31), ~b & 0xFFFFFFFF)


def topk_exact_missed(scores: torch.Tensor, selection: torch.Tensor, seq_lens: torch.Tensor,
                      page_table: torch.Tensor) -> int:
    """Over the rows past TOPK keys, the most slots of the exact top-TOPK of the row's
    own scores (descending, then lowest position) that its selection misses."""
    missed = 0
    for s, n in enumerate(seq_lens.tolist()):
        if n <= TOPK:
            continue
        pos = torch.sort(_radix_keys(scores[s, :n]), descending=True, stable=True).indices[:TOPK]
        want = page_table[s, pos // PAGE].long() * PAGE + pos % PAGE
        missed = max(missed, TOPK - int(torch.isin(want, selection[s].long()).sum()))
    return missed


def _topk_vs_sglang(ref_topk: torch.Tensor, selection: torch.Tensor, own: torch.Tensor) -> dict:
    rel, own_missed = 0.0, 0
    ref_topk, own = ref_topk.to(selection.device), own.to(selection.device)
    for s in range(selection.shape[0]):
        want = ref_topk[s][ref_topk[s] >= 0].long()
        if want.numel() == 0:
            continue
        missed = want[~torch.isin(want, selection[s].long())]
        rel = max(rel, missed.numel() / want.numel())
        own_missed = max(own_missed, int(torch.isin(missed, own).sum()))
    return {"topk": {"rel": rel}, "topk_own": {"max_abs": float(own_missed)}}


def _outside(name: str, value: float, bound: float) -> bool:
    """A cosine is bounded from below, every other metric from above; NaN is outside
    every bound."""
    if math.isnan(value):
        return True
    return value < bound if name.endswith(".cosine") else value > bound


def compare(L, ref: dict, out: torch.Tensor, inter: dict, seq_lens: torch.Tensor, page_table: torch.Tensor,
            positions: torch.Tensor, S: int, numerics) -> tuple[dict, list]:
    """Measure the launch (``out`` and the intermediates ``forward(keep=True)`` returned)
    against ``ref``: one INFO record with every value of the layer, one ERROR record per
    value outside its bound in ``numerics.bounds``. Returns (values, violations), the
    violations as (name, value, bound)."""
    regions = _Regions(L.caches, ref["slots"])
    got, want = regions.read(), ref["regions"]
    measured = {"streams": _distances(out[:S], ref["streams"])}
    if regions.slots.numel():
        measured["kv"] = _distances(_kv_values(got["kv"], got.get("kv_scale")),
                                    _kv_values(want["kv"], want.get("kv_scale")))
        measured["index"] = _distances(_index_values(got["ikv"], got["iks"]),
                                       _index_values(want["ikv"], want["iks"]))
    sel = inter["topk_slots"][:S]
    missed = topk_exact_missed(inter["index_scores"], sel, seq_lens[:S], page_table)
    measured["topk_exact"] = {"max_abs": float(missed)}
    if ref.get("topk") is not None:
        measured.update(_topk_vs_sglang(ref["topk"], sel, regions.slots))
    values = {f"layer.{part}.{metric}": v for part, ms in measured.items() for metric, v in ms.items()}
    lo, hi = int(positions[:S].min()), int(positions[:S].max())
    logger.info("check mode, layer %d against SGLang's module, %d rows at positions [%d, %d]: %s", L.i, S, lo, hi,
                ", ".join(f"{k}={v:.6g}" for k, v in values.items()))
    violations = [(k, values[k], b) for k, b in numerics.bounds.items() if k in values and _outside(k, values[k], b)]
    for k, v, b in violations:
        logger.error("check mode, layer %d: %s is %.6g, outside its bound %g", L.i, k, v, b)
    return values, violations
