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

import torch
import torch.nn.functional as F

from .attn import PAGE, TOPK

logger = logging.getLogger(__name__)

CHECK_ENV = "SGLANG_AMD_MONO_CHECK"
# SGLang's id of the shared expert it fuses after the routed ones
SHARED_EXPERT = 256
# E2M1 code -> value (codes 8..15 the negatives), two codes a byte, element 2i low
_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def _metrics(a: torch.Tensor, b: torch.Tensor) -> dict[str, float]:
    a, b = a.float().reshape(-1), b.float().reshape(-1)
    if a.numel() == 0:
        return {}
    return {
        "max_abs": float((a - b).abs().max()),
        "rel": float((a - b).norm() / b.norm().clamp_min(1e-30)),
        "cosine": float(F.cosine_similarity(a, b, dim=0)),
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


def _f32_routing(mlp, top_k: int, route_scale: float):
    """Hooks that route SGLang's MoE in f32 as the launch does (sigmoid scores, the 8
    largest of score + bias, weights the scores over their sum times the route scale)
    where the module's top-k would add the bias in bf16; the fused shared expert's
    entries keep SGLang's values. Returns the hook handles ([] when the module has no
    ``gate`` / ``topk`` submodules to hook)."""
    gate, topk = getattr(mlp, "gate", None), getattr(mlp, "topk", None)
    if not (hasattr(mlp, "register_forward_pre_hook") and hasattr(topk, "register_forward_hook")):
        return []
    seen = {}

    def take_input(mod, args):
        seen["x"] = args[0]

    def reroute(mod, args, out):
        x = seen.pop("x")
        scores = torch.sigmoid(x.float() @ gate.weight.float().t())
        ids = (scores + gate.e_score_correction_bias.float()).topk(top_k, -1).indices
        raw = scores.gather(1, ids)
        routed = out.topk_ids != SHARED_EXPERT
        new_ids, new_w = out.topk_ids.clone(), out.topk_weights.clone()
        new_ids[routed] = ids.to(new_ids.dtype).reshape(-1)
        new_w[routed] = (raw / raw.sum(-1, keepdim=True) * route_scale).to(new_w.dtype).reshape(-1)
        return out._replace(topk_weights=new_w, topk_ids=new_ids)

    return [mlp.register_forward_pre_hook(take_input), topk.register_forward_hook(reroute)]


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
    hooks = _f32_routing(getattr(L.module, "mlp", None), top_k, route_scale) + _selection_hook(L.module, seen)
    try:
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


def compare(L, ref: dict, out: torch.Tensor, inter: dict, seq_lens: torch.Tensor, page_table: torch.Tensor,
            positions: torch.Tensor, S: int, numerics) -> tuple[dict, list]:
    """Measure the launch (``out`` and the intermediates ``forward(keep=True)`` returned)
    against ``ref``; log every value and every violation of ``numerics.bounds``.
    Returns (values, violations) with violations as (name, value, bound)."""
    outputs = {"streams": _metrics(out[:S], ref["streams"])}
    regions = _Regions(L.caches, ref["slots"])
    got, want = regions.read(), ref["regions"]
    if regions.slots.numel():
        outputs["kv"] = _metrics(_kv_values(got["kv"], got.get("kv_scale")),
                                 _kv_values(want["kv"], want.get("kv_scale")))
        outputs["index"] = _metrics(_index_values(got["ikv"], got["iks"]), _index_values(want["ikv"], want["iks"]))
    sel = inter["topk_slots"][:S]
    outputs["topk_exact"] = {"max_abs": float(topk_exact_missed(inter["index_scores"], sel, seq_lens[:S],
                                                                 page_table))}
    if ref.get("topk") is not None:
        outputs.update(_topk_vs_sglang(ref["topk"], sel, regions.slots))
    values = {f"layer.{o}.{m}": v for o, ms in outputs.items() for m, v in ms.items()}
    pos = positions[:S]
    logger.info("monokernel check layer %d (%d rows, positions %d..%d): %s", L.i, S, int(pos.min()), int(pos.max()),
                " ".join(f"{k}={v:.6g}" for k, v in values.items()))
    violations = []
    for name, bound in numerics.bounds.items():
        v = values.get(name)
        if v is None:
            continue
        if not (v >= bound if name.endswith(".cosine") else v <= bound):
            violations.append((name, v, bound))
            logger.error("monokernel check violation: layer %d %s = %.6g, bound %g", L.i, name, v, bound)
    return values, violations
