"""The SGLang monokernel spec of this build and its forward (the plugin surface of the
reference: ``MonoSpec`` registered under backend ``amd``, sgl_amd_mono/glm53/spec.py:
584-616; ``_Built.forward`` routing by graph key, :277-317; the step tables built in the
graph, :467-496; ``_build`` once per rank at startup, :499-581).

Every covered layer (the MoE layers after ``first_k_dense_replace``) runs as the
layer runtime's launches (``layer.LayerRuntime``: front, sparse attention + back,
FP8 MoE); the embedding, the dense layers, the final norm and the logits stay on
SGLang's path. A decode or verify step whose rows exceed the runtime's widest step
runs the model's own forward. The kernels carry one GPU's TP=4 share of the layer
with the two TP all-reduces (after o_proj and after the MoE) replaced by a local
residual add, so a served model needs ``SGL_AMD_MONO_AMD_LOCAL_SHARE=1``: the
reduction over xGMI is not part of this build, and without it the spec refuses.
"""

from __future__ import annotations

import os

import torch

try:
    from sglang.kernels.plugin_kernels.amd.spec import (DeviceLimits, Feature, MonoSpec, Numerics, NumericsKind,
                                                        Requirements)
except ModuleNotFoundError:  # SGLang before the plugin-kernels package
    from sglang.srt.monokernels.spec import DeviceLimits, Feature, MonoSpec, Numerics, NumericsKind, Requirements

from . import sglang_bind
from .attn import PAGE, TOPK
from .layer import HEADS, HIDDEN, INDEX_DIM, INDEX_HEADS, KV_LORA, MAX_ROWS, NOPE_DIM, PE_DIM, Q_LORA, V_DIM
from .moe import FP8_MOE

# the model the kernels build in: DeepSeek-V3.2's shapes (config.json) with the
# reference's ungrouped sigmoid router (glm53/__init__.py:11-40: n_group 1)
HF_CONFIG = dict(
    hidden_size=HIDDEN,
    num_attention_heads=4 * HEADS,
    q_lora_rank=Q_LORA,
    kv_lora_rank=KV_LORA,
    qk_nope_head_dim=NOPE_DIM,
    qk_rope_head_dim=PE_DIM,
    v_head_dim=V_DIM,
    n_routed_experts=FP8_MOE.n_experts,
    num_experts_per_tok=FP8_MOE.top_k,
    n_shared_experts=1,
    moe_intermediate_size=4 * FP8_MOE.inter,
    routed_scaling_factor=FP8_MOE.route_scale,
    scoring_func="sigmoid",
    n_group=1,
    topk_group=1,
    norm_topk_prob=True,
    hidden_act="silu",
    rms_norm_eps=FP8_MOE.eps,
    index_n_heads=INDEX_HEADS,
    index_head_dim=INDEX_DIM,
    index_topk=TOPK,
)
# the rows a launch takes: any step up to MAX_ROWS runs at its own row count (no pad rows)
ROWS = tuple(range(1, MAX_ROWS + 1))
# the kernels carry one GPU's TP=4 share (32 heads, expert intermediate 512)
TP_SIZES = (4,)
# one persistent workgroup per CU of an MI355X
BLOCKS = 256
LOCAL_SHARE_ENV = "SGL_AMD_MONO_AMD_LOCAL_SHARE"
# the reference's test fault injection, rank:site[:after] (common/guard.py:79-88); site in
# the layer runtime's numbering (_lib.LAYER_SITES)
FAULT_INJECT_ENV = "SGLANG_AMD_MONO_FAULT_INJECT"
# a wait's deadline: below the server's watchdog, at most this long (common/guard.py:4-6)
MAX_DEADLINE_S = 60.0

# Each covered layer against SGLang's layer on the same input and caches (check mode,
# SGLANG_AMD_MONO_CHECK=1, check.py): the stream it hands on, the MLA row and the FP4
# index key it writes; on the selection, every key of the step's own chain SGLang
# selects, and exactly the top-2048 of its own scores (score descending, then position)
NUMERICS = Numerics(
    NumericsKind.TOLERANCE,
    {
        "layer.streams.cosine": 0.995,
        "layer.streams.rel": 5e-2,
        "layer.kv.cosine": 0.995,
        # one E2M1 code step moves a value by up to a third of it
        "layer.index.cosine": 0.99,
        "layer.topk_own.max_abs": 0.0,
        "layer.topk_exact.max_abs": 0.0,
    },
)


def covered_layers(hf_config) -> list[int]:
    """The MoE layers: every layer from ``first_k_dense_replace`` on."""
    return list(range(hf_config.first_k_dense_replace, hf_config.num_hidden_layers))


def max_context(context_len: int) -> int:
    """Keys a row may hold, rounded up to whole 64-key pages (the runtime's max_ctx)."""
    return -(-context_len // PAGE) * PAGE


def config_disable_reasons(cfg, hf_config) -> list[str]:
    """Why this server's config cannot run the kernels ([] when it can); every rank
    computes the same list from the same config."""
    reasons = [
        f"needs {key} = {want!r}, got {getattr(hf_config, key, None)!r}"
        for key, want in HF_CONFIG.items()
        if getattr(hf_config, key, None) != want
    ]
    if getattr(hf_config, "moe_layer_freq", 1) != 1:
        reasons.append(f"moe_layer_freq {hf_config.moe_layer_freq}: a launch carries a routed MoE, so every "
                       "layer from first_k_dense_replace on must have one")
    quant = getattr(hf_config, "quantization_config", None) or {}
    if quant.get("quant_method") != "fp8" or list(quant.get("weight_block_size") or ()) != [128, 128]:
        reasons.append(f"needs the FP8 block-128 checkpoint, got {quant.get('quant_method')!r} "
                       f"{quant.get('weight_block_size')!r}")
    rope = getattr(hf_config, "rope_parameters", None) or getattr(hf_config, "rope_scaling", None) or {}
    rope_type = rope.get("rope_type", rope.get("type", "default"))
    if rope_type != "default":
        reasons.append(f"RoPE {rope_type!r}: the kernels' softmax scale is unscaled")
    if getattr(cfg, "page_size", None) not in (None, PAGE):
        reasons.append(f"--page-size {cfg.page_size}: the DSA caches need {PAGE}")
    if getattr(cfg, "speculative_algorithm", None) is not None and (
        getattr(cfg, "speculative_eagle_topk", 1) != 1
        or cfg.speculative_num_draft_tokens != cfg.speculative_num_steps + 1
    ):
        reasons.append("speculative decoding: the launch's rows of a request must form one causal chain "
                       "(speculative_eagle_topk 1 and speculative_num_draft_tokens = speculative_num_steps + 1)")
    context_len = getattr(cfg, "context_length", None)
    if context_len is not None and max_context(context_len) > 32768:
        reasons.append(f"context {context_len}: a row holds at most 32768 keys on the kernels")
    if os.environ.get(LOCAL_SHARE_ENV) != "1":
        reasons.append(
            f"the kernels run one GPU's TP=4 share with a local residual add in place of the TP all-reduces "
            f"(the xGMI reduction is not built); set {LOCAL_SHARE_ENV}=1 to run that share alone"
        )
    return reasons


def model_disable_reasons(model, hf_config, copies: dict) -> list[str]:
    """Why the loaded model cannot run the kernels ([] when it can)."""
    reasons, row_major = [], {}
    for i in covered_layers(hf_config):
        layer = model.model.layers[i]
        why = sglang_bind.experts_reason(layer.mlp)
        if why is not None:
            reasons.append(f"layer {i}: {why}")
        if getattr(layer.self_attn, "indexer", None) is None:
            reasons.append(f"layer {i}: needs its own indexer")
            continue
        for name in sglang_bind.unshuffled(layer):
            row_major.setdefault(name, []).append(i)
    for name, ids in row_major.items():
        where = f"layer {ids[0]}" if len(ids) == 1 else f"{len(ids)} layers from {ids[0]}"
        reasons.append(f"{name} of {where} is row-major: the launches read FP8 weights in place in the "
                       "16 x 16 shuffled layout of SGLang's AITER block-FP8 path")
    return reasons


class _Layer:
    """One covered layer: its module and weights; its caches bind at its first launch
    and rebind if SGLang's pool moves them."""

    def __init__(self, i: int, module, weights):
        self.i, self.module, self.w = i, module, weights
        self.caches = None


class _Step:
    """The rows of one step as the launches read them, built on the device (in the
    graph when SGLang captures one) once per step."""

    def __init__(self, width: int, device):
        self.seq_lens = torch.zeros(width, dtype=torch.int32, device=device)
        self.page_table = None


class _Built:
    """One rank's monokernels: the layer runtime, each covered layer's weights, the
    rotary table, the step table, and the forward."""

    def __init__(self, lm, layers: dict, runtime, cos, sin, device, context_len: int):
        from .check import CHECK_ENV

        self.lm, self.model = lm, lm.model
        # check mode: each covered layer also runs SGLang's module and is measured against it
        self.check_layers = os.environ.get(CHECK_ENV) == "1"
        self._layers, self.runtime = layers, runtime
        self.first, self.last = min(layers), max(layers)
        self.max_rows = MAX_ROWS if runtime is None else runtime.max_rows
        self.max_position = context_len - 1
        self.cos, self.sin = cos, sin
        self.step = _Step(self.max_rows, device)

    def forward(self, plan, input_ids, positions, forward_batch, input_embeds=None, pp_proxy_tensors=None):
        """``DeepseekV2ForCausalLM.forward`` for a decode or verify step; a step wider
        than the runtime runs the model's own forward."""
        lm = self.lm
        # a launch that stopped earlier: raise before this step runs (the runtime's
        # fail-stop watcher ends the process within a millisecond or so of the stop,
        # also for replayed steps; this check catches an eager step inside that window)
        if self.runtime is not None:
            self.runtime.raise_pending()
        if plan.key.rows > self.max_rows:
            return type(lm).forward(lm, input_ids, positions, forward_batch, input_embeds, pp_proxy_tensors)
        hidden = self._backbone(plan, input_ids, positions, forward_batch, input_embeds)
        return lm.logits_processor(input_ids, hidden, lm.lm_head, forward_batch)

    def _backbone(self, plan, input_ids, positions, forward_batch, input_embeds):
        """``DeepseekV2Model.forward``: the embedding and the dense layers on SGLang's
        path (``layer(positions, hidden, forward_batch, residual)`` -> ``(hidden,
        residual)``), each covered layer as a launch on the whole stream, then the
        final norm."""
        m = self.model
        hidden = m.embed_tokens(input_ids) if input_embeds is None else input_embeds
        residual = None
        S = plan.key.rows
        for i in range(len(m.layers)):
            L = self._layers.get(i)
            if L is None:
                hidden, residual = m.layers[i](positions, hidden, forward_batch, residual)
                continue
            if residual is not None:  # the stream the dense layers left in two parts
                hidden, residual = hidden + residual, None
            hidden = self._layer(L, plan, positions, hidden[:S].contiguous(), forward_batch)
        if residual is not None:
            hidden, _ = m.norm(hidden, residual)
        else:
            hidden = m.norm(hidden)
        return hidden

    def _layer(self, L: _Layer, plan, positions, h, forward_batch):
        """One covered layer's launches on the stream ``h`` [S, 7168] bf16."""
        from sglang.srt.model_executor.forward_context import get_token_to_kv_pool

        S = h.shape[0]
        step = self._step(plan, positions, forward_batch, S)
        self._bind(L, get_token_to_kv_pool())
        args = (h, step.seq_lens[:S], step.page_table, L.caches, L.w, self.cos, self.sin)
        if not self.check_layers or (h.is_cuda and torch.cuda.is_current_stream_capturing()):
            return self.runtime.forward(*args, check_weights=False)
        from . import check  # eager steps only: the check reads results on the host

        ref = check.reference(L, positions, h, forward_batch, S, FP8_MOE.top_k, FP8_MOE.route_scale)
        out, inter = self.runtime.forward(*args, check_weights=False, keep=True)
        check.compare(L, ref, out, inter, step.seq_lens[:S], step.page_table, positions, S, NUMERICS)
        return out

    @staticmethod
    def _bind(L: _Layer, pool) -> None:
        kv = pool.get_key_buffer(L.i)
        if L.caches is not None and L.caches.kv.data_ptr() == kv.data_ptr():
            return
        L.caches = sglang_bind.caches(pool, L.i)

    def _step(self, plan, positions, forward_batch, S: int) -> _Step:
        """The step's rows for every launch, built once a step on the device (no host
        reads, so SGLang can capture it): a row at position p sees keys 0 ..= p of its
        request's pages (a verify row sees its draft chain up to itself); a pad row
        (SGLang's padding slot 0) gets 0 keys and writes no cache."""
        if "step" not in plan.state:
            from sglang.srt.model_executor.forward_context import get_attn_backend

            st = self.step
            loc = forward_batch.out_cache_loc[:S].to(torch.int64)
            pos = positions[:S].to(torch.int64).clamp(max=self.max_position)
            st.seq_lens[:S] = torch.where(loc != 0, pos + 1, 0).to(torch.int32)
            st.page_table = get_attn_backend().forward_metadata.real_page_table[:S]
            plan.state["step"] = st
        return plan.state["step"]


def _build(model, hf_config, ctx) -> _Built:
    """Bind every covered layer's weights (in place, the copies logged in
    ``ctx.copies``), read the rotary table, and create the layer runtime for the
    widest routed step, once and outside graph capture."""
    from sglang.srt.runtime_context import get_parallel, process_model_config

    from .layer import LayerRuntime

    p = get_parallel()
    if p.tp_size not in TP_SIZES:
        raise ValueError(f"monokernel: TP{p.tp_size}; the kernels carry one GPU's share at TP {TP_SIZES}")
    covered = covered_layers(hf_config)
    layers = {i: _Layer(i, model.model.layers[i], sglang_bind.layer_weights(model.model.layers[i], i, ctx.copies))
              for i in covered}
    cos, sin = sglang_bind.rope_tables([model.model.layers[i] for i in covered], ctx.copies)
    context_len = process_model_config().context_len
    if cos.shape[0] < context_len:
        raise ValueError(f"monokernel: the rotary table holds {cos.shape[0]} positions, the context is {context_len}")
    widths = [w for w in ctx.widths if w <= MAX_ROWS]
    if not widths:
        raise ValueError(f"monokernel: the kernels run at most {MAX_ROWS} rows; this server routes {sorted(ctx.widths)}")
    device = cos.device
    rt = LayerRuntime(max(widths), max_context(context_len), device)
    rt.set_deadline(deadline_seconds(ctx))
    fault = fault_injection(p.tp_rank)
    if fault is not None:
        rt.handle.set_fault(*fault)
    # a stopped launch ends the process, also in steps replayed from a graph
    rt.watch()
    return _Built(model, layers, rt, cos, sin, device, context_len)


def deadline_seconds(ctx) -> float:
    """Every wait's deadline: the framework's own (``ctx.deadline_s``, half its watchdog
    at most 60 s, as the reference's build takes it, glm53/spec.py:569), else half of
    ``ctx.watchdog_timeout`` at most 60 s, else 60 s."""
    given = getattr(ctx, "deadline_s", None)
    if given:
        return float(given)
    watchdog = getattr(ctx, "watchdog_timeout", None)
    return min(0.5 * float(watchdog), MAX_DEADLINE_S) if watchdog else MAX_DEADLINE_S


def fault_injection(rank: int):
    """This rank's test fault from ``SGLANG_AMD_MONO_FAULT_INJECT=rank:site[:after]``:
    (site, after) for ``LayerHandle.set_fault``, or None (the reference's
    common/guard.py:79-88: once ``after`` launches have run, the wait at ``site``
    fails)."""
    spec = os.environ.get(FAULT_INJECT_ENV, "")
    if not spec:
        return None
    parts = (spec.split(":") + ["0", "0"])[:3]
    try:
        r, site, after = (int(x or 0) for x in parts)
    except ValueError:
        raise ValueError(f"{FAULT_INJECT_ENV}={spec!r}: expected rank:site[:after] integers") from None
    return (site, after) if r == rank else None


SPEC = MonoSpec(
    name="mono_layer_gfx950",
    devices={"gfx950": DeviceLimits(widths=ROWS, tp_sizes=TP_SIZES, resident_blocks=BLOCKS)},
    features=frozenset({Feature.SPECULATIVE_DECODING}),
    requires=Requirements(
        dtypes=frozenset({"bfloat16"}),
        attention_backends=frozenset({"dsa"}),
        server_args={
            # the launches write SGLang's raw E4M3 MLA rows
            "kv_cache_dtype": frozenset({"fp8_e4m3"}),
            "moe_runner_backend": frozenset({"auto", "aiter"}),
            "speculative_algorithm": frozenset({None, "EAGLE"}),
            "enable_hisparse": frozenset({False}),
            "expert_distribution_recorder_mode": frozenset({None}),
        },
        env={
            "SGLANG_SIMULATE_UNIFORM_EXPERTS": False,
            "SGLANG_SIMULATE_ROUND_ROBIN_EXPERTS": False,
        },
    ),
    numerics=NUMERICS,
    model_disable_reasons=model_disable_reasons,
    build=_build,
    api_version=1,
    config_disable_reasons=config_disable_reasons,
)
