"""The SGLang spec's forward on the GPU (sgl_amd_mono_amd.spec) through the stand-in
registry: a three-layer model (one dense layer on "SGLang's" path, two covered layers)
whose tensors sit in SGLang's module layout and DSA pools, built by ``SPEC.build`` and
run by ``_Built.forward`` for a 4-row decode step. The covered layers' output must be
bit for bit what the layer runtime gives when called directly on the same bound
weights, caches and step, and a 17-row step must run the model's own forward."""

import sys
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "fake_sglang"))

from sglang.kernels.plugin_kernels.amd import spec as registry  # noqa: E402
from sglang.srt import runtime_context  # noqa: E402
from sglang.srt.model_executor import forward_context  # noqa: E402

from oracle import codecs as ocodecs  # noqa: E402
from sgl_amd_mono_amd import workloads  # noqa: E402
from sgl_amd_mono_amd.layer import LayerRuntime  # noqa: E402
from sgl_amd_mono_amd.moe import FP8_MOE  # noqa: E402

pytestmark = pytest.mark.gpu

CTX, ROWS = 4096, 4


def _linear(w, s):
    lin = SimpleNamespace(weight=w.view(torch.float8_e4m3fn), weight_scale_inv=s)
    lin.aiter_bpreshuffled = True
    return lin


def _sglang_layer(seed, dev, rot):
    """Synthetic weights of one layer in SGLang's module names (FP8 linears already in
    the (16, 16) layout, the shared expert fused as expert 256)."""
    return _sglang_layer_of(workloads.proj_weights(dev, seed=seed), workloads.fp8_moe_weights(FP8_MOE, dev, seed=seed + 1),
                            dev, rot)


def _sglang_layer_of(p, m, dev, rot):
    uk = ocodecs.aiter_unshuffle(p.w_uk.cpu()).reshape(32, 512, 128)
    uv = ocodecs.aiter_unshuffle(p.w_uv.cpu()).reshape(32, 128, 512)
    iw = ocodecs.aiter_unshuffle(p.w_iw.cpu().view(torch.uint8)).view(torch.bfloat16)
    ind = SimpleNamespace(wk=_linear(p.w_ik, p.s_ik), wq_b=_linear(p.w_iq, p.s_iq),
                          weights_proj=SimpleNamespace(weight=iw.to(dev)),
                          k_norm=SimpleNamespace(weight=p.g_ik, bias=p.b_ik), rotary_emb=rot)
    attn = SimpleNamespace(
        fused_qkv_a_proj_with_mqa=_linear(p.w_qkv, p.s_qkv), q_b_proj=_linear(p.w_qb, p.s_qb),
        o_proj=_linear(p.w_o, p.s_o), w_kc=uk.transpose(1, 2).contiguous().view(torch.float8_e4m3fn).to(dev),
        w_vc=uv.transpose(1, 2).contiguous().view(torch.float8_e4m3fn).to(dev),
        w_scale=torch.tensor(0.004, device=dev), indexer=ind, rotary_emb=rot,
        q_a_layernorm=SimpleNamespace(weight=p.g_q), kv_a_layernorm=SimpleNamespace(weight=p.g_kv),
    )  # fmt: skip
    experts = SimpleNamespace(w13_weight=m.w13.view(torch.float8_e4m3fn), w13_weight_scale_inv=m.s13,
                              w2_weight=m.w2.view(torch.float8_e4m3fn), w2_weight_scale_inv=m.s2, is_shuffled=True)
    gate = SimpleNamespace(weight=m.w_router, e_score_correction_bias=m.bias)
    return SimpleNamespace(self_attn=attn, mlp=SimpleNamespace(experts=experts, gate=gate),
                           input_layernorm=SimpleNamespace(weight=p.g_in),
                           post_attention_layernorm=SimpleNamespace(weight=m.g_post))


def test_spec_forward_runs_the_launches(gpu_device, monkeypatch):
    from sgl_amd_mono_amd import spec as mono

    dev = gpu_device
    monkeypatch.setenv(mono.LOCAL_SHARE_ENV, "1")
    cos, sin = workloads.rope_tables(CTX, dev)
    rot = SimpleNamespace(cos_sin_cache=torch.cat([cos, sin], -1))
    print("[spec] building a 3-layer SGLang-shaped model", flush=True)
    dense_calls = []

    def dense(positions, hidden, batch, residual):
        dense_calls.append(hidden.shape)
        return hidden * 0.5, hidden * 0.5

    layers = [dense, _sglang_layer(11, dev, rot), _sglang_layer(12, dev, rot)]
    model = SimpleNamespace(embed_tokens=lambda ids: workloads.rows_bf16(ROWS, 7168, dev, seed=13), layers=layers,
                            norm=lambda h, r=None: (h + r, None) if r is not None else h)
    lm = SimpleNamespace(model=model, lm_head=None, logits_processor=lambda ids, h, head, batch: h)
    hf = SimpleNamespace(first_k_dense_replace=1, num_hidden_layers=3)
    lens = [4096, 1500, 65, 2049]
    step, c1 = workloads.attn_case(lens, dev, seed=14, max_ctx=CTX)
    _, c2 = workloads.attn_case(lens, dev, seed=14, max_ctx=CTX)
    pools = {}
    for i, c in ((1, c1), (2, c2)):
        pools[i] = (c.kv.view(-1, 1, 576), c.ikv.view(-1, 1, 4, 64, 16), c.iks.view(-1, 1, 4, 64))
    forward_context.POOL = SimpleNamespace(get_key_buffer=lambda i: pools[i][0],
                                           get_index_k_fp4_payload_buffer=lambda i: pools[i][1],
                                           get_index_k_fp4_scale_buffer=lambda i: pools[i][2])
    forward_context.ATTN_BACKEND = SimpleNamespace(forward_metadata=SimpleNamespace(real_page_table=step.page_table))
    runtime_context.PARALLEL = SimpleNamespace(tp_size=4, tp_rank=0, tp_group=None)
    runtime_context.MODEL_CONFIG = SimpleNamespace(context_len=CTX)
    assert mono.model_disable_reasons(lm, hf, {}) == []
    copies = {}
    built = mono.SPEC.build(lm, hf, SimpleNamespace(widths=[1, 2, 4], copies=copies, deadline_s=2.0))
    try:
        pos = step.seq_lens.long() - 1
        slots = step.page_table.gather(1, (pos // 64)[:, None]).squeeze(1).long() * 64 + pos % 64
        batch = SimpleNamespace(out_cache_loc=slots)
        key = registry.ShapeKey(forward_mode="decode", batch_size=ROWS, tokens_per_request=1)
        print("[spec] forward", flush=True)
        out = built.forward(registry.Plan(key=key), None, pos, batch)
        torch.cuda.synchronize()
        built.runtime.check_errors()
        assert len(dense_calls) == 1
        # the covered layers by hand, on the same bound weights and caches
        x = workloads.rows_bf16(ROWS, 7168, dev, seed=13)
        rt = LayerRuntime(ROWS, CTX, dev)
        try:
            for i in (1, 2):
                L = built._layers[i]
                x = rt.forward(x, step.seq_lens, step.page_table, L.caches, L.w, built.cos, built.sin)
            torch.cuda.synchronize()
        finally:
            rt.close()
        print(f"  spec forward vs direct: max diff {float((out.float() - x.float()).abs().max()):.3e}", flush=True)
        assert torch.equal(out, x)
        assert built._layers[1].caches.kv_scale is None
        # a step wider than the runtime runs the model's own forward
        ran = []

        class Own:
            def forward(self, *a):
                ran.append(a)
                return "own"

        built.lm = Own()
        wide = registry.ShapeKey(forward_mode="decode", batch_size=17, tokens_per_request=1)
        assert built.forward(registry.Plan(key=wide), None, pos, batch) == "own" and len(ran) == 1
    finally:
        built.runtime.close()


class _OracleIndexer(torch.nn.Module):
    """The stand-in indexer: its forward hands on the selection (KV slots, -1 past a
    row's keys), where check mode's hook reads SGLang's selection."""

    def __init__(self, ns):
        super().__init__()
        for k, v in vars(ns).items():
            setattr(self, k, v)

    def forward(self, selection):
        return selection


class _OracleLayer:
    """SGLang's layer module stood in by the CPU oracle chain (front, cache write,
    index scores, exact top-2048, sparse MLA, back, FP8 MoE) on the same weights:
    ``(positions, hidden, batch, residual) -> (hidden, None)``, writing its cache rows
    into the layer's pools like SGLang's layer."""

    def __init__(self, i, seed, dev, rot, cos, sin):
        from test_gpu_layer import CpuExperts, _cpu_proj

        from sgl_amd_mono_amd import sglang_bind

        ns, p, m = _sglang_parts(seed, dev, rot)
        vars(self).update(vars(ns))
        self.self_attn.indexer = _OracleIndexer(self.self_attn.indexer)
        self.i, self.cos, self.sin = i, cos.cpu(), sin.cpu()
        # the projections as the spec binds them (W_UK / W_UV with SGLang's per-tensor scale)
        self.proj = _cpu_proj(sglang_bind.layer_weights(self, i, {}).proj)
        self.m = m
        self.experts = (CpuExperts(m.w13, True), CpuExperts(m.s13), CpuExperts(m.w2, True), CpuExperts(m.s2))

    def __call__(self, positions, hidden, batch, residual):
        from oracle import attention as oatt
        from oracle import layer as ol
        from oracle import moe as omoe
        from sgl_amd_mono_amd import sglang_bind
        from sgl_amd_mono_amd.moe import FP8_MOE

        dev = hidden.device
        h, pos = hidden.cpu(), positions.cpu().long()
        pt = forward_context.ATTN_BACKEND.forward_metadata.real_page_table.cpu()[:h.shape[0]]
        f = ol.front(h, pos, pt, self.proj, self.cos, self.sin, kv_scaled=False)
        c = sglang_bind.caches(forward_context.POOL, self.i)
        cpu = {k: getattr(c, k).cpu() for k in ("ikv", "iks", "kv")}
        ol.write_caches(f, cpu["ikv"], cpu["iks"], cpu["kv"], None)
        for k in cpu:
            getattr(c, k).copy_(cpu[k])
        lens = pos.to(torch.int32) + 1
        scores = oatt.index_scores(f["iq"], f["iqs"], f["iw"], cpu["ikv"], cpu["iks"], pt, lens, CTX)
        sel = self.self_attn.indexer(oatt.select_topk(scores, lens, pt))
        o = oatt.sparse_mla(f["q"].to(torch.bfloat16), cpu["kv"], None, sel)
        a = ol.back(o.to(torch.bfloat16), h, self.proj)["a"]
        m = self.m
        out = omoe.fp8_moe_block(a, m.g_post.cpu(), m.w_router.cpu(), m.bias.cpu(), *self.experts, eps=FP8_MOE.eps,
                                 top_k=FP8_MOE.top_k, inter=FP8_MOE.inter)["out"]
        return out.to(dev), None


def _sglang_parts(seed, dev, rot):
    p = workloads.proj_weights(dev, seed=seed)
    m = workloads.fp8_moe_weights(FP8_MOE, dev, seed=seed + 1)
    return _sglang_layer_of(p, m, dev, rot), p, m


def test_check_mode_against_the_oracle_layer(gpu_device, monkeypatch, caplog):
    """SGLANG_AMD_MONO_CHECK=1 with the CPU oracle chain standing in for SGLang's layer
    module: every covered layer's stream, MLA rows, index keys and selection are
    measured against it, and none violates the spec's NUMERICS bounds."""
    from sgl_amd_mono_amd import check
    from sgl_amd_mono_amd import spec as mono

    dev = gpu_device
    monkeypatch.setenv(mono.LOCAL_SHARE_ENV, "1")
    monkeypatch.setenv(check.CHECK_ENV, "1")
    caplog.set_level("INFO", logger="sgl_amd_mono_amd.check")
    cos, sin = workloads.rope_tables(CTX, dev)
    rot = SimpleNamespace(cos_sin_cache=torch.cat([cos, sin], -1))
    print("[check mode] building a 2-layer model with oracle stand-in layers", flush=True)
    layers = [_OracleLayer(0, 21, dev, rot, cos, sin), _OracleLayer(1, 22, dev, rot, cos, sin)]
    model = SimpleNamespace(embed_tokens=lambda ids: workloads.rows_bf16(ROWS, 7168, dev, seed=23), layers=layers,
                            norm=lambda h, r=None: h)
    lm = SimpleNamespace(model=model, lm_head=None, logits_processor=lambda ids, h, head, batch: h)
    hf = SimpleNamespace(first_k_dense_replace=0, num_hidden_layers=2)
    lens = [4096, 1500, 65, 3000]
    step, c0 = workloads.attn_case(lens, dev, seed=24, max_ctx=CTX)
    _, c1 = workloads.attn_case(lens, dev, seed=25, max_ctx=CTX)
    c0.kv_scale = c1.kv_scale = None
    pools = {i: (c.kv.view(-1, 1, 576), c.ikv.view(-1, 1, 4, 64, 16), c.iks.view(-1, 1, 4, 64))
             for i, c in ((0, c0), (1, c1))}
    forward_context.POOL = SimpleNamespace(get_key_buffer=lambda i: pools[i][0],
                                           get_index_k_fp4_payload_buffer=lambda i: pools[i][1],
                                           get_index_k_fp4_scale_buffer=lambda i: pools[i][2])
    forward_context.ATTN_BACKEND = SimpleNamespace(forward_metadata=SimpleNamespace(real_page_table=step.page_table))
    runtime_context.PARALLEL = SimpleNamespace(tp_size=4, tp_rank=0, tp_group=None)
    runtime_context.MODEL_CONFIG = SimpleNamespace(context_len=CTX)
    built = mono.SPEC.build(lm, hf, SimpleNamespace(widths=[4], copies={}, deadline_s=2.0))
    try:
        assert built.check_layers
        pos = step.seq_lens.long() - 1
        slots = step.page_table.gather(1, (pos // 64)[:, None]).squeeze(1).long() * 64 + pos % 64
        key = registry.ShapeKey(forward_mode="decode", batch_size=ROWS, tokens_per_request=1)
        print("[check mode] forward", flush=True)
        built.forward(registry.Plan(key=key), None, pos, SimpleNamespace(out_cache_loc=slots))
        torch.cuda.synchronize()
        built.runtime.check_errors()
    finally:
        built.runtime.close()
    info = [r.getMessage() for r in caplog.records if r.levelname == "INFO"]
    for line in info:
        print("  " + line, flush=True)
    assert len(info) == 2 and all("layer.topk_own.max_abs" in line for line in info)
    errors = [r.getMessage() for r in caplog.records if r.levelname == "ERROR"]
    assert not errors, errors
