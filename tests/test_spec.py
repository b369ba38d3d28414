"""The SGLang plugin surface on CPU (sgl_amd_mono_amd.spec, sglang_bind) against a
stand-in registry (tests/fake_sglang: SGLang is not installed in this image): the
entry point's registration and lookup by architecture and ISA, the config and model
refusal reasons, routing by graph key (a step wider than the runtime runs the model's
own forward), the step table built on the device, the backbone around the covered
layers, and in-place binding of SGLang-shaped weights and caches with errors that name
the tensor (the reference's test design: test/unit/test_glm53_spec.py)."""

import os
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "fake_sglang"))

from sglang.kernels.plugin_kernels.amd import spec as registry  # noqa: E402
from sglang.srt.model_executor import forward_context  # noqa: E402

import sgl_amd_mono_amd  # noqa: E402
from oracle import codecs as ocodecs  # noqa: E402
from sgl_amd_mono_amd import sglang_bind  # noqa: E402
from sgl_amd_mono_amd import spec as mono  # noqa: E402

# DeepSeek-V3.2's layer structure with the ungrouped router the kernels run
DSV32 = SimpleNamespace(
    **mono.HF_CONFIG,
    model_type="deepseek_v32",
    num_hidden_layers=61,
    first_k_dense_replace=3,
    moe_layer_freq=1,
    quantization_config={"quant_method": "fp8", "weight_block_size": [128, 128]},
    rope_scaling=None,
    architectures=["DeepseekV32ForCausalLM"],
)
CFG = SimpleNamespace(page_size=64, speculative_algorithm=None, context_length=32768)


@pytest.fixture
def local_share(monkeypatch):
    monkeypatch.setenv(mono.LOCAL_SHARE_ENV, "1")


def test_the_forward_covers_the_moe_layers():
    assert mono.covered_layers(DSV32) == list(range(3, 61))


def test_the_plugin_registers_the_spec():
    sgl_amd_mono_amd.register_specs()
    arch = ["DeepseekV32ForCausalLM"]
    found, why = registry.find_spec(backend=sgl_amd_mono_amd.BACKEND, architectures=arch, isa="gfx950",
                                    model_type="deepseek_v32")
    assert found is mono.SPEC, why
    assert mono.SPEC.devices["gfx950"].tp_sizes == (4,)
    assert mono.SPEC.devices["gfx950"].widths == tuple(range(1, 17))
    found, why = registry.find_spec(backend="amd", architectures=arch, isa="gfx942", model_type="deepseek_v32")
    assert found is None and "gfx942" in why


def test_config_refusals(local_share):
    assert mono.config_disable_reasons(CFG, DSV32) == []
    grouped = SimpleNamespace(**{**vars(DSV32), "n_group": 8, "topk_group": 4})
    why = mono.config_disable_reasons(CFG, grouped)
    assert any("n_group = 1" in r for r in why) and any("topk_group = 1" in r for r in why)
    bf16 = SimpleNamespace(**{**vars(DSV32), "quantization_config": None})
    assert any("FP8 block-128" in r for r in mono.config_disable_reasons(CFG, bf16))
    yarn = SimpleNamespace(**{**vars(DSV32), "rope_scaling": {"type": "yarn", "factor": 40}})
    assert any("yarn" in r for r in mono.config_disable_reasons(CFG, yarn))
    pages = SimpleNamespace(**{**vars(CFG), "page_size": 32})
    assert any("--page-size 32" in r for r in mono.config_disable_reasons(pages, DSV32))
    mtp = SimpleNamespace(**{**vars(CFG), "speculative_algorithm": "EAGLE", "speculative_eagle_topk": 2,
                             "speculative_num_steps": 3, "speculative_num_draft_tokens": 4})
    assert any("one causal chain" in r for r in mono.config_disable_reasons(mtp, DSV32))
    chain = SimpleNamespace(**{**vars(mtp), "speculative_eagle_topk": 1})
    assert mono.config_disable_reasons(chain, DSV32) == []
    long = SimpleNamespace(**{**vars(CFG), "context_length": 163840})
    assert any("32768 keys" in r for r in mono.config_disable_reasons(long, DSV32))


def test_refuses_without_the_local_share_flag(monkeypatch):
    monkeypatch.delenv(mono.LOCAL_SHARE_ENV, raising=False)
    why = mono.config_disable_reasons(CFG, DSV32)
    assert len(why) == 1 and mono.LOCAL_SHARE_ENV in why[0]


class _Lm:
    """A model whose own forward records that it ran."""

    def __init__(self, model=None):
        self.model, self.ran = model or SimpleNamespace(), []

    def forward(self, *args):
        self.ran.append(args)
        return "the model's forward"


def test_a_wider_step_runs_the_model_forward():
    lm = _Lm()
    built = mono._Built(lm, {3: None}, None, None, None, "cpu", context_len=32768)
    key = registry.ShapeKey(forward_mode="decode", batch_size=17, tokens_per_request=1)
    assert built.forward(registry.Plan(key=key), "ids", "positions", "batch") == "the model's forward"
    assert lm.ran == [("ids", "positions", "batch", None, None)]


def test_step_table_rows_keys_and_pad_rows():
    built = mono._Built(_Lm(), {3: None}, None, None, None, "cpu", context_len=4096)
    table = torch.arange(4 * 64, dtype=torch.int32).reshape(4, 64)
    forward_context.ATTN_BACKEND = SimpleNamespace(forward_metadata=SimpleNamespace(real_page_table=table))
    key = registry.ShapeKey(forward_mode="target_verify", batch_size=1, tokens_per_request=4)
    plan = registry.Plan(key=key)
    batch = SimpleNamespace(out_cache_loc=torch.tensor([700, 701, 0, 9000]))
    st = built._step(plan, torch.tensor([60, 61, 62, 5000]), batch, 4)
    # a row at position p sees keys 0 ..= p; the padding slot 0 marks a pad row; positions
    # past the context clamp to its last one
    assert st.seq_lens.tolist()[:4] == [61, 62, 0, 4096]
    assert torch.equal(st.page_table, table[:4])
    # built once a step: the second layer reuses it
    assert built._step(plan, torch.tensor([0, 0, 0, 0]), batch, 4) is st
    assert st.seq_lens.tolist()[:4] == [61, 62, 0, 4096]


class _Runtime:
    """Records each covered layer's launch; returns h + 1 as the layer's output.
    ``pending`` stands for the pinned host word a stopped launch sets."""

    max_rows = 16

    def __init__(self, pending: int = 0):
        self.calls, self.pending = [], pending

    def raise_pending(self):
        if self.pending:
            from sgl_amd_mono_amd import _lib

            raise _lib.MonoError(_lib.MONO_ESTATE, f"a layer launch stopped at wait {self.pending - 1}")

    def forward(self, h, seq_lens, page_table, caches, w, cos, sin, check_weights=True):
        self.calls.append((h.clone(), seq_lens.clone(), caches, w))
        return h + 1


def test_backbone_runs_dense_layers_then_launches():
    S, Hd = 2, 7168
    dense_calls = []

    def dense(i):
        def f(positions, hidden, batch, residual):
            dense_calls.append(i)
            return hidden * 2, (hidden if residual is None else residual + hidden)
        return f

    layers = [dense(0), dense(1), dense(2), "L3", "L4"]
    model = SimpleNamespace(embed_tokens=lambda ids: torch.ones(S, Hd), layers=layers,
                            norm=lambda h, r=None: (h + r, None) if r is not None else h * 10)
    lm = _Lm(model)
    lm.logits_processor = lambda ids, hidden, head, batch: ("logits", hidden)
    lm.lm_head = None
    rt = _Runtime()
    covered = {i: mono._Layer(i, None, f"w{i}") for i in (3, 4)}
    built = mono._Built(lm, covered, rt, None, None, "cpu", context_len=4096)
    kv = torch.zeros(64, 1, 576, dtype=torch.uint8)
    pool = SimpleNamespace(get_key_buffer=lambda i: kv,
                           get_index_k_fp4_payload_buffer=lambda i: torch.zeros(1, 1, 4, 64, 16, dtype=torch.uint8),
                           get_index_k_fp4_scale_buffer=lambda i: torch.zeros(1, 1, 4, 64, dtype=torch.uint8))
    forward_context.POOL = pool
    forward_context.ATTN_BACKEND = SimpleNamespace(
        forward_metadata=SimpleNamespace(real_page_table=torch.zeros(S, 64, dtype=torch.int32)))
    key = registry.ShapeKey(forward_mode="decode", batch_size=S, tokens_per_request=1)
    batch = SimpleNamespace(out_cache_loc=torch.tensor([5, 6]))
    out = built.forward(registry.Plan(key=key), "ids", torch.tensor([4, 5]), batch)
    assert dense_calls == [0, 1, 2]
    # hidden after the dense layers: 8 (1 doubled three times), residual 1 + 2 + 4 = 7:
    # the first launch takes the whole stream 15, the second 16; the final norm x 10
    assert [float(c[0][0, 0]) for c in rt.calls] == [15.0, 16.0]
    assert [c[3] for c in rt.calls] == ["w3", "w4"]
    assert rt.calls[0][1].tolist() == [5, 6]
    assert out[0] == "logits" and float(out[1][0, 0]) == 170.0
    # each layer bound its caches once, scale-less E4M3 rows
    assert covered[3].caches.kv_scale is None and covered[3].caches.kv.shape == (64, 576)


def test_a_stopped_launch_raises_instead_of_serving():
    """A launch that failed a wait (or was refused after one) sets the runtime's pinned
    host word; the next eager forward raises before anything runs. (The step whose
    launch failed, and steps replayed from a graph, are the fail-stop watcher's: it
    ends the process, see test_fail_stop_watch_*.)"""
    from sgl_amd_mono_amd import _lib

    lm = _Lm(SimpleNamespace(embed_tokens=lambda ids: torch.ones(1, 7168), layers=[], norm=lambda h: h))
    rt = _Runtime(pending=9)  # expert outputs
    built = mono._Built(lm, {3: None}, rt, None, None, "cpu", context_len=4096)
    key = registry.ShapeKey(forward_mode="decode", batch_size=1, tokens_per_request=1)
    with pytest.raises(_lib.MonoError, match="stopped at wait 8"):
        built.forward(registry.Plan(key=key), "ids", torch.tensor([3]), SimpleNamespace())
    assert rt.calls == [] and lm.ran == []
    # a step wider than the runtime raises as well: the model's forward would run the
    # dense layers on the same GPU whose launch stopped
    key = registry.ShapeKey(forward_mode="decode", batch_size=17, tokens_per_request=1)
    with pytest.raises(_lib.MonoError):
        built.forward(registry.Plan(key=key), "ids", "positions", "batch")


def test_deadline_follows_the_watchdog():
    """The framework's deadline when it gives one, else half the watchdog at most 60 s
    (common/guard.py:4-6), else 60 s."""
    assert mono.deadline_seconds(SimpleNamespace(deadline_s=12.5)) == 12.5
    assert mono.deadline_seconds(SimpleNamespace(watchdog_timeout=30)) == 15.0
    assert mono.deadline_seconds(SimpleNamespace(watchdog_timeout=300)) == 60.0
    assert mono.deadline_seconds(SimpleNamespace()) == 60.0


def test_fault_injection_env(monkeypatch):
    """SGLANG_AMD_MONO_FAULT_INJECT=rank:site[:after], the reference's format."""
    monkeypatch.delenv(mono.FAULT_INJECT_ENV, raising=False)
    assert mono.fault_injection(0) is None
    monkeypatch.setenv(mono.FAULT_INJECT_ENV, "1:8:40")
    assert mono.fault_injection(1) == (8, 40) and mono.fault_injection(0) is None
    monkeypatch.setenv(mono.FAULT_INJECT_ENV, "0:17")
    assert mono.fault_injection(0) == (17, 0)
    monkeypatch.setenv(mono.FAULT_INJECT_ENV, "0:x")
    with pytest.raises(ValueError, match="rank:site"):
        mono.fault_injection(0)


# ---- binding SGLang-shaped tensors in place ----

def _fp8_linear(rows, cols, shuffled=True):
    lin = SimpleNamespace(weight=torch.empty(rows, cols, dtype=torch.float8_e4m3fn),
                          weight_scale_inv=torch.rand(-(-rows // 128), -(-cols // 128)))
    lin.aiter_bpreshuffled = shuffled
    return lin


def _sglang_layer(shuffled=True, fused_shared=True):
    bf = torch.bfloat16
    H = 7168
    g = torch.Generator().manual_seed(0)
    ind = SimpleNamespace(wk=_fp8_linear(128, H, shuffled), wq_b=_fp8_linear(64 * 128, 1536, shuffled),
                          weights_proj=SimpleNamespace(weight=torch.randn(64, H, generator=g).to(bf)),
                          k_norm=SimpleNamespace(weight=torch.ones(128, dtype=bf), bias=torch.zeros(128, dtype=bf)))
    codes = lambda *s: torch.randint(0, 120, s, generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)  # noqa
    attn = SimpleNamespace(
        fused_qkv_a_proj_with_mqa=_fp8_linear(1536 + 512 + 64, H, shuffled), q_b_proj=_fp8_linear(32 * 192, 1536, shuffled),
        o_proj=_fp8_linear(H, 32 * 128, shuffled), w_kc=codes(32, 128, 512), w_vc=codes(32, 512, 128),
        w_scale=torch.tensor(0.03), indexer=ind, q_a_layernorm=SimpleNamespace(weight=torch.ones(1536, dtype=bf)),
        kv_a_layernorm=SimpleNamespace(weight=torch.ones(512, dtype=bf)),
    )  # fmt: skip
    E1 = 257 if fused_shared else 256
    experts = SimpleNamespace(w13_weight=torch.empty(E1, 1024, H, dtype=torch.float8_e4m3fn),
                              w13_weight_scale_inv=torch.empty(E1, 8, 56), w2_weight=torch.empty(E1, H, 512, dtype=torch.float8_e4m3fn),
                              w2_weight_scale_inv=torch.empty(E1, 56, 4), is_shuffled=True)
    gate = SimpleNamespace(weight=torch.empty(256, H, dtype=bf), e_score_correction_bias=torch.zeros(256))
    return SimpleNamespace(self_attn=attn, mlp=SimpleNamespace(experts=experts, gate=gate),
                           input_layernorm=SimpleNamespace(weight=torch.ones(H, dtype=bf)),
                           post_attention_layernorm=SimpleNamespace(weight=torch.ones(H, dtype=bf)))


def test_weights_bind_in_place_and_pack_the_copies():
    layer = _sglang_layer()
    copies = {}
    w = sglang_bind.layer_weights(layer, 3, copies)
    attn, ex = layer.self_attn, layer.mlp.experts
    # in place: the same storage, viewed as bytes
    assert w.proj.w_qkv.data_ptr() == attn.fused_qkv_a_proj_with_mqa.weight.data_ptr()
    assert w.proj.w_o.data_ptr() == attn.o_proj.weight.data_ptr()
    assert w.proj.s_qb.data_ptr() == attn.q_b_proj.weight_scale_inv.data_ptr()
    assert w.moe.w13.data_ptr() == ex.w13_weight.data_ptr() and w.moe.w13.dtype == torch.uint8
    assert w.moe.w_router.data_ptr() == layer.mlp.gate.weight.data_ptr()
    # the copies: W_UK[(h, c), d] = w_kc[h, d, c] and W_UV[(h, v), c] = w_vc[h, c, v] in the
    # (16, 16) layout, their scale planes the per-tensor scale
    uk = ocodecs.aiter_unshuffle(w.proj.w_uk).reshape(32, 512, 128)
    assert torch.equal(uk[5, 17], attn.w_kc[5, :, 17].view(torch.uint8))
    uv = ocodecs.aiter_unshuffle(w.proj.w_uv).reshape(32, 128, 512)
    assert torch.equal(uv[31, 100], attn.w_vc[31, :, 100].view(torch.uint8))
    assert w.proj.s_uk.shape == (128, 1) and bool((w.proj.s_uk == 0.03).all())
    assert w.proj.s_uv.shape == (32, 4) and bool((w.proj.s_uv == 0.03).all())
    iw = ocodecs.aiter_unshuffle(w.proj.w_iw.view(torch.uint8)).view(torch.bfloat16)
    assert torch.equal(iw, attn.indexer.weights_proj.weight)
    assert w.proj.g_ik.dtype == torch.float32
    assert {k[1] for k in copies} == {"w_uk", "s_uk", "w_uv", "s_uv", "w_iw", "g_ik", "b_ik"}


def test_binding_errors_name_the_tensor():
    layer = _sglang_layer()
    layer.self_attn.o_proj.weight_scale_inv = torch.rand(56, 16)
    with pytest.raises(sglang_bind.BindError, match=r"layer 7: needs o_proj.weight_scale_inv .*\(56, 32\)"):
        sglang_bind.layer_weights(layer, 7, {})
    with pytest.raises(sglang_bind.BindError, match="shared expert fused"):
        sglang_bind.layer_weights(_sglang_layer(fused_shared=False), 3, {})
    with pytest.raises(sglang_bind.BindError, match=r"fused_qkv_a_proj_with_mqa in AITER.s \(16, 16\)"):
        sglang_bind.layer_weights(_sglang_layer(shuffled=False), 3, {})


def test_model_refusals_list_row_major_projections():
    model = SimpleNamespace(model=SimpleNamespace(layers=[None] * 3 + [_sglang_layer(shuffled=False)] * 58))
    why = mono.model_disable_reasons(model, DSV32, {})
    assert any(r.startswith("fused_qkv_a_proj_with_mqa of 58 layers from 3") for r in why)
    ok = SimpleNamespace(model=SimpleNamespace(layers=[None] * 3 + [_sglang_layer()] * 58))
    assert mono.model_disable_reasons(ok, DSV32, {}) == []


def test_caches_bind_sglang_pools_in_place():
    kv = torch.zeros(128, 1, 576, dtype=torch.float8_e4m3fn)
    pay = torch.zeros(2, 1, 4, 64, 16, dtype=torch.uint8)
    sc = torch.zeros(2, 1, 4, 64, dtype=torch.uint8)
    pool = SimpleNamespace(get_key_buffer=lambda i: kv, get_index_k_fp4_payload_buffer=lambda i: pay,
                           get_index_k_fp4_scale_buffer=lambda i: sc)
    c = sglang_bind.caches(pool, 4)
    assert c.kv.data_ptr() == kv.data_ptr() and c.kv.shape == (128, 576) and c.kv_scale is None
    assert c.ikv.data_ptr() == pay.data_ptr() and c.ikv.shape == (2, 4, 64, 16)
    assert c.iks.shape == (2, 4, 64)
    bad = SimpleNamespace(get_key_buffer=lambda i: torch.zeros(128, 1, 656, dtype=torch.uint8),
                          get_index_k_fp4_payload_buffer=lambda i: pay, get_index_k_fp4_scale_buffer=lambda i: sc)
    with pytest.raises(sglang_bind.BindError, match="layer 4: MLA cache"):
        sglang_bind.caches(bad, 4)


def test_rope_tables_from_the_rotary_cache():
    cache = torch.randn(4096, 64)
    rot = SimpleNamespace(cos_sin_cache=cache)
    layer = SimpleNamespace(self_attn=SimpleNamespace(rotary_emb=rot, indexer=SimpleNamespace(rotary_emb=rot)))
    cos, sin = sglang_bind.rope_tables([layer, layer], {})
    assert torch.equal(cos, cache[:, :32]) and torch.equal(sin, cache[:, 32:]) and cos.is_contiguous()
    other = SimpleNamespace(cos_sin_cache=torch.randn(4096, 64))
    bad = SimpleNamespace(self_attn=SimpleNamespace(rotary_emb=rot, indexer=SimpleNamespace(rotary_emb=other)))
    with pytest.raises(sglang_bind.BindError, match="rotary"):
        sglang_bind.rope_tables([layer, bad], {})


# ---- check mode (SGLANG_AMD_MONO_CHECK=1) ----

class _CheckModule:
    """SGLang's layer as check mode calls it: ``(positions, hidden, batch, residual)``
    -> ``(hidden, residual)``; it writes ``rows`` into the caches at the step's slots
    and records the cache rows it saw."""

    def __init__(self, caches_of, rows):
        self.caches_of, self.rows, self.saw = caches_of, rows, []

    def __call__(self, positions, hidden, batch, residual):
        c, slots = self.caches_of(), batch.out_cache_loc.long()
        self.saw.append(c.kv[slots].clone())
        c.kv[slots] = self.rows["kv"]
        c.ikv[slots // 64, :, slots % 64] = self.rows["ikv"]
        return hidden * 2, hidden


class _CheckRuntime(_Runtime):
    """A launch that writes ``rows`` and returns 3 h (+ ``bump``) with the given
    index scores and selection as its kept intermediates."""

    def __init__(self, caches_of, rows, scores, selection, bump=0.0):
        super().__init__()
        self.caches_of, self.rows, self.scores, self.sel, self.bump = caches_of, rows, scores, selection, bump
        self.saw = []

    def forward(self, h, seq_lens, page_table, caches, w, cos, sin, check_weights=True, keep=False):
        assert keep
        self.saw.append(caches.kv[self.rows["slots"]].clone())
        caches.kv[self.rows["slots"]] = self.rows["kv"]
        caches.ikv[self.rows["slots"] // 64, :, self.rows["slots"] % 64] = self.rows["ikv"]
        return h * 3 + self.bump, dict(index_scores=self.scores, topk_slots=self.sel)


def _check_case(monkeypatch, bump=0.0, kv_delta=0, swap_selected=False):
    """Two rows at positions 2999 and 99 of two requests over 50 pages each; scores
    fall with position, so a row's exact top-2048 is its first 2048 positions."""
    from sgl_amd_mono_amd import check

    monkeypatch.setenv(check.CHECK_ENV, "1")
    S, pages, ctx = 2, 100, 3200
    g = torch.Generator().manual_seed(3)
    kv = torch.randint(0, 120, (pages * 64, 1, 576), generator=g, dtype=torch.uint8)
    pay = torch.randint(0, 256, (pages, 1, 4, 64, 16), generator=g, dtype=torch.uint8)
    sc = torch.randint(120, 130, (pages, 1, 4, 64), generator=g, dtype=torch.uint8)
    pool = SimpleNamespace(get_key_buffer=lambda i: kv, get_index_k_fp4_payload_buffer=lambda i: pay,
                           get_index_k_fp4_scale_buffer=lambda i: sc)
    forward_context.POOL = pool
    table = torch.cat([torch.arange(50, 100), torch.arange(0, 50)]).to(torch.int32).reshape(2, 50)
    forward_context.ATTN_BACKEND = SimpleNamespace(forward_metadata=SimpleNamespace(real_page_table=table))
    pos = torch.tensor([2999, 99])
    slots = table[torch.arange(2), pos // 64].long() * 64 + pos % 64
    rows = dict(slots=slots, kv=torch.randint(0, 120, (2, 576), generator=g, dtype=torch.uint8),
                ikv=torch.randint(0, 256, (2, 4, 16), generator=g, dtype=torch.uint8))
    launch_rows = dict(rows, kv=rows["kv"] + kv_delta)
    scores = -torch.arange(ctx, dtype=torch.float32).repeat(S, 1)
    first = torch.arange(2048)
    sel = torch.full((S, 2048), -1, dtype=torch.int32)
    sel[0] = (table[0, first // 64].long() * 64 + first % 64).to(torch.int32)
    sel[1, :100] = (table[1, first[:100] // 64].long() * 64 + first[:100] % 64).to(torch.int32)
    if swap_selected:
        sel[0, 5] = int(table[0, 2100 // 64]) * 64 + 2100 % 64
    layer = mono._Layer(0, None, "w0")  # one covered layer, no dense ones
    bound = lambda: layer.caches  # noqa: E731
    layer.module = _CheckModule(bound, rows)
    rt = _CheckRuntime(bound, launch_rows, scores, sel, bump)
    model = SimpleNamespace(embed_tokens=lambda ids: torch.ones(S, 7168), layers=["L0"], norm=lambda h: h)
    lm = _Lm(model)
    lm.logits_processor = lambda ids, hidden, head, batch: hidden
    lm.lm_head = None
    built = mono._Built(lm, {0: layer}, rt, None, None, "cpu", context_len=ctx)
    before = kv.view(-1, 576)[slots].clone()
    key = registry.ShapeKey(forward_mode="decode", batch_size=S, tokens_per_request=1)
    out = built.forward(registry.Plan(key=key), "ids", pos, SimpleNamespace(out_cache_loc=slots))
    return out, before, layer.module, rt, kv.view(-1, 576)[slots].clone(), launch_rows


def test_check_mode_measures_the_launch_against_sglangs_layer(monkeypatch, caplog):
    """SGLang's module runs first on the caches as they were, its rows are restored, the
    launch writes its own; every metric is logged and none is violated."""
    caplog.set_level("INFO", logger="sgl_amd_mono_amd.check")
    out, before, module, rt, after, launch_rows = _check_case(monkeypatch)
    assert torch.equal(module.saw[0], before) and torch.equal(rt.saw[0], before)
    assert torch.equal(after, launch_rows["kv"]) and float(out[0, 0]) == 3.0
    info = [r.getMessage() for r in caplog.records if r.levelname == "INFO"]
    assert len(info) == 1 and "layer.streams.cosine=1" in info[0] and "layer.topk_exact.max_abs=0" in info[0]
    assert "layer.kv.cosine=1" in info[0] and "layer.index.cosine=1" in info[0]
    assert not [r for r in caplog.records if r.levelname == "ERROR"]


@pytest.mark.parametrize("plant, metric", [
    (dict(bump=0.5), "layer.streams.rel"),
    (dict(kv_delta=9), "layer.kv.cosine"),
    (dict(swap_selected=True), "layer.topk_exact.max_abs"),
])
def test_check_mode_reports_violations(monkeypatch, caplog, plant, metric):
    """A planted difference (the stream shifted, other MLA rows written, one key of the
    exact top-2048 swapped for a lower one) is logged as that metric's violation."""
    caplog.set_level("INFO", logger="sgl_amd_mono_amd.check")
    _check_case(monkeypatch, **plant)
    errors = [r.getMessage() for r in caplog.records if r.levelname == "ERROR"]
    assert any(metric in e for e in errors), errors


def test_check_mode_is_off_by_default(monkeypatch):
    from sgl_amd_mono_amd import check

    monkeypatch.delenv(check.CHECK_ENV, raising=False)
    built = mono._Built(_Lm(), {3: None}, None, None, None, "cpu", context_len=4096)
    assert built.check_layers is False


def test_fail_stop_watch_reports_once_and_stops():
    """The watcher polls the pinned word without touching the GPU and calls on_fail
    once with the first non-zero code; stop() ends it and is idempotent."""
    import threading
    import time

    from sgl_amd_mono_amd.layer import FailStopWatch

    words = iter([0, 0, 0, 12, 12, 12])
    last = [0]

    def pending():
        last[0] = next(words, last[0])
        return last[0]

    hit = threading.Event()
    seen = []
    w = FailStopWatch(pending, on_fail=lambda c: (seen.append(c), hit.set()), interval=1e-3)
    assert hit.wait(5.0)
    time.sleep(0.02)
    assert seen == [12] and w.code == 12
    w.stop()
    w.stop()
    # a quiet word never calls on_fail, and stop() ends the thread
    quiet = FailStopWatch(lambda: 0, on_fail=seen.append, interval=1e-3)
    time.sleep(0.02)
    quiet.stop()
    assert seen == [12] and not quiet._thread.is_alive()


def test_fail_stop_watch_default_ends_the_process():
    """The default on_fail logs the wait site and ends the process with exit status
    FAIL_STOP_EXIT, as the reference's null-page store ends it (common/guard.py:91-97)."""
    import subprocess
    import sys

    from sgl_amd_mono_amd.layer import FAIL_STOP_EXIT

    code = (
        "import time\n"
        "from sgl_amd_mono_amd.layer import FailStopWatch\n"
        "FailStopWatch(lambda: 10, interval=1e-3)\n"
        "time.sleep(30)\n"
        "print('served')\n"
    )
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120,
                       cwd=str(__import__("pathlib").Path(__file__).resolve().parent.parent))
    assert r.returncode == FAIL_STOP_EXIT, (r.returncode, r.stderr[-2000:])
    assert "served" not in r.stdout
    assert "expert outputs" in r.stderr


def test_check_mode_routes_sglangs_moe_as_the_launch():
    """In check mode SGLang's MoE routes by the launch's f32 rule: the hook on its
    ``topk`` submodule replaces the routed columns by the 8 largest f32 sigmoid + bias
    (weights their scores over their sum x 2.5) and keeps the fused shared expert's
    column. A bias that bf16 cannot tell apart from its neighbour decides the pick."""
    from collections import namedtuple

    from sgl_amd_mono_amd import check

    TopK = namedtuple("TopK", "topk_weights topk_ids router_logits")
    g = torch.Generator().manual_seed(4)
    S, H, E = 3, 64, 32
    gate = torch.nn.Linear(H, E, bias=False)
    gate.weight.data = torch.randn(E, H, generator=g) * 0.1
    gate.weight.data[6] = gate.weight.data[5]  # equal scores: the bias alone orders 5 and 6
    gate.e_score_correction_bias = torch.zeros(E)
    gate.e_score_correction_bias[5] = 34.0 + 1 / 64  # bf16(34 + 1/64) == 34
    gate.e_score_correction_bias[6] = 34.0

    class SglangTopK(torch.nn.Module):  # bf16 bias, fused shared expert appended
        def forward(self, hidden_states, router_logits):
            s = router_logits.float().sigmoid()
            ids = (s.bfloat16() + gate.e_score_correction_bias.bfloat16()).float().topk(8, -1).indices
            w = torch.full((hidden_states.shape[0], 9), 0.1)
            ids = torch.cat([ids, torch.full((hidden_states.shape[0], 1), check.SHARED_EXPERT)], 1)
            return TopK(w, ids.int(), router_logits)

    mlp = torch.nn.Module()
    mlp.gate, mlp.topk = gate, SglangTopK()
    x = torch.randn(S, H, generator=g)
    with check._RouteAsTheLaunch(mlp, 8, 2.5):
        out = mlp.topk(x, gate(x))
    plain = mlp.topk(x, gate(x))  # the hook is gone afterwards
    ids, w = check.launch_routing(x, gate.weight, gate.e_score_correction_bias, 8, 2.5)
    assert torch.equal(out.topk_ids[:, :8].long(), ids) and bool((out.topk_ids[:, 8] == check.SHARED_EXPERT).all())
    assert torch.allclose(out.topk_weights[:, :8], w) and torch.allclose(out.topk_weights[:, :8].sum(-1), torch.full((S,), 2.5))
    assert bool((out.topk_weights[:, 8] == 0.1).all())
    # the f32 rule ranks expert 5 (bias 34 + 1/64) above 6; rows differ from SGLang's bf16 order
    assert bool((ids[:, 0] == 5).all()) and bool((ids[:, 1] == 6).all())
    assert not torch.equal(plain.topk_ids[:, :8].long(), ids)
    # scores by hand in float64
    sc = torch.sigmoid(x.double() @ gate.weight.double().t())
    pick = sc.gather(1, ids)
    assert torch.allclose(w.double(), pick / pick.sum(-1, keepdim=True) * 2.5, atol=1e-6)
