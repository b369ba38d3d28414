"""ctypes binding of libmono_gfx950.so (the C-ABI declared in include/mono.h).

The library is built in-tree by ``sgl_amd_mono_amd.build``. There is no fallback:
if the library is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmono_gfx950.so"
ABI_VERSION = 4

MONO_OK, MONO_EINVAL, MONO_EHIP, MONO_ESTATE, MONO_ENOMEM = 0, 1, 2, 3, 4
ROUTER_SIGMOID_BIAS, ROUTER_SOFTMAX = 0, 1
WEIGHT_FP8_BLOCK128, WEIGHT_MXFP4 = 0, 1

_VP, _I32, _F32 = C.c_void_p, C.c_int32, C.c_float


class MoeConfig(C.Structure):
    _fields_ = [
        ("device", _I32), ("max_rows", _I32), ("hidden", _I32), ("n_experts", _I32),
        ("top_k", _I32), ("inter", _I32), ("weight_format", _I32), ("router", _I32),
        ("route_scale", _F32), ("eps", _F32),
    ]


class MoeFp8Args(C.Structure):
    _fields_ = [
        ("a", _VP), ("g_post", _VP), ("w_router", _VP), ("bias", _VP),
        ("w13", _VP), ("s13", _VP), ("w2", _VP), ("s2", _VP), ("out", _VP),
        ("rows", _I32), ("y", _VP), ("scores", _VP), ("topk_ids", _VP), ("topk_w", _VP),
    ]


class MoeMxfp4Args(C.Structure):
    _fields_ = [
        ("x", _VP), ("logits", _VP), ("w13", _VP), ("s13", _VP), ("w2", _VP), ("s2", _VP),
        ("out", _VP), ("rows", _I32), ("y", _VP), ("topk_ids", _VP), ("topk_w", _VP), ("timeline", _VP),
    ]


class AttnConfig(C.Structure):
    _fields_ = [("device", _I32), ("max_rows", _I32), ("max_ctx", _I32), ("softmax_scale", _F32)]


class AttnArgs(C.Structure):
    _fields_ = [
        ("iq", _VP), ("iqs", _VP), ("iw", _VP), ("ikv", _VP), ("iks", _VP), ("q", _VP), ("kv", _VP),
        ("kv_scale", _VP), ("page_table", _VP), ("seq_lens", _VP), ("pt_stride", _I32),
        ("n_pages", _I32), ("out", _VP), ("rows", _I32), ("scores", _VP), ("topk", _VP),
        ("timeline", _VP),
    ]


class ProjConfig(C.Structure):
    _fields_ = [("device", _I32), ("max_rows", _I32)]


PROJ_WEIGHT_FIELDS = (
    "g_in", "w_qkv", "s_qkv", "w_ik", "s_ik", "w_iw", "g_q", "g_kv", "g_ik", "b_ik",
    "w_qb", "s_qb", "w_iq", "s_iq", "w_uk", "s_uk", "w_uv", "s_uv", "w_o", "s_o",
)


class ProjWeights(C.Structure):
    _fields_ = [(n, _VP) for n in PROJ_WEIGHT_FIELDS]


class FrontArgs(C.Structure):
    _fields_ = [
        ("h", _VP), ("seq_lens", _VP), ("page_table", _VP), ("pt_stride", _I32), ("n_pages", _I32),
        ("rope_cos", _VP), ("rope_sin", _VP), ("max_pos", _I32),
        ("ikv", _VP), ("iks", _VP), ("kv", _VP), ("kv_scale", _VP),
        ("q", _VP), ("iq", _VP), ("iqs", _VP), ("iw", _VP), ("rows", _I32), ("timeline", _VP),
    ]


class BackArgs(C.Structure):
    _fields_ = [("o_lat", _VP), ("h", _VP), ("a", _VP), ("o", _VP), ("rows", _I32), ("timeline", _VP)]


class LayerConfig(C.Structure):
    _fields_ = [("device", _I32), ("max_rows", _I32), ("max_ctx", _I32), ("softmax_scale", _F32),
                ("route_scale", _F32), ("eps", _F32), ("max_layers", _I32)]


class LayerArgs(C.Structure):
    _fields_ = [("front", C.POINTER(FrontArgs)), ("attn", C.POINTER(AttnArgs)), ("back", C.POINTER(BackArgs)),
                ("moe", C.POINTER(MoeFp8Args)), ("ticks", _VP)]


# the phase boundaries a one-launch layer stamps per workgroup (mono_layer_args.ticks)
LAYER_TICKS = ("begin", "front", "attn", "back", "plan", "end", "a_seen", "norm", "router", "route", "quant")
LAYER_TICK_WORDS = 16


# entry point -> (restype, argtypes); every name include/mono.h declares
SIGNATURES = {
    "mono_abi_version": (C.c_int, []),
    "mono_last_error": (C.c_char_p, []),
    "mono_moe_create": (C.c_int, [C.POINTER(MoeConfig), C.POINTER(_VP)]),
    "mono_moe_destroy": (C.c_int, [_VP]),
    "mono_moe_fp8_forward": (C.c_int, [_VP, C.POINTER(MoeFp8Args), _VP]),
    "mono_moe_mxfp4_forward": (C.c_int, [_VP, C.POINTER(MoeMxfp4Args), _VP]),
    "mono_moe_set_deadline": (C.c_int, [_VP, C.c_double]),
    "mono_moe_read_errors": (C.c_int, [_VP, C.POINTER(C.c_int32)]),
    "mono_moe_clear_errors": (C.c_int, [_VP]),
    "mono_moe_set_fault": (C.c_int, [_VP, C.c_int32]),
    "mono_attn_create": (C.c_int, [C.POINTER(AttnConfig), C.POINTER(_VP)]),
    "mono_attn_destroy": (C.c_int, [_VP]),
    "mono_attn_forward": (C.c_int, [_VP, C.POINTER(AttnArgs), _VP]),
    "mono_attn_forward_noalloc": (C.c_int, [C.POINTER(AttnArgs), C.c_float, _VP]),
    "mono_attn_set_deadline": (C.c_int, [_VP, C.c_double]),
    "mono_attn_read_errors": (C.c_int, [_VP, C.POINTER(C.c_int32)]),
    "mono_attn_clear_errors": (C.c_int, [_VP]),
    "mono_attn_set_fault": (C.c_int, [_VP, C.c_int32]),
    "mono_proj_create": (C.c_int, [C.POINTER(ProjConfig), C.POINTER(_VP)]),
    "mono_proj_destroy": (C.c_int, [_VP]),
    "mono_front_forward": (C.c_int, [_VP, C.POINTER(ProjWeights), C.POINTER(FrontArgs), _VP]),
    "mono_back_forward": (C.c_int, [_VP, C.POINTER(ProjWeights), C.POINTER(BackArgs), _VP]),
    "mono_attn_back_forward": (C.c_int, [_VP, C.POINTER(AttnArgs), C.POINTER(ProjWeights), C.POINTER(BackArgs), _VP]),
    "mono_proj_set_deadline": (C.c_int, [_VP, C.c_double]),
    "mono_proj_read_errors": (C.c_int, [_VP, C.POINTER(C.c_int32)]),
    "mono_proj_clear_errors": (C.c_int, [_VP]),
    "mono_proj_set_fault": (C.c_int, [_VP, C.c_int32]),
    "mono_layer_create": (C.c_int, [C.POINTER(LayerConfig), C.POINTER(_VP)]),
    "mono_layer_destroy": (C.c_int, [_VP]),
    "mono_layer_forward": (C.c_int, [_VP, C.POINTER(ProjWeights), C.POINTER(LayerArgs), _VP]),
    "mono_layer_front_forward": (C.c_int, [_VP, C.POINTER(ProjWeights), C.POINTER(LayerArgs), _VP]),
    "mono_layer_tail_forward": (C.c_int, [_VP, C.POINTER(ProjWeights), C.POINTER(LayerArgs), _VP]),
    "mono_layer_stack_set": (C.c_int, [_VP, _I32, C.POINTER(C.POINTER(ProjWeights)),
                                       C.POINTER(C.POINTER(LayerArgs))]),
    "mono_layer_stack_forward": (C.c_int, [_VP, _VP]),
    "mono_layer_set_deadline": (C.c_int, [_VP, C.c_double]),
    "mono_layer_read_errors": (C.c_int, [_VP, C.POINTER(C.c_int32)]),
    "mono_layer_pending_error": (C.c_int32, [_VP]),
    "mono_layer_clear_errors": (C.c_int, [_VP]),
    "mono_layer_set_fault": (C.c_int, [_VP, C.c_int32, C.c_int64]),
    "mono_layer_set_launch_ordinal": (C.c_int, [_VP, C.c_uint64]),
}
GUARD_WORDS = 8
# guard words: tag epochs, error (1 + site), failing tag, failing workgroup, u64 launches begun
G_EPOCH, G_ERROR, G_FAIL_TAG, G_FAIL_BLOCK, G_TICKET = 0, 1, 2, 3, 4
# tags repeat every TAG_PERIOD launches (a launch's tag is ordinal % TAG_PERIOD + 1)
TAG_PERIOD = 2**32 - 2
SCRUB_SITE = 31
# wait sites of the launches (guard word 1 = site + 1)
MOE_SITES = {0: "router tasks", 1: "(not used)", 2: "expert mid activations", 3: "expert outputs"}
ATTN_SITES = {0: "index scores", 1: "selected slots", 2: "split partials", 3: "top-k team"}
PROJ_SITES = {0: "stage-A partial sums", 1: "stage-A q_a tiles", 2: "q_nope", 3: "raw index query", 4: "W_UV output"}
# every launch of a layer runtime (one guard)
LAYER_SITES = {**ATTN_SITES, 4: "W_UV output", 5: "attention output", 6: "router tasks", 7: "(not used)",
               8: "expert mid activations", 9: "expert outputs", 10: "attention block output rows",
               **{11 + k: f"front: {v}" for k, v in {**PROJ_SITES, 5: "normed input rows"}.items()},
               17: "front index query and keys", 18: "front q",
               19: "the layer before's output rows (multi-layer launch)", SCRUB_SITE: "tag-epoch scrub"}
# the front's own sites in a layer runtime's numbering
LAYER_FRONT_SITE0 = 11

_lock = threading.Lock()
_lib = None


class MonoError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[mono error {code}] {msg}")
        self.code = code


def lib() -> C.CDLL:
    """The loaded library (loads on first use; raises if it is not built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built: run `python -m sgl_amd_mono_amd.build` "
                    "(the HIP path has no CPU fallback)"
                )
            h = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype, fn.argtypes = res, args
            got = h.mono_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH}: ABI version {got}, this binding expects {ABI_VERSION}")
            _lib = h
        return _lib


def check(rc: int) -> None:
    if rc != MONO_OK:
        msg = lib().mono_last_error().decode(errors="replace")
        if rc == MONO_EINVAL:
            raise ValueError(msg)
        raise MonoError(rc, msg)


def ptr(t) -> int | None:
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()
