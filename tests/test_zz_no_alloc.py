"""The attention entry point that allocates nothing (mono_attn_forward_noalloc, its
mailboxes in the library's static per-GPU scratch) against mono_attn_forward on a
runtime of the same limits (8 rows, 32768 keys): bit for bit on the output, the index
scores and the selected slots, call after call with the input shrinking, and the
limits refused with errors that name them."""

import ctypes as C

import pytest
import torch

from sgl_amd_mono_amd import _lib, workloads
from sgl_amd_mono_amd.attn import SOFTMAX_SCALE, AttnRuntime, attn_args

pytestmark = pytest.mark.gpu

CTX = 32768


def _noalloc():
    return _lib.lib().mono_attn_forward_noalloc


def _call(fn, step, caches, dev):
    args, out, dbg = attn_args(dev, 8, CTX, step, caches, None, True, None)
    _lib.check(fn(C.byref(args), SOFTMAX_SCALE, torch.cuda.current_stream(dev).cuda_stream))
    return out, dbg


def test_noalloc_attention_equals_the_runtime(gpu_device):
    fn = _noalloc()
    rt = AttnRuntime(8, CTX, device=gpu_device)
    cases = [
        ([CTX, 9000, 2049, 300, CTX - 5, 2048, 16000, 64], True, 301),  # 8 rows, per-token scales
        ([5000, 1025, 2047], True, 303),                                  # 3 shorter rows
        ([700, 20000], False, 305),                                       # 2 rows, raw E4M3 rows
    ]
    try:
        for lens, scaled, seed in cases:
            print(f"[no-alloc] rows {len(lens)} lens {lens} scaled {scaled}", flush=True)
            step, caches = workloads.attn_case(lens, gpu_device, seed=seed, max_ctx=CTX)
            if not scaled:
                caches.kv_scale = None
            got, gdbg = _call(fn, step, caches, gpu_device)
            want, wdbg = rt.forward(step, caches, debug=True)
            torch.cuda.synchronize()
            rt.check_errors()
            assert not bool(got.isnan().any()), "the no-alloc launch failed a wait"
            assert torch.equal(got, want), float((got.float() - want.float()).abs().max())
            assert torch.equal(gdbg["topk"], wdbg["topk"])
            assert torch.equal(gdbg["scores"], wdbg["scores"])
    finally:
        rt.close()


def test_noalloc_attention_refuses_past_its_limits(gpu_device):
    fn = _noalloc()
    step, caches = workloads.attn_case([100] * 9, gpu_device, seed=307, max_ctx=CTX)
    args, _, _ = attn_args(gpu_device, 9, CTX, step, caches, None, False, None)
    stream = torch.cuda.current_stream(gpu_device).cuda_stream
    with pytest.raises(ValueError, match=r"rows must be in \[1, 8\]"):
        _lib.check(fn(C.byref(args), SOFTMAX_SCALE, stream))
    args.rows = 8
    args.pt_stride = 100
    with pytest.raises(ValueError, match="pt_stride must cover"):
        _lib.check(fn(C.byref(args), SOFTMAX_SCALE, stream))
    args.pt_stride = CTX // 64
    with pytest.raises(ValueError, match="softmax_scale"):
        _lib.check(fn(C.byref(args), -1.0, stream))
    args.q = None
    with pytest.raises(ValueError, match="args->q"):
        _lib.check(fn(C.byref(args), SOFTMAX_SCALE, stream))
