"""The C-ABI library loads on the CPU and exports every entry point include/mono.h
declares (no compute call: there is no GPU here)."""

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mono.h"


def declared_entry_points():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mono_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_entry_points()
    assert "mono_moe_fp8_forward" in names and "mono_last_error" in names


def test_library_exports_every_declared_symbol():
    from sgl_amd_mono_amd import _lib

    assert _lib.LIB_PATH.exists(), "build the library first (python -m sgl_amd_mono_amd.build)"
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_entry_points() if not hasattr(raw, n)]
    assert not missing, f"declared in mono.h but not exported: {missing}"
    # the Python binding covers the same set
    assert set(_lib.SIGNATURES) == set(declared_entry_points())


def test_abi_version_and_error_string():
    from sgl_amd_mono_amd import _lib

    h = _lib.lib()
    assert h.mono_abi_version() == _lib.ABI_VERSION
    assert isinstance(h.mono_last_error(), bytes)


def test_create_rejects_bad_config_without_touching_the_gpu():
    """Argument checks run before any HIP call, so they are testable on the CPU."""
    import pytest

    from sgl_amd_mono_amd import _lib

    cfg = _lib.MoeConfig(device=0, max_rows=99, hidden=7168, n_experts=256, top_k=8, inter=512,
                         weight_format=0, router=0, route_scale=2.5, eps=1e-6)
    h = ctypes.c_void_p()
    with pytest.raises(ValueError, match="max_rows"):
        _lib.check(_lib.lib().mono_moe_create(ctypes.byref(cfg), ctypes.byref(h)))
    cfg.max_rows = 8
    cfg.hidden = 1000
    with pytest.raises(ValueError, match="hidden"):
        _lib.check(_lib.lib().mono_moe_create(ctypes.byref(cfg), ctypes.byref(h)))
    # destroying NULL is a no-op
    _lib.check(_lib.lib().mono_moe_destroy(None))
