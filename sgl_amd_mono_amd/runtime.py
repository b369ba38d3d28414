"""What every C-ABI runtime handle shares on the host: lifetime and the guard.

The guard is the reference's fail-stop machinery (sgl_amd_mono/common/guard.py:100-241,
``Glm53Runtime.set_deadline`` glm53/gfx950/runner.py:197-204): every inter-workgroup
wait of a launch has a deadline; the first one to pass it records its site in the
runtime's guard words and the runtime refuses launches until the host clears it.
"""

from __future__ import annotations

import ctypes as C

import torch

from . import _lib


class Runtime:
    """Base of the MoE and attention runtimes: ``PREFIX`` names the C-ABI family
    (``mono_moe`` / ``mono_attn``) and ``SITES`` its wait sites."""

    PREFIX = ""
    SITES: dict = {}
    KIND = ""

    def __init__(self, device):
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"{type(self).__name__} needs a GPU device, got {self.device}")
        self._h = C.c_void_p()

    def _fn(self, name):
        return getattr(_lib.lib(), f"{self.PREFIX}_{name}")

    def _create(self, cfg) -> None:
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(self._fn("create")(C.byref(cfg), C.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.check(self._fn("destroy")(self._h))
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def set_deadline(self, seconds: float) -> None:
        """Deadline of every inter-workgroup wait of later launches."""
        _lib.check(self._fn("set_deadline")(self._h, float(seconds)))

    def set_fault(self, site: int) -> None:
        """Tests of the fail-stop path: every wait at ``site`` fails at once (-1: off)."""
        _lib.check(self._fn("set_fault")(self._h, int(site)))

    def error_words(self) -> list[int]:
        """The guard words (synchronises): [tag epochs, 1 + failed wait site or 0, failing
        launch tag, failing workgroup, launches begun (u64, two words), scrub barrier,
        reserved]."""
        words = (C.c_int32 * _lib.GUARD_WORDS)()
        with torch.cuda.device(self.device):
            _lib.check(self._fn("read_errors")(self._h, words))
        return list(words)

    def check_errors(self) -> None:
        """Raise MonoError if a launch of this runtime stopped at a wait (fail-stop)."""
        w = self.error_words()
        if w[1]:
            site = w[1] - 1
            raise _lib.MonoError(
                _lib.MONO_ESTATE,
                f"{self.KIND} launch (tag {w[2]}) stopped: wait '{self.SITES.get(site, site)}' passed its "
                f"deadline in workgroup {w[3]}; the runtime refuses launches until clear_errors()",
            )

    def clear_errors(self) -> None:
        with torch.cuda.device(self.device):
            _lib.check(self._fn("clear_errors")(self._h))


def need(t: torch.Tensor, name: str, shape: tuple, dtypes, device: torch.device) -> None:
    """Raise ValueError naming the tensor unless it has this shape / dtype and is a
    contiguous tensor on ``device`` (the checks of glm53/gfx950/runner.py:250-273)."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a tensor, got {type(t).__name__}")
    dtypes = dtypes if isinstance(dtypes, tuple) else (dtypes,)
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.dtype not in dtypes:
        raise ValueError(f"{name}: expected dtype {' or '.join(map(str, dtypes))}, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name}: expected device {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous tensor (strides {t.stride()})")
