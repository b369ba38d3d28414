"""A stand-in for SGLang's monokernel registry (the names sgl_amd_mono reads:
``register``, ``DeviceLimits``, ``Feature``, ``MonoSpec``, ``Numerics``,
``NumericsKind``, ``Requirements``; sgl_amd_mono/__init__.py:33-55,
glm53/spec.py:34-51), for CPU tests of the plugin surface. SGLang is not installed in
this image; this module only records registrations and looks them up the way a
server would: by backend, architecture, model type and ISA."""

from __future__ import annotations

import enum
import importlib
from dataclasses import dataclass, field

_REGISTRY: dict = {}


@dataclass(frozen=True)
class DeviceLimits:
    widths: tuple
    tp_sizes: tuple
    resident_blocks: int


class Feature(enum.Enum):
    SPECULATIVE_DECODING = "speculative_decoding"


class NumericsKind(enum.Enum):
    TOLERANCE = "tolerance"
    EXACT = "exact"


@dataclass(frozen=True)
class Numerics:
    kind: NumericsKind
    bounds: dict


@dataclass(frozen=True)
class Requirements:
    dtypes: frozenset = frozenset()
    attention_backends: frozenset = frozenset()
    server_args: dict = field(default_factory=dict)
    env: dict = field(default_factory=dict)


@dataclass(frozen=True)
class MonoSpec:
    name: str
    devices: dict
    features: frozenset
    requires: Requirements
    numerics: Numerics
    model_disable_reasons: object
    build: object
    api_version: int
    config_disable_reasons: object = None


@dataclass(frozen=True)
class ShapeKey:
    forward_mode: str
    batch_size: int
    tokens_per_request: int

    @property
    def rows(self) -> int:
        return self.batch_size * self.tokens_per_request


@dataclass
class Plan:
    key: ShapeKey
    state: dict = field(default_factory=dict)


def register(backend: str, architecture: str, path: str, model_type=None) -> None:
    _REGISTRY[backend, architecture, model_type] = path


def find_spec(backend: str, architectures, isa: str, model_type=None):
    """(spec, "") or (None, why)."""
    for arch in architectures:
        path = _REGISTRY.get((backend, arch, model_type)) or _REGISTRY.get((backend, arch, None))
        if path is None:
            continue
        mod, _, attr = path.partition(":")
        spec = getattr(importlib.import_module(mod), attr)
        if isa not in spec.devices:
            return None, f"{spec.name} has no limits for {isa}"
        return spec, ""
    return None, f"no {backend} spec for {list(architectures)}"
