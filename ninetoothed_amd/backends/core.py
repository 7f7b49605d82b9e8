"""Backend registry and artifact contracts.

Same shape as the reference's plugin interface (``src/ninetoothed/backends/core.py:11-163``):
``Target``, ``Capability``, ``Artifact``, ``BuiltArtifact``, ``Backend`` (with
``normalize_options`` / ``prepare_for_emission`` / ``emit``) and ``Registry``.  The
reference's ``Target`` enumerates triton/tilelang/cuda; this package's enumerates the
one backend it implements, ``hip`` (aliases ``rocm``, ``mi355x``, ``gfx950``).
"""

import json
from dataclasses import dataclass, field
from enum import Enum
from pathlib import Path
from typing import Any, Mapping, MutableMapping


class Target(str, Enum):
    HIP = "hip"


_CANONICAL_BACKEND_NAMES = {
    None: Target.HIP,
    "hip": Target.HIP,
    "rocm": Target.HIP,
    "mi355x": Target.HIP,
    "gfx950": Target.HIP,
}


@dataclass(frozen=True, kw_only=True)
class Capability:
    name: Target | str
    emits_source: bool
    can_execute: bool
    requires_external_compiler: bool = False
    notes: tuple[str, ...] = ()


@dataclass(frozen=True, kw_only=True)
class Artifact:
    """The output of lowering a kernel to a backend: here a launch plan, not source."""

    backend: Target
    kernel_name: str
    language: str
    sources: Mapping[str, str]
    entrypoint: str | None = None
    metadata: Mapping[str, Any] = field(default_factory=dict)

    @property
    def primary_source_name(self) -> str:
        return next(iter(self.sources))

    @property
    def primary_source(self) -> str:
        return self.sources[self.primary_source_name]

    def write_to(self, output_dir):
        output_path = Path(output_dir)
        output_path.mkdir(parents=True, exist_ok=True)
        paths = []
        for name, content in self.sources.items():
            path = output_path / name
            path.write_text(content, encoding="utf-8")
            paths.append(path)
        return tuple(paths)


@dataclass(frozen=True, kw_only=True)
class BuiltArtifact:
    source: Artifact
    cache_key: str
    source_path: str
    binary_path: str | None
    manifest_path: str
    abi: Mapping[str, Any]


class Backend:
    name: Target | str
    capability: Capability
    supported_options: frozenset = frozenset()

    def normalize_options(self, options: Mapping[str, Any]) -> Mapping[str, Any]:
        unknown = sorted(set(options) - self.supported_options)
        if unknown:
            names = ", ".join(f"`{name}`" for name in unknown)
            raise TypeError(f"Unsupported {backend_id_for(self.name)} backend option(s): {names}.")
        return dict(options)

    def prepare_for_emission(self, kernel):
        return kernel

    def emit(self, kernel) -> Artifact:
        raise NotImplementedError


class Registry:
    def __init__(self):
        self._backends: MutableMapping[str, Backend] = {}

    def register(self, backend: Backend, *, replace: bool = False) -> None:
        backend_id = backend_id_for(backend.name)
        if backend_id in self._backends and not replace:
            raise ValueError(f"Backend `{backend_id}` is already registered.")
        self._backends[backend_id] = backend

    def get(self, name) -> Backend:
        normalized = backend_id_for(normalize_target(name))
        try:
            return self._backends[normalized]
        except KeyError as exc:
            available = ", ".join(sorted(self._backends))
            raise ValueError(f"Unsupported backend `{normalized}`. Available backends: {available}.") from exc

    def capabilities(self):
        return tuple(b.capability for b in self._backends.values())

    def names(self):
        return tuple(sorted(self._backends))


def backend_id_for(name) -> str:
    value = name.value if isinstance(name, Target) else str(name)
    backend_id = value.strip().lower()
    if not backend_id:
        raise ValueError("Backend id must not be empty.")
    return backend_id


def normalize_target(name) -> Target:
    if isinstance(name, Target):
        return name
    key = None if name is None else str(name).lower()
    try:
        return _CANONICAL_BACKEND_NAMES[key]
    except KeyError as exc:
        supported = ", ".join(sorted(a for a in _CANONICAL_BACKEND_NAMES if isinstance(a, str)))
        raise ValueError(f"Unsupported backend `{name}`. Supported backends: {supported}.") from exc


def dump_json(value) -> str:
    return json.dumps(value, indent=1, sort_keys=True, default=str)
