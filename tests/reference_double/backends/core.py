"""Backend, Capability, Artifact and Registry with the reference's fields (test double)."""

from dataclasses import dataclass, field
from typing import Any, Mapping


@dataclass(frozen=True, kw_only=True)
class Capability:
    name: Any
    emits_source: bool
    can_execute: bool
    requires_external_compiler: bool = False
    notes: tuple = ()


@dataclass(frozen=True, kw_only=True)
class Artifact:
    backend: Any
    kernel_name: str
    language: str
    sources: Mapping[str, str]
    entrypoint: str = None
    metadata: Mapping[str, Any] = field(default_factory=dict)


class Backend:
    name = None
    capability = None

    def emit(self, kernel):
        raise NotImplementedError


class Registry:
    def __init__(self):
        self._items = {}

    def register(self, item, *, replace=False):
        key = str(getattr(item, "name", None) or item.target).lower()
        if key in self._items and not replace:
            raise ValueError(f"`{key}` is already registered.")
        self._items[key] = item

    def get(self, name):
        return self._items[str(name).lower()]
