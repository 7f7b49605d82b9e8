"""materializer_for over a lazily built default registry (test double)."""

from . import core

_DEFAULT_REGISTRY = None


def materializer_for(target):
    global _DEFAULT_REGISTRY
    if _DEFAULT_REGISTRY is None:
        _DEFAULT_REGISTRY = core.Registry()
    return _DEFAULT_REGISTRY._items.get(str(target).lower())
