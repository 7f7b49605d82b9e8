"""Backend and materializer registries (reference ``src/ninetoothed/backends/__init__.py:22-85``)."""

from ninetoothed_amd.backends.core import (  # noqa: F401
    Artifact,
    Backend,
    BuiltArtifact,
    Capability,
    Registry,
    Target,
    backend_id_for,
    normalize_target,
)

_DEFAULT = None


def create_default_registry():
    from ninetoothed_amd.backends.hip import HipBackend

    registry = Registry()
    registry.register(HipBackend())
    return registry


def default_registry():
    global _DEFAULT
    if _DEFAULT is None:
        _DEFAULT = create_default_registry()
    return _DEFAULT
