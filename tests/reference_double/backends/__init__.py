"""A backend registry with the reference's register / get contract (test double)."""

from . import core, materializers  # noqa: F401

_DEFAULT = None


def default_registry():
    global _DEFAULT
    if _DEFAULT is None:
        _DEFAULT = core.Registry()
    return _DEFAULT
