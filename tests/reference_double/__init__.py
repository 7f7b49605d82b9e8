"""A test double of the reference package's object model, for the adapter's tests only.

The reference cannot be imported in this suite, so this small package of our own plays the
parts the adapter reads: a ``Symbol`` whose name carries its constexpr / meta role as a
prefix and whose bounds are attributes (as reference src/ninetoothed/symbol.py:20-95 and
naming.py:8-52 describe), a ``Tensor`` with the attributes of reference tensor.py:27-120,
``block_size``, a ``language`` module of named functions, and the two registries of
reference backends/__init__.py:22-43 and backends/materializers/__init__.py:7-29.
"""

import ast
import itertools
from dataclasses import dataclass

from . import backends, compiler, language  # noqa: F401

_count = itertools.count()


def _prefixed(name, role):
    return f"ninetoothed_{role}_prefix_{name}"


class Symbol:
    def __init__(self, expr, constexpr=None, meta=None, lower_bound=None, upper_bound=None, power_of_two=None):
        self._node = ast.parse(str(expr), mode="eval").body
        if isinstance(self._node, ast.Name):
            if meta:
                self._node.id = _prefixed(self._node.id, "meta")
            if constexpr:
                self._node.id = _prefixed(self._node.id, "constexpr")
            self._node.symbol = self
        self.lower_bound = lower_bound if lower_bound is not None else (32 if meta else (1 if constexpr else None))
        self.upper_bound = upper_bound if upper_bound is not None else (1024 if meta else (2**20 if constexpr else None))
        self.power_of_two = power_of_two if power_of_two is not None else (True if meta else (False if constexpr else None))

    def __mul__(self, other):
        out = Symbol("0")
        out._node = ast.BinOp(self._node, ast.Mult(), ast.Constant(other) if isinstance(other, int) else other._node)
        return out

    def __str__(self):
        return ast.unparse(self._node)


class Tensor:
    def __init__(self, ndim=None, shape=None, dtype=None, jagged_dim=None, other=None, shape_options=None,
                 constexpr=None, value=None, name=None):
        ndim = len(shape) if ndim is None else ndim
        shape = shape if shape is not None else (None,) * ndim
        options = shape_options if isinstance(shape_options, (tuple, list)) else (shape_options or {},) * ndim
        self.name = name or f"tensor_{next(_count)}"
        self.shape = tuple(s if s is not None else Symbol(f"{self.name}_size_{i}", **(o or {}))
                           for i, (s, o) in enumerate(zip(shape, options)))
        self.ndim = ndim
        self.dtype, self.jagged_dim, self.other = dtype, jagged_dim, other
        self.constexpr, self.value = constexpr, value
        self.source = self


def block_size(lower_bound=None, upper_bound=None):
    return Symbol(f"BLOCK_SIZE_{next(_count)}", meta=True, lower_bound=lower_bound, upper_bound=upper_bound)


@dataclass(frozen=True)
class Compilation:
    request: object
