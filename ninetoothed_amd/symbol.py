"""Symbols: named sizes, block sizes and integer expressions over them.

Same public surface as the reference's ``Symbol`` (``src/ninetoothed/symbol.py:9-271``):
``Symbol(expr, constexpr=, meta=, lower_bound=, upper_bound=, power_of_two=)`` and
``block_size(lower_bound, upper_bound)``, with the reference's defaults for meta
symbols (power-of-two block sizes in [32, 1024]) and non-meta constexpr symbols
([1, 2**20]).  Arithmetic builds an expression tree that folds constants eagerly;
``evaluate(env)`` substitutes concrete integers by name.  ``==`` is structural, as
in the reference, so arrangement code can test ``size == -1`` on symbolic sizes.

The representation is this package's own: a small tuple-based expression tree, no
Python AST and no sympy.
"""

import ast
import itertools
import math
import numbers
import operator

_BINARY = {
    "add": operator.add,
    "sub": operator.sub,
    "mul": operator.mul,
    "floordiv": operator.floordiv,
    "mod": operator.mod,
    "lt": operator.lt,
    "le": operator.le,
    "gt": operator.gt,
    "ge": operator.ge,
    "and": operator.and_,
    "max": max,
    "min": min,
}
_TEXT = {
    "add": "+",
    "sub": "-",
    "mul": "*",
    "floordiv": "//",
    "mod": "%",
    "lt": "<",
    "le": "<=",
    "gt": ">",
    "ge": ">=",
    "and": "&",
}

META_LOWER_BOUND = 2**5
META_UPPER_BOUND = 2**10
CONSTEXPR_LOWER_BOUND = 1
CONSTEXPR_UPPER_BOUND = 2**20


class Symbol:
    """A named value or an integer expression over named values."""

    __slots__ = ("_op", "_args", "constexpr", "meta", "lower_bound", "upper_bound", "power_of_two")

    def __init__(self, expr, constexpr=None, meta=None, lower_bound=None, upper_bound=None, power_of_two=None):
        self.constexpr = None
        self.meta = None
        self.lower_bound = None
        self.upper_bound = None
        self.power_of_two = None
        if isinstance(expr, Symbol):
            self._op, self._args = expr._op, expr._args
            for attr in ("constexpr", "meta", "lower_bound", "upper_bound", "power_of_two"):
                setattr(self, attr, getattr(expr, attr))
            return
        if isinstance(expr, tuple) and len(expr) == 2 and isinstance(expr[0], str) and isinstance(expr[1], tuple):
            self._op, self._args = expr  # internal node constructor
            return
        if isinstance(expr, bool) or isinstance(expr, numbers.Number):
            self._op, self._args = "const", (expr,)
        elif isinstance(expr, str):
            text = expr.strip()
            if text.isidentifier():
                self._op, self._args = "name", (text,)
            else:
                parsed = _from_python(ast.parse(text, mode="eval").body)
                self._op, self._args = parsed._op, parsed._args
        else:
            raise TypeError(f"cannot make a Symbol from {type(expr).__name__}")

        if (constexpr or meta) and self._op != "name":
            raise ValueError("The `constexpr` and `meta` options are properties of name symbols.")
        if meta and constexpr is False:
            raise ValueError("Non-constexpr meta symbol is not supported.")
        self.meta = bool(meta) if meta is not None else None
        self.constexpr = True if meta else constexpr
        if lower_bound is not None:
            self.lower_bound = lower_bound
        elif meta:
            self.lower_bound = META_LOWER_BOUND
        elif constexpr:
            self.lower_bound = CONSTEXPR_LOWER_BOUND
        if upper_bound is not None:
            self.upper_bound = upper_bound
        elif meta:
            self.upper_bound = META_UPPER_BOUND
        elif constexpr:
            self.upper_bound = CONSTEXPR_UPPER_BOUND
        if power_of_two is not None:
            self.power_of_two = power_of_two
        elif meta:
            self.power_of_two = True
        elif constexpr:
            self.power_of_two = False

    # ------------------------------------------------------------------ queries
    @property
    def name(self):
        return self._args[0] if self._op == "name" else None

    def is_constant(self):
        return self._op == "const"

    @property
    def value(self):
        if self._op != "const":
            raise ValueError(f"{self} is not a constant")
        return self._args[0]

    def names(self):
        """Names of the symbols this expression depends on."""
        if self._op == "name":
            return {self._args[0]}
        if self._op == "const":
            return set()
        out = set()
        for a in self._args:
            if isinstance(a, Symbol):
                out |= a.names()
        return out

    def evaluate(self, env):
        """Substitute names from ``env`` (name -> number) and compute the value."""
        op, args = self._op, self._args
        if op == "const":
            return args[0]
        if op == "name":
            try:
                return env[args[0]]
            except KeyError:
                raise KeyError(f"no value for symbol `{args[0]}`") from None
        if op == "neg":
            return -evaluate(args[0], env)
        return _BINARY[op](evaluate(args[0], env), evaluate(args[1], env))

    # --------------------------------------------------------------- arithmetic
    def _binary(self, op, other, swap=False):
        lhs, rhs = (Symbol(other), self) if swap else (self, Symbol(other))
        if lhs._op == "const" and rhs._op == "const":
            return Symbol(_BINARY[op](lhs.value, rhs.value))
        if op == "add":
            if lhs == 0:
                return rhs
            if rhs == 0:
                return lhs
        elif op == "sub":
            if rhs == 0:
                return lhs
        elif op == "mul":
            if lhs == 1:
                return rhs
            if rhs == 1:
                return lhs
            if lhs == 0 or rhs == 0:
                return Symbol(0)
        elif op == "floordiv":
            if rhs == 1:
                return lhs
        return Symbol((op, (lhs, rhs)))

    def __add__(self, other):
        return self._binary("add", other)

    def __radd__(self, other):
        return self._binary("add", other, swap=True)

    def __sub__(self, other):
        return self._binary("sub", other)

    def __rsub__(self, other):
        return self._binary("sub", other, swap=True)

    def __mul__(self, other):
        return self._binary("mul", other)

    def __rmul__(self, other):
        return self._binary("mul", other, swap=True)

    def __floordiv__(self, other):
        return self._binary("floordiv", other)

    def __rfloordiv__(self, other):
        return self._binary("floordiv", other, swap=True)

    def __mod__(self, other):
        return self._binary("mod", other)

    def __rmod__(self, other):
        return self._binary("mod", other, swap=True)

    def __neg__(self):
        if self._op == "const":
            return Symbol(-self.value)
        return Symbol(("neg", (self,)))

    def __lt__(self, other):
        return self._binary("lt", other)

    def __le__(self, other):
        return self._binary("le", other)

    def __gt__(self, other):
        return self._binary("gt", other)

    def __ge__(self, other):
        return self._binary("ge", other)

    def __and__(self, other):
        return self._binary("and", other)

    def __rand__(self, other):
        return self._binary("and", other, swap=True)

    def __eq__(self, other):
        if isinstance(other, Symbol):
            return self._op == other._op and self._args == other._args
        if isinstance(other, numbers.Number):
            return self._op == "const" and self._args[0] == other
        return NotImplemented

    def __hash__(self):
        return hash((self._op, self._args))

    def __index__(self):
        if self._op == "const" and isinstance(self.value, int):
            return self.value
        raise TypeError(f"symbolic value `{self}` has no concrete integer value yet")

    def __repr__(self):
        op, args = self._op, self._args
        if op == "const":
            return repr(args[0])
        if op == "name":
            return args[0]
        if op == "neg":
            return f"(-{args[0]!r})"
        if op in ("max", "min"):
            return f"{op}({args[0]!r}, {args[1]!r})"
        return f"({args[0]!r} {_TEXT[op]} {args[1]!r})"


def evaluate(value, env):
    """Evaluate a Symbol, number or nested tuple/list of them."""
    if isinstance(value, Symbol):
        return value.evaluate(env)
    if isinstance(value, (tuple, list)):
        return type(value)(evaluate(v, env) for v in value)
    return value


def names_in(value):
    if isinstance(value, Symbol):
        return value.names()
    if isinstance(value, (tuple, list)):
        out = set()
        for v in value:
            out |= names_in(v)
        return out
    return set()


def prod(values):
    result = 1
    for v in values:
        result = result * v
    return result


def _from_python(node):
    """A Python expression AST -> Symbol (integer arithmetic and names only)."""
    if isinstance(node, ast.Constant):
        return Symbol(node.value)
    if isinstance(node, ast.Name):
        return Symbol(node.id)
    if isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.USub):
        return -_from_python(node.operand)
    if isinstance(node, ast.BinOp):
        ops = {ast.Add: "__add__", ast.Sub: "__sub__", ast.Mult: "__mul__", ast.FloorDiv: "__floordiv__", ast.Mod: "__mod__"}
        name = ops.get(type(node.op))
        if name is not None:
            return getattr(_from_python(node.left), name)(_from_python(node.right))
    raise ValueError(f"unsupported symbol expression: {ast.unparse(node)}")


_block_size_counter = itertools.count()


def block_size(lower_bound=None, upper_bound=None):
    """A fresh block-size meta symbol (reference ``src/ninetoothed/symbol.py:257-271``), named as
    the reference names generated symbols (``naming.py:4-5``), so a call's meta keywords agree."""
    return Symbol(f"ninetoothed_BLOCK_SIZE_{next(_block_size_counter)}", meta=True, lower_bound=lower_bound,
                  upper_bound=upper_bound)


def default_meta_value(symbol, preferred=64):
    """The value this backend gives a meta symbol nobody set: ``preferred`` clamped
    into the symbol's bounds (kept a power of two when the symbol asks for one).

    Meta symbols only choose how the reference tiles its launch grid; the MI355X
    kernels pick their own tiles, so any legal value yields the same computation.
    """
    lo = symbol.lower_bound if symbol.lower_bound is not None else 1
    hi = symbol.upper_bound if symbol.upper_bound is not None else max(preferred, lo)
    value = min(max(preferred, lo), hi)
    if symbol.power_of_two:
        p = 1 << max(0, math.ceil(math.log2(max(value, 1))))
        if p > hi:
            p >>= 1
        value = max(p, 1)
    return int(value)
