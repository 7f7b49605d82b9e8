"""Application frontend: a parsed (never executed) application body -> value graph.

Plays the role of the reference's ``from_application``
(``src/ninetoothed/frontend/python.py:37-91``): the body of an application is parsed
with ``ast`` and lowered once per specialization (concrete constexpr values fold
``if`` statements, as the reference's runtime specialization does for non-Triton
backends, ``src/ninetoothed/compiler/runtime.py:158-243``).  Supported constructs are
those of the hot-path applications: assignments and augmented assignments, ``for _ in
range(...)`` loops with loop-carried values, constexpr ``if``, calls to ``ntl``
functions, ``.to(dtype)``, ``.offsets(dim)``, ``.shape`` / ``.source.shape`` / ``.dtype``,
level indexing ``x[k]``, broadcasting subscripts ``x[:, None]``, arithmetic and
comparisons, ``float("-inf")``, and calls to helper applications, which are inlined
(reference ``_InlineHelperCalls``, ``frontend/python.py:94-306``: a helper that assigns
to one of its parameters assigns to the caller's variable or tensor it was given).

The result is a graph of hash-consed ``Value`` nodes (structurally equal expressions
are the same object), plus the loops and the stores (assignments to parameters).
Family matchers in ``ninetoothed_amd.families`` read this graph.
"""

import ast
import builtins
import inspect
import math
import textwrap
from dataclasses import dataclass, field

from ninetoothed_amd import language as ntl
from ninetoothed_amd.dtype import normalize_dtype
from ninetoothed_amd.errors import LoweringError


class Value:
    __slots__ = ("op", "args", "__weakref__")

    def __init__(self, op, args):
        self.op = op
        self.args = args

    def __repr__(self):
        return f"{self.op}({', '.join(_short(a) for a in self.args)})"


def _short(a):
    if isinstance(a, Value):
        return repr(a) if a.op in ("param", "const", "dtype", "loop_index", "carried") else f"<{a.op}>"
    return repr(a)


VIEW_OPS = ("param", "index")


@dataclass
class Loop:
    id: int
    var: str
    trip: Value
    init: dict = field(default_factory=dict)
    update: dict = field(default_factory=dict)
    parent: int = None  # id of the symbolic loop whose body holds this one
    effects: tuple = (0, 0)  # [start, end) of the program's effects recorded in the body


@dataclass
class Program:
    params: tuple
    stores: dict  # param name -> stored value (last store)
    loops: dict  # loop id -> Loop
    store_order: list
    # side effects outside the arranged tile stores, in program order:
    # ("src_store", param, indices, value), ("ptr_store", ptr, value), ("atomic_add", ptr, value)
    effects: list = field(default_factory=list)


@dataclass
class ParamInfo:
    """What the frontend needs to know about one application parameter."""

    name: str
    level_ndims: tuple  # ndim of each level below the program level (level 1 first)
    source_ndim: int
    constexpr: bool = False
    constexpr_value: object = None


class _Builder:
    def __init__(self):
        self._interned = {}

    def make(self, op, *args):
        key = (op,) + tuple(id(a) if isinstance(a, Value) else ("#", _freeze(a)) for a in args)
        v = self._interned.get(key)
        if v is None:
            v = Value(op, args)
            self._interned[key] = v
        return v


def _freeze(a):
    if isinstance(a, (list, tuple)):
        return tuple(_freeze(x) for x in a)
    if isinstance(a, float) and math.isnan(a):
        return "nan"
    return a


class _Shape:
    """``x.shape`` of a view or of a value with a known shape."""

    def __init__(self, items):
        self.items = tuple(items)

    def __getitem__(self, i):
        return self.items[i]


class _Source:
    def __init__(self, param, ndim):
        self.param = param
        self.ndim = ndim


class _Method:
    def __init__(self, name, target):
        self.name = name
        self.target = target


class _Alias:
    """A helper parameter bound to the caller's local variable or tensor parameter."""

    def __init__(self, kind, name, frame):
        self.kind = kind  # "local" | "param"
        self.name = name
        self.frame = frame


_NTL_BY_ID = {id(getattr(ntl, name)): name for name in ntl._FUNCTIONS}
_NTL_BY_ID.update({id(getattr(ntl.libdevice, name)): f"libdevice.{name}" for name in ntl.libdevice.FUNCTIONS})
_DTYPE_NAMES = {"float8_e4m3fn", "float8_e5m2", "float16", "bfloat16", "float32", "float64", "int8", "int16", "int32",
                "int64", "uint8"}

_BINOPS = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div", ast.FloorDiv: "floordiv", ast.Mod: "mod"}
_CMPOPS = {ast.Lt: "lt", ast.LtE: "le", ast.Gt: "gt", ast.GtE: "ge", ast.Eq: "eq", ast.NotEq: "ne"}


class _Frame:
    def __init__(self, func, node, bindings, param_names):
        self.func = func
        self.node = node
        self.env = dict(bindings)
        self.param_names = set(param_names)
        self.globals = getattr(func, "__globals__", {})
        closure = inspect.getclosurevars(func) if func is not None else None
        self.nonlocals = dict(closure.nonlocals) if closure is not None else {}


def parse_function(func):
    try:
        source = textwrap.dedent(inspect.getsource(func))
    except (OSError, TypeError) as exc:
        raise LoweringError(f"cannot read the source of application `{getattr(func, '__name__', func)}`") from exc
    module = ast.parse(source)
    for node in module.body:
        if isinstance(node, (ast.FunctionDef, ast.AsyncFunctionDef)) and node.name == func.__name__:
            return node
    for node in ast.walk(module):
        if isinstance(node, ast.FunctionDef):
            return node
    raise LoweringError(f"no function definition found for `{func.__name__}`")


def parameter_names(func):
    node = parse_function(func)
    return tuple(a.arg for a in node.args.args)


class Lowerer:
    def __init__(self, application, params, unroll=None):
        self.unroll = unroll  # trip Value -> int, or None: loops are lowered symbolically
        self.b = _Builder()
        self.params = {p.name: p for p in params}
        self.loops = {}
        self.stores = {}
        self.store_order = []
        self.effects = []
        self.written = {}  # param -> the whole tile last assigned to it
        self._loop_ids = 0
        self._loop_stack = []  # ids of the symbolic loops being lowered, outermost first
        self.application = application

    # ----------------------------------------------------------------- driver
    def lower(self):
        node = parse_function(self.application)
        names = tuple(a.arg for a in node.args.args)
        if set(names) != set(self.params):
            raise LoweringError(f"application parameters {names} do not match the arranged tensors {tuple(self.params)}")
        bindings = {}
        for name in names:
            info = self.params[name]
            if info.constexpr:
                bindings[name] = info.constexpr_value
            else:
                bindings[name] = self.b.make("param", name)
        frame = _Frame(self.application, node, bindings, names)
        self._block(frame, node.body)
        return Program(names, dict(self.stores), dict(self.loops), list(self.store_order), list(self.effects))

    # ----------------------------------------------------------------- values
    def const(self, v):
        return self.b.make("const", float(v) if isinstance(v, float) else v)

    def view_level(self, v):
        if v.op == "param":
            return 1
        if v.op == "index":
            return self.view_level(v.args[0]) + 1
        raise LoweringError("not a tensor view")

    def view_param(self, v):
        while v.op == "index":
            v = v.args[0]
        return v.args[0]

    def view_ndim(self, v):
        info = self.params[self.view_param(v)]
        level = self.view_level(v)
        if level - 1 >= len(info.level_ndims):
            return 0
        return info.level_ndims[level - 1]

    def data(self, v):
        """A value used as data: tensor views are loaded.  A parameter read after the
        application assigned it reads back what it stored (the reference loads it after its
        store, in program order), in the parameter's dtype."""
        if isinstance(v, Value):
            if v.op == "param" and v.args[0] in self.written:
                return self.b.make("cast", self.written[v.args[0]], self.b.make("dtype_of", v))
            if v.op in VIEW_OPS:
                return self.b.make("load", v)
            return v
        if isinstance(v, bool):
            return self.const(v)
        if isinstance(v, (int, float)):
            return self.const(v)
        raise LoweringError(f"cannot use {v!r} as a tensor value")

    def dtype_value(self, d):
        if isinstance(d, Value) and d.op in ("dtype_of", "dtype"):
            return d
        if isinstance(d, str):
            name = normalize_dtype(d)
            if name not in _DTYPE_NAMES:
                raise LoweringError(f"unknown dtype {d!r}")
            return self.b.make("dtype", name)
        raise LoweringError(f"unsupported dtype expression {d!r}")

    # -------------------------------------------------------------- statements
    def _block(self, frame, stmts):
        for s in stmts:
            self._stmt(frame, s)

    def _assign_name(self, frame, name, value):
        cur = frame.env.get(name)
        if isinstance(cur, _Alias):
            if cur.kind == "local":
                self._assign_name(cur.frame, cur.name, value)
            else:
                self._store(cur.name, value)
            return
        if name in frame.param_names and isinstance(cur, Value) and cur.op == "param":
            self._store(cur.args[0], value)
            return
        frame.env[name] = value

    @staticmethod
    def _is_param_binding(frame, name):
        """Whether ``name`` still names an application parameter: assigning it stores into
        the parameter (never a loop-carried local)."""
        v = frame.env.get(name)
        return name in frame.param_names and isinstance(v, Value) and v.op == "param"

    def _store(self, param, value):
        if self._loop_stack:
            # a whole arranged output assigned inside a loop that stays a loop: every iteration
            # stores its tile, as the reference's loop body does; a later read of the parameter
            # reads the tensor (a program that also reads it is refused by the tile kernels)
            self.effects.append(("view_store", self.b.make("param", param), self.data(value)))
            self.store_order.append(param)
            self.written.pop(param, None)
            return
        self.stores[param] = self.data(value)
        self.store_order.append(param)
        self.written[param] = self.stores[param]

    def _stmt(self, frame, s):
        if isinstance(s, ast.Expr):
            if isinstance(s.value, ast.Constant):
                return  # docstring
            self._expr(frame, s.value)
            return
        if isinstance(s, ast.Pass):
            return
        if isinstance(s, ast.Return):
            if s.value is not None:
                raise LoweringError("applications do not return values (a helper may end with `return value`)")
            return
        if isinstance(s, ast.Assign):
            if len(s.targets) != 1:
                raise LoweringError("chained assignment is not supported")
            value = self._expr(frame, s.value)
            self._target(frame, s.targets[0], value)
            return
        if isinstance(s, ast.AnnAssign):
            self._target(frame, s.target, self._expr(frame, s.value))
            return
        if isinstance(s, ast.AugAssign):
            cur = self._expr(frame, s.target)
            op = _BINOPS.get(type(s.op))
            if op is None:
                raise LoweringError(f"unsupported augmented operator {type(s.op).__name__}")
            self._target(frame, s.target, self._binop(op, cur, self._expr(frame, s.value)))
            return
        if isinstance(s, ast.If):
            test = self._expr(frame, s.test)
            if isinstance(test, Value):
                if test.op == "const":
                    test = test.args[0]
                else:
                    raise LoweringError("`if` on run-time data is not supported; branch on constexpr values only")
            self._block(frame, s.body if test else s.orelse)
            return
        if isinstance(s, ast.For):
            self._for(frame, s)
            return
        raise LoweringError(f"unsupported statement `{type(s).__name__}` in an application")

    def _target(self, frame, target, value):
        if isinstance(target, ast.Name):
            self._assign_name(frame, target.id, value)
            return
        if isinstance(target, ast.Tuple):
            if not isinstance(value, tuple) or len(value) != len(target.elts):
                raise LoweringError("tuple unpacking needs a tuple of the same length")
            for t, v in zip(target.elts, value):
                self._target(frame, t, v)
            return
        if isinstance(target, ast.Subscript):
            base = self._expr(frame, target.value)
            if isinstance(base, Value) and base.op in VIEW_OPS and not isinstance(target.slice, ast.Slice):
                # `out[i] = v`: a store into one element (a tile) of a level
                view = self._subscript(frame, base, target.slice)
                if not (isinstance(view, Value) and view.op == "index"):
                    raise LoweringError("only level indexing `out[i] = ...` can be assigned")
                self.effects.append(("view_store", view, self.data(value)))
                self.store_order.append(self.view_param(view))
                return
            if isinstance(base, _Source):
                indices = self._source_indices(frame, base, target.slice)
                self.effects.append(("src_store", base.param, indices, self.data(value)))
                self.store_order.append(base.param)
                return
        raise LoweringError("only simple names can be assigned in an application")

    def _for(self, frame, s):
        it = s.iter
        if not (isinstance(it, ast.Call) and isinstance(it.func, ast.Name) and it.func.id == "range" and len(it.args) == 1):
            raise LoweringError("only `for _ in range(n)` loops are supported")
        if s.orelse:
            raise LoweringError("`for ... else` is not supported")
        if not isinstance(s.target, ast.Name):
            raise LoweringError("loop variables must be simple names")
        trip = self.data(self._expr(frame, it.args[0])) if not isinstance(self._expr(frame, it.args[0]), Value) else self._expr(frame, it.args[0])
        count = self.unroll(trip) if self.unroll is not None else None
        if count is not None:
            # unrolled: the body runs `count` times with the loop variable a constant.  Values
            # carried from one iteration to the next are wrapped in `unmask` at every boundary:
            # like the results of a loop, they carry no load mask into later reductions.
            carried = [n for n in sorted(_assigned_names(s.body))
                       if isinstance(frame.env.get(n), Value) and not self._is_param_binding(frame, n)]

            def boundary():
                for n in carried:
                    if isinstance(frame.env.get(n), Value):
                        frame.env[n] = self.b.make("unmask", frame.env[n])

            for k in range(count):
                boundary()
                frame.env[s.target.id] = self.const(k)
                self._block(frame, s.body)
            boundary()
            return
        loop_id = self._loop_ids
        self._loop_ids += 1
        assigned = _assigned_names(s.body)
        carried = [n for n in sorted(assigned) if n in frame.env and not isinstance(frame.env[n], (_Alias,))
                   and not self._is_param_binding(frame, n)]
        alias_carried = [n for n in sorted(assigned) if isinstance(frame.env.get(n), _Alias) and frame.env[n].kind == "local"]
        loop = Loop(loop_id, s.target.id, trip, parent=self._loop_stack[-1] if self._loop_stack else None)
        saved = {}
        for n in carried:
            loop.init[n] = frame.env[n]
            saved[n] = frame.env[n]
            frame.env[n] = self.b.make("carried", loop_id, n)
        for n in alias_carried:
            a = frame.env[n]
            loop.init[n] = a.frame.env[a.name]
            a.frame.env[a.name] = self.b.make("carried", loop_id, n)
        frame.env[s.target.id] = self.b.make("loop_index", loop_id)
        start = len(self.effects)
        self._loop_stack.append(loop_id)
        try:
            self._block(frame, s.body)
        finally:
            self._loop_stack.pop()
        loop.effects = (start, len(self.effects))
        for n in carried:
            loop.update[n] = frame.env[n]
            frame.env[n] = self.b.make("loop_out", loop_id, n)
        for n in alias_carried:
            a = frame.env[n]
            loop.update[n] = a.frame.env[a.name]
            a.frame.env[a.name] = self.b.make("loop_out", loop_id, n)
        self.loops[loop_id] = loop

    # ------------------------------------------------------------- expressions
    def _lookup(self, frame, name):
        if name in frame.env:
            v = frame.env[name]
            if isinstance(v, _Alias):
                if v.kind == "local":
                    return self._lookup(v.frame, v.name)
                return v.frame.env[v.name] if v.name in v.frame.env else self.b.make("param", v.name)
            return v
        if name in frame.nonlocals:
            return frame.nonlocals[name]
        if name in frame.globals:
            return frame.globals[name]
        if hasattr(builtins, name):
            return getattr(builtins, name)
        raise LoweringError(f"name `{name}` is not defined in the application")

    def _expr(self, frame, e):
        if isinstance(e, ast.Constant):
            return e.value
        if isinstance(e, ast.Name):
            return self._lookup(frame, e.id)
        if isinstance(e, ast.Tuple):
            return tuple(self._expr(frame, x) for x in e.elts)
        if isinstance(e, ast.Attribute):
            return self._attribute(frame, self._expr(frame, e.value), e.attr)
        if isinstance(e, ast.BinOp):
            op = _BINOPS.get(type(e.op))
            if op is None:
                raise LoweringError(f"unsupported operator {type(e.op).__name__}")
            return self._binop(op, self._expr(frame, e.left), self._expr(frame, e.right))
        if isinstance(e, ast.UnaryOp):
            v = self._expr(frame, e.operand)
            if isinstance(e.op, ast.USub):
                if isinstance(v, (int, float)):
                    return -v
                return self.b.make("neg", self.data(v))
            if isinstance(e.op, ast.Not) and isinstance(v, (bool, int)):
                return not v
            if isinstance(e.op, ast.UAdd):
                return v
            raise LoweringError(f"unsupported unary operator {type(e.op).__name__}")
        if isinstance(e, ast.Compare):
            if len(e.ops) != 1:
                raise LoweringError("chained comparisons are not supported")
            op = _CMPOPS.get(type(e.ops[0]))
            lhs, rhs = self._expr(frame, e.left), self._expr(frame, e.comparators[0])
            if not isinstance(lhs, Value) and not isinstance(rhs, Value):
                return {"lt": lhs < rhs, "le": lhs <= rhs, "gt": lhs > rhs, "ge": lhs >= rhs, "eq": lhs == rhs, "ne": lhs != rhs}[op]
            return self.b.make(op, self.data(lhs), self.data(rhs))
        if isinstance(e, ast.BoolOp):
            vals = [self._expr(frame, x) for x in e.values]
            if all(not isinstance(v, Value) for v in vals):
                return all(vals) if isinstance(e.op, ast.And) else any(vals)
            raise LoweringError("boolean operators on tensors are not supported; use `&` / `|`")
        if isinstance(e, ast.Subscript):
            return self._subscript(frame, self._expr(frame, e.value), e.slice)
        if isinstance(e, ast.Call):
            return self._call(frame, e)
        if isinstance(e, ast.List):
            return tuple(self._expr(frame, x) for x in e.elts)
        raise LoweringError(f"unsupported expression `{ast.unparse(e)}`")

    def _binop(self, op, lhs, rhs):
        if not isinstance(lhs, Value) and not isinstance(rhs, Value):
            return {
                "add": lambda a, b: a + b, "sub": lambda a, b: a - b, "mul": lambda a, b: a * b,
                "div": lambda a, b: a / b, "floordiv": lambda a, b: a // b, "mod": lambda a, b: a % b,
            }[op](lhs, rhs)
        return self.b.make(op, self.data(lhs), self.data(rhs))

    def _attribute(self, frame, base, attr):
        if isinstance(base, Value):
            if attr == "shape":
                if base.op in VIEW_OPS:
                    nd = self.view_ndim(base)
                    return _Shape(self.b.make("shape", base, d) for d in range(nd))
                if base.op in ("zeros", "full"):
                    return _Shape(base.args[0])
                if base.op == "dtype_of":
                    # the shape of a level below a view (x.dtype.shape, x.dtype.dtype.shape, x[0].dtype.shape)
                    view, depth = base, 0
                    while view.op == "dtype_of":
                        view, depth = view.args[0], depth + 1
                    param, level = self.view_param(view), self.view_level(view) + depth
                    ndims = self.params[param].level_ndims
                    if level - 1 >= len(ndims):
                        raise LoweringError(f"`{param}` has no level {level}")
                    return _Shape(self.b.make("level_shape", param, level, d) for d in range(ndims[level - 1]))
                raise LoweringError("`.shape` is only known for tensor parameters and zeros/full values")
            if attr == "dtype":
                if base.op in VIEW_OPS or base.op == "dtype_of":
                    return self.b.make("dtype_of", base)
                raise LoweringError("`.dtype` is only supported on tensor parameters")
            if attr == "source":
                if base.op != "param":
                    raise LoweringError("`.source` is only supported on tensor parameters")
                return _Source(base.args[0], self.params[base.args[0]].source_ndim)
            if attr in ("to", "offsets"):
                return _Method(attr, base)
            raise LoweringError(f"unsupported attribute `.{attr}`")
        if isinstance(base, _Source):
            if attr == "shape":
                return _Shape(self.b.make("source_shape", base.param, d) for d in range(base.ndim))
            if attr in ("data_ptr", "stride"):
                return _Method(attr, base)
            raise LoweringError(f"unsupported attribute `.source.{attr}`")
        try:
            return getattr(base, attr)
        except AttributeError as exc:
            raise LoweringError(f"`{attr}` not found") from exc

    def _subscript(self, frame, base, sl):
        if isinstance(base, _Shape):
            idx = self._expr(frame, sl)
            if not isinstance(idx, int):
                raise LoweringError("shape index must be an integer")
            return base[idx]
        if isinstance(base, (tuple, list)):
            return base[self._expr(frame, sl)]
        if isinstance(base, _Source):
            return self.b.make("src_load", base.param, self._source_indices(frame, base, sl))
        if not isinstance(base, Value):
            raise LoweringError("unsupported subscript")
        items = sl.elts if isinstance(sl, ast.Tuple) else [sl]
        if any(isinstance(x, ast.Slice) or (isinstance(x, ast.Constant) and x.value is None) for x in items):
            pattern = []
            for x in items:
                if isinstance(x, ast.Slice):
                    if x.lower or x.upper or x.step:
                        raise LoweringError("only `:` and `None` are supported in broadcasting subscripts")
                    pattern.append(":")
                elif isinstance(x, ast.Constant) and x.value is None:
                    pattern.append(None)
                else:
                    raise LoweringError("mixed integer/broadcast subscripts are not supported")
            return self.b.make("bcast", self.data(base), tuple(pattern))
        if base.op not in VIEW_OPS:
            raise LoweringError("only tensor parameters can be indexed by level")
        if len(items) != 1:
            raise LoweringError("level indexing takes one index")
        idx = self._expr(frame, items[0])
        return self.b.make("index", base, self.data(idx) if not isinstance(idx, Value) else idx)

    def _source_indices(self, frame, src, sl):
        items = sl.elts if isinstance(sl, ast.Tuple) else [sl]
        if len(items) != src.ndim:
            raise LoweringError(f"`.source[...]` of a {src.ndim}-D tensor takes {src.ndim} indices")
        return tuple(self.data(self._expr(frame, x)) for x in items)

    def _norm_dim(self, d, ndim):
        if not isinstance(d, int):
            raise LoweringError("dimension arguments must be integers")
        return d + ndim if d < 0 else d

    def _call(self, frame, e):
        func = self._expr(frame, e.func)
        args = [self._expr(frame, a) for a in e.args]
        kwargs = {k.arg: self._expr(frame, k.value) for k in e.keywords}
        if isinstance(func, _Method) and isinstance(func.target, _Source):
            src = func.target
            if func.name == "data_ptr":
                return self.b.make("ptr", src.param)
            d = args[0] if args else kwargs.get("dim")
            if not isinstance(d, int):
                raise LoweringError("`.source.stride(dim)` needs an integer dimension")
            return self.b.make("source_stride", src.param, self._norm_dim(d, src.ndim))
        if isinstance(func, _Method):
            t = func.target
            if func.name == "to":
                dt = args[0] if args else kwargs.get("dtype")
                return self.b.make("cast", self.data(t), self.dtype_value(dt))
            if func.name == "offsets":
                if t.op not in VIEW_OPS:
                    raise LoweringError("`.offsets` is only supported on tensor parameters")
                src_nd = self.params[self.view_param(t)].source_ndim
                d = self._norm_dim(args[0] if args else kwargs.get("dim", 0), src_nd)
                return self.b.make("offsets", t, d)
        if func is float and len(args) == 1 and isinstance(args[0], str):
            return float(args[0])
        if func in (float, int, bool, min, max, abs) and all(not isinstance(a, Value) for a in args):
            return func(*args)
        name = _NTL_BY_ID.get(id(func))
        if name is not None:
            return self._ntl(name, args, kwargs)
        if inspect.isfunction(func):
            return self._inline(frame, func, e)
        raise LoweringError(f"unsupported call `{ast.unparse(e.func)}`")

    def _ntl(self, name, args, kwargs):
        b = self.b
        if name in ("zeros", "full"):
            shape = args[0] if args else kwargs["shape"]
            if isinstance(shape, _Shape):
                shape = shape.items
            shape = tuple(self.data(x) if not isinstance(x, Value) else x for x in shape)
            if name == "zeros":
                dt = args[1] if len(args) > 1 else kwargs.get("dtype", "float32")
                return b.make("zeros", shape, self.dtype_value(dt))
            value = args[1] if len(args) > 1 else kwargs["value"]
            dt = args[2] if len(args) > 2 else kwargs.get("dtype", "float32")
            return b.make("full", shape, float(value), self.dtype_value(dt))
        if name == "dot":
            return b.make("dot", self.data(args[0]), self.data(args[1]))
        if name == "trans":
            return b.make("trans", self.data(args[0]))
        if name == "where":
            return b.make("where", self.data(args[0]), self.data(args[1]), self.data(args[2]))
        if name in ("max", "min", "sum"):
            axis = args[1] if len(args) > 1 else kwargs.get("axis")
            return b.make("reduce", name, self.data(args[0]), axis)
        if name in ("maximum", "minimum"):
            return b.make(name, self.data(args[0]), self.data(args[1]))
        if name in ("exp", "exp2", "log", "log2", "sqrt", "rsqrt", "abs", "sigmoid"):
            return b.make("math", name, self.data(args[0]))
        if name == "cast":
            return b.make("cast", self.data(args[0]), self.dtype_value(args[1] if len(args) > 1 else kwargs["dtype"]))
        if name == "load":
            if len(args) != 1 or kwargs:
                raise LoweringError("ntl.load takes one pointer (masks are added by the backend)")
            return b.make("ptr_load", self.data(args[0]))
        if name in ("store", "atomic_add"):
            if len(args) != 2 or kwargs:
                raise LoweringError(f"ntl.{name} takes (pointer, value)")
            self.effects.append(("ptr_store" if name == "store" else "atomic_add", self.data(args[0]),
                                 self.data(args[1])))
            return None
        if name in ("rand", "randint", "randn"):
            # counter-based random numbers: (seed, offset) -> one value per offset element
            if len(args) != 2 or kwargs:
                raise LoweringError(f"ntl.{name} takes (seed, offset)")
            return b.make(name, self.data(args[0]), self.data(args[1]))
        if name.startswith("libdevice."):
            if kwargs:
                raise LoweringError(f"{name} takes positional arguments only")
            return b.make("libm", name[len("libdevice."):], tuple(self.data(a) for a in args))
        raise LoweringError(f"ntl.{name} is not supported by the MI355X backend")

    def _inline(self, frame, func, call):
        node = parse_function(func)
        names = [a.arg for a in node.args.args]
        if len(call.args) > len(names):
            raise LoweringError(f"too many arguments for helper `{func.__name__}`")
        bindings = {}
        for pname, arg in zip(names, call.args):
            if isinstance(arg, ast.Name) and arg.id in frame.env:
                cur = frame.env[arg.id]
                if isinstance(cur, Value) and cur.op == "param" and arg.id in frame.param_names:
                    bindings[pname] = _Alias("param", cur.args[0], frame)
                    continue
                bindings[pname] = _Alias("local", arg.id, frame)
            else:
                bindings[pname] = self._expr(frame, arg)
        for kw in call.keywords:
            bindings[kw.arg] = self._expr(frame, kw.value)
        for pname in names:
            if pname not in bindings:
                raise LoweringError(f"missing argument `{pname}` for helper `{func.__name__}`")
        callee = _Frame(func, node, bindings, names)
        body = list(node.body)
        # a trailing `return value` is the call's value (reference frontend/python.py:226-270)
        result = body.pop() if body and isinstance(body[-1], ast.Return) else None
        self._block(callee, body)
        if result is None or result.value is None:
            return None
        return self._expr(callee, result.value)


def _assigned_names(stmts):
    out = set()
    for s in stmts:
        for node in ast.walk(s):
            if isinstance(node, (ast.Assign, ast.AugAssign, ast.AnnAssign)):
                targets = node.targets if isinstance(node, ast.Assign) else [node.target]
                for t in targets:
                    out.update(_bound_names(t))
    return out


def _bound_names(target):
    """Names an assignment target rebinds (``out[i] = v`` and ``x.source[...] = v`` rebind none)."""
    if isinstance(target, ast.Name):
        return {target.id}
    if isinstance(target, (ast.Tuple, ast.List)):
        return set().union(*(_bound_names(t) for t in target.elts)) if target.elts else set()
    return set()


def pointer_param(v):
    """The tensor parameter whose ``source.data_ptr()`` a pointer expression starts from."""
    found = set()
    stack = [v]
    while stack:
        x = stack.pop()
        if not isinstance(x, Value):
            continue
        if x.op == "ptr":
            found.add(x.args[0])
        elif x.op in ("add", "sub"):
            stack.extend(x.args)
    if len(found) != 1:
        raise LoweringError("a pointer must be one tensor's `source.data_ptr()` plus integer offsets")
    return found.pop()


def effect_targets(program):
    """Parameters written by the program's side effects (scatter stores, pointer stores, atomics)."""
    out = []
    for eff in program.effects:
        if eff[0] == "src_store":
            out.append(eff[1])
        elif eff[0] == "view_store":
            v = eff[1]
            while v.op == "index":
                v = v.args[0]
            out.append(v.args[0])
        else:
            out.append(pointer_param(eff[1]))
    return out


def lower(application, params, unroll=None):
    """Lower ``application`` for parameters described by ``params`` (ParamInfo list);
    with ``unroll`` (trip Value -> int or None), loops with a known trip count are unrolled."""
    return Lowerer(application, params, unroll=unroll).lower()
