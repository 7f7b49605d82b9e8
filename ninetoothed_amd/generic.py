"""Generic kernels: element-parallel programs that match no hand-written family.

The reference emits source for any arrangement and application through its backends
(``src/ninetoothed/emitters/ssa.py``, ``emitters/cuda.py:245-381``) and compiles it at
run time (``backends/materializers/cuda.py:96-170``).  This module does the same for the
programs whose work is element by element: every tensor is used at its tile level
(``load(x)`` of the whole arranged view), the body is arithmetic, comparisons,
``where``, ``maximum``/``minimum``, casts, ``ntl`` math functions and
``libdevice`` functions on those values and on 0-d scalar parameters, and the results
are stored to arranged outputs.  Such a program computes each element independently,
so the kernel walks the flattened index space of the arranged hierarchy (program grid
and tile levels together) with one lane per element:

  * index maps: for every tensor, the source offset of every element of that space is
    evaluated on the host by the same evaluator the families use
    (``tensor.BoundView.probe``), with the call's strides; masked elements get -1.
    The tables (int32) are built once per bound launcher (shapes, strides, constexprs).
  * the body: the application's value graph is emitted as HIP C++ with the reference's
    typing rules (``src/ninetoothed/frontend/types.py``: ``_promote_dtype``, division
    promotes to at least float32, math functions keep their operand's type, Python
    literals are weakly typed); every value is computed in fp32 (fp64 for float64) and
    rounded to its type after each operation, so fp16/bf16 intermediates round where
    the reference's program rounds them.  Masked loads read the source's ``other`` (or
    0); masked outputs are not written.
  * the source is compiled for gfx950 once per distinct text with hipRTC and launched
    through ``nt_rtc_*`` of libnt_mi355x.so.

Programs with reductions (``ntl.sum/max/min``), ``ntl.dot``, broadcasting subscripts,
``offsets`` index vectors, source pointers and gathers, or loops over tile levels run as
tile programs (``TilePlan``, below): one workgroup per program instance, reductions through
LDS and wave64 shuffles.  Loops with up to ``MAX_UNROLL`` iterations known at the call are
unrolled; longer ones, and those whose trip counts are run-time scalars, run as loops in
the kernel, each loop-carried tile in two LDS buffers (iteration k reads buffer k % 2 and
writes the other), level indices by the loop variable guarded against the level's extent.
What neither form takes raises ``LoweringError``.  An arrangement that
maps several elements to one output element writes it from several lanes (the last write
is unspecified), as the reference's generated programs would.
"""

import copy
import ctypes
import dataclasses
import hashlib
import threading

import numpy as np

from ninetoothed_amd import _lib, jagged
from ninetoothed_amd.errors import KernelLaunchError, LoweringError
from ninetoothed_amd.frontend import Value, effect_targets
from ninetoothed_amd.frontend import pointer_param as frontend_pointer_param

MAX_ELEMENTS = 1 << 26
MAX_UNROLL = 64  # loops of up to this many known iterations are unrolled for the tile kernels; longer ones loop
_CONSTLIKE = ("const", "shape", "source_shape", "source_stride", "level_shape")  # values known at specialisation
# arithmetic on values known at specialisation is folded with Python's semantics, as the
# reference's constexpr arithmetic (so ``x.source.shape[1] - 1`` stays an exact integer)
_FOLD = {"add": lambda a, b: a + b, "sub": lambda a, b: a - b, "mul": lambda a, b: a * b,
         "div": lambda a, b: a / b, "floordiv": lambda a, b: a // b, "mod": lambda a, b: a % b,
         "neg": lambda a: -a}

_ALLOWED = {"load", "const", "param", "add", "sub", "mul", "div", "floordiv", "mod", "neg", "lt", "le", "gt", "ge",
            "eq", "ne", "where", "maximum", "minimum", "math", "libm", "cast", "dtype", "dtype_of", "zeros",
            "full", "offsets", "rand", "randint", "randn", "shape", "source_shape", "level_shape"}

_FLOAT = ("float16", "bfloat16", "float32", "float64")
_INT = ("int8", "int16", "int32", "int64", "uint8")
_RANK = {"bool": 0, "int8": 1, "uint8": 1, "int16": 2, "int32": 3, "int64": 4, "float8_e4m3fn": 5, "float8_e5m2": 5,
         "float16": 6, "bfloat16": 6, "float32": 7, "float64": 8}
_FP8 = ("float8_e4m3fn", "float8_e5m2")

# storage C type, working C type, load expression, store expression (of `v`)
_STORAGE = {
    "float8_e4m3fn": ("unsigned char", "float", "ld_e4m3({})", "st_e4m3({})"),
    "float8_e5m2": ("unsigned char", "float", "ld_e5m2({})", "st_e5m2({})"),
    "float16": ("unsigned short", "float", "ld_f16({})", "st_f16({})"),
    "bfloat16": ("unsigned short", "float", "ld_bf16({})", "st_bf16({})"),
    "float32": ("float", "float", "{}", "{}"),
    "float64": ("double", "double", "{}", "{}"),
    "int8": ("signed char", "long long", "(long long){}", "(signed char){}"),
    "uint8": ("unsigned char", "long long", "(long long){}", "(unsigned char){}"),
    "int16": ("short", "long long", "(long long){}", "(short){}"),
    "int32": ("int", "long long", "(long long){}", "(int){}"),
    "int64": ("long long", "long long", "{}", "{}"),
    "bool": ("bool", "bool", "{}", "{}"),
}

_PRELUDE = r"""
__device__ __forceinline__ float ld_f16(unsigned short b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ unsigned short st_f16(float x) { return __builtin_bit_cast(unsigned short, (_Float16)x); }
__device__ __forceinline__ float r_f16(float x) { return (float)(_Float16)x; }
__device__ __forceinline__ float r_bf16(float x) {
  unsigned u = __builtin_bit_cast(unsigned, x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __builtin_bit_cast(float, (u | 0x00400000u) & 0xffff0000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __builtin_bit_cast(float, u & 0xffff0000u);
}
// ntl.rand / randint / randn: Philox4x32-10 (Salmon et al., SC'11) on the counter
// (offset, 0, 0, 0) keyed by the 64-bit seed, as Triton's tl.rand family.
__device__ __forceinline__ void nt_philox(long long seed, long long offset, unsigned (&c)[4]) {
  unsigned k0 = (unsigned)(unsigned long long)seed, k1 = (unsigned)((unsigned long long)seed >> 32);
  c[0] = (unsigned)offset; c[1] = 0u; c[2] = 0u; c[3] = 0u;
  for (int r = 0; r < 10; ++r) {
    const unsigned long long p0 = 0xD2511F53ull * c[0], p1 = 0xCD9E8D57ull * c[2];
    const unsigned n0 = (unsigned)(p1 >> 32) ^ c[1] ^ k0, n2 = (unsigned)(p0 >> 32) ^ c[3] ^ k1;
    c[1] = (unsigned)p1; c[3] = (unsigned)p0; c[0] = n0; c[2] = n2;
    k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
  }
}
__device__ __forceinline__ float nt_uniform(unsigned w) {  // [0, 1): |int32| folded, times ~2^-31
  const int x = (int)w;
  return (float)(x < 0 ? ~x : x) * 4.6566127342e-10f;
}
__device__ __forceinline__ long long nt_randint(long long seed, long long offset) {
  unsigned c[4]; nt_philox(seed, offset, c); return (long long)c[0];
}
__device__ __forceinline__ float nt_rand(long long seed, long long offset) {
  unsigned c[4]; nt_philox(seed, offset, c); return nt_uniform(c[0]);
}
__device__ __forceinline__ float nt_randn(long long seed, long long offset) {
  unsigned c[4]; nt_philox(seed, offset, c);
  const float u1 = fmaxf(nt_uniform(c[0]), 1e-7f), u2 = nt_uniform(c[1]);
  return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}
__device__ __forceinline__ float ld_bf16(unsigned short b) { return __builtin_bit_cast(float, (unsigned)b << 16); }
typedef _Float16 nt_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 nt_bf16x8 __attribute__((ext_vector_type(8)));
typedef float nt_floatx16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ unsigned short st_bf16(float x) { return (unsigned short)(__builtin_bit_cast(unsigned, r_bf16(x)) >> 16); }
// fp8 (OCP formats, as torch's float8_e4m3fn and float8_e5m2): round to nearest, ties to
// even, on the exact value; e4m3fn has no infinity, so magnitudes from 480 (the midpoint
// past its largest value, 448) and NaN encode as NaN (0x7f with the sign); e5m2 rounds
// magnitudes from 61440 (the midpoint past 57344) to infinity.  Below the smallest normal
// the step is the subnormal quantum (2^-9 and 2^-16); a step that carries into the next
// binade gives that binade's first code, as the encodings are consecutive.
__device__ __forceinline__ unsigned char st_e4m3(float x) {
  const unsigned char sign = (unsigned char)((__builtin_bit_cast(unsigned, x) >> 24) & 0x80u);
  const float a = __builtin_fabsf(x);
  if (!(a < 480.0f)) return sign | 0x7f;
  if (a < 0.015625f) return sign | (unsigned char)__builtin_rintf(a * 512.0f);
  int e;
  const float m = __builtin_frexpf(a, &e);  // a = m 2^e, m in [0.5, 1)
  return sign | (unsigned char)((e + 6) * 8 + (int)__builtin_rintf((2.0f * m - 1.0f) * 8.0f));
}
__device__ __forceinline__ unsigned char st_e5m2(float x) {
  const unsigned char sign = (unsigned char)((__builtin_bit_cast(unsigned, x) >> 24) & 0x80u);
  const float a = __builtin_fabsf(x);
  if (a != a) return sign | 0x7f;
  if (a >= 61440.0f) return sign | 0x7c;
  if (a < 6.103515625e-05f) return sign | (unsigned char)__builtin_rintf(a * 65536.0f);
  int e;
  const float m = __builtin_frexpf(a, &e);
  return sign | (unsigned char)((e + 14) * 4 + (int)__builtin_rintf((2.0f * m - 1.0f) * 4.0f));
}
__device__ __forceinline__ float ld_e4m3(unsigned char b) {
  const int E = (b >> 3) & 15, M = b & 7;
  const float v = (E == 15 && M == 7) ? __builtin_nanf("") : (E == 0 ? __builtin_ldexpf((float)M, -9)
                                                                    : __builtin_ldexpf((float)(8 + M), E - 10));
  return (b & 0x80) ? -v : v;
}
__device__ __forceinline__ float ld_e5m2(unsigned char b) {  // the top byte of an fp16
  return (float)__builtin_bit_cast(_Float16, (unsigned short)((unsigned)b << 8));
}
__device__ __forceinline__ float r_e4m3(float x) { return ld_e4m3(st_e4m3(x)); }
__device__ __forceinline__ float r_e5m2(float x) { return ld_e5m2(st_e5m2(x)); }
"""

# ntl math functions (unary) and libdevice functions: C names for float / double
_MATH = {
    "exp": ("expf", "exp"), "exp2": ("exp2f", "exp2"), "log": ("logf", "log"), "log2": ("log2f", "log2"),
    "sqrt": ("sqrtf", "sqrt"), "rsqrt": ("rsqrtf", "rsqrt"), "abs": ("fabsf", "fabs"), "expm1": ("expm1f", "expm1"),
    "log10": ("log10f", "log10"), "log1p": ("log1pf", "log1p"), "sin": ("sinf", "sin"), "cos": ("cosf", "cos"),
    "tan": ("tanf", "tan"), "tanh": ("tanhf", "tanh"), "sinh": ("sinhf", "sinh"), "cosh": ("coshf", "cosh"),
    "asin": ("asinf", "asin"), "acos": ("acosf", "acos"), "atan": ("atanf", "atan"), "erf": ("erff", "erf"),
    "floor": ("floorf", "floor"), "ceil": ("ceilf", "ceil"), "trunc": ("truncf", "trunc"),
    "round": ("roundf", "round"), "fabs": ("fabsf", "fabs"), "pow": ("powf", "pow"), "atan2": ("atan2f", "atan2"),
    "fmax": ("fmaxf", "fmax"), "fmin": ("fminf", "fmin"), "fmod": ("fmodf", "fmod"), "hypot": ("hypotf", "hypot"),
}


def _torch_dtype_name(dtype):
    name = str(dtype).replace("torch.", "")
    if name == "bool":
        return "bool"
    if name not in _RANK:
        raise LoweringError(f"the generic kernels do not support tensors of dtype {dtype}")
    return name


def _promote(a, b):
    if a == "weak":
        return b if b != "weak" else "weak"
    if b == "weak":
        return a
    if a == b:
        return a
    if {a, b} == {"float16", "bfloat16"}:
        return "float32"
    return a if _RANK[a] >= _RANK[b] else b


def _walk(values):
    """Values reachable from ``values`` (dependencies first)."""
    order, seen = [], set()

    def visit(v):
        if not isinstance(v, Value) or id(v) in seen:
            return
        seen.add(id(v))
        for a in v.args:
            if isinstance(a, tuple):
                for x in a:
                    visit(x)
            else:
                visit(a)
        order.append(v)

    for v in values:
        visit(v)
    return order


class _Emitter:
    """Typed HIP C++ for the value graph of an element-parallel program."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.types = {}  # id(value) -> dtype name, "weak" or "bool"
        self.names = {}  # id(value) -> C expression / variable
        self.lines = []
        self.tensors = []  # loaded tensor params, in argument order
        self.scalars = []  # 0-d scalar params, in argument order
        self.offsets = []  # (tensor param, source dim) whose per-element offsets the body reads

    def tensor_dtype(self, name):
        return _torch_dtype_name(self.ctx.dtypes[name])

    def scalar_type(self, name):
        """0-d run-time parameters: Python ints are int64, everything else float32."""
        value = self.ctx.values[name]
        return "int64" if isinstance(value, int) and not isinstance(value, bool) else "float32"

    def dtype_name(self, d):
        if d.op == "dtype":
            return d.args[0]
        view = d.args[0]
        while view.op in ("index", "dtype_of"):
            view = view.args[0]
        return self.tensor_dtype(view.args[0])

    @staticmethod
    def ctx_const(value):
        return Value("const", (float(value),))

    def type_of(self, v):
        if not isinstance(v, Value):
            return "weak"
        return self.types[id(v)]

    def work(self, t):
        return _STORAGE["float32" if t == "weak" else t][1]

    def round_to(self, t, expr):
        if t == "float16":
            return f"r_f16({expr})"
        if t == "bfloat16":
            return f"r_bf16({expr})"
        if t == "float8_e4m3fn":
            return f"r_e4m3({expr})"
        if t == "float8_e5m2":
            return f"r_e5m2({expr})"
        return expr

    def const_value(self, v):
        """The Python value of a constant, ``x.shape[d]`` or ``x.source.shape[d]``; None otherwise."""
        if v.op == "const":
            return v.args[0]
        if v.op == "shape":
            view, d = v.args
            level = 1
            while view.op == "index":
                view, level = view.args[0], level + 1
            return int(self.ctx.views[view.args[0]].level_shapes[level][d])
        if v.op == "source_shape":
            return int(self.ctx.views[v.args[0]].source_shape[v.args[1]])
        if v.op == "source_stride":
            return int(self.ctx.values[v.args[0]].stride(v.args[1]))
        if v.op == "level_shape":
            return int(self.ctx.views[v.args[0]].level_shapes[v.args[1]][v.args[2]])
        if v.op in _FOLD:
            memo = self.__dict__.setdefault("_folded", {})
            if id(v) not in memo:
                xs = [self.const_value(a) if isinstance(a, Value) else a for a in v.args]
                c = None
                if all(isinstance(x, (int, float)) and not isinstance(x, bool) for x in xs):
                    try:
                        c = _FOLD[v.op](*xs)
                    except (ZeroDivisionError, OverflowError):
                        c = None
                memo[id(v)] = (v, c)  # the value is kept so that its id stays its own
            return memo[id(v)][1]
        return None

    def is_const(self, v):
        """Whether ``v`` is known at specialisation (a constant, a shape, or arithmetic on them)."""
        return v.op in _CONSTLIKE or (v.op in _FOLD and self.const_value(v) is not None)

    def operand(self, v, t):
        """Operand ``v`` as a value of working type for an operation in type ``t``."""
        if self.is_const(v):
            c = self.const_value(v)
            if isinstance(c, bool):
                return "true" if c else "false"
            w = self.work(t)
            if w == "long long":
                return f"((long long){int(c)})"
            if w == "bool":
                return "true" if c else "false"
            lit = repr(float(c))
            if lit in ("inf", "-inf", "nan"):
                lit = {"inf": "__builtin_huge_valf()", "-inf": "(-__builtin_huge_valf())", "nan": "__builtin_nanf(\"\")"}[lit]
                if w == "double":
                    lit = f"((double){lit})"
            elif w == "float":
                lit += "f"
            return self.round_to(t, f"(({w}){lit})")  # weakly typed literal: rounded to the operation's type
        expr = self.names[id(v)]
        src = self.types[id(v)]
        w = self.work(t)
        if self.work(src) != w:
            expr = f"(({w}){expr})"
        return expr

    def define(self, v, t, expr, exact=False):
        name = f"v{len(self.names)}"
        self.lines.append(f"    const {self.work(t)} {name} = {expr if exact else self.round_to(t, expr)};")
        self.names[id(v)] = name
        self.types[id(v)] = t

    def emit(self, v):
        op, args = v.op, v.args
        if self.is_const(v):
            self.types[id(v)] = "bool" if isinstance(self.const_value(v), bool) else "weak"
            return
        if op in ("dtype", "dtype_of", "param"):
            return
        if op in ("zeros", "full"):
            t = self.dtype_name(args[-1])
            fill = 0.0 if op == "zeros" else args[1]
            self.define(v, t, self.operand(self.ctx_const(fill), t))
            return
        if op == "load":
            view = args[0]
            if view.op != "param":
                raise LoweringError("the generic kernels load whole arranged tensors only (no level indexing)")
            name = view.args[0]
            info = self.ctx.params[name]
            if info.source_ndim == 0:
                if name not in self.scalars:
                    self.scalars.append(name)
                self.names[id(v)] = f"s_{name}"
                self.types[id(v)] = self.scalar_type(name)
                return
            if name not in self.tensors:
                self.tensors.append(name)
            t = self.tensor_dtype(name)
            st, w, ld, _ = _STORAGE[t]
            other = self.ctx.views[name].source.other
            other = 0.0 if other is None else float(other)
            o = repr(other) if other == other and abs(other) != float("inf") else (
                "__builtin_nanf(\"\")" if other != other else ("__builtin_huge_valf()" if other > 0 else "(-__builtin_huge_valf())"))
            # an element of the tensor, or `other`, is already a value of type t
            self.define(v, t, f"(i_{name} >= 0 ? ({w}){ld.format(f'p_{name}[i_{name}]')} : ({w}){o})", exact=True)
            return
        if op in ("add", "sub", "mul", "div", "floordiv", "mod", "maximum", "minimum"):
            a, b = args
            t = _promote(self.type_of(a), self.type_of(b))
            if t == "weak":
                t = "float32"
            if op == "div" and t not in ("float32", "float64"):
                t = "float32"
            if t == "bool":
                raise LoweringError(f"`{op}` on booleans is not supported")
            x, y = self.operand(a, t), self.operand(b, t)
            w = self.work(t)
            if op == "maximum":
                expr = f"fmax({x}, {y})" if w == "double" else (f"fmaxf({x}, {y})" if w == "float" else f"({x} > {y} ? {x} : {y})")
            elif op == "minimum":
                expr = f"fmin({x}, {y})" if w == "double" else (f"fminf({x}, {y})" if w == "float" else f"({x} < {y} ? {x} : {y})")
            elif op == "floordiv":
                expr = f"floor({x} / {y})" if w != "long long" else f"({x} / {y})"
            elif op == "mod":
                expr = f"fmod({x}, {y})" if w != "long long" else f"({x} % {y})"
            else:
                expr = f"({x} {dict(add='+', sub='-', mul='*', div='/')[op]} {y})"
            self.define(v, t, expr)
            return
        if op == "neg":
            t = self.type_of(args[0])
            t = "float32" if t == "weak" else t
            self.define(v, t, f"(-{self.operand(args[0], t)})")
            return
        if op in ("lt", "le", "gt", "ge", "eq", "ne"):
            a, b = args
            t = _promote(self.type_of(a), self.type_of(b))
            t = "float32" if t == "weak" else t
            sym = dict(lt="<", le="<=", gt=">", ge=">=", eq="==", ne="!=")[op]
            self.define(v, "bool", f"({self.operand(a, t)} {sym} {self.operand(b, t)})")
            return
        if op == "where":
            c, a, b = args
            t = _promote(self.type_of(a), self.type_of(b))
            t = "float32" if t == "weak" else t
            self.define(v, t, f"({self.operand(c, 'bool')} ? {self.operand(a, t)} : {self.operand(b, t)})")
            return
        if op == "cast":
            x, d = args
            t = self.dtype_name(d)
            src = self.type_of(x)
            src = "float32" if src == "weak" else src
            e = self.operand(x, src)
            self.define(v, t, f"(({self.work(t)}){e})")
            return
        if op in ("math", "libm"):
            fname = args[0]
            operands = (args[1],) if op == "math" else args[1]
            if op == "math" and fname == "sigmoid":
                t = self.type_of(operands[0])
                t = "float32" if t in ("weak", "bool") or t not in _FLOAT else t
                x = self.operand(operands[0], t)
                one = "1.0" if self.work(t) == "double" else "1.0f"
                ex = "exp" if self.work(t) == "double" else "expf"
                self.define(v, t, f"({one} / ({one} + {ex}(-{x})))")
                return
            if fname not in _MATH:
                raise LoweringError(f"math function `{fname}` is not supported by the generic kernels")
            t = "weak"
            for o in operands:
                t = _promote(t, self.type_of(o))
            if t in ("weak", "bool") or t not in _FLOAT:
                t = "float32"
            cf = _MATH[fname][1 if self.work(t) == "double" else 0]
            self.define(v, t, f"{cf}({', '.join(self.operand(o, t) for o in operands)})")
            return
        if op == "offsets":
            view, d = args
            if view.op != "param":
                raise LoweringError("the generic kernels take `offsets` of whole arranged tensors only")
            key = (view.args[0], int(d))
            if key not in self.offsets:
                self.offsets.append(key)
            self.names[id(v)] = f"q_{key[0]}_{key[1]}"
            self.types[id(v)] = "int32"
            return
        if op in ("rand", "randint", "randn"):
            seed, off = self.operand(args[0], "int64"), self.operand(args[1], "int64")
            self.define(v, "int64" if op == "randint" else "float32", f"nt_{op}({seed}, {off})", exact=True)
            return
        raise LoweringError(f"operation `{op}` is not supported by the generic kernels")


def _analyse(ctx):
    """(stores, ordered values, output names, loaded names) or None if the program is not element-parallel."""
    program = ctx.program
    if program.loops or program.effects:
        return None
    stores = program.stores
    values = _walk(list(stores.values()))
    for v in values:
        if v.op not in _ALLOWED:
            return None
        if v.op == "load" and v.args[0].op != "param":
            return None
        if v.op == "offsets" and v.args[0].op != "param":
            return None
    tensors = [n for n in list(stores) + [v.args[0].args[0] for v in values if v.op in ("load", "offsets")]
               if ctx.params[n].source_ndim != 0]
    shapes = {tuple(ctx.views[n].level_shapes) for n in tensors}
    if len(shapes) > 1:
        return None
    for n in stores:
        if ctx.params[n].source_ndim == 0:
            return None
    return stores, values


class GenericPlan:
    """A bound generic kernel (see the module docstring)."""

    family = "generic"
    _lock = threading.Lock()
    _functions = {}  # source digest -> loaded kernel handle
    _blobs = {}  # source digest -> code object (compiled here, or carried by a built artifact)

    def check(self, values):
        """The generic kernels take every dtype and size their emitter accepted."""

    def __init__(self, ctx, stores, values):
        self.ctx = ctx
        self.stores = stores
        em = _Emitter(ctx)
        for v in values:
            em.emit(v)
        self.loaded = list(em.tensors)
        self.scalars = list(em.scalars)
        self.offsets = list(em.offsets)
        self.outputs = list(stores)
        lines = []
        for out, v in stores.items():
            t = _torch_dtype_name(ctx.dtypes[out])
            src = em.type_of(v)
            src = "float32" if src == "weak" else src
            val = em.operand(v, src) if em.is_const(v) else em.names[id(v)]
            if em.work(src) != em.work(t):
                val = f"(({em.work(t)}){val})"
            lines.append(f"    if (o_{out} >= 0) p_{out}[o_{out}] = {_STORAGE[t][3].format(val)};")
        self.body = em.lines
        self.store_lines = lines
        self.index_names = list(dict.fromkeys(self.outputs + self.loaded))
        params = []
        for n in self.index_names:
            params.append(f"const int* __restrict__ t_{n}")
        for n, d in self.offsets:
            params.append(f"const int* __restrict__ f_{n}_{d}")
        for n in self.loaded:
            if n not in self.outputs:
                params.append(f"const {_STORAGE[_torch_dtype_name(ctx.dtypes[n])][0]}* __restrict__ p_{n}")
        for n in self.outputs:
            params.append(f"{_STORAGE[_torch_dtype_name(ctx.dtypes[n])][0]}* p_{n}")
        self.scalar_types = {n: em.scalar_type(n) for n in self.scalars}
        for n in self.scalars:
            params.append(f"{_STORAGE[self.scalar_types[n]][0]} s_{n}")
        params.append("long long total")
        self.params = params
        self.kernel_name = "nt_generic"

    def source(self, linear=None, linear_offsets=()):
        """Kernel source; ``linear[name] = n`` marks a tensor whose index table is e for e < n, -1 after;
        ``linear_offsets`` the (tensor, dim) offsets tables that equal e."""
        linear = linear or {}

        def index(n):
            return f"(e < {linear[n]}LL ? (int)e : -1)" if n in linear else f"t_{n}[e]"

        head = [f"    const int i_{n} = {index(n)};" for n in self.loaded]
        head += [f"    const int o_{n} = {index(n)};" for n in self.outputs]
        head += [f"    const long long q_{n}_{d} = {'e' if (n, d) in linear_offsets else f'(long long)f_{n}_{d}[e]'};"
                 for n, d in self.offsets]
        return (
            _PRELUDE
            + f'\nextern "C" __global__ void __launch_bounds__(256) {self.kernel_name}({", ".join(self.params)}) {{\n'
            + "  for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < total;"
            + " e += (long long)gridDim.x * 256) {\n"
            + "\n".join(head + self.body + self.store_lines)
            + "\n  }\n}\n"
        )

    def describe(self):
        return {"family": self.family, "outputs": self.outputs, "inputs": self.loaded, "scalars": self.scalars}

    # ------------------------------------------------------------ compile, tables, launch
    @classmethod
    def compile(cls, source):
        """Code object for ``source`` (hipRTC, gfx950); raises LoweringError with the log."""
        lib = _lib.load()
        code, size = ctypes.c_void_p(), ctypes.c_int64()
        log = ctypes.create_string_buffer(16384)
        status = lib.nt_rtc_compile(source.encode(), b"nt_generic.hip", ctypes.byref(code), ctypes.byref(size), log,
                                    len(log))
        if status != 0:
            raise LoweringError(f"hipRTC could not compile the generic kernel:\n{log.value.decode(errors='replace')}")
        try:
            return ctypes.string_at(code, size.value)
        finally:
            lib.nt_rtc_free(code)

    @staticmethod
    def digest(source):
        return hashlib.sha256(source.encode()).hexdigest()

    @classmethod
    def code_object(cls, source):
        """The code object of ``source``: from the cache, else compiled (needs no GPU)."""
        digest = cls.digest(source)
        with cls._lock:
            blob = cls._blobs.get(digest)
        if blob is None:
            blob = cls.compile(source)
            with cls._lock:
                cls._blobs[digest] = blob
        return blob

    def sources_for(self, values):
        """The kernel sources a call with ``values`` runs (strides decide the index tables)."""
        if not self.index_names:
            return []
        linear, linear_offsets = self._layout(values)[1:3]
        return [self.source(linear, linear_offsets)]

    def function(self, source):
        digest = self.digest(source)
        blob = self.code_object(source)
        with self._lock:
            fn = self._functions.get(digest)
            if fn is None:
                handle = ctypes.c_void_p()
                buf = ctypes.create_string_buffer(blob, len(blob))
                status = _lib.load().nt_rtc_load(buf, self.kernel_name.encode(), ctypes.byref(handle))
                if status != 0:
                    raise KernelLaunchError(status)
                fn = handle
                self._functions[digest] = fn
        return fn

    def _maps(self, name):
        """(source index arrays, mask, flattened level shape) of every element of ``name``'s arrangement."""
        view = self.ctx.views[name]
        shape = tuple(s for level in view.level_shapes for s in level)
        total = int(np.prod(shape)) if shape else 1
        if total > MAX_ELEMENTS:
            raise LoweringError(f"the generic kernels index at most {MAX_ELEMENTS} elements per launch ({total} here)")
        idx, mask = view.probe(view.full_index())
        return idx, mask, shape

    def _table(self, name, tensor, maps=None):
        idx, mask, shape = maps or self._maps(name)
        total = int(np.prod(shape)) if shape else 1
        if jagged.is_jagged(tensor):  # offsets into values(), masked past each batch's rows
            off, mask = jagged.element_offsets(tensor, idx, mask)
        else:
            off = np.zeros((), dtype=np.int64)
            for i, st in zip(idx, tensor.stride()):
                off = off + np.asarray(i, dtype=np.int64) * int(st)
        off = np.broadcast_to(np.where(mask, off, -1), shape).reshape(-1)
        if off.size and off.max() >= 2**31:
            raise LoweringError("the generic kernels address at most 2^31 elements of a tensor")
        return off.astype(np.int32), total

    def _offsets_table(self, name, dim, maps=None):
        """Source index along ``dim`` of every element (masked ones included), as ``offsets(dim)`` reads it."""
        idx, _, shape = maps or self._maps(name)
        q = np.broadcast_to(np.asarray(idx[dim], dtype=np.int64), shape).reshape(-1)
        if q.size and (q.max() >= 2**31 or q.min() < -(2**31)):
            raise LoweringError("the generic kernels take offsets within 32 bits")
        return q.astype(np.int32)

    def _layout(self, values):
        """Host index tables, the tensors walked linearly (no table), offsets tables, and the
        size of the index space."""
        tables, linear, total, maps = {}, {}, None, {}
        for n in self.index_names:
            maps[n] = self._maps(n)
            tab, tot = self._table(n, values[n], maps[n])
            if total is not None and tot != total:
                raise LoweringError("generic kernel operands do not share one index space")
            total = tot
            valid = int(np.count_nonzero(tab >= 0))
            if np.array_equal(tab[:valid], np.arange(valid, dtype=np.int32)) and not np.any(tab[valid:] >= 0):
                linear[n] = valid  # e -> e, masked from `valid` on: no table
            else:
                tables[n] = tab
        if tables and not self.offsets:
            # Every operand indexed by one table that is a permutation of 0..n-1: an
            # element-parallel program may visit the elements in memory order instead.
            ref = next(iter(tables.values()))
            same = all(np.array_equal(t, ref) for t in tables.values()) and len(tables) == len(self.index_names)
            if same:
                valid = ref[ref >= 0]
                if np.array_equal(np.sort(valid), np.arange(valid.size, dtype=valid.dtype)):
                    return {}, {n: int(valid.size) for n in self.index_names}, set(), {}, int(valid.size)
        offset_tables, linear_offsets = {}, set()
        for n, d in self.offsets:
            q = self._offsets_table(n, d, maps.get(n))
            if q.size != total:
                raise LoweringError("generic kernel operands do not share one index space")
            if np.array_equal(q, np.arange(q.size, dtype=np.int32)):
                linear_offsets.add((n, d))
            else:
                offset_tables[(n, d)] = q
        return tables, linear, linear_offsets, offset_tables, total

    def launch_spec(self, values):
        """One launch of this plan on ``values``: (kernel source, grid, kernel arguments in
        parameter order), or None when the program stores nothing.  An argument is ("table",
        int32 array, or None for a tensor walked linearly), ("tensor", name), ("scalar", name,
        "int64" or "float32") or ("i64", value)."""
        if not self.index_names:
            return None
        host_tables, linear, linear_offsets, host_offsets, total = self._layout(values)
        args = [("table", host_tables.get(n)) for n in self.index_names]
        args += [("table", host_offsets.get(k)) for k in self.offsets]
        args += [("tensor", n) for n in self.loaded if n not in self.outputs]
        args += [("tensor", n) for n in self.outputs]
        args += [("scalar", n, "int64" if self.scalar_types[n] == "int64" else "float32") for n in self.scalars]
        args.append(("i64", total))
        grid = max(1, min((total + 255) // 256, 256 * 64)) if total else 0
        return self.source(linear, linear_offsets), grid, args

    def bind(self, values, index):
        import torch

        spec = self.launch_spec(values)
        if spec is None:  # nothing is stored: the program has no effect
            return lambda args: None
        source, grid, spec_args = spec
        device = next(values[a[1]].device for a in spec_args if a[0] == "tensor")
        fn = self.function(source)
        tables, argv, ptrs, svals = [], [], [], {}
        for a in spec_args:
            if a[0] == "table":
                t = torch.from_numpy(a[1]).to(device) if a[1] is not None else None
                tables.append(t)
                argv.append(ctypes.c_void_p(t.data_ptr() if t is not None else None))
            elif a[0] == "tensor":
                slot = ctypes.c_void_p()
                ptrs.append((index[a[1]], slot))
                argv.append(slot)
            elif a[0] == "scalar":
                slot = ctypes.c_int64() if a[2] == "int64" else ctypes.c_float()
                svals[a[1]] = (index[a[1]], slot, a[2])
                argv.append(slot)
            else:
                argv.append(ctypes.c_int64(a[1]))
        params = (ctypes.c_void_p * len(argv))(*[ctypes.addressof(a) for a in argv])
        lib = _lib.load()

        def launch(args):
            for p, slot in ptrs:
                slot.value = jagged.data_ptr(args[p])
            for p, slot, kind in svals.values():
                v = args[p]
                v = v.item() if hasattr(v, "item") else v
                slot.value = int(v) if kind == "int64" else float(v)
            status = lib.nt_rtc_launch(fn, grid, 256, params, ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
            if status != 0:
                raise KernelLaunchError(status)

        launch.keep = (tables, argv, params)  # device tables and the argument block live with the launcher
        return launch

    def run(self, values):
        names = tuple(values)
        self.bind(values, {n: i for i, n in enumerate(names)})(tuple(values[n] for n in names))


# ============================================================================ tile programs
# Programs with reductions (``ntl.sum/max/min``) or broadcasting subscripts run one
# workgroup per program instance: reductions first, in dependency order, each into an LDS
# array (groups of G lanes per output element stride the reduced axis and combine with
# wave64 shuffles), then every output tile element by element.  Values between them are
# recomputed at the coordinates where they are read (loads through the index tables,
# reduction results from LDS).  A reduction operand element counts only where the load
# masks of every tensor it is computed from hold, else it is the reduction's identity
# (reference src/ninetoothed/backends/emitters/ssa.py:1834-1910, 2180-2210).

_TILE_ALLOWED = _ALLOWED | {"reduce", "mdot", "bcast", "ptr", "source_stride", "src_load", "ptr_load", "index",
                            "unmask", "loop_index", "carried", "loop_out"}
LDS_BYTES = 64 * 1024
_INT_LIMITS = {"int8": (-128, 127), "uint8": (0, 255), "int16": (-32768, 32767), "int32": (-(2**31), 2**31 - 1),
               "int64": (-(2**63), 2**63 - 1)}


def _value_operands(v):
    if v.op == "src_load":
        return list(v.args[1])
    if v.op == "ptr_load":
        return [v.args[0]]
    if v.op in ("ptr", "source_stride"):
        return []
    if v.op == "math":
        return [v.args[1]]
    if v.op == "libm":
        return list(v.args[1])
    if v.op in ("cast", "bcast", "unmask"):
        return [v.args[0]]
    if v.op == "load":  # the level indices that are values
        chain = _view_chain(v.args[0])
        return [k for k in chain[1] if isinstance(k, Value)] if chain else []
    if v.op in ("offsets", "reduce", "mdot", "const", "shape", "source_shape", "level_shape", "zeros", "full", "param",
                "dtype", "dtype_of", "loop_index", "carried", "loop_out"):
        return []
    return [a for a in v.args if isinstance(a, Value)]


def _view_chain(view):
    """(param, level indices) of ``param[k0][k1]...``, or None: constant indices as ints,
    the others (a loop index, a scalar parameter, an expression of them) as their values."""
    ks = []
    while view.op == "index":
        k = view.args[1]
        if not isinstance(k, Value):
            return None
        ks.append(k.args[0] if k.op == "const" and isinstance(k.args[0], int) else k)
        view = view.args[0]
    if view.op != "param":
        return None
    return view.args[0], tuple(reversed(ks))


def _bcast_shapes(*shapes):
    try:
        return tuple(int(x) for x in np.broadcast_shapes(*shapes))
    except ValueError:
        raise LoweringError(f"shapes {shapes} do not broadcast") from None


def _tile_shape(ctx, name):
    ls = ctx.views[name].level_shapes
    return tuple(ls[1]) if len(ls) > 1 else ()


def _shapes(ctx, values, const_value, carried=None):
    """Tile shape of every value: loads have their tensor's tile shape, reductions drop
    their axis (all axes for ``axis=None``), ``x[:, None]`` inserts unit dims, and
    elementwise operations broadcast as numpy does (right-aligned).  ``carried[(loop, name)]``
    is the shape of a loop-carried value (and of the loop's result)."""
    shp = {}
    for v in values:
        op, a = v.op, v.args
        if op in ("const", "dtype", "dtype_of", "shape", "source_shape", "source_stride", "level_shape", "param", "ptr",
                  "loop_index"):
            s = ()
        elif op in ("carried", "loop_out"):
            s = carried[(a[0], a[1])]
        elif op == "mdot":  # (x, y, x transposed, y transposed)
            sx, sy = shp[id(a[0])], shp[id(a[1])]
            s = ((sx[1] if a[2] else sx[0]), (sy[0] if a[3] else sy[1]))
        elif op == "load":
            name, ks = _view_chain(a[0])
            levels = ctx.views[name].level_shapes if ctx.params[name].source_ndim != 0 else []
            s = () if not levels else (tuple(levels[1 + len(ks)]) if 1 + len(ks) < len(levels) else ())
        elif op == "offsets":
            tile = _tile_shape(ctx, a[0].args[0])
            if len(tile) != ctx.params[a[0].args[0]].source_ndim:
                raise LoweringError("`offsets` in a tile program needs a tile with one dim per source dim")
            s = (tile[int(a[1])],) if tile else ()
        elif op == "reduce":
            src, axis = shp[id(a[1])], a[2]
            if axis is None:
                s = ()
            else:
                ax = axis + len(src) if axis < 0 else axis
                if not 0 <= ax < len(src):
                    raise LoweringError(f"reduction axis {axis} of a {len(src)}-D value")
                s = src[:ax] + src[ax + 1:]
        elif op == "bcast":
            src, pattern = list(shp[id(a[0])]), a[1]
            if any(isinstance(x, int) for x in pattern):  # axes named: a broadcast with the axes permuted
                if sorted(x for x in pattern if x is not None) != list(range(len(src))):
                    raise LoweringError("a permuting broadcast names every source axis once")
                s = tuple(src[x] if x is not None else 1 for x in pattern)
            else:
                if sum(1 for x in pattern if x == ":") != len(src):
                    raise LoweringError("a broadcasting subscript needs one `:` per dimension")
                it = iter(src)
                s = tuple(next(it) if x == ":" else 1 for x in pattern)
        elif op in ("zeros", "full"):
            dims = []
            for d in a[0]:
                c = const_value(d) if isinstance(d, Value) else d
                if not isinstance(c, int):
                    raise LoweringError("zeros/full need constant shapes")
                dims.append(c)
            s = tuple(dims)
        else:
            s = _bcast_shapes(*[shp[id(x)] for x in _value_operands(v)]) if _value_operands(v) else ()
        shp[id(v)] = s
    return shp


def _unravel(idx, shape):
    """C expressions of the coordinates of row-major element ``idx`` of ``shape``."""
    coords, stride = [], 1
    for size in reversed(shape):
        if size == 1:
            coords.append("0")
        else:
            coords.append(f"(({idx} / {stride}LL) % {size}LL)" if stride > 1 else f"({idx} % {size}LL)")
        stride *= size
    return tuple(reversed(coords))


def _ravel(coords, shape):
    terms, stride = [], 1
    for c, size in zip(reversed(coords), reversed(shape)):
        if size != 1:
            terms.append(f"{c} * {stride}LL" if stride > 1 else f"{c}")
        stride *= size
    return " + ".join(reversed(terms)) if terms else "0"


class _TileEmitter(_Emitter):
    """Code for one evaluation context: a root value at given coordinates, and every value
    it is computed from at the coordinates that implies."""

    def __init__(self, plan):
        super().__init__(plan.ctx)
        self.plan = plan
        self.types = plan.types
        self.shapes = plan.shapes

    def context(self, root, coords, tag, more=()):
        """Lines computing ``root`` at ``coords`` (and each (value, coords) of ``more``)."""
        self.names, self.lines, self.coords, self.masks, self.tag = {}, [], {}, {}, tag
        self.ptrs = {}
        self._assign(root, tuple(coords))
        for extra, extra_coords in more:
            self._assign(extra, tuple(extra_coords))
        for v in _walk([root] + [m[0] for m in more]):
            if id(v) in self.coords:
                self.emit(v)
        return self.lines

    def _canon(self, v, coords):
        return tuple("0" if size == 1 else c for size, c in zip(self.shapes[id(v)], coords))

    def _assign(self, v, coords):
        coords = self._canon(v, coords)
        prev = self.coords.get(id(v))
        if prev is not None:
            if prev != coords:
                raise LoweringError("a value is read at two different broadcast positions in one expression")
            return
        self.coords[id(v)] = coords
        if v.op == "bcast":
            pattern = v.args[1]
            if any(isinstance(x, int) for x in pattern):  # source axis x at this position
                src = [None] * sum(1 for x in pattern if x is not None)
                for c, x in zip(coords, pattern):
                    if x is not None:
                        src[x] = c
                self._assign(v.args[0], tuple(src))
            else:
                self._assign(v.args[0], tuple(c for c, x in zip(coords, pattern) if x == ":"))
            return
        for a in _value_operands(v):
            sa = self.shapes[id(a)]
            aligned = coords[len(coords) - len(sa):] if sa else ()
            self._assign(a, aligned)

    def define(self, v, t, expr, exact=False):
        name = f"{self.tag}{len(self.names)}"
        self.lines.append(f"      const {self.work(t)} {name} = {expr if exact else self.round_to(t, expr)};")
        self.names[id(v)] = name
        self.types[id(v)] = t

    def emit(self, v):
        op, args = v.op, v.args
        if self.emit_pointer(v):
            return
        if op == "ptr_load":
            if not self.is_pointer(args[0]):
                raise LoweringError("ntl.load needs a `source.data_ptr()` pointer")
            name, off = self.ptrs[id(args[0])]
            ox = off  # bounds: inside the tensor's storage extent, else 0
            self.raw_load(v, name, ox, f"({ox}) >= 0 && ({ox}) < {self.plan.extent(name)}LL")
            self.masks[id(v)] = frozenset()
            return
        if op == "src_load":
            name, indices = args
            off, cond = self.source_offset(name, indices)
            self.raw_load(v, name, off, cond)
            self.masks[id(v)] = frozenset([f"({cond})"])
            return
        chain = _view_chain(args[0]) if op == "load" else None
        if chain is not None and self.ctx.params[chain[0]].source_ndim != 0:
            name, ks = chain
            t = self.tensor_dtype(name)
            st, w, ld, _ = _STORAGE[t]
            entry = self.plan.level_index(name, ks, _ravel(self.coords[id(v)], self.shapes[id(v)]), self)
            ix = f"{self.tag}x{len(self.names)}"
            self.lines.append(f"      const int {ix} = {entry};")
            other = self.ctx.views[name].source.other
            other = 0.0 if other is None else float(other)
            o = repr(other) if other == other and abs(other) != float("inf") else (
                "__builtin_nanf(\"\")" if other != other else ("__builtin_huge_valf()" if other > 0 else "(-__builtin_huge_valf())"))
            self.define(v, t, f"({ix} >= 0 ? ({w}){ld.format(f'p_{name}[{ix}]')} : ({w}){o})", exact=True)
            self.masks[id(v)] = frozenset([f"({ix} >= 0)"])
            return
        if op == "offsets":
            name, d = args[0].args[0], int(args[1])
            lin = _ravel(self.coords[id(v)], self.shapes[id(v)])
            self.names[id(v)] = f"(long long)f_{name}_{d}[pbo_{name}_{d} + {lin}]"
            self.types[id(v)] = "int32"
            self.masks[id(v)] = frozenset()
            return
        if op in ("reduce", "mdot"):
            arr, oshape = self.plan.lds[id(v)]
            self.names[id(v)] = f"{arr}[{_ravel(self.coords[id(v)], oshape)}]"
            self.masks[id(v)] = frozenset()
            return
        if op == "bcast":
            self.names[id(v)] = self.names[id(args[0])]
            self.types[id(v)] = self.types[id(args[0])]
            self.masks[id(v)] = self.masks.get(id(args[0]), frozenset())
            return
        if op == "loop_index":
            self.names[id(v)] = f"li{args[0]}"
            self.types[id(v)] = "int32"
            self.masks[id(v)] = frozenset()
            return
        if op in ("carried", "loop_out"):  # this iteration's buffer, or the one the loop ended in
            i, n = args
            arr, size = self.plan.carried_arrays[(i, n)]
            buffer = f"pp{i}" if op == "carried" else f"po{i}"
            self.names[id(v)] = f"{arr}[{buffer} * {size}LL + {_ravel(self.coords[id(v)], self.shapes[id(v)])}]"
            self.types[id(v)] = self.plan.carried_type((i, n))
            self.masks[id(v)] = frozenset()  # as a loop's values: no load mask
            return
        if op == "unmask":  # a loop-carried value: the same value, no load mask
            self.names[id(v)] = self.names[id(args[0])]
            self.types[id(v)] = self.types[id(args[0])]
            self.masks[id(v)] = frozenset()
            return
        if op in ("zeros", "full"):
            t = self.dtype_name(args[-1])
            fill = 0.0 if op == "zeros" else args[1]
            self.define(v, t, self.operand(self.ctx_const(fill), t))
            self.masks[id(v)] = frozenset()
            return
        super().emit(v)
        m = frozenset()
        for a in _value_operands(v):
            m |= self.masks.get(id(a), frozenset())
        self.masks[id(v)] = m

    def mask_of(self, v):
        m = sorted(self.masks.get(id(v), frozenset()))
        return " && ".join(m) if m else None

    def is_pointer(self, v):
        return isinstance(v, Value) and id(v) in self.ptrs

    def source_offset(self, name, indices):
        """(C offset, C bounds condition) of ``source[indices]`` (each index already emitted)."""
        t = self.ctx.values[name]
        terms, conds = [], []
        for d, ix in enumerate(indices):
            e = self.operand(ix, "int64")
            terms.append(f"({e}) * {int(t.stride(d))}LL")
            conds.append(f"({e}) >= 0 && ({e}) < {int(t.shape[d])}LL")
        return " + ".join(terms) or "0LL", " && ".join(f"({c})" for c in conds) or "true"

    def emit_pointer(self, v):
        """Pointer arithmetic: record (tensor, C element offset) instead of a value."""
        if v.op == "ptr":
            self.ptrs[id(v)] = (v.args[0], "0LL")
            return True
        if v.op in ("add", "sub") and any(self.is_pointer(a) for a in v.args):
            a, b = v.args
            if v.op == "sub" and self.is_pointer(b):
                raise LoweringError("a pointer can only be offset, not subtracted from")
            p, q = (a, b) if self.is_pointer(a) else (b, a)
            if self.is_pointer(q):
                raise LoweringError("two pointers cannot be added")
            name, off = self.ptrs[id(p)]
            sign = "-" if v.op == "sub" else "+"
            self.ptrs[id(v)] = (name, f"({off} {sign} {self.operand(q, 'int64')})")
            return True
        return False

    def raw_load(self, v, name, off, cond):
        t = self.tensor_dtype(name)
        st, w, ld, _ = _STORAGE[t]
        ox = f"{self.tag}o{len(self.names)}"
        self.lines.append(f"      const long long {ox} = {off};")
        self.define(v, t, f"(({cond}) ? ({w}){ld.format(f'p_{name}[{ox}]')} : ({w})0)", exact=True)
        self.plan.raw_reads.add(name)


def _static_type(ctx, v):
    """The dtype of a loaded tensor or of a cast, as far as it is known without emitting."""
    if v.op == "load":
        chain = _view_chain(v.args[0])
        if chain is not None and ctx.params[chain[0]].source_ndim != 0:
            return _torch_dtype_name(ctx.dtypes[chain[0]])
    if v.op == "cast":
        d = v.args[1]
        if d.op == "dtype":
            return d.args[0]
        if d.op == "dtype_of":
            view = d.args[0]
            while view.op in ("index", "dtype_of"):
                view = view.args[0]
            return _torch_dtype_name(ctx.dtypes[view.args[0]]) if view.op == "param" else None
    return None


MDOT_LDS = 48 * 1024  # LDS a matrix-core dot may take (staged operands and the fp32 result)


def _mdot_stage_type(tx, ty):
    """The 16-bit type both operands of a matrix-core dot are staged in, or None: bf16 with
    bf16; fp16 and fp8 (e4m3fn, e5m2) in any mix as fp16, which holds every fp8 value exactly,
    so the products and their fp32 sums are those of an fp8 matrix multiply."""
    if tx == ty == "bfloat16":
        return "bfloat16"
    if tx in ("float16",) + _FP8 and ty in ("float16",) + _FP8:
        return "float16"
    return None


def _mdot_fits(ctx, x, y, tx, ty):
    """Whether ``dot`` of (inner) operands x, y runs on the matrix core: both 16-bit floats
    of one type, and the operands padded to M, N multiples of 32 and K of 16 plus the fp32
    result within MDOT_LDS."""
    if _mdot_stage_type(_static_type(ctx, x), _static_type(ctx, y)) is None:
        return False
    try:
        shp = _shapes(ctx, _walk([x, y]), _Emitter(ctx).const_value, {})
    except (KeyError, LoweringError):
        return False
    sx, sy = shp[id(x)], shp[id(y)]
    if len(sx) != 2 or len(sy) != 2:
        return False
    m, k = (sx[1], sx[0]) if tx else sx
    k2, n = (sy[1], sy[0]) if ty else sy
    mp, np_, kp = -(-m // 32) * 32, -(-n // 32) * 32, -(-k // 16) * 16
    return k == k2 and min(m, n, k) > 0 and (mp + np_) * (kp + 8) * 2 + m * n * 4 <= MDOT_LDS


def _lower_dots(program, ctx=None):
    """The program with every ``ntl.dot`` of two tiles rewritten: on the matrix core
    (``mdot``) where ``_mdot_fits``, else as an fp32 reduction.

    ``dot(x, y)`` of an [m, k] and a [k, n] tile is ``sum(x[:, :, None] * y[None, :, :],
    axis=1)`` with both operands first cast to float32 (the reference's ``tl.dot``
    accumulates in fp32 and returns fp32 for 16- and 32-bit floats: reference
    src/ninetoothed/backends/emitters/ssa.py:1455-1542).  A transposed operand takes the
    product in another axis order, so that no value is transposed: ``dot(x, trans(w))``
    with w [n, k] is ``sum(x[:, None, :] * w[None, :, :], axis=2)`` and ``dot(trans(u), y)``
    with u [k, m] is ``sum(u[:, :, None] * y[:, None, :], axis=0)``; ``dot(trans(u),
    trans(w))`` is the same sum over a [k, m, n] product whose w factor is broadcast with its
    axes permuted (a ``bcast`` naming source axes), so again nothing is transposed in memory.
    In every form a product counts only where
    both operands' load masks hold (the reference's dot emitter masks them the same way:
    src/ninetoothed/backends/emitters/ssa.py:1455-1542)."""
    roots = list(program.stores.values())
    for eff in program.effects:
        roots += [a for a in eff[1:] if isinstance(a, Value)] + [x for a in eff[1:] if isinstance(a, tuple)
                                                                    for x in a if isinstance(x, Value)]
    for lp in program.loops.values():
        roots += [lp.trip] + list(lp.init.values()) + list(lp.update.values())
    if not any(v.op == "dot" for v in _walk(roots)):
        return program
    f32 = Value("dtype", ("float32",))
    done = {}

    def rebuild(v):
        if not isinstance(v, Value):
            if isinstance(v, tuple):
                return tuple(rebuild(x) for x in v)
            return v
        if id(v) in done:
            return done[id(v)]
        if v.op == "dot":
            x, y = v.args
            tx, ty = x.op == "trans", y.op == "trans"
            xi, yi = rebuild(x.args[0] if tx else x), rebuild(y.args[0] if ty else y)
            if ctx is not None and _mdot_fits(ctx, xi, yi, tx, ty):
                out = Value("mdot", (xi, yi, tx, ty))
                done[id(v)] = out
                return out
            cx = Value("cast", (xi, f32))
            cy = Value("cast", (yi, f32))
            if tx and ty:  # u [k, m], w [n, k]: prod[k, m, n] = u[k, m] * w[n, k]
                prod = Value("mul", (Value("bcast", (cx, (":", ":", None))), Value("bcast", (cy, (1, None, 0)))))
                axis = 0
            elif ty:
                prod = Value("mul", (Value("bcast", (cx, (":", None, ":"))), Value("bcast", (cy, (None, ":", ":")))))
                axis = 2
            elif tx:
                prod = Value("mul", (Value("bcast", (cx, (":", ":", None))), Value("bcast", (cy, (":", None, ":")))))
                axis = 0
            else:
                prod = Value("mul", (Value("bcast", (cx, (":", ":", None))), Value("bcast", (cy, (None, ":", ":")))))
                axis = 1
            out = Value("reduce", ("sum", prod, axis))
        else:
            args = tuple(rebuild(a) for a in v.args)
            out = v if all(a is b for a, b in zip(args, v.args)) else Value(v.op, args)
        done[id(v)] = out
        return out

    lowered = copy.copy(program)
    lowered.stores = {k: rebuild(v) for k, v in program.stores.items()}
    lowered.effects = [tuple(rebuild(a) for a in eff) for eff in program.effects]
    lowered.loops = {i: dataclasses.replace(lp, trip=rebuild(lp.trip), init={n: rebuild(x) for n, x in lp.init.items()},
                                            update={n: rebuild(x) for n, x in lp.update.items()})
                     for i, lp in program.loops.items()}
    return lowered


def _constants(program):
    """The program with every loop's trip count, initial and updated values as values
    (a Python number there becomes a constant)."""
    if not program.loops:
        return program

    def val(x):
        return x if isinstance(x, Value) else Value("const", (x,))

    def trip(x):  # `range(n)` of a scalar parameter names the parameter itself: its value
        return Value("load", (x,)) if isinstance(x, Value) and x.op in ("param", "index") else val(x)

    out = copy.copy(program)
    out.loops = {i: dataclasses.replace(lp, trip=trip(lp.trip), init={n: val(x) for n, x in lp.init.items()},
                                        update={n: val(x) for n, x in lp.update.items()})
                 for i, lp in program.loops.items()}
    return out


def _effect_roots(eff):
    """The values a side effect reads (its view, with any level indices that are values)."""
    if eff[0] == "src_store":
        return list(eff[2]) + [eff[3]]
    return [eff[1], eff[2]]


class _LoopNest:
    """Where each value of a program with symbolic loops is computed.

    A value's scope is the innermost loop whose index or carried values it depends on (None:
    outside every loop); a loop's results belong to the loop's own enclosing scope.  The
    values a Python scope can see make these dependencies a chain, so the innermost is the
    deepest of them."""

    def __init__(self, program, values):
        self.program = program
        self.loops = program.loops
        self.depth = {}
        for i in sorted(self.loops):  # a loop's id is above its enclosing loop's
            p = self.loops[i].parent
            self.depth[i] = 0 if p is None else self.depth[p] + 1
        self.scopes = {}
        for v in values:  # dependencies first
            if v.op in ("loop_index", "carried"):
                sc = v.args[0]
            elif v.op == "loop_out":
                sc = self.loops[v.args[0]].parent
            else:
                sc = None
                for a in v.args:
                    for x in (a if isinstance(a, tuple) else (a,)):
                        if isinstance(x, Value):
                            sc = self.deeper(sc, self.scopes[id(x)])
            self.scopes[id(v)] = sc

    def deeper(self, a, b):
        if a is None:
            return b
        if b is None:
            return a
        return a if self.depth[a] >= self.depth[b] else b

    def inside(self, i, outer):
        """Whether loop ``i`` is ``outer`` or nested in it."""
        while i is not None:
            if i == outer:
                return True
            i = self.loops[i].parent
        return False

    def effect_scope(self, e):
        sc = None
        for i, lp in self.loops.items():
            if lp.effects[0] <= e < lp.effects[1]:
                sc = self.deeper(i, sc)
        return sc

    def items(self, scope):
        """The loops and side effects directly in ``scope``, in program order."""
        keyed = [((lp.effects[0], 0, i), ("loop", i)) for i, lp in self.loops.items() if lp.parent == scope]
        keyed += [((e, 1, 0), ("effect", e)) for e in range(len(self.program.effects)) if self.effect_scope(e) == scope]
        return [item for _, item in sorted(keyed)]

    def roots(self, i):
        """Every value loop ``i`` and the loops nested in it compute or store."""
        out = []
        for j, lp in self.loops.items():
            if self.inside(j, i):
                out += [lp.trip] + list(lp.init.values()) + list(lp.update.values())
        s, t = self.loops[i].effects
        for e in range(s, t):
            out += _effect_roots(self.program.effects[e])
        return out


def _analyse_tile(ctx):
    """(ctx, stores, values) of a tile program (ctx a copy whose program has its dots
    lowered, when it has any), or None."""
    program = _lower_dots(_constants(ctx.program), ctx)
    if program is not ctx.program:
        ctx = copy.copy(ctx)
        ctx.program = program
    stores = program.stores
    roots = list(stores.values())
    for eff in program.effects:
        if eff[0] == "view_store" and _view_chain(eff[1]) is None:
            return None
        roots += _effect_roots(eff)
    for lp in program.loops.values():
        roots += [lp.trip] + list(lp.init.values()) + list(lp.update.values())
    values = _walk(roots)
    if not stores and not program.effects:
        return None
    for v in values:
        if v.op not in _TILE_ALLOWED:
            return None
        if v.op == "load" and _view_chain(v.args[0]) is None:
            return None
        if v.op == "offsets" and v.args[0].op != "param":
            return None
    loaded = {_view_chain(v.args[0])[0] for v in values if v.op == "load"}
    loaded |= {v.args[0].args[0] for v in values if v.op == "offsets"}
    read_raw = {v.args[0] for v in values if v.op == "src_load"}
    read_raw |= {frontend_pointer_param(v.args[0]) for v in values if v.op == "ptr_load"}
    tensors = [n for n in list(stores) + sorted(loaded) if ctx.params[n].source_ndim != 0]
    for n in stores:
        if ctx.params[n].source_ndim == 0:
            return None
    targets = set(effect_targets(program))
    data_read = {_view_chain(v.args[0])[0] for v in values if v.op == "load"}  # offsets are indices, not data
    if targets & (data_read | read_raw):
        raise LoweringError("the generic tile kernels do not scatter into or store through a pointer to a tensor "
                            "they also read")
    if set(stores) & (data_read | read_raw) and targets & set(stores):
        raise LoweringError("a tile program that updates a tensor it reads may not also write its outputs "
                            "through pointers or level stores")
    if not tensors:
        raise LoweringError("a tile program needs an arranged tensor to set its program grid")
    indexed = {_view_chain(v.args[0])[0] for v in values if v.op == "load" and _view_chain(v.args[0])[1]}
    indexed |= {_view_chain(e[1])[0] for e in program.effects if e[0] == "view_store"}
    tensors += sorted({_view_chain(e[1])[0] for e in program.effects if e[0] == "view_store"})
    for n in tensors:
        depth = len(ctx.views[n].level_shapes)
        if depth > 3 or (depth == 3 and n not in indexed):
            raise LoweringError(f"`{n}` has {depth} levels; the generic tile kernels take 2, or 3 indexed by level")
    # one flat program id, unravelled by every tensor over its own outermost level
    if len({int(np.prod(ctx.views[n].level_shapes[0])) for n in tensors}) > 1:
        raise LoweringError("the arranged tensors have different numbers of programs")
    return ctx, stores, values


class TilePlan(GenericPlan):
    """A bound generic tile program (see the section comment above)."""

    family = "generic"

    def __init__(self, ctx, stores, values):
        self.ctx = ctx
        self.stores = stores
        probe = _Emitter(ctx)
        program = ctx.program
        self.nest = _LoopNest(program, values) if program.loops else None
        # a tile stored to a tensor the program also reads: every stored value is computed
        # into LDS before the first write, so that each load sees the tensor as it was
        read = {_view_chain(v.args[0])[0] for v in values if v.op == "load"}
        read |= {v.args[0] for v in values if v.op == "src_load"}
        read |= {frontend_pointer_param(v.args[0]) for v in values if v.op == "ptr_load"}
        self.inplace = bool(set(stores) & read)
        self.carried_shapes = self._settle_shapes(values, probe)
        self.shapes = _shapes(ctx, values, probe.const_value, self.carried_shapes)
        self.outputs = list(stores)
        self.kernel_name = "nt_generic_tile"
        arranged = self.outputs + sorted(
            {_view_chain(e[1])[0] for e in program.effects if e[0] == "view_store"}
            | {_view_chain(v.args[0])[0] for v in values if v.op == "load"
               and ctx.params[_view_chain(v.args[0])[0]].source_ndim != 0}
            | {v.args[0].args[0] for v in values if v.op == "offsets"})
        grid = tuple(ctx.views[arranged[0]].level_shapes[0])
        self.programs = int(np.prod(grid)) if grid else 1
        if self.nest is not None:
            for out, v in stores.items():
                if self.nest.scopes[id(v)] is not None:
                    raise LoweringError(f"`{out}` is assigned a value computed inside a loop; the generic tile kernels "
                                        "store a loop's results after it, or a level of the output inside it")
        # the types of the loop-carried values: the promotion of each one's initial and updated
        # types, found by emitting until they no longer change
        self.carried_types = {}
        for _ in range(8):
            found = self._emit(values)
            if found == self.carried_types:
                break
            self.carried_types = found
        else:
            raise LoweringError("the types of the loop-carried values do not settle")
        self.loaded = sorted({_view_chain(v.args[0])[0] for v in values if v.op == "load"
                              and ctx.params[_view_chain(v.args[0])[0]].source_ndim != 0} - set(stores))
        # tensors reached only through pointers or source indexing: a plain pointer argument
        self.raw = sorted((self.raw_reads | set(self.raw_writes)) - set(self.loaded) - set(self.outputs)
                          - set(self.view_targets))
        self.scalars = [v.args[0].args[0] for v in values if v.op == "load" and v.args[0].op == "param"
                        and ctx.params[v.args[0].args[0]].source_ndim == 0]
        self.scalars = list(dict.fromkeys(self.scalars))
        self.offsets = sorted({(v.args[0].args[0], int(v.args[1])) for v in values if v.op == "offsets"})
        self.index_names = list(dict.fromkeys(self.outputs + self.view_targets + self.loaded))
        self.tile_sizes = {n: int(np.prod([int(np.prod(l)) for l in ctx.views[n].level_shapes[1:]]))
                           for n in self.index_names}
        self.offset_lengths = {(n, d): (_tile_shape(ctx, n)[d] if _tile_shape(ctx, n) else 1) for n, d in self.offsets}
        self.scalar_types = {n: probe.scalar_type(n) for n in self.scalars}
        params = [f"const int* __restrict__ t_{n}" for n in self.index_names]
        params += [f"const int* __restrict__ f_{n}_{d}" for n, d in self.offsets]
        params += [f"const {_STORAGE[_torch_dtype_name(ctx.dtypes[n])][0]}* __restrict__ p_{n}" for n in self.loaded]
        params += [f"{_STORAGE[_torch_dtype_name(ctx.dtypes[n])][0]}* __restrict__ p_{n}"
                   for n in self.outputs + self.view_targets]
        params += [("" if n in self.raw_writes else "const ") + f"{_STORAGE[_torch_dtype_name(ctx.dtypes[n])][0]}* p_{n}"
                   for n in self.raw]
        params += [f"{_STORAGE[self.scalar_types[n]][0]} s_{n}" for n in self.scalars]
        params.append("long long programs")
        self.params = params

    def _settle_shapes(self, values, probe):
        """Shape of every loop-carried value: its initial value's, broadcast with its updated
        value's until that no longer changes."""
        program = self.ctx.program
        carried = {}
        for i in sorted(program.loops):  # an initial value sees only enclosing and earlier loops
            lp = program.loops[i]
            shp = _shapes(self.ctx, _walk(list(lp.init.values())), probe.const_value, carried)
            for n, x in lp.init.items():
                carried[(i, n)] = shp[id(x)]
        for _ in range(8):
            shp = _shapes(self.ctx, values, probe.const_value, carried)
            new = {(i, n): _bcast_shapes(carried[(i, n)], shp[id(u)])
                   for i, lp in program.loops.items() for n, u in lp.update.items()}
            if new == carried:
                return carried
            carried = new
        raise LoweringError("the shapes of the loop-carried values do not settle")

    def carried_type(self, key):
        return self.carried_types.get(key, "float32")

    def _emit(self, values):
        """Emit the kernel body (``self.blocks``, ``self.decls``) with the current carried
        types; returns the carried types the emission implies."""
        ctx, program = self.ctx, self.ctx.program
        self.types = {}
        self.lds = {}
        self.raw_reads = set()  # tensors read through source indexing or pointers
        self.raw_writes = []
        self.view_targets = sorted({_view_chain(e[1])[0] for e in program.effects if e[0] == "view_store"})
        self.decls, self.lds_bytes = [], 0
        self.carried_arrays = {}
        for (i, n), shape in sorted(self.carried_shapes.items()):
            size = int(np.prod(shape)) if shape else 1
            w = _STORAGE["float32" if self.carried_type((i, n)) == "weak" else self.carried_type((i, n))][1]
            arr = f"c{i}_{n}"
            self.decls.append(f"  __shared__ {w} {arr}[{2 * size}];  // loop {i}: `{n}`, two buffers")
            self.lds_bytes += 2 * size * (8 if w in ("double", "long long") else (1 if w == "bool" else 4))
            self.carried_arrays[(i, n)] = (arr, size)
        self.found_types = {}
        self.red_index = {id(r): k for k, r in enumerate(v for v in values if v.op in ("reduce", "mdot"))}
        self.emitted = set()
        em = _TileEmitter(self)
        if self.inplace:  # side effects (which read no stored tensor) first, then the staged stores
            items = (self.nest.items(None) if self.nest is not None
                     else [("effect", e) for e in range(len(program.effects))]) + [("staged", None)]
        elif self.nest is None:
            items = [("store", out) for out in self.stores] + [("effect", e) for e in range(len(program.effects))]
        else:
            items = self.nest.items(None) + [("store", out) for out in self.stores]
        self.blocks = self._scope_blocks(em, None, items)
        if self.lds_bytes > LDS_BYTES:
            raise LoweringError(f"the reductions and loop-carried values of this program need {self.lds_bytes} bytes "
                                f"of LDS (at most {LDS_BYTES})")
        return self.found_types

    def _scope_blocks(self, em, scope, items):
        """Blocks of the items of one scope, each preceded by the reductions of that scope it
        needs that no earlier item did."""
        program = self.ctx.program
        blocks = []
        for kind, x in items:
            if kind == "loop":
                roots = self.nest.roots(x)
            elif kind == "effect":
                roots = _effect_roots(program.effects[x])
            elif kind == "store":
                roots = [self.stores[x]]
            elif kind == "staged":
                roots = list(self.stores.values())
            else:  # "update": the carried values of loop x
                roots = list(program.loops[x].update.values())
            for v in _walk(roots):
                if v.op in ("reduce", "mdot") and id(v) not in self.emitted and (
                        self.nest is None or self.nest.scopes[id(v)] == scope):
                    self.emitted.add(id(v))
                    blocks.append(self._reduction_block(em, v) if v.op == "reduce" else self._mdot_block(em, v))
            if kind == "loop":
                blocks += self._loop_blocks(em, x)
            elif kind == "effect":
                blocks.append(self._effect(em, x, program.effects[x]))
            elif kind == "store":
                blocks.append(self._store_block(em, x, self.stores[x]))
            elif kind == "staged":
                blocks += self._staged_stores(em)
        return blocks

    def _reduction_block(self, em, r):
        k = self.red_index[id(r)]
        kind, operand, axis = r.args
        sshape = self.shapes[id(operand)]
        oshape = self.shapes[id(r)]
        if axis is None:
            n_out, extent = 1, int(np.prod(sshape)) if sshape else 1
        else:
            ax = axis + len(sshape) if axis < 0 else axis
            n_out, extent = int(np.prod(oshape)) if oshape else 1, sshape[ax]
        # operand coordinates from (o, l)
        if axis is None:
            coords = _unravel("l", sshape)
        else:
            oc = list(_unravel("o", oshape))
            coords = tuple(oc[:ax] + ["l"] + oc[ax:])
        body = em.context(operand, coords, f"r{k}_")
        t = em.type_of(operand)
        t = "float32" if t in ("weak", "bool") else t
        if kind == "sum" and t in ("int8", "int16", "uint8"):
            t = "int32"
        w = em.work(t)
        if w == "bool":
            raise LoweringError("reductions of booleans are not supported")
        ident, comb = self._combine(kind, t, w)
        val = em.operand(operand, t)
        mask = em.mask_of(operand)
        term = f"({mask}) ? {val} : {ident}" if mask else val
        lanes = 1 if n_out >= 256 else min(64, 1 << int(np.log2(256 // n_out)))
        lanes = max(1, min(lanes, 1 << int(np.ceil(np.log2(max(extent, 1))))))
        step = 256 // lanes
        o_pad = -(-n_out // step) * step
        arr = f"red{k}"
        self.decls.append(f"  __shared__ {w} {arr}[{max(n_out, 1)}];")
        self.lds_bytes += max(n_out, 1) * (8 if w in ("double", "long long") else 4)
        self.lds[id(r)] = (arr, oshape)
        self.types[id(r)] = t
        return "\n".join([
            f"    {{  // {kind} over {'all axes' if axis is None else f'axis {axis}'}: {n_out} x {extent}",
            f"      const int g = tid % {lanes};",
            f"      for (int o = tid / {lanes}; o < {o_pad}; o += {step}) {{",
            f"        {w} acc = {ident};",
            f"        if (o < {n_out}) {{",
            f"          for (long long l = g; l < {extent}LL; l += {lanes}) {{",
            *["    " + x for x in body],
            f"            acc = {comb.format(a='acc', b=f'({term})')};",
            "          }",
            "        }",
            *([f"        for (int s = {lanes // 2}; s > 0; s >>= 1) "
               f"acc = {comb.format(a='acc', b='__shfl_xor(acc, s, 64)')};"] if lanes > 1 else []),
            f"        if (g == 0 && o < {n_out}) {arr}[o] = {em.round_to(t, 'acc')};",
            "      }",
            "    }",
            "    __syncthreads();",
        ])

    def _staged_stores(self, em):
        """Every stored tile computed into LDS (in its storage type), one barrier, then written."""
        compute, write = [], []
        for out, v in self.stores.items():
            lines = self._store_block(em, out, v).split("\n")
            st = _STORAGE[_torch_dtype_name(self.ctx.dtypes[out])][0]
            n_tile = int(np.prod(_tile_shape(self.ctx, out)) or 1)
            arr = f"stage_{out}"
            self.decls.append(f"  __shared__ {st} {arr}[{n_tile}];  // `{out}` before it is written")
            self.lds_bytes += n_tile * {"double": 8, "long long": 8, "float": 4, "int": 4}.get(st, 2 if "short" in st else 1)
            # the store block's loop with its index lookup moved to the write pass
            head, lookup, skip, body, last, end = lines[0], lines[1], lines[2], lines[3:-2], lines[-2], lines[-1]
            value = last.split(" = ", 1)[1]
            compute.append("\n".join([head, *body, f"      {arr}[j] = {value}", end]))
            write.append("\n".join([head, lookup, skip, f"      p_{out}[oi] = {arr}[j];", end]))
        return compute + ["    __syncthreads();"] + write

    def _mdot_block(self, em, v):
        """``dot`` on the matrix core: both operands staged into LDS as [row][k] (k
        contiguous, rows padded by 16 bytes), masked elements as zero, and zero-padded to M, N
        multiples of 32 and K of 16; each wave takes 32 x 32 output blocks,
        ``v_mfma_f32_32x32x16`` per 16-deep k slice, and stores their elements inside [M, N]
        into an fp32 LDS array."""
        k_id = self.red_index[id(v)]
        x, y, tx, ty = v.args
        sx, sy = self.shapes[id(x)], self.shapes[id(y)]
        m, kk = (sx[1], sx[0]) if tx else sx
        n = sy[0] if ty else sy[1]
        mp, np_, kp = -(-m // 32) * 32, -(-n // 32) * 32, -(-kk // 16) * 16
        pitch = kp + 8
        a, b, arr = f"da{k_id}", f"db{k_id}", f"red{k_id}"
        lines = [f"    {{  // dot on the matrix core: [{m}, {kk}] x [{kk}, {n}]"]
        t = None
        for name, val, rows, rows_p, trans, tag in ((a, x, m, mp, tx, f"ma{k_id}_"), (b, y, n, np_, not ty, f"mb{k_id}_")):
            # element j of the staged (padded) operand: row j / kp, k j % kp; zero past [rows, kk]
            r, c = f"(j / {kp}LL)", f"(j % {kp}LL)"
            body = em.context(val, (c, r) if trans else (r, c), tag)
            if t is None:
                t = _mdot_stage_type(_static_type(self.ctx, x), _static_type(self.ctx, y))
                if t is None:
                    raise LoweringError("a matrix-core dot needs 16-bit or fp8 float operands (bf16 with bf16)")
            st = "st_f16" if t == "float16" else "st_bf16"
            mask = em.mask_of(val)
            value = f"{st}({em.operand(val, em.type_of(val))})"
            if mask:
                value = f"(({mask}) ? {value} : (unsigned short)0)"
            lines += [f"      for (long long j = tid; j < {rows_p * kp}LL; j += 256) {{",
                      f"        unsigned short staged = 0;",
                      f"        if ({r} < {rows}LL && {c} < {kk}LL) {{", *["    " + x for x in body],
                      f"          staged = {value};", "        }",
                      f"        {name}[(j / {kp}LL) * {pitch}LL + (j % {kp}LL)] = staged;", "      }"]
            self.decls.append(f"  __shared__ __attribute__((aligned(16))) unsigned short {name}[{rows_p * pitch}];")
            self.lds_bytes += rows_p * pitch * 2
        frag = "nt_half8" if t == "float16" else "nt_bf16x8"
        mfma = "__builtin_amdgcn_mfma_f32_32x32x16_" + ("f16" if t == "float16" else "bf16")
        nb = np_ // 32
        lines += [
            "      __syncthreads();",
            "      {",
            "        const int lane = tid & 63, wave = tid >> 6;",
            f"        for (int blk = wave; blk < {(mp // 32) * nb}; blk += 4) {{",
            f"          const int bm = blk / {nb}, bn = blk % {nb};",
            "          nt_floatx16 acc = {};",
            f"          for (int k0 = 0; k0 < {kp}; k0 += 16) {{",
            f"            const {frag} fa = *(const {frag}*)({a} + (bm * 32 + (lane & 31)) * {pitch} + k0 + 8 * (lane >> 5));",
            f"            const {frag} fb = *(const {frag}*)({b} + (bn * 32 + (lane & 31)) * {pitch} + k0 + 8 * (lane >> 5));",
            f"            acc = {mfma}(fa, fb, acc, 0, 0, 0);",
            "          }",
            "          for (int r = 0; r < 16; ++r) {",
            "            const int row = bm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), col = bn * 32 + (lane & 31);",
            f"            if (row < {m} && col < {n}) {arr}[row * {n} + col] = acc[r];",
            "          }",
            "        }",
            "      }",
            "    }",
            "    __syncthreads();",
        ]
        self.decls.append(f"  __shared__ float {arr}[{m * n}];")
        self.lds_bytes += m * n * 4
        self.lds[id(v)] = (arr, (m, n))
        self.types[id(v)] = "float32"
        return "\n".join(lines)

    def _store_block(self, em, out, v):
        ctx = self.ctx
        tshape = _tile_shape(ctx, out)
        sv = self.shapes[id(v)]
        if _bcast_shapes(sv, tshape) != tshape:
            raise LoweringError(f"a value of shape {sv} is stored to a tile of shape {tshape}")
        n_tile = int(np.prod(tshape)) if tshape else 1
        oc = _unravel("j", tshape)
        body = em.context(v, oc[len(oc) - len(sv):] if sv else (), f"s{out}_")
        t = _torch_dtype_name(ctx.dtypes[out])
        src = em.type_of(v)
        src = "float32" if src == "weak" else src
        val = em.operand(v, src) if em.is_const(v) else em.names[id(v)]
        if em.work(src) != em.work(t):
            val = f"(({em.work(t)}){val})"
        return "\n".join([
            f"    for (long long j = tid; j < {n_tile}LL; j += 256) {{",
            f"      const int oi = {self.index_expr(out, 'j')};",
            "      if (oi < 0) continue;",
            *body,
            f"      p_{out}[oi] = {_STORAGE[t][3].format(val)};",
            "    }",
        ])

    def _carried_write(self, em, i, n, v, tag, buffer):
        """Lines writing value ``v`` to every element of loop ``i``'s carried ``n`` in ``buffer``."""
        arr, size = self.carried_arrays[(i, n)]
        shape = self.carried_shapes[(i, n)]
        t = self.carried_type((i, n))
        coords = _unravel("j", shape)
        sv = self.shapes[id(v)]
        body = em.context(v, coords[len(coords) - len(sv):] if sv else (), tag)
        val = em.round_to(t, em.operand(v, t))
        return [
            f"    for (long long j = tid; j < {size}LL; j += 256) {{",
            *body,
            f"      {arr}[{buffer} * {size}LL + j] = {val};",
            "    }",
        ]

    @staticmethod
    def _settled_type(t, v):
        if t != "weak":
            return t
        c = v.args[0] if v.op == "const" else None
        return "bool" if isinstance(c, bool) else ("int32" if isinstance(c, int) else "float32")

    def _loop_blocks(self, em, i):
        """A symbolic loop: its carried values in two LDS buffers each (iteration k reads
        buffer k % 2 and writes the other), one barrier per iteration after the update."""
        lp = self.ctx.program.loops[i]
        lines = [f"    // loop {i} (`for {lp.var} in range(...)`)"]
        trip_lines = em.context(lp.trip, (), f"t{i}_")
        tt = em.type_of(lp.trip)
        if tt not in _INT and not (tt == "weak" and isinstance(em.const_value(lp.trip), int)):
            raise LoweringError("a loop's trip count must be an integer")
        lines += trip_lines + [f"    const long long n{i} = {em.operand(lp.trip, 'int64')};"]
        init_types = {}
        for n, x in sorted(lp.init.items()):
            lines += self._carried_write(em, i, n, x, f"i{i}_{n}_", "0")
            init_types[n] = self._settled_type(em.type_of(x), x)
        lines.append("    __syncthreads();")
        body = self._scope_blocks(em, i, self.nest.items(i) + [("update", i)])
        update = []
        for n, u in sorted(lp.update.items()):
            update += self._carried_write(em, i, n, u, f"u{i}_{n}_", f"(pp{i} ^ 1)")
            self.found_types[(i, n)] = _promote(init_types[n], self._settled_type(em.type_of(u), u))
        inner = [f"    const long long pp{i} = li{i} & 1;", *body, *update, "    __syncthreads();"]
        lines.append(f"    for (long long li{i} = 0; li{i} < n{i}; ++li{i}) {{")
        lines += ["  " + x for x in "\n".join(inner).split("\n")]
        lines.append("    }")
        lines.append(f"    const long long po{i} = (n{i} > 0 ? n{i} : 0) & 1;")
        return ["\n".join(lines)]

    def index_expr(self, name, lin):
        return f"t_{name}[pb_{name} + {lin}]"

    def level_index(self, name, ks, inner, em):
        """C index-table entry of element ``inner`` of the level of ``name`` reached by the
        level indices ``ks`` (ints, or values already emitted by ``em``); -1 (masked) where an
        index that is a value falls outside its level."""
        levels = [tuple(l) for l in self.ctx.views[name].level_shapes[1:]]
        terms, guards = [], []
        for i, k in enumerate(ks):
            if len(levels[i]) != 1:
                raise LoweringError(f"level index {k} of `{name}` needs a 1-D level")
            below = int(np.prod([int(np.prod(l)) for l in levels[i + 1:]]))
            if isinstance(k, Value):
                if self.shapes[id(k)] != ():
                    raise LoweringError(f"a level index of `{name}` must be a scalar")
                t = em.type_of(k)
                if t not in _INT and not (t == "weak" and isinstance(em.const_value(k), int)):
                    raise LoweringError(f"a level index of `{name}` must be an integer")
                e = em.operand(k, "int64")
                terms.append(f"({e}) * {below}LL")
                guards.append(f"({e}) >= 0 && ({e}) < {levels[i][0]}LL")
            else:
                if not 0 <= k < levels[i][0]:
                    raise LoweringError(f"level index {k} of `{name}` needs a 1-D level that holds it")
                terms.append(f"{k * below}LL")
        entry = self.index_expr(name, " + ".join(terms + [inner]) if terms else inner)
        return f"(({' && '.join(guards)}) ? {entry} : -1)" if guards else entry

    def extent(self, name):
        """Elements from a tensor's first to one past its last element (its storage span)."""
        return jagged.storage_extent(self.ctx.values[name])

    _ATOMIC = {"float32": "float", "float64": "double", "int32": "int"}

    def _effect(self, em, k, eff):
        """One side effect: a scatter into a source, a store or an atomic add through a pointer,
        element by element over the broadcast shape of its operands, masked to the tensor."""
        kind = eff[0]
        if kind == "view_store":
            name, ks = _view_chain(eff[1])
            value = eff[2]
            levels = self.ctx.views[name].level_shapes
            shape = tuple(levels[1 + len(ks)]) if 1 + len(ks) < len(levels) else ()
            sv = self.shapes[id(value)]
            if _bcast_shapes(sv, shape) != shape:
                raise LoweringError(f"a value of shape {sv} is stored to a level of shape {shape}")
            n = int(np.prod(shape)) if shape else 1
            coords = _unravel("j", shape)
            indices = [(x, ()) for x in ks if isinstance(x, Value)]
            body = em.context(value, coords[len(coords) - len(sv):] if sv else (), f"e{k}_", more=indices)
            t = _torch_dtype_name(self.ctx.dtypes[name])
            src = em.type_of(value)
            src = "float32" if src == "weak" else src
            val = em.operand(value, src) if em.is_const(value) else em.names[id(value)]
            if em.work(src) != em.work(t):
                val = f"(({em.work(t)}){val})"
            return "\n".join([
                f"    for (long long j = tid; j < {n}LL; j += 256) {{  // store into {name}{list(ks)}",
                f"      const int oi = {self.level_index(name, ks, 'j', em)};",
                "      if (oi < 0) continue;",
                *body,
                f"      p_{name}[oi] = {_STORAGE[t][3].format(val)};",
                "    }",
                "    __syncthreads();",
            ])
        if kind == "src_store":
            name, indices, value = eff[1], eff[2], eff[3]
            operands = list(indices) + [value]
        else:
            ptr, value = eff[1], eff[2]
            name = frontend_pointer_param(ptr)
            operands = [ptr, value]
        shape = _bcast_shapes(*[self.shapes[id(x)] for x in operands])
        n = int(np.prod(shape)) if shape else 1
        coords = _unravel("j", shape)
        roots = [(x, coords[len(coords) - len(self.shapes[id(x)]):] if self.shapes[id(x)] else ())
                 for x in operands]
        body = em.context(roots[0][0], roots[0][1], f"e{k}_", more=roots[1:])
        t = _torch_dtype_name(self.ctx.dtypes[name])
        src = em.type_of(value)
        src = "float32" if src in ("weak", "bool") else src
        val = em.operand(value, t)
        if kind == "src_store":
            off, cond = em.source_offset(name, indices)
        else:
            pname, off = em.ptrs[id(ptr)]
            cond = f"({off}) >= 0 && ({off}) < {self.extent(name)}LL"
        if kind == "atomic_add":
            ctype = self._ATOMIC.get(t)
            if ctype is None:
                raise LoweringError(f"ntl.atomic_add on {t} tensors is not supported (float32, float64, int32 are)")
            action = f"atomicAdd(p_{name} + o, ({ctype}){val});"
        else:
            action = f"p_{name}[o] = {_STORAGE[t][3].format(val)};"
        self.raw_writes.append(name)
        return "\n".join([
            f"    for (long long j = tid; j < {n}LL; j += 256) {{  // {kind} into {name}",
            *body,
            f"      const long long o = {off};",
            f"      if ({cond}) {action}",
            "    }",
            "    __syncthreads();",
        ])

    def sources_for(self, values):
        return [self.source()]

    @staticmethod
    def _combine(kind, t, w):
        if kind == "sum":
            return ("0" if w == "long long" else ("0.0" if w == "double" else "0.0f")), "({a} + {b})"
        lo, hi = _INT_LIMITS.get(t, (None, None))
        if w == "long long":
            ident = f"{lo}LL" if kind == "max" else f"{hi}LL"
            if t == "int64":
                ident = "(-9223372036854775807LL - 1)" if kind == "max" else "9223372036854775807LL"
            return ident, ("({b} > {a} ? {b} : {a})" if kind == "max" else "({b} < {a} ? {b} : {a})")
        inf = "__builtin_huge_val()" if w == "double" else "__builtin_huge_valf()"
        if t == "float8_e4m3fn":  # no infinity: its largest magnitude (reference ssa.py:2187-2192)
            inf = "448.0f"
        f = ("fmax" if kind == "max" else "fmin") + ("" if w == "double" else "f")
        return (f"(-{inf})" if kind == "max" else inf), f + "({a}, {b})"

    def source(self, linear=None, linear_offsets=()):
        bases = [f"    const long long pb_{n} = p * {self.tile_sizes[n]}LL;" for n in self.tile_sizes]
        bases += [f"    const long long pbo_{n}_{d} = p * {self.offset_lengths[(n, d)]}LL;" for n, d in self.offsets]
        return (
            _PRELUDE
            + f'\nextern "C" __global__ void __launch_bounds__(256) {self.kernel_name}({", ".join(self.params)}) {{\n'
            + "\n".join(self.decls) + "\n"
            + "  const int tid = threadIdx.x;\n"
            + "  for (long long p = blockIdx.x; p < programs; p += gridDim.x) {\n"
            + "\n".join(bases + self.blocks)
            + "\n    __syncthreads();\n  }\n}\n"
        )

    def describe(self):
        return {"family": self.family, "outputs": self.outputs, "inputs": self.loaded, "scalars": self.scalars,
                "reductions": len(self.lds)}

    def launch_spec(self, values):
        """As GenericPlan.launch_spec: the tables, the tensors (loaded, stored, read through
        pointers), the scalars and the number of programs."""
        maps, args = {}, []
        for n in self.index_names:
            maps[n] = self._maps(n)
            args.append(("table", self._table(n, values[n], maps[n])[0]))
        args += [("table", self._tile_offsets(n, d, maps.get(n))) for n, d in self.offsets]
        args += [("tensor", n) for n in self.loaded]
        args += [("tensor", n) for n in self.outputs + self.view_targets]
        args += [("tensor", n) for n in self.raw]
        args += [("scalar", n, "int64" if self.scalar_types[n] == "int64" else "float32") for n in self.scalars]
        args.append(("i64", self.programs))
        return self.source(), min(self.programs, 256 * 64), args

    def _tile_offsets(self, name, dim, maps=None):
        """``offsets(dim)`` per program: the source index along ``dim`` of the tile's elements
        along its dim ``dim`` ([programs, tile_shape[dim]]); it may not vary along the other
        tile dims."""
        idx, _, shape = maps or self._maps(name)
        grid = tuple(self.ctx.views[name].level_shapes[0])
        tile = _tile_shape(self.ctx, name)
        full = np.broadcast_to(np.asarray(idx[dim], dtype=np.int64), shape).reshape(
            (int(np.prod(grid)) if grid else 1,) + tile)
        sel = [slice(None)] + [slice(None) if i == dim else slice(0, 1) for i in range(len(tile))]
        vec = full[tuple(sel)]
        if not np.array_equal(np.broadcast_to(vec, full.shape), full):
            raise LoweringError(f"`{name}.offsets({dim})` varies along other tile dims; tile programs take it as a vector")
        vec = vec.reshape(full.shape[0], tile[dim] if tile else 1)
        if vec.size and (vec.max() >= 2**31 or vec.min() < -(2**31)):
            raise LoweringError("the generic kernels take offsets within 32 bits")
        return np.ascontiguousarray(vec, dtype=np.int32).reshape(-1)


def match_generic(ctx):
    """A generic kernel for the program, or None when it is neither element-parallel nor a tile program."""
    found = _analyse(ctx)
    if found is not None:
        return GenericPlan(ctx, *found)
    refused = None
    if ctx.program.loops and ctx.relower is not None:
        # loops with up to MAX_UNROLL iterations known now are unrolled (no loop-carried
        # buffers); longer ones, and those whose trip counts are run-time values, stay loops
        resolve = _Emitter(ctx).const_value

        def unroll(trip):
            c = resolve(trip) if isinstance(trip, Value) else trip
            return c if isinstance(c, int) and not isinstance(c, bool) and 0 <= c <= MAX_UNROLL else None

        program = ctx.relower(unroll)
        if len(program.loops) < len(ctx.program.loops):
            unrolled = copy.copy(ctx)
            unrolled.program = program
            try:
                found = _analyse_tile(unrolled)
                if found is not None:
                    return TilePlan(*found)
            except LoweringError as e:  # e.g. unrolled reductions beyond the LDS: try the loops
                refused = e
    found = _analyse_tile(ctx)
    if found is not None:
        return TilePlan(*found)
    if refused is not None:
        raise refused
    return None
