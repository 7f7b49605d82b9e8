"""Standalone C++ launchers for AOT builds (reference ``backends/materializers/cpp.py:26-333``).

For an AOT build whose shapes, strides and dtypes are fixed at definition, the kernel plan
chosen for that specialisation becomes a C++ function with the reference's standalone ABI

    NineToothedResult launch_<kernel>(NineToothedStream stream, NineToothedTensor tensor_0, ...);

(``ninetoothed.h``: ``NineToothedTensor {void *data; uint64_t *shape; int64_t *strides;}``,
the stream is a ``hipStream_t``, the result a ``hipError_t``).  Tensors are passed in the
application's parameter order; 0-d parameters point at a host scalar of their declared
dtype (``double`` for floating types).  The launcher checks every rank, shape and stride
against the specialisation (the plan was fitted to them) and returns NT_ERR_INVALID before
launching anything when one differs; an empty output returns 0.  It then calls the plan's
entry point of ``libnt_mi355x.so``, which it links.

A generic kernel's launcher embeds its code object (compiled for gfx950 by hipRTC at build
time) and its index tables (fixed by the specialisation's shapes and strides).  On its first
call on a device it loads the code object (``nt_rtc_load``) and copies the tables to that
device once (they stay allocated until the process ends); every call then launches through
``nt_rtc_launch`` with the kernel arguments the Python binding passes.  Tables above
MAX_TABLE_BYTES are not embedded (no launcher).
"""

import math
import re
import subprocess
from pathlib import Path

from ninetoothed_amd import _lib

HEADER = """#ifndef NINETOOTHED_H
#define NINETOOTHED_H

#include <stdint.h>

#define NINETOOTHED_TRUE 1
#define NINETOOTHED_FALSE 0
#define NINETOOTHED_NONE 0

enum NineToothedDataType {
    NINETOOTHED_INT8,
    NINETOOTHED_INT16,
    NINETOOTHED_INT32,
    NINETOOTHED_INT64,
    NINETOOTHED_UINT8,
    NINETOOTHED_UINT16,
    NINETOOTHED_UINT32,
    NINETOOTHED_UINT64,
    NINETOOTHED_FLOAT16,
    NINETOOTHED_BFLOAT16,
    NINETOOTHED_FLOAT32,
    NINETOOTHED_FLOAT64
};

typedef struct {
    void *data;
    uint64_t *shape;
    int64_t *strides;
} NineToothedTensor;

typedef void *NineToothedStream;
typedef int NineToothedResult;

#endif
"""

_SCALAR_C = {"float16": "double", "bfloat16": "double", "float32": "double", "float64": "double",
             "int8": "int8_t", "int16": "int16_t", "int32": "int32_t", "int64": "int64_t", "uint8": "uint8_t"}


MAX_TABLE_BYTES = 16 << 20


class Unsupported(Exception):
    """The plan or the specialisation has no C++ launcher (the reason is the message)."""


def _f(x):
    r = repr(float(x))
    if r in ("inf", "-inf", "nan"):
        raise Unsupported("non-finite constant")
    return r


class _Call:
    """Arguments of one C-ABI call: C expressions, tensors by parameter name."""

    def __init__(self, entry, index):
        self.entry, self.index, self.args, self.arrays = entry, index, [], []

    def ptr(self, name):
        self.args.append(f"tensor_{self.index[name]}.data" if name is not None else "nullptr")

    def i(self, v):
        self.args.append(f"{int(v)}LL")

    def f(self, expr):
        self.args.append(f"(float)({expr})")

    def arr(self, vals):
        name = f"a{len(self.arrays)}"
        self.arrays.append(f"  static const int64_t {name}[{len(vals)}] = {{{', '.join(f'{int(v)}LL' for v in vals)}}};")
        self.args.append(name)


def _coef(factors, scalar_expr):
    terms = []
    for term in factors:
        parts = [scalar_expr(f) if isinstance(f, str) else _f(f) for f in term]
        terms.append(" * ".join(parts) if parts else "1.0")
    return " + ".join(terms) if terms else "0.0"


def _call_for(plan, values, scalar_expr, index):
    """The entry point and argument expressions of ``plan`` for the static ``values``."""
    import torch

    fam = plan.describe()["family"]
    call = None

    def begin(entry):
        nonlocal call
        call = _Call(entry, index)
        return call

    if fam == "gemm":
        a, b, out = values[plan.a], values[plan.b], values[plan.out]
        c = values[plan.c] if plan.c else None
        m, k = a.shape
        n = b.shape[1]
        cl = begin(f"nt_gemm_{_lib.dtype_suffix(a.dtype)}")
        cl.ptr(plan.a), cl.i(a.stride(0)), cl.i(a.stride(1))
        cl.ptr(plan.b), cl.i(b.stride(0)), cl.i(b.stride(1))
        cl.ptr(plan.c if plan.c else None)
        cl.i(c.stride(0) if c is not None else 0), cl.i(c.stride(1) if c is not None else 0)
        cl.ptr(plan.out), cl.i(out.stride(0)), cl.i(out.stride(1))
        out_code = _lib.dtype_code(out.dtype)
        if c is not None and c.dtype != out.dtype:  # c in its own type (e.g. fp8), as kernels.bind_gemm passes it
            out_code |= (_lib.bias_dtype_code(c.dtype) + 1) << 8
        cl.args.append(str(out_code))
        cl.i(m), cl.i(n), cl.i(k)
        cl.f(_coef(plan.alpha_factors, scalar_expr))
        cl.f(_coef(plan.beta_factors, scalar_expr) if plan.c else "0.0")
        cl.args.append(str(_lib.DTYPE_NONE if plan.round_dtype is None else _lib.dtype_code(plan.round_dtype)))
    elif fam == "add":
        a, b, out = values[plan.a], values[plan.b], values[plan.out]
        flat = out.dim() != 1
        cl = begin(f"nt_add_{_lib.dtype_suffix(out.dtype)}")
        cl.ptr(plan.a), cl.i(1 if flat else a.stride(0))
        cl.ptr(plan.b), cl.i(1 if flat else b.stride(0))
        cl.ptr(plan.out), cl.i(1 if flat else out.stride(0))
        cl.i(out.numel())
    elif fam == "softmax":
        x, y = values[plan.x], values[plan.y]
        rows, cols = x.shape
        cl = begin(f"nt_softmax_{_lib.dtype_suffix(x.dtype)}")
        cl.ptr(plan.x), cl.i(x.stride(0)), cl.i(x.stride(1))
        cl.ptr(plan.y), cl.i(y.stride(0)), cl.i(y.stride(1))
        cl.i(rows), cl.i(cols), cl.i(max(cols if plan.block is None else int(plan.block), 1))
    elif fam == "max_pool2d":
        x, y = values[plan.x], values[plan.y]
        kh, kw = plan.window
        sh, sw = plan.stride if plan.stride is not None else plan.window
        cl = begin(f"nt_max_pool2d_{_lib.dtype_suffix(x.dtype)}")
        cl.ptr(plan.x), cl.arr(x.stride()), cl.ptr(plan.y), cl.arr(y.stride())
        for v in (*x.shape, y.shape[2], y.shape[3], kh, kw, sh, sw, *plan.padding, *plan.dilation):
            cl.i(v)
    elif fam == "attention":
        q, k, v, o = (values[n] for n in (plan.q, plan.k, plan.v, plan.o))
        scale = plan.scale
        if q.dtype in (torch.float16, torch.bfloat16):
            scale = float(torch.tensor(scale, dtype=q.dtype))
        cl = begin(f"nt_attention_{_lib.dtype_suffix(q.dtype)}")
        for name, t in ((plan.q, q), (plan.k, k), (plan.v, v), (plan.o, o)):
            cl.ptr(name), cl.arr(t.stride())
        cl.args.append(str(_lib.dtype_code(o.dtype)))
        for val in (q.shape[0], q.shape[1], q.shape[2], k.shape[2], q.shape[3]):
            cl.i(val)
        cl.f(_f(scale))
        cl.args.append("1" if plan.causal else "0")
    elif fam == "conv2d":
        x, w, y = values[plan.x], values[plan.w], values[plan.y]
        cl = begin(f"nt_conv2d_{_lib.dtype_suffix(x.dtype)}")
        cl.ptr(plan.x), cl.arr(x.stride()), cl.ptr(plan.w), cl.arr(w.stride()), cl.ptr(plan.y), cl.arr(y.stride())
        cl.args.append(str(_lib.dtype_code(y.dtype)))
        dims = (*x.shape, w.shape[0], w.shape[2], w.shape[3], y.shape[2], y.shape[3], *plan.padding, *plan.stride,
                *plan.dilation)
        for val in dims:
            cl.i(val)
        cl.args.append(str(_lib.DTYPE_NONE if plan.round_dtype is None else _lib.dtype_code(plan.round_dtype)))
        cl.args += ["nullptr", "0LL"]  # no re-layout workspace: the direct kernel
    else:
        raise Unsupported(f"the {fam} kernels have no standalone C++ launcher")
    return call


def source(kernel_name, plan, kernel, values, outputs):
    """C++ source of ``launch_<kernel_name>`` for ``plan`` specialised to ``values``."""
    if not re.fullmatch(r"[A-Za-z_][A-Za-z0-9_]*", kernel_name):
        raise Unsupported(f"`{kernel_name}` is not a C identifier")
    names = list(kernel.params)
    index = {n: i for i, n in enumerate(names)}
    specs = {s.name: s for s in kernel.param_specs}
    checks, reads, empty, nulls = [], [], [], []
    from ninetoothed_amd.dtype import normalize_dtype

    def scalar_expr(name):
        return f"s_{name}"

    for i, name in enumerate(names):
        spec, t = specs[name], f"tensor_{i}"
        if spec.source_ndim == 0:
            if spec.dtype is None:
                raise Unsupported(f"`{name}` needs a declared dtype for the C++ ABI")
            ctype = _SCALAR_C.get(normalize_dtype(spec.dtype))
            if ctype is None:
                raise Unsupported(f"scalar dtype {spec.dtype} of `{name}`")
            if spec.constexpr:
                checks.append(f"{t}.data != nullptr && *static_cast<const {ctype} *>({t}.data) != "
                              f"({ctype})({_f(spec.constexpr_value)})")
            else:
                nulls.append(f"{t}.data == nullptr")
                reads.append(f"  const double s_{name} = (double)*static_cast<const {ctype} *>({t}.data);")
            continue
        v = values[name]
        checks.append(f"{t}.shape == nullptr || {t}.strides == nullptr")
        for d, (size, stride) in enumerate(zip(v.shape, v.stride())):
            checks.append(f"{t}.shape[{d}] != {int(size)}ULL || {t}.strides[{d}] != {int(stride)}LL")
        nulls.append(f"{t}.data == nullptr")
        if name in outputs and math.prod(v.shape) == 0:
            empty.append("true")
    params = ", ".join(["NineToothedStream stream"] + [f"NineToothedTensor tensor_{i}" for i in range(len(names))])
    body = [f"  if ({c}) return NT_ERR_INVALID;" for c in checks]
    if empty:
        body.append("  return 0;  // an empty output: nothing to launch")
    body.append(f"  if ({' || '.join(nulls) or 'false'}) return NT_ERR_INVALID;")
    body += reads
    prelude = ""
    if plan.describe()["family"] == "generic":
        prelude, launch = _generic_launch(plan, values, index)
        body += launch
    else:
        call = _call_for(plan, values, scalar_expr, index)
        body += call.arrays
        body.append(f"  return {call.entry}({', '.join(call.args + ['static_cast<hipStream_t>(stream)'])});")
    return (
        "// Standalone launcher of an AOT-built NineToothed kernel for the MI355X backend.\n"
        '#include "ninetoothed.h"\n#include "nt_mi355x.h"\n\n' + prelude
        + f'extern "C" NineToothedResult launch_{kernel_name}({params}) {{\n' + "\n".join(body) + "\n}\n"
    )


def _bytes_c(data, per_line=24):
    items = [f"0x{b:02x}" for b in data]
    return ",\n".join(", ".join(items[i:i + per_line]) for i in range(0, len(items), per_line))


def _generic_launch(plan, values, index):
    """(file-scope code, launcher body lines) of a generic kernel plan on the static ``values``."""
    from ninetoothed_amd.generic import GenericPlan

    spec = plan.launch_spec(values)
    if spec is None:
        return "", ["  return 0;  // the program stores nothing"]
    source, grid, args = spec
    tables = [a[1] for a in args if a[0] == "table" and a[1] is not None]
    if sum(t.nbytes for t in tables) > MAX_TABLE_BYTES:
        raise Unsupported(f"the generic kernel's index tables exceed {MAX_TABLE_BYTES} bytes")
    code = GenericPlan.code_object(source)
    lines = ["#include <hip/hip_runtime.h>", "#include <mutex>", "", "namespace {",
             f"const unsigned char kCode[{len(code)}] = {{\n{_bytes_c(code)}}};"]
    for i, t in enumerate(tables):
        vals = ", ".join(str(int(x)) for x in t.tolist())
        lines.append(f"const int32_t kTable{i}[{t.size}] = {{{vals}}};")
    n_tab = len(tables)
    lines += [
        "// Per device: the loaded kernel and the device copies of the tables (kept until exit).",
        "struct Loaded {", "  void* fn = nullptr;", f"  void* tab[{max(n_tab, 1)}] = {{}};", "  int status = -1;", "};",
        "Loaded g_loaded[64];", "std::mutex g_lock;", "int prepare(Loaded& d) {",
        f'  int s = nt_rtc_load(kCode, "{plan.kernel_name}", &d.fn);', "  if (s) return s;"]
    for i, t in enumerate(tables):
        lines += [f"  s = (int)hipMalloc(&d.tab[{i}], sizeof(kTable{i}));", "  if (s) return s;",
                  f"  s = (int)hipMemcpy(d.tab[{i}], kTable{i}, sizeof(kTable{i}), hipMemcpyHostToDevice);",
                  "  if (s) return s;"]
    lines += ["  return 0;", "}", "}  // namespace", ""]
    body = ["  int dev = 0;", "  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return NT_ERR_INVALID;",
            "  Loaded& d = g_loaded[dev];", "  {", "    std::lock_guard<std::mutex> guard(g_lock);",
            "    if (d.status < 0) d.status = prepare(d);", "  }", "  if (d.status) return d.status;"]
    names, k = [], 0
    for i, a in enumerate(args):
        if a[0] == "table":
            if a[1] is None:
                body.append(f"  void* k{i} = nullptr;")
            else:
                body.append(f"  void* k{i} = d.tab[{k}];")
                k += 1
        elif a[0] == "tensor":
            body.append(f"  void* k{i} = tensor_{index[a[1]]}.data;")
        elif a[0] == "scalar":
            ctype = "long long" if a[2] == "int64" else "float"
            body.append(f"  {ctype} k{i} = ({ctype})s_{a[1]};")
        else:
            body.append(f"  long long k{i} = {int(a[1])}LL;")
        names.append(f"&k{i}")
    body.append(f"  void* argv[] = {{{', '.join(names)}}};")
    body.append(f"  return nt_rtc_launch(d.fn, {int(grid)}u, 256u, argv, static_cast<hipStream_t>(stream));")
    return "\n".join(lines) + "\n", body


def build(kernel_name, code, output_dir):
    """Write ninetoothed.h and the source, compile ``lib<kernel_name>.so``; its path."""
    out = Path(output_dir)
    (out / "ninetoothed.h").write_text(HEADER)
    src = out / f"{kernel_name}.launch.cpp"
    src.write_text(code)
    lib = out / f"lib{kernel_name}.so"
    include = Path(__file__).resolve().parents[2] / "include"
    libdir = _lib.LIBRARY_PATH.parent
    cmd = ["/opt/rocm/bin/hipcc", "-shared", "-fPIC", "-O2", "-std=c++17", f"-I{out}", f"-I{include}", str(src),
           f"-L{libdir}", "-lnt_mi355x", f"-Wl,-rpath,{libdir}", "-o", str(lib)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise Unsupported(f"hipcc failed: {r.stderr[-2000:]}")
    return lib
