"""``ninetoothed.build``: several configured variants of one kernel behind one dispatcher.

Contract (reference ``src/ninetoothed/build.py:127-257``, exercised by its
``tests/test_aot.py:233-310``):

    kernel = build(premake, configs, *, caller="cuda", output_dir, kernel_name=None,
                   meta_parameters=None, lazy=False, backend=None, platform=None,
                   compute_arch=None, pipeline=None, pass_options=None, **backend_options)

``configs`` is a sequence of ``(args, kwargs, compiler_options)``; each builds one variant
from ``premake(*args, **kwargs) -> (arrangement, application, tensors)``, AOT-materialised
into ``output_dir``.  A variant's *configuration* is the value of every parameter of
``premake`` (defaults included) except the ``meta_parameters``.  The returned dispatcher
is called with the kernel's arguments followed by one value per configuration parameter,
in ``premake``'s order; it runs the variant built for exactly that configuration and
raises ``ValueError`` when none was.  Variants sharing a configuration (they differ only in
meta parameters or compiler options) are auto-tuned against each other.  ``lazy=True``
defers all of it to the first call.

On the MI355X backend a variant is the compiled program plus its kernel plan; its
standalone C++ launcher exists when shapes, strides and dtypes are fixed
(``backends.cpp_export``).  When every variant has one, ``<kernel_name>.h`` /
``<kernel_name>.cpp`` and ``lib<kernel_name>.so`` hold a C++ dispatcher

    NineToothedResult launch_<kernel_name>(NineToothedStream stream, NineToothedTensor tensor_0, ...,
                                           int|double config_0, ...);

that compares the configuration values and calls the first variant built for them
(dtypes are passed as their ``NineToothedDataType`` enumerator, ``None`` as 0), or returns
NT_ERR_INVALID when none matches.
"""

import inspect
import math
import re
import subprocess
import threading
from pathlib import Path

from ninetoothed_amd.dtype import normalize_dtype

_ENUM = ("int8", "int16", "int32", "int64", "uint8", "uint16", "uint32", "uint64", "float16", "bfloat16",
         "float32", "float64")


def _normal(value):
    """A configuration value as a hashable plain value (what the dispatcher compares)."""
    if isinstance(value, (str, int, float, bool, type(None))):
        return value
    return str(value)


def _function_name(fn):
    while hasattr(fn, "func"):
        fn = fn.func
    return getattr(fn, "__name__", type(fn).__name__.lower())


class _Group:
    """The variants built for one configuration: one handle, or an auto-tuned choice among several."""

    def __init__(self, handles, labels, namespace):
        self.handles = tuple(handles)
        self.tuner = None
        if len(self.handles) > 1:
            from ninetoothed_amd.auto_tuner import AutoTuner

            first = self.handles[0]
            self.tuner = AutoTuner(self.handles, labels, cache_namespace=namespace,
                                   validator=lambda args, kwargs: first._public_values(args, kwargs))

    def __call__(self, *args, **kwargs):
        return self.handles[0](*args, **kwargs) if self.tuner is None else self.tuner(*args, **kwargs)


class BuiltKernel:
    """The dispatcher ``build`` returns."""

    def __init__(self, groups, config_names, handles, cpp=None):
        self._groups = groups  # configuration tuple -> _Group
        self._config_names = tuple(config_names)
        self.handles = tuple(handles)  # every variant, in build order
        self.cpp = cpp  # paths of the C++ dispatcher, or the reason there is none

    @property
    def configurations(self):
        return tuple(self._groups)

    def __call__(self, *args, **kwargs):
        n = len(self._config_names)
        if len(args) < n:
            raise TypeError(f"Expected the kernel arguments followed by {n} configuration values "
                            f"({', '.join(self._config_names)}).")
        config = tuple(_normal(v) for v in args[len(args) - n:]) if n else ()
        group = self._groups.get(config)
        if group is None:
            raise ValueError(f"No compiled kernel configuration matches {config}.")
        return group(*args[:len(args) - n], **kwargs)


class _Lazy:
    def __init__(self, factory):
        self._factory = factory
        self._built = None
        self._lock = threading.Lock()

    def __call__(self, *args, **kwargs):
        if self._built is None:
            with self._lock:
                if self._built is None:
                    self._built = self._factory()
        return self._built(*args, **kwargs)


def build(premake, configs, *, backend=None, platform=None, compute_arch=None, caller="cuda", output_dir,
          kernel_name=None, meta_parameters=None, lazy=False, pipeline=None, pass_options=None, **backend_options):
    """Compile every configured variant of ``premake`` and return one dispatcher (see the module docstring)."""
    configs = tuple(configs)
    meta = tuple(meta_parameters or ())
    if lazy:
        return _Lazy(lambda: build(premake, configs, backend=backend, platform=platform, compute_arch=compute_arch,
                                   caller=caller, output_dir=output_dir, kernel_name=kernel_name,
                                   meta_parameters=meta, pipeline=pipeline, pass_options=pass_options,
                                   **backend_options))
    if not configs:
        raise ValueError("At least one build configuration is required.")
    from ninetoothed_amd.compiler import DEFAULT_COMPILER, CompileRequest

    sig = inspect.signature(premake)
    names = tuple(p for p in sig.parameters if p not in meta)
    base = kernel_name or _function_name(premake)
    members, labels, order, handles = {}, {}, [], []
    for i, (args, kwargs, options) in enumerate(configs):
        bound = sig.bind(*args, **kwargs)
        bound.apply_defaults()
        config = tuple(_normal(bound.arguments[n]) for n in names)
        arrangement, application, tensors = premake(*args, **kwargs)
        options = dict(options or {})
        name = f"{base}_{i}" if len(configs) > 1 else base
        handle = DEFAULT_COMPILER.materialize(CompileRequest(
            arrangement=arrangement, application=application, tensors=tuple(tensors), backend=backend,
            platform=platform, compute_arch=compute_arch, caller=caller, kernel_name=name, output_dir=output_dir,
            num_warps=options.get("num_warps"), num_stages=options.get("num_stages"), max_num_configs=1,
            pipeline=options.get("pipeline", pipeline), pass_options=options.get("pass_options", pass_options),
            backend_options={**backend_options, **dict(options.get("backend_options", {}))},
        ), output_dir=output_dir, mode="aot")
        handles.append(handle)
        if config not in members:
            members[config], labels[config] = [], []
            order.append(config)
        members[config].append(handle)
        labels[config].append(f"{name}:{sorted(kwargs.items())!r}:{sorted(options.items())!r}")
    namespace = f"build_{base}_{backend or 'hip'}_{platform or 'mi355x'}_{compute_arch or 'gfx950'}"
    groups = {c: _Group(members[c], labels[c], namespace) for c in order}
    cpp = _write_cpp_dispatcher(base, names, [(c, members[c][0]) for c in order], Path(output_dir))
    return BuiltKernel(groups, names, handles, cpp)


# ------------------------------------------------------------------ C++ dispatcher
def _cpp_value(value):
    if isinstance(value, str):
        canonical = normalize_dtype(value)
        if canonical in _ENUM:
            return _ENUM.index(canonical)
        raise TypeError(f"configuration value {value!r} has no C++ form")
    if value is None:
        return 0
    if isinstance(value, bool):
        return int(value)
    if isinstance(value, int):
        if not -(1 << 31) <= value < (1 << 31):
            raise ValueError("C++ configuration integers must fit an int")
        return value
    if isinstance(value, float):
        if not math.isfinite(value):
            raise ValueError("C++ configuration values must be finite")
        return value
    raise TypeError(f"configuration value {value!r} has no C++ form")


def _write_cpp_dispatcher(base, names, variants, out):
    """Write and compile the dispatcher over the variants' launchers; a dict of its paths or the reason."""
    if not re.fullmatch(r"[A-Za-z_][A-Za-z0-9_]*", base):
        return {"unavailable": f"`{base}` is not a C identifier"}
    launchers = []
    for config, handle in variants:
        built = getattr(handle, "_built_artifact", None)
        manifest = _manifest(built)
        library = manifest.get("cpp", {}).get("library")
        if library is None:
            return {"unavailable": f"variant {handle._compilation.artifact.kernel_name}: "
                                   + manifest.get("cpp", {}).get("unavailable", "no C++ launcher")}
        launchers.append((config, handle._compilation.artifact.kernel_name, library,
                          len(handle._compilation.launch_abi["public_args"])))
    if len({n for *_, n in launchers}) != 1:
        return {"unavailable": "the variants take different numbers of arguments"}
    try:
        values = [tuple(_cpp_value(v) for v in config) for config, *_ in launchers]
    except (TypeError, ValueError) as exc:
        return {"unavailable": str(exc)}
    n_tensors = launchers[0][3]
    ctypes_ = ["double" if any(isinstance(v[i], float) for v in values) else "int" for i in range(len(names))]
    params = ", ".join(["NineToothedStream stream"] + [f"NineToothedTensor tensor_{i}" for i in range(n_tensors)]
                       + [f"{t} config_{i}" for i, t in enumerate(ctypes_)])
    proto = f"NineToothedResult launch_{base}({params})"
    forward = ", ".join(["stream"] + [f"tensor_{i}" for i in range(n_tensors)])
    variant_params = ", ".join(["NineToothedStream"] + ["NineToothedTensor"] * n_tensors)
    decls, branches, seen = [], [], set()
    for (config, name, _, _), v in zip(launchers, values):
        decls.append(f'extern "C" NineToothedResult launch_{name}({variant_params});')
        if v in seen:
            continue
        seen.add(v)
        cond = " && ".join(f"config_{i} == {repr(x) if isinstance(x, float) else int(x)}" for i, x in enumerate(v))
        branches.append(f"  if ({cond or 'true'}) return launch_{name}({forward});")
    guard = f"NINETOOTHED_{base.upper()}_H"
    header = (f"#ifndef {guard}\n#define {guard}\n\n#include \"ninetoothed.h\"\n\n#ifdef __cplusplus\nextern \"C\"\n"
              f"#endif\n{proto};\n\n#endif\n")
    source = (f'// Dispatcher over the configured variants of {base} (MI355X backend).\n#include "{base}.h"\n'
              '#include "nt_mi355x.h"\n\n' + "\n".join(decls) + f'\n\nextern "C" {proto} {{\n'
              + "\n".join(branches) + "\n  return NT_ERR_INVALID;  // no variant was built for this configuration\n}\n")
    from ninetoothed_amd.backends import cpp_export

    out.mkdir(parents=True, exist_ok=True)
    (out / "ninetoothed.h").write_text(cpp_export.HEADER)
    (out / f"{base}.h").write_text(header)
    src = out / f"{base}.cpp"
    src.write_text(source)
    lib = out / f"lib{base}.so"
    include = Path(__file__).resolve().parents[1] / "include"
    libs = sorted({str(Path(p)) for *_, p, _ in launchers})
    # Host code only (it calls the variants' launchers): the system C++ compiler, with the HIP
    # runtime API header for hipStream_t.
    cmd = ["g++", "-shared", "-fPIC", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{out}", f"-I{include}",
           "-I/opt/rocm/include", str(src), *libs, *sorted({f"-Wl,-rpath,{Path(p).parent}" for p in libs}),
           "-o", str(lib)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        return {"unavailable": f"g++ failed: {r.stderr[-2000:]}"}
    return {"header": str(out / f"{base}.h"), "source": str(src), "library": str(lib), "symbol": f"launch_{base}"}


def _manifest(built):
    import json

    if built is None or built.manifest_path is None:
        return {}
    try:
        return json.loads(Path(built.manifest_path).read_text())
    except (OSError, ValueError):
        return {}
