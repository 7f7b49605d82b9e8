"""Compiler driver: arrangement + application + tensors -> Compilation -> Handle.

Follows the reference's driver (``src/ninetoothed/compiler/driver.py``): ``make``
(176-216) runs the arrangement on deep copies of the symbolic tensors (283-287),
lowers the application, asks the selected backend to ``emit`` an ``Artifact``, derives
the launch ABI (416-495: public arguments in application order, meta/constexpr
keyword arguments, outputs) and materialises a ``Handle`` through the backend's
``Materializer``.  ``jit`` takes the arrangement from parameter annotations (272-281).

For the MI355X backend emission does not generate source: it records the program
(application parameters, arranged tensors, the symbols they use and the schedule
granularity) and the kernel family is chosen per call-time specialisation, when
dtypes, shapes, strides and constexpr values are known.
"""

import copy
import inspect
from dataclasses import dataclass, field, replace

from ninetoothed_amd import families, frontend, jagged
from ninetoothed_amd.backends import default_registry
from ninetoothed_amd.backends.materializers import materializer_for
from ninetoothed_amd.errors import LoweringError
from ninetoothed_amd.symbol import default_meta_value
from ninetoothed_amd.targets import resolve_target_context
from ninetoothed_amd.tensor import BoundView, Tensor


@dataclass(frozen=True)
class CompileRequest:
    application: object
    arrangement: object = None
    tensors: tuple = None
    backend: object = None
    platform: object = None
    compute_arch: object = None
    caller: str = "torch"
    kernel_name: str = None
    output_dir: object = None
    num_warps: object = None
    num_stages: object = None
    max_num_configs: object = None
    pipeline: object = None
    pass_options: object = None
    backend_options: dict = field(default_factory=dict)


@dataclass
class ParamSpec:
    name: str
    source_ndim: int
    level_ndims: tuple
    static_shape: tuple
    dtype: object
    constexpr: bool
    shape_symbols: tuple  # (symbol name or None) per source dim
    constexpr_value: object = None  # fixed at definition (``Tensor(0, constexpr=True, value=...)``)
    jagged_dim: object = None  # the ragged dim of a jagged source (ninetoothed_amd.jagged), else None


@dataclass
class Compilation:
    request: CompileRequest
    kernel: "KernelProgram"
    artifact: object
    target: object
    launch_abi: dict


class KernelProgram:
    """The arranged program, ready to be specialised at call time.

    The application is lowered once per set of constexpr values (their `if`s fold) and the
    lowered programs are cached; a program rebuilt from a built artifact (``from_bundle``)
    carries those lowered programs and needs the application only for constexpr values it
    was not built with (then it imports it by module and qualified name, if it can)."""

    def __init__(self, request, params, arranged, specs, symbols, granularity, outputs):
        self.request = request
        self.name = request.kernel_name or request.application.__name__
        self.params = params
        self.arranged = dict(zip(params, arranged))
        self.param_specs = specs
        self.symbols = symbols  # name -> Symbol (meta/constexpr flags)
        self.granularity = granularity
        self.outputs = outputs
        self.application = request.application
        self.application_ref = _application_ref(request.application)
        self._lowered = {}

    # ------------------------------------------------------------ built artifacts
    def bundle(self):
        """Everything call-time specialisation needs, as picklable data (no application)."""
        return {"name": self.name, "params": self.params, "arranged": self.arranged, "specs": self.param_specs,
                "symbols": self.symbols, "granularity": self.granularity, "outputs": self.outputs,
                "lowered": dict(self._lowered), "application_ref": self.application_ref}

    @classmethod
    def from_bundle(cls, bundle):
        self = cls.__new__(cls)
        self.request = None
        self.name = bundle["name"]
        self.params = bundle["params"]
        self.arranged = bundle["arranged"]
        self.param_specs = bundle["specs"]
        self.symbols = bundle["symbols"]
        self.granularity = bundle["granularity"]
        self.outputs = bundle["outputs"]
        self.application = None
        self.application_ref = bundle["application_ref"]
        self._lowered = dict(bundle["lowered"])
        return self

    def infos(self, public=None):
        """ParamInfo per parameter; constexpr values from ``public`` or fixed at definition."""
        infos = []
        for spec in self.param_specs:
            if spec.source_ndim == 0:
                value = public[spec.name] if public is not None and spec.name in public else spec.constexpr_value
                infos.append(frontend.ParamInfo(spec.name, (), 0, spec.constexpr,
                                                _plain(value) if spec.constexpr else None))
            else:
                infos.append(frontend.ParamInfo(spec.name, spec.level_ndims, spec.source_ndim))
        return infos

    def lowered(self, infos):
        key = tuple((i.name, repr(i.constexpr_value)) for i in infos if i.constexpr)
        program = self._lowered.get(key)
        if program is None:
            application = self.application or _import_application(self.application_ref)
            if application is None:
                raise LoweringError(
                    f"`{self.name}` was built for constexpr values {[dict(k) for k in self._lowered] or 'none'}; "
                    f"{dict(key)} needs its application, which cannot be imported"
                )
            program = frontend.lower(application, infos)
            self._lowered[key] = program
        return program

    def prelower(self):
        """Lower for the constexpr values fixed at definition (all of them, or nothing)."""
        if all(s.constexpr_value is not None for s in self.param_specs if s.constexpr):
            self.lowered(self.infos())

    def static_values(self):
        """Meta-device stand-ins for a call, when every shape and dtype is fixed at definition."""
        import torch

        from ninetoothed_amd.dtype import normalize_dtype

        public = {}
        for spec in self.param_specs:
            if spec.source_ndim == 0:
                if spec.constexpr:
                    if spec.constexpr_value is None:
                        return None
                    public[spec.name] = spec.constexpr_value
                else:
                    public[spec.name] = 0.0
                continue
            if spec.dtype is None or any(s is None for s in spec.static_shape):
                return None
            dtype = getattr(torch, normalize_dtype(spec.dtype), None)
            if dtype is None:
                return None
            public[spec.name] = torch.empty(spec.static_shape, dtype=dtype, device="meta")
        return public

    @property
    def meta_args(self):
        shape_names = {n for s in self.param_specs for n in s.shape_symbols if n}
        return tuple(sorted(n for n, sym in self.symbols.items() if n not in shape_names and (sym.meta or sym.constexpr)))

    def environment(self, public, meta):
        env = {}
        for spec in self.param_specs:
            if spec.source_ndim == 0:
                continue
            value = public[spec.name]
            shape = jagged.padded_shape(value) if jagged.is_jagged(value) else value.shape
            for name, size in zip(spec.shape_symbols, shape):
                if name is not None:
                    env[name] = int(size)
        shape_names = set(env)
        for name, sym in self.symbols.items():
            if name in shape_names:
                continue
            if name in meta:
                env[name] = int(meta[name])
            elif sym.meta:
                env[name] = default_meta_value(sym)
            elif sym.constexpr:
                raise TypeError(f"Missing launch meta-parameter `{name}`.")
            else:
                raise TypeError(f"No value for symbol `{name}`.")
        return env

    def specialize(self, public, meta, tune=False):
        """The kernel plan for a call; with ``tune``, a ``TunedPlan`` over every fitting plan
        when there are several and the program updates no tensor it reads."""
        ctx = self.context(public, meta)
        if tune and not families.updates_an_input(ctx.program):
            plans = families.candidates(ctx)
            if len(plans) > 1:
                return families.TunedPlan(plans, namespace=f"{self.name}:{self.application_ref}")
        return families.select(ctx)

    def context(self, public, meta):
        env = self.environment(public, meta)
        views, dtypes = {}, {}
        for spec in self.param_specs:
            if spec.source_ndim == 0:
                views[spec.name] = None
                continue
            views[spec.name] = BoundView(self.arranged[spec.name], env)
            dtypes[spec.name] = public[spec.name].dtype
        infos = self.infos(public)
        program = self.lowered(infos)
        ctx = families.CallContext(program, views, public, {i.name: i for i in infos}, dtypes)
        application = self.application or _import_application(self.application_ref)
        if application is not None:
            # the generic kernels re-lower with loops unrolled once trip counts are known
            ctx.relower = lambda unroll: frontend.lower(application, infos, unroll=unroll)
        return ctx


def _plain(v):
    if hasattr(v, "item"):
        return v.item()
    return v


def _application_ref(application):
    """(module, qualified name) of an importable application, else None."""
    module, qualname = getattr(application, "__module__", None), getattr(application, "__qualname__", "")
    if not module or "<" in qualname:
        return None
    return module, qualname


def _import_application(ref):
    if ref is None:
        return None
    import importlib

    try:
        obj = importlib.import_module(ref[0])
        for part in ref[1].split("."):
            obj = getattr(obj, part)
    except (ImportError, AttributeError):
        return None
    return obj


def _arrangement_from_annotations(application):
    sig = inspect.signature(application)
    annotated = []
    for name, p in sig.parameters.items():
        if not isinstance(p.annotation, Tensor):
            raise LoweringError(f"`jit` needs every parameter annotated with an arranged Tensor (`{name}` is not)")
        annotated.append(p.annotation)

    def arrangement(*tensors):
        return tuple(tensors)

    return arrangement, tuple(annotated)


def _shape_symbol_names(source):
    names = []
    for size in source.shape:
        names.append(size.name if hasattr(size, "name") and getattr(size, "name", None) else None)
    return tuple(names)


def _discover_outputs(application, params, arranged):
    """Parameters the application assigns (stores), any constexpr branch included."""
    infos = []
    for name, t in zip(params, arranged):
        if not isinstance(t, Tensor) or t.source.ndim == 0:
            infos.append(frontend.ParamInfo(name, (), 0, constexpr=bool(getattr(t, "constexpr", False)),
                                            constexpr_value=_BothBranches()))
        else:
            infos.append(frontend.ParamInfo(name, tuple(l.ndim for l in t.levels()[1:]), t.source.ndim))
    lowerer = _ExploringLowerer(application, infos)
    program = lowerer.lower()
    written = set(program.stores) | set(frontend.effect_targets(program))
    return tuple(n for n in params if n in written), program


class _BothBranches:
    """Marker constexpr value: output discovery walks both arms of an `if`."""


class _ExploringLowerer(frontend.Lowerer):
    def data(self, v):
        # a constexpr used as a value: any constant will do to find the stored parameters
        if isinstance(v, _BothBranches):
            return self.const(1)
        return super().data(v)

    def _stmt(self, frame, s):
        import ast

        if isinstance(s, ast.If):
            test = self._expr(frame, s.test)
            if isinstance(test, _BothBranches) or isinstance(test, frontend.Value):
                self._block(frame, s.body)
                self._block(frame, s.orelse)
                return
        super()._stmt(frame, s)


def _granularity(program):
    """Schedule granularity, in the reference's vocabulary (compiler/passes.py:1070-1084)."""
    ops = {v.op for value in list(program.stores.values()) + [u for l in program.loops.values() for u in l.update.values()]
           for v in families._walk(value)}
    if "dot" in ops and ("math" in ops or "reduce" in ops):
        return "exp-reduction-dot-region"
    if "dot" in ops:
        return "blocked-linalg"
    if "reduce" in ops:
        return "parallel-reduction"
    return "elementwise-grid"


def compile_kernel(request):
    target = resolve_target_context(request.backend, request.platform, request.compute_arch)
    backend = default_registry().get(target.backend)
    backend_options = backend.normalize_options(request.backend_options or {})
    application = request.application
    params = frontend.parameter_names(application)

    if request.arrangement is None:
        arrangement, tensors = _arrangement_from_annotations(application)
    else:
        # `tensors` are the arrangement's arguments: besides one Tensor per application
        # parameter they may carry other values the arrangement reads (e.g. slices).
        arrangement, tensors = request.arrangement, tuple(request.tensors)
    copies = copy.deepcopy(tensors)
    arranged = arrangement(*copies)
    if not isinstance(arranged, tuple):
        arranged = tuple(arranged) if isinstance(arranged, list) else (arranged,)
    if len(arranged) != len(params):
        raise LoweringError(f"the arrangement returns {len(arranged)} tensors for {len(params)} application parameters")

    specs, symbols = [], {}
    for name, original, t in zip(params, tensors, arranged):
        source = t.source if isinstance(t, Tensor) else t
        if not isinstance(source, Tensor):
            raise LoweringError(f"arranged parameter `{name}` is not a Tensor")
        static = tuple(s if isinstance(s, int) else None for s in source.shape)
        specs.append(ParamSpec(
            name=name,
            source_ndim=source.ndim,
            level_ndims=tuple(l.ndim for l in t.levels()[1:]) if source.ndim else (),
            static_shape=static,
            dtype=source.dtype if isinstance(source.dtype, str) else None,
            constexpr=bool(source.constexpr),
            shape_symbols=_shape_symbol_names(source),
            constexpr_value=source.value if source.constexpr else None,
            jagged_dim=getattr(source, "jagged_dim", None),
        ))
        if source.ndim:
            symbols.update(t.symbols())
    outputs, explored = _discover_outputs(application, params, arranged)
    granularity = _granularity(explored)
    kernel = KernelProgram(request, params, arranged, specs, symbols, granularity, outputs)
    kernel = backend.prepare_for_emission(kernel)
    artifact = backend.emit(kernel)
    abi = {
        "public_args": tuple(params),
        "meta_args": kernel.meta_args,
        "outputs": outputs,
        "options": dict(backend_options),
    }
    return Compilation(request=request, kernel=kernel, artifact=artifact, target=target, launch_abi=abi)


class Compiler:
    def compile(self, request):
        return compile_kernel(request)

    def materialize(self, request, *, output_dir=None, mode=None):
        """A Handle for a CompileRequest or an existing Compilation (reference
        ``compiler/runtime.py:1450-1472``): ``mode`` "jit" or "aot" (default: "jit" for
        ``caller="torch"``, else "aot"); AOT needs an output directory."""
        compilation = request if isinstance(request, Compilation) else self.compile(request)
        req = compilation.request
        output_dir = output_dir if output_dir is not None else req.output_dir
        materializer = materializer_for(compilation.target.backend)
        if mode is None:
            mode = "jit" if req.caller == "torch" else "aot"
        if mode == "aot":
            if output_dir is None:
                raise ValueError("AOT materialization requires an output directory.")
            return materializer.aot_build(compilation, output_dir=output_dir)
        if mode != "jit":
            raise ValueError(f"Unknown materialization mode `{mode}`.")
        return materializer.jit_materialize(compilation, output_dir=output_dir)


def load_built_artifact(built):
    """Reload a Handle from a built artifact without the application (reference
    ``compiler/runtime.py:1475-1481``)."""
    return materializer_for(built.source.backend).load_built_artifact(built)


DEFAULT_COMPILER = Compiler()


def make(arrangement, application, tensors, caller="torch", kernel_name=None, output_dir=None, num_warps=None,
         num_stages=None, max_num_configs=None, *, backend=None, platform=None, compute_arch=None, pipeline=None,
         pass_options=None, **backend_options):
    """``ninetoothed.make`` (reference ``src/ninetoothed/make.py:6-41``) for the MI355X backend.

    ``num_warps``, ``num_stages`` and ``max_num_configs`` are accepted for drop-in
    compatibility; the hand-written kernels choose their tiles themselves.
    """
    return DEFAULT_COMPILER.materialize(CompileRequest(
        application=application, arrangement=arrangement, tensors=tuple(tensors), backend=backend, platform=platform,
        compute_arch=compute_arch, caller=caller, kernel_name=kernel_name, output_dir=output_dir, num_warps=num_warps,
        num_stages=num_stages, max_num_configs=max_num_configs, pipeline=pipeline, pass_options=pass_options,
        backend_options=backend_options,
    ))


def jit(func=None, *, backend=None, platform=None, compute_arch=None, caller="torch", kernel_name=None, num_warps=None,
        num_stages=None, max_num_configs=None, pipeline=None, pass_options=None, _prettify=False, **backend_options):
    """``ninetoothed.jit`` (reference ``src/ninetoothed/compiler/jit.py:6-46``): annotations are the arrangement."""
    if _prettify:
        raise NotImplementedError("The legacy `_prettify` source rewrite is not supported.")

    def wrapper(application):
        return DEFAULT_COMPILER.materialize(CompileRequest(
            application=application, backend=backend, platform=platform, compute_arch=compute_arch, caller=caller,
            kernel_name=kernel_name or application.__name__, num_warps=num_warps, num_stages=num_stages,
            max_num_configs=max_num_configs, pipeline=pipeline, pass_options=pass_options,
            backend_options=backend_options,
        ))

    return wrapper if func is None else wrapper(func)
