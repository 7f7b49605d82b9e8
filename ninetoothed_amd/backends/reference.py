"""This backend behind the reference's own plugin points.

``register(ninetoothed)``, called with the imported reference package, installs this backend in
the reference's three registries:

* the SSA pass registry: the ``ssa.hip.optimize_schedule`` pass that the reference requires of
  every ``Target`` member (``backends/registry.py:24-55``; the default pipeline runs it by name,
  ``compiler/passes.py:846-858``), registered through ``register_pass_bundle``
  (``backends/registry.py:11-21``) into every pass registry the reference creates from then on
  and into the default one if it exists;
* the backend registry (``backends/__init__.py:22-43``): a ``Backend`` whose ``emit`` returns an
  ``Artifact`` carrying the metadata the reference's driver derives the launch ABI from
  (``variables``, ``outputs``, ``shape_params``, ``target``, ``tensors``, ``program_mode`` and the
  schedule of the pipeline: ``emitters/ssa.py:148-180``, ``compiler/driver.py:416-495``);
* the materializer registry (``backends/materializers/__init__.py:7-29``, contract
  ``materializers/base.py:9-48``): a ``Materializer`` that rebuilds the reference's
  ``CompileRequest`` (``compiler/driver.py:37-54``) for this package and returns the
  reference's own ``Handle`` type (``compiler/runtime.py:55-94``) around this package's Handle,
  so the reference's lazy per-dtype specialisation (``runtime.py:177-243``) can drive it.

The request is converted as follows:

* reference ``Tensor`` parameters (``tensor.py:27-127``: ``ndim``, ``shape``, ``dtype``,
  ``jagged_dim``, ``other``, ``constexpr``, ``value``) become this package's ``Tensor``; an
  arranged tensor (a ``jit`` annotation) is converted by converting its source and replaying
  the meta-operations the reference records in ``_history`` (``tensor.py:185-196``), level by
  level, as the reference's own ``eval`` does (``eval.py:72-94``);
* reference ``Symbol`` objects (``symbol.py:20-95``: a name carries its ``constexpr`` / ``meta``
  role as a name prefix, ``naming.py:8-52``, and its bounds as attributes) become this
  package's ``Symbol`` with the same role and bounds; expressions of them are rebuilt with
  the same operators;
* the arrangement and the application (and the plain Python helpers they call) are re-bound:
  copies whose globals, defaults, annotations and closure cells map the reference package,
  its ``language`` module and the names imported from either to this package's objects, so
  that ``ntl.sum``, ``block_size()`` or ``Symbol(...)`` in the user's module resolve here.

What the reference needs from its maintainer before ``register`` can work (this package
cannot add them from outside): a ``Target.HIP = "hip"`` member and its ``"hip"`` alias
(``backends/core.py:11-22``), a platform profile whose ``backend_modes`` name ``hip``
(``targets.py:16-204``), and a ``"hip"`` source suffix for ``Target.HIP`` in the lazy
materialisation's suffix table (``compiler/runtime.py:183-186``).
"""

import ast
import functools
import importlib
import json
import re
import types

import ninetoothed_amd
from ninetoothed_amd import language as ntl
from ninetoothed_amd.compiler import DEFAULT_COMPILER, CompileRequest
from ninetoothed_amd.compiler import load_built_artifact as _load_built_artifact
from ninetoothed_amd.symbol import Symbol
from ninetoothed_amd.tensor import Tensor

TARGET = "hip"
PASS_NAME = "ssa.hip.optimize_schedule"
_PREFIX = re.compile(r"ninetoothed_((?!_).*?)_prefix_")  # the reference's name-prefix pattern
_OPS = {ast.Add: lambda a, b: a + b, ast.Sub: lambda a, b: a - b, ast.Mult: lambda a, b: a * b,
        ast.FloorDiv: lambda a, b: a // b, ast.Mod: lambda a, b: a % b}


class _ModuleView(types.ModuleType):
    """A user module seen through ``ReferenceObjects``: attributes come back converted (an
    application calling ``matmul.application`` of another test module gets the re-bound copy)."""

    def __init__(self, module, objects):
        super().__init__(module.__name__, getattr(module, "__doc__", None))
        self._module, self._objects = module, objects

    def __getattr__(self, name):
        return self._objects.value(getattr(self._module, name))


class ReferenceObjects:
    """Maps the objects of one imported reference package to this package's."""

    def __init__(self, reference):
        self.reference = reference
        self.language = getattr(reference, "language", None)
        self._memo = {}
        self._modules = {}

    def _uses_reference(self, module):
        """Whether a module imports the reference package or its language module."""
        values = getattr(module, "__dict__", {}).values()
        return any(v is self.reference or (self.language is not None and v is self.language) for v in values)

    # ------------------------------------------------------------------ symbols and tensors
    def symbol(self, sym):
        return self._node(sym._node)

    def _node(self, node):
        if isinstance(node, ast.Constant):
            return node.value
        if isinstance(node, ast.Name):
            roles = set(_PREFIX.findall(node.id))
            ref = getattr(node, "symbol", None)
            bounds = {k: getattr(ref, k, None) for k in ("lower_bound", "upper_bound", "power_of_two")}
            return Symbol(_PREFIX.sub("", node.id), constexpr=("constexpr" in roles) or None,
                          meta=("meta" in roles) or None, **{k: v for k, v in bounds.items() if v is not None})
        if isinstance(node, ast.BinOp) and type(node.op) in _OPS:
            return _OPS[type(node.op)](self._node(node.left), self._node(node.right))
        if isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.USub):
            return -self._node(node.operand)
        raise NotImplementedError(f"reference symbol expression `{ast.unparse(node)}` is not supported")

    def tensor(self, t):
        if getattr(t, "source", t) is not t:
            return self._arranged(t)
        sizes = tuple(t.shape)
        shape = tuple(s if isinstance(s, int) else None for s in sizes)
        options = []
        for s in sizes:
            node = getattr(s, "_node", None)
            ref = getattr(node, "symbol", None)
            opts = {k: getattr(ref, k) for k in ("lower_bound", "upper_bound", "power_of_two")
                    if getattr(ref, k, None) is not None}
            if isinstance(node, ast.Name) and "constexpr" in _PREFIX.findall(node.id):
                opts["constexpr"] = True
            options.append(opts)
        return Tensor(len(sizes), shape=shape if any(s is not None for s in shape) else None, dtype=t.dtype,
                      jagged_dim=t.jagged_dim, other=t.other, shape_options=tuple(options),
                      constexpr=t.constexpr or None, value=t.value)

    def _replay(self, tensor, history):
        for func, args, kwargs in history:
            tensor = getattr(tensor, func.__name__)(*self.value(tuple(args)),
                                                    **{k: self.value(v) for k, v in kwargs.items()})
        return tensor

    def _arranged(self, t):
        """An arranged reference tensor: its source converted, then its recorded meta-operations
        replayed on it, and on every level below the outermost the same way."""
        ref_tensor = type(t)
        ours = self._replay(self.tensor(t.source), t._history)
        new, old = ours, t
        while isinstance(old.dtype, ref_tensor):
            new.dtype = self._replay(new.dtype, old.dtype._history)
            new, old = new.dtype, old.dtype
        return ours

    # ------------------------------------------------------------------ values and functions
    def value(self, v):
        ref, lang = self.reference, self.language
        if v is ref:
            return ninetoothed_amd
        if lang is not None and v is lang:
            return ntl
        if lang is not None and v is getattr(lang, "libdevice", None):
            return ntl.libdevice
        if isinstance(v, getattr(ref, "Symbol", ())):
            return self.symbol(v)
        if isinstance(v, getattr(ref, "Tensor", ())):
            return self.tensor(v)
        if isinstance(v, types.ModuleType):
            if v.__name__ not in self._modules:
                self._modules[v.__name__] = _ModuleView(v, self) if self._uses_reference(v) else v
            return self._modules[v.__name__]
        if isinstance(v, (tuple, list)):
            return type(v)(self.value(x) for x in v)
        if isinstance(v, functools.partial):
            return functools.partial(self.value(v.func), *self.value(v.args),
                                     **{k: self.value(x) for k, x in v.keywords.items()})
        if callable(v):
            for module, ours in ((ref, ninetoothed_amd), (lang, ntl)):
                name = getattr(v, "__name__", None)
                if module is not None and name and getattr(module, name, None) is v and hasattr(ours, name):
                    return getattr(ours, name)
            if isinstance(v, types.FunctionType):
                return self.function(v)
        return v

    def function(self, func):
        """A copy of a user function whose globals, defaults and closure cells are mapped."""
        if id(func) in self._memo:
            return self._memo[id(func)][1]
        scope = dict(func.__globals__)
        copy = types.FunctionType(func.__code__, scope, func.__name__, None, None)
        self._memo[id(func)] = (func, copy)  # first, so that recursion meets the copy
        names = set()

        def collect(code):
            names.update(code.co_names)
            for c in code.co_consts:
                if isinstance(c, types.CodeType):
                    collect(c)

        collect(func.__code__)
        for n in names & set(scope):
            scope[n] = self.value(scope[n])
        closure = None
        if func.__closure__:
            closure = tuple(types.CellType(self.value(c.cell_contents)) for c in func.__closure__)
        defaults = self.value(func.__defaults__) if func.__defaults__ else None
        rebuilt = types.FunctionType(func.__code__, scope, func.__name__, defaults, closure)
        rebuilt.__kwdefaults__ = {k: self.value(x) for k, x in (func.__kwdefaults__ or {}).items()} or None
        rebuilt.__qualname__, rebuilt.__module__ = func.__qualname__, func.__module__
        rebuilt.__annotations__ = {k: self.value(x) for k, x in func.__annotations__.items()}
        rebuilt.__dict__.update(func.__dict__)
        self._memo[id(func)] = (func, rebuilt)
        return rebuilt

    def request(self, req, output_dir=None):
        """This package's CompileRequest for a reference CompileRequest."""
        return CompileRequest(
            application=self.value(req.application),
            arrangement=self.value(req.arrangement) if req.arrangement is not None else None,
            tensors=tuple(self.tensor(t) for t in req.tensors) if req.tensors else None,
            backend=TARGET, caller=req.caller, kernel_name=req.kernel_name, output_dir=output_dir,
            num_warps=req.num_warps, num_stages=req.num_stages, max_num_configs=req.max_num_configs,
            backend_options=dict(req.backend_options or {}))


def _module(reference, path):
    return importlib.import_module(f"{reference.__name__}.{path}")


def hip_target(reference):
    """The reference's ``Target`` member for this backend (a maintainer's addition)."""
    core = _module(reference, "backends.core")
    try:
        return core.normalize_target(TARGET)
    except ValueError:
        raise RuntimeError(
            "the reference has no `hip` backend target: add `HIP = \"hip\"` to `Target` and the alias "
            "`\"hip\": Target.HIP` (ninetoothed/backends/core.py) before registering this backend") from None


def optimize_schedule_pass(reference):
    """The reference's per-backend schedule pass for ``hip`` (contract ``compiler/passes.py:408-540``).

    It proposes no schedule candidates and no tiles: the hand-written kernels choose their
    own tiling per call, as non-Triton backends may (``compiler/driver.py:328-333``).  Its
    policy keeps ``linalg.dot`` whole (``preserve_linalg``, read by ``DecomposeLinalg``,
    ``passes.py:335-366``) and records that the kernel family is chosen at call time; the
    granularity stays what the reference's ``SelectSchedule`` found."""
    passes = _module(reference, "compiler.passes")
    target = hip_target(reference)

    class HipOptimizeSchedule(passes.OptimizeSchedule):
        name = PASS_NAME
        supported_backends = (target,)

        def schedule_candidates(self, analysis, schedule, context):
            return ()

        def optimization_policy(self, backend, analysis, schedule):
            return {"preserve_linalg": bool(analysis.get("has_dot")), "kernel_selection": "family-at-call-time",
                    "library": "libnt_mi355x.so"}

    HipOptimizeSchedule.__qualname__ = HipOptimizeSchedule.__name__
    return HipOptimizeSchedule


def register_ssa_passes(registry, reference):
    """Register the ``hip`` schedule pass into one of the reference's pass registries, as each
    reference backend's ``register_ssa_passes`` does (e.g. ``backends/cuda.py:166-173``)."""
    _module(reference, "backends.registry").register_pass_bundle(
        registry, backend=hip_target(reference), optimize_schedule=optimize_schedule_pass(reference))


def _install_pass_bundle(reference):
    """Make every pass registry the reference creates carry the ``hip`` pass (its
    ``register_passes`` validates the contract for every ``Target`` member,
    ``backends/registry.py:24-55``), and add it to the default registry if one exists."""
    bundles = _module(reference, "backends.registry")
    original = bundles.register_passes
    if not getattr(original, "_ninetoothed_amd", False):
        def register_passes(registry):
            register_ssa_passes(registry, reference)
            original(registry)

        register_passes._ninetoothed_amd = True
        bundles.register_passes = register_passes
    passes = _module(reference, "compiler.passes")
    default = getattr(passes, "_DEFAULT_REGISTRY", None)
    if default is not None:
        try:
            default.get(PASS_NAME)
        except KeyError:
            register_ssa_passes(default, reference)


def _walk(operations):
    for op in operations:
        yield op
        for region in op.regions:
            yield from _walk(region.operations)


def artifact_metadata(kernel, reference):
    """What the reference's driver reads from an ``Artifact`` (``compiler/driver.py:416-495``,
    ``emitters/ssa.py:148-180``), for a reference ``Kernel`` after the ``hip`` pipeline.

    ``outputs`` are the tensors the application stores to (``mem.store``) or adds to
    atomically through a data pointer (``mem.atomic_add``), in program order;
    ``variables`` the other non-constexpr parameters; ``shape_params`` the symbols the
    tensors' shapes and access templates use, from the reference's own scan
    (``emitters/ssa.py:4131-4185``) so the launch ABI the driver derives is the one its
    other backends get."""
    program = kernel.ssa
    block = program.blocks[0] if program.blocks else None
    ops = tuple(_walk(block.operations)) if block is not None else ()
    by_result = {r.name: op for op in ops for r in op.results}
    outputs = []
    for op in ops:
        name = None
        if op.opcode == "mem.store" and len(op.operands) == 2:
            name = op.operands[1]
        elif op.opcode == "mem.atomic_add" and op.operands:
            ptr = by_result.get(op.operands[0])
            if ptr is not None and ptr.opcode == "mem.data_ptr" and ptr.operands:
                name = ptr.operands[0]
        if name is not None and name not in outputs:
            outputs.append(name)
    if not outputs:
        outputs = [v.name for v in program.outputs]
    variables = tuple(t.name for t in kernel.tensors if t.name not in outputs and not t.constexpr)
    emitter = _module(reference, "backends.emitters.ssa")
    shape_params = tuple(emitter._shape_params(kernel.tensors, block.operations if block is not None else ()))
    ir = _module(reference, "ir")
    schedule = dict(program.metadata.get("schedule", {}))
    granularity = schedule.get("granularity")
    return {
        "backend": TARGET,
        "target": dict(kernel.metadata.get("target", {})),
        "kernel_name": kernel.kernel_name,
        "lowering_ir": "ssa.Program",
        "source_route": "ninetoothed_amd families (hand-written gfx950 kernels, chosen per call)",
        "shape_params": shape_params,
        "variables": variables,
        "outputs": tuple(outputs),
        "auxiliary_bindings": (),
        "tensors": [ir.ir_to_dict(t) for t in kernel.tensors],
        "ssa_metadata": dict(program.metadata),
        "ssa_pass_trace": tuple(program.metadata.get("pass_trace", ())),
        "ssa_schedule": schedule,
        "ssa_optimization": dict(program.metadata.get("optimization", {})),
        # The kernels are hand-written per family; the grid is chosen by the library per call.
        "program_mode": {"block": granularity in ("blocked-linalg", "exp-reduction-dot-region"),
                         "cooperative_reduction": False, "scalar": False,
                         "vector": granularity in ("parallel-reduction", "elementwise-grid")},
        "library": "libnt_mi355x.so",
    }


def reference_backend(reference):
    """A ``Backend`` of the reference (``backends/core.py:81-105``) for ``hip``."""
    core = _module(reference, "backends.core")
    target = hip_target(reference)

    class HipReferenceBackend(core.Backend):
        name = target
        capability = core.Capability(name=target, emits_source=False, can_execute=True,
                                     notes=("hand-written gfx950 kernels in libnt_mi355x.so, chosen per call by "
                                            "ninetoothed_amd's family matchers",))
        supported_options = frozenset()

        def emit(self, kernel):
            metadata = artifact_metadata(kernel, reference)
            name = kernel.kernel_name
            source = ("// " + name + ": served by the hand-written gfx950 kernels of libnt_mi355x.so;\n"
                      "// the kernel family is chosen per call (ninetoothed_amd.families).\n")
            return core.Artifact(backend=target, kernel_name=name, language="hip",
                                 sources={f"{name}.hip": source,
                                          f"{name}.hip.json": json.dumps(
                                              {k: metadata[k] for k in ("variables", "outputs", "shape_params",
                                                                        "program_mode")}, default=list)},
                                 entrypoint=None, metadata=metadata)

    HipReferenceBackend.__qualname__ = HipReferenceBackend.__name__
    return HipReferenceBackend()


class _Specialized:
    """This package's Handle with the values the reference specialised its compilation on.

    The reference's lazy specialisation compiles per call-time key with the values of the
    launch ABI's constexpr and meta bindings substituted (``compiler/runtime.py:206-243``)
    and then passes on only the keywords the specialised ABI still lists
    (``runtime.py:1188-1195``): a constexpr such as conv2d's ``padding_h`` is dropped from
    the call.  This Handle specialises itself per call, so those values are handed back to
    it here, for every keyword it takes that the call leaves out."""

    def __init__(self, handle, request):
        self.handle = handle
        accepted = set(handle._abi["meta_args"]) | set(handle._abi["public_args"])
        values = {_PREFIX.sub("", str(k)): v for k, v in dict(request.specialization_values or {}).items()}
        self.fixed = {k: v for k, v in values.items() if k in accepted}
        self._built_artifact = getattr(handle, "_built_artifact", None)

    def __call__(self, *args, **kwargs):
        if self.fixed:
            given = set(self.handle._abi["public_args"][:len(args)]) | set(kwargs)
            kwargs = {**{k: v for k, v in self.fixed.items() if k not in given}, **kwargs}
        return self.handle(*args, **kwargs)


class ReferenceMaterializer:
    """The reference's ``Materializer`` contract (``materializers/base.py:9-48``) for ``hip``.

    Both materialisations return the reference's own ``Handle`` around this package's Handle
    (its source file, written to the reference's cache for JIT or to ``output_dir`` for AOT,
    is the artifact's one-line description).  AOT also writes this package's built artifact
    under ``output_dir/hip/``, which ``load_built_artifact`` reloads without the
    application."""

    target = TARGET

    def __init__(self, reference):
        self.reference = reference
        self.objects = ReferenceObjects(reference)

    def _wrap(self, compilation, ours, source_dir=None):
        from pathlib import Path

        runtime = _module(self.reference, "compiler.runtime")
        cache = _module(self.reference, "compiler.cache")
        artifact = compilation.artifact
        key = cache.compilation_cache_key(compilation)
        if source_dir is None:
            source = cache.write_source(artifact.kernel_name, artifact.primary_source, "hip", cache_key=key)
        else:
            source = Path(source_dir) / f"{artifact.kernel_name}.hip"
            source.parent.mkdir(parents=True, exist_ok=True)
            source.write_text(artifact.primary_source)
        return runtime.Handle(compilation, None, ours, source)

    def jit_materialize(self, compilation, *, output_dir=None):
        ours = DEFAULT_COMPILER.materialize(self.objects.request(compilation.request), mode="jit")
        return self._wrap(compilation, _Specialized(ours, compilation.request))

    def aot_build(self, compilation, *, output_dir):
        import pickle
        from pathlib import Path

        out = Path(output_dir) / "hip"
        ours = DEFAULT_COMPILER.materialize(self.objects.request(compilation.request, out), output_dir=out,
                                            mode="aot")
        (out / f"{compilation.artifact.kernel_name}.built.pkl").write_bytes(pickle.dumps(ours._built_artifact))
        return self._wrap(compilation, _Specialized(ours, compilation.request), source_dir=output_dir)

    def load_built_artifact(self, built):
        """This package's Handle for a reference ``BuiltArtifact`` written by ``aot_build``."""
        import pickle
        from pathlib import Path

        path = Path(built.source_path).parent / "hip" / f"{built.source.kernel_name}.built.pkl"
        return _load_built_artifact(pickle.loads(path.read_bytes()))


def register(reference, *, replace=False):
    """Install this backend in the reference's pass, backend and materializer registries;
    returns the ``Backend`` and the ``Materializer``."""
    _install_pass_bundle(reference)
    backend = reference_backend(reference)
    _module(reference, "backends").default_registry().register(backend, replace=replace)
    materializers = _module(reference, "backends.materializers")
    materializers.materializer_for("triton")  # builds the reference's default registry
    materializer = ReferenceMaterializer(reference)
    materializers._DEFAULT_REGISTRY.register(materializer, replace=replace)
    return backend, materializer
