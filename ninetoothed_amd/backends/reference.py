"""This backend behind the reference's own plugin points.

``register(ninetoothed)``, called with the imported reference package, adds two objects to the
reference's registries: a ``Backend`` for the ``"hip"`` target (the reference's
``backends/__init__.py:22-32`` registry; ``backend_id_for`` accepts plugin names,
``backends/core.py:134-140``) and a ``Materializer`` (``backends/materializers/__init__.py:7-29``,
contract ``materializers/base.py:9-48``).  The reference's compile driver lowers the request for
every target before it materializes (``compiler/driver.py:58-97``); this backend lowers the
application itself, so the ``Backend``'s artifact only names the kernel and the ``Materializer``
rebuilds the reference's ``CompileRequest`` (``compiler/driver.py:37-54``) for this package:

* reference ``Tensor`` parameters (``tensor.py:27-120``: ``ndim``, ``shape``, ``dtype``,
  ``jagged_dim``, ``other``, ``constexpr``, ``value``) become this package's ``Tensor``;
* reference ``Symbol`` objects (``symbol.py:20-95``: a name carries its ``constexpr`` / ``meta``
  role as a name prefix, ``naming.py:8-52``, and its bounds as attributes) become this
  package's ``Symbol`` with the same role and bounds; expressions of them are rebuilt with
  the same operators;
* the arrangement and the application (and the plain Python helpers they call) are re-bound:
  copies whose globals, defaults and closure cells map the reference package, its
  ``language`` module and the names imported from either to this package's objects, so that
  ``ntl.sum``, ``block_size()`` or ``Symbol(...)`` in the user's module resolve here.

The ``Target.HIP`` enum member and the ``amd-mi355x`` platform profile, which the reference's
target resolution needs before a request reaches the registries, are the maintainer's
additions to the reference (``backends/core.py:11-22``, ``targets.py:16-204``).
"""

import ast
import functools
import re
import types

import ninetoothed_amd
from ninetoothed_amd import language as ntl
from ninetoothed_amd.compiler import DEFAULT_COMPILER, CompileRequest
from ninetoothed_amd.compiler import load_built_artifact as _load_built_artifact
from ninetoothed_amd.symbol import Symbol
from ninetoothed_amd.tensor import Tensor

TARGET = "hip"
_PREFIX = re.compile(r"ninetoothed_((?!_).*?)_prefix_")  # the reference's name-prefix pattern
_OPS = {ast.Add: lambda a, b: a + b, ast.Sub: lambda a, b: a - b, ast.Mult: lambda a, b: a * b,
        ast.FloorDiv: lambda a, b: a // b, ast.Mod: lambda a, b: a % b}


class ReferenceObjects:
    """Maps the objects of one imported reference package to this package's."""

    def __init__(self, reference):
        self.reference = reference
        self.language = getattr(reference, "language", None)
        self._memo = {}

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
            raise NotImplementedError("arranged reference tensors (jit annotations) are not converted; "
                                      "pass an arrangement and plain tensors")
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


class ReferenceMaterializer:
    """The reference's ``Materializer`` contract (``materializers/base.py:9-48``) for ``"hip"``."""

    target = TARGET

    def __init__(self, reference):
        self.objects = ReferenceObjects(reference)

    def jit_materialize(self, compilation, *, output_dir=None):
        return DEFAULT_COMPILER.materialize(self.objects.request(compilation.request, output_dir),
                                            output_dir=output_dir, mode="jit")

    def aot_build(self, compilation, *, output_dir):
        return DEFAULT_COMPILER.materialize(self.objects.request(compilation.request, output_dir),
                                            output_dir=output_dir, mode="aot")

    def load_built_artifact(self, built):
        return _load_built_artifact(built)


def reference_backend(reference):
    """A ``Backend`` of the reference (``backends/core.py:85-110``) for ``"hip"``: no source of
    its own; its artifact names the kernel, and the materializer lowers the application."""
    core = reference.backends.core

    class HipReferenceBackend(core.Backend):
        name = TARGET
        capability = core.Capability(name=TARGET, emits_source=False, can_execute=True,
                                     notes=("lowered and run by ninetoothed_amd on MI355X",))
        supported_options = frozenset()

        def emit(self, kernel):
            name = getattr(kernel, "name", "kernel")
            return core.Artifact(backend=TARGET, kernel_name=name, language="hip", sources={f"{name}.hip": ""},
                                 metadata={})

    return HipReferenceBackend()


def register(reference, *, replace=False):
    """Register this backend's ``Backend`` and ``Materializer`` with the reference's default
    registries; returns the two objects."""
    backend = reference_backend(reference)
    reference.backends.default_registry().register(backend, replace=replace)
    materializers = reference.backends.materializers
    materializers.materializer_for("triton")  # builds the reference's default registry
    materializer = ReferenceMaterializer(reference)
    materializers._DEFAULT_REGISTRY.register(materializer, replace=replace)
    return backend, materializer
