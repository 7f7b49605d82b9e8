"""Materializers: turn a Compilation into a callable Handle.

Contract as the reference's ``Materializer`` (``src/ninetoothed/backends/materializers/base.py:9-48``):
``jit_materialize``, ``aot_build`` and ``load_built_artifact``, registered per backend id.
The HIP materializer loads the prebuilt ``libnt_mi355x.so`` (it never compiles at run
time) and wraps the compilation in a ``Handle``.  ``aot_build`` writes a program bundle
and a manifest into the caller's output directory; ``load_built_artifact`` rebuilds the
Handle from them without the application.
"""

import hashlib
import json
import pickle
from abc import ABC, abstractmethod
from pathlib import Path

from ninetoothed_amd import _lib
from ninetoothed_amd.backends.core import BuiltArtifact, Target, backend_id_for


class Materializer(ABC):
    target = None

    @abstractmethod
    def jit_materialize(self, compilation, *, output_dir=None):
        """Create a callable for interactive execution."""

    @abstractmethod
    def aot_build(self, compilation, *, output_dir):
        """Build (here: record) a reloadable artifact and return a callable."""

    @abstractmethod
    def load_built_artifact(self, built):
        """Load an existing artifact without recompiling it."""


class MaterializerRegistry:
    def __init__(self):
        self._materializers = {}

    def register(self, materializer, *, replace=False):
        backend_id = backend_id_for(materializer.target)
        if backend_id in self._materializers and not replace:
            raise ValueError(f"Materializer `{backend_id}` is already registered.")
        self._materializers[backend_id] = materializer

    def get(self, target):
        backend_id = backend_id_for(target)
        try:
            return self._materializers[backend_id]
        except KeyError as exc:
            available = ", ".join(sorted(self._materializers))
            raise ValueError(f"No materializer for `{backend_id}`. Available: {available}.") from exc


class HipMaterializer(Materializer):
    target = Target.HIP

    def jit_materialize(self, compilation, *, output_dir=None):
        from ninetoothed_amd.runtime import Handle

        if not _lib.LIBRARY_PATH.is_file():
            raise _lib.LibraryNotBuiltError(
                f"{_lib.LIBRARY_PATH} is not built; run `python __graft_entry__.py` first."
            )
        handle = Handle(compilation, library_path=_lib.LIBRARY_PATH)
        if output_dir is not None:
            compilation.artifact.write_to(output_dir)
        return handle

    def aot_build(self, compilation, *, output_dir):
        """Write a reloadable artifact under ``output_dir`` and return the Handle.

        The artifact is the kernel library (prebuilt, referenced by path) plus a program
        bundle: the arranged tensors, parameter specs and symbols, the application lowered
        for the constexpr values fixed at definition, and — when every shape and dtype is
        fixed too — the code objects of the generic kernels that call will run, so a reload
        compiles nothing.  ``<kernel>.manifest.json`` describes it for readers."""
        from ninetoothed_amd.generic import GenericPlan

        handle = self.jit_materialize(compilation, output_dir=output_dir)
        out = Path(output_dir)
        out.mkdir(parents=True, exist_ok=True)
        kernel = compilation.kernel
        kernel.prelower()
        code_objects, plans = {}, []
        name = compilation.artifact.kernel_name
        static = kernel.static_values()
        cpp = {"unavailable": "shapes, strides or dtypes are not all fixed at definition"}
        if static is not None:
            plan = kernel.specialize(static, {})
            plans.append(plan.describe())
            for source in getattr(plan, "sources_for", lambda values: [])(static):
                code_objects[GenericPlan.digest(source)] = GenericPlan.code_object(source)
            from ninetoothed_amd.backends import cpp_export

            try:
                code = cpp_export.source(name, plan, kernel, static, set(compilation.launch_abi["outputs"]))
                library = cpp_export.build(name, code, out)
                cpp = {"header": str(out / "ninetoothed.h"), "source": str(out / f"{name}.launch.cpp"),
                       "library": str(library), "symbol": f"launch_{name}"}
            except cpp_export.Unsupported as exc:
                cpp = {"unavailable": str(exc)}
        bundle_path = out / f"{name}.program.pkl"
        bundle = {"schema": 1, "abi_version": _lib.ABI_VERSION, "kernel": kernel.bundle(), "code_objects": code_objects}
        bundle_path.write_bytes(pickle.dumps(bundle))
        manifest = out / f"{name}.manifest.json"
        manifest.write_text(json.dumps({
            "schema": 2,
            "backend": compilation.target.backend.value,
            "kernel_name": name,
            "library": str(_lib.LIBRARY_PATH),
            "abi_version": _lib.ABI_VERSION,
            "program": str(bundle_path),
            "lowered_for": [dict(k) for k in kernel.bundle()["lowered"]],
            "plans": plans,
            "code_objects": sorted(code_objects),
            "cpp": cpp,
            "abi": {k: list(v) if isinstance(v, tuple) else v for k, v in compilation.launch_abi.items()},
            "artifact": dict(compilation.artifact.metadata),
        }, indent=1, default=str))
        cache_key = hashlib.sha256(bundle_path.read_bytes()).hexdigest()[:16]
        handle._built_artifact = BuiltArtifact(
            source=compilation.artifact, cache_key=cache_key, source_path=str(bundle_path),
            binary_path=str(_lib.LIBRARY_PATH), manifest_path=str(manifest), abi=dict(compilation.launch_abi),
        )
        return handle

    def load_built_artifact(self, built):
        """The Handle of a built artifact, from its program bundle alone (reference
        ``materializers/cuda.py:32-46``); the application is not needed."""
        from ninetoothed_amd.compiler import Compilation, KernelProgram
        from ninetoothed_amd.generic import GenericPlan
        from ninetoothed_amd.runtime import Handle
        from ninetoothed_amd.targets import resolve_target_context

        if built.binary_path is None or not Path(built.binary_path).is_file():
            raise _lib.LibraryNotBuiltError(f"the artifact's kernel library {built.binary_path} is missing")
        bundle = pickle.loads(Path(built.source_path).read_bytes())
        if bundle.get("abi_version") != _lib.ABI_VERSION:
            raise ValueError(f"the artifact was built against library ABI {bundle.get('abi_version')}, "
                             f"this library is {_lib.ABI_VERSION}")
        with GenericPlan._lock:
            for digest, blob in bundle["code_objects"].items():
                GenericPlan._blobs.setdefault(digest, blob)
        kernel = KernelProgram.from_bundle(bundle["kernel"])
        compilation = Compilation(request=None, kernel=kernel, artifact=built.source,
                                  target=resolve_target_context(built.source.backend, None, None),
                                  launch_abi=dict(built.abi))
        handle = Handle(compilation, library_path=built.binary_path)
        handle._built_artifact = built
        return handle


_REGISTRY = MaterializerRegistry()
_REGISTRY.register(HipMaterializer())


def materializer_for(target):
    return _REGISTRY.get(target)
