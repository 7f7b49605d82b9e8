"""Materializers: turn a Compilation into a callable Handle.

Contract as the reference's ``Materializer`` (``src/ninetoothed/backends/materializers/base.py:9-48``):
``jit_materialize``, ``aot_build`` and ``load_built_artifact``, registered per backend id.
The HIP materializer loads the prebuilt ``libnt_mi355x.so`` (it never compiles at run
time) and wraps the compilation in a ``Handle``.  ``aot_build`` writes the plan
manifest next to the caller's output directory and returns the same Handle.
"""

import json
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
        handle = self.jit_materialize(compilation, output_dir=output_dir)
        out = Path(output_dir)
        manifest = out / f"{compilation.artifact.kernel_name}.manifest.json"
        manifest.write_text(json.dumps({
            "schema": 1,
            "backend": compilation.target.backend.value,
            "library": str(_lib.LIBRARY_PATH),
            "abi": {k: list(v) if isinstance(v, tuple) else v for k, v in compilation.launch_abi.items()},
            "artifact": dict(compilation.artifact.metadata),
        }, indent=1, default=str))
        handle._built_artifact = BuiltArtifact(
            source=compilation.artifact, cache_key=compilation.artifact.kernel_name,
            source_path=str(out / compilation.artifact.primary_source_name), binary_path=str(_lib.LIBRARY_PATH),
            manifest_path=str(manifest), abi=dict(compilation.launch_abi),
        )
        return handle

    def load_built_artifact(self, built):
        raise NotImplementedError(
            "reloading a built artifact needs the application's Python source; call make() again "
            "(the kernel library itself is prebuilt and never recompiled)"
        )


_REGISTRY = MaterializerRegistry()
_REGISTRY.register(HipMaterializer())


def materializer_for(target):
    return _REGISTRY.get(target)
