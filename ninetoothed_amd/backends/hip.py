"""The MI355X (gfx950) backend.

Stands where the reference's Triton backend stands (``src/ninetoothed/backends/triton.py``):
``emit`` turns a compiled program into an ``Artifact``.  Instead of source text the
artifact carries the program description (application parameters, launch-ABI
metadata, schedule granularity) and names the prebuilt library ``libnt_mi355x.so``
whose hand-written kernels implement the families; the family itself is selected
when the call-time specialisation is known (``ninetoothed_amd.families``).

The per-backend schedule pass the reference requires (``ssa.<backend>.optimize_schedule``,
``src/ninetoothed/backends/registry.py:35-55``) is ``schedule_pass`` below: it records the
granularity class of the program (blocked-linalg, exp-reduction-dot-region,
parallel-reduction, elementwise-grid) that the family kernels are organised by.
"""

from ninetoothed_amd import _lib
from ninetoothed_amd.backends.core import Artifact, Backend, Capability, Target, dump_json

PASS_NAME = "ssa.hip.optimize_schedule"


def schedule_pass(kernel):
    return {"granularity": kernel.granularity}


class HipBackend(Backend):
    name = Target.HIP
    capability = Capability(
        name=Target.HIP,
        emits_source=False,
        can_execute=True,
        requires_external_compiler=False,
        notes=(
            "hand-written gfx950 HIP kernels in libnt_mi355x.so, bound with ctypes",
            "families: gemm/addmm, conv2d (implicit GEMM), attention, softmax, max_pool2d, add",
        ),
    )
    supported_options = frozenset()
    passes = {PASS_NAME: schedule_pass}

    def emit(self, kernel):
        schedule = schedule_pass(kernel)
        metadata = {
            "target": self.name.value,
            "library": str(_lib.LIBRARY_PATH),
            "abi_version": _lib.ABI_VERSION,
            "variables": list(kernel.params),
            "outputs": list(kernel.outputs),
            "shape_params": sorted({n for s in kernel.param_specs for n in s.shape_symbols if n}),
            "meta_params": list(kernel.meta_args),
            "program_mode": "family-dispatch",
            "schedule": schedule,
            "pass_trace": [PASS_NAME],
            "tensors": [
                {"name": s.name, "ndim": s.source_ndim, "levels": list(s.level_ndims), "dtype": s.dtype,
                 "constexpr": s.constexpr}
                for s in kernel.param_specs
            ],
        }
        return Artifact(
            backend=self.name,
            kernel_name=kernel.name,
            language="hip-family-plan",
            sources={f"{kernel.name}.plan.json": dump_json(metadata)},
            entrypoint=None,
            metadata=metadata,
        )
