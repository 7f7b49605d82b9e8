"""Writes tests/golden/reference_registry.json: this backend registered into the real reference.

Run once in this container, where the reference's source tree is present (the GPU box does
not have it, and no test imports it):

    python tests/golden/make_reference_registry.py

What it does, all in this one process:

1. Imports the reference from /root/reference/src and makes, in memory, the additions its
   maintainer would make for a new backend (``ninetoothed_amd.backends.reference`` names
   them): a ``Target.HIP`` member with its ``"hip"`` alias, an ``amd-mi355x`` platform profile
   whose backend modes name ``hip``, and the ``"hip"`` entry of the lazy materialisation's
   source-suffix table.  There is no GPU here, so the reference's device check for
   non-Triton backends (``runtime_device_types``, targets.py:756-766, which admits ``cuda``
   only) is widened in this process to the profile's device types, which also name
   ``cpu``: the reference's own argument checks then pass CPU tensors on to the
   materialized Handle.
2. Calls ``ninetoothed_amd.backends.reference.register(ninetoothed)``.
3. Runs the reference's own test wrappers (tests/test_matmul.py ``matmul``, test_addmm.py
   ``addmm``, test_conv2d.py ``conv2d``, test_attention.py ``attention``, test_softmax.py
   ``softmax``, test_max_pool2d.py ``max_pool2d``, test_add.py ``add``) with
   ``NINETOOTHED_BACKEND=hip`` on small CPU tensors.  Each goes through the reference's
   ``make``/``jit``, its pass pipeline (with the ``ssa.hip.optimize_schedule`` pass), this
   backend's ``emit``, the reference driver's launch ABI, the reference's lazy
   specialisation and this backend's materializer, and ends in this package's Handle, which
   refuses CPU tensors (the kernels run on the GPU): that ``TypeError`` is the expected end.
4. Records per program what the reference computed (schedule granularity, pass trace, the
   artifact metadata its driver read, the launch ABI it derived) and what this package made
   of the converted request (its ABI, granularity, the family chosen for the call, and the
   converted symbols with their roles and bounds).

``tests/test_reference_adapter.py`` compares this package's native programs against it.
"""

import dataclasses
import inspect
import json
import os
import sys
import textwrap
import traceback
from pathlib import Path

REFERENCE = Path("/root/reference")
sys.path.insert(0, str(REFERENCE / "src"))
sys.path.insert(0, str(REFERENCE))
sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

import torch  # noqa: E402

import ninetoothed  # noqa: E402  (the reference)
from ninetoothed.backends import core as ref_core  # noqa: E402


def _add_hip_target():
    """``Target.HIP = "hip"`` and its alias (reference backends/core.py:11-22)."""
    target = ref_core.Target
    if "HIP" not in target.__members__:
        member = str.__new__(target, "hip")
        member._name_, member._value_ = "HIP", "hip"
        member.__objclass__ = target
        target._member_map_["HIP"] = member
        target._value2member_map_["hip"] = member
        target._member_names_.append("HIP")  # Target.HIP and iteration read these tables
    ref_core._CANONICAL_BACKEND_NAMES["hip"] = target.HIP
    return target.HIP


HIP = _add_hip_target()

from ninetoothed import targets as ref_targets  # noqa: E402
from ninetoothed.compiler import runtime as ref_runtime  # noqa: E402

PROFILE = ref_targets.PlatformProfile(
    name="amd-mi355x", aliases=("mi355x",), accelerator_vendor="amd", accelerator_name="mi355x",
    compute_arch="gfx950", device_types=("cuda", "cpu"), backend_modes={"hip": frozenset({"jit", "aot"})},
    metadata={"wavefront_size": 64})
ref_targets.default_platform_registry().register(PROFILE, replace=True)

# the lazy materialisation's source-suffix table gains Target.HIP (compiler/runtime.py:183-186)
_source = inspect.getsource(ref_runtime._materialize_lazy)
assert 'Target.CUDA: "cu",' in _source
_source = _source.replace('Target.CUDA: "cu",', 'Target.CUDA: "cu",\n        Target.HIP: "hip",')
exec(compile(textwrap.dedent(_source), ref_runtime.__file__, "exec"), ref_runtime.__dict__)

_device_types = ref_runtime.runtime_device_types


def _runtime_device_types(value):
    context = getattr(value, "target", None)
    if getattr(context, "backend", None) == HIP:
        return context.device_types
    return _device_types(value)


ref_runtime.runtime_device_types = _runtime_device_types

os.environ["NINETOOTHED_BACKEND"] = "hip"
os.environ["NINETOOTHED_PLATFORM"] = "amd-mi355x"

from ninetoothed_amd.backends import reference as adapter  # noqa: E402

BACKEND, MATERIALIZER = adapter.register(ninetoothed)

from tests import (  # noqa: E402
    test_add,
    test_addmm,
    test_attention,
    test_conv2d,
    test_matmul,
    test_max_pool2d,
    test_softmax,
)


def _g(seed):
    return torch.Generator("cpu").manual_seed(seed)


def _t(shape, dtype=torch.float16, seed=0):
    return torch.randn(shape, generator=_g(seed)).to(dtype)


PROGRAMS = {
    "matmul": (lambda: test_matmul.matmul(_t((96, 80)), _t((80, 72), seed=1))),
    "addmm": (lambda: test_addmm.addmm(_t((64, 48)), _t((64, 32), seed=1), _t((32, 48), seed=2), 0.5, 1.0)),
    "conv2d": (lambda: test_conv2d.conv2d(_t((4, 64, 16, 16)), _t((512, 64, 3, 3), seed=1), padding=(1, 1))),
    "attention": (lambda: test_attention.attention(_t((2, 4, 100, 64)), _t((2, 4, 100, 64), seed=1),
                                                   _t((2, 4, 100, 64), seed=2), True)),
    "softmax": (lambda: test_softmax.softmax(torch.rand((10, 781), generator=_g(3)))),
    "max_pool2d": (lambda: test_max_pool2d.max_pool2d(_t((2, 3, 10, 11)), (3, 3), ceil_mode=True)),
    "add": (lambda: test_add.add(_t((1000,), torch.float32), _t((1000,), torch.float32, seed=1))),
}


def _frames(tb):
    while tb is not None:
        yield tb.tb_frame
        tb = tb.tb_next


def _symbol_entry(sym):
    return [sym.constexpr, sym.meta, sym.lower_bound, sym.upper_bound, sym.power_of_two]


def _describe(value):
    if hasattr(value, "shape"):
        return {"shape": list(value.shape), "dtype": str(value.dtype).replace("torch.", ""),
                "stride": list(value.stride())}
    return value


def record(name, run):
    try:
        run()
    except TypeError as exc:
        tb, message = exc.__traceback__, str(exc)
    else:
        raise AssertionError(f"{name}: the call ran; it should stop at this package's Handle (CPU tensors)")
    ours_frame = next(f for f in _frames(tb) if f.f_code.co_filename.endswith("ninetoothed_amd/runtime.py")
                      and f.f_code.co_name == "__call__")
    ours, args, kwargs = ours_frame.f_locals["self"], ours_frame.f_locals["args"], ours_frame.f_locals["kwargs"]
    lazy = next(f for f in _frames(tb) if f.f_code.co_name == "launch" and "specializations" in f.f_locals)
    reference_handle = lazy.f_locals["handle"]
    specialized = next(iter(lazy.f_locals["specializations"].values()))
    names = ours._abi["public_args"]
    public, meta = dict(zip(names, args)), {}
    for k, v in kwargs.items():
        (public if k in names else meta)[k] = v
    plan = ours._kernel.specialize(public, meta)
    metadata = reference_handle._compilation.artifact.metadata
    abi = reference_handle._compilation.launch_abi
    symbols = {}
    for spec in ours._kernel.param_specs:
        arranged = ours._kernel.arranged[spec.name]
        symbols[spec.name] = {n: _symbol_entry(s) for n, s in sorted(arranged.symbols().items())}
    return {
        "stopped_at": message,
        "reference": {
            "granularity": metadata["ssa_schedule"].get("granularity"),
            "pass_trace": list(metadata["ssa_pass_trace"]),
            "optimization": {k: v for k, v in metadata["ssa_optimization"].items() if k == "preserve_linalg"},
            "variables": list(metadata["variables"]),
            "outputs": list(metadata["outputs"]),
            "shape_params": list(metadata["shape_params"]),
            "program_mode": dict(metadata["program_mode"]),
            "launch_abi": {"public_args": list(abi.public_args), "outputs": list(abi.outputs),
                           "kernel_args": [[b.name, b.kind, b.source] for b in abi.kernel_args]},
            "specialized_backend": specialized._compilation.artifact.backend.value,
            "specialized_materialized_by": type(specialized).__module__ + "." + type(specialized).__name__,
        },
        "ours": {
            "public_args": list(names), "outputs": list(ours._abi["outputs"]),
            "granularity": ours._kernel.granularity, "family": plan.describe()["family"],
            "symbols": symbols,
        },
        "call": {"args": [_describe(a) for a in args], "kwargs": {k: _describe(v) for k, v in kwargs.items()}},
    }


def main():
    from ninetoothed.compiler import passes

    registry = passes.create_default_registry()  # validates every Target's pass contract
    descriptor = registry.get(adapter.PASS_NAME)
    out = {
        "reference_version": ninetoothed.__version__ if hasattr(ninetoothed, "__version__") else "0.26.0",
        "pass": {"name": descriptor.name, "supports_hip": descriptor.supports("hip"),
                 "supported_backends": [b.value for b in descriptor.supported_backends]},
        "backend_capability_notes": list(BACKEND.capability.notes),
        "programs": {},
    }
    for name, run in PROGRAMS.items():
        try:
            out["programs"][name] = record(name, run)
        except Exception:
            traceback.print_exc()
            raise
        p = out["programs"][name]
        print(f"{name}: reference {p['reference']['granularity']}, ours {p['ours']['granularity']}, "
              f"family {p['ours']['family']}", flush=True)
    path = Path(__file__).with_name("reference_registry.json")
    path.write_text(json.dumps(out, indent=1, sort_keys=True, default=str) + "\n")
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
