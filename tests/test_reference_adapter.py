"""This backend behind the reference's own plugin points (``ninetoothed_amd.backends.reference``).

``tests/golden/make_reference_registry.py`` registered the adapter into the real reference in
this container (with the maintainer's additions made in that process) and ran the reference's
own test wrappers for matmul, addmm, conv2d, attention, softmax, max_pool2d and add through
its ``make``/``jit``, its pass pipeline, this backend's ``emit``, its driver's launch ABI, its
lazy specialisation and this backend's materializer, down to this package's Handle.
``tests/golden/reference_registry.json`` holds what it recorded.  The reference cannot be
imported by a test, so the CPU tests here compare this package's native programs
(``tests/programs.py``) with that record: the reference's schedule granularity, the launch
ABI its driver derived from this backend's artifact, the family the converted program was
bound to for the same call, and the converted symbols' roles and bounds.  The GPU test runs
the part of the chain that needs no reference: the materializer's hand-back of the values
the reference specialised on (conv2d's ``padding_h``/``padding_w``).
"""

import functools
import json
import re
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

import ninetoothed_amd as ninetoothed
import programs as pg
from ninetoothed_amd.backends import reference as adapter

FIXTURE = json.loads((Path(__file__).parent / "golden" / "reference_registry.json").read_text())
# names a per-process counter numbers: tensor sizes, block_size() symbols
AUTO = re.compile(r"^(tensor_\d+_size_\d+|ninetoothed_BLOCK_SIZE_\d+)$")

NATIVE = {
    "matmul": lambda: ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors()),
    "addmm": lambda: ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors()),
    "conv2d": lambda: pg.make_conv2d(),
    "attention": lambda: ninetoothed.make(pg.attention_arrangement, pg.attention_application,
                                          pg.attention_tensors()),
    "softmax": lambda: pg.make_softmax(),
    "max_pool2d": lambda: ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=True),
                                           pg.max_pool2d_application, pg.max_pool2d_tensors()),
    "add": lambda: pg.make_add(),
}


def _value(d):
    if isinstance(d, dict) and "shape" in d:
        return torch.empty_strided(d["shape"], d["stride"], dtype=getattr(torch, d["dtype"]))
    return d


def _call(handle, record):
    names = handle._abi["public_args"]
    args = [_value(a) for a in record["call"]["args"]]
    public, meta = dict(zip(names, args)), {}
    for k, v in record["call"]["kwargs"].items():
        (public if k in names else meta)[k] = _value(v)
    return public, meta


def _symbols(handle):
    out = {}
    for spec in handle._kernel.param_specs:
        syms = handle._kernel.arranged[spec.name].symbols()
        out[spec.name] = {n: [s.constexpr, s.meta, s.lower_bound, s.upper_bound, s.power_of_two]
                          for n, s in syms.items()}
    return out


def _split(entries):
    named = {n: e for n, e in entries.items() if not AUTO.match(n)}
    auto = sorted(json.dumps(e) for n, e in entries.items() if AUTO.match(n))
    return named, auto


def test_fixture_covers_the_six_families():
    assert set(FIXTURE["programs"]) == set(NATIVE)
    assert FIXTURE["pass"] == {"name": adapter.PASS_NAME, "supported_backends": ["hip"], "supports_hip": True}


@pytest.mark.parametrize("name", sorted(NATIVE))
def test_reference_pipeline_runs_the_hip_schedule_pass(name):
    ref = FIXTURE["programs"][name]["reference"]
    assert ref["pass_trace"] == ["ssa.canonicalize", "ssa.analyze_effects", "ssa.select_schedule", adapter.PASS_NAME,
                                 "ssa.decompose_linalg", "ssa.validate_target_capabilities"]
    # the reference's lazy specialisation reached this backend's materializer and this package's Handle
    assert ref["specialized_backend"] == "hip"
    assert FIXTURE["programs"][name]["stopped_at"].endswith("must be on a CUDA device.")


@pytest.mark.parametrize("name", sorted(NATIVE))
def test_granularity_is_the_references(name):
    # reference compiler/passes.py:1070-1084, as computed by the reference's own SelectSchedule
    record = FIXTURE["programs"][name]
    assert NATIVE[name]()._kernel.granularity == record["reference"]["granularity"]
    assert record["ours"]["granularity"] == record["reference"]["granularity"]


@pytest.mark.parametrize("name", sorted(NATIVE))
def test_launch_abi_matches_what_the_reference_derived(name):
    record = FIXTURE["programs"][name]
    ref = record["reference"]
    h = NATIVE[name]()
    assert list(h._abi["public_args"]) == ref["launch_abi"]["public_args"] == record["ours"]["public_args"]
    assert list(h._abi["outputs"]) == ref["launch_abi"]["outputs"] == ref["outputs"] == record["ours"]["outputs"]
    # the artifact's variables: the public non-constexpr parameters that are not outputs
    assert ref["variables"] == [n for n in ref["launch_abi"]["public_args"]
                                if n not in ref["outputs"] and n in [b[0] for b in ref["launch_abi"]["kernel_args"]
                                                                     if b[1] == "tensor" or b[1] == "scalar"]]
    # every shape parameter became a binding of the reference's launch ABI
    bound = {b[0] for b in ref["launch_abi"]["kernel_args"]}
    assert set(ref["shape_params"]) <= bound


@pytest.mark.parametrize("name", sorted(NATIVE))
def test_converted_program_binds_the_same_family(name):
    record = FIXTURE["programs"][name]
    h = NATIVE[name]()
    public, meta = _call(h, record)
    assert h._kernel.specialize(public, meta).describe()["family"] == record["ours"]["family"] == name.replace(
        "matmul", "gemm").replace("addmm", "gemm")


@pytest.mark.parametrize("name", sorted(NATIVE))
def test_converted_symbols_keep_roles_and_bounds(name):
    record = FIXTURE["programs"][name]
    native = _symbols(NATIVE[name]())
    assert set(native) == set(record["ours"]["symbols"])
    for param, entries in record["ours"]["symbols"].items():
        assert _split(native[param]) == _split(entries), param


def test_specialisation_values_are_handed_back():
    # the reference drops a constexpr it specialised on from the call's keywords
    # (compiler/runtime.py:1188-1195); the materializer passes it on to this package's Handle
    h = pg.make_conv2d()
    request = SimpleNamespace(specialization_values={
        "ninetoothed_constexpr_prefix_padding_h": 1, "ninetoothed_constexpr_prefix_padding_w": 2,
        "ninetoothed_ninetoothed_tensor_93_size_0": 4, "ninetoothed_meta_prefix_BLOCK_SIZE_M": 64})
    wrapped = adapter._Specialized(h, request)
    assert wrapped.fixed == {"padding_h": 1, "padding_w": 2, "BLOCK_SIZE_M": 64}


@pytest.mark.gpu
def test_specialised_conv2d_runs_without_its_padding_keywords():
    h = pg.make_conv2d()
    request = SimpleNamespace(specialization_values={"ninetoothed_constexpr_prefix_padding_h": 1,
                                                     "ninetoothed_constexpr_prefix_padding_w": 1})
    wrapped = adapter._Specialized(h, request)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 64, 12, 12, generator=g).half().cuda()
    w = (torch.randn(96, 64, 3, 3, generator=g) / 24).half().cuda()
    y = torch.empty(2, 96, 12, 12, dtype=torch.float16, device="cuda")
    wrapped(x, w, y)  # as the reference's lazy launch calls it: no padding keywords
    assert torch.allclose(y.float(), F.conv2d(x.float(), w.float(), padding=1), atol=1e-2, rtol=1e-2)
