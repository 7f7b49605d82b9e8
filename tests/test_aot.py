"""AOT builds and their reload (reference tests/test_built_artifact_reload.py, test_aot.py).

CPU: an AOT build writes a program bundle and a manifest; ``load_built_artifact`` rebuilds
the Handle without the application (also in a fresh interpreter, from a pickled
BuiltArtifact) and specialises it to the same kernel family; a program whose shapes and
dtypes are fixed at definition carries the code objects of its generic kernels.  GPU: the
reloaded Handle computes what the original does.
"""

import json
import pickle
import subprocess
import sys
from pathlib import Path

import pytest
import torch

import ninetoothed_amd as ninetoothed
import ninetoothed_amd.language as ntl
from ninetoothed_amd import Tensor
from ninetoothed_amd.compiler import DEFAULT_COMPILER, CompileRequest, load_built_artifact

REPO = Path(__file__).resolve().parents[1]


def _compile(application, arrangement, tensors, name):
    return DEFAULT_COMPILER.compile(CompileRequest(application=application, arrangement=arrangement,
                                                   tensors=tensors, kernel_name=name))


def _add_kernel():
    # reference tests/test_built_artifact_reload.py:19-24 (a local application: it cannot be imported)
    def arrangement(input, other, output):
        return tuple(t.tile((64,)) for t in (input, other, output))

    def application(input, other, output):
        output = input + other  # noqa: F841

    tensors = tuple(Tensor(shape=(257,), dtype=ninetoothed.float32) for _ in range(3))
    return _compile(application, arrangement, tensors, "reload_hip")


def _pow_kernel():
    def arrangement(x, e, o):
        return tuple(t.tile((128,)) for t in (x, e, o))

    def application(x, e, o):
        o = ntl.libdevice.pow(x, e)  # noqa: F841

    tensors = tuple(Tensor(shape=(1000,), dtype=ninetoothed.float32) for _ in range(3))
    return _compile(application, arrangement, tensors, "pow_static")


def test_aot_build_writes_a_reloadable_artifact(tmp_path):
    handle = DEFAULT_COMPILER.materialize(_add_kernel(), output_dir=tmp_path, mode="aot")
    built = handle._built_artifact
    assert Path(built.source_path).is_file() and Path(built.manifest_path).is_file()
    assert built.binary_path is not None and Path(built.binary_path).is_file()
    manifest = json.loads(Path(built.manifest_path).read_text())
    assert manifest["kernel_name"] == "reload_hip" and manifest["plans"][0]["family"] == "add"
    reloaded = load_built_artifact(built)
    assert reloaded._kernel.application is None
    v = torch.empty(257)
    plan = reloaded._kernel.specialize({"input": v, "other": v, "output": v}, {})
    assert plan.describe()["family"] == "add"
    assert reloaded._abi["public_args"] == ("input", "other", "output")


def test_built_artifact_reloads_in_a_fresh_interpreter(tmp_path):
    handle = DEFAULT_COMPILER.materialize(_add_kernel(), output_dir=tmp_path, mode="aot")
    built_path = tmp_path / "built.pkl"
    built_path.write_bytes(pickle.dumps(handle._built_artifact))
    script = (
        "import pickle, sys, torch\n"
        "from ninetoothed_amd.compiler import load_built_artifact\n"
        "h = load_built_artifact(pickle.loads(open(sys.argv[1], 'rb').read()))\n"
        "v = torch.empty(257)\n"
        "print(h._kernel.specialize({'input': v, 'other': v, 'output': v}, {}).describe()['family'])\n"
    )
    r = subprocess.run([sys.executable, "-c", script, str(built_path)], cwd=REPO, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip().splitlines()[-1] == "add"


def test_static_generic_program_carries_its_code_objects(tmp_path):
    from ninetoothed_amd.generic import GenericPlan

    handle = DEFAULT_COMPILER.materialize(_pow_kernel(), output_dir=tmp_path, mode="aot")
    bundle = pickle.loads(Path(handle._built_artifact.source_path).read_bytes())
    assert len(bundle["code_objects"]) == 1
    digest, blob = next(iter(bundle["code_objects"].items()))
    assert len(blob) > 1000
    GenericPlan._blobs.pop(digest, None)
    reloaded = load_built_artifact(handle._built_artifact)
    assert GenericPlan._blobs[digest] == blob  # registered, so the reload compiles nothing
    v = torch.empty(1000)
    plan = reloaded._kernel.specialize({"x": v, "e": v, "o": v}, {})
    assert [GenericPlan.digest(s) for s in plan.sources_for({"x": v, "e": v, "o": v})] == [digest]


def test_constexpr_values_without_an_importable_application_are_refused(tmp_path):
    flag = Tensor(0, constexpr=True)

    def arrangement(x, f, o):
        return x.tile((32,)), f, o.tile((32,))

    def application(x, f, o):
        if f:
            o = x * 2.0 + 1.0  # noqa: F841
        else:
            o = x * 3.0  # noqa: F841

    c = _compile(application, arrangement, (Tensor(1), flag, Tensor(1)), "flagged")
    handle = DEFAULT_COMPILER.materialize(c, output_dir=tmp_path, mode="aot")
    reloaded = load_built_artifact(handle._built_artifact)
    v = torch.empty(64)
    with pytest.raises(ninetoothed.LoweringError, match="cannot be imported"):
        reloaded._kernel.specialize({"x": v, "f": True, "o": v}, {})
    # with the value fixed at definition, the bundle carries the lowered program
    fixed = _compile(application, arrangement, (Tensor(1), Tensor(0, constexpr=True, value=True), Tensor(1)), "fixed")
    handle = DEFAULT_COMPILER.materialize(fixed, output_dir=tmp_path / "fixed", mode="aot")
    plan = load_built_artifact(handle._built_artifact)._kernel.specialize({"x": v, "f": True, "o": v}, {})
    assert plan.describe()["family"] == "generic"


def test_importable_application_lowers_new_constexpr_values_after_reload(tmp_path):
    import programs as pg

    h = ninetoothed.make(pg.attention_arrangement, pg.attention_application, pg.attention_tensors(),
                         caller="hip", output_dir=tmp_path)
    reloaded = load_built_artifact(h._built_artifact)
    q = torch.empty((1, 2, 64, 64), dtype=torch.float16)
    for causal in (False, True):
        d = reloaded._kernel.specialize({"q": q, "k": q, "v": q, "is_causal": causal, "o": q}, {}).describe()
        assert d["family"] == "attention" and d["causal"] == causal


@pytest.mark.gpu
def test_reloaded_handles_compute_the_same(tmp_path):
    # reference tests/test_built_artifact_reload.py:28-66 (in this process; the subprocess reload is on the CPU)
    handle = DEFAULT_COMPILER.materialize(_add_kernel(), output_dir=tmp_path / "add", mode="aot")
    x, y = torch.randn(257, device="cuda"), torch.randn(257, device="cuda")
    out, out2 = torch.empty_like(x), torch.empty_like(x)
    handle(x, y, out)
    load_built_artifact(handle._built_artifact)(x, y, out2)
    assert torch.equal(out, x + y) and torch.equal(out2, out)

    handle = DEFAULT_COMPILER.materialize(_pow_kernel(), output_dir=tmp_path / "pow", mode="aot")
    x, e = torch.rand(1000, device="cuda"), torch.rand(1000, device="cuda")
    out, out2 = torch.empty_like(x), torch.empty_like(x)
    handle(x, e, out)
    load_built_artifact(handle._built_artifact)(x, e, out2)
    assert torch.allclose(out, torch.pow(x, e)) and torch.equal(out2, out)
