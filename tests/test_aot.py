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


# ------------------------------------------------------------------ standalone C++ launchers
import ctypes  # noqa: E402


class NineToothedTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("shape", ctypes.POINTER(ctypes.c_uint64)),
                ("strides", ctypes.POINTER(ctypes.c_int64))]


def _nt_tensor(t, keep):
    if t.dim() == 0 or not hasattr(t, "data_ptr"):
        raise TypeError
    shape = (ctypes.c_uint64 * t.dim())(*t.shape)
    strides = (ctypes.c_int64 * t.dim())(*t.stride())
    keep += [shape, strides]
    return NineToothedTensor(ctypes.c_void_p(t.data_ptr()), shape, strides)


def _nt_scalar(value, keep):
    v = ctypes.c_double(value)
    keep.append(v)
    return NineToothedTensor(ctypes.cast(ctypes.pointer(v), ctypes.c_void_p), None, None)


def _static_matmul(tmp_path, name="mm_static"):
    import programs as pg

    f16 = ninetoothed.float16
    tensors = (Tensor(shape=(256, 512), dtype=f16), Tensor(shape=(512, 128), dtype=f16),
               Tensor(shape=(256, 128), dtype=f16))
    c = DEFAULT_COMPILER.compile(CompileRequest(application=pg.matmul_application, arrangement=pg.matmul_arrangement,
                                                tensors=tensors, kernel_name=name))
    return DEFAULT_COMPILER.materialize(c, output_dir=tmp_path, mode="aot")


def test_cpp_launcher_is_built_and_checks_its_arguments(tmp_path):
    h = _static_matmul(tmp_path)
    manifest = json.loads(Path(h._built_artifact.manifest_path).read_text())
    cpp = manifest["cpp"]
    assert cpp["symbol"] == "launch_mm_static" and Path(cpp["library"]).is_file()
    assert "NineToothedTensor" in Path(cpp["header"]).read_text()
    lib = ctypes.CDLL(cpp["library"])
    fn = lib.launch_mm_static
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 3
    keep = []
    a, b, out = torch.empty(256, 512, dtype=torch.float16), torch.empty(512, 128, dtype=torch.float16), \
        torch.empty(256, 128, dtype=torch.float16)
    bad = torch.empty(256, 64, dtype=torch.float16)  # wrong shape: rejected before anything is launched
    assert fn(None, _nt_tensor(a, keep), _nt_tensor(b, keep), _nt_tensor(bad, keep)) == 1
    nulls = NineToothedTensor(None, _nt_tensor(out, keep).shape, _nt_tensor(out, keep).strides)
    assert fn(None, _nt_tensor(a, keep), _nt_tensor(b, keep), nulls) == 1


def test_cpp_launcher_reasons_are_recorded(tmp_path):
    # symbolic shapes: no launcher, with the reason in the manifest
    h = ninetoothed.make(lambda x, y, o: (x.tile((64,)), y.tile((64,)), o.tile((64,))), _add_app(), (
        Tensor(1), Tensor(1), Tensor(1)), caller="hip", output_dir=tmp_path / "sym")
    assert "not all fixed" in json.loads(Path(h._built_artifact.manifest_path).read_text())["cpp"]["unavailable"]


def test_generic_kernel_launcher_is_built_and_checks_its_arguments(tmp_path):
    # a generic kernel's launcher embeds its code object (and index tables, if any)
    h = DEFAULT_COMPILER.materialize(_pow_kernel(), output_dir=tmp_path / "pow", mode="aot")
    cpp = json.loads(Path(h._built_artifact.manifest_path).read_text())["cpp"]
    assert cpp["symbol"] == "launch_pow_static" and Path(cpp["library"]).is_file()
    assert "kCode[" in Path(cpp["source"]).read_text()
    fn = getattr(ctypes.CDLL(cpp["library"]), cpp["symbol"])
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 3
    keep = []
    x, bad = torch.empty(1000), torch.empty(999)
    assert fn(None, _nt_tensor(x, keep), _nt_tensor(x, keep), _nt_tensor(bad, keep)) == 1  # rejected unlaunched


def _add_app():
    def application(input, other, output):
        output = input + other  # noqa: F841

    return application


@pytest.mark.gpu
def test_cpp_launchers_compute(tmp_path):
    import programs as pg

    h = _static_matmul(tmp_path / "mm")
    cpp = json.loads(Path(h._built_artifact.manifest_path).read_text())["cpp"]
    fn = getattr(ctypes.CDLL(cpp["library"]), cpp["symbol"])
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 3
    a = torch.randn(256, 512, device="cuda", dtype=torch.float16)
    b = torch.randn(512, 128, device="cuda", dtype=torch.float16)
    out = torch.empty(256, 128, device="cuda", dtype=torch.float16)
    keep = []
    stream = torch.cuda.current_stream().cuda_stream
    assert fn(stream, _nt_tensor(a, keep), _nt_tensor(b, keep), _nt_tensor(out, keep)) == 0
    torch.cuda.synchronize()
    assert torch.allclose(out.float(), (a.float() @ b.float()).half().float(), atol=5e-2, rtol=1e-2)

    # addmm: 0-d alpha/beta are host doubles
    f16, f64 = ninetoothed.float16, ninetoothed.float64
    tensors = (Tensor(shape=(256, 128), dtype=f16), Tensor(shape=(256, 512), dtype=f16),
               Tensor(shape=(512, 128), dtype=f16), Tensor(0, dtype=f64), Tensor(0, dtype=f64),
               Tensor(shape=(256, 128), dtype=f16))
    c = DEFAULT_COMPILER.compile(CompileRequest(application=pg.addmm_application, arrangement=pg.addmm_arrangement,
                                                tensors=tensors, kernel_name="addmm_static"))
    h = DEFAULT_COMPILER.materialize(c, output_dir=tmp_path / "addmm", mode="aot")
    cpp = json.loads(Path(h._built_artifact.manifest_path).read_text())["cpp"]
    fn = getattr(ctypes.CDLL(cpp["library"]), cpp["symbol"])
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 6
    inp = torch.randn(256, 128, device="cuda", dtype=torch.float16)
    assert fn(stream, _nt_tensor(inp, keep), _nt_tensor(a, keep), _nt_tensor(b, keep), _nt_scalar(0.5, keep),
              _nt_scalar(2.0, keep), _nt_tensor(out, keep)) == 0
    torch.cuda.synchronize()
    ref = 0.5 * inp.float() + 2.0 * (a.float() @ b.float()).half().float()
    assert torch.allclose(out.float(), ref, atol=1e-1, rtol=1e-2)


@pytest.mark.gpu
def test_generic_kernel_launchers_compute(tmp_path):
    # an element-parallel program (libdevice.pow) and a tile program with index tables
    # (dot + a reduction), each through its standalone launcher
    h = DEFAULT_COMPILER.materialize(_pow_kernel(), output_dir=tmp_path / "pow", mode="aot")
    cpp = json.loads(Path(h._built_artifact.manifest_path).read_text())["cpp"]
    fn = getattr(ctypes.CDLL(cpp["library"]), cpp["symbol"])
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 3
    x, e = torch.rand(1000, device="cuda"), torch.rand(1000, device="cuda")
    out = torch.empty_like(x)
    keep = []
    stream = torch.cuda.current_stream().cuda_stream
    assert fn(stream, _nt_tensor(x, keep), _nt_tensor(e, keep), _nt_tensor(out, keep)) == 0
    torch.cuda.synchronize()
    assert torch.allclose(out, torch.pow(x, e))

    def arrangement(x, w, o):
        xt = x.tile((16, -1))
        return xt, w.tile((-1, -1)).expand((xt.shape[0], -1)), o.tile((16,))

    def application(x, w, o):
        o = ntl.sum(ntl.dot(x, w), axis=1)  # noqa: F841

    f16, f32 = ninetoothed.float16, ninetoothed.float32
    tensors = (Tensor(shape=(64, 40), dtype=f16), Tensor(shape=(40, 24), dtype=f16), Tensor(shape=(64,), dtype=f32))
    h = DEFAULT_COMPILER.materialize(_compile(application, arrangement, tensors, "dot_rows_static"),
                                     output_dir=tmp_path / "dot", mode="aot")
    cpp = json.loads(Path(h._built_artifact.manifest_path).read_text())["cpp"]
    assert "kTable0" in Path(cpp["source"]).read_text()
    fn = getattr(ctypes.CDLL(cpp["library"]), cpp["symbol"])
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 3
    a = (torch.randn(64, 40, device="cuda") / 4).half()
    w = (torch.randn(40, 24, device="cuda") / 4).half()
    rows = torch.empty(64, device="cuda")
    for _ in range(2):  # the second call reuses the loaded kernel and the device tables
        rows.fill_(float("nan"))
        assert fn(stream, _nt_tensor(a, keep), _nt_tensor(w, keep), _nt_tensor(rows, keep)) == 0
        torch.cuda.synchronize()
        assert torch.allclose(rows, (a.float() @ w.float()).sum(dim=1), atol=1e-3, rtol=1e-3)
