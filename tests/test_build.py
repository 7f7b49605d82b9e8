"""``ninetoothed_amd.build``: configured variants behind one dispatcher (reference tests/test_aot.py:219-310).

The reference's conv2d build leg: ``premake`` (reference tests/test_conv2d.py:50-85) builds
one variant per block-size configuration; the dispatcher is called with the kernel's
tensors followed by every premake parameter's value (sizes, dtype, block sizes) and runs
the variant built for exactly those values.  CPU: dispatch, errors, the C++ dispatcher's
source and its rejection of an unbuilt configuration, lazy builds.  GPU: the variants
compute F.conv2d within the reference's 1e-3, through Python and through the C++
dispatcher.
"""

import ctypes
import functools
import json
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

import ninetoothed_amd as ninetoothed
import programs as pg
from ninetoothed_amd import Tensor
from test_aot import NineToothedTensor, _nt_tensor

SIZES = {"n": 4, "c": 64, "h": 16, "w": 16, "k": 512, "r": 3, "s": 3}
CONFIGS = (((), {"block_size_m": 64, "block_size_n": 64, "block_size_k": 64}, {}),
           ((), {"block_size_m": 128, "block_size_n": 32, "block_size_k": 64}, {}))


def premake(n=None, c=None, h=None, w=None, k=None, r=None, s=None, dtype=None, block_size_m=64, block_size_n=64,
            block_size_k=64):
    arrangement = functools.partial(pg.conv2d_arrangement, BLOCK_SIZE_M=block_size_m, BLOCK_SIZE_N=block_size_n,
                                    BLOCK_SIZE_K=block_size_k)
    p = h - r + 1 if h is not None and r is not None else None
    q = w - s + 1 if w is not None and s is not None else None
    tensors = (Tensor(shape=(n, c, h, w), dtype=dtype), Tensor(shape=(k, c, r, s), dtype=dtype),
               Tensor(shape=(n, k, p, q), dtype=dtype))
    return arrangement, pg.matmul_application, tensors


def _build(tmp_path, constexpr_shapes, name, **options):
    sizes = SIZES if constexpr_shapes else dict.fromkeys(SIZES)
    kernel = ninetoothed.build(functools.partial(premake, **sizes, dtype=ninetoothed.float16), CONFIGS, caller="hip",
                               kernel_name=name, output_dir=tmp_path, **options)
    config = (*sizes.values(), ninetoothed.float16)
    return kernel, config


def test_build_dispatches_by_configuration(tmp_path):
    kernel, config = _build(tmp_path, False, "conv2d_dyn")
    assert len(kernel.handles) == 2 and len(kernel.configurations) == 2
    # every premake parameter is part of the configuration: sizes, dtype, then the block sizes
    assert kernel.configurations[0] == (None,) * 7 + ("fp16", 64, 64, 64)
    assert kernel.configurations[1][-3:] == (128, 32, 64)
    x = torch.empty(4, 64, 16, 16, dtype=torch.float16)
    with pytest.raises(ValueError, match="No compiled kernel configuration matches"):
        kernel(x, x, x, *config, 32, 32, 32)
    with pytest.raises(TypeError, match="configuration values"):
        kernel(x)
    # symbolic shapes: the variants have no standalone launcher, so neither has the dispatcher
    assert "unavailable" in kernel.cpp
    for h in kernel.handles:
        assert Path(h._built_artifact.manifest_path).is_file()


def test_meta_parameters_share_a_configuration(tmp_path):
    kernel, _ = _build(tmp_path, False, "conv2d_meta", meta_parameters=("block_size_m", "block_size_n", "block_size_k"))
    assert kernel.configurations == ((None,) * 7 + ("fp16",),)
    (group,) = kernel._groups.values()
    assert group.tuner is not None and len(group.handles) == 2


def test_lazy_build_compiles_on_first_call(tmp_path):
    kernel = ninetoothed.build(premake, CONFIGS, caller="hip", kernel_name="conv2d_lazy", output_dir=tmp_path,
                               lazy=True)
    assert not list(tmp_path.iterdir())  # nothing built yet
    with pytest.raises(ValueError, match="No compiled kernel configuration"):
        kernel(torch.empty(1), torch.empty(1), torch.empty(1), *([None] * 7), None, 1, 2, 3)
    assert list(tmp_path.glob("*.manifest.json"))


def test_cpp_dispatcher_is_written_and_checks_the_configuration(tmp_path):
    kernel, _ = _build(tmp_path, True, "conv2d_static")
    cpp = kernel.cpp
    assert cpp["symbol"] == "launch_conv2d_static", cpp
    header = Path(cpp["header"]).read_text()
    assert "NineToothedStream stream, NineToothedTensor tensor_0, NineToothedTensor tensor_1, " \
           "NineToothedTensor tensor_2, int config_0" in header and "int config_10" in header
    source = Path(cpp["source"]).read_text()
    # dtype configuration values are NineToothedDataType enumerators (float16 = 8)
    assert "config_7 == 8 && config_8 == 64 && config_9 == 64 && config_10 == 64" in source
    assert "launch_conv2d_static_0(" in source and "launch_conv2d_static_1(" in source
    fn = ctypes.CDLL(cpp["library"]).launch_conv2d_static
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 3 + [ctypes.c_int] * 11
    keep = []
    t = [_nt_tensor(torch.empty(2), keep) for _ in range(3)]
    assert fn(None, *t, *SIZES.values(), 8, 32, 32, 32) == 1  # no variant: NT_ERR_INVALID, nothing launched
    manifests = [json.loads(Path(h._built_artifact.manifest_path).read_text()) for h in kernel.handles]
    assert all(m["cpp"]["symbol"].startswith("launch_conv2d_static_") for m in manifests)


@pytest.mark.gpu
@pytest.mark.parametrize("constexpr_shapes", (False, True))
def test_build_conv2d_reference_case(tmp_path, constexpr_shapes):
    kernel, config = _build(tmp_path, constexpr_shapes, f"conv2d_build_{int(constexpr_shapes)}")
    g = torch.Generator().manual_seed(90)
    x = torch.randn(4, 64, 16, 16, generator=g).half().cuda()
    w = torch.randn(512, 64, 3, 3, generator=g).half().cuda()
    expected = F.conv2d(x.float(), w.float()).half()
    for _, kw, _ in CONFIGS:
        y = torch.empty(4, 512, 14, 14, dtype=torch.float16, device="cuda")
        kernel(x, w, y, *config, *kw.values())
        assert torch.allclose(y, expected, rtol=1e-3, atol=1e-3)
    if constexpr_shapes:
        fn = ctypes.CDLL(kernel.cpp["library"]).launch_conv2d_build_1
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p] + [NineToothedTensor] * 3 + [ctypes.c_int] * 11
        y = torch.empty(4, 512, 14, 14, dtype=torch.float16, device="cuda")
        keep = []
        stream = torch.cuda.current_stream().cuda_stream
        assert fn(stream, _nt_tensor(x, keep), _nt_tensor(w, keep), _nt_tensor(y, keep), *SIZES.values(), 8, 128, 32,
                  64) == 0
        torch.cuda.synchronize()
        assert torch.allclose(y, expected, rtol=1e-3, atol=1e-3)


@pytest.mark.gpu
def test_build_tunes_variants_of_one_configuration(tmp_path, monkeypatch):
    monkeypatch.setenv("NINETOOTHED_AMD_CACHE_DIR", str(tmp_path / "cache"))
    kernel, config = _build(tmp_path, False, "conv2d_tuned", meta_parameters=("block_size_m", "block_size_n",
                                                                               "block_size_k"))
    g = torch.Generator().manual_seed(91)
    x = torch.randn(4, 64, 16, 16, generator=g).half().cuda()
    w = torch.randn(512, 64, 3, 3, generator=g).half().cuda()
    y = torch.empty(4, 512, 14, 14, dtype=torch.float16, device="cuda")
    kernel(x, w, y, *config)
    assert torch.allclose(y, F.conv2d(x.float(), w.float()).half(), rtol=1e-3, atol=1e-3)
    (group,) = kernel._groups.values()
    assert len(group.tuner.timings(x, w, y)) == 2
