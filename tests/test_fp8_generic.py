"""fp8 tensors (torch float8_e4m3fn and float8_e5m2) in the generic kernels.

CPU: the kernels' own fp8 encode/decode functions (the emitted source's prelude, built for
the host with clang) against torch's conversions, bit for bit, on every code and on the
values where rounding decides (ties, binade edges, the overflow thresholds, subnormals,
NaN, infinities, signed zero) plus a random sample across the range; the reference's
typing (fp8 ranks below fp16, e4m3fn's reduction identity ±448); programs with fp8 operands
compile, their dots on the matrix core.  GPU: stores into fp8 outputs, loads of fp8 inputs,
fp8 arithmetic and a matrix-core dot of fp8 tiles against torch.
"""

import ctypes
import subprocess

import numpy as np
import pytest
import torch

import ninetoothed_amd as ninetoothed
import ninetoothed_amd.language as ntl
from ninetoothed_amd import Symbol, Tensor
from ninetoothed_amd import generic
from ninetoothed_amd.generic import GenericPlan

FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)
CLANG = "/opt/rocm/llvm/bin/clang++"


# ------------------------------------------------------------------ the conversions, on the host
@pytest.fixture(scope="module")
def host_fp8(tmp_path_factory):
    body = generic._PRELUDE
    start = body.index("__device__ __forceinline__ unsigned char st_e4m3")
    end = body.index("__device__ __forceinline__ float r_e4m3")
    src = body[start:end].replace("__device__ __forceinline__", "static inline")
    src += """
extern "C" unsigned char enc_e4m3(float x) { return st_e4m3(x); }
extern "C" unsigned char enc_e5m2(float x) { return st_e5m2(x); }
extern "C" float dec_e4m3(unsigned char b) { return ld_e4m3(b); }
extern "C" float dec_e5m2(unsigned char b) { return ld_e5m2(b); }
extern "C" void enc_many(const float* x, unsigned char* out, long n, int e5m2) {
  for (long i = 0; i < n; ++i) out[i] = e5m2 ? st_e5m2(x[i]) : st_e4m3(x[i]);
}
"""
    tmp = tmp_path_factory.mktemp("fp8")
    (tmp / "fp8.cpp").write_text(src)
    subprocess.run([CLANG, "-O2", "-shared", "-fPIC", str(tmp / "fp8.cpp"), "-o", str(tmp / "libfp8.so")], check=True)
    lib = ctypes.CDLL(str(tmp / "libfp8.so"))
    lib.dec_e4m3.restype = lib.dec_e5m2.restype = ctypes.c_float
    lib.dec_e4m3.argtypes = lib.dec_e5m2.argtypes = [ctypes.c_ubyte]
    lib.enc_many.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long, ctypes.c_int]
    return lib


def _torch_codes(x, dtype):
    return x.to(dtype).view(torch.uint8).numpy()


def _encode(lib, x, e5m2):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.uint8)
    lib.enc_many(x.ctypes.data, out.ctypes.data, x.size, int(e5m2))
    return out


@pytest.mark.parametrize("dtype", FP8)
def test_every_code_decodes_as_torch(host_fp8, dtype):
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(dtype).float().numpy()
    dec = host_fp8.dec_e5m2 if dtype == torch.float8_e5m2 else host_fp8.dec_e4m3
    got = np.array([dec(int(c)) for c in range(256)], dtype=np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))  # signed zeros too


@pytest.mark.parametrize("dtype", FP8)
def test_encoding_matches_torch(host_fp8, dtype):
    e5m2 = dtype == torch.float8_e5m2
    codes = torch.arange(256, dtype=torch.uint8).view(dtype).float()
    finite = codes[torch.isfinite(codes)].unique()
    mids = (finite[1:] + finite[:-1]) / 2  # the ties, and one float either side of them
    edges = torch.cat([finite, mids, torch.nextafter(mids, torch.tensor(float("inf"))),
                       torch.nextafter(mids, torch.tensor(float("-inf"))),
                       torch.nextafter(finite, torch.tensor(float("inf"))), torch.nextafter(finite, torch.tensor(0.0))])
    special = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 448.0, 464.0, 479.99997, 480.0,
                            480.00003, 57344.0, 61439.996, 61440.0, 61440.004, 65536.0, 1e30, 1e-30, 2.0 ** -9,
                            2.0 ** -10, 3 * 2.0 ** -11, 2.0 ** -16, 2.0 ** -17, 3 * 2.0 ** -18, 2.0 ** -6, 2.0 ** -14])
    g = torch.Generator().manual_seed(8)
    random = torch.cat([torch.randn(200000, generator=g) * s for s in (1e-5, 1e-3, 0.1, 1.0, 30.0, 500.0, 3e4, 1e5)])
    x = torch.cat([edges, -edges, special, -special, random]).float()
    got = _encode(host_fp8, x.numpy(), e5m2)
    want = _torch_codes(x, dtype)
    nan = np.isnan(x.to(dtype).float().numpy())
    bad = np.nonzero((got != want) & ~nan)[0]
    assert bad.size == 0, [(float(x[i]), int(got[i]), int(want[i])) for i in bad[:10]]
    # NaN results: both give a NaN code (the sign bit is not compared)
    got_nan = codes.numpy()[got[nan]] if nan.any() else np.array([])
    assert np.isnan(got_nan).all()


def test_fp8_typing_follows_the_reference():
    # ranks: fp8 (5) below the 16-bit floats (6) (reference frontend/types.py:441-468)
    assert generic._promote("float8_e4m3fn", "float16") == "float16"
    assert generic._promote("float8_e5m2", "float32") == "float32"
    assert generic._promote("float8_e4m3fn", "float8_e4m3fn") == "float8_e4m3fn"
    assert generic._promote("int32", "float8_e5m2") == "float8_e5m2"
    ident, _ = generic.TilePlan._combine("max", "float8_e4m3fn", "float")
    assert ident == "(-448.0f)"
    ident, _ = generic.TilePlan._combine("min", "float8_e5m2", "float")
    assert ident == "__builtin_huge_valf()"


# ------------------------------------------------------------------ programs
BS = Symbol("BS", meta=True)
DOT_BM = Symbol("DOT_BM", meta=True)


def copy_application(x, output):
    output = x  # noqa: F841


def add_application(x, y, output):
    output = x + y  # noqa: F841


def scale_application(x, output):
    output = x * 3 - 1.5  # noqa: F841


def _elementwise(application, n):
    return ninetoothed.make(lambda *ts: tuple(t.tile((BS,)) for t in ts), application, tuple(Tensor(1) for _ in range(n)))


def dot_arrangement(x, w, o):
    xt = x.tile((DOT_BM, -1))
    return xt, w.tile((-1, -1)).expand((xt.shape[0], -1)), o.tile((DOT_BM, -1))


def dot_application(x, w, o):
    o = ntl.dot(x, w)  # noqa: F841


def max_arrangement(x, o):
    return x.tile((1, -1)), o.tile((1,))


def max_application(x, o):
    o = ntl.max(x)  # noqa: F841


def _plan(handle, *args, **meta):
    names = handle._abi["public_args"]
    return handle._kernel.specialize(dict(zip(names, args)), meta)


def test_fp8_programs_compile():
    e4, e5 = torch.float8_e4m3fn, torch.float8_e5m2
    for dtype in FP8:
        plan = _plan(_elementwise(add_application, 3), torch.empty(100, dtype=dtype), torch.empty(100, dtype=dtype),
                     torch.empty(100, dtype=dtype), BS=64)
        src = plan.sources_for({"x": torch.empty(100, dtype=dtype), "y": torch.empty(100, dtype=dtype),
                                "output": torch.empty(100, dtype=dtype)})[0]
        body = src[src.index('extern "C" __global__'):]
        kind = "e4m3" if dtype == e4 else "e5m2"
        assert f"r_{kind}((v0 + v1))" in body and f"st_{kind}(" in body and f"ld_{kind}(" in body
        assert len(GenericPlan.compile(src)) > 1000
    h = ninetoothed.make(dot_arrangement, dot_application, (Tensor(2), Tensor(2), Tensor(2)))
    for tx, tw in ((e4, e4), (e5, e5), (e4, e5), (e4, torch.float16)):
        plan = _plan(h, torch.empty(64, 48, dtype=tx), torch.empty(48, 40, dtype=tw), torch.empty(64, 40), DOT_BM=32)
        assert plan.describe()["family"] == "generic"
        src = plan.source()
        assert "__builtin_amdgcn_mfma_f32_32x32x16_f16" in src  # fp8 staged exactly as fp16
        assert len(GenericPlan.compile(src)) > 1000


# ------------------------------------------------------------------ GPU
def _values(n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * torch.exp2(torch.randint(-18, 18, (n,), generator=g).float())
    x[:8] = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 464.0, 61440.0, 2.0 ** -10])
    return x


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", FP8)
def test_stores_into_fp8_match_torch(dtype):
    x = _values(100003, 3).cuda()
    out = torch.empty(x.shape, dtype=dtype, device="cuda")
    _elementwise(copy_application, 2)(x, out, BS=256)
    want = x.to(dtype)
    same = out.view(torch.uint8) == want.view(torch.uint8)
    both_nan = torch.isnan(out.float()) & torch.isnan(want.float())
    assert bool((same | both_nan).all())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", FP8)
def test_fp8_loads_and_arithmetic(dtype):
    codes = torch.arange(256, dtype=torch.uint8).repeat(40).cuda()
    x = codes.view(dtype)
    y = codes.roll(7).view(dtype)
    out32 = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    _elementwise(copy_application, 2)(x, out32, BS=256)
    assert torch.equal(torch.isnan(out32), torch.isnan(x.float()))
    ok = ~torch.isnan(out32)
    assert torch.equal(out32[ok], x.float()[ok])
    # fp8 + fp8 in fp8: the exact sum rounded once (torch: fp32 sum, then the cast)
    out = torch.empty(x.shape, dtype=dtype, device="cuda")
    _elementwise(add_application, 3)(x, y, out, BS=256)
    want = (x.float() + y.float()).to(dtype)
    same = out.view(torch.uint8) == want.view(torch.uint8)
    assert bool((same | (torch.isnan(out.float()) & torch.isnan(want.float()))).all())
    # a weak scalar expression on fp8 (each operation rounded to fp8, as the 16-bit types)
    small = torch.randn(4096, device="cuda").to(dtype)
    out = torch.empty_like(small)
    _elementwise(scale_application, 2)(small, out, BS=256)
    want = ((small.float() * 3).to(dtype).float() - 1.5).to(dtype)
    assert torch.equal(out.view(torch.uint8), want.view(torch.uint8))


@pytest.mark.gpu
@pytest.mark.parametrize("tx, tw", ((torch.float8_e4m3fn, torch.float8_e4m3fn), (torch.float8_e5m2, torch.float8_e5m2),
                                    (torch.float8_e4m3fn, torch.float8_e5m2), (torch.float8_e5m2, torch.float16)))
def test_fp8_dot_on_the_matrix_core(tx, tw):
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(96, 40, generator=g)).to(tx).cuda()
    w = (torch.randn(40, 24, generator=g)).to(tw).cuda()
    o = torch.full((96, 24), float("nan"), device="cuda")
    h = ninetoothed.make(dot_arrangement, dot_application, (Tensor(2), Tensor(2), Tensor(2)))
    assert "mfma" in _plan(h, x, w, o, DOT_BM=32).source()
    h(x, w, o, DOT_BM=32)
    torch.testing.assert_close(o, x.float() @ w.float(), rtol=1e-5, atol=1e-5)  # exact products, fp32 sums


@pytest.mark.gpu
def test_fp8_max_of_masked_rows_is_the_identity():
    # rows shorter than the tile: masked elements take e4m3fn's identity, -448, not -inf (which
    # would encode as NaN); an all-negative row's maximum is its own largest element
    x = (-torch.rand(6, 37, device="cuda") * 400 - 1).to(torch.float8_e4m3fn)
    o = torch.empty(6, dtype=torch.float8_e4m3fn, device="cuda")
    ninetoothed.make(lambda a, b: (a.tile((1, 64)), b.tile((1,))), max_application, (Tensor(2), Tensor(1)))(x, o)
    assert torch.equal(o.float(), x.float().max(dim=1).values)
