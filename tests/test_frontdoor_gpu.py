"""The reference's known-answer tests, run through the drop-in ``make``/``jit`` front door.

Each test builds the kernel exactly as a NineToothed user would (arrangement +
application + symbolic tensors, tests/programs.py), calls it on seeded GPU tensors,
and checks the result against (a) the reference test's own torch oracle and
tolerance where that is meaningful on MI355X, and (b) this build's CPU oracle
(``oracle.apply``, the tile-by-tile restatement of the application) on the same
inputs.  It also asserts that the call really went through libnt_mi355x.so.
"""

import functools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ninetoothed_amd as ninetoothed
import programs as pg
from ninetoothed_amd import _lib, kernels
from oracle import apply

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _gen(seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _randn(shape, dtype, seed, scale=1.0):
    return (torch.randn(shape, generator=_gen(seed)) * scale).to(dtype).to(DEV)


def _rand(shape, dtype, seed, lo=0.0, hi=1.0):
    return (torch.rand(shape, generator=_gen(seed)) * (hi - lo) + lo).to(dtype).to(DEV)


def _np(t):
    return t.float().cpu().numpy()


@pytest.fixture(autouse=True)
def _no_tf32():
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def test_native_library_is_loaded():
    import ctypes  # noqa: F401

    lib = _lib.load()
    assert lib.nt_abi_version() == _lib.ABI_VERSION
    maps = open("/proc/self/maps").read()
    assert "libnt_mi355x.so" in maps


# ------------------------------------------------------------------------ matmul
def test_matmul_reference_case():
    m = n = k = 512
    lhs, rhs = _randn((m, k), torch.float16, 1), _randn((k, n), torch.float16, 2)
    output = torch.empty((m, n), dtype=torch.float16, device=DEV)
    kernel = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    assert kernel(lhs, rhs, output) is output
    expected = torch.matmul(lhs.float(), rhs.float()).half()
    assert torch.allclose(output, expected, atol=1e-2, rtol=1e-2)
    ref = apply.matmul(_np(lhs), _np(rhs), "float16", pg.matmul_arrangement, block=(64, 64, 64))
    assert np.allclose(_np(output), ref, atol=1e-2, rtol=1e-2)
    assert kernel.plans()[0]["family"] == "gemm"


@pytest.mark.parametrize("dtype", (torch.float8_e5m2, torch.float8_e4m3fn))
def test_matmul_fp8_reference_case(dtype):
    # reference tests/test_matmul.py:64-88: fp8 lhs, column-major fp8 rhs (`other.T.to(dtype)`),
    # fp16 output, atol 0.125 against torch.matmul on the operands widened to fp16
    m = n = k = 512
    lhs = _randn((m, k), torch.float16, 11).to(dtype)
    rhs = _randn((k, n), torch.float16, 12).T.to(dtype)  # used as the (k, n) operand: column-major
    assert rhs.stride() == (1, k)
    output = torch.empty((m, n), dtype=torch.float16, device=DEV)
    kernel = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    kernel(lhs, rhs, output)
    expected = torch.matmul(lhs.to(torch.float16), rhs.to(torch.float16))
    assert torch.allclose(output, expected, atol=0.125)
    ref = apply.matmul(_np(lhs), _np(rhs), "float16", pg.matmul_arrangement, block=(64, 64, 64))
    assert np.allclose(_np(output), ref, atol=1e-2, rtol=1e-2)


def test_matmul_fp32_readme_case():
    lhs, rhs = _randn((512, 512), torch.float32, 3), _randn((512, 512), torch.float32, 4)
    output = torch.empty((512, 512), device=DEV)
    kernel = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application_fp32, pg.matmul_tensors())
    kernel(lhs, rhs, output)
    assert torch.allclose(output, (lhs.double() @ rhs.double()).float(), atol=1e-4, rtol=1e-4)


# ------------------------------------------------------------------------- addmm
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_addmm_reference_case(dtype):
    m = n = k = 512
    input, mat1, mat2 = _randn((m, n), dtype, 5), _randn((m, k), dtype, 6), _randn((k, n), dtype, 7)
    beta, alpha = 0.3723, 0.8391
    output = torch.empty((m, n), dtype=dtype, device=DEV)
    kernel = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    kernel(input, mat1, mat2, beta, alpha, output)
    ref = apply.addmm(_np(input), _np(mat1), _np(mat2), beta, alpha, "float16" if dtype == torch.float16 else "bfloat16",
                      pg.addmm_arrangement, block=(64, 64, 64))
    assert np.allclose(_np(output), ref, atol=2e-2, rtol=1e-2)
    if dtype == torch.float16:
        # The reference test's own oracle and tolerance.
        assert torch.allclose(output, torch.addmm(input, mat1, mat2, beta=beta, alpha=alpha), atol=0.075)


@pytest.mark.parametrize("dtype", (torch.float8_e5m2, torch.float8_e4m3fn))
def test_addmm_fp8_reference_case(dtype):
    # reference tests/test_addmm.py:57-90 (float8_e5m2 case): fp8 input and mat1, column-major
    # fp8 mat2 (`mat2.T.to(dtype)`), fp16 output, atol 0.125 against torch.addmm on the
    # operands widened to fp16
    m = n = k = 512
    input = _randn((m, n), torch.float16, 15).to(dtype)
    mat1 = _randn((m, k), torch.float16, 16).to(dtype)
    mat2 = _randn((k, n), torch.float16, 17).T.to(dtype)
    assert mat2.stride() == (1, k)
    beta, alpha = 0.6180, 0.4142
    output = torch.empty((m, n), dtype=torch.float16, device=DEV)
    kernel = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    kernel(input, mat1, mat2, beta, alpha, output)
    f16 = torch.float16
    expected = torch.addmm(input.to(f16), mat1.to(f16), mat2.to(f16), beta=beta, alpha=alpha)
    assert torch.allclose(output, expected, atol=0.125)
    ref = apply.addmm(_np(input), _np(mat1), _np(mat2), beta, alpha, "float16", pg.addmm_arrangement,
                      block=(64, 64, 64))
    assert np.allclose(_np(output), ref, atol=1e-2, rtol=1e-2)


def test_addmm_headline_shape():
    m = n = k = 4096
    s = 1.0 / math.sqrt(k)
    input, mat1, mat2 = (_randn((4096, 4096), torch.float16, 8 + i, s) for i in range(3))
    output = torch.empty_like(input)
    kernel = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    kernel(input, mat1, mat2, 0.5, 1.0, output)
    ref = (0.5 * input.float() + (mat1.float() @ mat2.float()).half().float()).half()
    assert torch.allclose(output, ref, atol=1e-2, rtol=1e-2)


# ------------------------------------------------------------------------ conv2d
@pytest.mark.parametrize("padding", (0, (1, 1), (0, 1), (2, 0)))
def test_conv2d_reference_case(padding):
    x, w = _rand((4, 64, 16, 16), torch.float16, 11), _rand((512, 64, 3, 3), torch.float16, 12)
    pad = (padding, padding) if isinstance(padding, int) else padding
    p, q = 16 + 2 * pad[0] - 2, 16 + 2 * pad[1] - 2
    y = torch.empty((4, 512, p, q), dtype=torch.float16, device=DEV)
    kernel = pg.make_conv2d()
    kernel(x, w, y, padding_h=pad[0], padding_w=pad[1])
    expected = F.conv2d(x.float(), w.float(), padding=pad).half()
    assert torch.allclose(y, expected, rtol=1e-3, atol=1e-3)  # the reference test's tolerance
    ref = apply.conv2d(_np(x), _np(w), pad, functools.partial(pg.conv2d_arrangement, enable_padding=True),
                       block=(64, 64, 64))
    assert np.allclose(_np(y), ref, rtol=1e-3, atol=1e-3)


def test_conv2d_headline_shape():
    x = _randn((16, 256, 56, 56), torch.float16, 13)
    w = _randn((256, 256, 3, 3), torch.float16, 14, 1.0 / math.sqrt(256 * 9))
    y = torch.empty_like(x)
    pg.make_conv2d()(x, w, y, padding_h=1, padding_w=1)
    assert torch.allclose(y.float(), F.conv2d(x.float(), w.float(), padding=1), atol=1e-2, rtol=1e-2)


# --------------------------------------------------------------------- attention
@pytest.mark.parametrize("is_causal", (False, True))
@pytest.mark.parametrize("seq_len", (1024, 1))
@pytest.mark.parametrize("dtype, tol", ((torch.float32, 0.025), (torch.float16, 0.01)))
def test_attention_reference_case(is_causal, seq_len, dtype, tol):
    q, k, v = (_randn((2, 4, seq_len, 64), dtype, 20 + i) for i in range(3))
    o = torch.empty_like(q)
    kernel = ninetoothed.make(pg.attention_arrangement, pg.attention_application, pg.attention_tensors())
    kernel(q, k, v, is_causal, o)
    expected = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=is_causal, scale=1)
    assert torch.allclose(o.float(), expected, rtol=tol, atol=tol)
    if dtype == torch.float16 and seq_len == 1024:
        ref = apply.attention(_np(q[:1, :2]), _np(k[:1, :2]), _np(v[:1, :2]), is_causal, pg.attention_arrangement,
                              block=(64, 64))
        assert np.allclose(_np(o[:1, :2]), ref, atol=5e-3, rtol=5e-3)


@pytest.mark.parametrize("is_causal", (False, True))
def test_attention_headline_scaled(is_causal):
    q, k, v = (_randn((4, 32, 4096, 128), torch.float16, 30 + i) for i in range(3))
    o = torch.empty_like(q)
    kernel = ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors())
    kernel(q, k, v, is_causal, o)
    _check_every_head(q, k, v, o, is_causal, 1 / math.sqrt(128))


def _check_every_head(q, k, v, o, causal, scale, tol=1e-2):
    """Compare every (batch, head) slice with an fp32 restatement of attention, one head at a time.

    The output comes from torch.empty, so a head the kernel's work order skips or writes
    twice fails here whichever XCD or head group it belongs to."""
    sq, sk = q.shape[2], k.shape[2]
    mask = None
    if causal:
        mask = torch.ones(sq, sk, dtype=torch.bool, device=q.device).tril().logical_not()  # key j <= query i
    bad = []
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            s = torch.matmul(q[b, h].float(), k[b, h].float().t().contiguous()) * scale
            if mask is not None:
                s.masked_fill_(mask, float("-inf"))
            ref = torch.matmul(torch.softmax(s, dim=-1), v[b, h].float())
            if not torch.allclose(o[b, h].float(), ref, atol=tol, rtol=tol):
                bad.append((b, h, float((o[b, h].float() - ref).abs().max())))
    assert not bad, f"heads outside tolerance (b, h, max error): {bad[:8]}"


# B*H = 64 and 24: with 64 (8 heads per XCD, two groups of four) both the grouped causal
# order and the per-XCD non-causal order run with every head checked; with 24 (3 heads per
# XCD) the causal launch takes the ungrouped per-XCD order; B*H = 6 takes the plain order.
@pytest.mark.parametrize("is_causal", (False, True))
@pytest.mark.parametrize("shape", ((2, 32, 1024, 128), (3, 8, 640, 64), (2, 3, 333, 128)))
def test_attention_work_orders_every_head(is_causal, shape):
    q, k, v = (_randn(shape, torch.float16, 70 + i) for i in range(3))
    o = torch.empty_like(q)
    kernel = ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors())
    kernel(q, k, v, is_causal, o)
    torch.cuda.synchronize()
    _check_every_head(q, k, v, o, is_causal, 1 / math.sqrt(128))  # the application's constant scale
    if shape[3] == 128:  # the pipelined kernel's work order too (same block order, its own grid)
        o.fill_(float("nan"))
        kernels.attention(q, k, v, o, causal=is_causal, q_scale=kernels.LOG2E / math.sqrt(128), config=1)
        _check_every_head(q, k, v, o, is_causal, 1 / math.sqrt(128))


# ----------------------------------------------------------------------- softmax
def test_softmax_reference_case():
    x = _rand((1823, 781), torch.float32, 40)
    y = pg.make_softmax()
    out = torch.empty_like(x)
    y(x, out, BLOCK_SIZE=x.shape[-1])
    assert torch.allclose(out, torch.softmax(x, dim=-1))
    assert np.allclose(_np(out), apply.softmax(_np(x), 781), atol=1e-6, rtol=1e-5)


def test_softmax_headline_shape():
    x = _randn((8192, 8192), torch.float16, 41, 2.0)
    out = torch.empty_like(x)
    pg.make_softmax()(x, out, BLOCK_SIZE=8192)
    assert torch.allclose(out.float(), torch.softmax(x.float(), -1), atol=1e-2, rtol=1e-2)


def test_softmax_partial_block():
    x = _randn((33, 1000), torch.float32, 42)
    out = torch.empty_like(x)
    pg.make_softmax()(x, out, BLOCK_SIZE=256)
    assert np.allclose(_np(out), apply.softmax(_np(x), 256), atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("layout", ("transposed", "every_other_column"))
@pytest.mark.parametrize("block", (781, 256))
def test_softmax_strided_columns(layout, block):
    # the reference passes strides to its kernel: softmax(x.t(), y) and softmax(x[:, ::2], y) run
    if layout == "transposed":
        x = _randn((781, 64), torch.float16, 21, 2.0).t()
    else:
        x = _randn((64, 1562), torch.float16, 21, 2.0)[:, ::2]
    assert x.stride(1) != 1
    y = torch.full(x.shape, float("nan"), dtype=torch.float16, device=DEV)
    pg.make_softmax()(x, y, BLOCK_SIZE=block)
    ref = apply.softmax(_np(x), block, "float16")
    assert np.allclose(_np(y), ref, atol=1e-3, rtol=1e-2)
    if block == 781:
        assert torch.allclose(y.float(), torch.softmax(x.float(), -1), atol=1e-3, rtol=1e-2)


@pytest.mark.parametrize("in_dtype, out_dtype", ((torch.float16, torch.float32), (torch.float32, torch.bfloat16),
                                                 (torch.bfloat16, torch.float16)))
def test_softmax_output_of_another_dtype(in_dtype, out_dtype):
    # the reference's store casts the fp32 quotient to the output's type
    x = _randn((129, 3000), in_dtype, 22, 2.0)
    y = torch.full(x.shape, float("nan"), dtype=out_dtype, device=DEV)
    pg.make_softmax()(x, y, BLOCK_SIZE=3000)
    names = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}
    ref = apply.softmax(_np(x), 3000, names[in_dtype], out_dtype=names[out_dtype])
    assert np.allclose(_np(y), ref, atol=1e-3, rtol=1e-2)
    # fp32 math throughout on the kernel's side: close to torch's float softmax of the same values
    assert torch.allclose(y.float(), torch.softmax(x.float(), -1).to(out_dtype).float(), atol=1e-5, rtol=1e-2)


# -------------------------------------------------------------------- max_pool2d
@pytest.mark.parametrize("in_dtype, out_dtype", ((torch.float16, torch.float32), (torch.float32, torch.float16),
                                                 (torch.bfloat16, torch.float32)))
@pytest.mark.parametrize("ceil_mode", (False, True))
def test_max_pool2d_output_of_another_dtype(in_dtype, out_dtype, ceil_mode):
    x = _rand((3, 5, 33, 34), in_dtype, 23, -1.0, 1.0)
    kernel = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=ceil_mode),
                              pg.max_pool2d_application, pg.max_pool2d_tensors())
    ref = F.max_pool2d(x, (2, 2), ceil_mode=ceil_mode)
    y = torch.full(ref.shape, float("nan"), dtype=out_dtype, device=DEV)
    kernel(x, y, WINDOW_HEIGHT=2, WINDOW_WIDTH=2)
    assert torch.equal(y, ref.to(out_dtype))  # bit-exact: rounding is monotone
    oracle = apply.max_pool2d(_np(x), (2, 2), ceil_mode,
                              functools.partial(pg.max_pool2d_arrangement, ceil_mode=ceil_mode))
    assert np.array_equal(_np(y), _np(torch.from_numpy(oracle).to(out_dtype)))


@pytest.mark.parametrize("ceil_mode", (False, True))
def test_max_pool2d_reference_case(ceil_mode):
    x = _randn((32, 3, 64, 64), torch.float16, 50)
    div = (lambda a, b: (a + b - 1) // b) if ceil_mode else (lambda a, b: a // b)
    p = q = div(64 - 3, 3) + 1
    y = torch.empty((32, 3, p, q), dtype=torch.float16, device=DEV)
    kernel = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=ceil_mode),
                              pg.max_pool2d_application, pg.max_pool2d_tensors())
    kernel(x, y, WINDOW_HEIGHT=3, WINDOW_WIDTH=3)
    assert torch.equal(y, F.max_pool2d(x, (3, 3), ceil_mode=ceil_mode))
    ref = apply.max_pool2d(_np(x), (3, 3), ceil_mode, functools.partial(pg.max_pool2d_arrangement, ceil_mode=ceil_mode))
    assert np.array_equal(_np(y), ref)


def test_max_pool2d_headline_shape():
    x = _rand((32, 128, 112, 112), torch.float16, 51, -1.0, 1.0)
    y = torch.empty((32, 128, 56, 56), dtype=torch.float16, device=DEV)
    kernel = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=False), pg.max_pool2d_application,
                              pg.max_pool2d_tensors())
    kernel(x, y, WINDOW_HEIGHT=2, WINDOW_WIDTH=2)
    assert torch.equal(y, F.max_pool2d(x, (2, 2)))


# --------------------------------------------------------------------------- add
@pytest.mark.parametrize("size", (98432, 1, 1000003))
def test_add_reference_case(size):
    lhs, rhs = _rand((size,), torch.float32, 60), _rand((size,), torch.float32, 61)
    out = torch.empty_like(lhs)
    pg.make_add()(lhs, rhs, out)
    assert torch.allclose(out, lhs + rhs)
    assert np.array_equal(_np(out), apply.add(_np(lhs), _np(rhs), 64))


def test_empty_output_launches_nothing():
    kernel = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    out = torch.empty((0, 8), dtype=torch.float16, device=DEV)
    assert kernel(torch.empty((0, 4), dtype=torch.float16, device=DEV),
                  torch.empty((4, 8), dtype=torch.float16, device=DEV), out) is out


# ----------------------------------------------------------- bound-launcher cache
def test_repeat_calls_take_new_data_and_scalars():
    kernel = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    output = torch.empty((256, 192), dtype=torch.float16, device=DEV)
    for i, (beta, alpha) in enumerate(((0.5, 1.25), (-1.0, 0.25), (0.0, 2.0))):
        input, mat1, mat2 = _randn((256, 192), torch.float16, 70 + i), _randn((256, 128), torch.float16, 80 + i), \
            _randn((128, 192), torch.float16, 90 + i)
        assert kernel(input, mat1, mat2, beta, alpha, output) is output
        ref = apply.addmm(_np(input), _np(mat1), _np(mat2), beta, alpha, "float16", pg.addmm_arrangement,
                          block=(64, 64, 64))
        assert np.allclose(_np(output), ref, atol=2e-2, rtol=1e-2), (beta, alpha)
    assert len(kernel.plans()) == 1


def test_stride_or_shape_change_rebinds():
    kernel = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    lhs = _randn((192, 320), torch.float16, 100)
    rhs = _randn((320, 256), torch.float16, 101)
    rhs_t = _randn((256, 320), torch.float16, 102).t()  # same shape as rhs, k-contiguous
    for a, b in ((lhs, rhs), (lhs, rhs_t), (lhs[:64], rhs), (lhs, rhs)):
        out = torch.empty((a.shape[0], b.shape[1]), dtype=torch.float16, device=DEV)
        kernel(a, b, out)
        assert torch.allclose(out.float(), a.float() @ b.float(), atol=2e-2, rtol=1e-2)
    assert len(kernel.plans()) == 3


def test_cached_key_still_checks_arguments():
    kernel = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    lhs, rhs = _randn((64, 64), torch.float16, 103), _randn((64, 64), torch.float16, 104)
    out = torch.empty((64, 64), dtype=torch.float16, device=DEV)
    kernel(lhs, rhs, out)
    with pytest.raises(TypeError):
        kernel(lhs.cpu(), rhs, out)
    with pytest.raises(TypeError):
        kernel(lhs, rhs)
    with pytest.raises(TypeError):
        kernel(lhs, rhs, out, output=out)
    out2 = torch.zeros_like(out)
    kernel(lhs, rhs, output=out2)  # public argument by keyword: the checked path
    assert torch.equal(out2, out)
