"""GPU parity of every libnt_mi355x.so entry point against torch fp32 references.

These call the C ABI through ``ninetoothed_amd.kernels`` directly (no front door),
on seeded CPU-generated inputs moved to the GPU.  Tolerances: bit-exact for
max_pool2d, 1e-2 (atol and rtol) for fp16/bf16 against fp32 accumulation, 1e-4 for
fp32, as the north-star contract states; attention in fp32 keeps the reference
test's 0.025 (tests/test_attention.py:99-117 of the reference).
"""

import math

import pytest
import torch
import torch.nn.functional as F

from ninetoothed_amd import kernels

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _gen(seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _randn(shape, dtype, seed, scale=1.0):
    return (torch.randn(shape, generator=_gen(seed), dtype=torch.float32) * scale).to(dtype).to(DEV)


def _rand(shape, dtype, seed, lo=0.0, hi=1.0):
    return (torch.rand(shape, generator=_gen(seed), dtype=torch.float32) * (hi - lo) + lo).to(dtype).to(DEV)


TOL = {torch.float16: 1e-2, torch.bfloat16: 1e-2, torch.float32: 1e-4}


@pytest.fixture(autouse=True, scope="module")
def _no_tf32():
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    yield


# --------------------------------------------------------------------------- add
@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, torch.bfloat16))
@pytest.mark.parametrize("n", (98432, 1, 7, 1000003))
def test_add(n, dtype):
    a = _rand((n,), dtype, 1)
    b = _rand((n,), dtype, 2)
    out = torch.empty_like(a)
    kernels.add(a, b, out)
    torch.cuda.synchronize()
    expected = (a.float() + b.float()).to(dtype)
    assert torch.equal(out, expected)


def test_add_strided():
    base = _rand((3000,), torch.float32, 3)
    a, b = base[::3], base[1::3]
    out = torch.empty(2000, device=DEV)[::2]
    kernels.add(a, b, out)
    assert torch.equal(out, a + b)


# ----------------------------------------------------------------------- softmax
def test_softmax_reference_case_fp32():
    # The reference's KAT: fp32 rand [1823, 781], torch.allclose defaults.
    x = _rand((1823, 781), torch.float32, 4)
    y = torch.empty_like(x)
    kernels.softmax(x, y)
    assert torch.allclose(y, torch.softmax(x, dim=-1))


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
@pytest.mark.parametrize("cols", (8192, 1000, 33, 20000, 70000))
def test_softmax_rows(cols, dtype):
    x = _randn((64, cols), dtype, 5, scale=2.0)
    y = torch.empty_like(x)
    kernels.softmax(x, y)
    ref = torch.softmax(x.float(), dim=-1)
    tol = TOL[dtype]
    assert torch.allclose(y.float(), ref, atol=tol, rtol=tol)
    assert torch.allclose(y.float().sum(-1), torch.ones(64, device=DEV), atol=3e-2 if dtype != torch.float32 else 1e-4)


def test_softmax_segments():
    # BLOCK_SIZE smaller than the row: each 128-wide segment is normalised alone.
    x = _randn((16, 1000), torch.float32, 6)
    y = torch.empty_like(x)
    kernels.softmax(x, y, block=128)
    xp = F.pad(x, (0, 1024 - 1000), value=float("-inf")).view(16, 8, 128)
    ref = torch.softmax(xp, dim=-1).view(16, 1024)[:, :1000]
    assert torch.allclose(y, ref, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("config", (0, 5))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_softmax_short_contiguous_widths(dtype, config):
    # Contiguous rows whose byte length is no multiple of 16: most rows start inside a 16-byte
    # vector, so the lane-group kernel splits off a head of up to V - 1 elements (7 for
    # 16-bit types, 3 for fp32), more than a group of 1, 2 or 4 lanes has.  y starts as NaN
    # so an element the kernel never writes shows.
    widths = range(2, 32) if dtype != torch.float32 else range(2, 16)
    for cols in widths:
        x = _randn((37, cols), dtype, 100 + cols, scale=2.0)
        y = torch.full_like(x, float("nan"))
        kernels.softmax(x, y, config=config)
        ref = torch.softmax(x.float(), dim=-1)
        assert not torch.isnan(y).any(), f"cols={cols}: unwritten outputs"
        assert torch.allclose(y.float(), ref, atol=TOL[dtype], rtol=TOL[dtype]), f"cols={cols}"


@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
@pytest.mark.parametrize("block", (None, 100))
def test_softmax_any_strides(dtype, block):
    # column strides other than 1 (a transposed view, every third column, both at once)
    # take the element-wise kernel; the forced vector kernels refuse them before launching
    base = _randn((450, 300), dtype, 15, scale=2.0)
    views = (base.t(), base[:, ::3], base.t()[::2, 1::3])
    for x in views:
        rows, cols = x.shape
        blk = cols if block is None else block
        nseg = -(-cols // blk)
        xp = F.pad(x.float(), (0, nseg * blk - cols), value=float("-inf")).view(rows, nseg, blk)
        ref = torch.softmax(xp, dim=-1).view(rows, nseg * blk)[:, :cols]
        for y in (torch.full((rows, cols), float("nan"), dtype=dtype, device=DEV),
                  torch.full((cols, rows), float("nan"), dtype=dtype, device=DEV).t()):
            kernels.softmax(x, y, block=block)
            assert torch.allclose(y.float(), ref, atol=TOL[dtype], rtol=TOL[dtype])
            y.fill_(float("nan"))
            kernels.softmax(x, y, block=block, config=kernels.SOFTMAX_ANY)
            assert torch.allclose(y.float(), ref, atol=TOL[dtype], rtol=TOL[dtype])
        with pytest.raises(ValueError):
            kernels.softmax(x, torch.empty(rows, cols, dtype=dtype, device=DEV), block=block, config=1)


def test_softmax_headline_shape():
    x = _randn((8192, 8192), torch.float16, 7, scale=2.0)
    y = torch.empty_like(x)
    kernels.softmax(x, y)
    ref = torch.softmax(x.float(), dim=-1)
    assert torch.allclose(y.float(), ref, atol=1e-2, rtol=1e-2)


# -------------------------------------------------------------------- max_pool2d
@pytest.mark.parametrize("ceil_mode", (False, True))
def test_max_pool2d_reference_case(ceil_mode):
    x = _randn((32, 3, 64, 64), torch.float16, 8)
    h = w = 64
    r = s = 3
    div = (lambda a, b: (a + b - 1) // b) if ceil_mode else (lambda a, b: a // b)
    p, q = div(h - r, r) + 1, div(w - s, s) + 1
    y = torch.empty((32, 3, p, q), dtype=torch.float16, device=DEV)
    kernels.max_pool2d(x, y, (r, s))
    assert torch.equal(y, F.max_pool2d(x, (r, s), ceil_mode=ceil_mode))


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_max_pool2d_headline(dtype):
    x = _rand((32, 128, 112, 112), dtype, 9, -1.0, 1.0)
    y = torch.empty((32, 128, 56, 56), dtype=dtype, device=DEV)
    kernels.max_pool2d(x, y, (2, 2))
    assert torch.equal(y, F.max_pool2d(x, (2, 2)))


def test_max_pool2d_padding_stride_dilation():
    x = _randn((2, 5, 17, 19), torch.float16, 10)
    ref = F.max_pool2d(x, (3, 2), stride=(2, 3), padding=(1, 1), dilation=(2, 1))
    y = torch.empty_like(ref)
    kernels.max_pool2d(x, y, (3, 2), stride=(2, 3), padding=(1, 1), dilation=(2, 1))
    assert torch.equal(y, ref)


# -------------------------------------------------------------------------- gemm
def _gemm_ref(a, b, c=None, alpha=1.0, beta=0.0, round_dtype=None, out_dtype=None):
    acc = a.double() @ b.double()
    acc = acc.float()
    if round_dtype is not None:
        acc = acc.to(round_dtype).float()
    v = alpha * acc
    if c is not None:
        v = v + beta * c.float()
    return v.to(out_dtype or a.dtype)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("mnk", ((512, 512, 512), (4096, 4096, 4096), (300, 200, 100), (256, 512, 1000), (1, 1, 1),
                                 (256, 256, 64), (256, 512, 128), (512, 256, 192), (768, 1024, 320)))
def test_gemm16(mnk, dtype):
    m, n, k = mnk
    a = _randn((m, k), dtype, 11)
    b = _randn((k, n), dtype, 12)
    out = torch.empty((m, n), dtype=dtype, device=DEV)
    kernels.gemm(a, b, out, round_dtype=torch.float16 if dtype == torch.float16 else None)
    ref = _gemm_ref(a, b, round_dtype=torch.float16 if dtype == torch.float16 else None)
    tol = 1e-2 * max(1.0, math.sqrt(k) / 8)
    assert torch.allclose(out.float(), ref.float(), atol=tol, rtol=1e-2)


_FP8 = (torch.float8_e5m2, torch.float8_e4m3fn)


@pytest.mark.parametrize("dtype", _FP8)
def test_gemm_fp8_every_finite_value_is_exact(dtype):
    # a holds every finite byte pattern once (inf/NaN would spread through the zero terms);
    # b is a one-hot matrix, so out = a exactly: pins the fp8 -> fp16 widening bit for bit
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    vals = codes.view(dtype).float()
    codes = torch.where(torch.isfinite(vals), codes, torch.zeros_like(codes))
    a = codes.view(dtype).reshape(4, 64).to(DEV)
    b = torch.eye(64, dtype=torch.float32).to(dtype).to(DEV)
    out = torch.empty((4, 64), dtype=torch.float32, device=DEV)
    kernels.gemm(a, b, out)
    assert torch.equal(out, a.float())


@pytest.mark.parametrize("dtype", _FP8)
@pytest.mark.parametrize("mnk", ((300, 200, 100), (256, 512, 1000), (1, 1, 1)))
def test_gemm_fp8_ragged_strided(mnk, dtype):
    m, n, k = mnk
    a = _randn((m, k), torch.float16, 21).to(dtype)
    b = _randn((n, k), torch.float16, 22).to(dtype).t()  # k-contiguous
    c = _randn((m, n), torch.float16, 23)
    out = torch.empty((m, n), dtype=torch.float16, device=DEV)
    kernels.gemm(a, b, out, c=c, alpha=0.5, beta=2.0, round_dtype=torch.float16)
    ref = _gemm_ref(a.to(torch.float16), b.to(torch.float16), c, 0.5, 2.0, torch.float16)
    tol = 1e-2 * max(1.0, math.sqrt(k) / 8)
    assert torch.allclose(out.float(), ref.float(), atol=tol, rtol=1e-2)


@pytest.mark.parametrize("dtype", _FP8)
def test_gemm_fp8_rate_kernel_every_finite_value(dtype):
    # a k-contiguous, b column-major, M, N multiples of 256 and K of 64 (at least 192): the
    # fp8-rate kernel (the matrix core multiplies the fp8 bytes themselves).  a is one-hot
    # (row m selects k = m % 192) and b^T holds every finite byte pattern many times, so
    # out = b[m % 192, :] exactly, which pins the operand lane layout and the format codes.
    m, n, k = 512, 256, 192
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    finite = codes[torch.isfinite(codes.view(dtype).float())]
    idx = torch.arange(n * k) % finite.numel()
    bt = finite[idx].reshape(n, k).view(dtype).to(DEV)
    b = bt.t()
    a = torch.zeros((m, k), dtype=torch.float32)
    a[torch.arange(m), torch.arange(m) % k] = 1.0
    a = a.to(dtype).to(DEV)
    out = torch.empty((m, n), dtype=torch.float32, device=DEV)
    kernels.gemm(a, b, out)
    assert torch.equal(out, b.float()[torch.arange(m, device=DEV) % k])


@pytest.mark.parametrize("dtype", _FP8)
@pytest.mark.parametrize("k", (192, 320, 1024))
@pytest.mark.parametrize("padded", (False, True))
def test_gemm_fp8_rate_kernel(k, padded, dtype):
    # The fp8-rate kernel on random data with the addmm epilogue; padded: a and b^T as views
    # of wider buffers (row strides K + 64 and K + 128), the kernel's offsets come from them.
    m, n = 512, 768
    pa, pb = (64, 128) if padded else (0, 0)
    a = _randn((m, k + pa), torch.float16, 24).to(dtype)[:, :k]
    b = _randn((n, k + pb), torch.float16, 25).to(dtype)[:, :k].t()
    c = _randn((m, n), torch.float16, 26)
    out = torch.empty((m, n), dtype=torch.float16, device=DEV)
    kernels.gemm(a, b, out, c=c, alpha=0.5, beta=2.0, round_dtype=torch.float16)
    ref = _gemm_ref(a.to(torch.float16), b.to(torch.float16), c, 0.5, 2.0, torch.float16)
    tol = 1e-2 * max(1.0, math.sqrt(k) / 8)
    assert torch.allclose(out.float(), ref.float(), atol=tol, rtol=1e-2)


def test_addmm_epilogue():
    m = n = k = 512
    c = _randn((m, n), torch.float16, 13)
    a = _randn((m, k), torch.float16, 14)
    b = _randn((k, n), torch.float16, 15)
    out = torch.empty_like(c)
    alpha, beta = 0.37, 0.81
    kernels.gemm(a, b, out, c=c, alpha=alpha, beta=beta, round_dtype=torch.float16)
    ref = _gemm_ref(a, b, c, alpha, beta, torch.float16)
    assert torch.allclose(out.float(), ref.float(), atol=0.075)
    # torch.addmm is the reference test's oracle (atol 0.075).
    assert torch.allclose(out, torch.addmm(c, a, b, beta=beta, alpha=alpha), atol=0.075)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("round_dtype", (None, torch.float16, torch.bfloat16))
@pytest.mark.parametrize("c_kind", ("dense", "strided", "broadcast", "none"))
def test_addmm_fast_epilogue_variants(dtype, round_dtype, c_kind):
    # M, N multiples of 256 and K a multiple of 64: the DMA kernel, whose fast epilogue
    # stages the accumulators through LDS and rounds, scales and adds c per variant (six
    # out x round variants); strided out rows and every kind of c row stride it accepts.
    m, n, k = 512, 768, 256
    a = _randn((m, k), dtype, 30)
    b = _randn((k, n), dtype, 31)
    c = None
    if c_kind == "dense":
        c = _randn((m, n), dtype, 32)
    elif c_kind == "strided":
        c = _randn((m, n + 64), dtype, 32)[:, :n]
    elif c_kind == "broadcast":
        c = _randn((1, n), dtype, 32).expand(m, n)
    out = torch.empty((m, n + 128), dtype=dtype, device=DEV)[:, :n]
    kernels.gemm(a, b, out, c=c, alpha=0.75, beta=-1.25, round_dtype=round_dtype)
    ref = _gemm_ref(a, b, c, 0.75, -1.25, round_dtype)
    assert torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("k", (128, 192, 576))
def test_gemm_dma_padded_leading_dims(k, dtype):
    # The DMA kernel's operand offsets come from the row strides: a, b, c and out as views
    # of wider buffers (row strides K + 64, N + 128, N + 32, N + 64), K with 4, 6 and 18
    # k-tiles of 32.
    m, n = 512, 768
    a = _randn((m, k + 64), dtype, 40)[:, :k]
    b = _randn((k, n + 128), dtype, 41)[:, :n]
    c = _randn((m, n + 32), dtype, 42)[:, :n]
    out = torch.empty((m, n + 64), dtype=dtype, device=DEV)[:, :n]
    kernels.gemm(a, b, out, c=c, alpha=1.5, beta=0.25, round_dtype=None)
    ref = _gemm_ref(a, b, c, 1.5, 0.25, None)
    assert torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("config", (1, 2, 3))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_gemm_kernel_configs(config, dtype):
    # Each forced kernel configuration (DMA, register-staged eight-wave, element-wise
    # loader) on a call all three admit.
    m, n, k = 512, 768, 256
    a, b, c = _randn((m, k), dtype, 50), _randn((k, n), dtype, 51), _randn((m, n), dtype, 52)
    out = torch.empty((m, n), dtype=dtype, device=DEV)
    kernels.gemm(a, b, out, c=c, alpha=0.5, beta=2.0, round_dtype=torch.float16, config=config)
    ref = _gemm_ref(a, b, c, 0.5, 2.0, torch.float16)
    assert torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("mnk", ((1000, 1024, 512), (1920, 1920, 1920), (264, 776, 1000), (300, 264, 104),
                                 (520, 2056, 96), (4000, 4000, 4096)))
def test_gemm_dma_ragged(mnk, dtype):
    # The DMA kernel (forced) on ragged shapes: M anything, N and K multiples of 8; its
    # buffer resources end at the last valid row and column, the last k-tile takes 8, 16 or
    # 24 valid k (K = 1000, 104, 1000 % 32 = 8), and the epilogue stores only inside out.
    m, n, k = mnk
    a, b, c = _randn((m, k), dtype, 60), _randn((k, n), dtype, 61), _randn((m, n), dtype, 62)
    rd = torch.float16 if dtype == torch.float16 else None
    out = torch.full((m, n), 7.0, dtype=dtype, device=DEV)
    kernels.gemm(a, b, out, c=c, alpha=0.5, beta=2.0, round_dtype=rd, config=1)
    ref = _gemm_ref(a, b, c, 0.5, 2.0, rd)
    tol = 1e-2 * max(1.0, math.sqrt(k) / 8)
    assert torch.allclose(out.float(), ref.float(), atol=tol, rtol=1e-2)
    # without c, fp32 out (the element-wise epilogue of the same kernel)
    out32 = torch.empty((m, n), dtype=torch.float32, device=DEV)
    kernels.gemm(a, b, out32, config=1)
    assert torch.allclose(out32, a.float() @ b.float(), atol=tol, rtol=1e-3)


@pytest.mark.parametrize("config", (1, 4))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_gemm_dma_ragged_reads_nothing_past_the_matrix(dtype, config):
    # a and b are views of larger buffers filled with inf past K (a's columns, b's rows) and
    # past N (b's columns); out is a view whose neighbours must stay untouched.  A value
    # past K reaching the product would give inf * 0 = nan; one past N, a wrong column.
    m, n, k = 300, 264, 200
    inf = float("inf")
    abuf = torch.full((m, k + 8), inf, dtype=dtype, device=DEV)
    abuf[:, :k] = _randn((m, k), dtype, 63)
    bbuf = torch.full((k + 8, n + 8), inf, dtype=dtype, device=DEV)
    bbuf[:k, :n] = _randn((k, n), dtype, 64)
    a, b = abuf[:, :k], bbuf[:k, :n]
    obuf = torch.full((m + 1, n + 8), 7.0, dtype=dtype, device=DEV)
    out = obuf[:m, :n]
    kernels.gemm(a, b, out, config=config)
    assert torch.isfinite(out).all()
    assert torch.allclose(out.float(), a.float() @ b.float(), atol=2e-2, rtol=1e-2)
    assert torch.all(obuf[:, n:] == 7.0) and torch.all(obuf[m:] == 7.0)


@pytest.mark.parametrize("config", (1, 4))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_gemm_dma_ragged_broadcast_bias(dtype, config):
    # c broadcast along rows (row stride 0) on a ragged shape: the fast epilogue's c resource.
    m, n, k = 777, 520, 264
    a, b = _randn((m, k), dtype, 65), _randn((k, n), dtype, 66)
    c = _randn((n,), dtype, 67).expand(m, n)
    out = torch.empty((m, n), dtype=dtype, device=DEV)
    kernels.gemm(a, b, out, c=c, alpha=1.0, beta=0.5, config=config)
    ref = _gemm_ref(a, b, c, 1.0, 0.5, None)
    assert torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("bt", (False, True))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("mnk", ((2048, 2048, 2048), (1000, 1024, 512), (264, 776, 1000), (300, 264, 104),
                                 (520, 2056, 96), (128, 128, 96), (1, 8, 96)))
def test_gemm_dma128(mnk, dtype, bt):
    # The DMA kernel on 128 x 128 tiles (forced): ragged M, N and K multiples of 8 with a
    # partial last k-tile (1000, 104), b row-major or k-contiguous, with and without c; out is
    # a view whose neighbouring columns and row must stay untouched.
    m, n, k = mnk
    a = _randn((m, k), dtype, 90)
    b = _randn((n, k), dtype, 91).t() if bt else _randn((k, n), dtype, 91)
    c = _randn((m, n), dtype, 92)
    rd = torch.float16 if dtype == torch.float16 else None
    obuf = torch.full((m + 1, n + 8), 7.0, dtype=dtype, device=DEV)
    out = obuf[:m, :n]
    kernels.gemm(a, b, out, c=c, alpha=0.5, beta=2.0, round_dtype=rd, config=4)
    ref = _gemm_ref(a, b.contiguous(), c, 0.5, 2.0, rd)
    tol = 1e-2 * max(1.0, math.sqrt(k) / 8)
    assert torch.allclose(out.float(), ref.float(), atol=tol, rtol=1e-2)
    assert torch.all(obuf[:, n:] == 7.0) and torch.all(obuf[m:] == 7.0)
    out2 = torch.empty((m, n), dtype=dtype, device=DEV)
    kernels.gemm(a, b, out2, config=4)
    assert torch.allclose(out2.float(), a.float() @ b.float(), atol=tol, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("mnk", ((1, 4096, 4096), (7, 100, 72), (32, 4096, 11008), (33, 256, 8), (64, 1000, 520),
                                 (2, 32, 4104)))
def test_gemm_few_rows(mnk, dtype):
    # The few-rows kernel (forced; also the default here): M <= 64 against b^T rows, ragged N
    # and K (multiples of 8, a last 16-deep step half past K), with c, alpha and beta, and an
    # fp32 out; out a view whose neighbours must stay untouched.
    m, n, k = mnk
    a = _randn((m, k), dtype, 110, 1.0 / math.sqrt(k))
    b = _randn((n, k), dtype, 111).t()
    c = _randn((m, n), dtype, 112)
    rd = torch.float16 if dtype == torch.float16 else None
    obuf = torch.full((m + 1, n + 3), 7.0, dtype=dtype, device=DEV)
    out = obuf[:m, :n]
    kernels.gemm(a, b, out, c=c, alpha=0.5, beta=2.0, round_dtype=rd, config=5)
    ref = _gemm_ref(a, b.contiguous(), c, 0.5, 2.0, rd)
    assert torch.allclose(out.float(), ref.float(), atol=2e-2, rtol=1e-2)
    assert torch.all(obuf[:, n:] == 7.0) and torch.all(obuf[m:] == 7.0)
    out0 = torch.empty((m, n), dtype=dtype, device=DEV)
    kernels.gemm(a, b, out0, c=c, alpha=0.5, beta=2.0, round_dtype=rd)
    assert torch.equal(out0, out)
    out32 = torch.empty((m, n), dtype=torch.float32, device=DEV)
    kernels.gemm(a, b, out32, config=5)
    assert torch.allclose(out32, a.float() @ b.float(), atol=1e-3, rtol=1e-3)


def test_gemm_few_rows_rejects_unfit_calls():
    from ninetoothed_amd.errors import KernelLaunchError

    a, bt = _randn((65, 256), torch.float16, 113), _randn((128, 256), torch.float16, 114)
    out = torch.full((65, 128), 7.0, dtype=torch.float16, device=DEV)
    with pytest.raises(KernelLaunchError):  # 65 rows
        kernels.gemm(a, bt.t(), out, config=5)
    with pytest.raises(KernelLaunchError):  # b row-major
        kernels.gemm(a[:64], _randn((256, 128), torch.float16, 115), out[:64], config=5)
    assert torch.all(out == 7.0)


def test_gemm_dma128_rejects_what_its_epilogue_cannot_store():
    from ninetoothed_amd.errors import KernelLaunchError

    a, b = _randn((256, 128), torch.float16, 93), _randn((128, 256), torch.float16, 94)
    out32 = torch.full((256, 256), 7.0, dtype=torch.float32, device=DEV)
    with pytest.raises(KernelLaunchError):  # fp32 out: the element-wise epilogue only
        kernels.gemm(a, b, out32, config=4)
    assert torch.all(out32 == 7.0)
    b_odd = _randn((128, 260), torch.float16, 95)[:, :252]  # N % 8 != 0
    out = torch.full((256, 252), 7.0, dtype=torch.float16, device=DEV)
    with pytest.raises(KernelLaunchError):
        kernels.gemm(a, b_odd, out, config=4)
    assert torch.all(out == 7.0)


def test_gemm_forced_config_rejects_unfit_call():
    from ninetoothed_amd.errors import KernelLaunchError

    a, b = _randn((300, 100), torch.float16, 53), _randn((100, 200), torch.float16, 54)
    out = torch.full((300, 200), 7.0, dtype=torch.float16, device=DEV)
    # K = 100 (rows of a not 16-byte aligned) fits neither the DMA kernels nor (M, N not
    # multiples of 256) the register-staged one: rejected before launching
    for config in (1, 2, 4):
        with pytest.raises(KernelLaunchError):
            kernels.gemm(a, b, out, config=config)
    assert torch.all(out == 7.0)
    kernels.gemm(a, b, out, config=3)
    assert torch.allclose(out.float(), _gemm_ref(a, b).float(), atol=2e-2, rtol=1e-2)


def test_addmm_headline_bf16():
    m = n = k = 4096
    g = 1.0 / math.sqrt(k)
    c = _randn((m, n), torch.bfloat16, 16, g)
    a = _randn((m, k), torch.bfloat16, 17, g)
    b = _randn((k, n), torch.bfloat16, 18, g)
    out = torch.empty_like(c)
    kernels.gemm(a, b, out, c=c, alpha=1.0, beta=0.5, round_dtype=torch.float16)
    ref = _gemm_ref(a, b, c, 1.0, 0.5, torch.float16)
    assert torch.allclose(out.float(), ref.float(), atol=1e-2, rtol=1e-2)


def test_gemm_transposed_operands():
    a = _randn((384, 256), torch.float16, 19).t()  # [256, 384], m-contiguous
    b = _randn((512, 384), torch.float16, 20).t()  # [384, 512], k-contiguous
    out = torch.empty((256, 512), dtype=torch.float16, device=DEV)
    kernels.gemm(a, b, out)
    assert torch.allclose(out.float(), _gemm_ref(a, b).float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("mnk", ((4096, 4096, 4096), (1000, 1000, 1000), (300, 777, 104), (256, 256, 96),
                                 (1920, 4100, 640)))
def test_gemm_dma_b_transposed(mnk, dtype):
    # b k-contiguous (b = w.t(), the layout of x @ w.t()) on the DMA kernel (forced): b^T
    # rows go to LDS as a's; any N (777, 4100: not multiples of 8, the element-wise
    # epilogue), K multiples of 8 with a partial last k-tile (1000, 104, 640 % 32 = 0).
    m, n, k = mnk
    a = _randn((m, k), dtype, 70)
    b = _randn((n, k), dtype, 71).t()
    c = _randn((m, n), dtype, 72)
    rd = torch.float16 if dtype == torch.float16 else None
    out = torch.full((m, n), 7.0, dtype=dtype, device=DEV)
    kernels.gemm(a, b, out, c=c, alpha=1.0, beta=0.5, round_dtype=rd, config=1)
    ref = _gemm_ref(a, b.contiguous(), c, 1.0, 0.5, rd)
    tol = 1e-2 * max(1.0, math.sqrt(k) / 8)
    assert torch.allclose(out.float(), ref.float(), atol=tol, rtol=1e-2)


def test_gemm_negative_row_strides():
    """Rows walked backwards through the C ABI (a and out with negative row strides, as a
    caller may pass for a flipped view; torch itself makes none): the aligned DMA kernels
    address panels with unsigned offsets, so such a call takes the any-strides kernel and
    must still match the product of the flipped matrices."""
    import ctypes

    from ninetoothed_amd import _lib

    lib = _lib.load()
    m, n, k = 512, 512, 512
    a = _randn((m, k), torch.float16, 80, 0.1)
    b = _randn((k, n), torch.float16, 81, 0.1)
    out = torch.zeros(m, n, dtype=torch.float16, device=DEV)
    es = a.element_size()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    code = lib.nt_gemm_f16(a.data_ptr() + (m - 1) * k * es, -k, 1, b.data_ptr(), n, 1, None, 0, 0,
                           out.data_ptr() + (m - 1) * n * es, -n, 1, _lib.dtype_code(torch.float16), m, n, k, 1.0, 0.0,
                           _lib.dtype_code(torch.float16), stream)
    torch.cuda.synchronize()
    assert code == 0
    ref = (a.float() @ b.float())  # row i of the flipped a times b lands in row i of the flipped out
    assert torch.allclose(out.float(), ref, atol=1e-2, rtol=1e-2), (out.float() - ref).abs().max()


@pytest.mark.parametrize("config", (1, 4))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_gemm_dma_b_transposed_reads_nothing_past_k(dtype, config):
    # b^T rows are a view of a wider buffer holding inf past K: those values must not
    # reach the product (the last k-tile's chunks past K read zeros).  N = 300 on the 256-wide
    # kernel (any N with b^T), 296 on the 128-wide one (its epilogue stores 8 columns a lane).
    m, n, k = 264, 300 if config == 1 else 296, 200
    bt_buf = torch.full((n, k + 8), float("inf"), dtype=dtype, device=DEV)
    bt_buf[:, :k] = _randn((n, k), dtype, 73)
    a, b = _randn((m, k), dtype, 74), bt_buf[:, :k].t()
    out = torch.empty((m, n), dtype=dtype, device=DEV)
    kernels.gemm(a, b, out, config=config)
    assert torch.isfinite(out).all()
    assert torch.allclose(out.float(), a.float() @ b.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("mnk", ((1024, 1024, 1024), (2048, 2048, 256), (1000, 1028, 516), (4096, 64, 100),
                                 (700, 900, 4)))
def test_gemm_f32_mfma(mnk):
    # fp32 on the matrix core (v_mfma_f32_32x32x2_f32): 128 x 128 tiles (2048^2: 256 of
    # them) or 64 x 64, ragged M, N, K (multiples of 4), with c, alpha and beta, and a and b
    # as views of wider rows; against fp64.
    m, n, k = mnk
    a = _randn((m, k + 4), torch.float32, 23)[:, :k]
    b = _randn((k, n + 8), torch.float32, 24)[:, :n]
    c = _randn((m, n), torch.float32, 25)
    out = torch.empty((m, n), device=DEV)
    kernels.gemm(a, b, out, c=c, alpha=0.5, beta=2.0)
    ref = (0.5 * (a.double() @ b.double()) + 2.0 * c.double()).float()
    assert torch.allclose(out, ref, atol=1e-4 * max(1.0, k ** 0.5 / 8), rtol=1e-4)


@pytest.mark.parametrize("mnk", ((512, 512, 512), (100, 70, 33), (256, 128, 1000), (64, 32, 260), (64, 64, 514)))
def test_gemm_f32(mnk):
    m, n, k = mnk
    a = _randn((m, k), torch.float32, 21)
    b = _randn((k, n), torch.float32, 22)
    out = torch.empty((m, n), device=DEV)
    kernels.gemm(a, b, out)
    ref = (a.double() @ b.double()).float()
    assert torch.allclose(out, ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("plain", (False, True))
@pytest.mark.parametrize("mnk", ((512, 512, 512), (96, 64, 1024), (32, 32, 2048), (64, 128, 512)))
def test_gemm_f32_whole_tiles(mnk, plain):
    # the split-k kernel's whole-tile instances (M, N multiples of 32, K of 512, unit inner
    # strides, 16-byte aligned a rows; K exactly 512 or a loop; plain: no c, alpha 1): a and
    # b as views of wider rows, c, alpha and beta, and an output that is a slice of wider
    # rows; against fp64.
    m, n, k = mnk
    a = _randn((m, k + 4), torch.float32, 26)[:, :k]
    b = _randn((k, n + 8), torch.float32, 27)[:, :n]
    c = _randn((m, n), torch.float32, 28)
    out = torch.full((m, n + 3), 7.0, device=DEV)
    if plain:
        kernels.gemm(a, b, out[:, 1:n + 1])
        ref = (a.double() @ b.double()).float()
    else:
        kernels.gemm(a, b, out[:, 1:n + 1], c=c, alpha=0.5, beta=2.0)
        ref = (0.5 * (a.double() @ b.double()) + 2.0 * c.double()).float()
    assert torch.allclose(out[:, 1:n + 1], ref, atol=1e-4 * max(1.0, k ** 0.5 / 8), rtol=1e-4)
    assert (out[:, 0] == 7.0).all() and (out[:, n + 1:] == 7.0).all()


# ------------------------------------------------------------------------ conv2d
def _workspace(x, w, padding):
    nbytes = kernels.conv2d_workspace_bytes(x, w, padding)
    return torch.empty(nbytes, dtype=torch.uint8, device=DEV) if nbytes else None


@pytest.mark.parametrize("relayout", (False, True))
@pytest.mark.parametrize("padding", ((0, 0), (1, 1), (0, 1), (2, 0)))
def test_conv2d_reference_case(padding, relayout):
    x = _rand((4, 64, 16, 16), torch.float16, 23)
    w = _rand((512, 64, 3, 3), torch.float16, 24)
    ph, pw = padding
    p, q = 16 + 2 * ph - 2, 16 + 2 * pw - 2
    y = torch.empty((4, 512, p, q), dtype=torch.float16, device=DEV)
    ws = _workspace(x, w, padding) if relayout else None
    assert (ws is not None) == relayout
    kernels.conv2d(x, w, y, padding=padding, round_dtype=torch.float16, workspace=ws)
    ref = F.conv2d(x.float(), w.float(), padding=padding)
    assert torch.allclose(y.float(), ref, atol=1e-2 * 4, rtol=1e-2)


@pytest.mark.parametrize("relayout", (False, True))
def test_conv2d_headline(relayout):
    x = _randn((16, 256, 56, 56), torch.float16, 25)
    w = _randn((256, 256, 3, 3), torch.float16, 26, 1.0 / math.sqrt(256 * 9))
    y = torch.empty_like(x)
    kernels.conv2d(x, w, y, padding=(1, 1), round_dtype=torch.float16,
                   workspace=_workspace(x, w, (1, 1)) if relayout else None)
    ref = F.conv2d(x.float(), w.float(), padding=1)
    assert torch.allclose(y.float(), ref, atol=1e-2, rtol=1e-2)


def test_conv2d_relayout_strided_ragged_bf16():
    # C = 64 takes the re-laid path; stride 2, dilation 2, K and N*P*Q not multiples of 256.
    x = _randn((3, 64, 23, 19), torch.bfloat16, 29)
    w = _randn((72, 64, 3, 2), torch.bfloat16, 30, 0.1)
    ref = F.conv2d(x.float(), w.float(), padding=(1, 2), stride=(2, 2), dilation=(2, 1))
    y = torch.empty(ref.shape, dtype=torch.bfloat16, device=DEV)
    ws = _workspace(x, w, (1, 2))
    assert ws is not None
    kernels.conv2d(x, w, y, padding=(1, 2), stride=(2, 2), dilation=(2, 1), workspace=ws)
    assert torch.allclose(y.float(), ref, atol=3e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", (
    # (N, C, H, W), (K, R, S), padding, stride, dilation: Q % 8 == 0 and C*R*S >= 96, the
    # re-laid DMA kernel; M and K not multiples of its 256 x 256 tile, 4, 6 and 36 k-tiles
    # of 32 (the pipeline's shortest and an odd count of 64-deep ones included).
    ((3, 128, 20, 16), (200, 3, 3), (1, 1), (1, 1), (1, 1)),
    ((2, 128, 33, 31), (64, 3, 3), (2, 2), (2, 2), (2, 2)),
    ((1, 64, 9, 45), (320, 1, 2), (0, 1), (1, 3), (1, 1)),
    ((2, 64, 12, 24), (96, 3, 1), (1, 0), (1, 1), (1, 1)),
    # 1,664 padded input rows: the re-layout's workgroups take three or four rows each
    ((64, 64, 24, 24), (64, 3, 3), (1, 1), (1, 1), (1, 1)),
))
def test_conv2d_relayout_dma(case, dtype):
    (n, c, h, w_), (k, r, s), padding, stride, dilation = case
    x = _randn((n, c, h, w_), dtype, 33)
    w = _randn((k, c, r, s), dtype, 34, 1.0 / math.sqrt(c * r * s))
    ref = F.conv2d(x.float(), w.float(), padding=padding, stride=stride, dilation=dilation)
    assert ref.shape[3] % 8 == 0 and c * r * s >= 96
    y = torch.empty(ref.shape, dtype=dtype, device=DEV)
    kernels.conv2d(x, w, y, padding=padding, stride=stride, dilation=dilation, round_dtype=torch.float16,
                   workspace=_workspace(x, w, padding))
    assert torch.allclose(y.float(), ref.to(torch.float16).float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("config", (1, 2, 3, 4, 7))
def test_conv2d_paths(config):
    # Each forced path (re-laid + DMA kernel, re-laid + N-H-W-C kernel, direct kernel,
    # re-laid + DMA kernel of 224-position tiles, re-laid + DMA kernel of 128 x 128 tiles) on a
    # call all five admit.
    x = _randn((2, 64, 16, 16), torch.float16, 60)
    w = _randn((96, 64, 3, 3), torch.float16, 61, 1.0 / math.sqrt(64 * 9))
    y = torch.empty((2, 96, 16, 16), dtype=torch.float16, device=DEV)
    ws = _workspace(x, w, (1, 1)) if config != 3 else None
    kernels.conv2d(x, w, y, padding=(1, 1), round_dtype=torch.float16, workspace=ws, config=config)
    ref = F.conv2d(x.float(), w.float(), padding=1)
    assert torch.allclose(y.float(), ref.to(torch.float16).float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", (
    # (N, C, H, W), (K, R, S), padding, config: channel counts that are no multiple of 64,
    # zero-filled to 32 (DMA kernel, config 1) or 64 (N-H-W-C kernel, config 2) in the
    # workspace; W % 8 == 0 (the one-launch re-layout) and not (the slab re-layout)
    ((2, 3, 32, 32), (64, 3, 3), (1, 1), 1),
    ((2, 3, 30, 30), (16, 7, 7), (3, 3), 2),
    ((3, 24, 16, 24), (40, 3, 3), (1, 1), 1),
    ((2, 96, 14, 16), (192, 3, 3), (1, 1), 1),
    ((2, 96, 14, 14), (100, 3, 3), (1, 1), 2),
    ((1, 100, 9, 13), (72, 3, 3), (1, 1), 0),
    ((2, 32, 28, 28), (64, 1, 1), (0, 0), 2),
))
def test_conv2d_padded_channels(case, dtype):
    (n, c, h, w_), (k, r, s), padding, config = case
    x = _randn((n, c, h, w_), dtype, 35)
    w = _randn((k, c, r, s), dtype, 36, 1.0 / math.sqrt(c * r * s))
    ref = F.conv2d(x.float(), w.float(), padding=padding)
    y = torch.full(ref.shape, 7.0, dtype=dtype, device=DEV)
    ws = _workspace(x, w, padding)
    assert ws is not None
    kernels.conv2d(x, w, y, padding=padding, round_dtype=torch.float16, workspace=ws, config=config)
    assert torch.allclose(y.float(), ref.to(torch.float16).float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", (
    # (N, C, H, W), (K, R, S), padding: outputs of 2 to 50 tiles of 256 x 256, so the DMA
    # kernel splits the reduction (16 splits of 9 k-tiles; 27 k-tiles in 6 splits, the last
    # shorter; 1,280 channels) and a second kernel sums the fp32 partials
    ((2, 512, 8, 8), (512, 3, 3), (1, 1)),
    ((4, 96, 28, 16), (192, 3, 3), (1, 1)),
    ((1, 1280, 8, 8), (1280, 3, 3), (1, 1)),
    ((4, 64, 16, 16), (512, 3, 3), (1, 1)),
    ((32, 512, 7, 7), (512, 3, 3), (1, 1)),   # Q = 7: partials of M rounded up to 8, stores one by one
    ((3, 96, 14, 14), (200, 3, 3), (1, 1)),
))
@pytest.mark.parametrize("config", (1, 7))
def test_conv2d_split_reduction(case, dtype, config):
    (n, c, h, w_), (k, r, s), padding = case
    x = _randn((n, c, h, w_), dtype, 37)
    w = _randn((k, c, r, s), dtype, 38, 1.0 / math.sqrt(c * r * s))
    ref = F.conv2d(x.float(), w.float(), padding=padding)
    y = torch.full(ref.shape, 7.0, dtype=dtype, device=DEV)
    kernels.conv2d(x, w, y, padding=padding, workspace=_workspace(x, w, padding), config=config)
    assert torch.allclose(y.float(), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", (
    # (N, C, H, W), (K, R, S), padding, stride: Q no multiple of 8 on the DMA kernel without
    # a split (the element-by-element epilogue: 8 positions that run across output rows)
    ((32, 128, 28, 28), (128, 3, 3), (1, 1), (1, 1)),
    ((16, 64, 15, 17), (300, 3, 3), (1, 1), (2, 2)),
    ((8, 256, 14, 14), (256, 1, 1), (0, 0), (1, 1)),
    ((8, 64, 28, 21), (128, 1, 1), (0, 0), (1, 1)),  # C*R*S = 64: re-laid with 96 channels
    ((4, 40, 9, 11), (72, 1, 1), (0, 0), (1, 1)),
))
@pytest.mark.parametrize("config", (1, 7))
def test_conv2d_dma_any_q(case, dtype, config):
    (n, c, h, w_), (k, r, s), padding, stride = case
    x = _randn((n, c, h, w_), dtype, 39)
    w = _randn((k, c, r, s), dtype, 40, 1.0 / math.sqrt(c * r * s))
    ref = F.conv2d(x.float(), w.float(), padding=padding, stride=stride)
    assert ref.shape[3] % 8 != 0
    y = torch.full(ref.shape, 7.0, dtype=dtype, device=DEV)
    kernels.conv2d(x, w, y, padding=padding, stride=stride, workspace=_workspace(x, w, padding), config=config)
    assert torch.allclose(y.float(), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", (
    # (N, C, H, W), (K, R, S), padding, stride, dilation through the DMA kernel of 224-position
    # tiles: M = N*P*Q no multiple of 224 (the last tile's upper waves wholly past M), K no
    # multiple of 256, the shortest pipeline (3 k-tiles), Q % 8 != 0 (element-by-element
    # stores), stride and dilation
    ((3, 128, 20, 16), (200, 3, 3), (1, 1), (1, 1), (1, 1)),
    ((2, 64, 12, 24), (96, 3, 1), (1, 0), (1, 1), (1, 1)),
    ((1, 32, 9, 45), (320, 1, 3), (0, 1), (1, 1), (1, 1)),
    ((32, 128, 28, 28), (128, 3, 3), (1, 1), (1, 1), (1, 1)),
    ((16, 64, 15, 17), (300, 3, 3), (1, 1), (2, 2), (1, 1)),
    ((2, 128, 33, 31), (64, 3, 3), (2, 2), (2, 2), (2, 2)),
))
def test_conv2d_dma224(case, dtype):
    (n, c, h, w_), (k, r, s), padding, stride, dilation = case
    x = _randn((n, c, h, w_), dtype, 41)
    w = _randn((k, c, r, s), dtype, 42, 1.0 / math.sqrt(c * r * s))
    ref = F.conv2d(x.float(), w.float(), padding=padding, stride=stride, dilation=dilation)
    y = torch.full(ref.shape, 7.0, dtype=dtype, device=DEV)
    kernels.conv2d(x, w, y, padding=padding, stride=stride, dilation=dilation, workspace=_workspace(x, w, padding),
                   config=4)
    assert torch.allclose(y.float(), ref, atol=2e-2, rtol=1e-2)


def test_conv2d_headline_takes_224_tiles():
    # [16,256,56,56] * [256,256,3,3]: 196 tiles of 256 positions or 224 of 224, one round of
    # 256 CUs either way; the default path takes the 224-position strip kernel (input read
    # in place) and agrees bit for bit with the 224- and 256-position kernels over the
    # re-laid input (same k order, same fp32 sums).
    x = _randn((16, 256, 56, 56), torch.float16, 43)
    w = _randn((256, 256, 3, 3), torch.float16, 44, 1.0 / math.sqrt(256 * 9))
    ws = _workspace(x, w, (1, 1))
    y0, y1, y4, y5 = (torch.empty_like(x) for _ in range(4))
    kernels.conv2d(x, w, y0, padding=(1, 1), workspace=ws)
    kernels.conv2d(x, w, y1, padding=(1, 1), workspace=ws, config=1)
    kernels.conv2d(x, w, y4, padding=(1, 1), workspace=ws, config=4)
    kernels.conv2d(x, w, y5, padding=(1, 1), workspace=ws, config=5)
    assert torch.equal(y0, y5) and torch.equal(y1, y4) and torch.equal(y4, y5)
    ref = F.conv2d(x.float(), w.float(), padding=1)
    assert torch.allclose(y5.float(), ref, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", (
    # (N, C, H, W), K, padding, input channel offset in a wider tensor, filter layout: the
    # strip kernel (config 5, 3 x 3 filters) against torch and, bit for bit, the re-laid
    # 224-position kernel (config 4).  Q = 56 / 16 / 32 (4, 14 and 7 output rows per tile),
    # two and three raw pieces per strip, one channel block, K no multiple of 256, no row
    # padding and two rows of it, an input that is a channel slice of a wider tensor (image
    # stride past C * H * W), a filter whose rows are not contiguous (re-laid by gathers), and
    # 75 32-channel filter blocks (the contiguous re-layout's last workgroup takes three of four),
    # and a contiguous filter starting 2 bytes past a 16-byte boundary (re-laid by gathers).
    ((3, 96, 56, 56), 64, (1, 1), 0, "dense"),
    ((2, 64, 14, 16), 96, (1, 1), 0, "dense"),
    ((1, 32, 14, 32), 200, (1, 1), 0, "dense"),
    ((2, 64, 58, 56), 32, (0, 1), 0, "dense"),
    ((1, 64, 54, 56), 40, (2, 1), 0, "dense"),
    ((2, 64, 56, 56), 300, (1, 1), 32, "dense"),
    ((2, 64, 56, 56), 96, (1, 1), 0, "krsc"),
    ((2, 32, 28, 56), 75, (1, 1), 0, "dense"),
    ((2, 64, 28, 56), 48, (1, 1), 0, "offset"),
))
def test_conv2d_strip224(case, dtype):
    (n, c, h, w_), k, padding, c_off, layout = case
    big = _randn((n, c + 2 * c_off, h, w_), dtype, 45)
    x = big[:, c_off:c_off + c]
    if layout == "dense":
        w = _randn((k, c, 3, 3), dtype, 46, 1.0 / math.sqrt(c * 9))
    elif layout == "offset":
        w = _randn((k * c * 9 + 1,), dtype, 46, 1.0 / math.sqrt(c * 9))[1:].view(k, c, 3, 3)
        assert w.is_contiguous() and w.data_ptr() % 16 == 2
    else:
        w = _randn((k, 3, 3, c), dtype, 46, 1.0 / math.sqrt(c * 9)).permute(0, 3, 1, 2)
    ref = F.conv2d(x.float(), w.float(), padding=padding)
    ws = _workspace(x, w, padding)
    y5 = torch.full(ref.shape, 7.0, dtype=dtype, device=DEV)
    y4 = torch.full(ref.shape, 7.0, dtype=dtype, device=DEV)
    kernels.conv2d(x, w, y5, padding=padding, workspace=ws, config=5)
    kernels.conv2d(x, w, y4, padding=padding, workspace=ws, config=4)
    assert torch.allclose(y5.float(), ref, atol=2e-2, rtol=1e-2)
    assert torch.equal(y5, y4)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", (
    # (N, C, H, W), K: 1 x 1 filters as a batch of products on the 128 x 128-tile GEMM kernel
    # (config 6): ResNet's bottleneck shapes, one image, a K no multiple of 8 (ragged M of the
    # products), C = 96 (three 32-deep k-tiles), H W = 8 (one 128-wide tile, mostly past N).
    ((4, 256, 56, 56), 64), ((4, 128, 56, 56), 256), ((8, 512, 28, 28), 128), ((1, 128, 16, 24), 200),
    ((3, 96, 4, 2), 37), ((2, 1024, 28, 28), 256),
    # H W no multiple of 8: the images through the workspace with rows padded to 8
    ((4, 1024, 14, 14), 256), ((8, 2048, 7, 7), 512), ((2, 96, 3, 5), 40), ((1, 256, 1, 1), 24),
))
def test_conv2d_1x1_as_batched_gemm(case, dtype):
    (n, c, h, w_), k = case
    x = _randn((n, c, h, w_), dtype, 96)
    w = _randn((k, c, 1, 1), dtype, 97, 1.0 / math.sqrt(c))
    ref = F.conv2d(x.float(), w.float())
    ybuf = torch.full((n, k + 1, h, w_), 7.0, dtype=dtype, device=DEV)
    y6 = ybuf[:, :k]  # image stride past K * H * W; the extra channel must stay untouched
    ws = _workspace(x, w, (0, 0)) if (h * w_) % 8 else None
    kernels.conv2d(x, w, y6, workspace=ws, config=6)
    y0 = torch.empty(ref.shape, dtype=dtype, device=DEV)
    kernels.conv2d(x, w, y0, workspace=ws)  # the default takes the same path
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-2
    assert torch.allclose(y6.float(), ref, atol=tol, rtol=tol)
    assert torch.equal(y0, y6)
    assert torch.all(ybuf[:, k:] == 7.0)


def test_conv2d_1x1_path_declines_what_it_cannot_take():
    from ninetoothed_amd.errors import KernelLaunchError

    def forced(xshape, wshape, padding=(0, 0), x=None):
        x = _randn(xshape, torch.float16, 98) if x is None else x
        w = _randn(wshape, torch.float16, 99, 0.05)
        ref = F.conv2d(x.float(), w.float(), padding=padding)
        y = torch.full(ref.shape, 7.0, dtype=torch.float16, device=DEV)
        with pytest.raises(KernelLaunchError):
            kernels.conv2d(x, w, y, padding=padding, config=6)
        assert torch.all(y == 7.0)
        kernels.conv2d(x, w, y, padding=padding, workspace=_workspace(x, w, padding))  # the default runs elsewhere
        assert torch.allclose(y.float(), ref, atol=2e-2, rtol=1e-2)

    forced((2, 128, 14, 14), (64, 128, 1, 1))               # H W = 196, no multiple of 8, and no workspace
    forced((2, 64, 16, 16), (64, 64, 1, 1))                 # C = 64 < 96
    forced((2, 128, 16, 16), (64, 128, 3, 3), (1, 1))       # a 3 x 3 filter
    forced((2, 128, 16, 16), (64, 128, 1, 1), (1, 1))       # padding
    forced(None, (64, 128, 1, 1), x=_randn((2, 128, 16, 16), torch.float16, 100).transpose(2, 3))  # w stride 16


def test_conv2d_strip224_reads_each_calls_filter():
    # Calls that reuse one workspace (which holds the re-laid filter) with a new filter each
    # time, back to back on one stream, must each see their own filter.
    x = _randn((16, 256, 56, 56), torch.float16, 50)
    ws = _workspace(x, torch.empty((256, 256, 3, 3), dtype=torch.float16, device=DEV), (1, 1))
    filters = [_randn((256, 256, 3, 3), torch.float16, 51 + i, 1.0 / math.sqrt(256 * 9)) for i in range(3)]
    ys = [torch.empty_like(x) for _ in filters]
    for w, y in zip(filters, ys):
        kernels.conv2d(x, w, y, padding=(1, 1), workspace=ws, config=5)
    for w, y in zip(filters, ys):
        y4 = torch.empty_like(x)
        kernels.conv2d(x, w, y4, padding=(1, 1), workspace=ws, config=4)
        assert torch.equal(y, y4)


def test_conv2d_strip224_rejects_unfit_calls():
    from ninetoothed_amd.errors import KernelLaunchError

    def call(xshape, wshape, padding=(1, 1), stride=(1, 1), x=None):
        x = _randn(xshape, torch.float16, 47) if x is None else x
        w = _randn((wshape[0], x.shape[1], *wshape[1:]), torch.float16, 48, 0.05)
        ref_shape = F.conv2d(x[:1, :, :, :].float().cpu(), w.float().cpu(), padding=padding, stride=stride).shape
        y = torch.full((x.shape[0], *ref_shape[1:]), 7.0, dtype=torch.float16, device=DEV)
        with pytest.raises(KernelLaunchError):
            kernels.conv2d(x, w, y, padding=padding, stride=stride, workspace=_workspace(x, w, padding), config=5)
        assert torch.all(y == 7.0)

    call((2, 64, 16, 16), (32, 3, 3))               # Q = 16, 14 rows per tile do not divide P = 16
    call((2, 48, 56, 56), (32, 3, 3))               # C % 32 != 0
    call((2, 64, 58, 58), (32, 3, 3), (0, 0))       # Q = 56, but W = 58 is no multiple of 8
    call((2, 64, 112, 112), (32, 3, 3), stride=(2, 2))  # stride 2
    call((1, 64, 56, 56), (32, 5, 5), (2, 2))       # a 5 x 5 filter
    call((1, 64, 56, 56), (32, 1, 1), (0, 0))       # a 1 x 1 filter
    xt = _randn((2, 64, 56, 56), torch.float16, 49).transpose(2, 3)  # w stride 56
    call(None, (32, 3, 3), x=xt)


@pytest.mark.parametrize("flip", ("w", "h"))
@pytest.mark.parametrize("config", (0, 1, 3, 4, 7))
@pytest.mark.parametrize("xshape", ((4, 64, 15, 13), (17, 64, 45, 45)))
def test_conv2d_flipped_output(flip, config, xshape):
    """An output flipped along w (q stride -1) or h (p stride -Q) through the C ABI, with
    Q % 8 != 0 so the DMA kernel stores element by element (the small shape splits the
    reduction, the large one does not): positions at negative offsets from the data
    pointer are valid outputs and must be written, on every path."""
    import ctypes

    from ninetoothed_amd import _lib

    lib = _lib.load()
    x = _randn(xshape, torch.float16, 64)
    w = _randn((128, 64, 3, 3), torch.float16, 65, 1.0 / math.sqrt(64 * 9))
    ref = F.conv2d(x.float(), w.float(), padding=1)
    n, k, p, q = ref.shape
    assert q % 8 != 0
    ybuf = torch.full(ref.shape, float("nan"), dtype=torch.float16, device=DEV)
    es = ybuf.element_size()
    if flip == "w":
        ptr, ys = ybuf.data_ptr() + (q - 1) * es, (k * p * q, p * q, q, -1)
    else:
        ptr, ys = ybuf.data_ptr() + (p - 1) * q * es, (k * p * q, p * q, -q, 1)
    nbytes = kernels.conv2d_workspace_bytes(x, w, (1, 1))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    code16 = _lib.dtype_code(torch.float16)
    args = (x.data_ptr(), _lib.int64_array(x.stride()), w.data_ptr(), _lib.int64_array(w.stride()), ptr,
            _lib.int64_array(ys), code16, *xshape, k, 3, 3, p, q, 1, 1, 1, 1, 1, 1, code16,
            ws.data_ptr() if config != 3 else None, nbytes if config != 3 else 0)
    if config:
        code = lib.nt_conv2d_config_f16(*args, config, stream)
    else:
        code = lib.nt_conv2d_f16(*args, stream)
    torch.cuda.synchronize()
    assert code == 0
    got = ybuf.flip(3) if flip == "w" else ybuf.flip(2)
    assert not torch.isnan(got).any()
    assert torch.allclose(got.float(), ref, atol=2e-2, rtol=1e-2)


def test_conv2d_empty_filter():
    """A filter with no taps (R or S zero) sums nothing: every output is zero, with or
    without a workspace (through the C ABI: torch refuses the shape, and an empty tensor has
    no data pointer).  The kernel choice must not divide by R * S."""
    import ctypes

    from ninetoothed_amd import _lib

    lib = _lib.load()
    x = _randn((2, 8, 6, 6), torch.float16, 60)
    w = torch.zeros(64, dtype=torch.float16, device=DEV)  # never read: the filter has no taps
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    code16 = _lib.dtype_code(torch.float16)
    for r, s_ in ((0, 3), (3, 0)):
        p, q = 6 + 2 - r + 1, 6 + 2 - s_ + 1
        y = torch.full((2, 4, p, q), float("nan"), dtype=torch.float16, device=DEV)
        for workspace, nbytes in ((None, 0), (ws.data_ptr(), ws.numel())):
            y.fill_(float("nan"))
            code = lib.nt_conv2d_f16(x.data_ptr(), _lib.int64_array(x.stride()), w.data_ptr(),
                                     _lib.int64_array((8 * r * s_, r * s_, s_, 1)), y.data_ptr(),
                                     _lib.int64_array(y.stride()), code16, 2, 8, 6, 6, 4, r, s_, p, q, 1, 1, 1, 1, 1, 1,
                                     code16, workspace, nbytes, stream)
            torch.cuda.synchronize()
            assert code == 0, (r, s_, workspace)
            assert (y == 0).all(), (r, s_, workspace)


def test_conv2d_forced_path_rejects_unfit_call():
    from ninetoothed_amd.errors import KernelLaunchError

    x = _randn((2, 24, 16, 16), torch.float16, 62)  # no workspace: no re-laid path
    w = _randn((40, 24, 3, 3), torch.float16, 63, 0.1)
    y = torch.full((2, 40, 14, 14), 7.0, dtype=torch.float16, device=DEV)
    for config in (1, 2, 4, 5):
        with pytest.raises(KernelLaunchError):
            kernels.conv2d(x, w, y, config=config)
    assert torch.all(y == 7.0)


def test_conv2d_strided_dilated_bf16():
    x = _randn((2, 24, 21, 19), torch.bfloat16, 27)
    w = _randn((40, 24, 3, 5), torch.bfloat16, 28, 0.1)
    ref = F.conv2d(x.float(), w.float(), padding=(2, 1), stride=(2, 3), dilation=(2, 1))
    y = torch.empty(ref.shape, dtype=torch.bfloat16, device=DEV)
    kernels.conv2d(x, w, y, padding=(2, 1), stride=(2, 3), dilation=(2, 1))
    assert torch.allclose(y.float(), ref, atol=3e-2, rtol=1e-2)


# --------------------------------------------------------------------- attention
def _sdpa_ref(q, k, v, causal, scale):
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=causal, scale=scale)


@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("seq", (1024, 1))
@pytest.mark.parametrize("dtype, tol", ((torch.float16, 1e-2), (torch.float32, 0.025)))
def test_attention_reference_case(seq, causal, dtype, tol):
    q, k, v = (_randn((2, 4, seq, 64), dtype, 30 + i) for i in range(3))
    o = torch.empty_like(q)
    # The reference test's dtypes.  fp16 follows the reference kernel's weak scalar
    # typing: the constant 1.44269504089 is rounded to fp16 before the multiply.
    c = float(torch.tensor(kernels.LOG2E, dtype=dtype)) if dtype == torch.float16 else kernels.LOG2E
    kernels.attention(q, k, v, o, causal=causal, q_scale=c)
    assert torch.allclose(o.float(), _sdpa_ref(q, k, v, causal, 1.0), atol=tol, rtol=tol)


@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_attention_d128_scaled(causal, dtype):
    q, k, v = (_randn((2, 3, 777, 128), dtype, 40 + i) for i in range(3))
    o = torch.empty_like(q)
    scale = 1.0 / math.sqrt(128)
    kernels.attention(q, k, v, o, causal=causal, q_scale=kernels.LOG2E * scale)
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    assert torch.allclose(o.float(), _sdpa_ref(q, k, v, causal, scale), atol=tol, rtol=tol)


def _attention_ref64(q, k, v, causal, q_scale):
    # The kernel's arithmetic in float64: q * q_scale rounded to the input type,
    # s = q . k in base 2, softmax by exp2, p rounded to the input type before p . v.
    qr = (q.float() * q_scale).to(q.dtype).double()
    s = qr @ k.double().transpose(-1, -2)
    if causal:
        sq, sk = s.shape[-2:]
        s = s.masked_fill(torch.ones(sq, sk, dtype=torch.bool, device=s.device).triu(1), -math.inf)
    p = torch.exp2(s - s.amax(-1, keepdim=True))
    l = p.sum(-1, keepdim=True)
    return (p.to(q.dtype).double() @ v.double()) / l


@pytest.mark.parametrize("d", (64, 128))
@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("sq, sk", ((700, 700), (300, 700), (129, 65)))
def test_attention_growing_scores(d, causal, sq, sk):
    # Scores rise along the keys by ~20 (log2 units) per 64-key tile and spread widely
    # within a tile, so the running max is raised on nearly every tile and exp2(s - m)
    # spans the whole range; ragged Sq, Sk exercise the key-range and causal masks.
    dtype = torch.float16
    u = _randn((d,), torch.float32, 60) / math.sqrt(d)
    q = (_randn((1, 2, sq, d), torch.float32, 61) + 2.0 * u).to(dtype)
    ramp = torch.arange(sk, device=DEV, dtype=torch.float32)[:, None] * (0.11 / math.sqrt(d)) * u * d
    k = (_randn((1, 2, sk, d), torch.float32, 62) + ramp).to(dtype)
    v = _randn((1, 2, sk, d), dtype, 63)
    o = torch.empty_like(q)
    qs = kernels.LOG2E / math.sqrt(d)
    kernels.attention(q, k, v, o, causal=causal, q_scale=qs)
    ref = _attention_ref64(q, k, v, causal, qs)
    assert torch.allclose(o.double(), ref, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("d", (8, 40, 80, 96, 112))
@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_attention_padded_head_dims(d, causal, dtype):
    # Head dims below 64 or 128 (multiples of 8) on the eight-wave kernel (forced), padded
    # with zeros: k, v and o as views of wider rows whose columns past d hold inf (k, v)
    # and a sentinel (o), so a value past d reaching the scores, or a store past d, shows.
    sq, sk = 300, 333
    pad = torch.full((1, 3, sk, d + 8), float("inf"), dtype=dtype, device=DEV)
    k, v = pad.clone(), pad.clone()
    k[..., :d] = _randn((1, 3, sk, d), dtype, 64)
    v[..., :d] = _randn((1, 3, sk, d), dtype, 65)
    k, v = k[..., :d], v[..., :d]
    q = _randn((1, 3, sq, d), dtype, 66)
    obuf = torch.full((1, 3, sq, d + 8), 7.0, dtype=dtype, device=DEV)
    o = obuf[..., :d]
    scale = 1.0 / math.sqrt(d)
    kernels.attention(q, k, v, o, causal=causal, q_scale=kernels.LOG2E * scale, config=2)
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=causal, scale=scale)
    assert torch.allclose(o.float(), ref, atol=2e-2, rtol=2e-2)
    assert torch.all(obuf[..., d:] == 7.0)


def test_attention_negative_row_strides():
    """Keys, values and queries walked backwards through the C ABI (negative row strides, as
    a caller may pass for a flipped view; torch itself makes none).  The fast kernels address
    a head's keys with unsigned buffer offsets, so such a call takes the four-wave kernels and
    must match attention over the flipped tensors."""
    import ctypes

    from ninetoothed_amd import _lib

    lib = _lib.load()
    b_, h_, s_, d_ = 1, 2, 256, 64
    q, k, v = (_randn((b_, h_, s_, d_), torch.float16, 90 + i) for i in range(3))
    o = torch.zeros_like(q)
    es = q.element_size()

    def flipped(t):  # pointer to row s-1 of head 0, row stride -D
        st = t.stride()
        return t.data_ptr() + (s_ - 1) * st[2] * es, _lib.int64_array((st[0], st[1], -st[2], st[3]))

    (qp, qs_), (kp, ks_), (vp, vs_), (op, os_) = (flipped(t) for t in (q, k, v, o))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    code = lib.nt_attention_f16(qp, qs_, kp, ks_, vp, vs_, op, os_, _lib.dtype_code(torch.float16), b_, h_, s_, s_,
                                d_, 1.4426950408889634 / d_ ** 0.5, 0, stream)
    torch.cuda.synchronize()
    assert code == 0
    # every row reversed in q, k, v and o: the softmax over keys is order-free, so o = attn(q, k, v)
    ref = F.scaled_dot_product_attention(q.float().cpu(), k.float().cpu(), v.float().cpu())
    assert torch.allclose(o.float().cpu(), ref, atol=1e-2, rtol=1e-2), (o.float().cpu() - ref).abs().max()


@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
def test_attention_empty_keys(dtype):
    """No keys: every output is zero, as F.scaled_dot_product_attention gives (the empty key
    tensors have no data pointer; the launcher needs none)."""
    q = _randn((2, 3, 5, 64), dtype, 70)
    k = torch.empty(2, 3, 0, 64, dtype=dtype, device=DEV)
    for causal in (False, True):
        o = torch.full_like(q, float("nan"))
        kernels.attention(q, k, k, o, causal)
        assert torch.equal(o, torch.zeros_like(q)), causal
        assert torch.equal(o.float().cpu(), F.scaled_dot_product_attention(q.float().cpu(), k.float().cpu(),
                                                                           k.float().cpu()))


@pytest.mark.parametrize("d", (24, 64, 100, 128))
@pytest.mark.parametrize("causal", (False, True))
def test_attention_f32(d, causal):
    # fp32 on the VALU kernel: one lane per query up to 64 dims, two above; ragged Sq, Sk;
    # k and v also as transposed copies (d stride != 1: element-wise tile loads); fp32 math,
    # so within 1e-4 of fp64.
    sq, sk = 130, 300
    q, k, v = (_randn((2, 3, s_, d), torch.float32, 80 + i) for i, s_ in enumerate((sq, sk, sk)))
    scale = 1.0 / math.sqrt(d)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), is_causal=causal, scale=scale)
    for kk, vv in ((k, v), (k.transpose(2, 3).contiguous().transpose(2, 3), v.transpose(2, 3).contiguous().transpose(2, 3))):
        o = torch.empty_like(q)
        kernels.attention(q, kk, vv, o, causal=causal, q_scale=kernels.LOG2E * scale)
        assert torch.allclose(o.double(), ref, atol=1e-4, rtol=1e-4), (d, causal)


def test_attention_headline_causal():
    q, k, v = (_randn((4, 32, 4096, 128), torch.float16, 50 + i) for i in range(3))
    o = torch.empty_like(q)
    scale = 1.0 / math.sqrt(128)
    kernels.attention(q, k, v, o, causal=True, q_scale=kernels.LOG2E * scale)
    # Every head against fp32 SDPA, one head at a time (64 MiB of scores each; all at once
    # would need 8 GiB).
    bad = []
    for b in range(4):
        for h in range(32):
            ref = _sdpa_ref(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1], True, scale)
            if not torch.allclose(o[b:b + 1, h:h + 1].float(), ref, atol=1e-2, rtol=1e-2):
                bad.append((b, h))
    assert not bad, f"heads outside tolerance: {bad[:8]}"


# Every kernel configuration of the 16-bit attention (config 1: one-wave-per-SIMD pipelined
# kernel, D = 128; 2: eight-wave kernel; 3: four-wave kernels) on ragged and causal shapes,
# with scores that rise along the keys (the lazy rescale fires on nearly every tile) and on
# random data, against the float64 restatement of the kernels' arithmetic.
@pytest.mark.parametrize("config", (1, 2, 3))
@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("sq, sk", ((700, 700), (300, 700), (129, 65), (64, 32), (257, 1000)))
def test_attention_configs(config, causal, sq, sk):
    d, dtype = 128, torch.float16
    u = _randn((d,), torch.float32, 80) / math.sqrt(d)
    q = (_randn((1, 3, sq, d), torch.float32, 81) + 2.0 * u).to(dtype)
    ramp = torch.arange(sk, device=DEV, dtype=torch.float32)[:, None] * (0.11 / math.sqrt(d)) * u * d
    k = (_randn((1, 3, sk, d), torch.float32, 82) + ramp).to(dtype)
    v = _randn((1, 3, sk, d), dtype, 83)
    qs = kernels.LOG2E / math.sqrt(d)
    for qq, kk in ((q, k), (_randn((1, 3, sq, d), dtype, 84), _randn((1, 3, sk, d), dtype, 85))):
        o = torch.empty_like(qq)
        kernels.attention(qq, kk, v, o, causal=causal, q_scale=qs, config=config)
        ref = _attention_ref64(qq, kk, v, causal, qs)
        assert torch.allclose(o.double(), ref, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("causal", (False, True))
def test_attention_pipe_bf16_against_eight_wave(causal):
    q, k, v = (_randn((2, 5, 613, 128), torch.bfloat16, 90 + i) for i in range(3))
    o1, o2 = torch.empty_like(q), torch.empty_like(q)
    scale = 1.0 / math.sqrt(128)
    kernels.attention(q, k, v, o1, causal=causal, q_scale=kernels.LOG2E * scale, config=1)
    kernels.attention(q, k, v, o2, causal=causal, q_scale=kernels.LOG2E * scale, config=2)
    ref = _sdpa_ref(q, k, v, causal, scale)
    assert torch.allclose(o1.float(), ref, atol=2e-2, rtol=2e-2)
    assert torch.allclose(o1.float(), o2.float(), atol=2e-2, rtol=2e-2)


def test_attention_config_conditions_are_checked():
    from ninetoothed_amd.errors import KernelLaunchError

    q, k, v = (_randn((1, 2, 100, 64), torch.float16, 95 + i) for i in range(3))
    o = torch.empty_like(q)
    with pytest.raises(KernelLaunchError):  # the pipelined kernel takes head dim 128 only
        kernels.attention(q, k, v, o, q_scale=kernels.LOG2E, config=1)
    qt = q.transpose(2, 3).contiguous().transpose(2, 3)  # d-stride != 1: four-wave kernels only
    with pytest.raises(KernelLaunchError):
        kernels.attention(qt, k, v, o, q_scale=kernels.LOG2E, config=2)
    kernels.attention(qt, k, v, o, q_scale=kernels.LOG2E, config=3)
    assert torch.allclose(o.float(), _sdpa_ref(q, k, v, False, 1.0), atol=1e-2, rtol=1e-2)


# Softmax kernel configurations (1, 2, 3: register path with four, eight, one wave per
# workgroup; 4: two-sweep kernel; 5: a group of lanes per segment) on whole rows, segments,
# an unaligned view and the headline width; a configuration whose kernel cannot hold the
# segment is refused.
@pytest.mark.parametrize("config", (1, 2, 3, 4, 5))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
@pytest.mark.parametrize("cols, block", ((8192, None), (1000, None), (33, None), (1000, 128), (5000, 777)))
def test_softmax_configs(config, dtype, cols, block):
    from ninetoothed_amd.errors import KernelLaunchError

    x = _randn((24, cols), dtype, 11, scale=2.0)
    blk = cols if block is None else block
    nseg = -(-cols // blk)
    xp = F.pad(x.float(), (0, nseg * blk - cols), value=float("-inf")).view(24, nseg, blk)
    ref = torch.softmax(xp, dim=-1).view(24, nseg * blk)[:, :cols]
    tol = TOL[dtype]
    for view in (x, _randn((24, cols + 1), dtype, 12, scale=2.0)[:, 1:]):  # aligned, then off by one element
        if view is not x:
            xp = F.pad(view.float(), (0, nseg * blk - cols), value=float("-inf")).view(24, nseg, blk)
            ref = torch.softmax(xp, dim=-1).view(24, nseg * blk)[:, :cols]
        y = torch.empty(24, cols, dtype=dtype, device=DEV)
        lanes = {1: 256, 2: 512, 3: 64, 5: 64}.get(config)
        vpt_max = 16 if view is x and (cols * x.element_size()) % 16 == 0 and (blk * x.element_size()) % 16 == 0 else 8
        if config == 5:
            vpt_max = 4
        if lanes is not None and min(blk, cols) > lanes * (16 // x.element_size()) * vpt_max:
            with pytest.raises(KernelLaunchError):
                kernels.softmax(view, y, block=block, config=config)
            continue
        kernels.softmax(view, y, block=block, config=config)
        assert torch.allclose(y.float(), ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
@pytest.mark.parametrize("rows, cols, block", ((3000, 128, None), (777, 24, None), (9, 300000, None),
                                               (700, 6000, 2000), (2, 1 << 20, None), (600, 40000, None)))
def test_softmax_shapes(rows, cols, block, dtype):
    # The library's own choice: lane groups for short segments (16 lanes per 128 fp16
    # columns, 4 segments of 24 per 16 lanes...), the register path, and the two-sweep
    # kernel with 1024 lanes (few segments) or 256 (many); also one column off alignment.
    x = _randn((rows, cols + 1), dtype, 14, scale=2.0)
    for view in (x[:, :cols], x[:, 1:]):
        blk = cols if block is None else block
        nseg = -(-cols // blk)
        xp = F.pad(view.float(), (0, nseg * blk - cols), value=float("-inf")).view(rows, nseg, blk)
        ref = torch.softmax(xp, dim=-1).view(rows, nseg * blk)[:, :cols]
        y = torch.empty(rows, cols, dtype=dtype, device=DEV)
        kernels.softmax(view, y, block=block)
        assert torch.allclose(y.float(), ref, atol=TOL[dtype], rtol=TOL[dtype]), (rows, cols)


def test_softmax_infinite_rows():
    # -inf entries: a row of -inf but one value, -inf prefixes across whole vectors, in the
    # lane-group kernel (128 columns) and the two-sweep kernel (300000 columns).
    for cols in (128, 300000):
        x = torch.randn(4, cols, device=DEV).half()
        x[0, :] = float("-inf")
        x[0, cols - 3] = 1.0
        x[1, : cols // 2] = float("-inf")
        y = torch.empty_like(x)
        kernels.softmax(x, y)
        assert torch.allclose(y.float(), torch.softmax(x.float(), -1), atol=1e-3, rtol=1e-2), cols


@pytest.mark.parametrize("config", (1, 2, 3, 4))
def test_max_pool2d_configs(config):
    from ninetoothed_amd.errors import KernelLaunchError

    x = _rand((4, 16, 112, 112), torch.float16, 13, -1.0, 1.0)
    y = torch.empty((4, 16, 56, 56), dtype=torch.float16, device=DEV)
    kernels.max_pool2d(x, y, (2, 2), config=config)
    assert torch.equal(y, F.max_pool2d(x, (2, 2)))
    # 2-high windows with Q a multiple of 4 but not of 8 (the pair-row kernel's, not the
    # flat kernel's), an input one column wider than the windows reach, a strided batch,
    # bf16, and a unit count that is no multiple of the grid's
    x3 = _rand((3, 7, 26, 48), torch.bfloat16, 15, -4.0, 4.0)[:, :, :, :41]
    ref3 = F.max_pool2d(x3, (2, 2))
    y3 = torch.empty_like(ref3)
    if config == 3:
        with pytest.raises(KernelLaunchError):
            kernels.max_pool2d(x3, y3, (2, 2), config=3)
    else:
        kernels.max_pool2d(x3, y3, (2, 2), config=config)
        assert torch.equal(y3, ref3)
    x2 = _randn((2, 5, 17, 19), torch.float16, 14)
    ref = F.max_pool2d(x2, (3, 2), stride=(2, 3), padding=(1, 1))
    y2 = torch.empty_like(ref)
    if config in (1, 3):  # the vector kernels take 2-wide windows of stride 2 only
        with pytest.raises(KernelLaunchError):
            kernels.max_pool2d(x2, y2, (3, 2), stride=(2, 3), padding=(1, 1), config=config)
    else:
        kernels.max_pool2d(x2, y2, (3, 2), stride=(2, 3), padding=(1, 1), config=config)
        assert torch.equal(y2, ref)


def test_max_pool2d_empty_input_plane():
    """A zero-width (or zero-height) input whose padding still gives outputs: every window
    lies in the padding, so every output is -inf (through the C ABI: torch refuses the shape,
    and an empty tensor has no data pointer).  The kernel choice must not divide by the
    empty row's size."""
    import ctypes

    from ninetoothed_amd import _lib

    lib = _lib.load()
    x = torch.zeros(64, dtype=torch.float16, device=DEV)  # never read: every window is padding
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for h, w, kh, kw, ph, pw, p, q in ((4, 0, 2, 2, 1, 1, 5, 1), (0, 6, 2, 2, 1, 1, 1, 7)):
        y = torch.zeros(2, 3, p, q, dtype=torch.float16, device=DEV)
        for config in (0, 2):
            code = lib.nt_max_pool2d_config_f16(x.data_ptr(), _lib.int64_array((3 * h * w, h * w, w, 1)), y.data_ptr(),
                                                _lib.int64_array(y.stride()), 2, 3, h, w, p, q, kh, kw, 1, 1, ph, pw,
                                                1, 1, stream, config)
            torch.cuda.synchronize()
            assert code == 0, (h, w, config)
            assert torch.isneginf(y).all(), (h, w, config)
            y.zero_()
        code = lib.nt_max_pool2d_config_f16(x.data_ptr(), _lib.int64_array((3 * h * w, h * w, w, 1)), y.data_ptr(),
                                            _lib.int64_array(y.stride()), 2, 3, h, w, p, q, kh, kw, 1, 1, ph, pw, 1, 1,
                                            stream, 4)
        assert code != 0, (h, w)  # the LDS kernel does not take an empty plane


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_max_pool2d_overlapping_windows(dtype):
    """Overlapping and padded windows (the LDS strip kernel) against F.max_pool2d, bit-exact:
    the ResNet stem pool (3x3, stride 2, padding 1) on rows of whole 16-byte vectors, an odd
    width (element-wise staging), ceil mode, dilation, a strided input, planes split into
    several strips, and a window too tall for the LDS (the element-wise kernel)."""
    cases = [
        ((4, 64, 112, 112), (3, 3), (2, 2), (1, 1), (1, 1), False),
        ((3, 5, 55, 55), (3, 3), (2, 2), (0, 0), (1, 1), True),
        ((2, 7, 33, 40), (3, 3), (1, 1), (1, 1), (1, 1), False),
        ((2, 3, 29, 24), (5, 3), (2, 1), (2, 1), (2, 3), True),
        ((1, 2, 300, 2048), (3, 3), (2, 2), (1, 1), (1, 1), False),
        ((1, 2, 40, 4096), (7, 2), (1, 2), (3, 0), (1, 1), False),
    ]
    for i, (shape, k, st, pad, dil, ceil) in enumerate(cases):
        x = _randn(shape, dtype, 40 + i)
        ref = F.max_pool2d(x, k, st, pad, dil, ceil_mode=ceil)
        y = torch.empty_like(ref)
        kernels.max_pool2d(x, y, k, st, pad, dil)
        assert torch.equal(y, ref), (shape, k, st, pad, dil, ceil)
        y.fill_(0)
        kernels.max_pool2d(x, y, k, st, pad, dil, config=2)
        assert torch.equal(y, ref), (shape, k, st, pad, dil, ceil)
    # many small planes: several whole planes per workgroup, a partial last group, ranges
    # starting at every 16-byte phase; and the same input into an output that is not
    # plane-contiguous (one plane per workgroup)
    x = _randn((3, 1111, 9, 14), dtype, 48)  # ceil mode adds an output column
    for ceil in (False, True):
        ref = F.max_pool2d(x, 3, 2, 1, ceil_mode=ceil)
        y = torch.empty_like(ref)
        kernels.max_pool2d(x, y, (3, 3), (2, 2), (1, 1))
        assert torch.equal(y, ref), ceil
        yt = torch.empty(ref.shape[2], ref.shape[3], 3, 1111, dtype=dtype, device=DEV).permute(2, 3, 0, 1)
        kernels.max_pool2d(x, yt, (3, 3), (2, 2), (1, 1))
        assert torch.equal(yt, ref), ceil
    base = _randn((3, 8, 60, 64), dtype, 50)
    for xs in (base[:, ::2, 1:, :], base[:, ::2, 1:, 2:]):  # strided channels, row and column offsets
        ref = F.max_pool2d(xs, 3, 2, 1)
        for config in (0, 4):
            y = torch.empty_like(ref)
            kernels.max_pool2d(xs, y, (3, 3), (2, 2), (1, 1), config=config)
            assert torch.equal(y, ref), (xs.shape, config)
