"""Seeded random shapes, layouts and dtypes through the drop-in ``make``/``jit`` Handles, against
torch in float32 (max_pool2d bit for bit).

The fixed cases elsewhere pin the reference's own tests and each kernel's edge conditions; this
sweep draws sizes that are no multiple of anything (and some that are), transposed operand
layouts, strided views and mixed output types, so that a path a fixed case never reaches is
still checked.  Every draw is seeded (the case id is the seed), so a failure names a case that
can be run again alone.  ``NT_SWEEP_CASES`` sets the number of draws per family (16).
"""

import functools
import math
import os
import random

import pytest
import torch
import torch.nn.functional as F

import ninetoothed_amd as ninetoothed
import programs as pg

pytestmark = pytest.mark.gpu

DEV = "cuda"
CASES = range(int(os.environ.get("NT_SWEEP_CASES", "16")))


@pytest.fixture(autouse=True)
def _no_tf32():
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def _gen(seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _randn(shape, dtype, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(DEV)


def _layout(t, rng):
    """The same values as ``t`` (2-D), stored row-major, column-major or as every other
    column of a wider row-major tensor."""
    u = rng.random()
    if u < 0.4:
        return t
    if u < 0.8:
        return t.t().contiguous().t()
    wide = torch.empty((t.shape[0], 2 * t.shape[1]), dtype=t.dtype, device=t.device)
    wide[:, ::2] = t
    return wide[:, ::2]


def _size(rng, hi):
    """A size in [1, hi]: half the draws a multiple of 8."""
    if rng.random() < 0.5:
        return 8 * rng.randint(1, max(1, hi // 8))
    return rng.randint(1, hi)


@functools.lru_cache(maxsize=None)
def _handle(name):
    if name == "matmul":
        return ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    if name == "matmul_fp32":
        return ninetoothed.make(pg.matmul_arrangement, pg.matmul_application_fp32, pg.matmul_tensors())
    if name == "addmm":
        return ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    if name == "conv2d":
        return pg.make_conv2d()
    if name == "attention":
        return ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors())
    if name == "softmax":
        return pg.make_softmax()
    raise KeyError(name)


@functools.lru_cache(maxsize=None)
def _pool_handle(ceil_mode):
    return ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=ceil_mode),
                            pg.max_pool2d_application, pg.max_pool2d_tensors())


@pytest.mark.parametrize("seed", CASES)
def test_matmul_random(seed):
    rng, g = random.Random(1000 + seed), _gen(1000 + seed)
    m, n, k = _size(rng, 700), _size(rng, 700), _size(rng, 700)
    dtype = rng.choice((torch.float16, torch.bfloat16, torch.float32))
    a = _layout(_randn((m, k), dtype, g, 1 / math.sqrt(k)), rng)
    b = _layout(_randn((k, n), dtype, g), rng)
    ref = a.float() @ b.float()
    if dtype == torch.float32:
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device=DEV)
        _handle("matmul_fp32")(a, b, out)
        assert torch.allclose(out, ref, atol=1e-4, rtol=1e-4), (m, n, k, a.stride(), b.stride())
    else:
        out = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
        _handle("matmul")(a, b, out)
        # the application rounds the fp32 accumulator to fp16
        assert torch.allclose(out.float(), ref.half().float(), atol=1e-2, rtol=1e-2), (m, n, k, dtype, a.stride(),
                                                                                      b.stride())


@pytest.mark.parametrize("seed", CASES)
def test_addmm_random(seed):
    rng, g = random.Random(2000 + seed), _gen(2000 + seed)
    m, n, k = _size(rng, 600), _size(rng, 600), _size(rng, 600)
    dtype = rng.choice((torch.float16, torch.bfloat16))
    beta, alpha = round(rng.uniform(-2, 2), 3), round(rng.uniform(-2, 2), 3)
    c = _layout(_randn((m, n), dtype, g), rng)
    a = _layout(_randn((m, k), dtype, g, 1 / math.sqrt(k)), rng)
    b = _layout(_randn((k, n), dtype, g), rng)
    out = torch.full((m, n), float("nan"), dtype=dtype, device=DEV)
    _handle("addmm")(c, a, b, beta, alpha, out)
    # beta * c + alpha * (a @ b rounded to fp16), in fp32, stored in the output's type
    ref = (beta * c.float() + alpha * (a.float() @ b.float()).half().float()).to(dtype).float()
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-2
    assert torch.allclose(out.float(), ref, atol=3 * tol, rtol=tol), (m, n, k, dtype, beta, alpha)


@pytest.mark.parametrize("seed", CASES)
def test_conv2d_random(seed):
    rng, g = random.Random(3000 + seed), _gen(3000 + seed)
    r, s = rng.randint(1, 5), rng.randint(1, 5)
    ph, pw = rng.randint(0, 2), rng.randint(0, 2)
    n, c, k = rng.randint(1, 3), rng.choice((rng.randint(1, 70), 32 * rng.randint(1, 3))), rng.randint(1, 90)
    h, w = rng.randint(max(1, r - 2 * ph), 40), rng.randint(max(1, s - 2 * pw), 40)
    dtype = rng.choice((torch.float16, torch.bfloat16))
    x = _randn((n, c, h, w), dtype, g)
    wt = _randn((k, c, r, s), dtype, g, 1 / math.sqrt(c * r * s))
    ref = F.conv2d(x.float(), wt.float(), padding=(ph, pw))
    y = torch.full(ref.shape, float("nan"), dtype=torch.float16, device=DEV)
    _handle("conv2d")(x, wt, y, padding_h=ph, padding_w=pw)
    assert torch.allclose(y.float(), ref.half().float(), atol=2e-2, rtol=1e-2), (x.shape, wt.shape, ph, pw, dtype)


@pytest.mark.parametrize("seed", CASES)
def test_attention_random(seed):
    rng, g = random.Random(4000 + seed), _gen(4000 + seed)
    bsz, heads = rng.randint(1, 2), rng.randint(1, 3)
    sq = rng.choice((rng.randint(1, 300), 64 * rng.randint(1, 4)))
    causal = rng.random() < 0.5
    sk = rng.choice((sq, rng.randint(1, 300)))
    d = rng.choice((16, 32, 40, 64, 80, 96, 112, 128))
    dtype = rng.choice((torch.float16, torch.bfloat16, torch.float32))
    q, k, v = (_randn((bsz, heads, s_, d), dtype, g) for s_ in (sq, sk, sk))
    o = torch.full_like(q, float("nan"))
    _handle("attention")(q, k, v, causal, o)
    # the application's constant is log2(e) / sqrt(128) whatever the head dim; reference on the
    # CPU in float32
    qc, kc, vc = (t.float().cpu() for t in (q, k, v))
    mask = torch.ones(sq, sk, dtype=torch.bool).tril() if causal else None
    ref = F.scaled_dot_product_attention(qc, kc, vc, attn_mask=mask, scale=1 / math.sqrt(128))
    tol = {torch.float16: 1e-2, torch.bfloat16: 2e-2, torch.float32: 1e-3}[dtype]
    assert torch.allclose(o.float().cpu(), ref, atol=tol, rtol=tol), (q.shape, sk, causal, dtype)


@pytest.mark.parametrize("seed", CASES)
def test_softmax_random(seed):
    rng, g = random.Random(5000 + seed), _gen(5000 + seed)
    rows, cols = rng.randint(1, 300), rng.choice((rng.randint(1, 3000), 8 * rng.randint(1, 300)))
    dtype = rng.choice((torch.float16, torch.bfloat16, torch.float32))
    out_dtype = rng.choice((dtype, torch.float32))
    view = rng.choice(("plain", "transposed", "every_other_column"))
    if view == "plain":
        x = _randn((rows, cols), dtype, g, 2.0)
    elif view == "transposed":
        x = _randn((cols, rows), dtype, g, 2.0).t()
    else:
        x = _randn((rows, 2 * cols), dtype, g, 2.0)[:, ::2]
    y = torch.full((rows, cols), float("nan"), dtype=out_dtype, device=DEV)
    block = 1 << (cols - 1).bit_length()
    _handle("softmax")(x, y, BLOCK_SIZE=block)
    ref = torch.softmax(x.float(), -1)
    tol = {torch.float16: 1e-3, torch.bfloat16: 8e-3, torch.float32: 1e-5}[out_dtype]
    assert torch.allclose(y.float(), ref, atol=tol, rtol=1e-2), (rows, cols, dtype, out_dtype, view)


@pytest.mark.parametrize("seed", CASES)
def test_max_pool2d_random(seed):
    rng, g = random.Random(6000 + seed), _gen(6000 + seed)
    wh, ww = rng.randint(1, 5), rng.randint(1, 5)
    n, c = rng.randint(1, 3), rng.randint(1, 8)
    h, w = rng.randint(wh, 60), rng.randint(ww, 60)
    ceil_mode = rng.random() < 0.5
    dtype = rng.choice((torch.float16, torch.bfloat16, torch.float32))
    x = _randn((n, c, h, w), dtype, g)
    ref = F.max_pool2d(x, (wh, ww), ceil_mode=ceil_mode)
    y = torch.full(ref.shape, float("nan"), dtype=dtype, device=DEV)
    _pool_handle(ceil_mode)(x, y, WINDOW_HEIGHT=wh, WINDOW_WIDTH=ww)
    assert torch.equal(y, ref), (x.shape, wh, ww, ceil_mode, dtype)


@pytest.mark.parametrize("seed", range(6))
def test_matmul_random_large(seed):
    # sizes the 256 x 256 DMA kernels take (and ragged ones around them)
    rng, g = random.Random(7000 + seed), _gen(7000 + seed)
    m = rng.choice((256 * rng.randint(1, 10), rng.randint(300, 2600)))
    n = 8 * rng.randint(32, 320)
    k = 8 * rng.randint(8, 320)
    dtype = rng.choice((torch.float16, torch.bfloat16))
    a = _randn((m, k), dtype, g, 1 / math.sqrt(k))
    b = _layout(_randn((k, n), dtype, g), rng)
    out = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
    _handle("matmul")(a, b, out)
    ref = (a.float() @ b.float()).half().float()
    assert torch.allclose(out.float(), ref, atol=1e-2, rtol=1e-2), (m, n, k, dtype, b.stride())


@pytest.mark.parametrize("seed", range(6))
def test_conv2d_random_large(seed):
    # 3 x 3 and 1 x 1 filters over 32-channel multiples at ResNet-like sizes: the strip and
    # re-laid DMA kernels
    rng, g = random.Random(8000 + seed), _gen(8000 + seed)
    r = rng.choice((1, 3))
    pad = (r - 1) // 2
    n, c, k = rng.randint(1, 4), 32 * rng.randint(1, 8), rng.choice((8 * rng.randint(1, 40), rng.randint(1, 300)))
    hw = rng.choice((7, 14, 28, 56, rng.randint(8, 60)))
    dtype = rng.choice((torch.float16, torch.bfloat16))
    x = _randn((n, c, hw, hw), dtype, g)
    wt = _randn((k, c, r, r), dtype, g, 1 / math.sqrt(c * r * r))
    ref = F.conv2d(x.float(), wt.float(), padding=pad)
    y = torch.full(ref.shape, float("nan"), dtype=torch.float16, device=DEV)
    _handle("conv2d")(x, wt, y, padding_h=pad, padding_w=pad)
    assert torch.allclose(y.float(), ref.half().float(), atol=2e-2, rtol=1e-2), (x.shape, wt.shape, dtype)
