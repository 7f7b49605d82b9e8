"""Seeded random sizes, block shapes and dtypes through the generic kernels (programs outside the
hand-written families), against torch with the reference's rounding after every operation.

Three programs: a 2-D element-wise chain over a row-major operand, a permuted one (stored
[N, M]) and a column-major one; a row reduction with one tile per row; a 1-D select with
run-time scalars.  The block shapes are powers of two that rarely divide the sizes, so the
masked edges of the index tables are exercised.  The case id is the seed.
"""

import math
import random

import pytest
import torch

import ninetoothed_amd as ninetoothed
import ninetoothed_amd.language as ntl
from ninetoothed_amd import Symbol, Tensor

pytestmark = pytest.mark.gpu

DEV = "cuda"
CASES = range(12)
BM = Symbol("BM", meta=True)
BN = Symbol("BN", meta=True)
BS = Symbol("BS", meta=True)
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-6}


def _gen(seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def chain_arrangement(a, b, c, o):
    return a.tile((BM, BN)), b.permute((1, 0)).tile((BM, BN)), c.tile((BM, BN)), o.tile((BM, BN))


def chain_application(a, b, c, o):
    o = ntl.maximum(a * b + c, a - c)  # noqa: F841


def rowsum_arrangement(x, o):
    return x.tile((1, BN)), o.tile((1,))


def rowsum_application(x, o):
    o = ntl.sum(x * x, axis=1)  # noqa: F841


def select_arrangement(x, s, t, o):
    return x.tile((BS,)), s, t, o.tile((BS,))


def select_application(x, s, t, o):
    o = ntl.where(x > t, x * s, -x)  # noqa: F841


_CHAIN = ninetoothed.make(chain_arrangement, chain_application, (Tensor(2), Tensor(2), Tensor(2), Tensor(2)))
_ROWSUM = ninetoothed.make(rowsum_arrangement, rowsum_application, (Tensor(2, other=0), Tensor(1)))
_SELECT = ninetoothed.make(select_arrangement, select_application, (Tensor(1), Tensor(0), Tensor(0), Tensor(1)))


@pytest.mark.parametrize("seed", CASES)
def test_chain_random(seed):
    rng, g = random.Random(9000 + seed), _gen(9000 + seed)
    m, n = rng.randint(1, 300), rng.randint(1, 300)
    bm, bn = 1 << rng.randint(0, 6), 1 << rng.randint(0, 6)
    dtype = rng.choice((torch.float16, torch.bfloat16, torch.float32))
    a = torch.randn((m, n), generator=g).to(dtype).to(DEV)
    b_store = torch.randn((n, m), generator=g).to(dtype).to(DEV)
    c = torch.randn((n, m), generator=g).to(dtype).to(DEV).t()  # column-major [M, N]
    o = torch.full((m, n), float("nan"), dtype=dtype, device=DEV)
    _CHAIN(a, b_store, c, o, BM=bm, BN=bn)
    ref = torch.maximum(a * b_store.t() + c, a - c)  # torch rounds each operation to the dtype, as the kernel
    assert torch.allclose(o, ref, atol=TOL[dtype], rtol=TOL[dtype]), (m, n, bm, bn, dtype)


@pytest.mark.parametrize("seed", CASES)
def test_rowsum_random(seed):
    rng, g = random.Random(9100 + seed), _gen(9100 + seed)
    rows, cols = rng.randint(1, 200), rng.randint(1, 1500)
    bn = 1 << (cols - 1).bit_length()
    dtype = rng.choice((torch.float16, torch.float32))
    x = (torch.randn((rows, cols), generator=g) / math.sqrt(cols)).to(dtype).to(DEV)
    o = torch.full((rows,), float("nan"), dtype=dtype, device=DEV)
    _ROWSUM(x, o, BN=bn)
    ref = (x * x).float().sum(1)  # squares rounded to the dtype, summed in fp32
    assert torch.allclose(o.float(), ref, atol=4 * TOL[dtype], rtol=4 * TOL[dtype]), (rows, cols, dtype)


@pytest.mark.parametrize("seed", CASES)
def test_select_random(seed):
    rng, g = random.Random(9200 + seed), _gen(9200 + seed)
    n = rng.choice((rng.randint(1, 5000), rng.randint(1, 300000)))
    bs = 1 << rng.randint(4, 10)
    dtype = rng.choice((torch.float16, torch.bfloat16, torch.float32))
    s, t = round(rng.uniform(-3, 3), 3), round(rng.uniform(-1, 1), 3)
    x = torch.randn((n,), generator=g).to(dtype).to(DEV)
    o = torch.full((n,), float("nan"), dtype=dtype, device=DEV)
    _SELECT(x, s, t, o, BS=bs)
    # the comparison and the product in fp32 (a Python float is a weakly typed fp32 scalar),
    # the product rounded to the dtype
    xf = x.float()
    ref = torch.where(xf > t, (xf * s).to(dtype).float(), -xf).to(dtype)
    assert torch.allclose(o.float(), ref.float(), atol=TOL[dtype], rtol=TOL[dtype]), (n, bs, s, t, dtype)
