"""Pin the oracle's tile-by-tile applications to closed forms, invariants and brute force.

Closed forms are torch CPU float64 (matmul, conv2d, softmax, max_pool2d,
scaled_dot_product_attention) computed from the same rounded inputs; a plausible
slip in the oracle (a transposed operand, a dropped padding row, a wrong causal
direction, a missing rescale by alpha, the divisor l) fails one of them.
"""

import functools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import programs as pg
from oracle import apply


def _rng(seed):
    return np.random.default_rng(seed)


def _f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("mnk,block", (((33, 20, 17), (16, 8, 4)), ((64, 48, 40), (16, 16, 16))))
def test_matmul_closed_form(mnk, block):
    m, n, k = mnk
    r = _rng(1)
    a, b = _f16(r.standard_normal((m, k))), _f16(r.standard_normal((k, n)))
    got = apply.matmul(a, b, "float16", pg.matmul_arrangement, block=block)
    ref = _f16(torch.from_numpy(a).double() @ torch.from_numpy(b).double())
    assert np.allclose(got, ref, atol=1e-2, rtol=1e-3)


def test_matmul_fp32_closed_form():
    r = _rng(2)
    a, b = r.standard_normal((40, 24)).astype(np.float32), r.standard_normal((24, 36)).astype(np.float32)
    got = apply.matmul(a, b, "float32", pg.matmul_arrangement, block=(16, 16, 8), round_dtype=None)
    assert np.allclose(got, a.astype(np.float64) @ b.astype(np.float64), atol=1e-4, rtol=1e-4)


def test_addmm_closed_form():
    r = _rng(3)
    c, a, b = (_f16(r.standard_normal(s)) for s in ((24, 20), (24, 30), (30, 20)))
    got = apply.addmm(c, a, b, 0.3, 0.7, "float16", pg.addmm_arrangement, block=(8, 8, 8))
    ref = torch.addmm(torch.from_numpy(c).double(), torch.from_numpy(a).double(), torch.from_numpy(b).double(),
                      beta=0.3, alpha=0.7).numpy()
    assert np.allclose(got, ref, atol=2e-2)


@pytest.mark.parametrize("padding", ((0, 0), (1, 1), (0, 1), (2, 0)))
def test_conv2d_closed_form(padding):
    r = _rng(4)
    x = _f16(r.random((2, 5, 7, 6)))
    w = _f16(r.random((6, 5, 3, 3)))
    arrangement = functools.partial(pg.conv2d_arrangement, enable_padding=True)
    got = apply.conv2d(x, w, padding, arrangement, block=(16, 8, 8))
    ref = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(), padding=padding).numpy()
    assert np.allclose(got, ref, atol=2e-2, rtol=2e-3)


def test_conv2d_delta_filter_is_identity():
    # A 3x3 filter with a single centre tap on channel c -> k is a channel copy (padding 1).
    r = _rng(5)
    x = _f16(r.random((1, 2, 5, 5)))
    w = np.zeros((2, 2, 3, 3), dtype=np.float32)
    w[0, 1, 1, 1] = 1.0
    w[1, 0, 1, 1] = 1.0
    arrangement = functools.partial(pg.conv2d_arrangement, enable_padding=True)
    got = apply.conv2d(x, w, (1, 1), arrangement, block=(8, 8, 8))
    assert np.array_equal(got[0, 0], x[0, 1]) and np.array_equal(got[0, 1], x[0, 0])


def _sdpa(q, k, v, causal, scale):
    t = [torch.from_numpy(a).double() for a in (q, k, v)]
    return F.scaled_dot_product_attention(*t, is_causal=causal, scale=scale).numpy()


@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("seq", (19, 1))
def test_attention_closed_form(seq, causal):
    r = _rng(6)
    q, k, v = (_f16(r.standard_normal((1, 2, seq, 8))) for _ in range(3))
    got = apply.attention(q, k, v, causal, pg.attention_arrangement, block=(8, 4))
    # The reference constant 1.44269504089 becomes the fp16 1.4423828125: scores are
    # scaled by c16 / log2(e) in the natural-exp softmax.
    c16 = float(np.float16(1.44269504089))
    ref = _sdpa(q, k, v, causal, c16 / math.log2(math.e))
    assert np.allclose(got, ref, atol=1e-2, rtol=1e-2)


def test_attention_invariants():
    r = _rng(7)
    q, k = (_f16(r.standard_normal((1, 1, 6, 4))) for _ in range(2))
    v = _f16(r.standard_normal((1, 1, 6, 4)))
    out = apply.attention(q, k, v, True, pg.attention_arrangement, block=(4, 2))
    assert np.allclose(out[0, 0, 0], v[0, 0, 0], atol=1e-3)  # causal row 0 sees only key 0
    same_keys = np.repeat(k[:, :, :1], 6, axis=2)
    out2 = apply.attention(q, same_keys, v, False, pg.attention_arrangement, block=(4, 2))
    assert np.allclose(out2[0, 0], np.broadcast_to(v[0, 0].mean(0), (6, 4)), atol=2e-3)  # equal keys -> mean(v)


@pytest.mark.parametrize("block", (781, 128))
def test_softmax_closed_form(block):
    r = _rng(8)
    x = r.random((9, 781)).astype(np.float32)
    got = apply.softmax(x, block)
    xp = np.pad(x, ((0, 0), (0, -(-781 // block) * block - 781)), constant_values=-np.inf)
    ref = torch.softmax(torch.from_numpy(xp).double().view(9, -1, block), -1).view(9, -1)[:, :781].numpy()
    assert np.allclose(got, ref, atol=1e-7, rtol=1e-5)
    if block == 781:
        assert np.allclose(got.sum(1), 1.0, atol=1e-5)


def test_softmax_fp16_input_fp32_output():
    # fp16 arithmetic up to the quotient, the quotient stored as fp32 (not rounded to fp16):
    # within fp16 precision of the float64 softmax, and not on the fp16 grid
    r = _rng(18)
    x = _f16(r.standard_normal((5, 300)) * 2)
    got = apply.softmax(x, 300, "float16", out_dtype="float32")
    ref = torch.softmax(torch.from_numpy(x).double(), -1).numpy()
    assert np.allclose(got, ref, atol=2e-4, rtol=4e-3)
    assert not np.array_equal(got, got.astype(np.float16).astype(np.float32))
    assert np.array_equal(apply.softmax(x, 300, "float16"), got.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("ceil_mode", (False, True))
def test_max_pool2d_closed_form(ceil_mode):
    r = _rng(9)
    x = _f16(r.standard_normal((2, 3, 10, 11)))
    arrangement = functools.partial(pg.max_pool2d_arrangement, ceil_mode=ceil_mode)
    got = apply.max_pool2d(x, (3, 3), ceil_mode, arrangement, block=8)
    ref = F.max_pool2d(torch.from_numpy(x), (3, 3), ceil_mode=ceil_mode).numpy()
    assert np.array_equal(got, ref)


def test_add_closed_form():
    r = _rng(10)
    a, b = r.random(1000).astype(np.float32), r.random(1000).astype(np.float32)
    assert np.array_equal(apply.add(a, b, 256), a + b)


# ------------------------------------------------------------------ ntl.rand / randint / randn
def test_philox_known_answers():
    # Random123's published known-answer vectors for philox4x32-10 (counter, key -> output)
    from oracle import philox

    kats = (
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    )
    for counter, key, expected in kats:
        assert tuple(int(x) for x in philox.philox4x32(counter, key)) == expected


def test_uniform_mapping_range_and_extremes():
    from oracle import philox

    words = np.array([0, 1, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF], dtype=np.uint32)
    u = philox.uniform(words)
    # int32 0 -> 0; 2^31 - 1 and its mirror -2^31 -> the largest value, still below 1
    assert u[0] == 0.0 and u[4] == 0.0 and u[2] == u[3] and 0.999 < u[2] < 1.0
    r = philox.rand(1234, np.arange(1 << 16))
    assert r.min() >= 0.0 and r.max() < 1.0 and abs(r.mean() - 0.5) < 0.01
    n = philox.randn(1234, np.arange(1 << 16))
    assert abs(n.mean()) < 0.02 and abs(n.std() - 1.0) < 0.02


def test_random_streams_match_tritons_generator():
    # The reference's ntl.rand/randint/randn forward to Triton (reference
    # src/ninetoothed/language.py:1-26); tests/golden/triton_random.json holds Triton 3.6.0's
    # own outputs (CPU interpreter) for six seeds (two above 2^32) and 32 offsets up to
    # 2^31 - 1: the oracle's seed/offset -> key/counter mapping and Box-Muller follow it.
    import json
    from pathlib import Path

    from oracle import philox

    fixture = json.loads((Path(__file__).parent / "golden" / "triton_random.json").read_text())
    for case in fixture["cases"]:
        off = np.asarray(case["offsets"], dtype=np.int64)
        got = philox.randint(case["seed"], off).astype(np.uint32).view(np.int32)
        assert got.tolist() == case["randint"], case["seed"]
        assert np.array_equal(philox.rand(case["seed"], off), np.asarray(case["rand"], dtype=np.float32))
        np.testing.assert_allclose(philox.randn(case["seed"], off), np.asarray(case["randn"], dtype=np.float32),
                                   rtol=1e-6, atol=1e-6)


def test_random_streams_are_distributed_and_independent():
    # What the mathematics fixes for the parts the known answers leave open (the seed and
    # offset -> key and counter mapping, Box-Muller): uniform and normal marginals
    # (Kolmogorov-Smirnov on 2^18 draws: a Box-Muller fed one word twice, or a uniform
    # map that drops the sign fold, fails), no correlation between neighbouring offsets or
    # between seeds that differ only in their high word (a mapping that ignored it, or put
    # the offset in the key, fails).
    from scipy import stats

    from oracle import philox

    off = np.arange(1 << 18)
    r = philox.rand(99, off).astype(np.float64)
    n = philox.randn(99, off).astype(np.float64)
    assert stats.kstest(r, "uniform").statistic < 0.005
    assert stats.kstest(n, "norm").statistic < 0.005
    assert abs(np.corrcoef(r[:-1], r[1:])[0, 1]) < 0.01
    hi = philox.rand(99 + (1 << 32), off).astype(np.float64)
    assert abs(np.corrcoef(r, hi)[0, 1]) < 0.01 and not np.array_equal(r, hi)
    # the pair (u1, u2) behind randn is not one word twice: normals of neighbouring offsets
    # are uncorrelated too, and their squares average 1
    assert abs(np.corrcoef(n[:-1], n[1:])[0, 1]) < 0.01 and abs((n * n).mean() - 1.0) < 0.01
