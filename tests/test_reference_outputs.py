"""Against the reference's own kernels' outputs.

tests/golden/reference_outputs.npz holds small seeded inputs and what the reference's generated
kernels computed from them on Triton's CPU interpreter (written by
tests/golden/make_reference_outputs.py; the reference's own programs from its test modules,
the README's fp32 matmul, one configuration each).  CPU: the oracle reproduces them bit for
bit for matmul (fp32 and fp16), addmm, conv2d, add and dropout (Philox stream, p = 0.3, a
seed of 1234567), and attention to 2 ulp (exp2 and the accumulation order).  GPU: the MI355X
kernels, through the Handle: fp16 matmul and conv2d to 1 ulp, addmm to 1 ulp of the rounded
product plus 1 of the output, attention to 2 ulps of max(|o|, 1) with at least 90 % bit for
bit, fp32 matmul to 1e-5, add and dropout bit for bit.  (The interpreter cannot run the
reference's softmax and max_pool2d kernels; those are pinned by torch closed forms, max_pool2d
bit for bit.)
"""

import functools
from pathlib import Path

import numpy as np
import pytest

import programs as pg
from oracle import apply, philox

_Z = np.load(Path(__file__).parent / "golden" / "reference_outputs.npz")
DROPOUT_P, DROPOUT_SEED = 0.3, 1234567  # the fixture script's call


def _arr(key):
    a = _Z[key]
    return a.view(np.float16) if str(_Z[key + "__dtype"]) == "float16" else a


def _f32(key):
    return _arr(key).astype(np.float32)


def _ulps(got, ref):
    """|got - ref| in units of fp16 spacing at ref."""
    ref16 = np.asarray(ref, dtype=np.float16)
    spacing = np.spacing(np.abs(ref16)).astype(np.float32)
    return np.abs(np.asarray(got, dtype=np.float32) - ref16.astype(np.float32)) / spacing


def _oracle(name):
    if name == "matmul_fp32":
        return apply.matmul(_f32("matmul_fp32_a"), _f32("matmul_fp32_b"), "float32", pg.matmul_arrangement,
                            block=(32, 32, 32), round_dtype=None)
    if name == "matmul_fp16":
        return apply.matmul(_f32("matmul_fp16_a"), _f32("matmul_fp16_b"), "float16", pg.matmul_arrangement,
                            block=(32, 32, 32))
    if name == "addmm":
        return apply.addmm(_f32("addmm_input"), _f32("addmm_mat1"), _f32("addmm_mat2"), 0.5, 1.0, "float16",
                           pg.addmm_arrangement, block=(32, 32, 32))
    if name == "conv2d":
        return apply.conv2d(_f32("conv2d_x"), _f32("conv2d_w"), (1, 1),
                            functools.partial(pg.conv2d_arrangement, enable_padding=True), block=(32, 32, 32))
    if name == "add":
        return apply.add(_f32("add_lhs"), _f32("add_rhs"), 64)
    if name == "dropout":
        # reference tests/test_dropout.py:16-17: fp16 / fp32 scalar computes in fp32, rounded
        # to fp16 at the store
        x = _f32("dropout_x")
        keep = philox.rand(DROPOUT_SEED, np.arange(x.size)) > np.float32(DROPOUT_P)
        return np.where(keep, x / (np.float32(1) - np.float32(DROPOUT_P)), np.float32(0)).astype(np.float16)
    causal = name.endswith("1")
    return apply.attention(_f32("attention_q"), _f32("attention_k"), _f32("attention_v"), causal,
                           pg.attention_arrangement, block=(32, 32))


_EXACT = ("matmul_fp32", "matmul_fp16", "addmm", "conv2d", "add", "dropout")
_OUT = {"matmul_fp32": "matmul_fp32_out", "matmul_fp16": "matmul_fp16_out", "addmm": "addmm_out",
        "conv2d": "conv2d_out", "add": "add_out", "dropout": "dropout_out", "attention_causal0": "attention_out_causal0",
        "attention_causal1": "attention_out_causal1"}


@pytest.mark.parametrize("name", _EXACT)
def test_oracle_reproduces_the_reference_kernels(name):
    assert np.array_equal(np.asarray(_oracle(name), dtype=np.float32), _f32(_OUT[name]))


@pytest.mark.parametrize("causal", (0, 1))
def test_oracle_attention_within_two_ulp_of_the_reference_kernel(causal):
    got, ref = _oracle(f"attention_causal{causal}"), _f32(f"attention_out_causal{causal}")
    u = _ulps(got, ref)
    assert u.max() <= 2.0 and (u == 0).mean() > 0.99


# ------------------------------------------------------------------ GPU
def _cuda(key):
    import torch

    return torch.from_numpy(_arr(key).copy()).cuda()


@pytest.mark.gpu
def test_kernels_match_the_reference_kernels():
    import torch

    import ninetoothed_amd as ninetoothed

    # fp32 matmul (the README program)
    a, b = _cuda("matmul_fp32_a"), _cuda("matmul_fp32_b")
    c = torch.empty(a.shape[0], b.shape[1], device="cuda")
    ninetoothed.make(pg.matmul_arrangement, pg.matmul_application_fp32, pg.matmul_tensors())(a, b, c)
    np.testing.assert_allclose(c.cpu().numpy(), _f32("matmul_fp32_out"), rtol=1e-5, atol=1e-5)
    # fp16 matmul and addmm: fp32 accumulation in another order, rounded once
    a, b = _cuda("matmul_fp16_a"), _cuda("matmul_fp16_b")
    c = torch.empty(a.shape[0], b.shape[1], dtype=torch.float16, device="cuda")
    ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())(a, b, c)
    assert _ulps(c.float().cpu().numpy(), _f32("matmul_fp16_out")).max() <= 1.0
    # addmm rounds A.B to fp16 before beta * C + alpha * (A.B): one ulp of A.B there (then one
    # of the output's own rounding) is what another accumulation order can change
    inp, m1, m2 = _cuda("addmm_input"), _cuda("addmm_mat1"), _cuda("addmm_mat2")
    c = torch.empty_like(inp)
    ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())(inp, m1, m2, 0.5, 1.0, c)
    ab = np.abs(_f32("addmm_mat1") @ _f32("addmm_mat2")).astype(np.float16)
    bound = np.spacing(ab).astype(np.float32) + np.spacing(np.abs(_arr("addmm_out"))).astype(np.float32)
    diff = np.abs(c.float().cpu().numpy() - _f32("addmm_out"))
    assert (diff <= bound).all(), float((diff / bound).max())
    # conv2d, padding 1
    x, w = _cuda("conv2d_x"), _cuda("conv2d_w")
    y = torch.empty(x.shape[0], w.shape[0], x.shape[2], x.shape[3], dtype=torch.float16, device="cuda")
    pg.make_conv2d()(x, w, y, padding_h=1, padding_w=1)
    assert _ulps(y.float().cpu().numpy(), _f32("conv2d_out")).max() <= 1.0
    # attention, both masks: the kernel rounds p against a running max that may trail the
    # true one (same relative precision), so the bar is 2 fp16 ulps of max(|o|, 1) (o is an
    # average of rows of v), with at least 90 % of the outputs bit for bit
    q, k, v = _cuda("attention_q"), _cuda("attention_k"), _cuda("attention_v")
    kernel = ninetoothed.make(pg.attention_arrangement, pg.attention_application, pg.attention_tensors())
    for causal in (0, 1):
        o = torch.empty_like(q)
        kernel(q, k, v, bool(causal), o)
        got, ref = o.float().cpu().numpy(), _f32(f"attention_out_causal{causal}")
        scale = np.maximum(np.abs(ref), 1.0).astype(np.float16)
        assert (np.abs(got - ref) <= 2 * np.spacing(scale).astype(np.float32)).all(), causal
        assert (got == ref).mean() >= 0.9, causal
    # add, bit for bit
    lhs, rhs = _cuda("add_lhs"), _cuda("add_rhs")
    out = torch.empty_like(lhs)
    pg.make_add()(lhs, rhs, out)
    assert np.array_equal(out.cpu().numpy(), _f32("add_out"))
    # dropout, bit for bit: the same Philox stream, the same fp32 quotient and rounding
    x = _cuda("dropout_x")
    y = torch.empty_like(x)
    pg.make_dropout()(x, DROPOUT_P, DROPOUT_SEED, y)
    assert np.array_equal(y.cpu().numpy().view(np.int16), _Z["dropout_out"])
