"""Every plan a family matcher hands out must launch: the binder may not reject it.

The matchers decide from the arrangement and the application; the binders in
``ninetoothed_amd.kernels`` then check dtypes, strides and sizes against what the
kernels take.  A call a matcher accepts but its binder rejects would raise where the
reference runs (its kernels take strides as arguments and its stores cast to the
output's type), so ``families.select`` asks each plan's ``check`` first and hands a
call its kernel would reject to the next family.  This test binds, on the CPU with a
stub library in place of the GPU one, the plan ``select`` picks and every tuning
candidate, across stride and dtype patterns of the six hot-path programs.
"""

import functools

import pytest
import torch

import ninetoothed_amd as ninetoothed
import programs as pg
from ninetoothed_amd import _lib, families, kernels


class _StubLibrary:
    """Stands in for libnt_mi355x.so: every entry point exists and returns 0."""

    def __getattr__(self, name):
        if name not in _lib.exported_symbols():
            raise AttributeError(name)

        def entry(*args):
            return 0

        entry.__name__ = name
        return entry


@pytest.fixture
def stub_library(monkeypatch):
    monkeypatch.setattr(_lib, "load", lambda: _StubLibrary())
    monkeypatch.setattr(kernels, "_check_device", lambda *tensors: torch.device("cpu"))
    monkeypatch.setattr(kernels, "_stream_of", lambda device: (lambda: None))


def _bind_all(handle, args, meta=None):
    """Bind the selected plan and every tuning candidate; return the selected family."""
    names = handle._abi["public_args"]
    public = dict(zip(names, args))
    index = {n: i for i, n in enumerate(names)}
    ctx = handle._kernel.context(public, meta or {})
    plan = families.select(ctx)
    if plan.family != "generic":
        plan.bind(public, index)
    bound = 0
    for cand in families.candidates(ctx):
        if cand.family == "generic":
            continue
        cand.bind(public, index)  # a candidate that passed check must bind
        bound += 1
    return plan.family, bound


def _t(shape, dtype=torch.float16):
    return torch.empty(shape, dtype=dtype)


F16, BF16, F32, F64 = torch.float16, torch.bfloat16, torch.float32, torch.float64


@pytest.mark.parametrize(
    "xs, ydtype, family",
    [
        ((F16, False, None), F16, "softmax"),
        ((F16, True, None), F16, "softmax"),  # x.t()
        ((F16, False, 2), F16, "softmax"),  # x[:, ::2]
        ((F16, False, None), F32, "softmax"),  # fp16 in, fp32 out
        ((F32, False, None), BF16, "softmax"),
        ((BF16, True, 3), F16, "softmax"),
        ((F64, False, None), F64, "generic"),  # no float64 softmax kernel: the generic kernels
    ],
)
def test_softmax_plans_bind(stub_library, xs, ydtype, family):
    dtype, transposed, step = xs
    rows, cols = 24, 50
    if transposed:
        x = _t((cols, rows), dtype).t()
    elif step:
        x = _t((rows, cols * step), dtype)[:, ::step]
    else:
        x = _t((rows, cols), dtype)
    y = _t((rows, cols), ydtype)
    for h in (pg.make_softmax(), pg.make_softmax(max_num_configs=5)):
        got, bound = _bind_all(h, (x, y), {"BLOCK_SIZE": cols})
        assert got == family
        assert bound >= (1 if family == "softmax" else 0)


@pytest.mark.parametrize(
    "xdtype, ydtype, strided, family",
    [
        (F16, F16, False, "max_pool2d"),
        (F16, F32, False, "max_pool2d"),
        (F32, F16, True, "max_pool2d"),
        (BF16, F32, True, "max_pool2d"),
        (F64, F64, False, "generic"),
    ],
)
def test_max_pool2d_plans_bind(stub_library, xdtype, ydtype, strided, family):
    h = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=False), pg.max_pool2d_application,
                         pg.max_pool2d_tensors())
    x = _t((2, 3, 16, 32), xdtype)[..., ::2] if strided else _t((2, 3, 16, 16), xdtype)
    y = _t((2, 3, 8, 8), ydtype)
    got, _ = _bind_all(h, (x, y), {"WINDOW_HEIGHT": 2, "WINDOW_WIDTH": 2})
    assert got == family


@pytest.mark.parametrize(
    "adtype, bdtype, odtype, bt, family",
    [
        (F16, F16, F16, False, "gemm"),
        (BF16, BF16, BF16, True, "gemm"),
        (F32, F32, F32, False, "gemm"),
        (F16, F16, F32, False, "gemm"),
        (F16, BF16, F16, False, "generic"),  # operands of two dtypes: no GEMM kernel takes them
        (F64, F64, F64, False, "generic"),
    ],
)
def test_matmul_plans_bind(stub_library, adtype, bdtype, odtype, bt, family):
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    b = _t((72, 80), bdtype).t() if bt else _t((80, 72), bdtype)
    got, _ = _bind_all(h, (_t((96, 80), adtype), b, _t((96, 72), odtype)))
    assert got == family


@pytest.mark.parametrize("cdtype, family", [(F16, "gemm"), (F32, "gemm"), (F64, "generic")])
def test_addmm_plans_bind(stub_library, cdtype, family):
    h = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    got, _ = _bind_all(h, (_t((64, 48), cdtype), _t((64, 32)), _t((32, 48)), 0.5, 2.0, _t((64, 48))))
    assert got == family


@pytest.mark.parametrize("dtype, family", [(F16, "conv2d"), (BF16, "conv2d"), (F32, "generic")])
def test_conv2d_plans_bind(stub_library, dtype, family):
    h = pg.make_conv2d()
    got, _ = _bind_all(h, (_t((2, 16, 8, 8), dtype), _t((32, 16, 3, 3), dtype), _t((2, 32, 8, 8), dtype)),
                       {"padding_h": 1, "padding_w": 1})
    assert got == family


@pytest.mark.parametrize("dtype, odtype", [(F16, F16), (F32, F32), (BF16, F32)])
def test_attention_plans_bind(stub_library, dtype, odtype):
    h = ninetoothed.make(pg.attention_arrangement, pg.attention_application, pg.attention_tensors())
    q = _t((1, 2, 64, 32), dtype)
    got, _ = _bind_all(h, (q, q, q, True, _t((1, 2, 64, 32), odtype)))
    assert got == "attention"


def test_float64_attention_is_refused_before_binding(stub_library):
    # no attention kernel takes float64 and the generic kernels do not take its loop: the
    # call is refused with the reason, never bound to a kernel that would reject it
    h = ninetoothed.make(pg.attention_arrangement, pg.attention_application, pg.attention_tensors())
    q = _t((1, 2, 64, 32), F64)
    with pytest.raises(ninetoothed.LoweringError, match="float64"):
        _bind_all(h, (q, q, q, True, q))


@pytest.mark.parametrize("dtype, family", [(F16, "add"), (F32, "add"), (F64, "generic")])
def test_add_plans_bind(stub_library, dtype, family):
    h = pg.make_add()
    x = _t((1000,), dtype)
    got, _ = _bind_all(h, (x, x, x))
    assert got == family
