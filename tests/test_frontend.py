"""Host logic on the CPU: lowering, family matching, launch ABI, call contract, registry."""

import functools
import json
import re
from pathlib import Path

import pytest
import torch

import ninetoothed_amd as ninetoothed
import ninetoothed_amd.language as ntl
import programs as pg
from ninetoothed_amd import Symbol, Tensor, _lib
from ninetoothed_amd.backends import Target, default_registry, normalize_target
from ninetoothed_amd.backends.core import Backend, Registry
from ninetoothed_amd.errors import LoweringError


def _specialize(handle, *args, **kwargs):
    names = handle._abi["public_args"]
    public, meta = dict(zip(names, args)), {}
    for k, v in kwargs.items():
        (public if k in names else meta)[k] = v
    return handle._kernel.specialize(public, meta).describe()


def _h(shape, dtype=torch.float16):
    return torch.empty(shape, dtype=dtype)


# The reference's own schedule granularity per program (compiler/passes.py:1070-1084), as its
# pipeline computed it for its test programs (tests/golden/make_reference_registry.py).
_REFERENCE = json.loads((Path(__file__).parent / "golden" / "reference_registry.json").read_text())["programs"]


def _granularity(program):
    return _REFERENCE[program]["reference"]["granularity"]


# ------------------------------------------------------------------- matching
def test_matmul_matches_gemm():
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    assert h._abi["public_args"] == ("lhs", "rhs", "output")
    assert h._abi["outputs"] == ("output",)
    assert h._kernel.granularity == _granularity("matmul")
    d = _specialize(h, _h((96, 80)), _h((80, 72)), _h((96, 72)))
    assert d["family"] == "gemm" and d["round"] == "torch.float16" and d["c"] is None


def test_matmul_transposed_view_matches():
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    b = _h((72, 80)).t()
    assert _specialize(h, _h((96, 80)), b, _h((96, 72)))["family"] == "gemm"


def test_addmm_epilogue_is_read():
    h = ninetoothed.make(pg.addmm_arrangement, pg.addmm_application, pg.addmm_tensors())
    d = _specialize(h, _h((64, 48)), _h((64, 32)), _h((32, 48)), 0.5, 2.0, _h((64, 48)))
    assert d == {"family": "gemm", "a": "mat1", "b": "mat2", "out": "output", "c": "input", "round": "torch.float16"}


@pytest.mark.parametrize("padding", ((0, 0), (1, 1), (0, 1), (2, 0)))
def test_conv2d_geometry_is_recovered(padding):
    h = pg.make_conv2d()
    ph, pw = padding
    d = _specialize(h, _h((4, 64, 16, 16)), _h((512, 64, 3, 3)), _h((4, 512, 14 + 2 * ph, 14 + 2 * pw)),
                    padding_h=ph, padding_w=pw)
    assert d["family"] == "conv2d" and d["padding"] == padding and d["stride"] == (1, 1)
    assert h._kernel.granularity == _granularity("conv2d")


@pytest.mark.parametrize("case", (
    # (H, W, R, S, padding): a filter axis of one tap, an output axis of one position, both
    ((16, 16, 1, 1, (0, 0)), (16, 16, 1, 3, (0, 1)), (16, 16, 5, 1, (2, 0)), (2, 14, 2, 4, (0, 0)),
     (1, 24, 1, 5, (0, 2)), (3, 3, 3, 3, (0, 0)), (1, 1, 1, 1, (0, 0)))
))
def test_conv2d_geometry_with_axes_of_one(case):
    # One tap (R or S of 1) leaves that axis' dilation undetermined by the index maps, one
    # output position (P or Q of 1) its stride: both are taken as 1, so these calls stay on
    # the conv2d kernels instead of the generic ones.
    h_, w_, r, s, (ph, pw) = case
    p, q = h_ + 2 * ph - r + 1, w_ + 2 * pw - s + 1
    d = _specialize(pg.make_conv2d(), _h((2, 32, h_, w_)), _h((40, 32, r, s)), _h((2, 40, p, q)), padding_h=ph,
                    padding_w=pw)
    assert d["family"] == "conv2d" and d["padding"] == (ph, pw)
    assert d["stride"] == (1, 1) and d["dilation"] == (1, 1)


@pytest.mark.parametrize("causal", (False, True))
def test_attention_matches(causal):
    h = ninetoothed.make(pg.attention_arrangement, pg.attention_application, pg.attention_tensors())
    assert h._kernel.granularity == _granularity("attention")
    q = _h((2, 4, 100, 64))
    d = _specialize(h, q, q, q, causal, q)
    assert d == {"family": "attention", "causal": causal, "scale": 1.44269504089}


def test_softmax_block_size_is_semantic():
    sm = pg.make_softmax()
    assert sm._kernel.granularity == _granularity("softmax")
    x = torch.empty(10, 100)
    assert _specialize(sm, x, torch.empty_like(x), BLOCK_SIZE=100)["block"] == 100
    assert _specialize(sm, x, torch.empty_like(x), BLOCK_SIZE=32)["block"] == 32


@pytest.mark.parametrize("ceil_mode", (False, True))
def test_max_pool2d_window(ceil_mode):
    h = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=ceil_mode), pg.max_pool2d_application,
                         pg.max_pool2d_tensors())
    p = (64 - 3 + (2 if ceil_mode else 0)) // 3 + 1
    d = _specialize(h, _h((32, 3, 64, 64)), _h((32, 3, p, p)), WINDOW_HEIGHT=3, WINDOW_WIDTH=3)
    assert d["family"] == "max_pool2d" and d["window"] == (3, 3) and d["stride"] == (3, 3)
    assert h._kernel.granularity == _granularity("max_pool2d")


def test_add_matches():
    add = pg.make_add()
    assert add._kernel.granularity == _granularity("add")
    v = torch.empty(98432)
    assert _specialize(add, v, v, v)["family"] == "add"


# ---------------------------------------------------------------- rejections
def test_elementwise_program_outside_the_families_is_generic():
    def app(lhs, rhs, output):
        output = ntl.sqrt(lhs) + rhs  # noqa: F841

    bs = Symbol("BS", meta=True)
    h = ninetoothed.make(lambda a, b, c: (a.tile((bs,)), b.tile((bs,)), c.tile((bs,))), app,
                         (Tensor(1), Tensor(1), Tensor(1)))
    assert _specialize(h, torch.empty(10), torch.empty(10), torch.empty(10))["family"] == "generic"


def _sum_of(a, b):
    s = a + b
    return s


def test_helper_with_a_trailing_return_is_inlined():
    # reference frontend/python.py:226-270: a helper's trailing `return value` is the call's value
    def app(lhs, rhs, output):
        output = _sum_of(lhs, rhs)  # noqa: F841

    bs = Symbol("BS", meta=True)
    h = ninetoothed.make(lambda a, b, c: (a.tile((bs,)), b.tile((bs,)), c.tile((bs,))), app,
                         (Tensor(1), Tensor(1), Tensor(1)))
    assert _specialize(h, torch.empty(10), torch.empty(10), torch.empty(10))["family"] == "add"


def test_reduction_program_is_generic():
    def app(lhs, rhs, output):
        output = ntl.sum(lhs, 0) + rhs  # noqa: F841

    bs = Symbol("BS", meta=True)
    h = ninetoothed.make(lambda a, b, c: (a.tile((bs,)), b.tile((bs,)), c.tile((bs,))), app,
                         (Tensor(1), Tensor(1), Tensor(1)))
    assert _specialize(h, torch.empty(10), torch.empty(10), torch.empty(10))["family"] == "generic"


def test_block_product_without_k_loop_is_a_tile_program():
    # a block product without the k loop of a matmul is no GEMM; the generic tile kernels
    # take it (ntl.dot as an fp32 reduction)
    def app(lhs, rhs, output):
        output = ntl.dot(lhs, rhs)  # noqa: F841

    h = ninetoothed.make(lambda a, b, c: (a.tile((16, 16)), b.tile((16, 16)), c.tile((16, 16))), app,
                         (Tensor(2), Tensor(2), Tensor(2)))
    described = _specialize(h, _h((16, 16)), _h((16, 16)), _h((16, 16)))
    assert described["family"] == "generic" and described["reductions"] == 1


def test_dot_of_two_transposed_tiles_is_a_tile_program():
    def app(lhs, rhs, output):
        output = ntl.dot(ntl.trans(lhs), ntl.trans(rhs))  # noqa: F841

    h = ninetoothed.make(lambda a, b, c: (a.tile((16, 16)), b.tile((16, 16)), c.tile((16, 16))), app,
                         (Tensor(2), Tensor(2), Tensor(2)))
    described = _specialize(h, _h((16, 16)), _h((16, 16)), _h((16, 16)))
    assert described["family"] == "generic" and described["reductions"] == 1


def test_unsupported_program_is_rejected():
    # a value computed inside a loop with a run-time trip count, stored after it: neither a
    # family nor the generic kernels (they store a loop's carried results after it)
    def app(lhs, n, output):
        for i in range(n):
            y = lhs * i
        output = y  # noqa: F841

    h = ninetoothed.make(lambda a, n, c: (a.tile((16, 16)), n, c.tile((16, 16))), app,
                         (Tensor(2), Tensor(0), Tensor(2)))
    with pytest.raises(LoweringError):
        _specialize(h, _h((16, 16)), 3, _h((16, 16)))


def test_output_assigned_in_an_unrolled_loop_keeps_the_last_store():
    def app(lhs, rhs, output):
        for i in range(3):
            output = lhs * i + rhs  # noqa: F841

    h = ninetoothed.make(lambda a, b, c: (a.tile((16, 16)), b.tile((16, 16)), c.tile((16, 16))), app,
                         (Tensor(2), Tensor(2), Tensor(2)))
    assert _specialize(h, _h((16, 16)), _h((16, 16)), _h((16, 16)))["family"] in ("generic", "add")


def test_data_dependent_if_is_rejected():
    def app(x, y):
        if x > 0:
            y = x  # noqa: F841

    h = ninetoothed.make(lambda a, b: (a.tile((4,)), b.tile((4,))), app, (Tensor(1), Tensor(1)))
    with pytest.raises(LoweringError, match="constexpr"):
        _specialize(h, torch.empty(8), torch.empty(8))


def test_mismatched_gemm_tiling_is_rejected():
    # `bad` only permutes twice (still a matmul); `bad2` swaps the output block shape.
    def bad(lhs, rhs, output, BM=16, BN=16, BK=16):
        out = output.tile((BM, BN))
        lt = lhs.tile((BM, BK)).tile((1, -1)).expand((-1, out.shape[1]))
        lt.dtype = lt.dtype.squeeze(0)
        rt = rhs.tile((BK, BN)).tile((-1, 1)).expand((out.shape[0], -1))
        rt.dtype = rt.dtype.squeeze(1)
        return lt, rt.permute((1, 0)).permute((1, 0)), out.permute((1, 0)).permute((1, 0))

    def bad2(lhs, rhs, output, BM=16, BN=32, BK=16):
        lt, rt, out = pg.matmul_arrangement(lhs, rhs, output, BM, BN, BK)
        return lt, rt, output.tile((BN, BM))  # swapped output block

    ok = ninetoothed.make(bad, pg.matmul_application, pg.matmul_tensors())
    assert _specialize(ok, _h((32, 48)), _h((48, 64)), _h((32, 64)))["family"] == "gemm"
    h = ninetoothed.make(bad2, pg.matmul_application, pg.matmul_tensors())
    with pytest.raises(LoweringError):
        _specialize(h, _h((32, 48)), _h((48, 64)), _h((32, 64)))


def test_overlapping_k_tiles_are_rejected():
    # k-tiles of stride 8 but size 16 visit each k twice: not a plain matmul.
    def overlap(lhs, rhs, output, BM=16, BN=16, BK=16):
        out = output.tile((BM, BN))
        lt = lhs.tile((BM, BK), strides=(-1, 8)).tile((1, -1)).expand((-1, out.shape[1]))
        lt.dtype = lt.dtype.squeeze(0)
        rt = rhs.tile((BK, BN), strides=(8, -1)).tile((-1, 1)).expand((out.shape[0], -1))
        rt.dtype = rt.dtype.squeeze(1)
        return lt, rt, out

    from ninetoothed_amd import families

    h = ninetoothed.make(overlap, pg.matmul_application, pg.matmul_tensors())
    ctx = h._kernel.context(dict(zip(h._abi["public_args"], (_h((32, 48)), _h((48, 64)), _h((32, 64))))), {})
    with pytest.raises(LoweringError, match="exactly once|disagree"):
        families.match_gemm(ctx)
    # the generic tile kernels take it as written (the loop unrolled, each dot a reduction)
    assert _specialize(h, _h((32, 48)), _h((48, 64)), _h((32, 64)))["family"] == "generic"


# ---------------------------------------------------------------- call contract
@pytest.fixture
def matmul_handle():
    return ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())


def test_contract_argument_errors(matmul_handle):
    a = _h((4, 4))
    with pytest.raises(TypeError, match="at most 3"):
        matmul_handle(a, a, a, a)
    with pytest.raises(TypeError, match="passed twice"):
        matmul_handle(a, a, a, lhs=a)
    with pytest.raises(TypeError, match="Unknown kernel arguments"):
        matmul_handle(a, a, a, nonsense=1)
    with pytest.raises(TypeError, match="Missing kernel arguments: output"):
        matmul_handle(a, a)


def test_contract_rank_device_dtype(matmul_handle):
    with pytest.raises(TypeError, match="rank 3; expected 2"):
        matmul_handle(_h((2, 2, 2)), _h((2, 2)), _h((2, 2)))
    with pytest.raises(TypeError, match="CUDA device"):
        matmul_handle(_h((2, 2)), _h((2, 2)), _h((2, 2)))
    typed = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application,
                             (Tensor(2, dtype=ninetoothed.float16), Tensor(2), Tensor(shape=(2, 3))))
    typed._device_types = ("cpu",)
    with pytest.raises(TypeError, match="dtype float32; expected float16"):
        typed(torch.empty(2, 2), _h((2, 3)), _h((2, 3)))
    with pytest.raises(TypeError, match="expected dimension 1 to be 3"):
        typed(_h((2, 2)), _h((2, 4)), _h((2, 4)))


def test_contract_empty_output_launches_nothing(matmul_handle):
    matmul_handle._device_types = ("cpu",)  # no GPU needed: the empty launch returns before any kernel
    out = _h((0, 5))
    assert matmul_handle(_h((0, 3)), _h((3, 5)), out) is out


def test_meta_kwargs_are_accepted():
    sm = pg.make_softmax()
    assert sm._abi["meta_args"] == ("BLOCK_SIZE",)
    h = pg.make_conv2d()
    assert {"padding_h", "padding_w"} <= set(h._abi["meta_args"])


def test_missing_constexpr_is_a_type_error():
    sm = pg.make_softmax()
    x = torch.empty(4, 8)
    with pytest.raises(TypeError, match="BLOCK_SIZE"):
        _specialize(sm, x, torch.empty_like(x))


# ----------------------------------------------------------------- registry
def test_registry_and_targets():
    reg = default_registry()
    assert reg.names() == ("hip",)
    assert normalize_target(None) is Target.HIP and normalize_target("rocm") is Target.HIP
    with pytest.raises(ValueError, match="Unsupported backend"):
        normalize_target("triton")
    with pytest.raises(TypeError, match="Unsupported hip backend option"):
        reg.get("hip").normalize_options({"num_ctas": 2})
    r = Registry()

    class Dummy(Backend):
        name = "dummy"

    r.register(Dummy())
    with pytest.raises(ValueError, match="already registered"):
        r.register(Dummy())


def test_artifact_metadata_contract():
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    md = h._artifact.metadata
    for key in ("variables", "outputs", "shape_params", "program_mode", "target", "tensors"):
        assert key in md
    assert md["schedule"]["granularity"] == "blocked-linalg"


# ------------------------------------------------------------------ library
def test_library_exports_every_declared_entry_point():
    header = (Path(__file__).resolve().parents[1] / "include" / "nt_mi355x.h").read_text()
    declared = set(re.findall(r"^(?:int|int64_t|void)\s+(nt_\w+)\(", header, re.M))
    assert declared == set(_lib.exported_symbols())
    lib = _lib.load()  # loads without a GPU; no compute call
    for name in declared:
        assert callable(getattr(lib, name))
    assert lib.nt_abi_version() == _lib.ABI_VERSION


def test_constexpr_used_as_a_value_is_lowered():
    # reference tests/test_scalar_element_reads.py: a constexpr scalar divides a row sum
    def app(x, scale, out):
        mean = ntl.sum(x, axis=1) / scale
        out = x - mean[:, None]  # noqa: F841

    scalar = Tensor(0, dtype="float32", constexpr=True, value=32.0)
    h = ninetoothed.make(lambda x, s, o: (x.tile((1, 32)), s, o.tile((1, 32))), app, (Tensor(2), scalar, Tensor(2)))
    assert h._abi["outputs"] == ("out",)
    x = torch.empty(3, 32)
    assert _specialize(h, x, 32.0, x)["family"] == "generic"
