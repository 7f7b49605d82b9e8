"""The generic element-parallel kernels (programs outside the hand-written families).

CPU: the reference's typing rules in the emitted source, the per-tensor index tables
(against numpy slicing / transposition of the same tensor), hipRTC compilation of the
emitted source for gfx950.  GPU: the reference's own elementwise tests (clone
application 0, ``libdevice.pow``, constant pad, expand of an empty tensor: reference
tests/test_clone.py, test_pow.py, test_pad.py, test_expand.py) and fp16/bf16 chains,
scalars, casts, in-place updates and transposed arrangements against torch.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ninetoothed_amd as ninetoothed
import ninetoothed_amd.language as ntl
from ninetoothed_amd import Symbol, Tensor, block_size
from ninetoothed_amd.generic import GenericPlan

BS = Symbol("BS", meta=True)


def _plan(handle, *args, **meta):
    names = handle._abi["public_args"]
    return handle._kernel.specialize(dict(zip(names, args)), meta)


def _tiled1(app, n):
    return ninetoothed.make(lambda *ts: tuple(t.tile((BS,)) for t in ts), app, tuple(Tensor(1) for _ in range(n)))


# ------------------------------------------------------------------ applications
def app_chain(x, y, output):
    output = ntl.maximum(x * 2 + y, 0.0) - ntl.exp(-x) / (1 + y * y)  # noqa: F841


def app_mixed(x, y, output):
    output = x + y  # noqa: F841


def app_div(x, y, output):
    output = x / y  # noqa: F841


def app_where(x, y, output):
    output = ntl.where(x > y, x, y * 0.5)  # noqa: F841


def app_scalars(x, alpha, beta, output):
    output = x * alpha + beta  # noqa: F841


def app_cast(x, output):
    output = (x > 0).to(ntl.float16) * ntl.sigmoid(x)  # noqa: F841


def app_inplace(x):
    x = x * x + 1  # noqa: F841


def app_int(x, y, output):
    output = x * 3 - y  # noqa: F841


def app_pow(input, exponent, output):
    output = ntl.libdevice.pow(input, exponent)  # noqa: F841


def app_copy(input, output):
    output = input  # noqa: F841


# ------------------------------------------------------------------ CPU: typing and source
def test_typing_follows_the_reference_rules():
    h = _tiled1(app_chain, 3)
    src = _plan(h, *(torch.empty(8, dtype=torch.float16) for _ in range(3))).source()
    # fp16 operations round after every step; the weakly typed literals stay fp16
    assert "r_f16((v" in src and "float v" in src and "double" not in src.split("nt_generic(")[1]
    mixed = _plan(_tiled1(app_mixed, 3), torch.empty(8, dtype=torch.float16), torch.empty(8, dtype=torch.bfloat16),
                  torch.empty(8, dtype=torch.float32)).source()
    body = mixed.split("nt_generic(")[1]
    assert "r_f16((v" not in body and "r_bf16((v" not in body  # fp16 + bf16 -> fp32
    div = _plan(_tiled1(app_div, 3), *(torch.empty(8, dtype=torch.float16) for _ in range(2)),
                torch.empty(8, dtype=torch.float16)).source()
    assert "r_f16((v0 / v1))" not in div and "(v0 / v1)" in div  # division promotes to fp32
    ints = _plan(_tiled1(app_int, 3), *(torch.empty(8, dtype=torch.int32) for _ in range(3))).source()
    assert "long long v" in ints


def test_scalar_parameters_are_typed_by_their_python_type():
    h = ninetoothed.make(lambda x, a, b, o: (x.tile((BS,)), a, b, o.tile((BS,))), app_scalars,
                         (Tensor(1), Tensor(0), Tensor(0), Tensor(1)))
    x = torch.empty(8)
    src = _plan(h, x, 0.5, 3, x).source()
    assert "float s_alpha" in src and "long long s_beta" in src


def test_index_tables_match_numpy_views():
    # a transposed, tiled source against numpy's transpose of the same offsets
    def arrange(src, dst):
        return src.permute((1, 0)).tile((16, 32)), dst.tile((16, 32))

    h = ninetoothed.make(arrange, app_copy, (Tensor(2), Tensor(2)))
    src = torch.empty_strided((70, 45), (50, 1))
    dst = torch.empty(45, 70)
    plan = _plan(h, src, dst)
    ts, total = plan._table("input", src)
    td, _ = plan._table("output", dst)
    assert total == ts.size == td.size
    offs = (np.arange(70)[:, None] * 50 + np.arange(45)[None, :]).T  # element (i, j) of the transposed view
    valid = td >= 0
    assert np.count_nonzero(valid) == 45 * 70
    # every output element (i, j) -> input element (j, i)
    i, j = np.divmod(td[valid], 70)
    assert np.array_equal(ts[valid], offs[i, j])
    assert np.all(ts[~valid] == -1)


def test_index_tables_of_sliced_arrangements():
    # reference tests/test_pad.py: input[input_slices] -> output[output_slices]
    def arrange(input, output, input_slices, output_slices):
        return input[input_slices], output[output_slices]

    isl, osl = (slice(1, 2), slice(0, 3)), (slice(1, 2), slice(1, 4))
    h = ninetoothed.make(arrange, app_copy, (Tensor(2), Tensor(2), isl, osl))
    inp, out = torch.empty(2, 3), torch.empty(3, 6)
    plan = _plan(h, inp, out)
    ti, _ = plan._table("input", inp)
    to, _ = plan._table("output", out)
    assert np.array_equal(ti, np.arange(6).reshape(2, 3)[isl].ravel())
    assert np.array_equal(to, np.arange(18).reshape(3, 6)[osl].ravel())


def test_tables_agree_with_eval():
    # ninetoothed.eval gives the contiguous source offset of every element of an arrangement
    def arrange(x, y):
        return x.tile((4, 8)), y.tile((4, 8))

    h = ninetoothed.make(arrange, app_copy, (Tensor(2), Tensor(2)))
    x = torch.empty(10, 20)
    t, _ = _plan(h, x, x)._table("input", x)
    src = Tensor(2)
    assert np.array_equal(t, ninetoothed.eval(src.tile((4, 8)), {src: {"shape": (10, 20)}}).reshape(-1))


def test_no_store_program_is_a_no_op():
    # reference tests/test_expand.py: the application only names its parameter
    def arrangement(x, BLOCK_SIZE=block_size()):
        return (x.expand((BLOCK_SIZE,)).tile((BLOCK_SIZE,)),)

    def application(x):
        x  # noqa: B018

    h = ninetoothed.make(arrangement, application, (Tensor(1),))
    x = torch.empty((0,))
    plan = _plan(h, x)
    assert plan.describe()["family"] == "generic" and plan.describe()["outputs"] == []
    assert plan.bind({"x": x}, {"x": 0})((x,)) is None


@pytest.mark.parametrize("app, n, dtype", ((app_chain, 3, torch.float16), (app_chain, 3, torch.bfloat16),
                                           (app_where, 3, torch.float32), (app_int, 3, torch.int32),
                                           (app_pow, 3, torch.float64)))
def test_emitted_source_compiles(app, n, dtype):
    plan = _plan(_tiled1(app, n), *(torch.empty(8, dtype=dtype) for _ in range(n)))
    blob = GenericPlan.compile(plan.source())
    assert len(blob) > 1000
    # the variant whose first operand is walked linearly (no index table)
    assert len(GenericPlan.compile(plan.source({plan.loaded[0]: 5}))) > 1000


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_clone_reference_case():
    # reference tests/test_clone.py:49-70 (application 0)
    def arrangement(input, output):
        block_shape = (block_size(), block_size())
        return input.tile(block_shape), output.tile(block_shape)

    kernel = ninetoothed.make(arrangement, app_copy, (Tensor(2), Tensor(2)))
    inp = torch.empty_strided((641, 280), (700, 300), device="cuda")
    inp.copy_(torch.randn(641, 280, device="cuda"))
    out = torch.empty_like(inp)
    kernel(inp, out)
    assert torch.equal(out, inp)


@pytest.mark.gpu
def test_pow_reference_case():
    # reference tests/test_pow.py:33-42
    kernel = _tiled1(app_pow, 3)
    inp = torch.rand(44925, device="cuda")
    exponent = torch.rand(44925, device="cuda")
    out = torch.empty_like(inp)
    kernel(inp, exponent, out)
    assert torch.allclose(out, torch.pow(inp, exponent), equal_nan=True)


def _pad_slices(shape, pad):
    out_shape, isl, osl = list(shape), [], []
    for i in range(len(shape)):
        left, right = pad[2 * (len(shape) - 1 - i)], pad[2 * (len(shape) - 1 - i) + 1]
        out_shape[i] += left + right
        isl.append(slice(max(0, -left), min(shape[i], shape[i] + right)))
        osl.append(slice(max(0, left), out_shape[i] - max(0, right)))
    return out_shape, tuple(isl), tuple(osl)


_PAD_KERNELS = {}


@pytest.mark.gpu
@pytest.mark.parametrize("dtype, atol", ((torch.float32, 1e-8), (torch.float16, 1e-3)))
@pytest.mark.parametrize("value", (0, 1, -1, float("-inf"), torch.pi, float(torch.sqrt(torch.tensor(2026)))))
@pytest.mark.parametrize("shape, pad", (((2026, 1207), (-100, 20, 99, -10)), ((2, 3), (1, 1, 1, 2)),
                                        ((2, 3, 4), (1, 3, 1, 0, 0, 0)), ((2, 3), (-1, -1, 0, 0))))
def test_pad_reference_cases(shape, pad, value, dtype, atol):
    # reference tests/test_pad.py:40-58 (arrangement input[slices] -> output[slices])
    def arrangement(input, output, input_slices, output_slices):
        return input[input_slices], output[output_slices]

    inp = torch.randn(shape, dtype=dtype, device="cuda")
    out_shape, isl, osl = _pad_slices(shape, pad)
    out = torch.full(out_shape, value, dtype=dtype, device="cuda")
    key = str((len(shape), isl, osl))
    if key not in _PAD_KERNELS:
        _PAD_KERNELS[key] = ninetoothed.make(arrangement, app_copy, (Tensor(len(shape)), Tensor(len(shape)), isl, osl))
    _PAD_KERNELS[key](inp, out)
    assert torch.allclose(out, F.pad(inp, pad, "constant", value), atol=atol)


@pytest.mark.gpu
def test_expand_of_empty_tensor():
    # reference tests/test_expand.py:16-22
    def arrangement(x, BLOCK_SIZE=block_size()):
        return (x.expand((BLOCK_SIZE,)).tile((BLOCK_SIZE,)),)

    def application(x):
        x  # noqa: B018

    kernel = ninetoothed.make(arrangement, application, (Tensor(1),))
    kernel(torch.empty((0,), device="cuda"))
    torch.cuda.synchronize()


def _chain_ref(x, y):
    x, y = x.float(), y.float()
    return torch.clamp_min(x * 2 + y, 0.0) - torch.exp(-x) / (1 + y * y)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
@pytest.mark.parametrize("n", (1, 1000, 65537))
def test_elementwise_chain(dtype, n):
    kernel = _tiled1(app_chain, 3)
    g = torch.Generator(device="cuda").manual_seed(n)
    x = torch.randn(n, device="cuda", generator=g).to(dtype)
    y = torch.randn(n, device="cuda", generator=g).to(dtype)
    out = torch.empty(n, dtype=dtype, device="cuda")
    kernel(x, y, out)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(out.float(), _chain_ref(x, y), atol=tol, rtol=tol)


@pytest.mark.gpu
def test_where_scalars_cast_inplace_int():
    n = 4099
    x = torch.randn(n, device="cuda")
    y = torch.randn(n, device="cuda")
    out = torch.empty_like(x)
    _tiled1(app_where, 3)(x, y, out)
    assert torch.equal(out, torch.where(x > y, x, y * 0.5))

    k = ninetoothed.make(lambda x, a, b, o: (x.tile((BS,)), a, b, o.tile((BS,))), app_scalars,
                         (Tensor(1), Tensor(0), Tensor(0), Tensor(1)))
    k(x, 0.25, 3, out)
    torch.testing.assert_close(out, x * 0.25 + 3, atol=1e-6, rtol=1e-6)
    k(x, -2.0, 5, out)  # same launcher, new scalar values
    torch.testing.assert_close(out, x * -2.0 + 5, atol=1e-6, rtol=1e-6)

    xh = x.half()
    oh = torch.empty_like(xh)
    _tiled1(app_cast, 2)(xh, oh)
    ref = (xh > 0).half() * torch.sigmoid(xh.float()).half()
    torch.testing.assert_close(oh.float(), ref.float(), atol=1e-3, rtol=1e-3)

    z = x.clone()
    ninetoothed.make(lambda t: (t.tile((BS,)),), app_inplace, (Tensor(1),))(z)
    torch.testing.assert_close(z, x * x + 1, atol=1e-6, rtol=1e-6)

    xi = torch.randint(-1000, 1000, (n,), device="cuda", dtype=torch.int32)
    yi = torch.randint(-1000, 1000, (n,), device="cuda", dtype=torch.int32)
    oi = torch.empty_like(xi)
    _tiled1(app_int, 3)(xi, yi, oi)
    assert torch.equal(oi, xi * 3 - yi)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
def test_transposed_copy(dtype):
    def arrange(src, dst):
        return src.permute((1, 0)).tile((16, 32)), dst.tile((16, 32))

    kernel = ninetoothed.make(arrange, app_copy, (Tensor(2), Tensor(2)))
    src = torch.randn(300, 257, device="cuda").to(dtype)
    dst = torch.empty(257, 300, dtype=dtype, device="cuda")
    kernel(src, dst)
    assert torch.equal(dst, src.t())


# ------------------------------------------------------------------ ntl.rand family (dropout)
def drop_arrangement(input, p, seed, output, BLOCK_SIZE=block_size()):
    return input.tile((BLOCK_SIZE,)), p, seed, output.tile((BLOCK_SIZE,))


def drop_application(input, p, seed, output):
    # reference tests/test_dropout.py:16-17
    output = ntl.where(ntl.rand(seed, input.offsets()) > p, input / (1 - p), 0)  # noqa: F841


def app_randint(seed, output):
    output = ntl.randint(seed, output.offsets())  # noqa: F841


def app_rand(seed, output):
    output = ntl.rand(seed, output.offsets())  # noqa: F841


def app_randn(seed, output):
    output = ntl.randn(seed, output.offsets())  # noqa: F841


def _rng_kernel(app):
    return ninetoothed.make(lambda s, o: (s, o.tile((BS,))), app, (Tensor(0), Tensor(1)))


def test_dropout_program_compiles():
    k = ninetoothed.make(drop_arrangement, drop_application, (Tensor(1), Tensor(0), Tensor(0), Tensor(1)))
    x = torch.empty(349, dtype=torch.float16)
    plan = _plan(k, x, 0.3, 12345, x)
    assert plan.offsets == [("input", 0)] and plan.scalar_types == {"seed": "int64", "p": "float32"}
    assert len(GenericPlan.compile(plan.source())) > 1000
    q = plan._offsets_table("input", 0)
    assert np.array_equal(q, np.arange(q.size))  # 1-D tiles: the offset of element e is e


@pytest.mark.gpu
def test_dropout_reference_case():
    # reference tests/test_dropout.py:33-48, plus the exact mask from the oracle's Philox
    from oracle import philox

    kernel = ninetoothed.make(drop_arrangement, drop_application, (Tensor(1), Tensor(0), Tensor(0), Tensor(1)))
    x = torch.randn(349, dtype=torch.float16, device="cuda")
    p, seed = 0.3, 1_234_567
    out = torch.empty_like(x)
    kernel(x, p, seed, out)
    assert abs(out.nonzero().numel() / x.numel() - (1 - p)) < 0.05
    assert torch.allclose(out[out != 0], x[out != 0] / (1 - p))
    keep = philox.rand(seed, np.arange(349)) > np.float32(p)
    xs = x.float().cpu().numpy()
    expected = np.where(keep, xs / (np.float32(1.0) - np.float32(p)), 0).astype(np.float16)
    assert np.array_equal(out.cpu().numpy(), expected)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", (0, 1, 2**31 - 1, 2**40 + 12345))
def test_random_streams_match_the_oracle(seed):
    from oracle import philox

    n = 100_003
    offs = np.arange(n)
    oi = torch.empty(n, dtype=torch.int64, device="cuda")
    _rng_kernel(app_randint)(seed, oi)
    assert np.array_equal(oi.cpu().numpy(), philox.randint(seed, offs).astype(np.int64))
    of = torch.empty(n, dtype=torch.float32, device="cuda")
    _rng_kernel(app_rand)(seed, of)
    assert np.array_equal(of.cpu().numpy(), philox.rand(seed, offs))
    _rng_kernel(app_randn)(seed, of)
    assert np.allclose(of.cpu().numpy(), philox.randn(seed, offs), atol=1e-5, rtol=1e-5)


# ------------------------------------------------------------------ tile programs with reductions
# The reduction programs of reference tests/test_triton_reduction_schedule.py:18-119,
# test_cuda_reduction_schedule.py:114-187 and test_triton_block_reductions.py:17-140.
WIDTH = Symbol("WIDTH", constexpr=True)
HEIGHT = Symbol("HEIGHT", constexpr=True)


def row_arrangement(x, out, WIDTH=WIDTH):
    return x.tile((1, WIDTH)), out.tile((1, WIDTH))


def row_reduced_arrangement(x, out, WIDTH=WIDTH):
    return x.tile((1, WIDTH)), out.tile((1,))


def column_arrangement(x, out, HEIGHT=HEIGHT):
    return x.tile((HEIGHT, 1)), out.tile((HEIGHT, 1))


def row_normalize(x, out):
    maximum = ntl.max(x, axis=1)
    numerator = ntl.exp(x - maximum[:, None])
    out = numerator / ntl.sum(numerator, axis=1)[:, None]  # noqa: F841


def row_layernorm(x, out):
    width = x.shape[1]
    mean = ntl.sum(x, axis=1) / width
    mean_square = ntl.sum(x * x, axis=1) / width
    variance = mean_square - mean * mean
    out = (x - mean[:, None]) * ntl.rsqrt(variance[:, None] + 1e-5)  # noqa: F841


def row_min(x, out):
    out = ntl.min(x, axis=1)  # noqa: F841


def row_sum(x, out):
    out = ntl.sum(x, axis=1)  # noqa: F841


def column_max_broadcast(x, out):
    out = x + ntl.max(x, axis=0)[None, :]  # noqa: F841


def middle_axis_sum(x, out):
    out = ntl.sum(x, axis=1)  # noqa: F841


def separate_reduction_outputs(x, rows, columns):
    rows = ntl.sum(x, axis=1)  # noqa: F841
    columns = ntl.max(x, axis=0)  # noqa: F841


def block_arrangement(x, out):
    x = x.tile((1, -1, -1))
    x.dtype = x.dtype.squeeze(0)
    out = out.tile((1, -1))
    out.dtype = out.dtype.squeeze(0)
    return x, out


def block_application(x, out):
    weights = ntl.sum(x, axis=1)
    out = ntl.sum(x * weights[:, None], axis=0)  # noqa: F841


def independent_arrangement(x, y, out):
    return x.tile((-1,)), y.tile((-1,)), out.tile((-1,))


def independent_application(x, y, out):
    out = x + ntl.sum(y, axis=0)  # noqa: F841


def _reduce_kernel(arrangement, application, *ndims, dtype=None):
    return ninetoothed.make(arrangement, application, tuple(Tensor(n, dtype=dtype) for n in ndims))


def test_tile_programs_compile():
    cases = ((row_reduced_arrangement, row_min, (2, 1), ((37, 127), (37,)), {"WIDTH": 127}),
             (row_arrangement, row_normalize, (2, 2), ((41, 781), (41, 781)), {"WIDTH": 781}),
             (row_arrangement, row_layernorm, (2, 2), ((29, 1127), (29, 1127)), {"WIDTH": 1127}),
             (column_arrangement, column_max_broadcast, (2, 2), ((193, 41), (193, 41)), {"HEIGHT": 193}),
             (block_arrangement, block_application, (3, 2), ((3, 8, 16), (3, 16)), {}))
    for arrangement, application, ndims, shapes, meta in cases:
        h = _reduce_kernel(arrangement, application, *ndims)
        plan = _plan(h, *(torch.empty(s) for s in shapes), **meta)
        assert plan.describe()["family"] == "generic" and plan.describe()["reductions"] >= 1
        assert len(GenericPlan.compile(plan.source())) > 1000


def inplace_two_outputs(x, out):
    x = x - ntl.max(x, axis=1)[:, None]  # noqa: F841
    out = x  # noqa: F841


def test_tile_program_rejections():
    # a program that updates a tensor it reads stages its stores; one that scatters into a
    # tensor it reads is refused
    h = _reduce_kernel(row_arrangement, inplace_two_outputs, 2, 2)
    plan = _plan(h, torch.empty(4, 8), torch.empty(4, 8), WIDTH=8)
    assert plan.inplace
    # `out = x` after `x = ...` reads back what was stored (the reference loads x after its
    # store), in x's dtype: no load of x's memory
    assert plan.stores["out"].op == "cast" and plan.stores["out"].args[0] is plan.stores["x"]

    def scatter_into_read(x, out):
        x.source[x.offsets(0)[:, None], x.offsets(1)[None, :]] = x * 2
        out = x  # noqa: F841

    h = _reduce_kernel(row_arrangement, scatter_into_read, 2, 2)
    with pytest.raises(ninetoothed.LoweringError, match="scatter into"):
        _plan(h, torch.empty(4, 8), torch.empty(4, 8), WIDTH=8)


@pytest.mark.gpu
def test_cooperative_reduction_reference_cases():
    # reference tests/test_cuda_reduction_schedule.py:114-187 (backend-neutral programs, same data shapes)
    f32, f16, bf16 = ninetoothed.float32, ninetoothed.float16, ninetoothed.bfloat16
    reduce_min = _reduce_kernel(row_reduced_arrangement, row_min, 2, 1, dtype=f32)
    base = torch.randn((37, 254), device="cuda")
    x = base[:, ::2]
    output = torch.empty((37,), device="cuda")
    reduce_min(x, output, WIDTH=127)
    torch.testing.assert_close(output, x.min(dim=1).values)

    normalize = ninetoothed.make(row_arrangement, row_normalize, (Tensor(2, dtype=f16), Tensor(2, dtype=f16)))
    x = torch.randn((41, 781), device="cuda", dtype=torch.float16)
    output = torch.empty_like(x)
    normalize(x, output, WIDTH=781)
    torch.testing.assert_close(output, torch.softmax(x, dim=1), rtol=2e-3, atol=2e-3)

    layernorm = ninetoothed.make(row_arrangement, row_layernorm, (Tensor(2, dtype=bf16), Tensor(2, dtype=bf16)))
    x = torch.randn((29, 1127), device="cuda", dtype=torch.bfloat16)
    output = torch.empty_like(x)
    layernorm(x, output, WIDTH=1127)
    torch.testing.assert_close(output, F.layer_norm(x, (1127,)), rtol=2e-2, atol=2e-2)

    reduce_sum = _reduce_kernel(row_reduced_arrangement, row_sum, 2, 1, dtype=f32)
    x = torch.randn((17, 4097), device="cuda")
    output = torch.empty((17,), device="cuda")
    reduce_sum(x, output, WIDTH=4097)
    torch.testing.assert_close(output, x.sum(dim=1), rtol=1e-4, atol=1e-4)

    column_max = _reduce_kernel(column_arrangement, column_max_broadcast, 2, 2, dtype=f32)
    x = torch.randn((193, 41), device="cuda")
    output = torch.empty_like(x)
    column_max(x, output, HEIGHT=193)
    torch.testing.assert_close(output, x + x.max(dim=0).values)

    x = torch.empty((0, 127), device="cuda", dtype=torch.float16)
    output = torch.empty_like(x)
    normalize(x, output, WIDTH=127)
    assert output.numel() == 0


@pytest.mark.gpu
def test_block_reduction_reference_cases():
    # reference tests/test_triton_block_reductions.py:82-140
    shape = (3, 8, 16)
    x = torch.randn((*shape[:-1], shape[-1] * 2), device="cuda")[..., ::2]
    output = torch.empty((shape[0], shape[2]), device="cuda")
    _reduce_kernel(block_arrangement, block_application, 3, 2)(x, output)
    expected = (x.double() * x.double().sum(dim=2, keepdim=True)).sum(dim=1)
    torch.testing.assert_close(output, expected.float(), rtol=2e-5, atol=2e-5)

    x = torch.zeros(8, device="cuda")
    y = torch.arange(16, device="cuda", dtype=torch.float32)
    out = torch.empty_like(x)
    ninetoothed.make(independent_arrangement, independent_application, (Tensor(1), Tensor(1), Tensor(1)))(x, y, out)
    torch.testing.assert_close(out, torch.full_like(out, 120), rtol=0, atol=0)


def mixed_outer_reductions(x, y, out_x, out_y):
    out_x = ntl.sum(x, axis=1)  # noqa: F841
    out_y = ntl.sum(y, axis=1)  # noqa: F841


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
def test_more_reduction_programs(dtype):
    # the other programs of reference tests/test_triton_reduction_schedule.py:43-109
    tol = 1e-2 if dtype == torch.float16 else 1e-5
    x = torch.randn((4, 8), device="cuda").to(dtype)
    rows = torch.empty(4, device="cuda", dtype=dtype)
    cols = torch.empty(8, device="cuda", dtype=dtype)
    ninetoothed.make(lambda x, r, c: (x.tile((4, 8)), r.tile((4,)), c.tile((8,))), separate_reduction_outputs,
                     (Tensor(2), Tensor(1), Tensor(1)))(x, rows, cols)
    torch.testing.assert_close(rows.float(), x.float().sum(dim=1), rtol=tol, atol=tol)
    assert torch.equal(cols, x.max(dim=0).values)

    x, y = torch.randn((5, 7), device="cuda").to(dtype), torch.randn((5, 7), device="cuda").to(dtype)
    ox, oy = torch.empty(5, device="cuda", dtype=dtype), torch.empty(5, device="cuda", dtype=dtype)
    ninetoothed.make(lambda x, y, a, b: (x.tile((1, 7)), y.tile((1, 7)), a.tile((1,)), b.tile((1,))),
                     mixed_outer_reductions, (Tensor(2), Tensor(2), Tensor(1), Tensor(1)))(x, y, ox, oy)
    torch.testing.assert_close(ox.float(), x.float().sum(dim=1), rtol=tol, atol=tol)
    torch.testing.assert_close(oy.float(), y.float().sum(dim=1), rtol=tol, atol=tol)

    k = ninetoothed.make(lambda x, o: (x.tile((2, 3, 5)), o.tile((2, 5))), middle_axis_sum, (Tensor(3), Tensor(2)))
    out = torch.empty((6, 10), device="cuda", dtype=dtype)
    with pytest.raises(ninetoothed.LoweringError):
        k(torch.randn((6, 9, 10), device="cuda").to(dtype), out)  # 18 programs for x against 6 for out
    x = torch.randn((6, 3, 10), device="cuda").to(dtype)
    k(x, out)
    torch.testing.assert_close(out.float(), x.float().sum(dim=1), rtol=tol, atol=tol)


def scalar_row_application(x, scale, out):
    mean = ntl.sum(x, axis=1) / scale
    out = x - mean[:, None]  # noqa: F841


@pytest.mark.gpu
@pytest.mark.parametrize("constexpr", (False, True))
def test_scalar_in_row_expression(constexpr):
    # reference tests/test_scalar_element_reads.py:9-30
    scalar = Tensor(0, dtype="float32", constexpr=constexpr, value=32.0 if constexpr else None)
    kernel = ninetoothed.make(lambda x, s, o: (x.tile((1, 32)), s, o.tile((1, 32))), scalar_row_application,
                              (Tensor(2), scalar, Tensor(2)), max_num_configs=1)
    x = torch.randn((3, 32), device="cuda")
    out = torch.full_like(x, -12345)
    kernel(x, 32.0, out)
    torch.testing.assert_close(out, x - x.mean(1, keepdim=True))


# ------------------------------------------------------------------ pointers, source indexing, atomics
def clone_application_1(input, output):
    output = ntl.load(  # noqa: F841
        input.source.data_ptr()
        + input.offsets(0)[:, None] * input.source.stride(0)
        + input.offsets(1)[None, :] * input.source.stride(1)
    )


def clone_application_2(input, output):
    output = input.source[input.offsets(0)[:, None], input.offsets(1)[None, :]]  # noqa: F841


def clone_application_3(input, output):
    output.source[output.offsets(0)[:, None], output.offsets(1)[None, :]] = input


def clone_arrangement(input, output):
    block_shape = (block_size(), block_size())
    return input.tile(block_shape), output.tile(block_shape)


def sum_arrangement(input, output, BLOCK_SIZE=1024):
    input_arranged = input.tile((BLOCK_SIZE,))
    return input_arranged, output.tile((-1,)).expand(input_arranged.shape)


def sum_application(input, output):
    ntl.atomic_add(output.source.data_ptr(), ntl.sum(input))


@pytest.mark.parametrize("app", (clone_application_1, clone_application_2, clone_application_3))
def test_pointer_and_source_programs_compile(app):
    k = ninetoothed.make(clone_arrangement, app, (Tensor(2), Tensor(2)))
    assert k._abi["outputs"] == ("output",)
    x = torch.empty_strided((641, 280), (700, 300))
    plan = _plan(k, x, torch.empty(641, 280))
    assert plan.describe()["family"] == "generic"
    assert len(GenericPlan.compile(plan.source())) > 1000


@pytest.mark.gpu
@pytest.mark.parametrize("app", (clone_application_1, clone_application_2, clone_application_3))
def test_clone_pointer_applications(app):
    # reference tests/test_clone.py:22-70 (applications 1-3) on its strided input
    kernel = ninetoothed.make(clone_arrangement, app, (Tensor(2), Tensor(2)))
    inp = torch.empty_strided((641, 280), (700, 300), device="cuda")
    inp.copy_(torch.randn(641, 280, device="cuda"))
    out = torch.empty_like(inp)
    kernel(inp, out)
    assert torch.equal(out, inp)


@pytest.mark.gpu
def test_data_ptr_atomic_sum():
    # reference tests/test_data_ptr.py:10-42
    kernel = ninetoothed.make(sum_arrangement, sum_application, (Tensor(1), Tensor(1)))
    inp = torch.randn(64180, device="cuda")
    out = torch.zeros(1, dtype=inp.dtype, device="cuda")
    kernel(inp, out)
    assert torch.allclose(out[0], torch.sum(inp), rtol=1e-4, atol=1e-3)


# ------------------------------------------------------------------ loops over tiles (unrolled up to 64 iterations)
def tiled_arrangement(x, out):
    arranged = []
    for tensor in (x, out):
        tensor = tensor.tile((1, 256)).tile((1, -1))
        tensor.dtype = tensor.dtype.squeeze((0,))
        tensor.dtype.dtype = tensor.dtype.dtype.squeeze((0,))
        arranged.append(tensor)
    return tuple(arranged)


def tiled_normalize(x, out):
    # reference tests/test_tiled_reduction_loops.py:22-31
    accumulator = ntl.zeros(x.dtype.shape, dtype=ntl.float32)
    for i in range(x.shape[0]):
        block = ntl.cast(x[i], ntl.float32)
        accumulator += block * block
    scale = ntl.rsqrt(ntl.sum(accumulator) / x.source.shape[1] + 1e-5)
    for i in range(x.shape[0]):
        out[i] = x[i] * scale


def test_tiled_reduction_loop_is_unrolled():
    k = ninetoothed.make(tiled_arrangement, tiled_normalize, (Tensor(2, other=0), Tensor(2)))
    assert k._abi["outputs"] == ("out",)
    x = torch.empty((7, 2050))[:, ::2]
    plan = _plan(k, x, torch.empty((7, 1025)))
    assert plan.describe()["family"] == "generic" and plan.describe()["reductions"] == 1
    src = plan.source()
    assert src.count("p_out[oi]") == 5  # one level store per column tile
    assert "acc = (acc + (" in src and ">= 0)) ?" not in src.split("acc = (acc")[1].split("\n")[0]
    assert len(GenericPlan.compile(src)) > 1000


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
@pytest.mark.parametrize("width", (17, 256, 1025))
def test_tiled_reduction_loop_runtime(dtype, width):
    # reference tests/test_tiled_reduction_loops.py:46-68
    kernel = ninetoothed.make(tiled_arrangement, tiled_normalize, (Tensor(2, other=0), Tensor(2)), max_num_configs=1)
    x = torch.randn((7, width * 2), device="cuda", dtype=dtype)[:, ::2]
    out = torch.empty((7, width), device="cuda", dtype=dtype)
    kernel(x, out)
    expected = x.float() * torch.rsqrt(x.float().square().mean(dim=1, keepdim=True) + 1e-5)
    torch.testing.assert_close(out, expected.to(dtype))


# ------------------------------------------------------------------ loops beyond the unroll limit (real loops)
def counted_normalize(x, n, out):
    # a run-time trip count: the first n column tiles of each row, scaled by a weight that
    # an inner loop counts up (a loop nested in a loop, both with run-time trip counts)
    accumulator = ntl.zeros(x.dtype.shape, dtype=ntl.float32)
    for i in range(n):
        weight = 0.0
        for j in range(n):
            weight = weight + 0.5
        accumulator += ntl.cast(x[i], ntl.float32) * weight
    total = ntl.sum(accumulator)
    for i in range(x.shape[0]):
        out[i] = x[i] * 0 + total


def _counted():
    return ninetoothed.make(lambda x, n, out: (tiled_arrangement(x, out)[0], n, tiled_arrangement(x, out)[1]),
                            counted_normalize, (Tensor(2, other=0), Tensor(0), Tensor(2)))


def test_long_tiled_loop_is_a_loop():
    # 70 column tiles of 256: beyond the unroll limit, so the kernel loops; the carried
    # accumulator lives in two LDS buffers, and each row's level stores sit inside the loop
    k = ninetoothed.make(tiled_arrangement, tiled_normalize, (Tensor(2, other=0), Tensor(2)))
    plan = _plan(k, torch.empty((3, 256 * 70)), torch.empty((3, 256 * 70)))
    assert plan.describe()["family"] == "generic" and plan.nest is not None
    src = plan.source()
    assert src.count("for (long long li") == 2 and src.count("p_out[oi]") == 1
    assert "__shared__ float c0_accumulator[512]" in src
    assert len(GenericPlan.compile(src)) > 1000
    # up to the limit the loops are unrolled (no carried buffers)
    plan = _plan(k, torch.empty((3, 256 * 64)), torch.empty((3, 256 * 64)))
    assert plan.nest is None and "for (long long li" not in plan.source()


def test_run_time_trip_counts_and_nested_loops_compile():
    plan = _plan(_counted(), torch.empty((2, 1000)), 3, torch.empty((2, 1000)))
    src = plan.source()
    assert plan.nest is not None and "const long long n0 = s_n;" in src and "const long long n1 = s_n;" in src
    assert "__shared__ float c1_weight[2]" in src  # the inner loop's scalar, carried in its own buffers
    assert len(GenericPlan.compile(src)) > 1000


def test_loop_rejections():
    # a value computed inside a loop may not be stored to a whole arranged output
    def stored_inside(x, out):
        for i in range(x.shape[0]):
            y = x[i] * 2
        out = y  # noqa: F841

    k = ninetoothed.make(lambda x, out: (tiled_arrangement(x, out)[0], out.tile((1, 256))), stored_inside,
                         (Tensor(2), Tensor(2)))
    with pytest.raises(ninetoothed.LoweringError):
        _plan(k, torch.empty((3, 256 * 70)), torch.empty((3, 256)))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
@pytest.mark.parametrize("width", (256 * 64 + 1, 40000))
def test_long_tiled_reduction_loop_runtime(dtype, width):
    # the reference's tiled reduction program (tests/test_tiled_reduction_loops.py:46-68) on
    # rows of 65 and 157 column tiles: real loops, checked against the reference test's formula
    kernel = ninetoothed.make(tiled_arrangement, tiled_normalize, (Tensor(2, other=0), Tensor(2)), max_num_configs=1)
    x = torch.randn((7, width * 2), device="cuda", dtype=dtype)[:, ::2]
    out = torch.empty((7, width), device="cuda", dtype=dtype)
    kernel(x, out)
    expected = x.float() * torch.rsqrt(x.float().square().mean(dim=1, keepdim=True) + 1e-5)
    torch.testing.assert_close(out, expected.to(dtype))


@pytest.mark.gpu
def test_run_time_trip_counts_and_nested_loops():
    kernel = _counted()
    x = torch.randn((5, 3000), device="cuda")
    for n in (0, 1, 4, 14):  # the row has 12 tiles: 14 reads two tiles past it (masked to zero)
        out = torch.full_like(x, -1.0)
        kernel(x, n, out)
        expected = (x[:, :256 * n].sum(dim=1, keepdim=True) * (0.5 * n)).expand_as(x)
        torch.testing.assert_close(out, expected, rtol=1e-5, atol=1e-3)


@pytest.mark.gpu
def test_long_overlapping_k_loop_matmul():
    # the overlapping k-tiles program with K = 576: 71 k-tiles, each an fp32 dot, in a real
    # loop (checked against the oracle's evaluation of the same arrangement)
    import programs as pg

    def overlap(lhs, rhs, output, BM=16, BN=16, BK=16):
        out = output.tile((BM, BN))
        lt = lhs.tile((BM, BK), strides=(-1, 8)).tile((1, -1)).expand((-1, out.shape[1]))
        lt.dtype = lt.dtype.squeeze(0)
        rt = rhs.tile((BK, BN), strides=(8, -1)).tile((-1, 1)).expand((out.shape[0], -1))
        rt.dtype = rt.dtype.squeeze(1)
        return lt, rt, out

    g = torch.Generator().manual_seed(23)
    a = (torch.randn(32, 576, generator=g) / 8).half().cuda()
    b = (torch.randn(576, 48, generator=g) / 8).half().cuda()
    out = torch.empty(32, 48, dtype=torch.float16, device="cuda")
    h = ninetoothed.make(overlap, pg.matmul_application, pg.matmul_tensors())
    assert _plan(h, a, b, out).nest is not None
    h(a, b, out)
    from oracle import apply

    ref = apply.matmul(a.float().cpu().numpy(), b.float().cpu().numpy(), "float16", overlap, block=(16, 16, 16))
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref), rtol=1e-2, atol=1e-2)


# ------------------------------------------------------------------ tile programs that update a tensor they read
def inplace_center(x):
    x = x - ntl.max(x)  # noqa: F841


def inplace_reverse(x):
    # each element takes its row's mirror element: another lane's, so the loads must all
    # happen before the first write
    x = x.source[x.offsets(0)[:, None], (x.source.shape[1] - 1 - x.offsets(1))[None, :]]  # noqa: F841


def _rows(app):
    return ninetoothed.make(lambda x, BW=Symbol("BW", meta=True): (x.tile((1, BW)),), app, (Tensor(2),))


def test_inplace_tile_programs_stage_their_stores():
    for app in (inplace_center, inplace_reverse):
        plan = _plan(_rows(app), torch.empty((4, 300), dtype=torch.float16), BW=512)
        src = plan.source()
        assert plan.inplace and "__shared__ unsigned short stage_x[512]" in src
        compute, write = src.split("stage_x[j] = ")[1], src.split("p_x[oi] = stage_x[j];")[0]
        assert "__syncthreads();" in compute.split("p_x[oi]")[0] and "p_x[oi] = st_f16" not in write
        assert len(GenericPlan.compile(src)) > 1000


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.float32))
def test_inplace_tile_programs(dtype):
    g = torch.Generator().manual_seed(24)
    x0 = torch.randn(6, 300, generator=g).to(dtype).cuda()
    x = x0.clone()
    _rows(inplace_center)(x, BW=512)
    torch.testing.assert_close(x, (x0.float() - x0.float().max(dim=1, keepdim=True).values).to(dtype))
    x = x0.clone()
    _rows(inplace_reverse)(x, BW=512)
    assert torch.equal(x, x0.flip(1))
    x, out = x0.clone(), torch.empty_like(x0)
    _reduce_kernel(row_arrangement, inplace_two_outputs, 2, 2)(x, out, WIDTH=512)
    centred = (x0.float() - x0.float().max(dim=1, keepdim=True).values).to(dtype)
    torch.testing.assert_close(x, centred)
    torch.testing.assert_close(out, centred)


# ------------------------------------------------------------------ libdevice (reference tests/test_libdevice_calls.py)
def fmod_application(x, y, out):
    out = ntl.libdevice.fmod(x, y)  # noqa: F841


def fmod_reduction_application(x, y, out):
    out = ntl.sum(ntl.libdevice.fmod(x, y), axis=1)  # noqa: F841


@pytest.mark.gpu
def test_fmod_boundary_values():
    kernel = ninetoothed.make(lambda x, y, o: (x.tile((32,)), y.tile((32,)), o.tile((32,))), fmod_application,
                              (Tensor(1), Tensor(1), Tensor(1)), max_num_configs=1)
    y = torch.linspace(0.5, 3.5, 4096, device="cuda")
    x = torch.nextafter(17 * y, torch.full_like(y, -float("inf")))
    x[::2] = -x[::2]
    y[::3] = -y[::3]
    out = torch.full_like(x, -12345)
    kernel(x, y, out)
    torch.testing.assert_close(out, torch.fmod(x, y), atol=0, rtol=0)


@pytest.mark.gpu
def test_libdevice_call_inside_reduction():
    kernel = ninetoothed.make(lambda x, y, o: (x.tile((1, 32)), y.tile((1, 32)), o.tile((1,))),
                              fmod_reduction_application, (Tensor(2), Tensor(2, other=1.0), Tensor(1)),
                              max_num_configs=1)
    x = torch.randn((3, 32), device="cuda")
    y = torch.rand_like(x) + 0.5
    out = torch.full((3,), -12345.0, device="cuda")
    kernel(x, y, out)
    torch.testing.assert_close(out, torch.fmod(x, y).sum(1))


def app_axpy(x, y, out):
    out = x * 2.0 + y  # noqa: F841


def test_same_layout_operands_walk_memory_order():
    # 2-D tiles of three same-layout tensors: one permutation table for all -> no tables read
    k = ninetoothed.make(lambda x, y, o: (x.tile((16, 32)), y.tile((16, 32)), o.tile((16, 32))), app_axpy,
                         (Tensor(2), Tensor(2), Tensor(2)))
    v = torch.empty(70, 90)
    plan = _plan(k, v, v, v)
    (src,) = plan.sources_for({"x": v, "y": v, "out": v})
    body = src.split("nt_generic(")[1]
    assert "t_x[e]" not in body and "t_out[e]" not in body and "(e < 6300LL" in body
    # a transposed operand keeps its table
    w = torch.empty(90, 70).t()
    (src,) = plan.sources_for({"x": w, "y": v, "out": v})
    assert "t_x[e]" in src


@pytest.mark.gpu
def test_two_d_tiled_elementwise():
    k = ninetoothed.make(lambda x, y, o: (x.tile((16, 32)), y.tile((16, 32)), o.tile((16, 32))), app_axpy,
                         (Tensor(2), Tensor(2), Tensor(2)))
    x, y = torch.randn(70, 90, device="cuda"), torch.randn(70, 90, device="cuda")
    out = torch.empty_like(x)
    k(x, y, out)
    assert torch.equal(out, x * 2.0 + y)
    xt = torch.randn(90, 70, device="cuda").t()
    k(xt, y, out)
    assert torch.equal(out, xt * 2.0 + y)


# ------------------------------------------------------------------ dot in tile programs
# ``ntl.dot`` outside a GEMM loop: a tile program runs it as an fp32 reduction over the
# shared axis of a broadcast product (as the reference's ``tl.dot``, fp32 accumulation).
DOT_BM = Symbol("DOT_BM", constexpr=True)


def dot_arrangement(x, w, o):
    xt = x.tile((DOT_BM, -1))
    return xt, w.tile((-1, -1)).expand((xt.shape[0], -1)), o.tile((DOT_BM, -1))


def dot_rows_arrangement(x, w, o):
    xt = x.tile((DOT_BM, -1))
    return xt, w.tile((-1, -1)).expand((xt.shape[0], -1)), o.tile((DOT_BM,))


def dot_application(x, w, o):
    o = ntl.dot(x, w)  # noqa: F841


def dot_trans_application(x, w, o):
    o = ntl.dot(x, ntl.trans(w)) * 0.5 + 1.0  # noqa: F841


def dot_row_sum_application(x, w, o):
    o = ntl.sum(ntl.dot(x, w), axis=1)  # noqa: F841


def test_dot_tile_programs_compile():
    cases = ((dot_arrangement, dot_application, ((64, 40), (40, 24), (64, 24))),
             (dot_arrangement, dot_trans_application, ((64, 40), (24, 40), (64, 24))),
             (dot_rows_arrangement, dot_row_sum_application, ((64, 40), (40, 24), (64,))))
    for arrangement, application, shapes in cases:
        h = ninetoothed.make(arrangement, application, tuple(Tensor(len(s)) for s in shapes))
        plan = _plan(h, *(torch.empty(s) for s in shapes), DOT_BM=16)
        assert plan.describe()["family"] == "generic" and plan.describe()["reductions"] >= 1
        assert len(GenericPlan.compile(plan.source())) > 1000


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_dot_tile_programs(dtype):
    tol = 1e-2 if dtype != torch.float32 else 1e-4
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(64, 40, generator=g) / 4).to(dtype).cuda()
    w = (torch.randn(40, 24, generator=g) / 4).to(dtype).cuda()
    ref = x.float() @ w.float()
    # dot alone, and with an epilogue on a transposed operand
    o = torch.empty(64, 24, dtype=dtype, device="cuda")
    ninetoothed.make(dot_arrangement, dot_application, (Tensor(2), Tensor(2), Tensor(2)))(x, w, o, DOT_BM=16)
    torch.testing.assert_close(o.float(), ref, rtol=tol, atol=tol)
    wt = w.t().contiguous()
    o2 = torch.empty(64, 24, dtype=torch.float32, device="cuda")
    ninetoothed.make(dot_arrangement, dot_trans_application, (Tensor(2), Tensor(2), Tensor(2)))(x, wt, o2, DOT_BM=32)
    torch.testing.assert_close(o2, ref * 0.5 + 1.0, rtol=tol, atol=tol)
    # dot then a reduction of its result (row sums)
    rows = torch.empty(64, dtype=torch.float32, device="cuda")
    ninetoothed.make(dot_rows_arrangement, dot_row_sum_application, (Tensor(2), Tensor(2), Tensor(1)))(x, w, rows,
                                                                                                      DOT_BM=16)
    torch.testing.assert_close(rows, ref.sum(dim=1), rtol=tol, atol=tol * 8)


def dot_tt_arrangement(x, w, o):
    # x [K, M] in column tiles (programs along M), w [N, K] whole, o [M, N] in row tiles
    xt = x.tile((-1, DOT_BM)).permute((1, 0))
    return xt, w.tile((-1, -1)).expand((xt.shape[0], -1)), o.tile((DOT_BM, -1))


def dot_tt_application(x, w, o):
    o = ntl.dot(ntl.trans(x), ntl.trans(w))  # noqa: F841


def test_dot_of_two_transposed_tiles_compiles():
    # fp32 operands: the fp32 reduction over a [k, m, n] product, w's factor broadcast with its
    # axes permuted; 16-bit operands on the 32 x 32 x 16 grid: the matrix core, both staged by
    # axis order
    h = ninetoothed.make(dot_tt_arrangement, dot_tt_application, (Tensor(2), Tensor(2), Tensor(2)))
    for dtype, mfma in ((torch.float32, False), (torch.float16, True)):
        plan = _plan(h, torch.empty((64, 128), dtype=dtype), torch.empty((96, 64), dtype=dtype),
                     torch.empty(128, 96), DOT_BM=32)
        assert plan.describe()["family"] == "generic"
        src = plan.source()
        assert ("mfma" in src) == mfma
        assert len(GenericPlan.compile(src)) > 1000


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, torch.bfloat16))
def test_dot_of_two_transposed_tiles(dtype):
    g = torch.Generator().manual_seed(27)
    x = (torch.randn(64, 128, generator=g) / 4).to(dtype).cuda()  # [K, M]
    w = (torch.randn(96, 64, generator=g) / 4).to(dtype).cuda()   # [N, K]
    ref = x.float().t() @ w.float().t()
    o = torch.empty(128, 96, dtype=torch.float32, device="cuda")
    ninetoothed.make(dot_tt_arrangement, dot_tt_application, (Tensor(2), Tensor(2), Tensor(2)))(x, w, o, DOT_BM=32)
    tol = 1e-4 if dtype == torch.float32 else 1e-4 * 8
    torch.testing.assert_close(o, ref, rtol=tol, atol=tol)  # 16-bit products are exact, sums fp32


DOT_K, DOT_N = Symbol("DOT_K", meta=True), Symbol("DOT_N", meta=True)


def dot_padded_arrangement(x, w, o):
    # one k-tile of DOT_K over a K that may be shorter (masked columns of x, rows of w)
    xt = x.tile((DOT_BM, DOT_K))
    return xt, w.tile((DOT_K, DOT_N)).expand((xt.shape[0], -1)), o.tile((DOT_BM, DOT_N))


def test_matrix_core_dot_programs_compile():
    # 16-bit operands with M, N multiples of 32 and K of 16: the dot runs on the matrix core
    cases = ((dot_application, (128, 64), (64, 96), "f16", torch.float16),
             (dot_trans_application, (128, 64), (96, 64), "bf16", torch.bfloat16))
    for application, sx, sw, suffix, dtype in cases:
        h = ninetoothed.make(dot_arrangement, application, (Tensor(2), Tensor(2), Tensor(2)))
        plan = _plan(h, torch.empty(sx, dtype=dtype), torch.empty(sw, dtype=dtype), torch.empty(128, 96), DOT_BM=32)
        src = plan.source()
        assert f"__builtin_amdgcn_mfma_f32_32x32x16_{suffix}" in src and "__shared__ float red0[3072]" in src
        assert len(GenericPlan.compile(src)) > 1000
    # shapes off the 32 x 32 x 16 grid run on the matrix core zero-padded to it; fp32 operands
    # keep the fp32 reduction
    h = ninetoothed.make(dot_arrangement, dot_application, (Tensor(2), Tensor(2), Tensor(2)))
    for dtype, sw, mfma in ((torch.float32, (64, 96), False), (torch.float16, (64, 24), True),
                            (torch.bfloat16, (40, 24), True)):
        plan = _plan(h, torch.empty((128, sw[0]), dtype=dtype), torch.empty(sw, dtype=dtype), torch.empty(128, sw[1]),
                     DOT_BM=32)
        src = plan.source()
        assert ("mfma" in src) == mfma
        assert len(GenericPlan.compile(src)) > 1000


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("shape", ((48, 40, 20), (16, 40, 24), (96, 8, 72)))
def test_matrix_core_dot_off_the_grid(dtype, shape):
    # M, N off multiples of 32 and K off 16: operands zero-padded in LDS, results inside [M, N]
    bm, k, n = shape
    g = torch.Generator().manual_seed(29)
    x = (torch.randn(2 * bm, k, generator=g) / 4).to(dtype).cuda()
    w = (torch.randn(k, n, generator=g) / 4).to(dtype).cuda()
    o = torch.full((2 * bm, n), float("nan"), dtype=torch.float32, device="cuda")
    h = ninetoothed.make(dot_arrangement, dot_application, (Tensor(2), Tensor(2), Tensor(2)))
    assert "mfma" in _plan(h, x, w, o, DOT_BM=bm).source()
    h(x, w, o, DOT_BM=bm)
    torch.testing.assert_close(o, x.float() @ w.float(), rtol=1e-4, atol=1e-4)  # exact products, fp32 sums


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_matrix_core_dot_programs(dtype):
    g = torch.Generator().manual_seed(25)
    x = (torch.randn(128, 64, generator=g) / 4).to(dtype).cuda()
    w = (torch.randn(64, 96, generator=g) / 4).to(dtype).cuda()
    ref = x.float() @ w.float()
    o = torch.empty(128, 96, dtype=torch.float32, device="cuda")
    ninetoothed.make(dot_arrangement, dot_application, (Tensor(2), Tensor(2), Tensor(2)))(x, w, o, DOT_BM=32)
    torch.testing.assert_close(o, ref, rtol=1e-4, atol=1e-4)  # exact products, fp32 sums
    o2 = torch.empty(128, 96, dtype=dtype, device="cuda")
    ninetoothed.make(dot_arrangement, dot_trans_application, (Tensor(2), Tensor(2), Tensor(2)))(
        x, w.t().contiguous(), o2, DOT_BM=64)
    torch.testing.assert_close(o2.float(), (ref * 0.5 + 1.0).to(dtype).float(), rtol=1e-2, atol=1e-2)
    # K = 50 in one 64-deep k-tile: the masked columns of x (other = 1) and rows of w
    # take no part, as in the reference's dot emitter
    xp = (torch.randn(96, 50, generator=g) / 4).to(dtype).cuda()
    wp = (torch.randn(50, 64, generator=g) / 4).to(dtype).cuda()
    op = torch.empty(96, 64, dtype=torch.float32, device="cuda")
    ninetoothed.make(dot_padded_arrangement, dot_application, (Tensor(2, other=1.0), Tensor(2, other=1.0), Tensor(2)))(
        xp, wp, op, DOT_BM=32, DOT_K=64, DOT_N=64)
    torch.testing.assert_close(op, xp.float() @ wp.float(), rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
def test_matrix_core_dot_in_a_long_loop():
    # the overlapping k-tiles matmul with 32 x 32 x 16 tiles and K = 576: 71 matrix-core dots
    # in a real loop (checked against the oracle's evaluation of the same arrangement)
    import programs as pg

    def overlap(lhs, rhs, output, BM=32, BN=32, BK=16):
        out = output.tile((BM, BN))
        lt = lhs.tile((BM, BK), strides=(-1, 8)).tile((1, -1)).expand((-1, out.shape[1]))
        lt.dtype = lt.dtype.squeeze(0)
        rt = rhs.tile((BK, BN), strides=(8, -1)).tile((-1, 1)).expand((out.shape[0], -1))
        rt.dtype = rt.dtype.squeeze(1)
        return lt, rt, out

    g = torch.Generator().manual_seed(26)
    a = (torch.randn(64, 576, generator=g) / 8).half().cuda()
    b = (torch.randn(576, 96, generator=g) / 8).half().cuda()
    out = torch.empty(64, 96, dtype=torch.float16, device="cuda")
    h = ninetoothed.make(overlap, pg.matmul_application, pg.matmul_tensors())
    plan = _plan(h, a, b, out)
    assert plan.nest is not None and "mfma_f32_32x32x16_f16" in plan.source()
    h(a, b, out)
    from oracle import apply

    ref = apply.matmul(a.float().cpu().numpy(), b.float().cpu().numpy(), "float16", overlap, block=(32, 32, 16))
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref), rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_overlapping_k_tiles_matmul_runs_as_written():
    # k-tiles of size 16 at stride 8 (each k visited twice, the last tiles masked past K):
    # not a GEMM, so the generic kernels run the loop as the program states.
    import programs as pg

    def overlap(lhs, rhs, output, BM=16, BN=16, BK=16):
        out = output.tile((BM, BN))
        lt = lhs.tile((BM, BK), strides=(-1, 8)).tile((1, -1)).expand((-1, out.shape[1]))
        lt.dtype = lt.dtype.squeeze(0)
        rt = rhs.tile((BK, BN), strides=(8, -1)).tile((-1, 1)).expand((out.shape[0], -1))
        rt.dtype = rt.dtype.squeeze(1)
        return lt, rt, out

    g = torch.Generator().manual_seed(22)
    a = (torch.randn(32, 48, generator=g) / 4).half().cuda()
    b = (torch.randn(48, 64, generator=g) / 4).half().cuda()
    out = torch.empty(32, 64, dtype=torch.float16, device="cuda")
    ninetoothed.make(overlap, pg.matmul_application, pg.matmul_tensors())(a, b, out)
    from oracle import apply

    # the oracle evaluates the same arrangement: five k-tiles, at k = 0, 8, ..., 32
    ref = apply.matmul(a.float().cpu().numpy(), b.float().cpu().numpy(), "float16", overlap, block=(16, 16, 16))
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref), rtol=1e-2, atol=1e-2)
    five = sum(a[:, 8 * t:8 * t + 16].float() @ b[8 * t:8 * t + 16, :].float() for t in range(5))
    torch.testing.assert_close(out.float(), five.half().float(), rtol=1e-2, atol=1e-2)


# ------------------------------------------------------------------ a whole output assigned inside a real loop
def assigned_each_iteration(x, n, out):
    for i in range(n):
        out = x * 2.0 + i  # noqa: F841  (every iteration stores; the last one stays)


def _assigned_each_iteration():
    return ninetoothed.make(lambda x, n, out: (x.tile((BS,)), n, out.tile((BS,))), assigned_each_iteration,
                            (Tensor(1), Tensor(0), Tensor(1)))


def test_output_assigned_inside_a_loop_compiles():
    plan = _plan(_assigned_each_iteration(), torch.empty(1000), 5, torch.empty(1000), BS=256)
    assert plan.describe()["family"] == "generic" and plan.nest is not None
    src = plan.source()
    assert "store into out[]" in src and len(GenericPlan.compile(src)) > 1000


@pytest.mark.gpu
def test_output_assigned_inside_a_loop():
    kernel = _assigned_each_iteration()
    x = torch.randn(1000, device="cuda")
    for n in (0, 1, 7):
        out = torch.full_like(x, -3.0)
        kernel(x, n, out, BS=256)
        expected = torch.full_like(x, -3.0) if n == 0 else x * 2.0 + (n - 1)
        torch.testing.assert_close(out, expected)


def assigned_in_unrolled_loop(x, out):
    for i in range(3):
        out = x * 2.0 + i  # noqa: F841


@pytest.mark.gpu
def test_output_assigned_in_an_unrolled_loop():
    kernel = ninetoothed.make(lambda x, out: (x.tile((BS,)), out.tile((BS,))), assigned_in_unrolled_loop,
                              (Tensor(1), Tensor(1)))
    x = torch.randn(1000, device="cuda")
    out = torch.empty_like(x)
    kernel(x, out, BS=128)
    torch.testing.assert_close(out, x * 2.0 + 2)
