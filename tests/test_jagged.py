"""Jagged tensors (``Tensor(ndim, jagged_dim=...)`` bound to torch nested tensors of the
``torch.jagged`` layout), the reference's tests/test_jagged.py programs.

CPU: the argument contract (jagged_dim range, nested vs strided arguments), the plan a
jagged call takes (the generic kernels) and its index tables against offsets computed
from the batches themselves.  GPU: to_padded_tensor (a jagged input with ``other`` as the
padding, copied into a dense output) and the expand copy (a dense source broadcast into a
jagged destination), against the batches, as the reference checks them.  The reference
draws batch sizes up to 1024 per dim; here they are seeded and up to 256, plus one case at
the full range, because the generic kernels build their index tables on the host.
"""

import functools
import random

import numpy as np
import pytest
import torch

import ninetoothed_amd as ninetoothed
from ninetoothed_amd import Symbol, Tensor

DEV = "cuda"
BLOCK = Symbol("block_size", constexpr=True)


def padded_arrangement(input, output, block_size=BLOCK):
    tile = (1,) + tuple(block_size for _ in range(1, input.ndim))
    return input.tile(tile), output.tile(tile)


def padded_application(input, output):
    output = input  # noqa: F841


def make_to_padded(ndim, padding, jagged_dim):
    tensors = (Tensor(ndim, jagged_dim=jagged_dim, other=padding), Tensor(ndim))
    return ninetoothed.make(padded_arrangement, padded_application, tensors)


def copy_arrangement(dst, src, jagged_dim, block_size=BLOCK):
    tile = (1,) + tuple(block_size for _ in range(1, dst.ndim))
    sizes = tuple(-1 if d != jagged_dim else dst.shape[d] for d in range(src.ndim))
    return dst.tile(tile), src.expand(sizes).tile(tile)


def copy_application(dst, src):
    dst = src  # noqa: F841


def make_copy(ndim, jagged_dim):
    tensors = (Tensor(ndim, jagged_dim=jagged_dim), Tensor(ndim))
    return ninetoothed.make(functools.partial(copy_arrangement, jagged_dim=jagged_dim), copy_application, tensors)


def _batches(ndim, jagged_dim, num_batches, seed, upper=256, device="cpu"):
    rng = random.Random(seed)
    shape = tuple(rng.randint(1, upper) for _ in range(ndim - 1))
    g = torch.Generator().manual_seed(seed)
    return tuple(
        torch.randn(shape[: jagged_dim - 1] + (rng.randint(1, upper),) + shape[jagged_dim:], generator=g).to(device)
        for _ in range(num_batches)
    )


def _padded_reference(batches, shape, padding, jagged_dim):
    expected = torch.full(shape, padding, dtype=batches[0].dtype)
    for b, batch in enumerate(batches):
        index = [b] + [slice(None)] * (len(shape) - 1)
        index[jagged_dim] = slice(0, batch.shape[jagged_dim - 1])
        expected[tuple(index)] = batch.cpu()
    return expected


def _plan(handle, *args, **meta):
    names = handle._abi["public_args"]
    return handle._kernel.specialize(dict(zip(names, args)), meta)


# ------------------------------------------------------------------------------- CPU
def test_jagged_dim_must_follow_the_batch_dim():
    Tensor(3, jagged_dim=1)
    Tensor(3, jagged_dim=2)
    for bad in (0, 3, -1, 1.0):
        with pytest.raises(ValueError):
            Tensor(3, jagged_dim=bad)


@pytest.mark.parametrize("jagged_dim", (1, 2))
def test_jagged_tables_follow_each_batch(jagged_dim):
    batches = _batches(3, jagged_dim, 5, 7, upper=40)
    nested = torch.nested.nested_tensor(batches, layout=torch.jagged)
    longest = max(b.shape[jagged_dim - 1] for b in batches)
    shape = tuple(longest if d == jagged_dim else int(s) for d, s in enumerate(nested.shape))
    output = torch.empty(shape)
    h = make_to_padded(3, -1.0, jagged_dim)
    plan = _plan(h, nested, output, block_size=16)
    assert plan.describe()["family"] == "generic"
    ti, total = plan._table("input", nested)
    to, _ = plan._table("output", output)
    assert ti.size == to.size == total
    # expected: output element (b, i1, i2) -> its place in values(), or -1 past the batch's rows
    values = nested.values()
    offsets = nested.offsets().numpy()
    expect = np.full(shape, -1, dtype=np.int64)
    for b, batch in enumerate(batches):
        n = batch.shape[jagged_dim - 1]
        grid = np.indices(batch.shape)
        rows = grid[jagged_dim - 1] + offsets[b]
        other = grid[2 - jagged_dim]
        vs = values.stride()
        if jagged_dim == 1:
            off = rows * vs[0] + other * vs[1]
            expect[b, :n, :] = off
        else:
            off = other * vs[0] + rows * vs[1]
            expect[b, :, :n] = off
    valid = to >= 0
    assert np.count_nonzero(valid) == output.numel()
    got = np.full(output.numel(), -2, dtype=np.int64)
    got[to[valid]] = ti[valid]
    assert np.array_equal(got.reshape(shape), expect)


def test_jagged_arguments_are_checked():
    h = make_to_padded(3, -1.0, 1)
    dense = torch.empty(2, 4, 4)
    with pytest.raises(TypeError, match="jagged nested tensor ragged in dimension 1"):
        h(dense, torch.empty(2, 4, 4), block_size=16)
    nested = torch.nested.nested_tensor(_batches(3, 2, 2, 3, upper=8), layout=torch.jagged)
    with pytest.raises(TypeError, match="ragged in dimension 1"):
        h(nested, torch.empty(2, 8, 8), block_size=16)  # ragged in dim 2, declared 1
    plain = ninetoothed.make(padded_arrangement, padded_application, (Tensor(3), Tensor(3)))
    nested1 = torch.nested.nested_tensor(_batches(3, 1, 2, 3, upper=8), layout=torch.jagged)
    with pytest.raises(TypeError, match="strided tensor"):
        plain(nested1, torch.empty(2, 8, 8), block_size=16)


# ------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("padding", (-1,))
@pytest.mark.parametrize("num_batches", (2, 3, 7, 16))
@pytest.mark.parametrize("jagged_dim", (1, 2))
def test_to_padded_tensor(jagged_dim, num_batches, padding):
    batches = _batches(3, jagged_dim, num_batches, 100 * jagged_dim + num_batches, device=DEV)
    nested = torch.nested.nested_tensor(batches, layout=torch.jagged)
    longest = int(nested.offsets().diff().max())
    shape = tuple(longest if d == jagged_dim else int(s) for d, s in enumerate(nested.shape))
    output = torch.empty(shape, device=DEV)
    make_to_padded(3, padding, jagged_dim)(nested, output, block_size=32)
    expected = _padded_reference(batches, shape, padding, jagged_dim)
    assert torch.equal(output.cpu(), expected)


@pytest.mark.gpu
def test_to_padded_tensor_full_range():
    batches = _batches(3, 1, 3, 2024, upper=1024, device=DEV)
    nested = torch.nested.nested_tensor(batches, layout=torch.jagged)
    longest = int(nested.offsets().diff().max())
    shape = (3, longest, int(nested.shape[2]))
    output = torch.empty(shape, device=DEV)
    make_to_padded(3, -1, 1)(nested, output, block_size=32)
    assert torch.equal(output.cpu(), _padded_reference(batches, shape, -1, 1))


@pytest.mark.gpu
@pytest.mark.parametrize("num_batches", (2, 3, 7, 16))
@pytest.mark.parametrize("jagged_dim", (1, 2))
def test_expand(jagged_dim, num_batches):
    batches = _batches(3, jagged_dim, num_batches, 300 * jagged_dim + num_batches, device=DEV)
    dst = torch.nested.nested_tensor(batches, layout=torch.jagged)
    src = torch.randn(tuple(int(s) if d != jagged_dim else 1 for d, s in enumerate(dst.shape)), device=DEV)
    make_copy(3, jagged_dim)(dst, src, block_size=32)
    for b, actual in enumerate(dst.unbind()):
        assert torch.equal(actual, src[b].expand_as(actual))


@pytest.mark.gpu
def test_jagged_calls_with_new_offsets_each_time():
    # one handle, three calls whose batches differ in number and length: the index tables
    # follow each call's offsets (a jagged call is never served from the bound-launcher cache)
    h = make_to_padded(3, -1, 1)
    for seed, n in ((1, 2), (2, 5), (3, 2)):
        batches = _batches(3, 1, n, seed, upper=64, device=DEV)
        nested = torch.nested.nested_tensor(batches, layout=torch.jagged)
        longest = int(nested.offsets().diff().max())
        shape = (n, longest, int(nested.shape[2]))
        output = torch.empty(shape, device=DEV)
        h(nested, output, block_size=32)
        assert torch.equal(output.cpu(), _padded_reference(batches, shape, -1, 1))
