"""The allocation-free conv2d entry point against the workspace entry point (both through the C ABI).

nt_conv2d_noalloc_* runs the same kernels as nt_conv2d_* with a caller-provided workspace,
so the outputs must be identical bit for bit.  Two calls in a row on the shared static
scratch, the second with a smaller input (whatever the first left in the scratch must not
leak into the second), then a shape whose re-layout needs more than the static scratch,
which is refused before anything is launched.
"""

import ctypes

import pytest
import torch

from ninetoothed_amd import _lib

DEV = "cuda"
SCRATCH_BYTES = 32 << 20  # NT_CONV2D_SCRATCH_BYTES
NT_ERR_SCRATCH = 2


def _i64(values):
    return _lib.int64_array(values)


def _args(x, w, y, pad):
    n, c, h, wd = x.shape
    k, _, r, s = w.shape
    p, q = y.shape[2], y.shape[3]
    return [x.data_ptr(), _i64(x.stride()), w.data_ptr(), _i64(w.stride()), y.data_ptr(), _i64(y.stride()),
            _lib.dtype_code(y.dtype), n, c, h, wd, k, r, s, p, q, pad, pad, 1, 1, 1, 1, _lib.dtype_code(y.dtype)]


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _with_workspace(x, w, y, pad):
    lib = _lib.load()
    suffix = _lib.dtype_suffix(x.dtype)
    n, c, h, wd = x.shape
    k, _, r, s = w.shape
    need = lib.nt_conv2d_workspace_size(n, c, h, wd, k, r, s, pad, pad, _lib.dtype_code(x.dtype))
    assert 0 < need <= SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    code = getattr(lib, f"nt_conv2d_{suffix}")(*_args(x, w, y, pad), ws.data_ptr(), need, _stream())
    assert code == 0
    return ws


def _no_alloc(x, w, y, pad):
    lib = _lib.load()
    return getattr(lib, f"nt_conv2d_noalloc_{_lib.dtype_suffix(x.dtype)}")(*_args(x, w, y, pad), _stream())


def _case(shape, k, pad, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g).to(dtype).to(DEV)
    w = (torch.randn(k, shape[1], 3, 3, generator=g) / (shape[1] * 9) ** 0.5).to(dtype).to(DEV)
    p, q = shape[2] + 2 * pad - 2, shape[3] + 2 * pad - 2
    return x, w, p, q


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_no_alloc_matches_the_workspace_entry_point(dtype):
    # The headline conv2d shape (a 28.7 MB re-layout), then a smaller one on the same scratch.
    for shape, k, pad, seed in (((16, 256, 56, 56), 256, 1, 100), ((2, 64, 20, 24), 128, 1, 101)):
        x, w, p, q = _case(shape, k, pad, dtype, seed)
        print(f"no-alloc conv2d {tuple(shape)} k={k} pad={pad} {dtype}", flush=True)
        ref = torch.full((shape[0], k, p, q), float("nan"), dtype=dtype, device=DEV)
        got = torch.full_like(ref, float("nan"))
        ws = _with_workspace(x, w, ref, pad)
        assert _no_alloc(x, w, got, pad) == 0
        torch.cuda.synchronize()
        del ws
        assert torch.equal(got, ref), f"max diff {(got.float() - ref.float()).abs().max()}"
        assert not torch.isnan(got.float()).any()


@pytest.mark.gpu
def test_no_alloc_refuses_shapes_beyond_its_scratch():
    # [64, 256, 56, 56] needs 64 * 58 * 58 * 256 * 2 + ... > 32 MiB: refused on the host.
    x = torch.empty(64, 256, 56, 56, dtype=torch.float16, device=DEV)
    w = torch.empty(256, 256, 3, 3, dtype=torch.float16, device=DEV)
    y = torch.empty(64, 256, 56, 56, dtype=torch.float16, device=DEV)
    assert _no_alloc(x, w, y, 1) == NT_ERR_SCRATCH
