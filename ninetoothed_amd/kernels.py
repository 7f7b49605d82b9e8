"""Tensor-level launchers over the C ABI of libnt_mi355x.so.

Each function takes PyTorch-ROCm tensors that already live on the GPU, checks
what the kernel assumes (device, dtype, rank, sizes), and calls the matching
``nt_*`` entry point on the caller's current stream.  Nothing here computes on the
CPU and nothing falls back: an unsupported case raises, a non-zero status from the
library raises :class:`KernelLaunchError` (the reference's error type,
``src/ninetoothed/compiler/runtime.py:31-35``).
"""

import ctypes

from ninetoothed_amd import _lib
from ninetoothed_amd.errors import KernelLaunchError

LOG2E = 1.44269504089


def _check_device(*tensors):
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise TypeError("MI355X kernels need tensors on the GPU (torch device type `cuda`).")
        if device is None:
            device = t.device
        elif t.device != device:
            raise TypeError("All tensor arguments must use the same GPU.")
    return device


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _status(code, name):
    if code != 0:
        raise KernelLaunchError(code, name)


def add(lhs, rhs, out):
    """out = lhs + rhs over 1-D tensors of equal length (any strides)."""
    _check_device(lhs, rhs, out)
    if not (lhs.dim() == rhs.dim() == out.dim() == 1):
        raise ValueError("add expects 1-D tensors")
    n = out.shape[0]
    if lhs.shape[0] != n or rhs.shape[0] != n:
        raise ValueError("add operands differ in length")
    if not (lhs.dtype == rhs.dtype == out.dtype):
        raise TypeError("add operands must share one dtype")
    lib = _lib.load()
    fn = getattr(lib, f"nt_add_{_lib.dtype_suffix(out.dtype)}")
    with_stream = _lib.current_stream(out.device)
    _status(fn(_ptr(lhs), lhs.stride(0), _ptr(rhs), rhs.stride(0), _ptr(out), out.stride(0), n, with_stream), fn.__name__)
    return out


def softmax(x, y, block=None):
    """Row softmax of a 2-D tensor over segments of ``block`` columns (default: whole rows)."""
    _check_device(x, y)
    if x.dim() != 2 or y.shape != x.shape:
        raise ValueError("softmax expects matching 2-D tensors")
    if x.dtype != y.dtype:
        raise TypeError("softmax input and output must share one dtype")
    rows, cols = x.shape
    block = cols if block is None else int(block)
    if cols > 1 and (x.stride(1) != 1 or y.stride(1) != 1):
        raise ValueError("softmax needs unit column stride")
    lib = _lib.load()
    fn = getattr(lib, f"nt_softmax_{_lib.dtype_suffix(x.dtype)}")
    _status(
        fn(_ptr(x), x.stride(0), x.stride(1), _ptr(y), y.stride(0), y.stride(1), rows, cols, max(block, 1),
           _lib.current_stream(x.device)),
        fn.__name__,
    )
    return y


def max_pool2d(x, y, window, stride=None, padding=(0, 0), dilation=(1, 1)):
    """y = max_pool2d(x) with -inf outside the input (any strides, N-C-H-W indexing)."""
    _check_device(x, y)
    if x.dim() != 4 or y.dim() != 4:
        raise ValueError("max_pool2d expects 4-D tensors")
    if x.dtype != y.dtype:
        raise TypeError("max_pool2d input and output must share one dtype")
    kh, kw = window
    sh, sw = stride if stride is not None else window
    ph, pw = padding
    dh, dw = dilation
    n, c, h, w = x.shape
    if y.shape[0] != n or y.shape[1] != c:
        raise ValueError("max_pool2d batch/channel sizes differ")
    p, q = y.shape[2], y.shape[3]
    lib = _lib.load()
    fn = getattr(lib, f"nt_max_pool2d_{_lib.dtype_suffix(x.dtype)}")
    _status(
        fn(_ptr(x), _lib.int64_array(x.stride()), _ptr(y), _lib.int64_array(y.stride()), n, c, h, w, p, q, kh, kw, sh,
           sw, ph, pw, dh, dw, _lib.current_stream(x.device)),
        fn.__name__,
    )
    return y


def gemm(a, b, out, c=None, alpha=1.0, beta=0.0, round_dtype=None):
    """out = cast(beta * c + alpha * round(a @ b)); fp32 accumulation; any strides."""
    _check_device(a, b, out, c)
    if a.dim() != 2 or b.dim() != 2 or out.dim() != 2:
        raise ValueError("gemm expects 2-D tensors")
    m, k = a.shape
    if b.shape[0] != k or out.shape[0] != m or out.shape[1] != b.shape[1]:
        raise ValueError(f"gemm shape mismatch: {tuple(a.shape)} @ {tuple(b.shape)} -> {tuple(out.shape)}")
    n = b.shape[1]
    if a.dtype != b.dtype:
        raise TypeError("gemm operands must share one dtype")
    if c is not None:
        if tuple(c.shape) != (m, n):
            raise ValueError("gemm bias shape mismatch")
        if c.dtype != out.dtype:
            raise TypeError("gemm bias and output must share one dtype")
    rd = _lib.DTYPE_NONE if round_dtype is None else _lib.dtype_code(round_dtype)
    lib = _lib.load()
    fn = getattr(lib, f"nt_gemm_{_lib.dtype_suffix(a.dtype)}")
    sc = c.stride() if c is not None else (0, 0)
    _status(
        fn(_ptr(a), a.stride(0), a.stride(1), _ptr(b), b.stride(0), b.stride(1), _ptr(c), sc[0], sc[1], _ptr(out),
           out.stride(0), out.stride(1), _lib.dtype_code(out.dtype), m, n, k, float(alpha), float(beta), rd,
           _lib.current_stream(a.device)),
        fn.__name__,
    )
    return out


def conv2d(x, w, y, padding=(0, 0), stride=(1, 1), dilation=(1, 1), round_dtype=None, workspace=None):
    """y = cast(round(conv2d(x, w))) as an implicit GEMM (cross-correlation, zero padding)."""
    _check_device(x, w, y, workspace)
    if x.dim() != 4 or w.dim() != 4 or y.dim() != 4:
        raise ValueError("conv2d expects 4-D tensors")
    if x.dtype != w.dtype:
        raise TypeError("conv2d input and filter must share one dtype")
    n, c, h, wd = x.shape
    k, c2, r, s = w.shape
    if c2 != c or y.shape[0] != n or y.shape[1] != k:
        raise ValueError("conv2d shape mismatch")
    p, q = y.shape[2], y.shape[3]
    ph, pw = padding
    sh, sw = stride
    dh, dw = dilation
    rd = _lib.DTYPE_NONE if round_dtype is None else _lib.dtype_code(round_dtype)
    lib = _lib.load()
    fn = getattr(lib, f"nt_conv2d_{_lib.dtype_suffix(x.dtype)}")
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _status(
        fn(_ptr(x), _lib.int64_array(x.stride()), _ptr(w), _lib.int64_array(w.stride()), _ptr(y),
           _lib.int64_array(y.stride()), _lib.dtype_code(y.dtype), n, c, h, wd, k, r, s, p, q, ph, pw, sh, sw, dh, dw,
           rd, _ptr(workspace), ws_bytes, _lib.current_stream(x.device)),
        fn.__name__,
    )
    return y


def conv2d_workspace_bytes(x, w, padding=(0, 0)):
    lib = _lib.load()
    n, c, h, wd = x.shape
    k, _, r, s = w.shape
    return int(lib.nt_conv2d_workspace_size(n, c, h, wd, k, r, s, padding[0], padding[1], _lib.dtype_code(x.dtype)))


def attention(q, k, v, o, causal=False, q_scale=LOG2E):
    """Flash attention forward of the reference application; q pre-scaled by ``q_scale``."""
    _check_device(q, k, v, o)
    if not (q.dim() == k.dim() == v.dim() == o.dim() == 4):
        raise ValueError("attention expects [B, H, S, D] tensors")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("attention q, k, v must share one dtype")
    bsz, heads, sq, d = q.shape
    sk = k.shape[2]
    if k.shape != (bsz, heads, sk, d) or v.shape != (bsz, heads, sk, d) or o.shape != q.shape:
        raise ValueError("attention shape mismatch")
    if d > 128:
        raise ValueError("attention head dim must be <= 128")
    lib = _lib.load()
    fn = getattr(lib, f"nt_attention_{_lib.dtype_suffix(q.dtype)}")
    _status(
        fn(_ptr(q), _lib.int64_array(q.stride()), _ptr(k), _lib.int64_array(k.stride()), _ptr(v),
           _lib.int64_array(v.stride()), _ptr(o), _lib.int64_array(o.stride()), _lib.dtype_code(o.dtype), bsz, heads,
           sq, sk, d, float(q_scale), 1 if causal else 0, _lib.current_stream(q.device)),
        fn.__name__,
    )
    return o
