"""Tensor-level launchers over the C ABI of libnt_mi355x.so.

Each operation comes in two forms:

- ``bind_<op>(...)`` takes sample tensors, checks what the kernel assumes (device,
  dtype, rank, sizes) and returns a launcher closed over everything that depends
  only on dtypes, shapes and strides (entry point, dims, stride arrays, device).
  A launcher reads only data pointers, scalar values and the caller's current
  stream, so a call costs a few microseconds of host time (the GEMM's about one: its
  constant arguments are packed once for ``nt_gemm_packed``).  Callers re-bind
  whenever a dtype, shape, stride or device changes (``runtime.Handle`` keys its
  cache on exactly those).
- ``<op>(...)`` binds and launches once.

Nothing here computes on the CPU and nothing falls back: an unsupported case
raises, a non-zero status from the library raises :class:`KernelLaunchError` (the
reference's error type, ``src/ninetoothed/compiler/runtime.py:31-35``).
"""

import ctypes
import struct

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


def _stream_of(device):
    """A zero-argument function returning the raw handle of ``device``'s current stream."""
    import torch

    index = device.index if device.index is not None else torch.cuda.current_device()
    raw = torch._C._cuda_getCurrentRawStream
    return lambda: raw(index)


def _entry_name(prefix, dtype):
    """The entry point ``<prefix>_<dtype>``; ``TypeError`` when the library has none for ``dtype``."""
    name = f"{prefix}_{_lib.dtype_suffix(dtype)}"
    if name not in _lib.exported_symbols():
        raise TypeError(f"no {prefix} kernel takes {dtype} operands")
    return name


def _entry(name):
    fn = getattr(_lib.load(), name)
    return fn, fn.__name__


def _raise(code, name):
    raise KernelLaunchError(code, name)


try:  # the packed launch (csrc/fastkey.cpp, built by ninetoothed_amd._build); else ctypes per argument
    from ninetoothed_amd import _fastkey
except ImportError:
    _fastkey = None


def _packed_address(name):
    """Address of the packed entry point ``name`` (``int name(const int64_t*)``), or None when
    the library does not export it or the packed launch module is missing."""
    if _fastkey is None or name not in _lib.exported_symbols():
        return None
    fn = getattr(_lib.load(), name, None)
    if not isinstance(fn, ctypes._CFuncPtr):
        return None
    return ctypes.cast(fn, ctypes.c_void_p).value


_F32 = struct.Struct("<f")
_U32 = struct.Struct("<I")
_float_bits_seen = {}


def _float_bits(x):
    """The bits of ``x`` as an fp32, as the packed entry points take alpha and beta."""
    bits = _float_bits_seen.get(x) if x else None  # (0.0 and -0.0 compare equal: not cached)
    if bits is None:
        bits = _U32.unpack(_F32.pack(x))[0]
        if x and len(_float_bits_seen) < 256:
            _float_bits_seen[x] = bits
    return bits


# ------------------------------------------------------------------------- add
# Each ``check_<op>`` validates what the kernels assume about dtypes, ranks and sizes
# without touching a device or the library (``TypeError`` / ``ValueError``), so a family
# matcher can decline a call its kernel would reject (``families.select``); ``bind_<op>``
# runs the same check before it binds.
def check_add(lhs, rhs, out):
    if not (lhs.dim() == rhs.dim() == out.dim() == 1):
        raise ValueError("add expects 1-D tensors")
    n = out.shape[0]
    if lhs.shape[0] != n or rhs.shape[0] != n:
        raise ValueError("add operands differ in length")
    if not (lhs.dtype == rhs.dtype == out.dtype):
        raise TypeError("add operands must share one dtype")
    return _entry_name("nt_add", out.dtype)


def bind_add(lhs, rhs, out):
    """launch(lhs, rhs, out): out = lhs + rhs over 1-D tensors of equal length (any strides)."""
    entry = check_add(lhs, rhs, out)
    device = _check_device(lhs, rhs, out)
    n = out.shape[0]
    fn, name = _entry(entry)
    sl, sr, so = lhs.stride(0), rhs.stride(0), out.stride(0)
    stream = _stream_of(device)

    def launch(lhs, rhs, out):
        code = fn(lhs.data_ptr(), sl, rhs.data_ptr(), sr, out.data_ptr(), so, n, stream())
        if code:
            _raise(code, name)

    return launch


def add(lhs, rhs, out):
    bind_add(lhs, rhs, out)(lhs, rhs, out)
    return out


# --------------------------------------------------------------------- softmax
# Kernel configurations of the softmax that ``config`` can force (0: the lane-group kernel for
# segments of at most four 16-byte vectors per lane of a wave, else the four-wave register
# path where the segment fits, else the two-sweep kernel; the element-wise kernel for a
# column stride other than 1 or an output of another dtype): the register path with
# workgroups of four, eight or one wave (the reference's num_warps candidates 4, 8, 1), the
# two-sweep kernel, the lane-group kernel, the element-wise kernel.
SOFTMAX_CONFIGS = (1, 2, 3, 4, 5, 6)
SOFTMAX_ANY = 6  # the configuration that takes any strides and any output dtype


def check_softmax(x, y, config=0):
    if x.dim() != 2 or y.shape != x.shape:
        raise ValueError("softmax expects matching 2-D tensors")
    if config and config not in SOFTMAX_CONFIGS:
        raise TypeError(f"softmax config {config} is not one of {SOFTMAX_CONFIGS}")
    cols = x.shape[1]
    unit = cols <= 1 or (x.stride(1) == 1 and y.stride(1) == 1)
    if config not in (0, SOFTMAX_ANY):
        if x.dtype != y.dtype:
            raise TypeError(f"softmax config {config} needs input and output of one dtype")
        if not unit:
            raise ValueError(f"softmax config {config} needs unit column strides")
    if x.dtype != y.dtype:
        _lib.dtype_code(x.dtype), _lib.dtype_code(y.dtype)  # TypeError for other dtypes
        return "nt_softmax_cast"
    return _entry_name("nt_softmax_config" if config else "nt_softmax", x.dtype)


def bind_softmax(x, y, block=None, config=0):
    """launch(x, y): row softmax of a 2-D tensor over segments of ``block`` columns (default: whole rows).

    Any strides; ``y`` may have another float dtype than ``x`` (the quotient is stored in
    y's type, as the reference's store casts it).  A nonzero ``config`` forces one kernel:
    configurations 1-5 need unit column strides and one dtype (``ValueError`` /
    ``TypeError`` here otherwise); a call a forced kernel does not admit raises
    ``KernelLaunchError`` without launching."""
    entry = check_softmax(x, y, config)
    device = _check_device(x, y)
    rows, cols = x.shape
    block = max(cols if block is None else int(block), 1)
    (xr, xc), (yr, yc) = x.stride(), y.stride()
    stream = _stream_of(device)
    if x.dtype != y.dtype:
        fn, name = _entry(entry)
        xcode, ycode = _lib.dtype_code(x.dtype), _lib.dtype_code(y.dtype)

        def launch(x, y):
            code = fn(x.data_ptr(), xcode, xr, xc, y.data_ptr(), ycode, yr, yc, rows, cols, block, stream())
            if code:
                _raise(code, name)

        return launch
    fn, name = _entry(entry)
    extra = (int(config),) if config else ()

    def launch(x, y):
        code = fn(x.data_ptr(), xr, xc, y.data_ptr(), yr, yc, rows, cols, block, stream(), *extra)
        if code:
            _raise(code, name)

    return launch


def softmax(x, y, block=None, config=0):
    bind_softmax(x, y, block, config)(x, y)
    return y


# ------------------------------------------------------------------ max_pool2d
# Kernel configurations of max_pool2d that ``config`` can force (0: the library's choice):
# 1 the vector kernels (pair-row kernel for 2-high windows, else one workgroup per plane),
# 2 the element-wise kernel, 3 the flat kernel (2-high windows, 8 outputs per unit),
# 4 the LDS strip kernel (any window whose input rows fit 32 KiB of LDS).
POOL_CONFIGS = (1, 2, 3, 4)
POOL_ANY = 2  # the configuration that takes any strides and any output dtype


def check_max_pool2d(x, y, config=0):
    if x.dim() != 4 or y.dim() != 4:
        raise ValueError("max_pool2d expects 4-D tensors")
    if config and config not in POOL_CONFIGS:
        raise TypeError(f"max_pool2d config {config} is not one of {POOL_CONFIGS}")
    if x.shape[0] != y.shape[0] or x.shape[1] != y.shape[1]:
        raise ValueError("max_pool2d batch/channel sizes differ")
    if x.dtype != y.dtype:
        if config not in (0, POOL_ANY):
            raise TypeError(f"max_pool2d config {config} needs input and output of one dtype")
        _lib.dtype_code(x.dtype), _lib.dtype_code(y.dtype)  # TypeError for other dtypes
        return "nt_max_pool2d_cast"
    return _entry_name("nt_max_pool2d_config" if config else "nt_max_pool2d", x.dtype)


def bind_max_pool2d(x, y, window, stride=None, padding=(0, 0), dilation=(1, 1), config=0):
    """launch(x, y): y = max_pool2d(x) with -inf outside the input (any strides, N-C-H-W indexing).

    ``y`` may have another float dtype than ``x`` (the window max is stored in y's type, as
    the reference's store casts it; still exact, rounding is monotone): that takes the
    element-wise kernel, so configurations other than 0 and 2 raise ``TypeError`` here.
    A nonzero ``config`` forces one kernel; a call it does not admit raises
    ``KernelLaunchError`` without launching."""
    entry = check_max_pool2d(x, y, config)
    device = _check_device(x, y)
    kh, kw = window
    sh, sw = stride if stride is not None else window
    ph, pw = padding
    dh, dw = dilation
    n, c, h, w = x.shape
    p, q = y.shape[2], y.shape[3]
    xs, ys = _lib.int64_array(x.stride()), _lib.int64_array(y.stride())
    dims = (n, c, h, w, p, q, kh, kw, sh, sw, ph, pw, dh, dw)
    stream = _stream_of(device)
    if x.dtype != y.dtype:
        fn, name = _entry(entry)
        xcode, ycode = _lib.dtype_code(x.dtype), _lib.dtype_code(y.dtype)

        def launch(x, y):
            code = fn(x.data_ptr(), xcode, xs, y.data_ptr(), ycode, ys, *dims, stream())
            if code:
                _raise(code, name)

        return launch
    fn, name = _entry(entry)
    extra = (int(config),) if config else ()

    def launch(x, y):
        code = fn(x.data_ptr(), xs, y.data_ptr(), ys, *dims, stream(), *extra)
        if code:
            _raise(code, name)

    return launch


def max_pool2d(x, y, window, stride=None, padding=(0, 0), dilation=(1, 1), config=0):
    bind_max_pool2d(x, y, window, stride, padding, dilation, config)(x, y)
    return y


# ------------------------------------------------------------------------ gemm
# Kernel configurations of the 16-bit GEMM that ``config`` can force (0: the fastest whose
# conditions hold): the DMA kernel, the register-staged eight-wave kernel, the element-wise
# loader kernel, the DMA kernel on 128 x 128 tiles, the few-rows kernel (M <= 64, b^T rows).
GEMM_CONFIGS = (1, 2, 3, 4, 5)


def check_gemm(a, b, out, c=None, round_dtype=None, config=0):
    """(entry point, out/c type argument, rounding type code) of a GEMM call."""
    if a.dim() != 2 or b.dim() != 2 or out.dim() != 2:
        raise ValueError("gemm expects 2-D tensors")
    m, k = a.shape
    if b.shape[0] != k or out.shape[0] != m or out.shape[1] != b.shape[1]:
        raise ValueError(f"gemm shape mismatch: {tuple(a.shape)} @ {tuple(b.shape)} -> {tuple(out.shape)}")
    n = b.shape[1]
    if a.dtype != b.dtype:
        raise TypeError("gemm operands must share one dtype")
    out_code = _lib.dtype_code(out.dtype)
    if c is not None:
        if tuple(c.shape) != (m, n):
            raise ValueError("gemm bias shape mismatch")
        if c.dtype != out.dtype:
            # c of another type (e.g. the reference's fp8 addmm input with an fp16 output) is
            # read in its own type: its code + 1 in bits 8-15 of the output-type argument.
            c_code = _lib.bias_dtype_code(c.dtype)
            if c_code in (_lib.DTYPE_E5M2, _lib.DTYPE_E4M3) and _lib.dtype_suffix(a.dtype) not in ("e5m2", "e4m3"):
                raise TypeError("an fp8 gemm bias needs fp8 operands")
            out_code |= (c_code + 1) << 8
    rd = _lib.DTYPE_NONE if round_dtype is None else _lib.dtype_code(round_dtype)
    if config:
        if config not in GEMM_CONFIGS or _lib.dtype_suffix(a.dtype) not in ("f16", "bf16"):
            raise TypeError(f"gemm config {config} needs fp16/bf16 operands and one of {GEMM_CONFIGS}")
        return _entry_name("nt_gemm_config", a.dtype), out_code, rd
    return _entry_name("nt_gemm", a.dtype), out_code, rd


def bind_gemm(a, b, out, c=None, round_dtype=None, config=0):
    """launch(a, b, out, c, alpha, beta): out = cast(beta * c + alpha * round(a @ b)).

    fp32 accumulation; any strides; ``c`` is None exactly when it was None here.  A nonzero
    ``config`` (fp16/bf16 operands only) forces one kernel; a call its conditions do not
    admit raises ``KernelLaunchError`` without launching."""
    entry, out_code, rd = check_gemm(a, b, out, c, round_dtype, config)
    device = _check_device(a, b, out, c)
    m, k = a.shape
    n = b.shape[1]
    fn, name = _entry(entry)
    extra = (int(config),) if config else ()
    (sa_m, sa_k), (sb_k, sb_n), (so_m, so_n) = a.stride(), b.stride(), out.stride()
    sc_m, sc_n = c.stride() if c is not None else (0, 0)
    stream = _stream_of(device)

    addr = _packed_address("nt_gemm_packed")
    if addr is not None:
        # nt_gemm_packed: the constant arguments packed once; per call the C++ helper writes
        # the four data pointers, alpha, beta and the stream into their slots and calls it.
        which = _PACKED_GEMM_ENTRY[entry]
        template = struct.pack("<22q", which, 0, sa_m, sa_k, 0, sb_k, sb_n, 0, sc_m, sc_n, 0, so_m, so_n, out_code, m,
                               n, k, 0, 0, rd, int(config), 0)
        call = _fastkey.call

        def launch(a, b, out, c, alpha, beta):
            code = call(addr, template, _GEMM_POINTER_SLOTS, (a, b, c, out), _GEMM_VALUE_SLOTS,
                        (_float_bits(alpha), _float_bits(beta), stream() or 0))
            if code:
                _raise(code, name)

        return launch

    def launch(a, b, out, c, alpha, beta):
        code = fn(a.data_ptr(), sa_m, sa_k, b.data_ptr(), sb_k, sb_n, c.data_ptr() if c is not None else None, sc_m,
                  sc_n, out.data_ptr(), so_m, so_n, out_code, m, n, k, alpha, beta, rd, *extra, stream())
        if code:
            _raise(code, name)

    return launch


# nt_gemm_packed: v[0] per entry point; slots of a, b, c, out and of alpha, beta, the stream
_PACKED_GEMM_ENTRY = {"nt_gemm_f16": 0, "nt_gemm_bf16": 1, "nt_gemm_f32": 2, "nt_gemm_e5m2": 3, "nt_gemm_e4m3": 4,
                      "nt_gemm_config_f16": 0, "nt_gemm_config_bf16": 1}
_GEMM_POINTER_SLOTS = (1, 4, 7, 10)
_GEMM_VALUE_SLOTS = (17, 18, 21)


def gemm(a, b, out, c=None, alpha=1.0, beta=0.0, round_dtype=None, config=0):
    bind_gemm(a, b, out, c, round_dtype, config)(a, b, out, c, float(alpha), float(beta))
    return out


# ---------------------------------------------------------------------- conv2d
def conv2d_workspace_bytes(x, w, padding=(0, 0)):
    """Bytes of the workspace that lets conv2d take its re-layout path (0: none needed)."""
    lib = _lib.load()
    n, c, h, wd = x.shape
    k, _, r, s = w.shape
    return int(lib.nt_conv2d_workspace_size(n, c, h, wd, k, r, s, padding[0], padding[1], _lib.dtype_code(x.dtype)))


# Paths of the 16-bit convolution that ``config`` can force (0: the fastest whose conditions
# hold): re-laid input through the DMA kernel, re-laid input through the N-H-W-C kernel,
# the direct kernel (no workspace), re-laid input through the DMA kernel of 224-position
# tiles, the input read in place by the 224-position strip kernel (only the filter re-laid),
# 1 x 1 filters as a batch of products on the 128 x 128-tile GEMM kernel, re-laid input
# through the DMA kernel of 128 x 128 tiles.
CONV_CONFIGS = (1, 2, 3, 4, 5, 6, 7)


def check_conv2d(x, w, y, round_dtype=None, config=0):
    """(entry point, rounding type code) of a conv2d call (fp16/bf16 input and filter)."""
    if x.dim() != 4 or w.dim() != 4 or y.dim() != 4:
        raise ValueError("conv2d expects 4-D tensors")
    if x.dtype != w.dtype:
        raise TypeError("conv2d input and filter must share one dtype")
    n, c = x.shape[:2]
    k, c2 = w.shape[:2]
    if c2 != c or y.shape[0] != n or y.shape[1] != k:
        raise ValueError("conv2d shape mismatch")
    _lib.dtype_code(y.dtype)
    rd = _lib.DTYPE_NONE if round_dtype is None else _lib.dtype_code(round_dtype)
    if config and config not in CONV_CONFIGS:
        raise TypeError(f"conv2d config {config} is not one of {CONV_CONFIGS}")
    return _entry_name("nt_conv2d_config" if config else "nt_conv2d", x.dtype), rd


def bind_conv2d(x, w, y, padding=(0, 0), stride=(1, 1), dilation=(1, 1), round_dtype=None, workspace_bytes=0,
                config=0):
    """launch(x, w, y, workspace): y = cast(round(conv2d(x, w))) as an implicit GEMM.

    Cross-correlation with zero padding.  ``workspace`` is a device buffer of at
    least ``workspace_bytes`` bytes, or None when ``workspace_bytes`` is 0.  A nonzero
    ``config`` forces one path; a call its conditions do not admit raises
    ``KernelLaunchError`` without launching."""
    entry, rd = check_conv2d(x, w, y, round_dtype, config)
    device = _check_device(x, w, y)
    n, c, h, wd = x.shape
    k, c2, r, s = w.shape
    p, q = y.shape[2], y.shape[3]
    ph, pw = padding
    sh, sw = stride
    dh, dw = dilation
    fn, name = _entry(entry)
    extra = (int(config),) if config else ()
    xs, ws, ys = (_lib.int64_array(t.stride()) for t in (x, w, y))
    dims = (_lib.dtype_code(y.dtype), n, c, h, wd, k, r, s, p, q, ph, pw, sh, sw, dh, dw, rd)
    stream = _stream_of(device)

    def launch(x, w, y, workspace):
        wp = None
        if workspace is not None:
            if workspace.device != device:
                raise TypeError("All tensor arguments must use the same GPU.")
            wp = workspace.data_ptr()
        code = fn(x.data_ptr(), xs, w.data_ptr(), ws, y.data_ptr(), ys, *dims, wp, workspace_bytes, *extra, stream())
        if code:
            _raise(code, name)

    return launch


def conv2d(x, w, y, padding=(0, 0), stride=(1, 1), dilation=(1, 1), round_dtype=None, workspace=None, config=0):
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if workspace is not None:
        _check_device(x, workspace)
    bind_conv2d(x, w, y, padding, stride, dilation, round_dtype, nbytes, config)(x, w, y, workspace)
    return y


# ------------------------------------------------------------------- attention
# Kernel configurations of the 16-bit attention that ``config`` can force (0: the eight-wave
# kernel where its conditions hold): the one-wave-per-SIMD pipelined kernel (head dim 128),
# the eight-wave kernel, the four-wave kernels (any strides).
ATTENTION_CONFIGS = (1, 2, 3)


def check_attention(q, k, v, o, config=0):
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
    _lib.dtype_code(o.dtype)
    if config:
        if config not in ATTENTION_CONFIGS or _lib.dtype_suffix(q.dtype) not in ("f16", "bf16"):
            raise TypeError(f"attention config {config} needs fp16/bf16 operands and one of {ATTENTION_CONFIGS}")
        return _entry_name("nt_attention_config", q.dtype)
    return _entry_name("nt_attention", q.dtype)


def bind_attention(q, k, v, o, causal=False, q_scale=LOG2E, config=0):
    """launch(q, k, v, o): flash attention forward of the reference application; q pre-scaled by ``q_scale``.

    A nonzero ``config`` (fp16/bf16 only) forces one kernel; a call its conditions do not
    admit raises ``KernelLaunchError`` without launching."""
    entry = check_attention(q, k, v, o, config)
    device = _check_device(q, k, v, o)
    bsz, heads, sq, d = q.shape
    sk = k.shape[2]
    fn, name = _entry(entry)
    extra = (int(config),) if config else ()
    qs, ks, vs, os_ = (_lib.int64_array(t.stride()) for t in (q, k, v, o))
    tail = (_lib.dtype_code(o.dtype), bsz, heads, sq, sk, d, float(q_scale), 1 if causal else 0)
    stream = _stream_of(device)

    def launch(q, k, v, o):
        code = fn(q.data_ptr(), qs, k.data_ptr(), ks, v.data_ptr(), vs, o.data_ptr(), os_, *tail, stream(), *extra)
        if code:
            _raise(code, name)

    return launch


def attention(q, k, v, o, causal=False, q_scale=LOG2E, config=0):
    bind_attention(q, k, v, o, causal, q_scale, config)(q, k, v, o)
    return o
