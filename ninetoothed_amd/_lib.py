"""ctypes binding of libnt_mi355x.so (declared in ``include/nt_mi355x.h``).

This mirrors how the reference binds the CUDA backend's compiled launcher
(reference ``src/ninetoothed/backends/materializers/cuda.py:49-130``): ``ctypes.CDLL``,
``restype = c_int``, device pointers as ``c_void_p``, dims as ``c_int64`` and the
caller's current stream last.  Here the library is prebuilt from hand-written HIP
sources instead of generated per kernel.

The library is loaded after ``torch`` so that it binds to the HIP runtime that
PyTorch-ROCm already has in the process (both name ``libamdhip64.so.7``); device
pointers and streams then mean the same thing on both sides.  A missing library is
an error, never a fallback.
"""

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libnt_mi355x.so"
ABI_VERSION = 1

DTYPE_NONE = -1
DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_E5M2 = 3  # GEMM bias (c) only
DTYPE_E4M3 = 4

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_I64P = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (restype is c_int unless listed in _RESTYPES)
_SIGNATURES = {
    "nt_abi_version": (),
    **{
        f"nt_add_{t}": (_P, _I64, _P, _I64, _P, _I64, _I64, _P)
        for t in ("f32", "f16", "bf16")
    },
    **{
        f"nt_softmax_{t}": (_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P)
        for t in ("f32", "f16", "bf16")
    },
    **{
        f"nt_softmax_config_{t}": (_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I)
        for t in ("f32", "f16", "bf16")
    },
    "nt_softmax_cast": (_P, _I, _I64, _I64, _P, _I, _I64, _I64, _I64, _I64, _I64, _P),
    "nt_max_pool2d_cast": (_P, _I, _I64P, _P, _I, _I64P) + (_I64,) * 14 + (_P,),
    **{
        f"nt_max_pool2d_{t}": (_P, _I64P, _P, _I64P) + (_I64,) * 14 + (_P,)
        for t in ("f32", "f16", "bf16")
    },
    **{
        f"nt_max_pool2d_config_{t}": (_P, _I64P, _P, _I64P) + (_I64,) * 14 + (_P, _I)
        for t in ("f32", "f16", "bf16")
    },
    **{
        f"nt_gemm_{t}": (_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I, _I64, _I64, _I64, _F, _F, _I, _P)
        for t in ("f32", "f16", "bf16", "e5m2", "e4m3")
    },
    **{
        f"nt_gemm_config_{t}": (_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I, _I64, _I64, _I64, _F,
                                _F, _I, _I, _P)
        for t in ("f16", "bf16")
    },
    "nt_gemm_packed": (_I64P,),
    "nt_conv2d_workspace_size": (_I64,) * 9 + (_I,),
    **{
        f"nt_conv2d_noalloc_{t}": (_P, _I64P, _P, _I64P, _P, _I64P, _I) + (_I64,) * 15 + (_I, _P)
        for t in ("f16", "bf16")
    },
    **{
        f"nt_conv2d_{t}": (_P, _I64P, _P, _I64P, _P, _I64P, _I) + (_I64,) * 15 + (_I, _P, _I64, _P)
        for t in ("f16", "bf16")
    },
    **{
        f"nt_conv2d_config_{t}": (_P, _I64P, _P, _I64P, _P, _I64P, _I) + (_I64,) * 15 + (_I, _P, _I64, _I, _P)
        for t in ("f16", "bf16")
    },
    **{
        f"nt_attention_{t}": (_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I64, _I64, _I64, _I64, _I64, _F, _I, _P)
        for t in ("f32", "f16", "bf16")
    },
    **{
        f"nt_attention_config_{t}": (_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _I64, _I64, _I64, _I64, _I64, _F, _I,
                                     _P, _I)
        for t in ("f16", "bf16")
    },
    "nt_rtc_compile": (ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_P), _I64P, ctypes.c_char_p, _I64),
    "nt_rtc_free": (_P,),
    "nt_rtc_load": (_P, ctypes.c_char_p, ctypes.POINTER(_P)),
    "nt_rtc_launch": (_P, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(_P), _P),
}
_RESTYPES = {"nt_conv2d_workspace_size": ctypes.c_int64, "nt_rtc_free": None}

_lock = threading.Lock()
_library = None


class LibraryNotBuiltError(RuntimeError):
    pass


def exported_symbols() -> tuple[str, ...]:
    return tuple(_SIGNATURES)


def load():
    """Load (once) and return the configured ``ctypes.CDLL``."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is not None:
            return _library
        if not LIBRARY_PATH.is_file():
            raise LibraryNotBuiltError(
                f"{LIBRARY_PATH} is not built; run `python __graft_entry__.py` "
                "(or ninetoothed_amd._build.build()) first."
            )
        import torch  # noqa: F401  (bind to the HIP runtime torch already loaded)

        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = list(argtypes)
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        version = lib.nt_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libnt_mi355x.so ABI {version}, expected {ABI_VERSION}; rebuild it.")
        _library = lib
        return lib


def int64_array(values):
    values = tuple(int(v) for v in values)
    return (ctypes.c_int64 * len(values))(*values)


def dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}
    try:
        return codes[dtype]
    except KeyError:
        raise TypeError(f"dtype {dtype} is not supported by the MI355X kernels") from None


def bias_dtype_code(dtype) -> int:
    """Element-type code of a GEMM's c operand: the float codes plus the fp8 formats."""
    import torch

    fp8 = {getattr(torch, "float8_e5m2", None): DTYPE_E5M2, getattr(torch, "float8_e4m3fn", None): DTYPE_E4M3}
    if dtype in fp8 and dtype is not None:
        return fp8[dtype]
    return dtype_code(dtype)


def dtype_suffix(dtype) -> str:
    import torch

    fp8 = {getattr(torch, "float8_e5m2", None): "e5m2", getattr(torch, "float8_e4m3fn", None): "e4m3"}
    if dtype in fp8 and dtype is not None:
        return fp8[dtype]
    return {DTYPE_F32: "f32", DTYPE_F16: "f16", DTYPE_BF16: "bf16"}[dtype_code(dtype)]


def current_stream(device=None):
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
