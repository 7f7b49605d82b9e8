"""ninetoothed_amd: an MI355X-native (gfx950) backend for NineToothed's arrange-and-apply kernels.

Drop-in surface of ``ninetoothed`` for the hot path (``import ninetoothed_amd as
ninetoothed``): ``make``, ``jit``, ``build``, ``Tensor``, ``Symbol``, ``block_size``, the dtype
aliases, ``eval`` and ``subs``; application bodies use ``ninetoothed_amd.language``
as ``ntl``.  Kernels run from the prebuilt ``libnt_mi355x.so``.
"""

from ninetoothed_amd.build import build
from ninetoothed_amd.compiler import jit, make
from ninetoothed_amd.dtype import (
    bfloat16,
    float16,
    float32,
    float64,
    int8,
    int16,
    int32,
    int64,
    uint8,
    uint16,
    uint32,
    uint64,
)
from ninetoothed_amd.errors import KernelLaunchError, LoweringError
from ninetoothed_amd.symbol import Symbol, block_size
from ninetoothed_amd.tensor import Tensor
from ninetoothed_amd.tensor import _eval as eval  # noqa: A001
from ninetoothed_amd.tensor import _subs as subs

__all__ = [
    "KernelLaunchError",
    "LoweringError",
    "Symbol",
    "Tensor",
    "bfloat16",
    "block_size",
    "build",
    "eval",
    "float16",
    "float32",
    "float64",
    "int8",
    "int16",
    "int32",
    "int64",
    "jit",
    "make",
    "subs",
    "uint8",
    "uint16",
    "uint32",
    "uint64",
]
