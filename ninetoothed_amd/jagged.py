"""Jagged tensors (torch nested tensors of the ``torch.jagged`` layout) as the kernels address them.

A jagged tensor of logical shape [B, ..., j, ...] (the ragged dim j, 1 <= j < ndim) keeps
its elements in ``values()``, whose dims are the logical dims 1 .. ndim-1 with dim j
running over every batch's rows back to back, and ``offsets()`` [B + 1]: batch b owns
rows offsets[b] .. offsets[b + 1] - 1 of that dim.  As the reference lowers it
(``src/ninetoothed/tensor.py:614-630``: the batch dim has stride 0 and the pointer is the
values'; ``src/ninetoothed/frontend/layout.py:55-70``: the element offset gains
``seq_start * stride(jagged_dim)``; ``src/ninetoothed/backends/emitters/ssa.py:3395-3450``:
``seq_start = offsets[b]``, ``seq_len = offsets[b + 1] - offsets[b]``), element
(b, i_1, ..., i_{n-1}) lives at

    sum_{d >= 1} i_d * values().stride(d - 1) + offsets[b] * values().stride(j - 1)

and exists only where i_j < seq_len(b).  The arrangement sees the ragged dim with the
call's longest batch as its size (the reference's ``max_seq_len``,
``compiler/runtime.py:1382-1389``); positions past a batch's own length are masked, so
loads there give the tensor's ``other`` and stores there write nothing.
"""

import numpy as np


def is_jagged(value):
    """Whether ``value`` is a nested tensor of the jagged layout."""
    if not getattr(value, "is_nested", False):
        return False
    import torch

    return getattr(value, "layout", None) is torch.jagged


def ragged_dim(value):
    """The dim of a jagged tensor whose size varies across the batch."""
    dims = [i for i, s in enumerate(value.shape) if not isinstance(s, int)]
    if len(dims) != 1:
        raise TypeError("a jagged tensor has exactly one ragged dimension")
    return dims[0]


def host_offsets(value):
    """offsets() as host int64 (one device-to-host copy, as the reference's ``max_seq_len``)."""
    import torch

    return value.offsets().to("cpu", torch.int64).numpy()


def padded_shape(value, offsets=None):
    """The logical shape with the ragged dim at the longest batch's length."""
    offs = host_offsets(value) if offsets is None else offsets
    longest = int(np.diff(offs).max()) if offs.size > 1 else 0
    j = ragged_dim(value)
    return tuple(longest if d == j else int(s) for d, s in enumerate(value.shape))


def data_ptr(value):
    """The address the kernels index from: the values' for a jagged tensor."""
    return value.values().data_ptr() if is_jagged(value) else value.data_ptr()


def element_offsets(value, idx, mask):
    """Element offsets (in elements from ``values()``) and mask for logical index arrays.

    ``idx`` holds one integer array per logical dim (broadcast alike), ``mask`` the
    arrangement's own mask; positions past their batch's length are masked out."""
    offs = host_offsets(value)
    j = ragged_dim(value)
    vstrides = value.values().stride()
    batches = offs.size - 1
    b = np.asarray(idx[0], dtype=np.int64)
    inside = mask & (b >= 0) & (b < batches)
    bc = np.clip(b, 0, max(batches - 1, 0))
    start = offs[bc] if batches else np.zeros_like(bc)
    length = offs[np.minimum(bc + 1, batches)] - start if batches else np.zeros_like(bc)
    rows = np.asarray(idx[j], dtype=np.int64)
    inside = inside & (rows < length)
    off = start * int(vstrides[j - 1])
    for d in range(1, len(idx)):
        off = off + np.asarray(idx[d], dtype=np.int64) * int(vstrides[d - 1])
    return np.broadcast_to(off, inside.shape), inside


def storage_extent(value):
    """Elements from the first to one past the last element of the values."""
    v = value.values() if is_jagged(value) else value
    if v.numel() == 0:
        return 0
    return 1 + sum((int(n) - 1) * int(st) for n, st in zip(v.shape, v.stride()))
