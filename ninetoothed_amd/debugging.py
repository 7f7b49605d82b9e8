"""Debugging aids: ``simulate_arrangement`` (reference ``src/ninetoothed/debugging.py:16-60``).

For each tensor, the source is an arange of its shape and the target holds, for every
element of the arranged hierarchy (outermost level flattened into one axis), the index of
the source element it refers to, -1 where the arrangement masks it.  The reference runs a
generated kernel to fill the targets; here they come from the same index evaluator that
fits the kernels' geometry (``tensor.BoundView``), so they show exactly what the MI355X
kernels are given.
"""

import math

import numpy as np

from ninetoothed_amd.tensor import Tensor


def simulate_arrangement(arrangement, tensors, device=None):
    """(source tensors, target tensors), in the arrangement's parameter order."""
    import torch

    device = "cuda" if device is None else device
    sources, targets = [], []
    for tensor, arranged in zip(tensors, arrangement(*tensors)):
        if tensor.ndim == 0:
            sources.append(torch.tensor(0, device=device))
            targets.append(torch.tensor(0, device=device))
            continue
        shape = tuple(int(s) for s in tensor.shape)
        sources.append(torch.arange(math.prod(shape), device=device).view(shape))
        levels = arranged.levels() if isinstance(arranged, Tensor) else []
        index = np.asarray(arranged.eval())
        outer = len(levels[0].shape) if levels else 0
        flat = index.reshape((int(np.prod(index.shape[:outer])),) + index.shape[outer:])
        targets.append(torch.from_numpy(np.ascontiguousarray(flat)).to(torch.int64).to(device))
    return tuple(sources), tuple(targets)
