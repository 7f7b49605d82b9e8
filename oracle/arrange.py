"""Oracle restatement of arrangement index semantics (test infrastructure only).

Restates the meta-operations of the reference's ``Tensor`` (``src/ninetoothed/tensor.py``:
tile 200-286, expand 288-320, unsqueeze 322-352, squeeze 354-391, permute 393-422,
flatten 424-480, ravel 482-536, pad 538-563, _slice_dim/__getitem__ 677-730) and the
mask rule of ``offsets`` (565-578: every derived index must lie in [0, size)).

Algorithm (deliberately not the product's): an ``OTensor`` holds its whole hierarchy
MATERIALISED as a table — for every element of every level, the source multi-index
and a validity flag.  A meta-operation on a level builds the new table by gathering
from the old one (index arithmetic on the enumerated new indices, out-of-range
gathers clipped and marked invalid).  ``ravel`` only regroups level boundaries.
Symbols are bound up front: sizes and block sizes must be plain integers or
objects with ``evaluate(env)``.

Masked (invalid) entries hold unspecified indices; ``eval`` writes -1 there, as the
reference's ``eval`` does (``src/ninetoothed/eval.py:15-55``).

Pinned by: the reference's golden maps (addmm arrangement in test_debugging.py:41-239,
eval cases in test_eval.py:11-198; tests/test_oracle_arrange.py) and closed forms.
"""

import numpy as np


def _int(v, env):
    if hasattr(v, "evaluate"):
        return int(v.evaluate(env))
    return int(v)


class OTensor:
    """A materialised hierarchy: ``table[..., d]`` = source index d, ``valid[...]``."""

    def __init__(self, shape, env=None, other=None, _table=None, _valid=None, _levels=None, _level=0, _src_shape=None):
        self.env = env or {}
        if _table is None:
            shape = tuple(_int(s, self.env) for s in shape)
            grids = np.meshgrid(*[np.arange(s) for s in shape], indexing="ij") if shape else []
            self.table = np.stack(grids, axis=-1) if shape else np.zeros((0,), dtype=np.int64)
            self.valid = np.ones(shape, dtype=bool)
            self.levels = [shape]
            self.src_shape = shape
        else:
            self.table, self.valid, self.levels, self.src_shape = _table, _valid, _levels, _src_shape
        self.level = _level  # which level this object stands for
        self.other = other
        self._owner = None  # (parent OTensor) for dtype assignment

    # ----------------------------------------------------------- hierarchy view
    @property
    def shape(self):
        return self.levels[self.level]

    @property
    def ndim(self):
        return len(self.levels[self.level])

    @property
    def dtype(self):
        if self.level + 1 >= len(self.levels):
            return None
        d = OTensor(None, self.env, self.other, self.table, self.valid, self.levels, self.level + 1, self.src_shape)
        d._owner = self
        return d

    @dtype.setter
    def dtype(self, inner):
        if inner is None or not isinstance(inner, OTensor):
            return
        # inner was derived from this tensor's inner level: adopt its table
        if inner.levels[: self.level + 1] != self.levels[: self.level + 1]:
            raise ValueError("inner level does not belong to this hierarchy")
        self.table, self.valid, self.levels = inner.table, inner.valid, inner.levels
        if self._owner is not None:  # this object is a view of an outer level's inner level
            self._owner.dtype = self

    def _axis0(self):
        return sum(len(l) for l in self.levels[: self.level])

    def _replace(self, new_levels_here, new_table, new_valid, keep_rest=True):
        levels = self.levels[: self.level] + new_levels_here + (self.levels[self.level + 1 :] if keep_rest else [])
        return OTensor(None, self.env, self.other, new_table, new_valid, levels, self.level, self.src_shape)

    def _gather_level(self, new_dims, index_fns):
        """Build a level with dims ``new_dims`` whose element maps to old level index
        ``(fn(new_idx) for fn in index_fns)``; out-of-range old indices are invalid."""
        a0 = self._axis0()
        old_shape = self.levels[self.level]
        n_old = len(old_shape)
        grids = np.meshgrid(*[np.arange(s) for s in new_dims], indexing="ij") if new_dims else []
        new_idx = [g for g in grids]
        old_idx = [fn(new_idx) for fn in index_fns]
        ok = np.ones(tuple(new_dims), dtype=bool)
        clipped = []
        for i, size in zip(old_idx, old_shape):
            i = np.broadcast_to(np.asarray(i), tuple(new_dims))
            ok = ok & (i >= 0) & (i < size)
            clipped.append(np.clip(i, 0, max(size - 1, 0)))
        # move the level's axes to the front, gather, move back
        t = np.moveaxis(self.table, list(range(a0, a0 + n_old)), list(range(n_old)))
        v = np.moveaxis(self.valid, list(range(a0, a0 + n_old)), list(range(n_old)))
        if n_old:
            t = t[tuple(clipped)]
            v = v[tuple(clipped)]
        else:
            t = np.broadcast_to(t, tuple(new_dims) + t.shape)
            v = np.broadcast_to(v, tuple(new_dims) + v.shape)
        extra = tuple([slice(None)] * len(new_dims)) + (None,) * (v.ndim - len(new_dims))
        v = v & ok[extra]
        k = len(new_dims)
        t = np.moveaxis(t, list(range(k)), list(range(a0, a0 + k)))
        v = np.moveaxis(v, list(range(k)), list(range(a0, a0 + k)))
        return t, v

    # ---------------------------------------------------------- meta-operations
    def tile(self, tile_shape, strides=None, dilation=None, floor_mode=False):
        env = self.env
        shape = self.shape
        n = len(shape)
        strides = [-1] * n if strides is None else [_int(s, env) for s in strides]
        dilation = [1] * n if dilation is None else [_int(d, env) for d in dilation]
        tile_shape = [_int(t, env) for t in tile_shape]
        outer, inner, steps = [], [], []
        for size, t, st, dl in zip(shape, tile_shape, strides, dilation):
            t = size if t == -1 else t
            st = t if st == -1 else st
            span = size - dl * (t - 1) - 1
            cnt = (span // st if floor_mode else -(-span // st)) + 1
            outer.append(cnt)
            inner.append(t)
            steps.append(st)
        dims = outer + inner
        fns = [
            (lambda idx, d=d: idx[d] * steps[d] + idx[n + d] * dilation[d]) for d in range(n)
        ]
        t, v = self._gather_level(dims, fns)
        return self._replace([tuple(outer), tuple(inner)], t, v)

    def expand(self, shape):
        env = self.env
        shape = [_int(s, env) for s in shape]
        new = [old if s == -1 else s for old, s in zip(self.shape, shape)]
        fns = [(lambda idx, d=d: idx[d] if shape[d] == -1 else idx[d] * 0) for d in range(len(new))]
        t, v = self._gather_level(new, fns)
        return self._replace([tuple(new)], t, v)

    def squeeze(self, dim):
        dims = dim if isinstance(dim, tuple) else (dim,)
        dims = [d + self.ndim if d < 0 else d for d in dims]
        new = [s for d, s in enumerate(self.shape) if d not in dims]
        kept = [d for d in range(self.ndim) if d not in dims]
        fns = []
        for d in range(self.ndim):
            if d in dims:
                fns.append(lambda idx: 0)
            else:
                fns.append(lambda idx, j=kept.index(d): idx[j])
        t, v = self._gather_level(new, fns)
        return self._replace([tuple(new)], t, v)

    def unsqueeze(self, dim):
        new = list(self.shape)
        new.insert(dim, 1)
        fns = [(lambda idx, j=(d if d < dim else d + 1): idx[j]) for d in range(self.ndim)]
        t, v = self._gather_level(new, fns)
        return self._replace([tuple(new)], t, v)

    def permute(self, dims):
        new = [self.shape[d] for d in dims]
        fns = [(lambda idx, j=list(dims).index(d): idx[j]) for d in range(self.ndim)]
        t, v = self._gather_level(new, fns)
        return self._replace([tuple(new)], t, v)

    def flatten(self, start_dim=None, end_dim=None):
        n = self.ndim
        s = 0 if start_dim is None else (start_dim + n if start_dim < 0 else start_dim)
        e = n if end_dim is None else (end_dim + n if end_dim < 0 else end_dim)
        sizes = list(self.shape[s:e])
        merged = int(np.prod(sizes)) if sizes else 1
        new = list(self.shape[:s]) + [merged] + list(self.shape[e:])

        def unravel(flat, k):
            stride = int(np.prod(sizes[k + 1 :])) if k + 1 < len(sizes) else 1
            return (flat // stride) % sizes[k] if k > 0 else flat // stride

        fns = []
        for d in range(n):
            if d < s:
                fns.append(lambda idx, d=d: idx[d])
            elif d < e:
                fns.append(lambda idx, k=d - s: unravel(idx[s], k))
            else:
                fns.append(lambda idx, d=d: idx[d - (e - s) + 1])
        t, v = self._gather_level(new, fns)
        return self._replace([tuple(new)], t, v)

    def ravel(self):
        merged = tuple(x for lvl in self.levels[self.level :] for x in lvl)
        levels = self.levels[: self.level] + [merged]
        return OTensor(None, self.env, self.other, self.table, self.valid, levels, self.level, self.src_shape)

    def pad(self, pad):
        pad = [(_int(lo, self.env), _int(hi, self.env)) for lo, hi in pad]
        new = [s + lo + hi for s, (lo, hi) in zip(self.shape, pad)]
        fns = [(lambda idx, d=d: idx[d] - pad[d][0]) for d in range(self.ndim)]
        t, v = self._gather_level(new, fns)
        return self._replace([tuple(new)], t, v)

    def __getitem__(self, index):
        raise NotImplementedError("the oracle restates the meta-operations the hot-path arrangements use")

    # ------------------------------------------------------------------ output
    def flat_levels(self):
        return [x for lvl in self.levels[self.level :] for x in lvl]

    def eval(self):
        """Linear source offsets with contiguous strides, -1 where invalid."""
        strides = np.cumprod((1,) + tuple(reversed(self.src_shape[1:])))[::-1] if self.src_shape else ()
        linear = (self.table * np.asarray(strides, dtype=np.int64)).sum(-1) if self.src_shape else 0
        return np.where(self.valid, linear, -1)


def source(shape, env=None, other=None):
    """An oracle source tensor of concrete ``shape``."""
    return OTensor(shape, env=env, other=other)


class Scalar:
    """Stand-in for a 0-d tensor parameter (arrangements pass it through unchanged)."""

    ndim = 0
