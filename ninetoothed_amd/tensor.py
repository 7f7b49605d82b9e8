"""Symbolic hierarchical tensors: the arrangement DSL.

Public surface as the reference's ``Tensor`` (``src/ninetoothed/tensor.py:11-730``):
``Tensor(ndim, shape, dtype, jagged_dim, other, shape_options, constexpr, value,
name)`` and the meta-operations ``tile``, ``expand``, ``squeeze``, ``unsqueeze``,
``permute``, ``flatten``, ``ravel``, ``pad`` and ``__getitem__``.  A tensor is one
level of a hierarchy; ``tensor.dtype`` is the next (inner) level or the element type.

Index semantics (what the reference computes in ``offsets``/``offsets_and_mask``,
``src/ninetoothed/tensor.py:565-578`` and ``src/ninetoothed/frontend/layout.py:72-97``):
every tensor derived by a meta-operation holds *links* to the tensor(s) it came
from, each link mapping this tensor's index to a contribution to the parent's
index.  Evaluating an arranged hierarchy assigns an index to every level, then
visits tensors newest-first; a visited tensor sums the contributions it received,
checks 0 <= index < size on every dimension (the conjunction of those checks is the
mask), and forwards contributions along its links until the source is reached.
Tiles contribute ``outer * stride`` and ``inner * dilation`` to the same parent
index; ``ravel`` splits its index across the levels it flattened.

The evaluator is vectorised over numpy index arrays and takes an environment that
binds every size symbol, block size and constexpr by name; it is used both to fit
kernel geometry at call time and by ``eval``.
"""

import copy
import itertools
import math

import numpy as np

from ninetoothed_amd.symbol import Symbol, evaluate, names_in, prod

_ids = itertools.count()


class _Link:
    """How a derived tensor's index contributes to one parent tensor's index."""

    __slots__ = ("target", "kind", "params")

    def __init__(self, target, kind, params):
        self.target = target
        self.kind = kind
        self.params = params

    def apply(self, idx, env):
        kind, p = self.kind, self.params
        if kind == "scale":  # tile levels: index * factor per dim
            factors = evaluate(p, env)
            return tuple(i * f for i, f in zip(idx, factors))
        if kind == "expand":  # expanded dims contribute 0
            return tuple(i if keep else i * 0 for i, keep in zip(idx, p))
        if kind == "squeeze":  # re-insert removed singleton dims as 0
            removed, parent_ndim = p
            it = iter(idx)
            zero = np.zeros((), dtype=np.int64)
            return tuple(zero if d in removed else next(it) for d in range(parent_ndim))
        if kind == "unsqueeze":
            return tuple(i for d, i in enumerate(idx) if d != p)
        if kind == "permute":  # parent[dims[i]] = idx[i]
            dims = p
            out = [None] * len(dims)
            for i, d in enumerate(dims):
                out[d] = idx[i]
            return tuple(out)
        if kind == "flatten":
            start, sizes = p
            sizes = evaluate(sizes, env)
            return tuple(idx[:start]) + _unravel(idx[start], sizes) + tuple(idx[start + 1 :])
        if kind == "slice":  # ravel: a window of the flat index
            start, stop = p
            return tuple(idx[start:stop])
        if kind == "shift":  # pad: index - low padding
            lows = evaluate(p, env)
            return tuple(i - lo for i, lo in zip(idx, lows))
        if kind == "affine_dim":  # getitem slice: parent[dim] = start + idx[dim] * step
            dim, start, step = p
            start, step = evaluate(start, env), evaluate(step, env)
            out = list(idx)
            out[dim] = start + idx[dim] * step
            return tuple(out)
        raise AssertionError(kind)


def _unravel(index, sizes):
    out = []
    for k in range(len(sizes)):
        stride = 1
        for s in sizes[k + 1 :]:
            stride *= s
        out.append(index // stride)
        index = index % stride
    return tuple(out)


def _as_size(value):
    if isinstance(value, Symbol) and value.is_constant():
        return value.value
    return value


class Tensor:
    """A symbolic tensor (one level of an arranged hierarchy)."""

    def __init__(
        self,
        ndim=None,
        shape=None,
        dtype=None,
        jagged_dim=None,
        other=None,
        shape_options=None,
        constexpr=None,
        value=None,
        name=None,
        *,
        _source=None,
        _links=(),
        _shape=None,
    ):
        self._id = next(_ids)
        if _shape is not None:  # derived tensor
            self.name = name if name is not None else _source.name
            self.shape = _shape
            self.dtype = dtype
            self.source = _source
            self.other = other if other is not None else _source.other
            self.jagged_dim = None
            self.constexpr = False
            self.value = None
            self._links = tuple(_links)
            return

        if ndim is None and shape is None:
            raise AssertionError("Either `ndim` or `shape` must be provided.")
        if ndim is None:
            ndim = len(shape)
        if shape is None:
            shape = (None,) * ndim
        if shape_options is None:
            shape_options = tuple({} for _ in range(ndim))
        elif isinstance(shape_options, dict):
            shape_options = tuple(shape_options for _ in range(ndim))
        shape_options = tuple(o if o is not None else {} for o in shape_options)
        self.name = name if name is not None else f"tensor_{self._id}"
        self.shape = tuple(
            _as_size(size) if size is not None else Symbol(f"{self.name}_size_{i}", **opts)
            for i, (size, opts) in enumerate(zip(shape, shape_options))
        )
        self.dtype = dtype
        # A jagged source (reference src/ninetoothed/tensor.py:17-45): dim `jagged_dim` varies
        # across the batch (dim 0); it is bound to a torch nested tensor of the jagged layout
        # (ninetoothed_amd.jagged), its size to the call's longest batch.
        if jagged_dim is not None and not (isinstance(jagged_dim, int) and 1 <= jagged_dim < ndim):
            raise ValueError("`jagged_dim` must be a dimension after the batch dimension (1 .. ndim - 1).")
        self.jagged_dim = jagged_dim
        self.other = other
        if constexpr and self.ndim != 0:
            raise ValueError("The `constexpr` option can only be set for zero-dimensional tensors.")
        self.constexpr = bool(constexpr)
        if not constexpr and value is not None:
            raise ValueError("The `value` option can only be set for constexpr tensors.")
        self.value = value
        self.source = self
        self._links = ()

    # --------------------------------------------------------------- structure
    @property
    def shape(self):
        return self._shape

    @shape.setter
    def shape(self, value):
        self._shape = tuple(_as_size(v) for v in value)

    @property
    def ndim(self):
        return len(self._shape)

    def size(self, dim=None):
        return self.shape if dim is None else self.shape[dim]

    def innermost(self):
        return self.dtype.innermost() if isinstance(self.dtype, Tensor) else self

    def levels(self):
        """This tensor and its inner levels, outermost first."""
        out, cur = [], self
        while isinstance(cur, Tensor):
            out.append(cur)
            cur = cur.dtype
        return out

    def element_dtype(self):
        return self.innermost().dtype

    def _derive(self, shape, links, dtype=None, **kw):
        return Tensor(_source=self.source, _links=links, _shape=tuple(shape), dtype=dtype, **kw)

    def __deepcopy__(self, memo):
        # Deep copies keep the ids of the tensors they copy: a copied hierarchy is
        # evaluated on its own, and every tensor an arrangement derives from a copy
        # gets a fresh (larger) id, so newest-first order still holds.
        cls = type(self)
        new = cls.__new__(cls)
        memo[id(self)] = new
        for k, v in self.__dict__.items():
            setattr(new, k, copy.deepcopy(v, memo))
        return new

    # -------------------------------------------------------- meta-operations
    def tile(self, tile_shape, strides=None, dilation=None, floor_mode=False):
        """Tile into a two-level hierarchy (reference ``tensor.py:200-286``)."""
        n = self.ndim
        strides = [-1] * n if strides is None else list(strides)
        dilation = [1] * n if dilation is None else list(dilation)
        outer_shape, outer_steps, inner_shape = [], [], []
        for size, tsz, stride, spacing in zip(self.shape, tile_shape, strides, dilation):
            tsz = size if _eq(tsz, -1) else tsz
            stride = tsz if _eq(stride, -1) else stride
            if _eq(stride, 0):
                count = -1
            else:
                span = size - spacing * (tsz - 1) - 1
                count = (span // stride if floor_mode else (span + stride - 1) // stride) + 1
            outer_shape.append(count)
            outer_steps.append(stride)
            inner_shape.append(tsz)
        inner = self._derive(inner_shape, (_Link(self, "scale", tuple(dilation)),), dtype=self.dtype)
        return self._derive(outer_shape, (_Link(self, "scale", tuple(outer_steps)),), dtype=inner)

    def expand(self, shape):
        """Broadcast singleton dims to ``shape`` (-1 keeps a dim; reference ``tensor.py:288-320``)."""
        new_shape = [old if _eq(new, -1) else new for old, new in zip(self.shape, shape)]
        keep = tuple(_eq(new, -1) for new in shape)
        return self._derive(new_shape, (_Link(self, "expand", keep),), dtype=self.dtype)

    def unsqueeze(self, dim):
        new_shape = list(self.shape)
        new_shape.insert(dim, 1)
        return self._derive(new_shape, (_Link(self, "unsqueeze", dim),), dtype=self.dtype)

    def squeeze(self, dim):
        dims = dim if isinstance(dim, tuple) else (dim,)
        dims = tuple(d + self.ndim if d < 0 else d for d in dims)
        new_shape = [s for d, s in enumerate(self.shape) if d not in dims]
        return self._derive(new_shape, (_Link(self, "squeeze", (frozenset(dims), self.ndim)),), dtype=self.dtype)

    def permute(self, dims):
        new_shape = [self.shape[d] for d in dims]
        return self._derive(new_shape, (_Link(self, "permute", tuple(dims)),), dtype=self.dtype)

    def flatten(self, start_dim=None, end_dim=None):
        """Merge dims [start_dim, end_dim) of this level (end exclusive, as the reference)."""
        n = self.ndim
        start = 0 if start_dim is None else (start_dim + n if start_dim < 0 else start_dim)
        end = n if end_dim is None else (end_dim + n if end_dim < 0 else end_dim)
        sizes = tuple(self.shape[start:end])
        new_shape = self.shape[:start] + (prod(sizes),) + self.shape[end:]
        return self._derive(new_shape, (_Link(self, "flatten", (start, sizes)),), dtype=self.dtype)

    def ravel(self):
        """Flatten the hierarchy into one level (reference ``tensor.py:482-536``)."""
        shape, links, pos = [], [], 0
        for level in self.levels():
            links.append(_Link(level, "slice", (pos, pos + level.ndim)))
            shape.extend(level.shape)
            pos += level.ndim
        return self._derive(shape, tuple(links), dtype=None, other=self.source.other, name=self.source.name)

    def pad(self, pad):
        new_shape = [size + lo + hi for size, (lo, hi) in zip(self.shape, pad)]
        return self._derive(new_shape, (_Link(self, "shift", tuple(lo for lo, _ in pad)),), dtype=self.dtype)

    def _slice_dim(self, dim, start, stop=None, step=None):
        if dim < 0:
            dim += self.ndim
        step = 1 if step is None else step
        size = self.shape[dim]
        if start is None:
            start = 0 if step > 0 else size - 1
        if stop is None:
            stop = size if step > 0 else -1
        if isinstance(start, int) and start < 0:
            start += size
        if isinstance(stop, int) and (stop < 0 if step > 0 else stop < -1):
            stop += size
        new_shape = list(self.shape)
        new_shape[dim] = (stop - start + step - (1 if step > 0 else -1)) // step
        return self._derive(new_shape, (_Link(self, "affine_dim", (dim, start, step)),), dtype=self.dtype)

    def __getitem__(self, indices):
        if not isinstance(indices, tuple):
            indices = (indices,)
        if indices.count(...) > 1:
            raise ValueError("Only one `Ellipsis` is allowed.")
        effective = len(indices) - indices.count(None) - indices.count(...)
        if effective > self.ndim:
            raise IndexError(f"Index `{indices}` is out of bounds for tensor of shape `{self.shape}`.")
        expanded = []
        for index in indices:
            if index is Ellipsis:
                expanded.extend([slice(None)] * (self.ndim - effective))
            else:
                expanded.append(index)
        out, dim = self, 0
        for index in expanded:
            if index is None:
                out = out.unsqueeze(dim)
                dim += 1
            elif isinstance(index, int):
                out = out._slice_dim(dim, index, index + 1).squeeze(dim)
            elif isinstance(index, slice):
                out = out._slice_dim(dim, index.start, index.stop, index.step)
                dim += 1
            else:
                raise TypeError(f"Index `{index}` must be an `int`, `slice`, or `None`, not `{type(index).__name__}`.")
        return out

    # ------------------------------------------------------------- inspection
    def symbol_names(self):
        """Names of every symbol the hierarchy's shapes and meta-op parameters use."""
        names = set()
        for node in _graph(self.levels()):
            names |= names_in(node.shape)
            for link in node._links:
                names |= names_in(link.params) if link.kind not in ("squeeze", "expand") else set()
        return names

    def symbols(self):
        """Symbol objects (with their constexpr/meta flags) used by the hierarchy."""
        found = {}

        def visit(v):
            if isinstance(v, Symbol):
                if v._op == "name":
                    prev = found.get(v.name)
                    if prev is None or (v.meta or v.constexpr):
                        found[v.name] = v
                else:
                    for a in v._args:
                        visit(a)
            elif isinstance(v, (tuple, list, frozenset)):
                for x in v:
                    visit(x)

        for node in _graph(self.levels()):
            visit(node.shape)
            for link in node._links:
                visit(link.params)
        return found

    def __repr__(self):
        return f"Tensor({self.name}, shape={self.shape})"

    # eval / subs are attached below (module functions with the reference's names)


def _eq(a, b):
    if isinstance(a, Symbol):
        return a == b
    return a == b


def _graph(levels):
    """Every tensor reachable from ``levels`` through links, newest first."""
    seen, stack = {}, list(levels)
    while stack:
        t = stack.pop()
        if t._id in seen:
            continue
        seen[t._id] = t
        for link in t._links:
            stack.append(link.target)
    return [seen[k] for k in sorted(seen, reverse=True)]


class BoundView:
    """An arranged hierarchy with every symbol bound: concrete shapes and index maps."""

    def __init__(self, top, env):
        self.top = top
        self.env = dict(env)
        self.levels = top.levels() if isinstance(top, Tensor) else []
        self.level_shapes = [tuple(int(v) for v in evaluate(t.shape, self.env)) for t in self.levels]
        self.source = top.source if isinstance(top, Tensor) else None
        self.source_shape = tuple(int(v) for v in evaluate(self.source.shape, self.env)) if self.source is not None else ()
        self._graph = _graph(self.levels)

    def probe(self, level_indices, record=None):
        """Source multi-index and mask for index arrays given per level.

        ``level_indices[i]`` is a tuple of integer arrays (one per dim of level i),
        all mutually broadcastable.  Returns (tuple of arrays over source dims, mask).
        """
        env = self.env
        contrib = {}
        for t, idx in zip(self.levels, level_indices):
            if len(idx) != t.ndim:
                raise ValueError(f"level {t} expects {t.ndim} indices, got {len(idx)}")
            contrib.setdefault(t._id, []).append(tuple(np.asarray(i, dtype=np.int64) for i in idx))
        mask = np.ones((), dtype=bool)
        source_idx = None
        for node in self._graph:
            parts = contrib.pop(node._id, None)
            if parts is None:
                continue
            idx = tuple(sum(p[d] for p in parts) for d in range(node.ndim))
            sizes = evaluate(node.shape, env)
            for i, s in zip(idx, sizes):
                mask = mask & (i >= 0) & (i < s)
            if record is not None:
                record[node._id] = idx
            if node._id == self.source._id:
                source_idx = idx
                continue
            for link in node._links:
                contrib.setdefault(link.target._id, []).append(link.apply(idx, env))
        if source_idx is None:
            raise RuntimeError("arranged tensor does not reach its source")
        shape = np.broadcast_shapes(mask.shape, *(np.shape(i) for i in source_idx))
        return tuple(np.broadcast_to(i, shape) for i in source_idx), np.broadcast_to(mask, shape)

    def full_index(self):
        """Index arrays enumerating every element of every level (open grid)."""
        dims = [s for shape in self.level_shapes for s in shape]
        grids = np.ix_(*[np.arange(s, dtype=np.int64) for s in dims]) if dims else ()
        out, pos = [], 0
        for shape in self.level_shapes:
            out.append(tuple(grids[pos : pos + len(shape)]))
            pos += len(shape)
        return out


def _default_env(tensor, subs=None):
    """Bindings for ``eval``: source shapes from ``subs`` (or concrete shapes), symbols by name."""
    env = {}
    subs = subs or {}
    for key, val in subs.items():
        if isinstance(key, Tensor):
            shape = val.shape if isinstance(val, Tensor) else val["shape"]
            for sym, size in zip(key.shape, shape):
                if isinstance(sym, Symbol) and sym.name:
                    env[sym.name] = int(evaluate(size, env))
        elif isinstance(key, Symbol):
            env[key.name] = val
        else:
            env[str(key)] = val
    return env


def _eval(tensor, subs=None):
    """Linear source offsets (contiguous strides) of every element, -1 where masked.

    The reference's ``ninetoothed.eval`` (``src/ninetoothed/eval.py:15-55``): the result
    has one axis per dimension of every level, outermost first.
    """
    if tensor.source.ndim == 0:
        return np.array(0, dtype=np.intp)
    env = dict(getattr(tensor, "_subs_env", {}))
    env.update(_default_env(tensor, subs))
    view = BoundView(tensor, env)
    idx, mask = view.probe(view.full_index())
    strides, acc = [], 1
    for s in reversed(view.source_shape):
        strides.append(acc)
        acc *= s
    strides.reverse()
    linear = sum(i * st for i, st in zip(idx, strides))
    shape = tuple(s for level in view.level_shapes for s in level)
    return np.broadcast_to(np.where(mask, linear, -1), shape).astype(np.intp)


def _subs(tensor, subs):
    """The tensor with symbol values recorded for later ``eval`` (reference ``eval.py:58-95``)."""
    out = copy.copy(tensor)
    env = dict(getattr(tensor, "_subs_env", {}))
    env.update(_default_env(tensor, subs))
    out._subs_env = env
    return out


Tensor.eval = _eval
Tensor.subs = _subs


def level_dims(tensor):
    return [t.ndim for t in tensor.levels()] if isinstance(tensor, Tensor) else []


def source_of(tensor):
    return tensor.source if isinstance(tensor, Tensor) else None


def numel(shape):
    return math.prod(shape)
