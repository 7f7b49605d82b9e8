"""Kernel families: recognise a lowered program and fit its arrangement to a kernel.

The MI355X backend has one hand-written kernel per family (GEMM with the addmm
epilogue, implicit-GEMM conv2d, fused attention, segmented row softmax, max_pool2d,
elementwise add).  Matching works in two steps, both structural, never by name (the
reference forbids operator dispatch in emitters, tests/test_emitter_boundaries.py:6-23):

1. Application: the frontend's value graph is matched against the family's dataflow
   pattern (``_match``: hash-consed nodes, commutative ``add``/``mul``/``maximum``
   tried both ways).  GEMM epilogues are read as a linear form
   ``beta * c + alpha * round(acc)`` over loaded blocks and scalar parameters.
2. Arrangement: the arranged tensors are evaluated at call time (``BoundView.probe``)
   on a few thousand sampled index points plus full sweeps of the reduction and
   output ranges, and the family's geometry hypothesis is checked exactly:
   e.g. for GEMM that the output element (m, n), the lhs element (m, k) and the rhs
   element (k, n) line up for every sampled program/k-step/block index, that masks
   are exactly the source bounds, and that every k < K is visited once.  Conv2d
   fits h = p*sh + r*dh - ph and w = q*sw + s*dw - pw by least squares and then checks
   the fit exactly.  A program that passes becomes a ``Plan`` bound to the kernel.

Anything that does not match raises ``LoweringError`` naming the family tried.
"""

import math

import numpy as np

from ninetoothed_amd import jagged
from ninetoothed_amd.errors import LoweringError
from ninetoothed_amd.frontend import Value

LOG2E = 1.44269504089

# ----------------------------------------------------------------------------- patterns


class _Any:
    def __repr__(self):
        return "_"


ANY = _Any()


class B:
    """Bind the matched value to ``name`` (same name twice must be the same node)."""

    def __init__(self, name, pat=ANY):
        self.name = name
        self.pat = pat


class P:
    """Match a node with operator ``op`` and argument patterns ``args``."""

    COMMUTATIVE = {"add", "mul", "maximum", "minimum", "eq", "ne"}

    def __init__(self, op, *args):
        self.op = op
        self.args = args


def _match(pat, v, b):
    """Return extended bindings or None."""
    if pat is ANY:
        return b
    if isinstance(pat, B):
        if pat.name in b:
            prev = b[pat.name]
            same = prev is v if isinstance(prev, Value) or isinstance(v, Value) else prev == v
            return b if same else None
        r = _match(pat.pat, v, b)
        if r is None:
            return None
        r = dict(r)
        r[pat.name] = v
        return r
    if isinstance(pat, P):
        if not isinstance(v, Value) or v.op != pat.op or len(v.args) != len(pat.args):
            return None
        orders = [v.args]
        if pat.op in P.COMMUTATIVE and len(v.args) == 2:
            orders.append((v.args[1], v.args[0]))
        for args in orders:
            r = b
            for pa, va in zip(pat.args, args):
                r = _match(pa, va, r)
                if r is None:
                    break
            if r is not None:
                return r
        return None
    if callable(pat) and not isinstance(pat, (int, float, str, tuple)):
        return b if pat(v) else None
    return b if pat == v else None


def _const(value):
    return P("const", value)


def _is_neg_inf(v):
    return isinstance(v, Value) and v.op == "const" and v.args[0] == float("-inf")


NEG_INF = _is_neg_inf


# ----------------------------------------------------------------------------- context


class CallContext:
    """Everything known at call time: the program, the bound views and the values."""

    def __init__(self, program, views, values, params, dtypes):
        self.program = program
        self.views = views  # param name -> BoundView (None for 0-d)
        self.values = values  # param name -> runtime value
        self.params = params  # param name -> ParamInfo
        self.dtypes = dtypes  # param name -> torch dtype (tensors only)
        self.relower = None  # unroll -> Program: the application lowered with loops unrolled

    def view(self, name):
        return self.views[name]


def _param_of_load(v, level=None):
    """``load(param x)`` (level 1) or ``load(index(param x, i))`` -> x."""
    if not (isinstance(v, Value) and v.op == "load"):
        return None
    t = v.args[0]
    if t.op == "param":
        return t.args[0] if level in (None, 1) else None
    return None


def _single_store(ctx):
    stores = ctx.program.stores
    if len(stores) != 1:
        raise LoweringError(f"expected exactly one output tensor, the application stores {sorted(stores)}")
    (name, value), = stores.items()
    return name, value


def _single_loop(ctx):
    if len(ctx.program.loops) != 1:
        return None
    return next(iter(ctx.program.loops.values()))


# ----------------------------------------------------------------------------- probing helpers

_RNG_SEED = 20250101


def _rand_idx(rng, shape, n):
    """n random multi-indices over ``shape`` plus the all-zero and all-max corners."""
    cols = []
    for s in shape:
        c = rng.integers(0, max(s, 1), size=n)
        c[0] = 0
        c[1] = max(s - 1, 0)
        cols.append(c.astype(np.int64))
    return tuple(cols)


def _inbounds(src, shape):
    ok = np.ones(np.shape(src[0]), dtype=bool)
    for i, s in zip(src, shape):
        ok &= (i >= 0) & (i < s)
    return ok


def _require(cond, family, why):
    if not cond:
        raise LoweringError(f"arrangement does not fit the {family} kernel: {why}")


def _levels(view, family, expect):
    shapes = view.level_shapes
    _require(len(shapes) == len(expect), family, f"tensor `{view.source.name}` has {len(shapes)} levels, expected {len(expect)}")
    for shape, nd in zip(shapes, expect):
        if nd is not None:
            _require(len(shape) == nd, family, f"level shape {shape} of `{view.source.name}` is not {nd}-D")
    return shapes


def _scalar_value(v):
    if hasattr(v, "item"):
        return float(v.item())
    return float(v)


# ----------------------------------------------------------------------------- plans


class Plan:
    """A matched program bound to one kernel family.

    ``bind(values, index)`` validates the sample ``values`` (parameter name -> value)
    against the kernel and returns ``launch(args)``, where ``args`` is a sequence
    laid out by ``index`` (parameter name -> position).  The launcher stays valid
    for every call whose tensors agree with the sample in dtype, shape, strides
    and device, and whose constexpr/meta values are the same.  ``run(values)``
    binds and launches once."""

    family = "?"

    def bind(self, values, index):
        raise NotImplementedError

    def check(self, values):
        """Raise ``TypeError`` / ``ValueError`` where the family's kernel would reject the
        call's dtypes or sizes (the check ``bind`` runs first), touching no device, so that
        ``select`` can hand such a call to the next family instead."""

    def run(self, values):
        names = tuple(values)
        self.bind(values, {n: i for i, n in enumerate(names)})(tuple(values[n] for n in names))

    def describe(self):
        return {"family": self.family}


# ============================================================================ GEMM / conv2d


def _lin_epilogue(v, acc_out, out_param, scalar_params):
    """Read ``v`` as sum_t coef_t * term_t; terms: ('acc', round_dtype) and ('c', param).

    Coefficients are lists of factors (floats or scalar-parameter names)."""
    if v is acc_out:
        return {("acc", None): [[1.0]]}
    if v.op == "cast" and v.args[0] is acc_out and v.args[1].op == "dtype":
        return {("acc", v.args[1].args[0]): [[1.0]]}
    if v.op == "load" and v.args[0].op == "param":
        name = v.args[0].args[0]
        if name in scalar_params:
            return {("scalar",): [[name]]}
        return {("c", name): [[1.0]]}
    if v.op == "const" and isinstance(v.args[0], (int, float)) and not isinstance(v.args[0], bool):
        return {("scalar",): [[float(v.args[0])]]}
    if v.op in ("add", "sub"):
        lhs = _lin_epilogue(v.args[0], acc_out, out_param, scalar_params)
        rhs = _lin_epilogue(v.args[1], acc_out, out_param, scalar_params)
        out = {k: list(c) for k, c in lhs.items()}
        for k, coefs in rhs.items():
            if v.op == "sub":
                coefs = [[-1.0] + c for c in coefs]
            out.setdefault(k, []).extend(coefs)
        return out
    if v.op == "neg":
        inner = _lin_epilogue(v.args[0], acc_out, out_param, scalar_params)
        return {k: [[-1.0] + c for c in coefs] for k, coefs in inner.items()}
    if v.op == "mul":
        lhs = _lin_epilogue(v.args[0], acc_out, out_param, scalar_params)
        rhs = _lin_epilogue(v.args[1], acc_out, out_param, scalar_params)
        for s, t in ((lhs, rhs), (rhs, lhs)):
            if set(s) == {("scalar",)}:
                return {k: [c1 + c2 for c1 in s[("scalar",)] for c2 in coefs] for k, coefs in t.items()}
        raise LoweringError("GEMM epilogue multiplies two tensors; only scalar scaling is supported")
    raise LoweringError(f"unsupported GEMM epilogue operation `{v.op}`")


class GemmPlan(Plan):
    family = "gemm"

    def __init__(self, a, b, out, c, alpha_factors, beta_factors, round_dtype, config=0):
        self.a, self.b, self.out, self.c = a, b, out, c
        self.alpha_factors, self.beta_factors = alpha_factors, beta_factors
        self.round_dtype = round_dtype
        self.config = config  # 0: the library picks the kernel; else one forced kernel

    def with_config(self, config):
        return GemmPlan(self.a, self.b, self.out, self.c, self.alpha_factors, self.beta_factors, self.round_dtype,
                        config)

    @staticmethod
    def _coef_fn(factors, index):
        """args -> sum over terms of the product of its factors (constants or scalar arguments)."""
        const, terms = 0.0, []
        for term in factors:
            x, names = 1.0, []
            for f in term:
                if isinstance(f, str):
                    names.append(index[f])
                else:
                    x *= f
            if names:
                terms.append((x, tuple(names)))
            else:
                const += x
        if not terms:
            return lambda args: const

        def coef(args):
            total = const
            for x, positions in terms:
                for i in positions:
                    x *= _scalar_value(args[i])
                total += x
            return total

        return coef

    def check(self, values):
        from ninetoothed_amd import kernels

        kernels.check_gemm(values[self.a], values[self.b], values[self.out], values[self.c] if self.c else None,
                           self.round_dtype, self.config)

    def bind(self, values, index):
        from ninetoothed_amd import kernels

        launch = kernels.bind_gemm(values[self.a], values[self.b], values[self.out],
                                   values[self.c] if self.c else None, round_dtype=self.round_dtype,
                                   config=self.config)
        ia, ib, io = index[self.a], index[self.b], index[self.out]
        ic = index[self.c] if self.c else None
        alpha = self._coef_fn(self.alpha_factors, index)
        beta = self._coef_fn(self.beta_factors, index) if self.c else (lambda args: 0.0)

        def run(args):
            launch(args[ia], args[ib], args[io], args[ic] if ic is not None else None, alpha(args), beta(args))

        return run

    def describe(self):
        d = {"family": "gemm", "a": self.a, "b": self.b, "out": self.out, "c": self.c, "round": str(self.round_dtype)}
        if self.config:
            d["config"] = self.config
        return d


class ConvPlan(Plan):
    family = "conv2d"

    def __init__(self, x, w, y, padding, stride, dilation, round_dtype, config=0):
        self.x, self.w, self.y = x, w, y
        self.padding, self.stride, self.dilation = padding, stride, dilation
        self.round_dtype = round_dtype
        self.config = config  # 0: the library picks the path; else one forced path

    def with_config(self, config):
        return ConvPlan(self.x, self.w, self.y, self.padding, self.stride, self.dilation, self.round_dtype, config)

    def check(self, values):
        from ninetoothed_amd import kernels

        kernels.check_conv2d(values[self.x], values[self.w], values[self.y], self.round_dtype, self.config)

    def bind(self, values, index):
        import torch

        from ninetoothed_amd import kernels

        x, w, y = values[self.x], values[self.w], values[self.y]
        nbytes = 0 if self.config == 3 else kernels.conv2d_workspace_bytes(x, w, self.padding)
        launch = kernels.bind_conv2d(x, w, y, padding=self.padding, stride=self.stride, dilation=self.dilation,
                                     round_dtype=self.round_dtype, workspace_bytes=nbytes, config=self.config)
        ix, iw, iy = index[self.x], index[self.w], index[self.y]
        device = x.device

        def run(args):
            # The re-layout workspace comes from torch's stream-ordered caching allocator
            # on every call, so calls on different streams never share one.
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None
            launch(args[ix], args[iw], args[iy], workspace)

        return run

    def describe(self):
        d = {"family": "conv2d", "padding": self.padding, "stride": self.stride, "dilation": self.dilation,
             "round": str(self.round_dtype)}
        if self.config:
            d["config"] = self.config
        return d


def _torch_dtype(name):
    import torch

    return {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}.get(name)


def match_gemm(ctx):
    family = "gemm"
    out, value = _single_store(ctx)
    loop = _single_loop(ctx)
    if loop is None:
        return None
    acc_name = None
    for name, upd in loop.update.items():
        b = _match(
            P("add", P("carried", loop.id, name),
              P("dot", P("load", P("index", P("param", B("A")), P("loop_index", loop.id))),
                P("load", P("index", P("param", B("B")), P("loop_index", loop.id))))),
            upd, {})
        if b is not None:
            acc_name, binds = name, b
            break
    if acc_name is None:
        return None
    init = loop.init[acc_name]
    if not (isinstance(init, Value) and init.op == "zeros" and init.args[1].op == "dtype" and init.args[1].args[0] == "float32"):
        return None
    a_name, b_name = binds["A"], binds["B"]
    if _match(P("shape", P("param", a_name), 0), loop.trip, {}) is None and _match(P("shape", P("param", b_name), 0), loop.trip, {}) is None:
        return None
    if len(loop.update) != 1:
        return None
    acc_out = None
    for v in _walk(value):
        if v.op == "loop_out" and v.args == (loop.id, acc_name):
            acc_out = v
    if acc_out is None:
        return None
    scalars = {n for n, p in ctx.params.items() if p.source_ndim == 0 and not p.constexpr}
    lin = _lin_epilogue(value, acc_out, out, scalars)
    acc_terms = [k for k in lin if k[0] == "acc"]
    c_terms = [k for k in lin if k[0] == "c"]
    if len(acc_terms) != 1 or len(c_terms) > 1 or ("scalar",) in lin:
        raise LoweringError("GEMM epilogue must be alpha * acc (+ beta * c)")
    round_name = acc_terms[0][1]
    round_dtype = _torch_dtype(round_name) if round_name else None
    if round_name and round_dtype is None:
        raise LoweringError(f"GEMM accumulator cast to {round_name} is not supported")
    c_name = c_terms[0][1] if c_terms else None
    alpha = lin[acc_terms[0]]
    beta = lin[c_terms[0]] if c_terms else [[0.0]]

    va, vb, vo = ctx.view(a_name), ctx.view(b_name), ctx.view(out)
    src_nd = (len(va.source_shape), len(vb.source_shape), len(vo.source_shape))
    if src_nd == (2, 2, 2):
        _fit_plain_gemm(ctx, va, vb, vo, c_name)
        return GemmPlan(a_name, b_name, out, c_name, alpha, beta, round_dtype)
    if src_nd == (4, 4, 4) and c_name is None:
        if any(len(t) != 1 or t[0] != 1.0 for t in alpha):
            raise LoweringError("conv2d epilogue scaling is not supported")
        padding, stride, dilation = _fit_conv(ctx, va, vb, vo)
        return ConvPlan(a_name, b_name, out, padding, stride, dilation, round_dtype)
    raise LoweringError(f"GEMM operands with source ranks {src_nd} fit neither the GEMM nor the conv2d kernel")


def _walk(v, seen=None):
    seen = set() if seen is None else seen
    stack = [v]
    while stack:
        x = stack.pop()
        if not isinstance(x, Value) or id(x) in seen:
            continue
        seen.add(id(x))
        yield x
        for a in x.args:
            if isinstance(a, Value):
                stack.append(a)
            elif isinstance(a, tuple):
                stack.extend(y for y in a if isinstance(y, Value))


def _gemm_samples(family, va, vb, vo, n=4096):
    so = _levels(vo, family, (None, 2))
    sa = _levels(va, family, (None, 1, 2))
    sb = _levels(vb, family, (None, 1, 2))
    _require(sa[0] == so[0] and sb[0] == so[0], family, "operands disagree on the launch grid")
    _require(sa[1] == sb[1], family, "operands disagree on the number of k-steps")
    bm, bn = so[1]
    _require(sa[2][0] == bm and sb[2][1] == bn and sa[2][1] == sb[2][0], family, "block shapes do not chain")
    bk = sa[2][1]
    rng = np.random.default_rng(_RNG_SEED)
    g = _rand_idx(rng, so[0], n)
    (kk,) = _rand_idx(rng, sa[1], n)
    (i,) = _rand_idx(rng, (bm,), n)
    (j,) = _rand_idx(rng, (bn,), n)
    (l,) = _rand_idx(rng, (bk,), n)
    return so, sa, sb, g, kk, i, j, l


def _fit_plain_gemm(ctx, va, vb, vo, c_name):
    family = "gemm"
    so, sa, sb, g, kk, i, j, l = _gemm_samples(family, va, vb, vo)
    o_src, o_mask = vo.probe([g, (i, j)])
    a_src, a_mask = va.probe([g, (kk,), (i, l)])
    b_src, b_mask = vb.probe([g, (kk,), (l, j)])
    _require(np.array_equal(a_src[0], o_src[0]), family, "lhs rows do not follow output rows")
    _require(np.array_equal(b_src[1], o_src[1]), family, "rhs columns do not follow output columns")
    _require(np.array_equal(a_src[1], b_src[0]), family, "lhs and rhs disagree on k")
    for src, mask, view in ((o_src, o_mask, vo), (a_src, a_mask, va), (b_src, b_mask, vb)):
        _require(np.array_equal(mask, _inbounds(src, view.source_shape)), family, f"mask of `{view.source.name}` is not its bounds")
    M, N = vo.source_shape
    K = va.source_shape[1]
    _require(va.source_shape[0] == M and vb.source_shape == (K, N), family, "operand shapes do not chain")
    _check_k_coverage(family, va, vb, g, i, j, o_mask, K, lambda a, b: a[1], lambda a, b: b[0])
    _check_output_coverage(family, vo, so, (M, N))
    if c_name is not None:
        vc = ctx.view(c_name)
        _require(vc.level_shapes == vo.level_shapes, family, "bias operand is not arranged like the output")
        c_src, c_mask = vc.probe([g, (i, j)])
        _require(all(np.array_equal(x, y) for x, y in zip(c_src, o_src)) and np.array_equal(c_mask, o_mask),
                 family, "bias operand does not line up with the output")


def _check_k_coverage(family, va, vb, g, i, j, o_mask, K, k_of_a, k_of_b, extra=None, masks_agree=True):
    """At one in-bounds output element every reduction index must be visited once.

    A reduction step counts as visited where the rhs element is in bounds; the lhs
    may be masked there only when it reads zero-filled padding (conv2d)."""
    valid = np.nonzero(o_mask)[0]
    _require(valid.size > 0, family, "no in-bounds output sample")
    s = valid[0]
    g1 = tuple(np.array([x[s]]) for x in g)
    nk = va.level_shapes[1][0]
    bk = va.level_shapes[2][1]
    kk = np.arange(nk, dtype=np.int64)[:, None]
    ll = np.arange(bk, dtype=np.int64)[None, :]
    ii = np.array([[i[s]]])
    jj = np.array([[j[s]]])
    a_src, a_mask = va.probe([tuple(x[:, None] for x in g1), (kk,), (ii, ll)])
    b_src, b_mask = vb.probe([tuple(x[:, None] for x in g1), (kk,), (ll, jj)])
    if masks_agree:
        _require(np.array_equal(a_mask, b_mask), family, "lhs and rhs disagree on which reduction steps exist")
    ka = k_of_a(a_src, b_src)[b_mask]
    kb = k_of_b(a_src, b_src)[b_mask]
    _require(np.array_equal(ka, kb), family, "lhs/rhs reduction indices differ")
    if extra is not None:
        extra(a_src, b_src, b_mask)
    _require(np.array_equal(np.sort(ka), np.arange(K)), family, "reduction does not visit every index exactly once")


_EXHAUSTIVE_LIMIT = 1 << 21


def _check_output_coverage(family, vo, so, full_shape, block_axis=None):
    """Every output element is written exactly once by the launch grid.

    Exhaustive for up to 2**21 grid x block positions; above that, 64 sampled programs
    (plus the first and last) are swept whole and must write distinct in-bounds
    elements, and the grid must have the capacity to cover the output."""
    grid, block = so[0], so[1]
    total = math.prod(grid) * math.prod(block)
    numel = math.prod(vo.source_shape)
    bi = np.indices(block).reshape(len(block), -1)
    b = tuple(x[None, :] for x in bi)
    if total <= _EXHAUSTIVE_LIMIT:
        gi = np.indices(grid).reshape(len(grid), -1)
    else:
        _require(total >= numel, family, "the launch grid is too small for the output")
        rng = np.random.default_rng(_RNG_SEED)
        count = math.prod(grid)
        picks = np.unique(np.concatenate([[0, count - 1], rng.integers(0, count, 64)]))
        gi = np.stack(np.unravel_index(picks, grid))
    g = tuple(x[:, None] for x in gi)
    src, mask = vo.probe([g, b])
    flat = np.ravel_multi_index(tuple(np.broadcast_to(x, mask.shape)[mask] for x in src), vo.source_shape)
    _require(np.unique(flat).size == flat.size, family, "two program positions write the same output element")
    if total <= _EXHAUSTIVE_LIMIT:
        _require(flat.size == numel, family, "the launch grid does not write every output element")


def _fit_conv(ctx, vx, vw, vy):
    family = "conv2d"
    so, sa, sb, g, kk, i, j, l = _gemm_samples(family, vx, vw, vy)
    y_src, y_mask = vy.probe([g, (i, j)])
    x_src, x_mask = vx.probe([g, (kk,), (i, l)])
    w_src, w_mask = vw.probe([g, (kk,), (l, j)])
    n, ko, p, q = y_src
    n2, c, h, w = x_src
    ko2, c2, r, s = w_src
    _require(np.array_equal(n, n2), family, "input batch index does not follow the output's")
    _require(np.array_equal(ko, ko2), family, "filter rows do not follow output channels")
    _require(np.array_equal(c, c2), family, "input and filter channels differ")

    N, K, P, Q = vy.source_shape
    _, C, H, W = vx.source_shape
    K2, C2, R, S = vw.source_shape

    def fit(out_pos, win, coord, n_out, n_win):
        # coord = out_pos * stride + win * dilation - padding.  An axis of one output position
        # (P or Q of 1) leaves the stride free, a filter axis of one tap (R or S of 1) the
        # dilation: such an index is 0 throughout, so its coefficient is taken as 1 and only
        # the others are fitted.
        free_st, free_dl = n_out == 1, n_win == 1
        cols = [c for c, free in ((out_pos, free_st), (win, free_dl)) if not free]
        A = np.stack(cols + [np.ones_like(out_pos)], axis=1).astype(np.float64)
        sol = iter(int(round(x)) for x in np.linalg.lstsq(A, coord.astype(np.float64), rcond=None)[0])
        st = 1 if free_st else next(sol)
        dl = 1 if free_dl else next(sol)
        off = next(sol)
        _require(np.array_equal(out_pos * st + win * dl + off, coord), family, "window positions are not affine")
        return st, dl, -off

    sh, dh, ph = fit(p, r, h, P, R)
    sw, dw, pw = fit(q, s, w, Q, S)
    _require(K2 == K and C2 == C, family, "filter shape does not match the input/output channels")
    _require(sh > 0 and sw > 0 and dh > 0 and dw > 0 and ph >= 0 and pw >= 0, family, "unsupported stride/padding")
    for src, mask, view in ((y_src, y_mask, vy), (w_src, w_mask, vw), (x_src, x_mask, vx)):
        _require(np.array_equal(mask, _inbounds(src, view.source_shape)), family, f"mask of `{view.source.name}` is not its bounds")

    def crs(a, b, both):
        key = (b[1] * R + b[2]) * S + b[3]
        _require(np.array_equal(np.sort(key[both]), np.arange(C * R * S)), family, "filter taps are not each visited once")

    _check_k_coverage(family, vx, vw, g, i, j, y_mask, C * R * S,
                      lambda a, b: (b[1] * R + b[2]) * S + b[3], lambda a, b: (b[1] * R + b[2]) * S + b[3], extra=crs,
                      masks_agree=False)
    _check_output_coverage(family, vy, so, vy.source_shape)
    return (ph, pw), (sh, sw), (dh, dw)


# ============================================================================ attention


def _attention_pattern(loop_id, causal):
    q = P("param", B("q"))
    ki = P("index", P("param", B("k")), P("loop_index", loop_id))
    vi = P("index", P("param", B("v")), P("loop_index", loop_id))
    q_loaded = P("cast", P("mul", P("load", q), B("scale", P("const", ANY))), P("dtype_of", q))
    dot_qk = P("dot", q_loaded, P("trans", P("load", ki)))
    bounds = P("lt", P("offsets", ki, 2), P("source_shape", B("k"), 2))
    qk0 = P("where", bounds, dot_qk, NEG_INF)
    if causal:
        cmask = P("ge", P("bcast", P("offsets", q, 2), (":", None)), P("bcast", P("offsets", ki, 2), (None, ":")))
        qk = P("where", cmask, qk0, NEG_INF)
    else:
        qk = qk0
    return q, ki, vi, qk


def match_attention(ctx):
    family = "attention"
    out, value = _single_store(ctx)
    loop = _single_loop(ctx)
    if loop is None or len(loop.update) != 3:
        return None
    # identify carried names by role through the update structure
    upd = loop.update
    names = list(upd)
    result = None
    for causal in (False, True):
        q, ki, vi, qk = _attention_pattern(loop.id, causal)
        for acc_n in names:
            for m_n in names:
                for l_n in names:
                    if len({acc_n, m_n, l_n}) != 3:
                        continue
                    m_ij = P("maximum", P("carried", loop.id, m_n), P("reduce", "max", qk, 1))
                    b = _match(B("m_ij", m_ij), upd[m_n], {})
                    if b is None:
                        continue
                    p = P("math", "exp2", P("sub", qk, P("bcast", B("m_ij"), (":", None))))
                    alpha = P("math", "exp2", P("sub", P("carried", loop.id, m_n), B("m_ij")))
                    l_pat = P("add", P("mul", P("carried", loop.id, l_n), alpha), P("reduce", "sum", p, 1))
                    b2 = _match(l_pat, upd[l_n], b)
                    if b2 is None:
                        continue
                    acc_pat = P("add", P("mul", P("carried", loop.id, acc_n), P("bcast", alpha, (":", None))),
                                P("dot", P("cast", p, P("dtype_of", vi)), P("load", vi)))
                    b3 = _match(acc_pat, upd[acc_n], b2)
                    if b3 is None:
                        continue
                    fin = P("div", P("loop_out", loop.id, acc_n), P("bcast", P("loop_out", loop.id, l_n), (":", None)))
                    b4 = _match(fin, value, b3)
                    if b4 is None:
                        continue
                    result = (causal, b4, acc_n, m_n, l_n)
                    break
                if result:
                    break
            if result:
                break
        if result:
            break
    if result is None:
        return None
    causal, b, acc_n, m_n, l_n = result
    # initial values: acc = zeros(fp32), l = full(1), m = full(-inf)
    init = loop.init
    ok = (init[acc_n].op == "zeros" and init[l_n].op == "full" and init[l_n].args[1] == 1.0
          and init[m_n].op == "full" and init[m_n].args[1] == float("-inf"))
    if not ok:
        raise LoweringError("attention accumulators have unexpected initial values")
    if _match(P("shape", P("param", b["k"]), 0), loop.trip, {}) is None:
        return None
    qn, kn, vn = b["q"], b["k"], b["v"]
    scale = float(b["scale"].args[0])
    _fit_attention(ctx, qn, kn, vn, out)
    return AttentionPlan(qn, kn, vn, out, scale, causal)


class AttentionPlan(Plan):
    family = "attention"

    def __init__(self, q, k, v, o, scale, causal, config=0):
        self.q, self.k, self.v, self.o = q, k, v, o
        self.scale = scale
        self.causal = causal
        self.config = config  # 0: the library picks the kernel; else one forced kernel

    def with_config(self, config):
        return AttentionPlan(self.q, self.k, self.v, self.o, self.scale, self.causal, config)

    def check(self, values):
        from ninetoothed_amd import kernels

        kernels.check_attention(values[self.q], values[self.k], values[self.v], values[self.o], self.config)

    def bind(self, values, index):
        import torch

        from ninetoothed_amd import kernels

        q = values[self.q]
        scale = self.scale
        if q.dtype in (torch.float16, torch.bfloat16):
            # A Python float literal in `q * c` takes the tensor's type (weak typing of
            # scalars in the reference's generated kernel): c is rounded to q's dtype.
            scale = float(torch.tensor(scale, dtype=q.dtype))
        launch = kernels.bind_attention(q, values[self.k], values[self.v], values[self.o], causal=self.causal,
                                        q_scale=scale, config=self.config)
        iq, ik, iv, io = index[self.q], index[self.k], index[self.v], index[self.o]

        def run(args):
            launch(args[iq], args[ik], args[iv], args[io])

        return run

    def describe(self):
        d = {"family": "attention", "causal": self.causal, "scale": self.scale}
        if self.config:
            d["config"] = self.config
        return d


def _fit_attention(ctx, qn, kn, vn, on):
    family = "attention"
    vq, vk, vv, vo = (ctx.view(x) for x in (qn, kn, vn, on))
    sq = _levels(vq, family, (4, 2))
    sk = _levels(vk, family, (4, 1, 2))
    _require(_levels(vo, family, (4, 2)) == sq and _levels(vv, family, (4, 1, 2)) == sk, family,
             "q/o or k/v are arranged differently")
    _require(sk[0] == sq[0], family, "k/v are not broadcast over the query programs")
    Bq, Hq, Sq, D = vq.source_shape
    _require(vo.source_shape == vq.source_shape, family, "output shape differs from q")
    _require(vk.source_shape[:2] == (Bq, Hq) and vv.source_shape == vk.source_shape and vk.source_shape[3] == D, family,
             "k/v shapes do not match q")
    Sk = vk.source_shape[2]
    bm, dq = sq[1]
    bn, dk = sk[2]
    _require(dq == D and dk == D, family, "the head dimension is tiled; the kernel needs whole rows")
    rng = np.random.default_rng(_RNG_SEED)
    n = 4096
    g = _rand_idx(rng, sq[0], n)
    (kk,) = _rand_idx(rng, sk[1], n)
    (i,) = _rand_idx(rng, (bm,), n)
    (j,) = _rand_idx(rng, (bn,), n)
    (d,) = _rand_idx(rng, (D,), n)
    q_src, q_mask = vq.probe([g, (i, d)])
    o_src, o_mask = vo.probe([g, (i, d)])
    k_src, k_mask = vk.probe([g, (kk,), (j, d)])
    v_src, v_mask = vv.probe([g, (kk,), (j, d)])
    _require(all(np.array_equal(x, y) for x, y in zip(q_src, o_src)), family, "o is not arranged like q")
    _require(all(np.array_equal(x, y) for x, y in zip(k_src, v_src)), family, "v is not arranged like k")
    _require(np.array_equal(k_src[0], q_src[0]) and np.array_equal(k_src[1], q_src[1]), family,
             "keys come from another batch/head than the queries")
    _require(np.array_equal(q_src[3], d) and np.array_equal(k_src[3], d), family, "head-dimension index is permuted")
    for src, mask, view in ((q_src, q_mask, vq), (k_src, k_mask, vk)):
        _require(np.array_equal(mask, _inbounds(src, view.source_shape)), family, f"mask of `{view.source.name}` is not its bounds")
    # every key visited once per query program
    valid = np.nonzero(q_mask)[0]
    _require(valid.size > 0, family, "no in-bounds query sample")
    s = valid[0]
    g1 = tuple(np.array([[x[s]]]) for x in g)
    kk_all = np.arange(sk[1][0])[:, None]
    jj = np.arange(bn)[None, :]
    src, mask = vk.probe([g1, (kk_all,), (jj, np.zeros((1, 1), dtype=np.int64))])
    keys = src[2][mask]
    _require(np.array_equal(np.sort(keys), np.arange(Sk)), family, "key blocks do not cover every key exactly once")
    _check_output_coverage(family, vo, sq, vo.source_shape)


# ============================================================================ softmax


class SoftmaxPlan(Plan):
    family = "softmax"

    def __init__(self, x, y, block, config=0):
        self.x, self.y, self.block = x, y, block
        self.config = config  # 0: the library picks the kernel; else one forced kernel

    def with_config(self, config):
        return SoftmaxPlan(self.x, self.y, self.block, config)

    def check(self, values):
        from ninetoothed_amd import kernels

        kernels.check_softmax(values[self.x], values[self.y], self.config)

    def bind(self, values, index):
        from ninetoothed_amd import kernels

        launch = kernels.bind_softmax(values[self.x], values[self.y], block=self.block, config=self.config)
        ix, iy = index[self.x], index[self.y]

        def run(args):
            launch(args[ix], args[iy])

        return run

    def describe(self):
        d = {"family": "softmax", "block": self.block}
        if self.config:
            d["config"] = self.config
        return d


def match_softmax(ctx):
    family = "softmax"
    out, value = _single_store(ctx)
    if ctx.program.loops:
        return None
    x = P("load", P("param", B("x")))
    num = P("math", "exp", P("sub", x, P("reduce", "max", x, None)))
    pat = P("div", B("num", num), P("reduce", "sum", B("num"), None))
    b = _match(pat, value, {})
    if b is None:
        return None
    xn = b["x"]
    vx, vy = ctx.view(xn), ctx.view(out)
    sx = _levels(vx, family, (2, 2))
    _require(_levels(vy, family, (2, 2)) == sx, family, "input and output are arranged differently")
    _require(sx[1][0] == 1, family, "a program must cover part of a single row")
    R, C = vx.source_shape
    _require(vy.source_shape == (R, C), family, "input and output shapes differ")
    bs = sx[1][1]
    rng = np.random.default_rng(_RNG_SEED)
    g = _rand_idx(rng, sx[0], 4096)
    (t,) = _rand_idx(rng, (bs,), 4096)
    z = np.zeros_like(t)
    x_src, x_mask = vx.probe([g, (z, t)])
    y_src, y_mask = vy.probe([g, (z, t)])
    _require(all(np.array_equal(a, b) for a, b in zip(x_src, y_src)) and np.array_equal(x_mask, y_mask), family,
             "input and output elements do not line up")
    _require(np.array_equal(x_src[0], g[0]) and np.array_equal(x_src[1], g[1] * bs + t), family,
             "programs are not (row, segment of BLOCK_SIZE columns)")
    _require(sx[0] == (R, -(-C // bs)), family, "launch grid does not cover rows x segments")
    _require(np.array_equal(x_mask, _inbounds(x_src, (R, C))), family, "mask is not the input bounds")
    other = vx.source.other
    if C % bs != 0:
        _require(other is not None and float(other) == float("-inf"), family,
                 "a partial segment needs other=-inf to be excluded from the softmax")
    return SoftmaxPlan(xn, out, bs)


# ============================================================================ max_pool2d


class MaxPoolPlan(Plan):
    family = "max_pool2d"

    def __init__(self, x, y, window, stride, padding, dilation, config=0):
        self.x, self.y = x, y
        self.window, self.stride, self.padding, self.dilation = window, stride, padding, dilation
        self.config = config  # 0: the library picks the kernel; else one forced kernel

    def with_config(self, config):
        return MaxPoolPlan(self.x, self.y, self.window, self.stride, self.padding, self.dilation, config)

    def check(self, values):
        from ninetoothed_amd import kernels

        kernels.check_max_pool2d(values[self.x], values[self.y], self.config)

    def bind(self, values, index):
        from ninetoothed_amd import kernels

        launch = kernels.bind_max_pool2d(values[self.x], values[self.y], self.window, stride=self.stride,
                                         padding=self.padding, dilation=self.dilation, config=self.config)
        ix, iy = index[self.x], index[self.y]

        def run(args):
            launch(args[ix], args[iy])

        return run

    def describe(self):
        d = {"family": "max_pool2d", "window": self.window, "stride": self.stride, "padding": self.padding}
        if self.config:
            d["config"] = self.config
        return d


def match_max_pool2d(ctx):
    family = "max_pool2d"
    out, value = _single_store(ctx)
    if ctx.program.loops:
        return None
    b = _match(P("reduce", "max", P("load", P("param", B("x"))), 1), value, {})
    if b is None:
        return None
    xn = b["x"]
    vx, vy = ctx.view(xn), ctx.view(out)
    if len(vx.source_shape) != 4 or len(vy.source_shape) != 4:
        return None
    sx = _levels(vx, family, (None, 2))
    sy = _levels(vy, family, (None, 1))
    _require(sx[0] == sy[0] and sx[1][0] == sy[1][0], family, "input and output disagree on programs")
    bs, win = sx[1]
    rng = np.random.default_rng(_RNG_SEED)
    n = 4096
    g = _rand_idx(rng, sx[0], n)
    (o,) = _rand_idx(rng, (bs,), n)
    (t,) = _rand_idx(rng, (win,), n)
    y_src, y_mask = vy.probe([g, (o,)])
    x_src, x_mask = vx.probe([g, (o, t)])
    n_, c, p, q = y_src
    n2, c2, h, w = x_src
    _require(np.array_equal(n_, n2) and np.array_equal(c, c2), family, "windows leave their (batch, channel) plane")
    # stride from t == 0 samples, then per-tap offsets
    z = np.zeros_like(o)
    x0, _ = vx.probe([g, (o, z)])
    sh = _slope(p, x0[2], family)
    sw = _slope(q, x0[3], family)
    off_h = h - p * sh
    off_w = w - q * sw
    taps = np.arange(win)
    g0 = tuple(np.full(win, x[0]) for x in g)
    xt, _ = vx.probe([g0, (np.full(win, o[0]), taps)])
    yt, _ = vy.probe([tuple(np.array([x[0]]) for x in g), (np.array([o[0]]),)])
    tap_h = xt[2] - yt[2][0] * sh
    tap_w = xt[3] - yt[3][0] * sw
    _require(np.array_equal(off_h, tap_h[t]) and np.array_equal(off_w, tap_w[t]), family, "window taps are not fixed offsets")
    hs, ws = np.unique(tap_h), np.unique(tap_w)
    kh, kw = hs.size, ws.size
    dh = int(hs[1] - hs[0]) if kh > 1 else 1
    dw = int(ws[1] - ws[0]) if kw > 1 else 1
    ph, pw = int(-hs[0]), int(-ws[0])
    grid_taps = {(int(-ph + r * dh), int(-pw + s * dw)) for r in range(kh) for s in range(kw)}
    _require(set(zip(tap_h.tolist(), tap_w.tolist())) == grid_taps and win == kh * kw, family,
             "window taps do not form a (dilated) rectangle")
    _require(ph >= 0 and pw >= 0, family, "windows start after their output position")
    _require(np.array_equal(y_mask, _inbounds(y_src, vy.source_shape)), family, "output mask is not its bounds")
    _require(np.array_equal(x_mask, _inbounds(x_src, vx.source_shape) & y_mask), family, "input mask is not its bounds")
    N, C, H, W = vx.source_shape
    N2, C2, P_, Q_ = vy.source_shape
    _require((N, C) == (N2, C2), family, "batch/channel sizes differ")
    outside = bool(((h < 0) | (h >= H) | (w < 0) | (w >= W))[y_mask].any())
    other = vx.source.other
    if outside:
        _require(other is not None and float(other) == float("-inf"), family,
                 "windows reach outside the input, which needs other=-inf")
    _check_output_coverage(family, vy, sy, vy.source_shape)
    return MaxPoolPlan(xn, out, (kh, kw), (sh, sw), (ph, pw), (dh, dw))


def _slope(pos, coord, family):
    A = np.stack([pos, np.ones_like(pos)], axis=1).astype(np.float64)
    sol, *_ = np.linalg.lstsq(A, coord.astype(np.float64), rcond=None)
    st = int(round(sol[0]))
    _require(st > 0, family, "non-positive window stride")
    return st


# ============================================================================ add


class AddPlan(Plan):
    family = "add"

    def __init__(self, a, b, out):
        self.a, self.b, self.out = a, b, out

    def check(self, values):
        from ninetoothed_amd import kernels

        a, b, o = values[self.a], values[self.b], values[self.out]
        kernels.check_add(a.reshape(-1), b.reshape(-1), o.reshape(-1))

    def bind(self, values, index):
        from ninetoothed_amd import kernels

        a, b, o = values[self.a], values[self.b], values[self.out]
        if o.dim() != 1:
            # Same-shaped operands walked as one flat range: each must be viewable as 1-D
            # (a view keeps its data pointer, so the launcher takes the original tensors).
            a, b, o = a.view(-1), b.view(-1), o.view(-1)
        launch = kernels.bind_add(a, b, o)
        ia, ib, io = index[self.a], index[self.b], index[self.out]

        def run(args):
            launch(args[ia], args[ib], args[io])

        return run

    def describe(self):
        return {"family": "add"}


def match_add(ctx):
    family = "add"
    out, value = _single_store(ctx)
    if ctx.program.loops:
        return None
    b = _match(P("add", P("load", P("param", B("a"))), P("load", P("param", B("b")))), value, {})
    if b is None:
        return None
    an, bn = b["a"], b["b"]
    import torch

    dts = {ctx.dtypes.get(n) for n in (an, bn, out)}
    if len(dts) != 1 or dts.pop() not in (torch.float32, torch.float16, torch.bfloat16):
        return None  # mixed or other dtypes: the generic kernels promote as the reference does
    va, vb, vo = ctx.view(an), ctx.view(bn), ctx.view(out)
    _require(va.level_shapes == vo.level_shapes == vb.level_shapes, family, "operands are arranged differently")
    _require(va.source_shape == vb.source_shape == vo.source_shape, family, "operand shapes differ")
    rng = np.random.default_rng(_RNG_SEED)
    idx = [_rand_idx(rng, s, 4096) for s in vo.level_shapes]
    srcs = [v.probe(idx) for v in (va, vb, vo)]
    _require(all(all(np.array_equal(x, y) for x, y in zip(s[0], srcs[2][0])) and np.array_equal(s[1], srcs[2][1])
                 for s in srcs), family, "operand elements do not line up")
    _require(np.array_equal(srcs[2][1], _inbounds(srcs[2][0], vo.source_shape)), family, "mask is not the bounds")
    _check_output_coverage(family, vo, vo.level_shapes[:2] if len(vo.level_shapes) == 2 else vo.level_shapes,
                           vo.source_shape)
    if len(vo.source_shape) != 1:
        for n in (an, bn, out):
            _require(ctx.values[n].is_contiguous(), family, "multi-dimensional operands must be contiguous")
    return AddPlan(an, bn, out)


def match_generic(ctx):
    from ninetoothed_amd import generic

    return generic.match_generic(ctx)


FAMILIES = (match_attention, match_gemm, match_softmax, match_max_pool2d, match_add, match_generic)


def _families_for(ctx):
    """The families a call may take: a call with a jagged tensor takes the generic kernels,
    whose index tables follow each batch's rows (ninetoothed_amd.jagged); the hand-written
    kernels address strided tensors only."""
    if any(jagged.is_jagged(v) for v in ctx.values.values()):
        return (match_generic,)
    return FAMILIES


def candidates(ctx):
    """Every family plan whose pattern and geometry fit, in the order ``select`` tries them.

    A GEMM plan stands for each of the 16-bit GEMM's kernel configurations (the DMA kernel,
    the register-staged one, the element-wise loader one), a conv2d plan for each of the
    convolution's paths (re-laid input through the DMA or the N-H-W-C kernel, the direct
    kernel), an attention plan for each attention kernel (pipelined one-wave-per-SIMD,
    eight-wave, four-wave), a softmax plan for each softmax kernel (register path with four,
    eight or one wave per workgroup, two-sweep) and a max_pool2d plan for each pooling kernel
    (pair-row or plane, element-wise, flat, LDS strip): configurations the call's
    operands do not admit fail when bound or launched and drop out of the timing.  A generic
    tile program with real loops is a candidate only where no other plan fits."""
    from ninetoothed_amd import kernels

    plans = []
    for matcher in _families_for(ctx):
        try:
            plan = matcher(ctx)
            if plan is not None:
                plan.check(ctx.values)
        except (LoweringError, TypeError, ValueError):
            plan = None
        if isinstance(plan, GemmPlan) and not plan.config:
            plans.extend(plan.with_config(cfg) for cfg in kernels.GEMM_CONFIGS)
        elif isinstance(plan, ConvPlan) and not plan.config:
            plans.extend(plan.with_config(cfg) for cfg in kernels.CONV_CONFIGS)
        elif isinstance(plan, AttentionPlan) and not plan.config:
            plans.extend(plan.with_config(cfg) for cfg in kernels.ATTENTION_CONFIGS)
        elif isinstance(plan, SoftmaxPlan) and not plan.config:
            plans.extend(plan.with_config(cfg) for cfg in kernels.SOFTMAX_CONFIGS)
        elif isinstance(plan, MaxPoolPlan) and not plan.config:
            plans.extend(plan.with_config(cfg) for cfg in kernels.POOL_CONFIGS)
        elif plan is not None:
            plans.append(plan)
    plans = [p for p in plans if _admits(p, ctx.values)]
    # a generic tile program that runs real loops is the fallback for programs no hand-written
    # kernel fits; beside one it is no candidate (timing it would only slow the tuning down)
    if any(p.family != "generic" for p in plans):
        plans = [p for p in plans if getattr(p, "nest", None) is None]
    return plans


def _admits(plan, values):
    try:
        plan.check(values)
    except (TypeError, ValueError):
        return False
    return True


def updates_an_input(program):
    """Whether the program stores to a tensor it also reads (re-running it changes the result)."""
    read = set()
    for value in program.stores.values():
        for v in _walk(value):
            if v.op in ("load", "offsets"):
                t = v.args[0]
                while t.op == "index":
                    t = t.args[0]
                read.add(t.args[0])
    return bool(read & set(program.stores))


class TunedPlan(Plan):
    """Several fitting plans; each bound call picks the fastest with ``AutoTuner``."""

    family = "tuned"

    def __init__(self, plans, namespace):
        self.plans = plans
        self.namespace = namespace
        self.chosen = {}

    def bind(self, values, index):
        import json

        from ninetoothed_amd.auto_tuner import AutoTuner, signature

        bound, keys = [], []
        for plan in self.plans:
            try:
                launch = plan.bind(values, index)
            except (LoweringError, TypeError, ValueError):
                continue
            bound.append(launch)
            keys.append(json.dumps(plan.describe(), sort_keys=True, default=str))
        if not bound:
            raise LoweringError("no candidate kernel accepts these arguments")
        if len(bound) == 1:
            return bound[0]
        names = sorted(index, key=index.get)
        args = tuple(values[n] for n in names)
        funcs = [lambda *a, _launch=launch: _launch(a) for launch in bound]
        tuner = AutoTuner(funcs, keys, cache_namespace=self.namespace)
        best = tuner.choose(*args)
        self.chosen[signature(args, {})] = keys[best]
        return bound[best]

    def describe(self):
        return {"family": "tuned", "candidates": [p.describe() for p in self.plans],
                "chosen": sorted(set(self.chosen.values()))}


def select(ctx):
    """Return the Plan of the first family whose pattern and geometry fit.

    A family whose pattern matches but whose geometry does not raises ``LoweringError``,
    and a plan whose kernel would reject the call's dtypes or sizes (``Plan.check``) is
    declined too; the next families are still tried (an elementwise program the add kernel
    cannot take runs on the generic kernels) and the reasons are reported if none fits."""
    tried, reasons = [], []
    for matcher in _families_for(ctx):
        name = matcher.__name__[len("match_"):]
        try:
            plan = matcher(ctx)
            if plan is not None:
                plan.check(ctx.values)  # a call the family's kernel would reject goes on
        except (LoweringError, TypeError, ValueError) as exc:
            reasons.append(f"{name}: {exc}")
            plan = None
        if plan is not None:
            return plan
        tried.append(name)
    detail = "; ".join(reasons)
    raise LoweringError(
        "the application matches none of the MI355X kernel families "
        f"({', '.join(tried)}); see ninetoothed_amd.families for the supported programs"
        + (f" ({detail})" if detail else "")
    )
