"""Oracle: the hot-path applications executed tile by tile on the CPU (TEST ONLY).

Each function runs an arrangement through the oracle's materialised index tables
(``oracle.arrange``), then executes the application body program by program with
numpy, following the reference application it cites and the dtype rules of the
reference's generated kernels:
  - ``ntl.dot`` of fp16/bf16 blocks accumulates in fp32
    (reference src/ninetoothed/frontend/types.py:283-295);
  - a Python float literal times a 16-bit tensor computes in the tensor's type
    (weak scalar typing, so ``q * 1.44269504089`` rounds the constant and the product);
    a 0-d scalar *parameter* (alpha, beta) is fp32 and promotes the product to fp32;
  - ``/`` of 16-bit operands computes in fp32 (types.py:319-324);
  - masked loads read ``other`` (default 0) and masked stores are skipped.
Reduction order inside ``tl.sum``/``tl.max`` of the generated kernel is unspecified
upstream; the oracle sums in fp32 (pairwise, numpy).

Pinned by closed forms on small inputs in tests/test_oracle_apply.py (torch float64
matmul/addmm/conv2d/attention/softmax/max_pool2d/add) and by invariants.
"""

import numpy as np

from oracle.arrange import OTensor, Scalar

_NP16 = {"float16": np.float16, "float32": np.float32, "float64": np.float64}


def _bf16_round(x):
    """Round float32 values to bfloat16 (nearest even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    out = (u & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def round_to(x, dtype):
    """Round float32 array ``x`` to ``dtype`` ('float16', 'bfloat16', 'float32') -> float32."""
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return _bf16_round(x)
    return np.asarray(x, dtype=np.float32)


def _gather(values, table, valid, other=0.0):
    """Gather ``values`` (a numpy array with the source shape) at ``table`` where valid."""
    idx = tuple(np.clip(table[..., d], 0, values.shape[d] - 1) for d in range(values.ndim))
    out = values[idx].astype(np.float32)
    return np.where(valid, out, np.float32(other))


def _scatter(dest, table, valid, vals):
    idx = tuple(table[..., d][valid] for d in range(dest.ndim))
    dest[idx] = vals[valid]


def _split_grid(t, n_grid_dims):
    """Flatten the program grid (first level) of a materialised table."""
    shape = t.table.shape
    g = int(np.prod(shape[:n_grid_dims])) if n_grid_dims else 1
    return t.table.reshape((g,) + shape[n_grid_dims:]), t.valid.reshape((g,) + t.valid.shape[n_grid_dims:])


# ----------------------------------------------------------------------------- GEMM family
def gemm_program(lhs_t, rhs_t, out_t, lhs, rhs, round_dtype="float16", epilogue=None, programs=None):
    """matmul application (reference tests/test_matmul.py:41-47; README.md:56-62 without
    the cast) over arranged tables; ``epilogue(out_tile_fp32, program_index)`` may
    rewrite the rounded accumulator tile (addmm).  Returns the output values and the
    output tables for the scatter."""
    ng = len(out_t.levels[0])
    ta, va = _split_grid(lhs_t, ng)  # (G, nk, BM, BK, 2)
    tb, vb = _split_grid(rhs_t, ng)  # (G, nk, BK, BN, 2)
    to, vo = _split_grid(out_t, ng)  # (G, BM, BN, 2)
    G = to.shape[0]
    sel = range(G) if programs is None else programs
    results = []
    for g in sel:
        a = _gather(lhs, ta[g], va[g])  # (nk, BM, BK)
        b = _gather(rhs, tb[g], vb[g])  # (nk, BK, BN)
        acc = np.zeros(to.shape[1:3], dtype=np.float32)
        for k in range(a.shape[0]):
            acc += a[k] @ b[k]  # fp32 accumulation of the block product
        tile = round_to(acc, round_dtype) if round_dtype else acc
        if epilogue is not None:
            tile = epilogue(tile, g)
        results.append((g, tile))
    return results, to, vo


def matmul(lhs, rhs, out_dtype, arrangement, block=(16, 16, 16), round_dtype="float16", programs=None):
    """C = A @ B through ``arrangement`` (the matmul arrangement or one built on it)."""
    M, K = lhs.shape
    N = rhs.shape[1]
    bm, bn, bk = block
    lt, rt, ot = arrangement(OTensor((M, K)), OTensor((K, N)), OTensor((M, N)), bm, bn, bk)
    out = np.zeros((M, N), dtype=np.float32)
    results, to, vo = gemm_program(lt, rt, ot, lhs, rhs, round_dtype, programs=programs)
    for g, tile in results:
        _scatter(out, to[g], vo[g], tile)
    return round_to(out, out_dtype)


def addmm(input, mat1, mat2, beta, alpha, out_dtype, arrangement, block=(16, 16, 16), programs=None):
    """addmm application (reference tests/test_addmm.py:35-38): beta*input + alpha*fp16(acc),
    in fp32 because beta and alpha are fp32 scalar parameters."""
    M, K = mat1.shape
    N = mat2.shape[1]
    bm, bn, bk = block
    it, at, bt, _, _, ot = arrangement(OTensor((M, N)), OTensor((M, K)), OTensor((K, N)), Scalar(), Scalar(),
                                       OTensor((M, N)), bm, bn, bk)
    ti, vi = _split_grid(it, len(ot.levels[0]))
    beta32, alpha32 = np.float32(beta), np.float32(alpha)

    def epilogue(tile, g):
        c = _gather(input, ti[g], vi[g])
        return beta32 * c + alpha32 * tile

    out = np.zeros((M, N), dtype=np.float32)
    results, to, vo = gemm_program(at, bt, ot, mat1, mat2, "float16", epilogue=epilogue, programs=programs)
    for g, tile in results:
        _scatter(out, to[g], vo[g], tile)
    return round_to(out, out_dtype)


def conv2d(x, w, padding, arrangement, out_dtype="float16", block=(16, 16, 16), programs=None):
    """conv2d program (reference tests/test_conv2d.py:14-49 with the matmul application):
    the arranged implicit GEMM, padding read as 0."""
    N, C, H, W = x.shape
    K, _, R, S = w.shape
    ph, pw = padding
    P, Q = H + 2 * ph - R + 1, W + 2 * pw - S + 1
    env = {"padding_h": ph, "padding_w": pw}
    bm, bn, bk = block
    xt, wt, yt = arrangement(OTensor((N, C, H, W), env), OTensor((K, C, R, S), env), OTensor((N, K, P, Q), env),
                             BLOCK_SIZE_M=bm, BLOCK_SIZE_N=bn, BLOCK_SIZE_K=bk)
    out = np.zeros((N, K, P, Q), dtype=np.float32)
    results, to, vo = gemm_program(xt, wt, yt, x, w, "float16", programs=programs)
    for g, tile in results:
        _scatter(out, to[g], vo[g], tile)
    return round_to(out, out_dtype)


# ----------------------------------------------------------------------------- attention
def attention(q, k, v, is_causal, arrangement, scale_const=1.44269504089, in_dtype="float16", block=(16, 16),
              programs=None):
    """attention application (reference tests/test_attention.py:45-70), online softmax in base 2."""
    B, H, S, D = q.shape
    Sk = k.shape[2]
    bm, bn = block
    qt, kt, vt, _, ot = arrangement(OTensor((B, H, S, D)), OTensor((B, H, Sk, D)), OTensor((B, H, Sk, D)), Scalar(),
                                    OTensor((B, H, S, D)), bm, bn)
    ng = len(ot.levels[0])
    tq, vq = _split_grid(qt, ng)  # (G, BM, D, 4)
    tk, vk = _split_grid(kt, ng)  # (G, nk, BN, D, 4)
    tv, vv = _split_grid(vt, ng)
    to, vo = _split_grid(ot, ng)
    out = np.zeros(q.shape, dtype=np.float32)
    c = np.float32(round_to(np.float32(scale_const), in_dtype)) if in_dtype != "float32" else np.float32(scale_const)
    sel = range(to.shape[0]) if programs is None else programs
    for g in sel:
        qb = _gather(q, tq[g], vq[g])
        q_loaded = round_to(round_to(qb * c, in_dtype), in_dtype)  # weak-typed literal product, then .to(q.dtype)
        q_pos = tq[g][:, 0, 2]
        acc = np.zeros((qb.shape[0], D), dtype=np.float32)
        l_i = np.ones(qb.shape[0], dtype=np.float32)
        m_i = np.full(qb.shape[0], -np.inf, dtype=np.float32)
        for i in range(tk.shape[1]):
            kb = _gather(k, tk[g][i], vk[g][i])
            vb = _gather(v, tv[g][i], vv[g][i])
            k_pos = tk[g][i][:, 0, 2]
            qk = q_loaded @ kb.T
            # `k[i].offsets(-2) < k.source.shape[-2]`: the oracle's tables clip invalid
            # positions, so the bound is read from the key rows' validity instead.
            k_in = vk[g][i][:, 0]
            qk = np.where(k_in[None, :], qk, -np.inf)
            if is_causal:
                qk = np.where(q_pos[:, None] >= k_pos[None, :], qk, -np.inf)
            m_ij = np.maximum(m_i, qk.max(axis=1))
            with np.errstate(invalid="ignore"):
                p = np.exp2(qk - m_ij[:, None]).astype(np.float32)
                alpha = np.exp2(m_i - m_ij).astype(np.float32)
            l_ij = p.sum(axis=1, dtype=np.float32)
            acc = acc * alpha[:, None] + round_to(p, in_dtype) @ vb
            m_i = m_ij
            l_i = l_i * alpha + l_ij
        acc = acc / l_i[:, None]
        _scatter(out, to[g], vo[g], acc)
    return round_to(out, in_dtype)


# ----------------------------------------------------------------------------- softmax
def softmax(x, block_size, in_dtype="float32", out_dtype=None):
    """softmax_kernel (reference tests/test_softmax.py:13-21) over (1, BLOCK_SIZE) tiles with
    other=-inf: x - max, exp, sum, divide (the divide in fp32), stored in ``out_dtype``
    (default ``in_dtype``; the reference's store casts the fp32 quotient to the output's type)."""
    R, C = x.shape
    xt = OTensor((R, C), other=float("-inf")).tile((1, block_size))
    t, valid = _split_grid(xt, 2)  # (G, 1, BS, 2)
    vals = _gather(x, t, valid, other=-np.inf)
    xr = round_to(vals, in_dtype)
    mx = xr.max(axis=(1, 2), keepdims=True)
    with np.errstate(invalid="ignore"):
        num = round_to(np.exp(round_to(xr - mx, in_dtype)), in_dtype)
    den = round_to(num.sum(axis=(1, 2), keepdims=True, dtype=np.float32), in_dtype)
    y = num / den
    out = np.zeros((R, C), dtype=np.float32)
    _scatter(out, t, valid, y)
    return round_to(out, in_dtype if out_dtype is None else out_dtype)


# ----------------------------------------------------------------------------- max_pool2d
def max_pool2d(x, window, ceil_mode, arrangement, block=64):
    """max_pool2d application (reference tests/test_max_pool2d.py:33-36): max over window
    elements, other=-inf."""
    N, C, H, W = x.shape
    r, s = window
    div = (lambda a, b: -(-a // b)) if ceil_mode else (lambda a, b: a // b)
    P, Q = div(H - r, r) + 1, div(W - s, s) + 1
    env = {"WINDOW_HEIGHT": r, "WINDOW_WIDTH": s, "BLOCK_SIZE": block}
    xt, yt = arrangement(OTensor((N, C, H, W), env, other=float("-inf")), OTensor((N, C, P, Q), env))
    tx, vx = _split_grid(xt, len(xt.levels[0]))
    ty, vy = _split_grid(yt, len(yt.levels[0]))
    vals = _gather(x, tx, vx, other=-np.inf)  # (G, BS, WIN)
    out = np.zeros((N, C, P, Q), dtype=np.float32)
    _scatter(out, ty, vy, vals.max(axis=-1))
    return out


# ----------------------------------------------------------------------------- add
def add(lhs, rhs, block, in_dtype="float32"):
    """add_kernel (reference tests/test_add.py:12-20): output = lhs + rhs per BLOCK_SIZE tile."""
    n = lhs.shape[0]
    t = OTensor((n,)).tile((block,))
    tb, vb = _split_grid(t, 1)
    a = _gather(lhs, tb, vb)
    b = _gather(rhs, tb, vb)
    out = np.zeros(n, dtype=np.float32)
    _scatter(out, tb, vb, round_to(a + b, in_dtype))
    return out
