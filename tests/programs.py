"""The hot path's user programs, written against ``ninetoothed_amd``'s drop-in API.

These are the arrangements and applications a NineToothed user writes for the six
kernel families; they restate the programs of the reference's tests (file:line on
each) in the same DSL, because a drop-in backend must accept exactly these programs.
The same arrangement functions also run on the oracle's materialised tensors
(``oracle.arrange.OTensor``), which is how the product's index maps are checked.
"""

import functools

import ninetoothed_amd as ninetoothed
import ninetoothed_amd.language as ntl
from ninetoothed_amd import Symbol, Tensor

BLOCK_SIZE_M = Symbol("BLOCK_SIZE_M", meta=True)
BLOCK_SIZE_N = Symbol("BLOCK_SIZE_N", meta=True)
BLOCK_SIZE_K = Symbol("BLOCK_SIZE_K", meta=True)


# --------------------------------------------------------------- matmul (reference tests/test_matmul.py:14-47)
def matmul_arrangement(lhs, rhs, output, BLOCK_SIZE_M=BLOCK_SIZE_M, BLOCK_SIZE_N=BLOCK_SIZE_N, BLOCK_SIZE_K=BLOCK_SIZE_K):
    output_tiled = output.tile((BLOCK_SIZE_M, BLOCK_SIZE_N))

    lhs_tiled = lhs.tile((BLOCK_SIZE_M, BLOCK_SIZE_K)).tile((1, -1)).expand((-1, output_tiled.shape[1]))
    lhs_tiled.dtype = lhs_tiled.dtype.squeeze(0)

    rhs_tiled = rhs.tile((BLOCK_SIZE_K, BLOCK_SIZE_N)).tile((-1, 1)).expand((output_tiled.shape[0], -1))
    rhs_tiled.dtype = rhs_tiled.dtype.squeeze(1)

    return lhs_tiled, rhs_tiled, output_tiled


def matmul_application(lhs, rhs, output):
    accumulator = ntl.zeros(output.shape, dtype=ntl.float32)
    for k in range(lhs.shape[0]):
        accumulator += ntl.dot(lhs[k], rhs[k])
    output = accumulator.to(ntl.float16)  # noqa: F841


def matmul_application_fp32(lhs, rhs, output):
    # README variant (reference README.md:56-62): the accumulator is stored as is.
    accumulator = ntl.zeros(output.shape, dtype=ntl.float32)
    for k in range(lhs.shape[0]):
        accumulator += ntl.dot(lhs[k], rhs[k])
    output = accumulator  # noqa: F841


def matmul_tensors():
    return (Tensor(2), Tensor(2), Tensor(2))


# ---------------------------------------------------------------- addmm (reference tests/test_addmm.py:13-38)
def addmm_arrangement(input, mat1, mat2, beta, alpha, output, BLOCK_SIZE_M=BLOCK_SIZE_M, BLOCK_SIZE_N=BLOCK_SIZE_N,
                      BLOCK_SIZE_K=BLOCK_SIZE_K):
    _, _, input_arranged = matmul_arrangement(mat1, mat2, input, BLOCK_SIZE_M, BLOCK_SIZE_N, BLOCK_SIZE_K)
    mat1_arranged, mat2_arranged, output_arranged = matmul_arrangement(mat1, mat2, output, BLOCK_SIZE_M, BLOCK_SIZE_N,
                                                                       BLOCK_SIZE_K)
    return input_arranged, mat1_arranged, mat2_arranged, beta, alpha, output_arranged


def addmm_application(input, mat1, mat2, beta, alpha, output):
    matmul_output = ntl.zeros(output.shape, dtype=ntl.float32)
    matmul_application(mat1, mat2, matmul_output)
    output = beta * input + alpha * matmul_output  # noqa: F841


def addmm_tensors():
    return (Tensor(2), Tensor(2), Tensor(2), Tensor(0), Tensor(0), Tensor(2))


# --------------------------------------------------------------- conv2d (reference tests/test_conv2d.py:14-49)
def conv2d_arrangement(input, filter, output, enable_padding=False, BLOCK_SIZE_M=BLOCK_SIZE_M,
                       BLOCK_SIZE_N=BLOCK_SIZE_N, BLOCK_SIZE_K=BLOCK_SIZE_K):
    if enable_padding:
        padding_h = Symbol("padding_h", constexpr=True)
        padding_w = Symbol("padding_w", constexpr=True)
        input_padded = input.pad(((0, 0), (0, 0), (padding_h, padding_h), (padding_w, padding_w)))
    else:
        input_padded = input

    input_tiled = input_padded.tile((1, *filter.shape[1:]), strides=(-1, -1, 1, 1))
    input_squeezed = input_tiled.squeeze(1)
    input_squeezed.dtype = input_squeezed.dtype.squeeze(0)
    input_raveled = input_squeezed.ravel()
    input_flattened = input_raveled.flatten(end_dim=3).flatten(start_dim=1)

    filter_flattened = filter.flatten(start_dim=1)
    filter_permuted = filter_flattened.permute((1, 0))

    output_flattened = output.permute((0, 2, 3, 1)).flatten(end_dim=3)

    return functools.partial(matmul_arrangement, BLOCK_SIZE_M=BLOCK_SIZE_M, BLOCK_SIZE_N=BLOCK_SIZE_N,
                             BLOCK_SIZE_K=BLOCK_SIZE_K)(input_flattened, filter_permuted, output_flattened)


def conv2d_tensors():
    return (Tensor(4), Tensor(4, shape_options={"constexpr": True}), Tensor(4))


def make_conv2d(**make_options):
    return ninetoothed.make(functools.partial(conv2d_arrangement, enable_padding=True), matmul_application,
                            conv2d_tensors(), **make_options)


# ------------------------------------------------------------ attention (reference tests/test_attention.py:10-70)
ATT_BLOCK_SIZE_M = ninetoothed.block_size(lower_bound=64, upper_bound=128)
ATT_BLOCK_SIZE_N = ninetoothed.block_size(lower_bound=32, upper_bound=64)


def attention_arrangement(q, k, v, is_causal, o, BLOCK_SIZE_M=ATT_BLOCK_SIZE_M, BLOCK_SIZE_N=ATT_BLOCK_SIZE_N):
    def arrange_q_or_o(input):
        arranged = input.tile((1, 1, BLOCK_SIZE_M, -1))
        arranged.dtype = arranged.dtype.squeeze((0, 1))
        return arranged

    def arrange_k_or_v(input):
        arranged = input.tile((1, 1, BLOCK_SIZE_N, -1)).tile((1, 1, -1, -1)).expand((-1, -1, q_arranged.shape[-2], -1))
        arranged.dtype = arranged.dtype.squeeze((0, 1, 3))
        arranged.dtype.dtype = arranged.dtype.dtype.squeeze((0, 1))
        return arranged

    q_arranged = arrange_q_or_o(q)
    return q_arranged, arrange_k_or_v(k), arrange_k_or_v(v), is_causal, arrange_q_or_o(o)


def attention_application(q, k, v, is_causal, o):
    q_loaded = (q * 1.44269504089).to(q.dtype)

    acc = ntl.zeros((q.shape[-2], q.shape[-1]), dtype=ntl.float32)
    l_i = ntl.full((q.shape[-2],), 1, dtype=ntl.float32)
    m_i = ntl.full((q.shape[-2],), float("-inf"), dtype=ntl.float32)

    for i in range(k.shape[0]):
        qk = ntl.dot(q_loaded, ntl.trans(k[i]))
        qk = ntl.where(k[i].offsets(-2) < k.source.shape[-2], qk, float("-inf"))

        if is_causal:
            mask = q.offsets(-2)[:, None] >= k[i].offsets(-2)[None, :]
            qk = ntl.where(mask, qk, float("-inf"))

        m_ij = ntl.maximum(m_i, ntl.max(qk, 1))
        p = ntl.exp2(qk - m_ij[:, None])
        l_ij = ntl.sum(p, 1)

        alpha = ntl.exp2(m_i - m_ij)
        acc = acc * alpha[:, None] + ntl.dot(p.to(v[i].dtype), v[i])
        m_i = m_ij
        l_i = l_i * alpha + l_ij

    acc /= l_i[:, None]
    o = acc  # noqa: F841


def attention_application_scaled(q, k, v, is_causal, o):
    # The 1/sqrt(128) configuration: the pre-scale constant is log2(e) / sqrt(128).
    q_loaded = (q * 0.12752981786465204).to(q.dtype)

    acc = ntl.zeros((q.shape[-2], q.shape[-1]), dtype=ntl.float32)
    l_i = ntl.full((q.shape[-2],), 1, dtype=ntl.float32)
    m_i = ntl.full((q.shape[-2],), float("-inf"), dtype=ntl.float32)

    for i in range(k.shape[0]):
        qk = ntl.dot(q_loaded, ntl.trans(k[i]))
        qk = ntl.where(k[i].offsets(-2) < k.source.shape[-2], qk, float("-inf"))

        if is_causal:
            mask = q.offsets(-2)[:, None] >= k[i].offsets(-2)[None, :]
            qk = ntl.where(mask, qk, float("-inf"))

        m_ij = ntl.maximum(m_i, ntl.max(qk, 1))
        p = ntl.exp2(qk - m_ij[:, None])
        l_ij = ntl.sum(p, 1)

        alpha = ntl.exp2(m_i - m_ij)
        acc = acc * alpha[:, None] + ntl.dot(p.to(v[i].dtype), v[i])
        m_i = m_ij
        l_i = l_i * alpha + l_ij

    acc /= l_i[:, None]
    o = acc  # noqa: F841


def attention_tensors():
    qkvo = tuple(
        Tensor(4, shape_options=(None, None, {"constexpr": True}, {"constexpr": True, "upper_bound": 128}))
        for _ in range(4)
    )
    q, k, v, o = qkvo
    return (q, k, v, Tensor(0, constexpr=True), o)


# -------------------------------------------------------------- softmax (reference tests/test_softmax.py:10-27)
def make_softmax(**jit_options):
    BLOCK_SIZE = Symbol("BLOCK_SIZE", constexpr=True)

    @ninetoothed.jit(**jit_options)
    def softmax_kernel(
        input_row: Tensor(2, other=float("-inf")).tile((1, BLOCK_SIZE)),
        output_row: Tensor(2).tile((1, BLOCK_SIZE)),
    ):
        row_minus_max = input_row - ntl.max(input_row)
        numerator = ntl.exp(row_minus_max)
        denominator = ntl.sum(numerator)
        output_row = numerator / denominator  # noqa: F841

    return softmax_kernel


# ----------------------------------------------------------- max_pool2d (reference tests/test_max_pool2d.py:13-64)
def max_pool2d_arrangement(input, output, ceil_mode=False):
    BLOCK_SIZE = Symbol("BLOCK_SIZE", meta=True)
    WINDOW_HEIGHT = Symbol("WINDOW_HEIGHT", constexpr=True, upper_bound=16)
    WINDOW_WIDTH = Symbol("WINDOW_WIDTH", constexpr=True, upper_bound=16)

    input_arranged = input.tile((1, 1, WINDOW_HEIGHT, WINDOW_WIDTH), floor_mode=not ceil_mode)
    input_arranged = input_arranged.ravel()
    input_arranged = input_arranged.flatten(end_dim=4).flatten(start_dim=1)
    input_arranged = input_arranged.tile((BLOCK_SIZE, -1))

    output_arranged = output.tile((1, 1, 1, 1))
    output_arranged = output_arranged.ravel()
    output_arranged = output_arranged.flatten(end_dim=4).flatten(start_dim=1)
    output_arranged = output_arranged.tile((BLOCK_SIZE, -1))
    output_arranged.dtype = output_arranged.dtype.squeeze(1)

    return input_arranged, output_arranged


def max_pool2d_application(input, output):
    output = ntl.max(input, axis=1)  # noqa: F841


def max_pool2d_tensors():
    return (Tensor(4, other=float("-inf")), Tensor(4))


# ------------------------------------------------------------------- add (reference tests/test_add.py:9-24)
def make_add():
    BLOCK_SIZE = Symbol("BLOCK_SIZE", meta=True)

    @ninetoothed.jit
    def add_kernel(
        lhs: Tensor(1).tile((BLOCK_SIZE,)),
        rhs: Tensor(1).tile((BLOCK_SIZE,)),
        output: Tensor(1).tile((BLOCK_SIZE,)),
    ):
        output = lhs + rhs  # noqa: F841

    return add_kernel


# ------------------------------------------------------------------- dropout (reference tests/test_dropout.py:10-24)
def make_dropout():
    def arrangement(input, p, seed, output, BLOCK_SIZE=ninetoothed.block_size()):
        return input.tile((BLOCK_SIZE,)), p, seed, output.tile((BLOCK_SIZE,))

    def application(input, p, seed, output):
        output = ntl.where(ntl.rand(seed, input.offsets()) > p, input / (1 - p), 0)  # noqa: F841

    return ninetoothed.make(arrangement, application, (Tensor(1), Tensor(0), Tensor(0), Tensor(1)))
