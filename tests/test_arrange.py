"""Arrangement index semantics: product DSL and oracle against the reference's golden
maps, against each other on every hot-path arrangement, and against closed forms."""

import functools
import json
from pathlib import Path

import numpy as np
import pytest

import ninetoothed_amd as ninetoothed
import programs as pg
from ninetoothed_amd import Tensor
from oracle.arrange import OTensor, Scalar

GOLDEN = json.loads((Path(__file__).parent / "golden" / "index_maps.json").read_text())


# ------------------------------------------------------------------ golden: eval
@pytest.mark.parametrize("shape_options", (None, {"constexpr": True}))
@pytest.mark.parametrize("subs_before_eval", (False, True))
@pytest.mark.parametrize("use_tensor_in_subs", (False, True))
def test_eval_golden(use_tensor_in_subs, subs_before_eval, shape_options):
    g = GOLDEN["eval_5x6"]
    assert (Tensor(shape=(2, 3)).eval() == np.array(g["plain_2x3"])).all()
    x = Tensor(2, shape_options=shape_options)
    bm, bn = ninetoothed.block_size(), ninetoothed.block_size()
    subs = {x: {"shape": (5, 6)}, bm: 2, bn: 3}
    if use_tensor_in_subs:
        subs[x] = Tensor(shape=(5, 6))

    def ev(t):
        return t.subs(subs).eval() if subs_before_eval else t.eval(subs)

    assert (ev(x) == np.array(g["plain"])).all()
    assert (ev(x.permute((1, 0))) == np.array(g["permuted"])).all()
    tiled = x.tile((bm, bn))
    assert (ev(tiled) == np.array(g["tiled"])).all()
    tt = tiled.tile((bm, bn))
    assert (ev(tt) == np.array(g["tiled_tiled"])).all()
    tt.dtype = tt.dtype.flatten()
    assert (ev(tt) == np.array(g["tiled_tiled_mid_flattened"])).all()
    tt.dtype.dtype = tt.dtype.dtype.flatten()
    assert (ev(tt) == np.array(g["tiled_tiled_both_flattened"])).all()


def test_eval_golden_oracle():
    g = GOLDEN["eval_5x6"]
    x = OTensor((5, 6))
    assert (x.eval() == np.array(g["plain"])).all()
    assert (x.permute((1, 0)).eval() == np.array(g["permuted"])).all()
    tiled = x.tile((2, 3))
    assert (tiled.eval() == np.array(g["tiled"])).all()
    tt = tiled.tile((2, 3))
    assert (tt.eval() == np.array(g["tiled_tiled"])).all()
    tt.dtype = tt.dtype.flatten()
    assert (tt.eval() == np.array(g["tiled_tiled_mid_flattened"])).all()
    tt.dtype.dtype = tt.dtype.dtype.flatten()
    assert (tt.eval() == np.array(g["tiled_tiled_both_flattened"])).all()


# ------------------------------------------------------------- golden: addmm maps
def _addmm_golden():
    g = GOLDEN["addmm_debugging"]
    return g, [np.array(t) for t in g["target_tensors"]]


def test_addmm_arrangement_golden_product():
    g, targets = _addmm_golden()
    m, n, k, b = g["m"], g["n"], g["k"], g["block_size"]
    arrangement = functools.partial(pg.addmm_arrangement, BLOCK_SIZE_M=b, BLOCK_SIZE_N=b, BLOCK_SIZE_K=b)
    tensors = (Tensor(shape=(m, n)), Tensor(shape=(m, k)), Tensor(shape=(k, n)), Tensor(0), Tensor(0),
               Tensor(shape=(m, n)))
    for arranged, expected in zip(arrangement(*tensors), targets):
        got = arranged.flatten().eval() if arranged.ndim != 0 else arranged.eval()
        assert np.array_equal(got, expected)


def test_addmm_arrangement_golden_oracle():
    g, targets = _addmm_golden()
    m, n, k, b = g["m"], g["n"], g["k"], g["block_size"]
    arranged = pg.addmm_arrangement(OTensor((m, n)), OTensor((m, k)), OTensor((k, n)), Scalar(), Scalar(),
                                    OTensor((m, n)), b, b, b)
    for t, expected in zip(arranged, targets):
        if isinstance(t, Scalar):
            assert expected.ndim == 0
            continue
        assert np.array_equal(t.flatten().eval(), expected)


def test_simulate_arrangement_sources_are_aranges():
    # The reference's simulate_arrangement source tensors are aranges of each shape.
    g, _ = _addmm_golden()
    shapes = [(g["m"], g["n"]), (g["m"], g["k"]), (g["k"], g["n"]), (), (), (g["m"], g["n"])]
    for shape, src in zip(shapes, g["source_tensors"]):
        assert np.array_equal(np.array(src), np.arange(int(np.prod(shape))).reshape(shape) if shape else np.array(0))


# ------------------------------------------- product == oracle on hot-path arrangements
def _product_eval(arranged):
    return [t.eval() if t.ndim or t.source.ndim else t.eval() for t in arranged]


def _same(product_tensors, oracle_tensors):
    for p, o in zip(product_tensors, oracle_tensors):
        if isinstance(o, Scalar):
            continue
        assert np.array_equal(p.eval(), o.eval())


@pytest.mark.parametrize("mnk,blocks", (((33, 20, 17), (16, 8, 4)), ((8, 8, 8), (4, 4, 8))))
def test_matmul_arrangement_matches_oracle(mnk, blocks):
    m, n, k = mnk
    prod_ = pg.matmul_arrangement(Tensor(shape=(m, k)), Tensor(shape=(k, n)), Tensor(shape=(m, n)), *blocks)
    orac = pg.matmul_arrangement(OTensor((m, k)), OTensor((k, n)), OTensor((m, n)), *blocks)
    _same(prod_, orac)


@pytest.mark.parametrize("padding", ((0, 0), (1, 1), (0, 1), (2, 0)))
def test_conv2d_arrangement_matches_oracle(padding):
    n, c, h, w, k, r, s = 2, 3, 6, 5, 4, 3, 2
    ph, pw = padding
    p, q = h + 2 * ph - r + 1, w + 2 * pw - s + 1
    env = {"padding_h": ph, "padding_w": pw}
    blocks = dict(BLOCK_SIZE_M=8, BLOCK_SIZE_N=4, BLOCK_SIZE_K=4)
    prod_ = pg.conv2d_arrangement(Tensor(shape=(n, c, h, w)), Tensor(shape=(k, c, r, s)), Tensor(shape=(n, k, p, q)),
                                  enable_padding=True, **blocks)
    orac = pg.conv2d_arrangement(OTensor((n, c, h, w), env), OTensor((k, c, r, s), env), OTensor((n, k, p, q), env),
                                 enable_padding=True, **blocks)
    for pt, ot in zip(prod_, orac):
        assert np.array_equal(pt.eval(env), ot.eval())


@pytest.mark.parametrize("seq", (10, 1))
def test_attention_arrangement_matches_oracle(seq):
    shape = (2, 3, seq, 4)
    prod_ = pg.attention_arrangement(*(Tensor(shape=shape) for _ in range(3)), Tensor(0, constexpr=True),
                                     Tensor(shape=shape), 4, 2)
    orac = pg.attention_arrangement(*(OTensor(shape) for _ in range(3)), Scalar(), OTensor(shape), 4, 2)
    _same(prod_, orac)


@pytest.mark.parametrize("ceil_mode", (False, True))
def test_max_pool2d_arrangement_matches_oracle(ceil_mode):
    x_shape = (2, 2, 7, 8)
    r = s = 3
    div = (lambda a, b: -(-a // b)) if ceil_mode else (lambda a, b: a // b)
    y_shape = (2, 2, div(7 - r, r) + 1, div(8 - s, s) + 1)
    env = {"WINDOW_HEIGHT": r, "WINDOW_WIDTH": s, "BLOCK_SIZE": 4}
    prod_ = pg.max_pool2d_arrangement(Tensor(shape=x_shape, other=float("-inf")), Tensor(shape=y_shape), ceil_mode)
    orac = pg.max_pool2d_arrangement(OTensor(x_shape, env), OTensor(y_shape, env), ceil_mode)
    for pt, ot in zip(prod_, orac):
        assert np.array_equal(pt.eval(env), ot.eval())


def test_softmax_and_add_tiles_match_oracle():
    bs = ninetoothed.Symbol("BLOCK_SIZE", constexpr=True)
    x = Tensor(shape=(5, 11)).tile((1, bs))
    assert np.array_equal(x.eval({bs: 4}), OTensor((5, 11)).tile((1, 4)).eval())
    y = Tensor(shape=(23,)).tile((8,))
    assert np.array_equal(y.eval(), OTensor((23,)).tile((8,)).eval())


# ---------------------------------------------------------------- closed forms
def test_tile_strides_dilation_floor_closed_form():
    # 1-D length 10, tiles of 3 with stride 2 and dilation 2: tile o, element i -> 2*o + 2*i.
    for make in (lambda: Tensor(shape=(10,)), lambda: OTensor((10,))):
        t = make().tile((3,), strides=(2,), dilation=(2,), floor_mode=True)
        got = t.eval()
        # floor((10 - 2*(3-1) - 1) / 2) + 1 = 3 tiles
        expected = np.array([[2 * o + 2 * i for i in range(3)] for o in range(3)])
        assert np.array_equal(got, expected)
        t2 = make().tile((3,), strides=(2,), dilation=(2,))  # ceil mode: 4 tiles, the last partly masked
        exp2 = np.array([[2 * o + 2 * i if 2 * o + 2 * i < 10 else -1 for i in range(3)] for o in range(4)])
        assert np.array_equal(t2.eval(), exp2)


def test_pad_expand_squeeze_closed_form():
    for make in (lambda: Tensor(shape=(2, 3)), lambda: OTensor((2, 3))):
        padded = make().pad(((1, 0), (0, 2)))
        expected = -np.ones((3, 5), dtype=int)
        expected[1:, :3] = np.arange(6).reshape(2, 3)
        assert np.array_equal(padded.eval(), expected)
    t = Tensor(shape=(1, 4)).expand((3, -1))
    assert np.array_equal(t.eval(), np.tile(np.arange(4), (3, 1)))
    assert np.array_equal(OTensor((1, 4)).expand((3, -1)).eval(), np.tile(np.arange(4), (3, 1)))
    sq = Tensor(shape=(1, 4)).squeeze(0)
    assert np.array_equal(sq.eval(), np.arange(4))


def test_getitem_and_ravel():
    t = Tensor(shape=(4, 6))
    assert np.array_equal(t[1].eval(), np.arange(6, 12))
    assert np.array_equal(t[:, 1:4].eval(), np.arange(24).reshape(4, 6)[:, 1:4])
    assert np.array_equal(t[None].eval(), np.arange(24).reshape(1, 4, 6))
    r = t.tile((2, 3)).ravel()
    assert r.shape == (2, 2, 2, 3)
    # element (tile row, tile col, i, j) = (2 * tile_row + i) * 6 + 3 * tile_col + j
    assert np.array_equal(r.eval(), np.arange(24).reshape(2, 2, 2, 3).transpose(0, 2, 1, 3))


@pytest.mark.parametrize("shape, indices", (
    # the cases of reference tests/test_getitem.py:7-24, checked against numpy's own indexing
    ((3, 4, 2), slice(None, None, None)),
    ((3, 4, 2), slice(0, -1, 2)),
    ((2, 3, 4, 5), slice(1, None, 2)),
    ((3, 4, 2), (slice(None), 1, slice(None))),
    ((3, 4, 2), (1, slice(None), None)),
    ((3, 4, 2), (slice(None, None, -1), 0, slice(1, -1))),
    ((3, 4, 2), (..., 1)),
    ((3, 4, 2), (None, slice(None), 1, slice(None))),
    ((6, 5), (slice(2, 4, None), slice(1, 4, None))),
))
def test_getitem_matches_numpy(shape, indices):
    out = Tensor(shape=shape)[indices].eval()
    assert np.array_equal(out, np.arange(int(np.prod(shape))).reshape(shape)[indices])


def test_unsqueeze_golden():
    # the expected arrays of reference tests/test_unsqueeze.py:7-57
    x = Tensor(1)
    bm, bn = ninetoothed.block_size(), ninetoothed.block_size()
    subs = {x: {"shape": (5,)}, bm: 2, bn: 3}
    u = x.unsqueeze(0)
    assert np.array_equal(u.eval(subs), np.array([[0, 1, 2, 3, 4]]))
    ue = u.expand((3, -1))
    assert np.array_equal(ue.eval(subs), np.array([[0, 1, 2, 3, 4]] * 3))
    assert np.array_equal(ue.tile((bm, bn)).eval(subs), np.array([
        [[[0, 1, 2], [0, 1, 2]], [[3, 4, -1], [3, 4, -1]]],
        [[[0, 1, 2], [-1, -1, -1]], [[3, 4, -1], [-1, -1, -1]]],
    ]))
    assert np.array_equal(x.tile((bn,)).unsqueeze(0).eval(subs), np.array([[[0, 1, 2], [3, 4, -1]]]))


def test_simulate_arrangement_golden():
    # reference tests/test_debugging.py:14-251: the addmm arrangement's source and target tensors
    import torch

    from ninetoothed_amd.debugging import simulate_arrangement

    g, targets = _addmm_golden()
    m, n, k, b = g["m"], g["n"], g["k"], g["block_size"]
    arrangement = functools.partial(pg.addmm_arrangement, BLOCK_SIZE_M=b, BLOCK_SIZE_N=b, BLOCK_SIZE_K=b)
    tensors = (Tensor(shape=(m, n)), Tensor(shape=(m, k)), Tensor(shape=(k, n)), Tensor(0), Tensor(0),
               Tensor(shape=(m, n)))
    sources, got = simulate_arrangement(arrangement, tensors, device="cpu")
    for t, expected in zip(sources, g["source_tensors"]):
        assert torch.equal(t, torch.tensor(expected))
    for t, expected in zip(got, targets):
        assert torch.equal(t, torch.from_numpy(expected).to(torch.int64))
