"""AutoTuner (reference tests/test_auto_tuner.py) and tuned Handles.

CPU: the contract of the reference's AutoTuner — every candidate benchmarked once per
argument key, the selection persisted so a new tuner with the same namespace and
candidates benchmarks nothing, failing candidates recorded as infinite timings (and timed
again by the next election), an error naming every reason when all fail.  Programs that update a tensor they read are never
tuned.  GPU: a Handle made with ``max_num_configs`` > 1 times the fitting kernels (the add
kernel and the generic kernel) and computes the same result.
"""

import uuid

import pytest
import torch

import ninetoothed_amd as ninetoothed
import ninetoothed_amd.language as ntl
import programs as pg
from ninetoothed_amd import Symbol, Tensor, families
from ninetoothed_amd.auto_tuner import AutoTuner, signature


@pytest.fixture(autouse=True)
def _cache_dir(tmp_path, monkeypatch):
    monkeypatch.setenv("NINETOOTHED_AMD_CACHE_DIR", str(tmp_path / "cache"))


def _foo(*args, **kwargs):
    return "foo"


def _bar(*args, **kwargs):
    return "bar"


def _deterministic(function, args, kwargs):
    return {_foo: 2.0, _bar: 1.0}.get(function, 3.0)


@pytest.mark.parametrize("kwargs", ({"a": 2, "b": 4}, {"a": 2, "b": 4, "c": 6, "d": 8}))
@pytest.mark.parametrize("args", ((1,), (1, 3, 5)))
def test_auto_tuner(args, kwargs):
    calls = []

    def benchmark(function, a, k):
        calls.append(function)
        return _deterministic(function, a, k)

    namespace = f"test_{uuid.uuid4().hex}"
    tuner = AutoTuner((_foo, _bar), ("_foo", "_bar"), benchmark=benchmark, cache_namespace=namespace)
    assert not tuner.book.path.exists()
    assert tuner(*args, **kwargs) == "bar"
    assert calls == [_foo, _bar]
    assert tuner(*args, **kwargs) == "bar" and calls == [_foo, _bar]  # no new benchmarks
    assert tuner.book.path.exists()
    assert tuner.timings(*args, **kwargs) == {"_foo": 2.0, "_bar": 1.0}

    again = []
    cached = AutoTuner((_foo, _bar), ("_foo", "_bar"), benchmark=lambda *c: again.append(c) or 0.0,
                       cache_namespace=namespace)
    assert cached(*args, **kwargs) == "bar" and not again  # a new tuner reads the book
    # another argument signature is benchmarked anew, and only that one
    cached(*args, 99, **kwargs)
    assert len(again) == 2
    # other candidate keys or another namespace are another book
    assert AutoTuner((_foo, _bar), ("x", "y"), cache_namespace=namespace).book.path != tuner.book.path
    assert AutoTuner((_foo, _bar), ("_foo", "_bar"), cache_namespace="other").book.path != tuner.book.path


def test_failing_candidates_are_skipped_and_reported():
    def broken(*a, **k):
        raise RuntimeError("boom")

    def benchmark(function, a, k):
        if function is broken:
            raise RuntimeError("boom")
        return 1.0

    tuner = AutoTuner((broken, _foo), ("broken", "_foo"), benchmark=benchmark, cache_namespace=uuid.uuid4().hex)
    assert tuner(1) == "foo"
    assert tuner.timings(1)["broken"].startswith("error: RuntimeError: boom")
    all_broken = AutoTuner((broken, broken), ("first", "second"), benchmark=benchmark,
                           cache_namespace=uuid.uuid4().hex)
    with pytest.raises(RuntimeError, match="All auto-tuning candidates failed: first: RuntimeError: boom; "
                                           "second: RuntimeError: boom"):
        all_broken(1)


def test_failed_candidate_is_retimed_by_a_new_election():
    # a candidate that failed once (a transient error, a kernel bug fixed since) is timed
    # again by the next tuner on the same book, and wins when it is now the fastest
    namespace = uuid.uuid4().hex
    state = {"fail": True}

    def flaky(*a, **k):
        return "flaky"

    def benchmark(function, a, k):
        if function is flaky:
            if state["fail"]:
                raise RuntimeError("device busy")
            return 0.5
        return 1.0

    first = AutoTuner((flaky, _foo), ("flaky", "_foo"), benchmark=benchmark, cache_namespace=namespace)
    assert first(1) == "foo"
    assert first.timings(1)["flaky"].startswith("error: RuntimeError: device busy")
    state["fail"] = False
    second = AutoTuner((flaky, _foo), ("flaky", "_foo"), benchmark=benchmark, cache_namespace=namespace)
    assert second(1) == "flaky"
    assert second.timings(1) == {"flaky": 0.5, "_foo": 1.0}
    # a row where every candidate failed is not final either
    all_failed = uuid.uuid4().hex
    state["fail"] = True
    with pytest.raises(RuntimeError, match="All auto-tuning candidates failed"):
        AutoTuner((flaky,), ("flaky",), benchmark=benchmark, cache_namespace=all_failed)(1)
    state["fail"] = False
    assert AutoTuner((flaky,), ("flaky",), benchmark=benchmark, cache_namespace=all_failed)(1) == "flaky"


def test_book_is_keyed_by_library_build(monkeypatch):
    from ninetoothed_amd import auto_tuner

    book = AutoTuner((_foo,), ("_foo",), cache_namespace="ns").book.path
    monkeypatch.setattr(auto_tuner, "_BUILD", "another-build")
    assert AutoTuner((_foo,), ("_foo",), cache_namespace="ns").book.path != book


def test_winner_that_raises_is_not_kept():
    def fails(*a, **k):
        raise RuntimeError("Winner invocation failed.")

    tuner = AutoTuner((fails,), ("winner",), benchmark=lambda *c: 1.0, cache_namespace=uuid.uuid4().hex)
    with pytest.raises(RuntimeError, match="Winner invocation failed"):
        tuner(1)
    assert tuner._winners == {}


def test_validator_and_key_checks():
    with pytest.raises(ValueError, match="one key for every candidate"):
        AutoTuner((_foo, _bar), ("_foo",))
    seen = []
    tuner = AutoTuner((_foo,), ("_foo",), benchmark=lambda *c: 1.0, validator=lambda a, k: seen.append(a),
                      cache_namespace=uuid.uuid4().hex)
    tuner(3)
    assert seen == [(3,)]
    sig = signature((torch.empty(2, 3),), {"x": 1})
    assert "[2,3]" in sig and "[3,1]" in sig and '"x"' in sig


def test_signature_tells_alignment_apart():
    # A launcher tuned on aligned operands may have chosen a kernel that needs them: a
    # misaligned view of the same shape and strides is a different signature.
    base = torch.empty(1025, dtype=torch.float16)
    aligned, shifted = base[:1024], base[1:]
    assert aligned.shape == shifted.shape and aligned.stride() == shifted.stride()
    assert signature((aligned,), {}) != signature((shifted,), {})
    assert signature((aligned,), {}) == signature((base[:1024].clone(),), {})


def _add_handle(**options):
    bs = Symbol("BS", meta=True)

    def app(a, b, out):
        out = a + b  # noqa: F841

    return ninetoothed.make(lambda a, b, o: (a.tile((bs,)), b.tile((bs,)), o.tile((bs,))), app,
                            (Tensor(1), Tensor(1), Tensor(1)), **options)


def test_candidates_and_in_place_programs():
    h = _add_handle()
    v = torch.empty(1000)
    ctx = h._kernel.context({"a": v, "b": v, "out": v}, {})
    assert [p.describe()["family"] for p in families.candidates(ctx)] == ["add", "generic"]
    assert not families.updates_an_input(ctx.program)
    tuned = h._kernel.specialize({"a": v, "b": v, "out": v}, {}, tune=True)
    assert tuned.describe()["family"] == "tuned"

    def inplace(x):
        x = x + 1.0  # noqa: F841

    bs = Symbol("BS", meta=True)
    k = ninetoothed.make(lambda x: (x.tile((bs,)),), inplace, (Tensor(1),))
    ctx = k._kernel.context({"x": v}, {})
    assert families.updates_an_input(ctx.program)
    assert k._kernel.specialize({"x": v}, {}, tune=True).describe()["family"] == "generic"


@pytest.mark.gpu
def test_tuned_handle_picks_a_kernel_and_computes():
    h = _add_handle(max_num_configs=4)
    a, b = torch.randn(100_000, device="cuda"), torch.randn(100_000, device="cuda")
    out = torch.empty_like(a)
    h(a, b, out)
    assert torch.equal(out, a + b)
    (plan,) = h.plans()
    assert plan["family"] == "tuned" and len(plan["chosen"]) == 1
    out2 = torch.empty_like(a)
    h(a, b, out2)  # the bound winner, no new benchmark
    assert torch.equal(out2, a + b)


def test_gemm_plans_expand_into_kernel_configs():
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    t = torch.empty(512, 512, dtype=torch.float16)
    ctx = h._kernel.context({"lhs": t, "rhs": t, "output": t}, {})
    described = [p.describe() for p in families.candidates(ctx)]
    assert [d["family"] for d in described] == ["gemm"] * 5
    assert [d["config"] for d in described] == [1, 2, 3, 4, 5]
    assert "config" not in families.select(ctx).describe()  # untuned: the library picks


@pytest.mark.gpu
def test_tuned_matmul_picks_a_kernel_config():
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors(), max_num_configs=4)
    g = torch.Generator().manual_seed(5)
    a, b = (torch.randn(512, 512, generator=g).half().cuda() for _ in range(2))
    out = torch.empty(512, 512, dtype=torch.float16, device="cuda")
    h(a, b, out)
    assert torch.allclose(out.float(), (a.float() @ b.float()).half().float(), atol=2e-2, rtol=1e-2)
    (plan,) = h.plans()
    assert plan["family"] == "tuned" and len(plan["chosen"]) == 1 and '"config"' in plan["chosen"][0]


def test_handle_key_tells_alignment_apart():
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors())
    base = torch.empty(512 * 512 + 8, dtype=torch.float16)
    aligned, shifted = base[:512 * 512].view(512, 512), base[1:512 * 512 + 1].view(512, 512)
    assert aligned.stride() == shifted.stride()
    assert h._fast_key((aligned,) * 3, {}) != h._fast_key((shifted,) * 3, {})


@pytest.mark.gpu
def test_tuned_matmul_then_misaligned_view():
    # The aligned call may bind a kernel that needs 16-byte aligned operands; a later call
    # with the same shapes and strides but a misaligned view must not reuse that launcher.
    h = ninetoothed.make(pg.matmul_arrangement, pg.matmul_application, pg.matmul_tensors(), max_num_configs=4)
    g = torch.Generator().manual_seed(6)
    base = torch.randn(2, 512 * 512 + 8, generator=g).half().cuda()
    a, b = base[0, :512 * 512].view(512, 512), base[1, :512 * 512].view(512, 512)
    a1, b1 = base[0, 1:512 * 512 + 1].view(512, 512), base[1, 1:512 * 512 + 1].view(512, 512)
    for x, y in ((a, b), (a1, b1)):
        out = torch.empty(512, 512, dtype=torch.float16, device="cuda")
        h(x, y, out)
        assert torch.allclose(out.float(), (x.float() @ y.float()).half().float(), atol=2e-2, rtol=1e-2)


def test_conv_plans_expand_into_paths():
    h = pg.make_conv2d()
    x = torch.empty(2, 64, 16, 16, dtype=torch.float16)
    w = torch.empty(96, 64, 3, 3, dtype=torch.float16)
    y = torch.empty(2, 96, 16, 16, dtype=torch.float16)
    names = list(h._kernel.params)
    ctx = h._kernel.context(dict(zip(names, (x, w, y))), {"padding_h": 1, "padding_w": 1})
    described = [p.describe() for p in families.candidates(ctx)]
    assert [(d["family"], d["config"]) for d in described] == [("conv2d", 1), ("conv2d", 2), ("conv2d", 3),
                                                                ("conv2d", 4), ("conv2d", 5), ("conv2d", 6),
                                                                ("conv2d", 7)]


@pytest.mark.gpu
def test_tuned_conv_picks_a_path():
    import torch.nn.functional as F

    h = pg.make_conv2d(max_num_configs=4)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 64, 16, 16, generator=g).half().cuda()
    w = (torch.randn(96, 64, 3, 3, generator=g) / 24).half().cuda()
    y = torch.empty(2, 96, 16, 16, dtype=torch.float16, device="cuda")
    h(x, w, y, padding_h=1, padding_w=1)
    ref = F.conv2d(x.float(), w.float(), padding=1).half().float()
    assert torch.allclose(y.float(), ref, atol=2e-2, rtol=1e-2)
    (plan,) = h.plans()
    assert plan["family"] == "tuned" and len(plan["chosen"]) == 1 and '"config"' in plan["chosen"][0]


def test_attention_plans_expand_into_kernels():
    h = ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors())
    q = torch.empty(1, 2, 256, 128, dtype=torch.float16)
    names = list(h._kernel.params)
    ctx = h._kernel.context(dict(zip(names, (q, q, q, True, q))), {})
    described = [p.describe() for p in families.candidates(ctx)]
    assert [(d["family"], d["config"]) for d in described] == [("attention", 1), ("attention", 2), ("attention", 3)]


@pytest.mark.gpu
def test_tuned_attention_picks_a_kernel():
    import math

    import torch.nn.functional as F

    h = ninetoothed.make(pg.attention_arrangement, pg.attention_application_scaled, pg.attention_tensors(),
                         max_num_configs=4)
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(1, 4, 512, 128, generator=g).half().cuda() for _ in range(3))
    o = torch.empty_like(q)
    h(q, k, v, True, o)
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True, scale=1 / math.sqrt(128))
    assert torch.allclose(o.float(), ref, atol=1e-2, rtol=1e-2)
    (plan,) = h.plans()
    assert plan["family"] == "tuned" and len(plan["chosen"]) == 1 and '"attention"' in plan["chosen"][0]


def test_softmax_and_pool_plans_expand_into_kernels():
    import functools

    sm = pg.make_softmax()
    x = torch.empty(8, 300)
    ctx = sm._kernel.context(dict(zip(list(sm._kernel.params), (x, x))), {"BLOCK_SIZE": 300})
    described = [p.describe() for p in families.candidates(ctx)]
    assert [(d["family"], d.get("config")) for d in described] == [
        ("softmax", 1), ("softmax", 2), ("softmax", 3), ("softmax", 4), ("softmax", 5), ("softmax", 6),
        ("generic", None)]
    # a transposed input or an output of another dtype: only the element-wise kernel admits it
    xt = torch.empty(300, 8).t()
    ctx = sm._kernel.context(dict(zip(list(sm._kernel.params), (xt, x))), {"BLOCK_SIZE": 300})
    assert [(d["family"], d.get("config")) for d in map(lambda p: p.describe(), families.candidates(ctx))] == [
        ("softmax", 6), ("generic", None)]
    ctx = sm._kernel.context(dict(zip(list(sm._kernel.params), (x.half(), x))), {"BLOCK_SIZE": 300})
    assert [(d["family"], d.get("config")) for d in map(lambda p: p.describe(), families.candidates(ctx))] == [
        ("softmax", 6), ("generic", None)]
    pool = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=False), pg.max_pool2d_application,
                            pg.max_pool2d_tensors())
    xi, yo = torch.empty(2, 3, 16, 16, dtype=torch.float16), torch.empty(2, 3, 8, 8, dtype=torch.float16)
    ctx = pool._kernel.context(dict(zip(list(pool._kernel.params), (xi, yo))), {"WINDOW_HEIGHT": 2, "WINDOW_WIDTH": 2})
    described = [p.describe() for p in families.candidates(ctx)]
    assert [(d["family"], d.get("config")) for d in described][:4] == [
        ("max_pool2d", 1), ("max_pool2d", 2), ("max_pool2d", 3), ("max_pool2d", 4)]
    ctx = pool._kernel.context(dict(zip(list(pool._kernel.params), (xi, yo.float()))),
                               {"WINDOW_HEIGHT": 2, "WINDOW_WIDTH": 2})
    described = [p.describe() for p in families.candidates(ctx)]
    assert [(d["family"], d.get("config")) for d in described][:1] == [("max_pool2d", 2)]
    assert all(d["family"] != "max_pool2d" for d in described[1:])


@pytest.mark.gpu
def test_tuned_softmax_and_pool_pick_a_kernel():
    import functools

    import torch.nn.functional as F

    sm = pg.make_softmax(max_num_configs=5)
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(64, 3000, generator=g) * 2).half().cuda()
    y = torch.empty_like(x)
    sm(x, y, BLOCK_SIZE=3000)
    assert torch.allclose(y.float(), torch.softmax(x.float(), -1), atol=1e-2, rtol=1e-2)
    (plan,) = sm.plans()
    assert plan["family"] == "tuned" and len(plan["chosen"]) == 1
    pool = ninetoothed.make(functools.partial(pg.max_pool2d_arrangement, ceil_mode=False), pg.max_pool2d_application,
                            pg.max_pool2d_tensors(), max_num_configs=3)
    xi = (torch.rand(4, 8, 64, 64, generator=g) * 2 - 1).half().cuda()
    yo = torch.empty(4, 8, 32, 32, dtype=torch.float16, device="cuda")
    pool(xi, yo, WINDOW_HEIGHT=2, WINDOW_WIDTH=2)
    assert torch.equal(yo, F.max_pool2d(xi, (2, 2)))
    (plan,) = pool.plans()
    assert plan["family"] == "tuned" and len(plan["chosen"]) == 1
