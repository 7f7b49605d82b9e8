"""This backend behind the reference's plugin points (``ninetoothed_amd.backends.reference``).

The reference cannot be imported here, so ``reference_double`` (a package of our own with the
reference's object model for what the adapter reads) stands for it, and
``reference_user_programs`` holds programs written against its API as a reference user writes
them.  CPU: symbol and tensor conversion (roles, bounds, fixed sizes), registration in both
registries, re-bound programs (the application's ``ntl`` and a helper's resolve to this
package) matched to the add and softmax kernels.  GPU: both run through the adapter's Handle.
"""

import pytest
import torch

import ninetoothed_amd as ninetoothed
import reference_double as ref
import reference_user_programs as user
from ninetoothed_amd.backends import reference as adapter


def _request(arrangement, application, tensors, name):
    return ref.Compilation(request=ref.compiler.CompileRequest(
        arrangement=arrangement, application=application, tensors=tensors, caller="torch", kernel_name=name))


def _add():
    return _request(user.add_arrangement, user.add_application, (ref.Tensor(1), ref.Tensor(1), ref.Tensor(1)), "add")


def _softmax():
    # the reference's softmax input: masked elements read -inf (reference tests/test_softmax.py)
    return _request(user.softmax_arrangement, user.softmax_application,
                    (ref.Tensor(2, other=float("-inf")), ref.Tensor(2)), "softmax")


def test_symbols_and_tensors_convert_with_their_roles_and_bounds():
    objects = adapter.ReferenceObjects(ref)
    s = objects.symbol(user.BLOCK_SIZE)
    assert isinstance(s, ninetoothed.Symbol) and str(s) == "BLOCK_SIZE"
    assert s.meta and s.constexpr and (s.lower_bound, s.upper_bound, s.power_of_two) == (32, 1024, True)
    c = objects.symbol(ref.Symbol("N", constexpr=True, upper_bound=64))
    assert not c.meta and c.constexpr and c.upper_bound == 64
    e = objects.symbol(ref.Symbol("K", meta=True) * 2)
    assert isinstance(e, ninetoothed.Symbol) and "K" in str(e)
    t = objects.tensor(ref.Tensor(shape=(None, 8), dtype="float16", other=0.0))
    assert isinstance(t, ninetoothed.Tensor) and t.ndim == 2 and t.shape[1] == 8 and t.other == 0.0
    assert objects.value(ref) is ninetoothed and objects.value(ref.language) is ninetoothed.language
    assert objects.value(ref.block_size) is ninetoothed.block_size
    with pytest.raises(NotImplementedError):
        arranged = ref.Tensor(1)
        arranged.source = ref.Tensor(1)
        objects.tensor(arranged)


def test_register_adds_backend_and_materializer():
    backend, materializer = adapter.register(ref, replace=True)
    assert ref.backends.default_registry().get("hip") is backend
    assert ref.backends.materializers.materializer_for("hip") is materializer
    assert backend.capability.can_execute and backend.emit(type("K", (), {"name": "add"})()).kernel_name == "add"


def test_reference_programs_match_the_kernels():
    m = adapter.ReferenceMaterializer(ref)
    add = m.jit_materialize(_add())
    x = torch.empty(4096, dtype=torch.float16)
    names = add._abi["public_args"]
    assert add._kernel.specialize(dict(zip(names, (x, x, x))), {"BLOCK_SIZE": 1024}).describe()["family"] == "add"
    sm = m.jit_materialize(_softmax())
    y = torch.empty(64, 300, dtype=torch.float16)
    names = sm._abi["public_args"]
    plan = sm._kernel.specialize(dict(zip(names, (y, y))), {p: 512 for p in sm._abi["meta_args"]})
    assert plan.describe()["family"] == "softmax"


@pytest.mark.gpu
def test_reference_programs_run_through_the_adapter():
    m = adapter.ReferenceMaterializer(ref)
    add = m.jit_materialize(_add())
    a = torch.randn(10000, device="cuda", dtype=torch.float16)
    b = torch.randn(10000, device="cuda", dtype=torch.float16)
    out = torch.empty_like(a)
    add(a, b, out, BLOCK_SIZE=1024)
    assert torch.equal(out, a + b)
    sm = m.jit_materialize(_softmax())
    x = torch.randn(64, 300, device="cuda", dtype=torch.float16)
    y = torch.empty_like(x)
    sm(x, y, **{n: 512 for n in sm._abi["meta_args"]})
    torch.testing.assert_close(y.float(), torch.softmax(x.float(), dim=1), rtol=1e-2, atol=1e-3)
