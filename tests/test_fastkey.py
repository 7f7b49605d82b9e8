"""The Handle's call key in C++ (ninetoothed_amd._fastkey): equal bytes exactly when every
tensor's dtype, shape, strides, device and data-pointer alignment agree."""

import pytest
import torch

_fastkey = pytest.importorskip("ninetoothed_amd._fastkey")


def test_equal_metadata_gives_equal_keys():
    a, b = torch.empty(64, 32), torch.empty(64, 32)
    assert _fastkey.key((a, b)) == _fastkey.key((torch.empty(64, 32), torch.empty(64, 32)))
    assert isinstance(_fastkey.key((a,)), bytes)
    assert _fastkey.key(()) == b""


@pytest.mark.parametrize("other", [
    lambda a: a.half(),                    # dtype
    lambda a: a.reshape(32, 64),           # shape
    lambda a: a.t().contiguous().t(),      # strides
    lambda a: a[:, 1:].contiguous()[:, :31].reshape(64, 31),  # shape again, another rank size
    lambda a: torch.empty(64 * 32 + 1)[1:].view(64, 32),      # data pointer 4 bytes past 16-byte alignment
    lambda a: a.unsqueeze(0),              # rank
])
def test_each_field_changes_the_key(other):
    a = torch.empty(64, 32)
    assert _fastkey.key((a,)) != _fastkey.key((other(a),))


def test_order_matters():
    a, b = torch.empty(8, 8), torch.empty(8, 8, dtype=torch.float16)
    assert _fastkey.key((a, b)) != _fastkey.key((b, a))


def test_non_tensors_and_tensors_without_strides_give_none():
    a = torch.empty(4)
    assert _fastkey.key((a, 1.0)) is None
    sparse = torch.sparse_coo_tensor(torch.tensor([[0, 1]]), torch.tensor([1.0, 2.0]), (4,))
    assert _fastkey.key((sparse,)) is None
    with pytest.raises(TypeError):
        _fastkey.key([a])


@pytest.fixture(scope="module")
def echo_library(tmp_path_factory):
    """A host library whose entry point records the packed array it is called with."""
    import ctypes
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("no host C compiler")
    d = tmp_path_factory.mktemp("echo")
    (d / "echo.c").write_text(
        "#include <stdint.h>\n#include <string.h>\nstatic int64_t seen[22];\n"
        "int echo(const int64_t* v) { memcpy(seen, v, sizeof(seen)); return (int)v[0]; }\n"
        "const int64_t* last(void) { return seen; }\n")
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", str(d / "echo.c"), "-o", str(d / "libecho.so")], check=True)
    lib = ctypes.CDLL(str(d / "libecho.so"))
    lib.last.restype = ctypes.POINTER(ctypes.c_int64)
    return lib, ctypes.cast(lib.echo, ctypes.c_void_p).value


def test_call_fills_slots(echo_library):
    import struct

    lib, addr = echo_library
    a, b = torch.empty(16), torch.empty(16, dtype=torch.float16)
    template = struct.pack("<22q", 7, *range(100, 121))
    rc = _fastkey.call(addr, template, (1, 4, 7), (a, None, b), (17, 21), (0x3F000000, 2**64 - 1))
    assert rc == 7
    seen = lib.last()[:22]
    assert seen[1] == a.data_ptr() and seen[4] == 0 and seen[7] == b.data_ptr()
    assert seen[17] == 0x3F000000 and seen[21] == -1
    untouched = [i for i in range(22) if i not in (0, 1, 4, 7, 17, 21)]
    assert [seen[i] for i in untouched] == [100 + i - 1 for i in untouched]


def test_malformed_calls_raise(echo_library):
    import struct

    _, addr = echo_library
    t = torch.empty(4)
    template = struct.pack("<22q", *range(22))
    with pytest.raises(ValueError):
        _fastkey.call(addr, template[:-1], (), (), (), ())
    with pytest.raises(ValueError):
        _fastkey.call(addr, template, (22,), (t,), (), ())
    with pytest.raises(ValueError):
        _fastkey.call(addr, template, (), (), (-1,), (0,))
    with pytest.raises(TypeError):
        _fastkey.call(addr, template, (1,), (3,), (), ())
    with pytest.raises(ValueError):
        _fastkey.call(0, template, (), (), (), ())


def test_packed_gemm_rejects_unknown_entries_before_launching():
    import struct

    from ninetoothed_amd import _lib, kernels

    if "nt_gemm_packed" not in _lib.exported_symbols():
        pytest.skip("library not built")
    addr = kernels._packed_address("nt_gemm_packed")
    assert addr is not None
    nt_err_invalid = 1  # include/nt_mi355x.h
    for which, config in ((9, 0), (2, 1), (-1, 0)):  # no such entry; a config on an fp32 GEMM
        template = struct.pack("<22q", which, *([0] * 19), config, 0)
        assert _fastkey.call(addr, template, (), (), (), ()) == nt_err_invalid
