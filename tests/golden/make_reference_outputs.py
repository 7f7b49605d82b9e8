"""Writes tests/golden/reference_outputs.npz: the reference's own generated kernels' outputs for
the hot-path programs, on small seeded inputs (stored beside them).

Run once in this container, where the reference's source tree and Triton are present (the
GPU box has neither, and no test needs them):

    python tests/golden/make_reference_outputs.py

The reference runs on Triton's CPU interpreter (TRITON_INTERPRET=1).  Its ``generic`` platform
profile accepts CUDA tensors only (reference src/ninetoothed/targets.py:461-469), so this
script re-registers that profile for CPU tensors in its own process.  Every program is the
reference's own, imported from its test modules (tests/test_matmul.py, test_addmm.py,
test_conv2d.py, test_attention.py, test_dropout.py, test_add.py), except
the fp32 matmul of the README (README.md:35-67), whose five-line application is restated
below.  Kernels are made with one configuration each: the interpreter is too slow to tune.
"""

import dataclasses
import functools
import os
import sys
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"
REFERENCE = Path("/root/reference")
sys.path.insert(0, str(REFERENCE / "src"))
sys.path.insert(0, str(REFERENCE))

import numpy as np  # noqa: E402
import torch  # noqa: E402

import ninetoothed  # noqa: E402  (the reference)
import ninetoothed.language as ntl  # noqa: E402
from ninetoothed import Tensor  # noqa: E402
from ninetoothed.targets import default_platform_registry  # noqa: E402

_registry = default_platform_registry()
_registry.register(dataclasses.replace(_registry.get("generic"), device_types=("cpu",)), replace=True)

from tests import test_add, test_addmm, test_attention, test_conv2d, test_dropout, test_matmul  # noqa: E402


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def _randn(shape, dtype, seed, scale=1.0):
    return (torch.randn(shape, generator=_gen(seed)) * scale).to(dtype)


def _rand(shape, dtype, seed, lo=0.0, hi=1.0):
    return (torch.rand(shape, generator=_gen(seed)) * (hi - lo) + lo).to(dtype)


def readme_matmul_application(input, other, output):
    # the README's fp32 matmul (README.md:56-62): the accumulator is the output
    accumulator = ntl.zeros(output.shape, dtype=ntl.float32)
    for k in range(input.shape[0]):
        accumulator += ntl.dot(input[k], other[k])
    output = accumulator  # noqa: F841


def main():
    out = {}
    import time

    t0 = time.time()

    def done(name):
        print(f"{name}: {time.time() - t0:.1f} s", flush=True)

    # matmul, fp32 (README) and fp16 (tests/test_matmul.py): ragged against every block size
    a, b = _randn((96, 80), torch.float32, 1), _randn((80, 112), torch.float32, 2)
    c = torch.empty((96, 112))
    k = ninetoothed.make(test_matmul.arrangement, readme_matmul_application, (Tensor(2), Tensor(2), Tensor(2)),
                         max_num_configs=1)
    k(a, b, c)
    out.update(matmul_fp32_a=a, matmul_fp32_b=b, matmul_fp32_out=c)
    a, b = _randn((64, 96), torch.float16, 3), _randn((96, 80), torch.float16, 4)
    c = torch.empty((64, 80), dtype=torch.float16)
    k = ninetoothed.make(test_matmul.arrangement, test_matmul.application, (Tensor(2), Tensor(2), Tensor(2)),
                         max_num_configs=1)
    k(a, b, c)
    out.update(matmul_fp16_a=a, matmul_fp16_b=b, matmul_fp16_out=c)
    done("matmul")

    # addmm fp16 (tests/test_addmm.py), beta 0.5, alpha 1.0 (0-d parameters)
    inp, m1, m2 = _randn((64, 80), torch.float16, 5), _randn((64, 96), torch.float16, 6), \
        _randn((96, 80), torch.float16, 7)
    c = torch.empty((64, 80), dtype=torch.float16)
    k = ninetoothed.make(test_addmm.arrangement, test_addmm.application,
                         (Tensor(2), Tensor(2), Tensor(2), Tensor(0), Tensor(0), Tensor(2)), max_num_configs=1)
    k(inp, m1, m2, 0.5, 1.0, c)
    out.update(addmm_input=inp, addmm_mat1=m1, addmm_mat2=m2, addmm_out=c)
    done("addmm")

    # conv2d fp16, padding (1, 1) (tests/test_conv2d.py:92-116, one configuration)
    x, w = _rand((2, 16, 10, 10), torch.float16, 8), _rand((32, 16, 3, 3), torch.float16, 9)
    y = torch.empty((2, 32, 10, 10), dtype=torch.float16)
    k = ninetoothed.make(functools.partial(test_conv2d.arrangement, enable_padding=True),
                         test_conv2d.matmul.application,
                         (Tensor(4), Tensor(4, shape_options={"constexpr": True}), Tensor(4)), max_num_configs=1)
    k(x, w, y, padding_h=1, padding_w=1)
    out.update(conv2d_x=x, conv2d_w=w, conv2d_out=y)
    done("conv2d")

    # attention fp16, causal and not (tests/test_attention.py:73-96, one configuration): 96
    # queries and keys
    q, kk, v = (_randn((1, 2, 96, 64), torch.float16, s) for s in (10, 11, 12))
    out.update(attention_q=q, attention_k=kk, attention_v=v)
    specs = tuple(Tensor(4, shape_options=(None, None, {"constexpr": True}, {"constexpr": True, "upper_bound": 128}))
                  for _ in range(4))
    k = ninetoothed.make(test_attention.arrangement, test_attention.application,
                         specs[:3] + (Tensor(0, constexpr=True),) + specs[3:], max_num_configs=1)
    for causal in (False, True):
        o = torch.empty_like(q)
        k(q, kk, v, causal, o)
        out[f"attention_out_causal{int(causal)}"] = o
    done("attention")
    # (softmax and max_pool2d, tests/test_softmax.py:10-27 and test_max_pool2d.py:39-64, are
    # not here: Triton 3.6's interpreter fails on the reductions in the kernels the reference
    # generates for them, with an AttributeError inside the interpreter.  max_pool2d is pinned
    # bit for bit by F.max_pool2d; softmax by torch.softmax within tolerance.)

    # dropout fp16, p = 0.3, a fixed seed (tests/test_dropout.py:10-24): ntl.rand through the
    # whole program, x / (1 - p) in the reference's typing
    x = _randn((349,), torch.float16, 17)
    y = torch.empty_like(x)
    k = ninetoothed.make(test_dropout.arrangement, test_dropout.application,
                         (Tensor(1), Tensor(0), Tensor(0), Tensor(1)), max_num_configs=1)
    k(x, 0.3, 1234567, y)
    out.update(dropout_x=x, dropout_out=y)

    # add fp32 (tests/test_add.py:9-24)
    lhs, rhs = _randn((1000,), torch.float32, 15), _randn((1000,), torch.float32, 16)
    out.update(add_lhs=lhs, add_rhs=rhs, add_out=test_add.add(lhs, rhs))

    arrays = {}
    for key, t in out.items():
        t = t.contiguous()
        # 16-bit tensors as their bits, so that the fixture loads without torch
        arrays[key] = t.view(torch.int16).numpy() if t.dtype == torch.float16 else t.numpy()
        arrays[key + "__dtype"] = np.array(str(t.dtype).replace("torch.", ""))
    path = Path(__file__).with_name("reference_outputs.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
