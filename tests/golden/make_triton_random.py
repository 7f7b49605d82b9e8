"""Writes tests/golden/triton_random.json: Triton's own ``tl.randint`` / ``tl.rand`` /
``tl.randn`` outputs, which the reference's ``ntl.rand`` family forwards to (reference
src/ninetoothed/language.py:1-26; its dropout test calls ``ntl.rand(seed, offsets)``,
tests/test_dropout.py:16-17).

Run once in a container where Triton is installed (it is not needed by any test), on the CPU
interpreter:  TRITON_INTERPRET=1 python tests/golden/make_triton_random.py
The fixture pins the oracle's (seed, offset) -> (key, counter) mapping and its Box-Muller
composition (oracle/philox.py) against the generator itself.
"""

import json
import os
from pathlib import Path

assert os.environ.get("TRITON_INTERPRET") == "1", "run with TRITON_INTERPRET=1 (CPU interpreter)"

import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402


@triton.jit
def _draw(offsets, out_i, out_u, out_n, seed, N: tl.constexpr):
    i = tl.arange(0, N)
    o = tl.load(offsets + i)
    tl.store(out_i + i, tl.randint(seed, o))
    tl.store(out_u + i, tl.rand(seed, o))
    tl.store(out_n + i, tl.randn(seed, o))


SEEDS = (0, 1, 1234, 2**31 - 1, 2**32 + 7, 0x0123456789ABCDEF)
OFFSETS = [0, 1, 2, 3, 63, 64, 1000, 65535, 65536, 2**24 + 1, 2**31 - 1] + list(range(100, 121))


def main():
    n = 64
    offs = np.zeros(n, dtype=np.int32)
    offs[: len(OFFSETS)] = OFFSETS
    cases = []
    for seed in SEEDS:
        oi, ou, on = torch.empty(n, dtype=torch.int32), torch.empty(n), torch.empty(n)
        _draw[(1,)](torch.from_numpy(offs), oi, ou, on, seed, N=n)
        k = len(OFFSETS)
        cases.append({"seed": seed, "offsets": OFFSETS, "randint": oi[:k].tolist(),
                      "rand": ou[:k].tolist(), "randn": on[:k].tolist()})
    out = {"generator": f"triton {triton.__version__} (TRITON_INTERPRET=1)", "cases": cases}
    path = Path(__file__).with_name("triton_random.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
