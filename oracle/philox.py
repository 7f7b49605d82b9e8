"""Oracle: the counter-based random numbers of ``ntl.rand`` / ``randint`` / ``randn`` (TEST ONLY).

The reference's ``ninetoothed.language`` forwards these names to Triton
(``src/ninetoothed/language.py:1-26``; the dropout test calls
``ntl.rand(seed, input.offsets())``, reference tests/test_dropout.py:16-17).  Triton
(pinned by the reference's environment; not installed here) documents them as Philox4x32
with 10 rounds, keyed by the 64-bit seed (low word, high word) on the counter
(offset, 0, 0, 0).  This module restates that published generator (Salmon, Moraes, Dror,
Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11; the Random123 multipliers
and Weyl key increments) with numpy uint64 arithmetic:

  round:  (c0, c1, c2, c3) <- (hi(B*c2) ^ c1 ^ k0,  lo(B*c2),  hi(A*c0) ^ c3 ^ k1,  lo(A*c0))
  key:    (k0, k1) <- (k0 + 0x9E3779B9, k1 + 0xBB67AE85)         (mod 2^32, after each round)
  A = 0xD2511F53, B = 0xCD9E8D57

``randint`` is the first word of the output.  ``rand`` maps it to [0, 1): reinterpret as
int32 x, take x if x >= 0 else -x - 1, convert to float32 (nearest) and multiply by the
float32 constant 4.6566127342e-10 (just below 2^-31).  ``randn`` is Box-Muller on the first
two words mapped that way: u1 = max(u1, 1e-7), r = sqrt(-2 log u1), r * cos(2 pi u2).

Pinned against the Random123 known-answer vectors for philox4x32-10 in
tests/test_oracle_apply.py::test_philox_known_answers, and end to end (the (seed, offset) ->
(key, counter) mapping, the uniform map and Box-Muller) against Triton 3.6.0's own outputs in
tests/golden/triton_random.json (written by tests/golden/make_triton_random.py on Triton's
CPU interpreter; randint and rand bit for bit, randn to 1e-6) in
tests/test_oracle_apply.py::test_random_streams_match_tritons_generator.
"""

import numpy as np

_A, _B = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_KA, _KB = np.uint64(0x9E3779B9), np.uint64(0xBB67AE85)
_M32 = np.uint64(0xFFFFFFFF)
_S32 = np.uint64(32)


def philox4x32(counter, key, rounds=10):
    """Philox4x32-``rounds``: counter (4 uint32 arrays), key (2 uint32 arrays) -> 4 uint32 arrays."""
    c = [np.asarray(x, dtype=np.uint64) & _M32 for x in counter]
    k0, k1 = (np.asarray(x, dtype=np.uint64) & _M32 for x in key)
    for _ in range(rounds):
        p0 = _A * c[0]
        p1 = _B * c[2]
        c = [((p1 >> _S32) ^ c[1] ^ k0) & _M32, p1 & _M32, ((p0 >> _S32) ^ c[3] ^ k1) & _M32, p0 & _M32]
        k0 = (k0 + _KA) & _M32
        k1 = (k1 + _KB) & _M32
    return tuple(x.astype(np.uint32) for x in c)


def _words(seed, offset):
    seed = np.uint64(int(seed) & 0xFFFFFFFFFFFFFFFF)
    offset = np.asarray(offset, dtype=np.int64).astype(np.uint64) & _M32
    zero = np.zeros_like(offset)
    return philox4x32((offset, zero, zero, zero), (seed & _M32, (seed >> _S32) & _M32))


def uniform(words):
    """uint32 -> float32 in [0, 1), as ``rand`` maps them."""
    x = np.asarray(words, dtype=np.uint32).view(np.int32).astype(np.int64)
    x = np.where(x < 0, -x - 1, x)
    return x.astype(np.float32) * np.float32(4.6566127342e-10)


def randint(seed, offset):
    return _words(seed, offset)[0]


def rand(seed, offset):
    return uniform(randint(seed, offset))


def randn(seed, offset):
    w = _words(seed, offset)
    u1 = np.maximum(uniform(w[0]), np.float32(1e-7))
    u2 = uniform(w[1])
    th = np.float32(6.283185307179586) * u2
    r = np.sqrt(np.float32(-2.0) * np.log(u1))
    return (r * np.cos(th)).astype(np.float32)
