"""The kernels' 32-bit requantisation path equals the reference's 64-bit one.

cpu_int_kernels.py:5-14 computes floor((a * m0) / 2**s) in int64.  For
m0 < 2**31 and s >= 32 the HIP epilogue computes mulhi(a, m0) >> (s - 32)
(signed 32x32 high product, arithmetic shift), and rewrites m0 == 2**31 as
(2**30, s - 1).  Both rewrites are checked here against exact integers.
"""

import numpy as np


def floor_shift(a, m, s):
    return (a * m) >> s                       # python ints: exact floor


def mulhi_path(a, m, s):
    prod = a * m
    hi = prod >> 32                           # signed high word (floor)
    return hi >> (s - 32)


def test_fast_path_identity_random_and_edges():
    rng = np.random.default_rng(0)
    a_vals = [-(2**31), -(2**31) + 1, -1, 0, 1, 2**31 - 1] + list(rng.integers(-2**31, 2**31, 3000))
    m_vals = [0, 1, 2**30, 2**31 - 1] + list(rng.integers(0, 2**31, 300))
    for s in (32, 33, 35, 38, 41, 50, 63):
        for m in m_vals[:60]:
            for a in a_vals[:400]:
                assert floor_shift(int(a), int(m), s) == mulhi_path(int(a), int(m), s)


def test_m0_two_pow_31_rewrite():
    rng = np.random.default_rng(1)
    for s in range(1, 64):
        for a in list(rng.integers(-2**31, 2**31, 200)) + [-(2**31), 2**31 - 1, -1, 0]:
            a = int(a)
            assert floor_shift(a, 2**31, s) == floor_shift(a, 2**30, s - 1)



def test_clamp_before_shift_identity():
    """Per-tensor path: x = mulhi(acc, m0) clamped to [0, hi] and then
    shifted by sh = shift - 32 equals the clamp of x >> sh to [0, 127], with
    hi = 128 * 2**sh - 1 capped at 2**31 - 1 (the int32 range of the
    register; for sh >= 24 every int32 x has x >> sh < 128)."""
    rng = np.random.default_rng(2)
    xs = [-(2**31), -(2**31) + 1, -1, 0, 1, 2**31 - 1] + [int(v) for v in rng.integers(-2**31, 2**31, 4000)]
    for sh in range(32):
        hi = min(128 * 2**sh - 1, 2**31 - 1)
        edges = [hi - 1, hi, hi + 1, 127 * 2**sh - 1, 127 * 2**sh, 128 * 2**sh]
        for x in xs + [e for e in edges if -(2**31) <= e < 2**31]:
            assert min(max(x >> sh, 0), 127) == (min(max(x, 0), hi) >> sh)


def test_signed_clamp_before_shift_identity():
    """Output layer (no ReLU) with per-tensor constants: x clamped to
    [lo, hi] and shifted arithmetically by sh equals the clamp of x >> sh to
    [-128, 127], with lo = -128 * 2**sh capped at -2**31 and hi as above."""
    rng = np.random.default_rng(3)
    xs = [-(2**31), -(2**31) + 1, -1, 0, 1, 2**31 - 1] + [int(v) for v in rng.integers(-2**31, 2**31, 4000)]
    for sh in range(32):
        hi = min(128 * 2**sh - 1, 2**31 - 1)
        lo = max(-128 * 2**sh, -(2**31))
        edges = [lo - 1, lo, lo + 1, hi - 1, hi, hi + 1, -127 * 2**sh, -127 * 2**sh - 1]
        for x in xs + [e for e in edges if -(2**31) <= e < 2**31]:
            assert min(max(x >> sh, -128), 127) == (min(max(x, lo), hi) >> sh)
