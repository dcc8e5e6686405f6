"""The kernels' 32-bit requantisation path equals the reference's 64-bit one,
and clamping before the per-channel shift equals clamping after it.

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


def clamp_then_shift(x, sh, lo_out):
    """The kernels' order (rq_clamp / rq_insert): clamp the int32 high
    product to [lo_out * 2**sh, 128 * 2**sh - 1] held inside the int32 range
    (hi = INT32_MAX for sh >= 24, lo = ~hi = -hi - 1 without ReLU), then
    shift arithmetically."""
    hi = 2**31 - 1 if sh >= 24 else (128 << sh) - 1
    lo = 0 if lo_out == 0 else -hi - 1
    return min(max(x, lo), hi) >> sh


def test_clamp_before_shift_identity():
    """min(max(x >> sh, lo), 127) == clamp_then_shift(x, sh, lo) for every
    int32 x near each clamp boundary and random x, all sh in [0, 31], with
    ReLU (lo = 0) and without (lo = -128)."""
    rng = np.random.default_rng(2)
    rand = [int(v) for v in rng.integers(-2**31, 2**31, 2000)]
    for sh in range(32):
        edges = []
        for b in (128 << sh, -128 << sh, 127 << sh, -127 << sh, 0):
            edges += [b - 2, b - 1, b, b + 1]
        xs = [x for x in edges + rand + [-(2**31), 2**31 - 1] if -(2**31) <= x < 2**31]
        for lo_out in (0, -128):
            for x in xs:
                assert min(max(x >> sh, lo_out), 127) == clamp_then_shift(x, sh, lo_out), (x, sh, lo_out)
