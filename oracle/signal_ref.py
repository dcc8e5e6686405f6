"""Signal transforms around the codec: numpy restatement of the reference,
TEST INFRASTRUCTURE ONLY (the checker for sigcomp_amd.signal, which runs them
in C++ through libsigcomp_host.so).  Imported by tests/ and
tests/golden/make_golden.py only.

Restates ``main.py:129-171`` (delta / zigzag / lossy LSB transforms) and
``main.py:504-546`` (small/large split and reassembly), function by function:

* ``np.diff`` on int16 wraps modulo 2**16; zigzag maps the int16 deltas to
  uint16; values < 256 are the "small" tokens, the rest are "large"
  (stored as ``value - 256``) with gap-coded uint32 positions.
* The lossy path rounds to a multiple of ``2**bit`` and keeps the upper bits.

Pinned by closed forms and invariants in tests/test_host.py (exhaustive int16
zigzag, wrap-around deltas, round trips) and by the reference's own golden
framed reads (tests/golden/e2e_reads.npz).
"""

from __future__ import annotations

import numpy as np


def diff_encode(signal: np.ndarray) -> np.ndarray:
    """``main.py:129-130``."""
    return np.diff(np.asarray(signal, dtype=np.int16)).astype(np.int16)


def diff_decode(sig0: int, deltas: np.ndarray) -> np.ndarray:
    """``main.py:133-137``: int16 prefix sum (wraps modulo 2**16)."""
    signal = np.empty(len(deltas) + 1, dtype=np.int16)
    signal[0] = sig0
    signal[1:] = sig0 + np.cumsum(deltas).astype(np.int16)
    return signal


def zigzag_encode(values: np.ndarray) -> np.ndarray:
    """``main.py:140-142``."""
    v = np.asarray(values).astype(np.int32)
    return ((v << 1) ^ (v >> 31)).astype(np.uint16)


def zigzag_decode(values: np.ndarray) -> np.ndarray:
    """``main.py:145-147``."""
    v = np.asarray(values).astype(np.uint32)
    return ((v >> 1) ^ -(v & 1)).astype(np.int16)


def reduce_lsb(signal: np.ndarray, bit: int) -> np.ndarray:
    """``main.py:158-163``: round half up to a multiple of ``2**bit``."""
    v = np.asarray(signal).astype(np.int32)
    step = 1 << bit
    rounding = ((v >> (bit - 1)) & 1) * step
    upper = v & (~(step - 1))
    return (upper + rounding).astype(np.int16)


def lossy_encode(signal: np.ndarray, bit: int) -> np.ndarray:
    """``main.py:166-167``."""
    return (np.asarray(signal).astype(np.int32) >> bit).astype(np.int16)


def lossy_decode(signal: np.ndarray, bit: int) -> np.ndarray:
    """``main.py:170-171``."""
    return (np.asarray(signal).astype(np.int32) << bit).astype(np.int16)


def prepare_signal(signal: np.ndarray, lsb: int) -> np.ndarray:
    """The compress-side transform applied before splitting (``main.py:862-864``)."""
    signal = np.asarray(signal, dtype=np.int16)
    if lsb > 0:
        signal = lossy_encode(reduce_lsb(signal, lsb), lsb)
    return signal


def split_signal(sig: np.ndarray):
    """``main.py:504-521``: -> (sig0, small uint8 tokens, large-256 uint16, gap-coded uint32 positions)."""
    sig = np.asarray(sig, dtype=np.int16)
    zz = zigzag_encode(diff_encode(sig))
    is_large = zz >= 256
    small_vals = zz[~is_large].astype(np.uint8)
    large_vals = zz[is_large].astype(np.uint16)
    large_pos = np.where(is_large)[0].astype(np.uint32)
    if len(large_pos) > 0:
        large_pos_deltas = np.empty_like(large_pos)
        large_pos_deltas[0] = large_pos[0]
        if len(large_pos) > 1:
            large_pos_deltas[1:] = np.diff(large_pos) - 1
    else:
        large_pos_deltas = np.array([], dtype=np.uint32)
    return int(sig[0]), small_vals, (large_vals - 256).astype(np.uint16), large_pos_deltas


def reassemble_signal(sig0: int, n: int, small_vals, large_adj, large_pos_deltas) -> np.ndarray:
    """``main.py:524-546`` with the Rice-decoded large values and gaps given."""
    large_vals = np.asarray(large_adj, dtype=np.uint16).astype(np.uint16) + np.uint16(256)
    deltas = np.asarray(large_pos_deltas, dtype=np.uint32).copy()
    if len(deltas) > 1:
        deltas[1:] += 1
    large_pos = np.cumsum(deltas).astype(np.int64) if len(deltas) else np.array([], np.int64)
    zz = np.zeros(n - 1, dtype=np.uint16)
    small_mask = np.ones(n - 1, dtype=bool)
    if len(large_pos) > 0:
        idx = large_pos.astype(np.intp)
        zz[idx] = large_vals
        small_mask[idx] = False
    zz[small_mask] = np.asarray(small_vals, dtype=np.uint8)
    return diff_decode(sig0, zigzag_decode(zz))
