"""Rice coding of the large deltas and their gap-coded positions (host C++,
``sc_rice_*`` in libsigcomp_host.so, include/sigcomp_host.h).

The reference Rice-codes the two side streams of ``_split_signal`` with the
third-party ``fast-rice==0.1.0`` package through ``_rice_compress`` /
``_rice_decompress`` (``main.py:174-186``): the large values minus 256 with
``fallback_bits=16`` and the gap-coded positions with ``fallback_bits=32``
(``main.py:884-885``, decoded at ``main.py:527-529``), ``max_quotient=31``.
That package's byte format is not available here, so the blobs written by
this module use the library's own format (the header of sigcomp_host.h
specifies it): they round-trip exactly, but are not byte-identical with the
reference's.  The empty case is the reference's own: one zero byte
(``main.py:176-177``), and a count of 0 decodes to an empty array without
reading the blob (``main.py:184-185``); the record count of large values is ``N - 1 - c_small`` (``main.py:562``).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _host

LARGE_FALLBACK_BITS = 16    # main.py:884
POS_FALLBACK_BITS = 32      # main.py:885
MAX_QUOTIENT = 31           # main.py:175,183


def _u32(vals) -> np.ndarray:
    a = np.asarray(vals)
    if a.ndim != 1:
        raise ValueError("Rice coding takes a 1-D array")
    if a.size and a.dtype.kind == "i" and int(a.min()) < 0:
        raise ValueError("Rice coding takes non-negative values")
    if a.size and int(a.max()) > 0xFFFFFFFF:
        raise ValueError("value does not fit the Rice fallback width")
    return np.ascontiguousarray(a, np.uint32)


def encode_many(arrays, fallback_bits: int = 32, max_quotient: int = MAX_QUOTIENT,
                n_threads: int = 0) -> list:
    """Rice blobs of several arrays (one thread per array, up to n_threads)."""
    arrs = [_u32(a) for a in arrays]
    n = len(arrs)
    counts = np.fromiter((len(a) for a in arrs), np.int64, count=n)
    off = _host._excl_scan(counts)
    vals = np.concatenate(arrs) if n and counts.sum() else np.zeros(1, np.uint32)
    L = _host.lib()
    caps = np.fromiter((L.sc_rice_bound(int(c), int(fallback_bits), int(max_quotient)) for c in counts), np.int64,
                       count=n)
    out_off = _host._excl_scan(caps)
    out = np.empty(max(int(caps.sum()), 1), np.uint8)
    out_len = np.zeros(max(n, 1), np.int64)
    bad = ctypes.c_int64(-1)
    _host._check(L.sc_rice_encode(_host._p(vals), _host._p(off), _host._p(counts), n, int(fallback_bits),
                                  int(max_quotient), _host._p(out), _host._p(out_off), _host._p(out_len),
                                  int(n_threads), ctypes.byref(bad)), bad, "array")
    return [out[o:o + int(m)].tobytes() for o, m in zip(out_off, out_len[:n])]


def decode_many(blobs, counts, fallback_bits: int = 32, max_quotient: int = MAX_QUOTIENT,
                n_threads: int = 0) -> list:
    """Inverse of encode_many: blob i holds counts[i] values -> uint32 arrays."""
    n = len(blobs)
    counts = np.ascontiguousarray(counts, np.int64)
    if len(counts) != n:
        raise ValueError("one count per blob")
    if n and int(counts.min()) < 0:
        raise ValueError("Rice value counts must be non-negative")
    kept = [np.frombuffer(bytes(b), np.uint8) if len(b) else np.zeros(1, np.uint8) for b in blobs]
    ptrs = np.fromiter((a.ctypes.data for a in kept), np.uint64, count=n)
    lens = np.fromiter((len(b) for b in blobs), np.int64, count=n)
    out_off = _host._excl_scan(counts)
    out = np.empty(max(int(counts.sum()), 1), np.uint32)
    bad = ctypes.c_int64(-1)
    _host._check(_host.lib().sc_rice_decode(_host._p(ptrs), _host._p(lens), _host._p(counts), n, int(fallback_bits),
                                            int(max_quotient), _host._p(out), _host._p(out_off), int(n_threads),
                                            ctypes.byref(bad)), bad, "blob")
    return [out[o:o + int(c)] for o, c in zip(out_off, counts)]


def rice_encode(vals, fallback_bits: int = 32, max_quotient: int = MAX_QUOTIENT) -> bytes:
    """One array -> its blob (the role of ``fast_rice.rice_encode``)."""
    return encode_many([vals], fallback_bits, max_quotient, n_threads=1)[0]


def rice_decode(buf, count: int, fallback_bits: int = 32, max_quotient: int = MAX_QUOTIENT) -> np.ndarray:
    """Blob of ``count`` values -> uint32 array (the role of ``fast_rice.rice_decode``)."""
    return decode_many([buf], [int(count)], fallback_bits, max_quotient, n_threads=1)[0]


def rice_compress(vals, fallback_bits: int = 32, max_quotient: int = MAX_QUOTIENT) -> bytes:
    """``_rice_compress`` (main.py:174-179)."""
    return rice_encode(vals, fallback_bits, max_quotient)


def rice_decompress(buf, count: int, fallback_bits: int = 32, max_quotient: int = MAX_QUOTIENT) -> np.ndarray:
    """``_rice_decompress`` (main.py:182-186)."""
    if count == 0:
        return np.array([], dtype=np.uint32)
    return rice_decode(buf, count, fallback_bits, max_quotient)


def encode_split(split: dict, n_threads: int = 0):
    """The two Rice blobs of every read of a ``signal.split_reads`` result:
    -> (large-value blobs, position blobs), as main.py:884-885 writes them."""
    la, lg, o, n = split["large_adj"], split["large_gap"], split["large_off"], split["n_large"]
    l_blobs = encode_many([la[a:a + c] for a, c in zip(o, n)], LARGE_FALLBACK_BITS, n_threads=n_threads)
    p_blobs = encode_many([lg[a:a + c] for a, c in zip(o, n)], POS_FALLBACK_BITS, n_threads=n_threads)
    return l_blobs, p_blobs


def decode_split(l_blobs, p_blobs, n_large, n_threads: int = 0):
    """Inverse of encode_split -> (large_adj uint16, large_gap uint32, large_off)
    concatenated in read order, the fields ``signal.reassemble_reads`` takes."""
    n_large = np.ascontiguousarray(n_large, np.int64)
    la = decode_many(l_blobs, n_large, LARGE_FALLBACK_BITS, n_threads=n_threads)
    lg = decode_many(p_blobs, n_large, POS_FALLBACK_BITS, n_threads=n_threads)
    cat = lambda xs, dt: np.concatenate(xs).astype(dt) if len(xs) and n_large.sum() else np.zeros(0, dt)
    return cat(la, np.uint16), cat(lg, np.uint32), _host._excl_scan(n_large)
