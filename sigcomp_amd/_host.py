"""ctypes binding of libsigcomp_host.so (include/sigcomp_host.h): signal
split / reassembly and SIG2 chunk framing on the host, multithreaded.

The library is built by ``sigcomp_amd.build`` (``__graft_entry__.build()``);
a missing library raises ``HostError``.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libsigcomp_host.so"

SC_OK = 0
SC_ERR_ARG = 1
ERR_FRAME_LENGTH = 10
ERR_FRAME = 11
ERR_TRAILING = 12
ERR_OVERSIZE = 13
ERR_COUNTS = 14
ERR_POSITION = 15
ERR_EMPTY_READ = 16
ERR_RICE = 24
ERR_RICE_RANGE = 25

EXPORTED = ("sc_host_last_error", "sc_host_split_count", "sc_host_split_fill", "sc_host_reassemble",
            "sc_host_frame", "sc_host_parse", "sc_host_parse_v", "sc_rice_bound", "sc_rice_encode",
            "sc_rice_decode")

# the exception type the reference raises for each failure
_MESSAGES = {
    ERR_FRAME_LENGTH: (ValueError, "Truncated SIG2 chunk length"),
    ERR_FRAME: (ValueError, "Invalid or truncated SIG2 range-coded chunk"),
    ERR_TRAILING: (ValueError, "Trailing SIG2 chunk data disagrees with token length"),
    ERR_OVERSIZE: (ValueError, "Compressed chunk exceeds the SIG2 uint16 frame; compress with a smaller "
                               "--chunk-len"),
    ERR_COUNTS: (ValueError, "small and large value counts disagree with the read length"),
    ERR_POSITION: (IndexError, "large-value position outside the read"),
    ERR_EMPTY_READ: (IndexError, "a read has no samples"),
    ERR_RICE: (ValueError, "Invalid or truncated Rice-coded blob"),
    ERR_RICE_RANGE: (ValueError, "value does not fit the Rice fallback width"),
}


class HostError(RuntimeError):
    pass


_LIB = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise HostError(f"{LIB_PATH} is missing; build it with `python -m sigcomp_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        L.sc_host_last_error.restype = ctypes.c_char_p
        L.sc_host_split_count.argtypes = [_P, _P, _I64, _I32, _P, _P, _P, _I32, _P]
        L.sc_host_split_fill.argtypes = [_P, _P, _I64, _I32, _P, _P, _P, _P, _P, _I32, _P]
        L.sc_host_reassemble.argtypes = [_P, _P, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _P]
        L.sc_host_frame.argtypes = [_P, _P, _P, _I64, _P, _P, _I32, _P]
        L.sc_host_parse.argtypes = [_P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P, _P, _I32, _P]
        L.sc_host_parse_v.argtypes = [_P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P, _P, _I32, _P]
        L.sc_rice_bound.argtypes = [_I64, _I32, _I32]
        L.sc_rice_encode.argtypes = [_P, _P, _P, _I64, _I32, _I32, _P, _P, _P, _I32, _P]
        L.sc_rice_decode.argtypes = [_P, _P, _P, _I64, _I32, _I32, _P, _P, _I32, _P]
        for name in EXPORTED[1:]:
            getattr(L, name).restype = ctypes.c_int
        L.sc_rice_bound.restype = ctypes.c_int64
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    # numpy gives even an empty array a valid (non-NULL) buffer.  The caller
    # must keep `a` referenced until the C call returns (never pass a
    # temporary: it is freed as soon as this returns)
    return a.ctypes.data


def _check(rc: int, bad: ctypes.c_int64, what: str = "item") -> None:
    if rc == SC_OK:
        return
    if rc in _MESSAGES:
        exc, msg = _MESSAGES[rc]
        raise exc(f"{msg} ({what} {bad.value})")
    raise HostError(lib().sc_host_last_error().decode(errors="replace") or f"host library error {rc}")


def _excl_scan(counts: np.ndarray) -> np.ndarray:
    off = np.zeros(len(counts), np.int64)
    if len(counts) > 1:
        np.cumsum(counts[:-1], out=off[1:])
    return off


def read_pointers(reads):
    """-> (kept int16 arrays, uint64 array of their data pointers, int64 lengths); no copy
    for reads that already are contiguous int16 arrays."""
    kept = [np.ascontiguousarray(r, np.int16) for r in reads]
    ptrs = np.fromiter((a.ctypes.data for a in kept), np.uint64, count=len(kept))
    lens = np.fromiter((len(a) for a in kept), np.int64, count=len(kept))
    return kept, ptrs, lens


def split(reads, lsb: int = 0, n_threads: int = 0) -> dict:
    """Split a list of int16 reads (see sc_host_split_count / _fill)."""
    kept, ptrs, lens = read_pointers(reads)
    n = len(lens)
    sig0 = np.zeros(n, np.int16)
    n_small = np.zeros(n, np.int64)
    n_large = np.zeros(n, np.int64)
    bad = ctypes.c_int64(-1)
    L = lib()
    _check(L.sc_host_split_count(_p(ptrs), _p(lens), n, int(lsb), _p(sig0), _p(n_small), _p(n_large),
                                 int(n_threads), ctypes.byref(bad)), bad, "read")
    small_off, large_off = _excl_scan(n_small), _excl_scan(n_large)
    small = np.empty(int(n_small.sum()), np.uint8)
    large_adj = np.empty(int(n_large.sum()), np.uint16)
    large_gap = np.empty(int(n_large.sum()), np.uint32)
    _check(L.sc_host_split_fill(_p(ptrs), _p(lens), n, int(lsb), _p(small_off), _p(large_off),
                                _p(small), _p(large_adj), _p(large_gap), int(n_threads), ctypes.byref(bad)),
           bad, "read")
    del kept
    return {"sig0": sig0, "len": lens, "small": small, "small_off": small_off, "n_small": n_small,
            "large_adj": large_adj, "large_gap": large_gap, "large_off": large_off, "n_large": n_large}


def reassemble(sig0, lens, small, small_off, n_small, large_adj, large_gap, large_off, n_large, lsb: int = 0,
               n_threads: int = 0):
    """Inverse of ``split`` -> (int16 samples concatenated, offsets)."""
    sig0 = np.ascontiguousarray(sig0, np.int16)
    lens = np.ascontiguousarray(lens, np.int64)
    small = np.ascontiguousarray(small, np.uint8)
    small_off = np.ascontiguousarray(small_off, np.int64)
    n_small = np.ascontiguousarray(n_small, np.int64)
    large_adj = np.ascontiguousarray(large_adj, np.uint16)
    large_gap = np.ascontiguousarray(large_gap, np.uint32)
    large_off = np.ascontiguousarray(large_off, np.int64)
    n_large = np.ascontiguousarray(n_large, np.int64)
    n = len(lens)
    if len(sig0) != n or len(small_off) != n or len(n_small) != n or len(large_off) != n or len(n_large) != n:
        raise ValueError("per-read arrays must have one entry per read")
    if n and (np.any(small_off < 0) or np.any(small_off + n_small > len(small)) or np.any(large_off < 0)
              or np.any(large_off + n_large > min(len(large_adj), len(large_gap)))):
        raise ValueError("per-read ranges exceed the value arrays")
    out_off = _excl_scan(lens)
    out = np.empty(int(lens.sum()), np.int16)
    bad = ctypes.c_int64(-1)
    _check(lib().sc_host_reassemble(_p(sig0), _p(lens), n, int(lsb), _p(small), _p(small_off), _p(n_small),
                                    _p(large_adj), _p(large_gap), _p(large_off), _p(n_large), _p(out),
                                    _p(out_off), int(n_threads), ctypes.byref(bad)), bad, "read")
    return out, out_off


def frame(words: np.ndarray, word_off: np.ndarray, word_cnt: np.ndarray, n_threads: int = 0):
    """Frame chunks -> (bytes buffer, per-chunk frame offsets incl. the end)."""
    words = np.ascontiguousarray(words, np.uint32)
    word_off = np.ascontiguousarray(word_off, np.int64)
    word_cnt = np.ascontiguousarray(word_cnt, np.int32)
    n = len(word_cnt)
    if n and (np.any(word_off < 0) or np.any(word_cnt < 0) or np.any(word_off + word_cnt > len(words))):
        raise ValueError("chunk word ranges exceed the word array")
    sizes = 2 + 4 * word_cnt.astype(np.int64)
    bounds = np.zeros(n + 1, np.int64)
    np.cumsum(sizes, out=bounds[1:])
    out = np.empty(int(bounds[-1]), np.uint8)
    bad = ctypes.c_int64(-1)
    starts = np.ascontiguousarray(bounds[:-1])      # kept alive across the call
    _check(lib().sc_host_frame(_p(words), _p(word_off), _p(word_cnt), n, _p(out), _p(starts),
                               int(n_threads), ctypes.byref(bad)), bad, "chunk")
    return out, bounds


def parse_word_count(payloads) -> int:
    """Words parse() writes for these payloads (its words_out size)."""
    return int(sum(len(p) // 4 for p in payloads))


def parse(payloads, tokens, chunk_len: int, n_threads: int = 0, words_out=None) -> dict:
    """Parse framed per-read payloads (list of bytes) with their token counts.
    words_out: optional uint32 array of at least parse_word_count(payloads)
    elements (e.g. pinned memory for the device copy) to hold the words."""
    n = len(payloads)
    tokens = np.asarray(tokens, np.int64).reshape(-1)
    if len(tokens) != n:
        raise ValueError("Compressed read and token length counts differ")
    if n and int(tokens.min()) < 0:
        raise ValueError("token counts must be non-negative")
    if int(chunk_len) < 1:
        raise ValueError("chunk_len must be positive")
    data_len = np.fromiter((len(p) for p in payloads), np.int64, count=n)
    # each payload's own buffer, no joined copy: bytes objects through
    # c_char_p (their internal buffer), anything else as a uint8 view
    views = []

    def addr(p):
        if type(p) is bytes:
            return ctypes.cast(ctypes.c_char_p(p), ctypes.c_void_p).value or 0
        a = np.frombuffer(p, np.uint8)
        views.append(a)
        return a.ctypes.data

    payload_ptr = np.fromiter((addr(p) for p in payloads), np.uint64, count=n) if n else np.zeros(1, np.uint64)
    frames = (tokens + chunk_len - 1) // chunk_len
    chunk_begin = _excl_scan(frames)
    n_chunks = int(frames.sum())
    read_word_off = _excl_scan(data_len // 4)
    n_words = max(int((data_len // 4).sum()), 1)
    if words_out is not None:
        if words_out.dtype != np.uint32 or words_out.ndim != 1 or len(words_out) < n_words \
                or not words_out.flags.c_contiguous:
            raise ValueError("words_out must be a contiguous uint32 array of the parse's word count")
        words = words_out[:n_words]
    else:
        words = np.empty(n_words, np.uint32)
    word_off = np.zeros(n_chunks, np.int64)
    word_cnt = np.zeros(n_chunks, np.int32)
    tok_cnt = np.zeros(n_chunks, np.int32)
    bad = ctypes.c_int64(-1)
    _check(lib().sc_host_parse_v(_p(payload_ptr), _p(data_len), _p(tokens), n, int(chunk_len),
                                 _p(chunk_begin), _p(read_word_off), _p(words), _p(word_off), _p(word_cnt),
                                 _p(tok_cnt), int(n_threads), ctypes.byref(bad)), bad, "read")
    del views, payload_ptr   # (the payloads themselves are the caller's)
    return {"words": words, "word_off": word_off, "word_cnt": word_cnt, "tok_cnt": tok_cnt,
            "chunk_begin": chunk_begin, "frames": frames}
