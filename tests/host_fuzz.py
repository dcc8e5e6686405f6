"""Seeded mutation fuzz of libsigcomp_host.so's entry points that take
untrusted bytes or counts: chunk payload parsing (sc_host_parse_v), Rice
decoding (sc_rice_decode), reassembly from side streams (sc_host_reassemble),
SIG2 record scanning (sc_sig2_scan_records) and the SIG2 index
(sc_sig2_read_index).

Each case starts from a valid encoding written by the library itself, then
corrupts bytes, truncates, inserts, or swaps a count.  The only allowed
outcomes are a result or the documented exception types; the memory safety
of the C++ is what the run under AddressSanitizer / UBSan checks
(tests/test_host_sanitized.py runs this file in a child process with the
sanitizer runtimes preloaded and a sanitized build of the library).  The raw
C-ABI cases pass argument arrays whose bad entries would, unchecked, index
outside the caller's buffers; each such buffer is a slice of a larger array
whose guard elements must stay untouched.

Usage: python tests/host_fuzz.py [--lib PATH] [--seed S] [--iters N]
"""

from __future__ import annotations

import argparse
import ctypes
import random
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[1]


def _modules(lib_path=None):
    if str(REPO) not in sys.path:
        sys.path.insert(0, str(REPO))
    from sigcomp_amd import _host, rice, sig2
    if lib_path is not None:
        if _host._LIB is not None and Path(lib_path) != _host.LIB_PATH:
            raise RuntimeError("the host library is already loaded from another path")
        _host.LIB_PATH = Path(lib_path)
    return _host, rice, sig2


def _mutate(rng: random.Random, b: bytes) -> bytes:
    b = bytearray(b)
    for _ in range(rng.randint(1, 4)):
        op = rng.randint(0, 3)
        if op == 0 and b:
            b[rng.randrange(len(b))] = rng.randrange(256)
        elif op == 1 and b:
            del b[rng.randrange(len(b)):]
        elif op == 2:
            i = rng.randint(0, len(b))
            b[i:i] = bytes(rng.randrange(256) for _ in range(rng.randint(1, 8)))
        elif op == 3 and len(b) > 2:
            i = rng.randrange(len(b) - 1)
            b[i] = b[i + 1] = 0xFF
    return bytes(b)


def _raw_abi_cases(_host) -> None:
    """Entry points called directly with counts that the Python wrappers
    refuse: each must fail with nothing written."""
    L = _host.lib()
    P = _host._p
    # parse: a negative token count, whose chunk_begin layout would make the
    # next read's first chunk index -1
    guard = np.full(4, -7, np.int64)
    word_off = guard[1:]
    wc_g, tc_g = np.full(4, -7, np.int32), np.full(4, -7, np.int32)
    pay = np.zeros(16, np.uint8)
    pay[0] = 4      # one 4-byte chunk of read 1
    ptrs = np.array([pay.ctypes.data, pay.ctypes.data], np.uint64)
    lens = np.array([0, 6], np.int64)
    toks = np.array([-4, 4], np.int64)
    cb = np.array([0, -1], np.int64)
    rwo = np.array([0, 0], np.int64)
    words = np.zeros(4, np.uint32)
    bad = ctypes.c_int64(-1)
    rc = L.sc_host_parse_v(P(ptrs), P(lens), P(toks), 2, 4, P(cb), P(rwo), P(words), P(word_off),
                           P(wc_g[1:]), P(tc_g[1:]), 1, ctypes.byref(bad))
    assert rc == _host.SC_ERR_ARG and bad.value == 0, (rc, bad.value)
    assert (guard == -7).all() and (wc_g == -7).all() and (tc_g == -7).all()
    # reassemble: a negative length, whose out_off prefix sum would make the
    # next read start one sample before `out`
    out_g = np.full(8, 1234, np.int16)
    sig0 = np.array([5, 6], np.int16)
    rl = np.array([-1, 3], np.int64)
    small = np.zeros(4, np.uint8)
    soff = np.array([0, 0], np.int64)
    ns = np.array([0, 2], np.int64)
    la, lg = np.zeros(1, np.uint16), np.zeros(1, np.uint32)
    loff, nl = np.zeros(2, np.int64), np.zeros(2, np.int64)
    ooff = np.array([0, -1], np.int64)
    bad = ctypes.c_int64(-1)
    rc = L.sc_host_reassemble(P(sig0), P(rl), 2, 0, P(small), P(soff), P(ns), P(la), P(lg), P(loff), P(nl),
                              P(out_g[1:]), P(ooff), 1, ctypes.byref(bad))
    assert rc == _host.ERR_EMPTY_READ and bad.value == 0, (rc, bad.value)
    assert (out_g == 1234).all()


def run(seed: int = 0, iters: int = 600, lib_path=None) -> dict:
    _host, rice, sig2 = _modules(lib_path)
    rng = random.Random(seed)
    allowed = (ValueError, IndexError, OverflowError, _host.HostError)
    stats: dict = {}

    def attempt(name, f):
        try:
            f()
            stats[name + "_ok"] = stats.get(name + "_ok", 0) + 1
        except allowed:
            stats[name + "_err"] = stats.get(name + "_err", 0) + 1

    _raw_abi_cases(_host)

    for _ in range(iters):      # framed chunk payloads
        n, cl = rng.randint(1, 4), rng.choice([1, 3, 8, 4096])
        tokens = [rng.randint(0, 3 * cl) for _ in range(n)]
        pays = []
        for t in tokens:
            p = b""
            for _c in range(-(-t // cl)):
                w = rng.randint(1, 5)
                p += (4 * w).to_bytes(2, "little") + bytes(rng.randrange(256) for _ in range(4 * w))
            pays.append(p)
        if rng.random() < 0.7:
            i = rng.randrange(n)
            pays[i] = _mutate(rng, pays[i])
        if rng.random() < 0.3:
            i = rng.randrange(n)
            tokens[i] = rng.choice([-1, -cl, tokens[i] + 1, tokens[i] - 1, 1 << 20])
        attempt("parse", lambda: _host.parse(pays, tokens, cl, n_threads=rng.randint(1, 3)))

    for _ in range(iters):      # Rice blobs
        fb, n = rng.choice([16, 32]), rng.randint(0, 40)
        vals = np.array([rng.randrange(1 << rng.choice([1, 4, 9, fb])) for _ in range(n)], np.uint32)
        blob, cnt = rice.rice_encode(vals, fb), n
        if rng.random() < 0.8:
            blob = _mutate(rng, blob)
        if rng.random() < 0.3:
            cnt = rng.choice([n + 1, max(n - 1, 0), 10 ** 6, 0])
        attempt("rice", lambda: rice.decode_many([blob], [cnt], fb, n_threads=1))

    for _ in range(iters):      # side streams of split reads
        n, lsb = rng.randint(1, 3), rng.choice([0, 0, 3])
        reads = [np.array([rng.randrange(-32768, 32768) if rng.random() < 0.1 else rng.randrange(-50, 50)
                           for _ in range(rng.randint(1, 60))], np.int16) for _ in range(n)]
        s = _host.split(reads, lsb)
        a = {k: s[k].copy() for k in ("sig0", "small", "small_off", "n_small", "large_adj", "large_gap",
                                      "large_off", "n_large")}
        a["lens"] = np.array([len(r) for r in reads], np.int64)
        key = rng.choice(["lens", "n_small", "n_large", "large_gap", "small_off", "large_off"])
        if len(a[key]):
            i = rng.randrange(len(a[key]))
            a[key][i] = rng.choice([0, 1, 7, 100, 2 ** 31 - 1]) if a[key].dtype.kind == "u" \
                else rng.choice([-1, 0, 1, 7, 100, 10 ** 9])
        attempt("reassemble", lambda: _host.reassemble(a["sig0"], a["lens"], a["small"], a["small_off"],
                                                       a["n_small"], a["large_adj"], a["large_gap"],
                                                       a["large_off"], a["n_large"], lsb=lsb))

    for _ in range(iters):      # SIG2 read records
        fmt, n = rng.choice([sig2.POD5, sig2.BLOW5]), rng.randint(0, 3)

        def blob_():
            return bytes(rng.randrange(256) for _ in range(rng.randint(0, 12)))
        ns = [rng.randint(1, 50) for _ in range(n)]
        kw = ({"pod5": np.zeros(n, sig2.POD5_DTYPE)} if fmt == sig2.POD5
              else {"read_ids": [bytes(16)] * n, "metas": [blob_() for _ in range(n)]})
        data, _ = sig2.write_records(fmt, np.zeros(n, np.int16), ns, [x - 1 for x in ns],
                                     [blob_() for _ in range(n)], [blob_() for _ in range(n)],
                                     [blob_() for _ in range(n)], **kw)
        start = rng.randint(0, 3)
        data = bytes(start) + data
        if rng.random() < 0.8:
            data = _mutate(rng, data)
        nn = n if rng.random() < 0.7 else rng.randint(0, 5)
        attempt("scan", lambda: sig2.scan_records(data, start, nn, fmt, require_end=rng.random() < 0.5))

    for _ in range(iters):      # SIG2 index tables
        n = rng.randint(0, 4)
        offs = np.array(sorted(rng.randrange(8, 200) for _ in range(n)), np.uint64)
        idx = sig2.write_index(np.zeros((n, 16), np.uint8), offs)
        if rng.random() < 0.8:
            idx = _mutate(rng, idx)
        nn = n if rng.random() < 0.7 else rng.randint(0, 6)
        attempt("index", lambda: sig2.read_index(idx, nn, rng.randint(0, 10), rng.randint(0, 300)))
    return stats


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib", default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--iters", type=int, default=600)
    args = ap.parse_args()
    print(run(args.seed, args.iters, args.lib), flush=True)
