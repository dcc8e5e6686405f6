"""SIG2 archive records and the SIDX index (C++ in libsigcomp_host.so,
include/sigcomp_host.h).

An archive is ``b'SIG2'``, a uint32 length and the header blob, then one
record per read (``main.py:226-246,549-607``).  The header blob (the
zstd-compressed pickle of the global metadata), the BLOW5 per-read metadata
(a pickle) and the two Rice-coded blobs are opaque bytes here: the caller
produces them (the Rice blobs with ``sigcomp_amd.rice.encode_split``; the
reference uses ``numcodecs`` and ``fast-rice``).  The SIDX index is ``b'SIDX'``, a uint32 count and
per read the 16-byte read id and the uint64 record offset
(``main.py:1451-1502``).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _host

MAGIC = b"SIG2"
IDX_MAGIC = b"SIDX"
POD5 = 0
BLOW5 = 1
POD5_PREFIX = 62

# sc_pod5_record (natural C layout; serialized packed as REC_FMT '<16sddBBdIIIQ')
POD5_DTYPE = np.dtype([("read_id", "u1", (16,)), ("calibration_offset", "<f8"), ("calibration_scale", "<f8"),
                       ("end_reason_forced", "u1"), ("end_reason_index", "u1"), ("median_before", "<f8"),
                       ("pore", "<u4"), ("read_number", "<u4"), ("run_info", "<u4"),
                       ("start_sample", "<u8")], align=True)

_ERRORS = {
    20: "Truncated SIG2 read record",
    21: "Invalid sample or token count in SIG2 read record",
    22: "SIG2 read count disagrees with trailing file data",
    23: None,   # message from the library
}

_BOUND = False


def _lib():
    global _BOUND
    L = _host.lib()
    if not _BOUND:
        P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        L.sc_sig2_write_records.argtypes = [I32, I64, P, P, P, P, P, P, P, P, P, P, P, P, P, I32, P]
        L.sc_sig2_scan_records.argtypes = [P, I64, I64, I64, I32, I32, P, P, P, P, P, P, P, P, P, P, P]
        L.sc_sig2_write_index.argtypes = [I64, P, P, P]
        L.sc_sig2_read_index.argtypes = [P, I64, I64, I64, I64, P, P, P]
        for n in ("sc_sig2_write_records", "sc_sig2_scan_records", "sc_sig2_write_index", "sc_sig2_read_index"):
            getattr(L, n).restype = ctypes.c_int
        _BOUND = True
    return L


def _check(rc, bad):
    if rc == 0:
        return
    msg = _ERRORS.get(rc)
    if rc in _ERRORS:
        raise ValueError(f"{msg or _host.lib().sc_host_last_error().decode()} (read {bad.value})")
    _host._check(rc, bad, "read")


def _p(a):
    return a.ctypes.data


def _cat(blobs):
    lens = np.fromiter((len(b) for b in blobs), np.int64, count=len(blobs))
    off = np.zeros(len(blobs), np.int64)
    if len(blobs) > 1:
        np.cumsum(lens[:-1], out=off[1:])
    data = np.frombuffer(b"".join(bytes(b) for b in blobs), np.uint8) if blobs else np.zeros(0, np.uint8)
    return (data if data.size else np.zeros(1, np.uint8)), off, lens


def write_records(fmt, sig0, n_samples, n_small, s_blobs, l_blobs, p_blobs, pod5=None, read_ids=None,
                  metas=None, n_threads: int = 0):
    """Serialize records -> (bytes, record offsets with the end appended).

    POD5: ``pod5`` = array of POD5_DTYPE.  BLOW5: ``read_ids`` (16-byte
    bytes each) and ``metas`` (bytes each).  The three blob lists hold the
    framed small tokens, the Rice-coded large values and positions."""
    n = len(sig0)
    sig0 = np.ascontiguousarray(sig0, np.int16)
    n_samples = np.ascontiguousarray(n_samples, np.uint32)
    n_small = np.ascontiguousarray(n_small, np.uint32)
    if not (len(n_samples) == len(n_small) == len(s_blobs) == len(l_blobs) == len(p_blobs) == n):
        raise ValueError("per-read inputs differ in length")
    blobs = [b for trio in zip(s_blobs, l_blobs, p_blobs) for b in trio]
    bdata, boff, blen = _cat(blobs)
    if fmt == POD5:
        pod5 = np.ascontiguousarray(pod5, POD5_DTYPE)
        if len(pod5) != n:
            raise ValueError("one POD5 record per read")
        prefix = np.full(n, POD5_PREFIX, np.int64)
        ids = mdata = moff = mlen = np.zeros(1, np.int64)
        pod = pod5
    elif fmt == BLOW5:
        if len(read_ids) != n or len(metas) != n or any(len(r) != 16 for r in read_ids):
            raise ValueError("one 16-byte read id and one metadata blob per read")
        ids = np.frombuffer(b"".join(read_ids), np.uint8) if n else np.zeros(16, np.uint8)
        mdata, moff, mlen = _cat(metas)
        prefix = 20 + mlen
        pod = np.zeros(1, POD5_DTYPE)
    else:
        raise ValueError("format must be POD5 or BLOW5")
    sizes = prefix + 10 + 12 + blen.reshape(n, 3).sum(axis=1) if n else np.zeros(0, np.int64)
    bounds = np.zeros(n + 1, np.int64)
    np.cumsum(sizes, out=bounds[1:])
    out = np.empty(max(int(bounds[-1]), 1), np.uint8)
    starts = np.ascontiguousarray(bounds[:-1])
    bad = ctypes.c_int64(-1)
    _check(_lib().sc_sig2_write_records(fmt, n, _p(pod), _p(ids), _p(mdata), _p(moff), _p(mlen), _p(sig0),
                                        _p(n_samples), _p(n_small), _p(bdata), _p(boff), _p(blen), _p(out),
                                        _p(starts), int(n_threads), ctypes.byref(bad)), bad)
    return out[:bounds[-1]].tobytes(), bounds


def scan_records(data, start: int, n_reads: int, fmt: int, require_end: bool = True) -> dict:
    """Parse n_reads records of ``data`` from byte ``start`` (scan_archive,
    archive_shards.py:149-175)."""
    buf = np.frombuffer(data, np.uint8) if len(data) else np.zeros(1, np.uint8)
    size = len(data)
    n = int(n_reads)
    res = {"rec_off": np.zeros(n + 1, np.int64), "read_ids": np.zeros((max(n, 1), 16), np.uint8),
           "sig0": np.zeros(max(n, 1), np.int16), "n_samples": np.zeros(max(n, 1), np.uint32),
           "n_small": np.zeros(max(n, 1), np.uint32), "blob_off": np.zeros((max(n, 1), 3), np.int64),
           "blob_len": np.zeros((max(n, 1), 3), np.int64), "meta_off": np.zeros(max(n, 1), np.int64),
           "meta_len": np.zeros(max(n, 1), np.int64), "pod5": np.zeros(max(n, 1), POD5_DTYPE)}
    bad = ctypes.c_int64(-1)
    _check(_lib().sc_sig2_scan_records(_p(buf), size, int(start), n, int(fmt), int(bool(require_end)),
                                       _p(res["rec_off"]), _p(res["read_ids"]), _p(res["sig0"]),
                                       _p(res["n_samples"]), _p(res["n_small"]), _p(res["blob_off"]),
                                       _p(res["blob_len"]), _p(res["meta_off"]), _p(res["meta_len"]),
                                       _p(res["pod5"]), ctypes.byref(bad)), bad)
    for k in res:
        if k != "rec_off":
            res[k] = res[k][:n]
    res["data"] = buf
    return res


def blob(scan: dict, r: int, k: int) -> bytes:
    """Blob k (0 small tokens, 1 large values, 2 positions) of scanned record r."""
    o, n = scan["blob_off"][r, k], scan["blob_len"][r, k]
    return scan["data"][o:o + n].tobytes()


def header_bytes(header_blob: bytes) -> bytes:
    """MAGIC + uint32 length + the (opaque) header blob (_write_header, main.py:226-233)."""
    return MAGIC + len(header_blob).to_bytes(4, "little") + bytes(header_blob)


def split_header(data: bytes):
    """-> (header blob, offset of the first record) (_read_header, main.py:236-246)."""
    if data[:4] != MAGIC:
        raise ValueError(f"Not a SIGCOMP file (magic={bytes(data[:4])!r}). ")
    if len(data) < 8:
        raise ValueError("Truncated SIG2 header")
    n = int.from_bytes(data[4:8], "little")
    if 8 + n > len(data):
        raise ValueError("Truncated SIG2 header")
    return bytes(data[8:8 + n]), 8 + n


def write_index(read_ids, offsets) -> bytes:
    ids = np.ascontiguousarray(read_ids, np.uint8).reshape(-1, 16)
    offs = np.ascontiguousarray(offsets, np.uint64)
    if len(ids) != len(offs):
        raise ValueError("one offset per read id")
    out = np.empty(8 + 24 * len(ids), np.uint8)
    rc = _lib().sc_sig2_write_index(len(ids), _p(ids if len(ids) else np.zeros(16, np.uint8)),
                                     _p(offs if len(offs) else np.zeros(1, np.uint64)), _p(out))
    _check(rc, ctypes.c_int64(-1))
    return out.tobytes()


def read_index(data: bytes, n_expected: int, data_start: int, file_size: int):
    """-> (read ids [n, 16] uint8, offsets uint64) with the reference's checks."""
    buf = np.frombuffer(data, np.uint8) if len(data) else np.zeros(1, np.uint8)
    n = int(n_expected)
    ids = np.zeros((max(n, 1), 16), np.uint8)
    offs = np.zeros(max(n, 1), np.uint64)
    bad = ctypes.c_int64(-1)
    rc = _lib().sc_sig2_read_index(_p(buf), len(data), n, int(data_start), int(file_size), _p(ids), _p(offs),
                                   ctypes.byref(bad))
    if rc:
        raise ValueError(_host.lib().sc_host_last_error().decode())
    return ids[:n], offs[:n]
