"""SIG2 records and the SIDX index (libsigcomp_host.so) against the
reference's struct layouts (main.py:55-62: REC_FMT '<16sddBBdIIIQ',
REC_FMT_BLOW5 '<16s', SPLIT_HDR_FMT '<hII', U32 '<I'; archive_shards.py:22
INDEX_ENTRY '<16sQ'), restated here with the struct module, the reference's
validation rules (archive_shards.py:130-175, main.py:427-444) and a full
read pipeline round trip through an archive."""

import struct

import numpy as np
import pytest

REC = struct.Struct("<16sddBBdIIIQ")
SPLIT = struct.Struct("<hII")
U32 = struct.Struct("<I")
ENTRY = struct.Struct("<16sQ")


def _sig2():
    from sigcomp_amd import _host, sig2
    if not _host.LIB_PATH.exists():
        pytest.skip("libsigcomp_host.so not built")
    return sig2


def _py_record_pod5(rec, sig0, n, ns, s, l, p):
    return (REC.pack(bytes(rec["read_id"]), float(rec["calibration_offset"]), float(rec["calibration_scale"]),
                     int(rec["end_reason_forced"]), int(rec["end_reason_index"]), float(rec["median_before"]),
                     int(rec["pore"]), int(rec["read_number"]), int(rec["run_info"]), int(rec["start_sample"]))
            + SPLIT.pack(sig0, n, ns) + U32.pack(len(s)) + s + U32.pack(len(l)) + l + U32.pack(len(p)) + p)


def _py_record_blow5(rid, meta, sig0, n, ns, s, l, p):
    return (rid + U32.pack(len(meta)) + meta + SPLIT.pack(sig0, n, ns) + U32.pack(len(s)) + s
            + U32.pack(len(l)) + l + U32.pack(len(p)) + p)


def _records(rng, n):
    sig2 = _sig2()
    pod = np.zeros(n, sig2.POD5_DTYPE)
    pod["read_id"] = rng.integers(0, 256, (n, 16))
    pod["calibration_offset"] = rng.normal(size=n) * 100
    pod["calibration_scale"] = rng.random(n)
    pod["end_reason_forced"] = rng.integers(0, 2, n)
    pod["end_reason_index"] = rng.integers(0, 6, n)
    pod["median_before"] = rng.random(n) * 300
    pod["pore"] = rng.integers(0, 2**32, n, dtype=np.uint64)
    pod["read_number"] = rng.integers(0, 2**32, n, dtype=np.uint64)
    pod["run_info"] = rng.integers(0, 8, n)
    pod["start_sample"] = rng.integers(0, 2**63, n, dtype=np.uint64)
    n_samples = rng.integers(1, 5000, n).astype(np.uint32)
    n_small = np.array([rng.integers(0, k) if k > 1 else 0 for k in n_samples], np.uint32)
    sig0 = rng.integers(-32768, 32768, n).astype(np.int16)
    blobs = [[rng.integers(0, 256, rng.integers(0, 40), dtype=np.uint8).tobytes() for _ in range(n)]
             for _ in range(3)]
    return pod, sig0, n_samples, n_small, blobs


def test_pod5_records_match_reference_layout_and_scan_back():
    sig2 = _sig2()
    rng = np.random.default_rng(1)
    pod, sig0, ns, nsm, (s, l, p) = _records(rng, 25)
    data, bounds = sig2.write_records(sig2.POD5, sig0, ns, nsm, s, l, p, pod5=pod)
    exp = b"".join(_py_record_pod5(pod[i], int(sig0[i]), int(ns[i]), int(nsm[i]), s[i], l[i], p[i])
                   for i in range(25))
    assert data == exp
    assert bounds[-1] == len(data)
    sc = sig2.scan_records(data, 0, 25, sig2.POD5)
    assert np.array_equal(sc["rec_off"], bounds)
    assert np.array_equal(sc["sig0"], sig0) and np.array_equal(sc["n_samples"], ns)
    assert np.array_equal(sc["n_small"], nsm) and np.array_equal(sc["read_ids"], pod["read_id"])
    for f in ("calibration_offset", "calibration_scale", "end_reason_forced", "end_reason_index",
              "median_before", "pore", "read_number", "run_info", "start_sample"):
        assert np.array_equal(sc["pod5"][f], pod[f]), f
    for i in range(25):
        assert sig2.blob(sc, i, 0) == s[i] and sig2.blob(sc, i, 1) == l[i] and sig2.blob(sc, i, 2) == p[i]


def test_blow5_records_match_reference_layout_and_scan_back():
    sig2 = _sig2()
    rng = np.random.default_rng(2)
    _, sig0, ns, nsm, (s, l, p) = _records(rng, 9)
    rids = [rng.integers(0, 256, 16, dtype=np.uint8).tobytes() for _ in range(9)]
    metas = [rng.integers(0, 256, rng.integers(0, 30), dtype=np.uint8).tobytes() for _ in range(9)]
    data, bounds = sig2.write_records(sig2.BLOW5, sig0, ns, nsm, s, l, p, read_ids=rids, metas=metas)
    exp = b"".join(_py_record_blow5(rids[i], metas[i], int(sig0[i]), int(ns[i]), int(nsm[i]), s[i], l[i], p[i])
                   for i in range(9))
    assert data == exp
    sc = sig2.scan_records(data, 0, 9, sig2.BLOW5)
    for i in range(9):
        o, n = sc["meta_off"][i], sc["meta_len"][i]
        assert sc["data"][o:o + n].tobytes() == metas[i] and sc["read_ids"][i].tobytes() == rids[i]


def test_scan_rejects_what_the_reference_rejects():
    sig2 = _sig2()
    rng = np.random.default_rng(3)
    pod, sig0, ns, nsm, (s, l, p) = _records(rng, 3)
    data, bounds = sig2.write_records(sig2.POD5, sig0, ns, nsm, s, l, p, pod5=pod)
    for cut in (1, 61, 62 + 5, int(bounds[1]) - 1, len(data) - 1):
        with pytest.raises(ValueError, match="Truncated"):
            sig2.scan_records(data[:cut], 0, 3, sig2.POD5)
    with pytest.raises(ValueError, match="trailing"):
        sig2.scan_records(data + b"\0", 0, 3, sig2.POD5)
    assert sig2.scan_records(data + b"\0", 0, 3, sig2.POD5, require_end=False)["rec_off"][-1] == len(data)
    bad = bytearray(data)
    bad[62 + 2:62 + 6] = U32.pack(0)                   # N = 0
    with pytest.raises(ValueError, match="sample or token count"):
        sig2.scan_records(bytes(bad), 0, 3, sig2.POD5)
    bad = bytearray(data)
    bad[62 + 6:62 + 10] = U32.pack(int(ns[0]))          # small tokens > N - 1
    with pytest.raises(ValueError, match="sample or token count"):
        sig2.scan_records(bytes(bad), 0, 3, sig2.POD5)
    with pytest.raises(ValueError, match="sample or token count"):
        sig2.write_records(sig2.POD5, sig0, np.zeros(3, np.uint32), nsm, s, l, p, pod5=pod)


def test_index_layout_and_checks():
    sig2 = _sig2()
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 256, (7, 16), dtype=np.uint8)
    offs = np.sort(rng.integers(100, 10**6, 7)).astype(np.uint64)
    idx = sig2.write_index(ids, offs)
    assert idx == b"SIDX" + U32.pack(7) + b"".join(ENTRY.pack(ids[i].tobytes(), int(offs[i])) for i in range(7))
    got_ids, got_offs = sig2.read_index(idx, 7, 100, 10**6)
    assert np.array_equal(got_ids, ids) and np.array_equal(got_offs, offs)
    with pytest.raises(ValueError, match="Not a valid SIDX"):
        sig2.read_index(b"SIDY" + idx[4:], 7, 100, 10**6)
    with pytest.raises(ValueError, match="count/size"):
        sig2.read_index(idx, 6, 100, 10**6)
    with pytest.raises(ValueError, match="count/size"):
        sig2.read_index(idx[:-1], 7, 100, 10**6)
    with pytest.raises(ValueError, match="outside archive records"):
        sig2.read_index(idx, 7, 100, int(offs[-1]))
    assert sig2.write_index(np.zeros((0, 16), np.uint8), np.zeros(0, np.uint64)) == b"SIDX" + U32.pack(0)


def test_archive_round_trip_through_the_read_pipeline(oracle_mod, oracle_models):
    """synthetic reads -> split -> framed range-coded tokens (the C oracle
    codec through the batched framing path) -> records -> archive bytes ->
    header + scan + index -> parse -> decode -> reassembly == the reads.
    The large values and gaps are Rice-coded by sigcomp_amd.rice (this
    library's own blob format: fast-rice 0.1.0's is third-party)."""
    sig2 = _sig2()
    from test_host import _OracleCodec
    from sigcomp_amd import rice, signal, synth
    from sigcomp_amd.framing import ReadFramingMixin

    class Codec(_OracleCodec, ReadFramingMixin):
        pass

    codec = Codec(oracle_mod, oracle_models["lossless"], chunk_len=512)
    reads = synth.synth_reads(5, 77, synth.DNA, lengths=[1, 300, 1200, 90, 2000])
    sp = signal.split_reads(reads)
    small = signal.reads_tokens(sp)
    s_bytes = codec.batch_inference_reads(list_of_reads=small)
    la, lg = rice.encode_split(sp)
    pod = np.zeros(len(reads), sig2.POD5_DTYPE)
    pod["read_id"] = np.arange(len(reads))[:, None] + np.arange(16)[None, :]
    recs, bounds = sig2.write_records(sig2.POD5, sp["sig0"], sp["len"], sp["n_small"], s_bytes, la, lg, pod5=pod)
    archive = sig2.header_bytes(b"opaque header blob") + recs
    hdr, start = sig2.split_header(archive)
    assert hdr == b"opaque header blob"
    sc = sig2.scan_records(archive, start, len(reads), sig2.POD5)
    idx = sig2.write_index(sc["read_ids"], sc["rec_off"][:-1].astype(np.uint64))
    ids, offs = sig2.read_index(idx, len(reads), start, len(archive))
    assert np.array_equal(offs, start + bounds[:-1])
    # random access through the index: read 3 alone
    one = sig2.scan_records(archive, int(offs[3]), 1, sig2.POD5, require_end=False)
    assert one["n_samples"][0] == len(reads[3])
    back = codec.batch_inference_reads(list_of_compressed_reads=[sig2.blob(sc, i, 0) for i in range(len(reads))],
                                       list_of_lengths=[int(x) for x in sc["n_small"]])
    # c_large = N - 1 - c_small (main.py:562)
    n_large = sc["n_samples"].astype(np.int64) - 1 - sc["n_small"].astype(np.int64)
    assert np.array_equal(n_large, sp["n_large"])
    large_adj, large_gap, large_off = rice.decode_split([sig2.blob(sc, i, 1) for i in range(len(reads))],
                                                        [sig2.blob(sc, i, 2) for i in range(len(reads))], n_large)
    split = {"sig0": sc["sig0"], "len": sc["n_samples"].astype(np.int64), "small_off": sp["small_off"],
             "n_small": sc["n_small"].astype(np.int64), "large_adj": large_adj, "large_gap": large_gap,
             "large_off": large_off, "n_large": n_large}
    out = signal.reassemble_reads(split, small=np.concatenate(back))
    assert all(np.array_equal(a, b) for a, b in zip(reads, out))


def test_host_library_exports_the_record_functions():
    import ctypes
    import re
    from conftest import REPO
    _sig2()
    from sigcomp_amd import _host
    text = re.sub(r"/\*.*?\*/", "", (REPO / "include" / "sigcomp_host.h").read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(sc_sig2_[a-z0-9_]+)\s*\(", text)))
    assert len(names) == 4
    lib = ctypes.CDLL(str(_host.LIB_PATH))
    assert [n for n in names if not hasattr(lib, n)] == []
