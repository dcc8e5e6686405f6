"""Rice coder of the large deltas and positions (sigcomp_amd.rice ->
sc_rice_* in libsigcomp_host.so).

The reference's blobs come from the third-party ``fast-rice==0.1.0``
(main.py:174-186), absent here: the byte format is this library's own
(include/sigcomp_host.h), so parity with the reference's Rice blobs is
unpinned.  What is pinned: the reference's own empty case (one zero byte,
main.py:176-177; count 0 decodes to an empty array, main.py:184-185), exact
round trips over the value ranges the call sites give it (uint16 large
values with fallback 16, uint32 gaps with fallback 32, main.py:884-885),
hand-computed blobs of the documented format, the size-optimal parameter
(brute force over every k), and strict rejection of malformed blobs.
"""

import numpy as np
import pytest

from sigcomp_amd import rice


def _bits(v, k, fb, mq):
    q = v.astype(np.uint64) >> np.uint64(k)
    return int(np.where(q < mq, q + 1 + k, mq + fb).sum())


def test_empty_is_one_zero_byte():
    assert rice.rice_compress(np.zeros(0, np.uint16), 16) == b"\x00"
    assert rice.rice_compress(np.zeros(0, np.uint32), 32) == b"\x00"
    out = rice.rice_decompress(b"not read at all", 0, 32)
    assert out.dtype == np.uint32 and out.size == 0


@pytest.mark.parametrize("vals, fb, blob", [
    # [0]: k = 0, bits '0' -> 0x00
    ([0], 16, bytes([0, 0x00])),
    # [5]: sizes k=0..3 are 6, 4, 4, 4 bits -> k = 1; q = 2: '1','1','0', low bit '1' -> 0b1011
    ([5], 16, bytes([1, 0x0B])),
    # [1, 1, 1]: k = 0 (2 bits each): '1','0' x 3 -> 0b010101
    ([1, 1, 1], 16, bytes([0, 0x15])),
    # [65535]: k = 11 (q = 31 -> escape: 31 ones then 16 bits) costs 47 bits;
    # k = 12..15 costs 15+1+12 = 28 .. 1+1+15 = 17; k = 16: q = 0 -> 17 bits;
    # smallest among the minima: k = 15 (q = 1: '1','0', then 15 low bits)
    ([65535], 16, bytes([15]) + (0b01 | (0x7FFF << 2)).to_bytes(3, "little")),
])
def test_known_blobs(vals, fb, blob):
    v = np.array(vals, np.uint32)
    assert rice.rice_encode(v, fb) == blob
    assert np.array_equal(rice.rice_decode(blob, len(vals), fb), v)


def test_escape_path():
    # one huge value among small ones: q >= 31 for the chosen k, written as
    # 31 ones and 32 raw bits
    v = np.array([3, 1, 0, 2, 4000000000, 1, 2], np.uint32)
    b = rice.rice_encode(v, 32)
    k = b[0]
    assert (int(v[4]) >> k) >= 31
    assert len(b) == 1 + (_bits(v, k, 32, 31) + 7) // 8
    assert np.array_equal(rice.rice_decode(b, len(v), 32), v)


@pytest.mark.parametrize("fb", [16, 32])
@pytest.mark.parametrize("dist", ["geometric", "uniform", "max", "equal", "mixed"])
def test_round_trip_and_optimal_parameter(fb, dist):
    rng = np.random.default_rng(fb * 7 + len(dist))
    hi = (1 << fb) - 1
    n = 3000
    if dist == "geometric":
        v = rng.geometric(0.003, n) - 1
    elif dist == "uniform":
        v = rng.integers(0, hi, n, endpoint=True)
    elif dist == "max":
        v = np.full(n, hi)
    elif dist == "equal":
        v = np.full(n, 37)
    else:
        v = np.concatenate([rng.geometric(0.05, n) - 1, rng.integers(0, hi, 40, endpoint=True)])
        rng.shuffle(v)
    v = np.minimum(v, hi).astype(np.uint32)
    b = rice.rice_encode(v, fb)
    sizes = [_bits(v, k, fb, 31) for k in range(min(fb, 31) + 1)]
    assert b[0] == int(np.argmin(sizes))
    assert len(b) == 1 + (min(sizes) + 7) // 8
    assert np.array_equal(rice.rice_decode(b, len(v), fb), v)


def test_many_arrays_threaded_equal_one_by_one():
    rng = np.random.default_rng(5)
    arrays = [(rng.geometric(0.01, int(n)) - 1).astype(np.uint32) for n in rng.integers(0, 300, 200)]
    blobs = rice.encode_many(arrays, 32, n_threads=8)
    assert blobs == [rice.rice_compress(a, 32) for a in arrays]
    back = rice.decode_many(blobs, [len(a) for a in arrays], 32, n_threads=8)
    assert all(np.array_equal(a, b) for a, b in zip(arrays, back))


def test_split_side_streams_round_trip():
    from sigcomp_amd import signal, synth
    reads = synth.synth_reads(6, 3, synth.DNA, lengths=[1, 2, 500, 3000, 20000, 7])
    reads[3][100:140] = np.int16(-32768)   # wrap-around deltas: large values near 65535
    sp = signal.split_reads(reads)
    la, lg = rice.encode_split(sp)
    assert all(b == b"\x00" for b, n in zip(la, sp["n_large"]) if n == 0)
    adj, gap, off = rice.decode_split(la, lg, sp["n_large"])
    assert np.array_equal(adj, sp["large_adj"]) and np.array_equal(gap, sp["large_gap"])
    assert np.array_equal(off, sp["large_off"])
    out = signal.reassemble_reads({**sp, "large_adj": adj, "large_gap": gap, "large_off": off})
    assert all(np.array_equal(a, b) for a, b in zip(reads, out))


@pytest.mark.parametrize("case", ["truncated", "trailing", "padding", "k", "short", "quotient", "fallback"])
def test_malformed_blobs_rejected(case):
    v = np.array([9, 2, 7, 300, 1], np.uint32)
    b = bytearray(rice.rice_encode(v, 16))
    n = len(v)
    if case == "truncated":
        b = b[:-1]
    elif case == "trailing":
        b += b"\x00"
    elif case == "padding":
        used = _bits(v, b[0], 16, 31)
        assert used % 8, "the test needs a padded last byte"
        b[-1] |= 0x80
    elif case == "k":
        b[0] = 17
    elif case == "short":
        b = b[:1]
    elif case == "fallback":
        # k = 16, q = 1, low bits 5: the value 65541 does not fit 16 bits
        b = bytearray([16, 0x15, 0x00, 0x00])
        n = 1
    else:
        # k = 31 and a quotient of 2: no 32-bit value has it
        b = bytearray([31, 0b011])
        n = 1
    with pytest.raises(ValueError, match="Rice"):
        rice.rice_decode(bytes(b), n, 16 if case != "quotient" else 32)


def test_negative_count_rejected_before_anything_is_written():
    """A negative count beside a valid item: the Python boundary raises, and
    the C ABI returns SC_ERR_ARG naming the item without writing any value
    (the output offsets after a negative count would not be valid)."""
    import ctypes
    from sigcomp_amd import _host
    blob = rice.rice_encode(np.array([1, 2, 3], np.uint32), 32)
    with pytest.raises(ValueError, match="non-negative"):
        rice.decode_many([b"\x00", blob], [-3, 3], 32)
    kept = [np.zeros(1, np.uint8), np.frombuffer(blob, np.uint8)]
    ptrs = np.array([a.ctypes.data for a in kept], np.uint64)
    lens = np.array([1, len(blob)], np.int64)
    counts = np.array([-3, 3], np.int64)
    out_off = np.array([0, 0], np.int64)
    out = np.full(8, 0xDEADBEEF, np.uint32)
    bad = ctypes.c_int64(-1)
    rc = _host.lib().sc_rice_decode(_host._p(ptrs), _host._p(lens), _host._p(counts), 2, 32, 31, _host._p(out),
                                    _host._p(out_off), 1, ctypes.byref(bad))
    assert rc != 0 and bad.value == 0
    assert (out == 0xDEADBEEF).all()


def test_value_outside_fallback_width_rejected():
    with pytest.raises(ValueError, match="fallback width"):
        rice.rice_encode(np.array([1, 65536], np.uint32), 16)
    with pytest.raises(ValueError):
        rice.rice_encode(np.array([-1]), 32)
