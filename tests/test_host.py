"""Host library (libsigcomp_host.so): signal split / reassembly and SIG2 chunk
framing, against the numpy restatement of main.py's transforms
(oracle/signal_ref.py), closed forms, the restated framing loop
(oracle/framing_ref.py, cpu_compression.py:28-84) and the reference's
golden framed reads."""

import numpy as np
import pytest

from conftest import GOLDEN, REPO

HEADER = REPO / "include" / "sigcomp_host.h"


def _lib_or_skip():
    from sigcomp_amd import _host
    if not _host.LIB_PATH.exists():
        pytest.skip("libsigcomp_host.so not built")
    return _host


def test_host_library_exports_every_declared_symbol():
    import ctypes
    import re
    _host = _lib_or_skip()
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(sc_(?:host|rice)_[a-z0-9_]+)\s*\(", text)))
    assert "sc_rice_encode" in names and "sc_rice_decode" in names
    lib = ctypes.CDLL(str(_host.LIB_PATH))
    assert [n for n in names if not hasattr(lib, n)] == []
    assert sorted(_host.EXPORTED) == names


def _reads(rng):
    from sigcomp_amd import synth
    out = [np.array([v], np.int16) for v in (-32768, 0, 32767)]
    out += [rng.integers(-32768, 32768, n).astype(np.int16) for n in (2, 3, 17, 1000)]
    out += [np.full(50, 123, np.int16), np.tile(np.array([-32768, 32767], np.int16), 40)]
    out += synth.synth_reads(6, 11, synth.DNA) + synth.synth_reads(3, 12, synth.RNA)
    return out


@pytest.mark.parametrize("lsb", [0, 1, 2, 3, 7, 15])
def test_split_matches_numpy_restatement(lsb):
    import signal_ref as ref
    _lib_or_skip()
    from sigcomp_amd import signal
    rng = np.random.default_rng(lsb)
    reads = _reads(rng)
    got = signal.split_reads(reads, lsb)
    for i, r in enumerate(reads):
        s0, sm, la, lg = ref.split_signal(ref.prepare_signal(r, lsb))
        o, n = got["small_off"][i], got["n_small"][i]
        lo, ln = got["large_off"][i], got["n_large"][i]
        assert int(got["sig0"][i]) == s0
        assert np.array_equal(got["small"][o:o + n], sm)
        assert np.array_equal(got["large_adj"][lo:lo + ln], la)
        assert np.array_equal(got["large_gap"][lo:lo + ln], lg)
        one = signal.split_signal(r, lsb)
        assert one[0] == s0 and np.array_equal(one[1], sm)


def test_zigzag_split_exhaustive_over_all_int16_deltas():
    """A read whose consecutive deltas are every int16 value once: zigzag
    z = (d << 1) ^ (d >> 31) mod 2**16, small iff d in [-128, 127]."""
    _lib_or_skip()
    from sigcomp_amd import signal
    d = np.arange(-32768, 32768, dtype=np.int64)
    sig = (np.concatenate([[5], 5 + np.cumsum(d)]) & 0xFFFF).astype(np.uint16).view(np.int16)
    sig0, small, large_adj, gaps = signal.split_signal(sig)
    z = ((d << 1) ^ (d >> 63)) & 0xFFFF
    is_small = (d >= -128) & (d <= 127)
    assert np.array_equal(is_small, z < 256)
    assert sig0 == 5
    assert np.array_equal(small, z[is_small].astype(np.uint8))
    assert np.array_equal(large_adj, (z[~is_small] - 256).astype(np.uint16))
    pos = np.flatnonzero(~is_small)
    exp_gaps = np.concatenate([[pos[0]], np.diff(pos) - 1])
    assert np.array_equal(gaps, exp_gaps.astype(np.uint32))
    back = signal.reassemble_signal(sig0, len(sig), small, large_adj, gaps)
    assert np.array_equal(back, sig)


@pytest.mark.parametrize("lsb", [0, 1, 3, 15])
def test_reassemble_inverts_split(lsb):
    import signal_ref as ref
    _lib_or_skip()
    from sigcomp_amd import signal
    reads = _reads(np.random.default_rng(100 + lsb))
    sp = signal.split_reads(reads, lsb)
    back = signal.reassemble_reads(sp, lsb=lsb)
    for r, b in zip(reads, back):
        exp = ref.lossy_decode(ref.prepare_signal(r, lsb), lsb) if lsb else r
        assert np.array_equal(b, exp)
        # the reference's own reassembly of the same pieces
        s0, sm, la, lg = ref.split_signal(ref.prepare_signal(r, lsb))
        rr = ref.reassemble_signal(s0, len(r), sm, la, lg)
        assert np.array_equal(b, ref.lossy_decode(rr, lsb) if lsb else rr)


def _wrap16(x):
    """Two's-complement int16 value of the integer x (x mod 2**16, signed)."""
    return ((x + 32768) % 65536) - 32768


def _lossy_closed_forms(b):
    """The lossy LSB transform of main.py:158-171 stated arithmetically, in
    int64 floor division rather than the reference's masks and shifts:
    reduce = round half up to a multiple of 2**b (floor((v + 2**(b-1)) / 2**b)
    * 2**b), wrapped to int16; encode = floor(x / 2**b); decode = x * 2**b
    wrapped to int16.  -> (v, reduce(v), encode(reduce(v)), decode(encode(...)))
    over every int16 value v."""
    v = np.arange(-32768, 32768, dtype=np.int64)
    step = 2 ** b
    red = _wrap16((v + step // 2) // step * step)
    enc = red // step
    dec = _wrap16(enc * step)
    return v, red, enc, dec


@pytest.mark.parametrize("lsb", list(range(1, 16)))
def test_lossy_transform_closed_form_every_int16(lsb):
    """Pins the oracle's lossy restatement (signal_ref.reduce_lsb /
    lossy_encode / lossy_decode) and the C++ split / reassembly against the
    closed form over all 65,536 int16 samples for lsb 1..15, incl. ties
    (v = k * 2**b + 2**(b-1) rounds up, also below zero) and the wrap of
    32767 rounded up past the int16 range."""
    import signal_ref as ref
    v, red, enc, dec = _lossy_closed_forms(lsb)
    v16 = v.astype(np.int16)
    assert np.array_equal(ref.reduce_lsb(v16, lsb).astype(np.int64), red)
    assert np.array_equal(ref.lossy_encode(red.astype(np.int16), lsb).astype(np.int64), enc)
    assert np.array_equal(ref.lossy_decode(enc.astype(np.int16), lsb).astype(np.int64), dec)
    assert np.array_equal(ref.prepare_signal(v16, lsb).astype(np.int64), enc)
    # special cases in plain Python integers
    half = 1 << (lsb - 1)
    assert int(ref.reduce_lsb(np.array([half], np.int16), lsb)[0]) == _wrap16(1 << lsb)   # tie rounds up
    assert int(ref.reduce_lsb(np.array([-half], np.int16), lsb)[0]) == 0                  # -1/2 rounds up to 0
    assert int(ref.reduce_lsb(np.array([half - 1], np.int16), lsb)[0]) == 0
    top = _wrap16(((32767 + half) >> lsb) << lsb)            # 32767 rounds to 2**15: wraps to -32768
    assert int(ref.reduce_lsb(np.array([32767], np.int16), lsb)[0]) == top == -32768
    assert int(ref.reduce_lsb(np.array([-32768], np.int16), lsb)[0]) == -32768
    # the C++ host library: one read of every int16 value (in order, then
    # shuffled, so the deltas vary), split with lsb and reassembled
    _lib_or_skip()
    from sigcomp_amd import signal
    perm = np.random.default_rng(lsb).permutation(65536)
    reads = [v16, v16[perm]]
    sp = signal.split_reads(reads, lsb)
    for i, (r, e) in enumerate(zip(reads, [enc, enc[perm]])):
        s0, sm, la, lg = ref.split_signal(e.astype(np.int16))
        o, n = sp["small_off"][i], sp["n_small"][i]
        assert int(sp["sig0"][i]) == s0 == int(e[0])
        assert np.array_equal(sp["small"][o:o + n], sm)
        lo, ln = sp["large_off"][i], sp["n_large"][i]
        assert np.array_equal(sp["large_adj"][lo:lo + ln], la)
        assert np.array_equal(sp["large_gap"][lo:lo + ln], lg)
    back = signal.reassemble_reads(sp, lsb=lsb)
    assert np.array_equal(back[0].astype(np.int64), dec)
    assert np.array_equal(back[1].astype(np.int64), dec[perm])


def test_lossy_closed_form_rejects_plausible_misreadings():
    """The closed form is not a restatement of itself: a round-half-down
    reading, a missing int16 wrap or a logical shift would each differ."""
    v, red, enc, dec = _lossy_closed_forms(3)
    half_down = _wrap16((v + 3) // 8 * 8)
    assert not np.array_equal(half_down, red)
    no_wrap = (v + 4) // 8 * 8
    assert not np.array_equal(no_wrap, red)
    logical = (red & 0xFFFF) >> 3
    assert not np.array_equal(logical, enc)


def test_reassemble_and_split_errors():
    _lib_or_skip()
    from sigcomp_amd import signal
    with pytest.raises(IndexError):
        signal.split_reads([np.zeros(3, np.int16), np.zeros(0, np.int16)])
    sig = np.array([0, 1000, 1000, -1000, 5], np.int16)
    s0, sm, la, lg = signal.split_signal(sig)
    with pytest.raises(ValueError):                   # one small token missing
        signal.reassemble_signal(s0, len(sig), sm[:-1], la, lg)
    bad = lg.copy()
    bad[-1] += 10                                      # last large position beyond the read
    with pytest.raises(IndexError):
        signal.reassemble_signal(s0, len(sig), sm, la, bad)
    assert np.array_equal(signal.reassemble_signal(s0, len(sig), sm, la, lg), sig)


def test_frame_matches_python_framing():
    _host = _lib_or_skip()
    from framing_ref import frame as frame_chunks
    rng = np.random.default_rng(3)
    cnt = rng.integers(1, 40, 50).astype(np.int32)
    cap = cnt + rng.integers(0, 3, 50)
    off = np.concatenate([[0], np.cumsum(cap)[:-1]]).astype(np.int64)
    words = rng.integers(0, 2**32, int(cap.sum()), dtype=np.uint64).astype(np.uint32)
    buf, bounds = _host.frame(words, off, cnt)
    chunks = [words[o:o + c].tobytes() for o, c in zip(off, cnt)]
    assert buf.tobytes() == frame_chunks(chunks)
    for k in range(len(cnt)):
        assert buf[bounds[k]:bounds[k + 1]].tobytes() == frame_chunks(chunks[k:k + 1])
    with pytest.raises(ValueError, match="uint16 frame"):
        _host.frame(np.zeros(20000, np.uint32), np.zeros(1, np.int64), np.array([16384], np.int32))


def _payload(rng, tokens, chunk_len):
    from framing_ref import frame as frame_chunks
    n = (tokens + chunk_len - 1) // chunk_len
    return frame_chunks([rng.integers(0, 2**32, rng.integers(1, 9), dtype=np.uint64).astype(np.uint32).tobytes()
                         for _ in range(n)])


def test_parse_matches_python_parse_and_errors():
    _host = _lib_or_skip()
    from framing_ref import parse as parse_framed
    rng = np.random.default_rng(4)
    tokens = [0, 1, 7, 8, 9, 30, 64]
    payloads = [_payload(rng, t, 8) for t in tokens]
    pr = _host.parse(payloads, tokens, 8)
    for r, (p, t) in enumerate(zip(payloads, tokens)):
        parts, counts = parse_framed(p, t, 8)
        c0 = pr["chunk_begin"][r]
        assert pr["frames"][r] == len(parts)
        for k, (part, cnt) in enumerate(zip(parts, counts)):
            c = c0 + k
            w = pr["words"][pr["word_off"][c]:pr["word_off"][c] + pr["word_cnt"][c]]
            assert w.tobytes() == part and pr["tok_cnt"][c] == cnt
    good = payloads[5]
    cases = [good[:1], good[:-1], good + b"\0", b"\0\0" + good[2:], b"\x06\x00" + good[2:]]
    for bad in cases:
        with pytest.raises(ValueError) as py_err:
            parse_framed(bad, 30, 8)
        with pytest.raises(ValueError) as host_err:
            _host.parse([payloads[0], bad], [0, 30], 8)
        assert str(host_err.value).startswith(str(py_err.value))
        assert "read 1" in str(host_err.value)


def test_parse_reads_payloads_in_place_from_any_buffer():
    """parse takes each payload where it lies (sc_host_parse_v, no joined
    copy): bytes, bytearray, memoryview and numpy payloads in one call give
    the words of sc_host_parse over the joined data, and the payloads are
    left as they were."""
    import ctypes
    _host = _lib_or_skip()
    rng = np.random.default_rng(9)
    tokens = [0, 5, 8, 17, 40, 3]
    payloads = [_payload(rng, t, 8) for t in tokens]
    mixed = [payloads[0], bytearray(payloads[1]), memoryview(payloads[2]),
             np.frombuffer(payloads[3], np.uint8).copy(), payloads[4], bytes(payloads[5])]
    before = [bytes(p) for p in mixed]
    pr = _host.parse(mixed, tokens, 8)
    assert [bytes(p) for p in mixed] == before
    # the joined-buffer entry point on the same data
    L = _host.lib()
    data = np.frombuffer(b"".join(payloads), np.uint8)
    lens = np.array([len(p) for p in payloads], np.int64)
    off = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    tk = np.array(tokens, np.int64)
    frames = (tk + 7) // 8
    cb = np.concatenate([[0], np.cumsum(frames)[:-1]]).astype(np.int64)
    rwo = np.concatenate([[0], np.cumsum(lens // 4)[:-1]]).astype(np.int64)
    nc = int(frames.sum())
    words = np.zeros(max(int((lens // 4).sum()), 1), np.uint32)
    wo, wc, tc = np.zeros(nc, np.int64), np.zeros(nc, np.int32), np.zeros(nc, np.int32)
    bad = ctypes.c_int64(-1)
    p = lambda a: a.ctypes.data
    assert L.sc_host_parse(p(data), p(off), p(lens), p(tk), len(tokens), 8, p(cb), p(rwo), p(words), p(wo), p(wc),
                           p(tc), 0, ctypes.byref(bad)) == 0
    assert np.array_equal(pr["word_off"], wo) and np.array_equal(pr["word_cnt"], wc)
    for c in range(nc):   # the words each chunk wrote (a read's slots past its frames are not written)
        assert np.array_equal(pr["words"][wo[c]:wo[c] + wc[c]], words[wo[c]:wo[c] + wc[c]])
    assert np.array_equal(pr["tok_cnt"], tc)


class _OracleCodec:
    """CPU codec around the C oracle with the GPU codec's flat interface, so
    that the batched framing path of ReadFramingMixin runs here."""

    def __init__(self, oracle_mod, om, chunk_len=2048):
        self.o, self.om, self.chunk_len = oracle_mod, om, chunk_len

    def compress_flat(self, tokens, lengths, max_batch_size=64, use_tqdm=False):
        off = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
        enc = self.o.compress_chunks(self.om, [tokens[o:o + n] for o, n in zip(off, lengths)])
        cnt = np.array([len(e) // 4 for e in enc], np.int32)
        words = np.frombuffer(b"".join(enc), np.uint32) if enc else np.zeros(0, np.uint32)
        return words, np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.int64), cnt

    def decompress_flat(self, words, word_off, word_cnt, lengths, use_tqdm=False):
        dec = self.o.decompress_chunks(self.om, [words[o:o + c].tobytes() for o, c in zip(word_off, word_cnt)],
                                       list(lengths))
        tok_off = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
        return (np.concatenate(dec) if dec else np.zeros(0, np.uint8)), tok_off


def test_batched_framing_matches_reference_golden_reads(oracle_mod, oracle_models):
    _lib_or_skip()
    from sigcomp_amd import signal
    from sigcomp_amd.framing import ReadFramingMixin

    class Codec(_OracleCodec, ReadFramingMixin):
        pass

    z = np.load(GOLDEN / "e2e_reads.npz")
    for name in ("lossless", "lossy"):
        lsb = int(z[f"{name}_lsb"])
        reads = [z[f"{name}_read{i}_signal"] for i in range(int(z[f"{name}_nreads"]))]
        codec = Codec(oracle_mod, oracle_models[name])
        small = signal.reads_tokens(signal.split_reads(reads, lsb))
        framed = codec.batch_inference_reads(list_of_reads=small + [np.zeros(0, np.uint8)], batch_size=7)
        for i in range(len(reads)):
            assert framed[i] == z[f"{name}_read{i}_sbytes"].tobytes(), (name, i)
        assert framed[-1] == b""
        back = codec.batch_inference_reads(list_of_compressed_reads=framed,
                                           list_of_lengths=[len(s) for s in small] + [0])
        assert all(np.array_equal(a, b) for a, b in zip(small, back)) and back[-1].size == 0
        with pytest.raises(ValueError):
            codec.batch_inference_reads(list_of_compressed_reads=framed[:2], list_of_lengths=[len(small[0]), -1])
