"""sc_decompress_chunks_static (the entry point that allocates nothing: its
decode state lives in a static device array of the library) against
sc_decompress_chunks on the same inputs, through the C ABI, bit-exact:
two calls in a row, the second with a smaller input, with the launch plan
from host lengths and from device lengths."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def codec(int_models):
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    return QuantMLPCompression(chunk_len=2048, gpu=0, model=int_models["lossless"])


def _inputs(codec, n, lo, hi, seed):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(lo, hi + 1, n).astype(np.int32)
    lengths[rng.choice(n, 3, replace=False)] = [0, 1, hi]
    tokens = rng.integers(0, 60, int(lengths.sum())).astype(np.uint8)
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    return tokens, lengths, words, woff, wcnt


def _decode(codec, entry, words, woff, wcnt, lengths, host_lengths):
    """One call of `entry` ("workspace" or "static") on chunks in the given
    order -> (tokens, status); outputs start as 0xAB / -1."""
    from sigcomp_amd import _hip
    L = _hip.lib()
    n = len(lengths)
    tok_off = np.zeros(n, np.int64)
    np.cumsum(lengths[:-1], dtype=np.int64, out=tok_off[1:])
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    t_words, t_woff, t_cnt = d(words.view(np.int32)), d(woff.astype(np.int64)), d(wcnt.astype(np.int32))
    t_len, t_toff = d(lengths.astype(np.int32)), d(tok_off)
    out = torch.full((max(int(lengths.sum()), 1),), 0xAB, dtype=torch.uint8, device="cuda")
    status = torch.full((n,), -1, dtype=torch.int32, device="cuda")
    len_host = np.ascontiguousarray(lengths, np.int32)
    hl = len_host.ctypes.data if host_lengths else None
    args = [codec.hip.handle, t_words.data_ptr(), t_woff.data_ptr(), t_cnt.data_ptr(), t_len.data_ptr(), n,
            out.data_ptr(), t_toff.data_ptr(), status.data_ptr(), hl]
    stream = torch.cuda.current_stream().cuda_stream
    if entry == "static":
        _hip.check(L.sc_decompress_chunks_static(*args, stream))
    else:
        ws = codec._decompress_workspace(n)
        _hip.check(L.sc_decompress_chunks(*args, ws.data_ptr(), ws.numel(), stream))
    torch.cuda.synchronize()
    return out.cpu().numpy()[:int(lengths.sum())], status.cpu().numpy()


@pytest.mark.parametrize("host_lengths", [True, False])
def test_static_entry_matches_workspace_entry(codec, monkeypatch, host_lengths):
    """Call 1: 2 * 32 * n_cu + 150 chunks of up to 700 tokens (full-wave
    launches, leftover chunks paired into the last one's rows, three 256-step
    segments whose state goes through the static array); call 2, smaller:
    900 chunks of up to 300 tokens (one launch of 32-chunk workgroups over
    two segments).  The second call runs over the first call's leftover
    state; both must equal the workspace entry point's output and the
    original tokens."""
    monkeypatch.delenv("SC_HIP_DEC_SEG", raising=False)
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    for n, hi, seed in ((2 * 32 * n_cu + 150, 700, 1), (900, 300, 2)):
        tokens, lengths, words, woff, wcnt = _inputs(codec, n, 1, hi, seed)
        src = np.concatenate([[0], np.cumsum(lengths[:-1])]).astype(np.int64)   # input chunk starts
        order = np.argsort(-lengths, kind="stable")            # longest first, as decompress_flat
        s_len, s_woff, s_wcnt = lengths[order], woff[order], wcnt[order]
        ref_tok, ref_st = _decode(codec, "workspace", words, s_woff, s_wcnt, s_len, host_lengths)
        got_tok, got_st = _decode(codec, "static", words, s_woff, s_wcnt, s_len, host_lengths)
        assert np.array_equal(got_st, ref_st) and not got_st.any()
        assert np.array_equal(got_tok, ref_tok)
        expect = np.concatenate([tokens[src[c]:src[c] + lengths[c]] for c in order])
        assert np.array_equal(got_tok, expect)


def test_static_entry_rejects_more_chunks_than_its_array(codec):
    from sigcomp_amd import _hip
    L = _hip.lib()
    n = _hip.STATIC_DEC_MAX_CHUNKS + 1
    dummy = torch.zeros(8, dtype=torch.int64, device="cuda")
    p = dummy.data_ptr()
    rc = L.sc_decompress_chunks_static(codec.hip.handle, p, p, p, p, n, p, p, p, None,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"at most" in L.sc_last_error()


def test_static_entry_under_graph_capture(codec):
    """The entry point's callers include code under HIP graph capture: 40
    chunks over two 256-step segments (a batch that decodes split when not
    captured; a capturing stream gets the unsplit launches) captured once
    and replayed three times, with eager work between the replays that
    overwrites the outputs; every replay equals the eager decode and the
    input."""
    from sigcomp_amd import _hip
    L = _hip.lib()
    tokens, lengths, words, woff, wcnt = _inputs(codec, 40, 300, 600, 5)
    ref_tok, ref_st = _decode(codec, "static", words, woff, wcnt, lengths, True)
    assert not ref_st.any()
    src = np.concatenate([[0], np.cumsum(lengths[:-1])]).astype(np.int64)
    assert np.array_equal(ref_tok, np.concatenate([tokens[src[c]:src[c] + lengths[c]] for c in range(40)]))
    n = len(lengths)
    tok_off = np.zeros(n, np.int64)
    np.cumsum(lengths[:-1], dtype=np.int64, out=tok_off[1:])
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    t_words, t_woff, t_cnt = d(words.view(np.int32)), d(woff.astype(np.int64)), d(wcnt.astype(np.int32))
    t_len, t_toff = d(lengths.astype(np.int32)), d(tok_off)
    out = torch.empty(int(lengths.sum()), dtype=torch.uint8, device="cuda")
    status = torch.empty(n, dtype=torch.int32, device="cuda")
    len_host = np.ascontiguousarray(lengths, np.int32)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=cap):
        _hip.check(L.sc_decompress_chunks_static(
            codec.hip.handle, t_words.data_ptr(), t_woff.data_ptr(), t_cnt.data_ptr(), t_len.data_ptr(), n,
            out.data_ptr(), t_toff.data_ptr(), status.data_ptr(), len_host.ctypes.data,
            torch.cuda.current_stream().cuda_stream))
    for rep in range(3):
        out.fill_(0xAB)
        status.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(status.cpu().numpy(), ref_st), rep
        assert np.array_equal(out.cpu().numpy(), ref_tok), rep


def test_device_lengths_refused_under_graph_capture(codec):
    """Without the host copy of the lengths the launch plan would read them
    back from the device, a wait that a capturing stream cannot hold: both
    decode entries return SC_ERR_ARG before enqueuing anything, so the
    caller's capture stays valid; a call with host lengths captured after
    the refused ones replays correctly."""
    from sigcomp_amd import _hip
    L = _hip.lib()
    tokens, lengths, words, woff, wcnt = _inputs(codec, 40, 100, 300, 7)
    n = len(lengths)
    ref_tok, ref_st = _decode(codec, "static", words, woff, wcnt, lengths, True)
    tok_off = np.zeros(n, np.int64)
    np.cumsum(lengths[:-1], dtype=np.int64, out=tok_off[1:])
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    t_words, t_woff, t_cnt = d(words.view(np.int32)), d(woff.astype(np.int64)), d(wcnt.astype(np.int32))
    t_len, t_toff = d(lengths.astype(np.int32)), d(tok_off)
    out = torch.empty(int(lengths.sum()), dtype=torch.uint8, device="cuda")
    status = torch.empty(n, dtype=torch.int32, device="cuda")
    ws = codec._decompress_workspace(n)
    len_host = np.ascontiguousarray(lengths, np.int32)
    torch.cuda.synchronize()
    args = lambda hl: [codec.hip.handle, t_words.data_ptr(), t_woff.data_ptr(), t_cnt.data_ptr(), t_len.data_ptr(),
                       n, out.data_ptr(), t_toff.data_ptr(), status.data_ptr(), hl]
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=cap):
        s = torch.cuda.current_stream().cuda_stream
        rc_static = L.sc_decompress_chunks_static(*args(None), s)
        err_static = L.sc_last_error()
        rc_ws = L.sc_decompress_chunks(*args(None), ws.data_ptr(), ws.numel(), s)
        _hip.check(L.sc_decompress_chunks_static(*args(len_host.ctypes.data), s))
    assert rc_static == _hip.SC_ERR_ARG and rc_ws == _hip.SC_ERR_ARG
    assert b"graph capture" in err_static
    for rep in range(2):
        out.fill_(0xAB)
        status.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(status.cpu().numpy(), ref_st), rep
        assert np.array_equal(out.cpu().numpy(), ref_tok), rep
