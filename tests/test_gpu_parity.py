"""GPU parity: the gfx950 kernels against the reference golden vectors and the
CPU oracle, bit-exact (integer / byte work has no tolerance)."""

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def codecs(int_models):
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    return {name: QuantMLPCompression(chunk_len=2048, gpu=0, model=m) for name, m in int_models.items()}


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_ar_step_matches_reference_logits(codecs, name):
    z = np.load(GOLDEN / f"mlp_{name}.npz")
    ctx = torch.from_numpy(z["ctx"]).cuda()
    got = codecs[name].gpu_engine._ar_step(ctx)[:, 0].cpu().numpy()
    assert np.array_equal(got, z["logits"])


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_fused_mlp_cdf_matches_reference(codecs, name):
    z = np.load(GOLDEN / f"mlp_{name}.npz")
    c = np.load(GOLDEN / f"cdf_{name}.npz")
    n = z["ctx"].shape[0]
    got = codecs[name].hip.forward_windows(torch.from_numpy(z["ctx"]).cuda(), "cdf").cpu().numpy()
    assert np.array_equal(got.astype(np.int64), c["cdf"][:n])


@pytest.mark.parametrize("rows", [1, 127, 128, 129, 1000])
def test_ar_step_matches_oracle_random_windows(codecs, oracle_mod, oracle_models, rows):
    rng = np.random.default_rng(rows)
    ctx = rng.integers(0, 257, (rows, 64))
    ctx[: rows // 3, : 20] = 256
    got = codecs["lossless"].gpu_engine._ar_step(torch.from_numpy(ctx).cuda())[:, 0].cpu().numpy()
    assert np.array_equal(got, oracle_mod.mlp_forward(oracle_models["lossless"], ctx))


def test_random_per_channel_model_matches_oracle(oracle_mod):
    from sigcomp_amd.model_io import random_int_model
    from sigcomp_amd.quant_mlp_export import HipModel
    m = random_int_model(seed=7, per_channel=True)
    hm = HipModel(m, torch.device("cuda:0"))
    rng = np.random.default_rng(9)
    ctx = rng.integers(0, 257, (300, 64))
    got = hm.forward_windows(torch.from_numpy(ctx).cuda(), "logits").cpu().numpy()
    om = oracle_mod.OracleModel(m)
    exp = oracle_mod.mlp_forward(om, ctx)
    assert np.array_equal(got, exp)
    assert len(np.unique(exp)) > 50          # activations are not saturated
    cdf = hm.forward_windows(torch.from_numpy(ctx).cuda(), "cdf").cpu().numpy()
    assert np.array_equal(cdf.astype(np.int64), oracle_mod.logits_to_cdf(exp, m.exp_lut))


def test_bad_context_token_raises(codecs):
    ctx = torch.full((3, 64), 256, dtype=torch.int64, device="cuda")
    ctx[1, 7] = 300
    with pytest.raises(ValueError):
        codecs["lossless"].gpu_engine._ar_step(ctx)


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_int8_logits_to_cdf_matches_reference(int_models, name):
    from sigcomp_amd.gpu_entropy_coding import int8_logits_to_cdf
    c = np.load(GOLDEN / f"cdf_{name}.npz")
    got = int8_logits_to_cdf(torch.from_numpy(c["logits"]).cuda(), int_models[name].exp_lut)
    assert np.array_equal(got.cpu().numpy(), c["cdf"])


def _adversarial_logits(rng):
    """Rows aimed at the frequency rule's corner cases: constant rows (every
    quotient an exact integer, the exact-division path), argmax ties inside
    one lane's 16 symbols and across lanes (first argmax wins), one-hot rows
    (with the lossy LUT's zero tail one frequency is 2**24 before the
    correction), two-level rows, narrow and wide random rows."""
    rows = [np.full(256, v) for v in (-128, -1, 0, 1, 127)]
    for pos in [(0,), (15,), (16,), (255,), (16, 17), (255, 16, 17), (31, 30), (240, 15), (3, 200)]:
        for hi, lo in ((127, -128), (5, 0), (-60, -128)):
            r = np.full(256, lo)
            r[list(pos)] = hi
            rows.append(r)
    idx = np.arange(256)
    for a, b in [(0, 1), (0, -1), (10, -10), (127, -128), (3, 2), (-128, 127)]:
        rows += [np.where(idx % 2 == 0, a, b), np.where(idx < 128, a, b), np.where(idx % 16 == 0, a, b),
                 np.where(idx % 16 == 15, a, b)]
    for spread in (1, 2, 4, 8, 32, 128):
        rows += list(rng.integers(-spread, spread + 1, (300, 256)) + rng.integers(-100, 100, (300, 1)))
    rows += list(rng.integers(-128, 128, (3000, 256)))
    return np.clip(np.array(rows), -128, 127).astype(np.int8)


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_logits_to_cdf_adversarial_rows_match_oracle(int_models, oracle_mod, name):
    from sigcomp_amd.gpu_entropy_coding import int8_logits_to_cdf
    lut = int_models[name].exp_lut
    rows = _adversarial_logits(np.random.default_rng(11))
    got = int8_logits_to_cdf(torch.from_numpy(rows).cuda(), lut).cpu().numpy()
    exp = oracle_mod.logits_to_cdf(rows, lut)
    assert got.shape == exp.shape
    bad = np.flatnonzero((got != exp).any(axis=1))
    assert bad.size == 0, f"rows {bad[:10]} differ"


def _golden_streams(name):
    z = np.load(GOLDEN / "coder_streams.npz")
    keys = sorted({k.rsplit("_", 1)[0] for k in z.files if k.startswith(name + "_")})
    return z, keys


# "0" / "1": the narrow (16 lanes per row) / wide (64 rows per wave) step kernels
STEP_PATHS = ["0", "1"]


@pytest.mark.parametrize("wide", STEP_PATHS)
@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_step_encoder_and_decoder_match_reference(int_models, name, wide, monkeypatch):
    monkeypatch.setenv("SC_HIP_STEP_WIDE", wide)
    from sigcomp_amd.gpu_entropy_coding import GpuRangeDecoder, GpuRangeStepEncoder
    z, keys = _golden_streams(name)
    lut = torch.from_numpy(int_models[name].exp_lut)
    B = len(keys)
    T = max(len(z[f"{k}_symbols"]) for k in keys)
    lg = np.zeros((B, T, 256), np.int8)
    sy = np.zeros((B, T), np.int64)
    valid = np.array([len(z[f"{k}_symbols"]) for k in keys], np.int64)
    for b, k in enumerate(keys):
        lg[b, :valid[b]] = z[f"{k}_logits"]
        sy[b, :valid[b]] = z[f"{k}_symbols"]
    enc = GpuRangeStepEncoder(B, T + 32, device="cuda")
    lg_d = torch.from_numpy(lg).cuda()
    sy_d = torch.from_numpy(sy).cuda()
    v_d = torch.from_numpy(valid).cuda()
    for t in range(T):
        enc.encode_step_int8(lg_d[:, t], lut, sy_d[:, t], v_d, t)
    words = enc.get_compressed()
    for b, k in enumerate(keys):
        assert np.array_equal(np.frombuffer(words[b], "<u4"), z[f"{k}_words"]), k
    dec = GpuRangeDecoder(words, device="cuda")
    got = np.zeros((B, T), np.int64)
    for t in range(T):
        got[:, t] = dec.decode_step_int8(lg_d[:, t], lut, v_d, t).cpu().numpy()
    dec.check()
    for b, k in enumerate(keys):
        assert np.array_equal(got[b, :valid[b]], z[f"{k}_decoded"]), k
        assert np.all(got[b, valid[b]:] == 256)


@pytest.mark.parametrize("wide", STEP_PATHS)
def test_step_api_many_streams(int_models, oracle_mod, wide, monkeypatch):
    """Large batches, as the coder benchmark runs them: 150,001 CDF rows
    (9,376 workgroups of 16 rows, the last one partial) against the oracle,
    and 70,001 streams x 3 encode / decode steps whose decoder returns every
    coded symbol, with every 1000th stream active for one step only."""
    monkeypatch.setenv("SC_HIP_STEP_WIDE", wide)
    from sigcomp_amd.gpu_entropy_coding import GpuRangeDecoder, GpuRangeStepEncoder, int8_logits_to_cdf
    lut_np = int_models["lossless"].exp_lut
    g = torch.Generator(device="cuda").manual_seed(3)
    rows = (torch.randn(150001, 256, generator=g, device="cuda") * 20).round().clamp(-128, 127).to(torch.int8)
    cdf = int8_logits_to_cdf(rows, lut_np).cpu().numpy()
    sub = np.r_[0:300, 65530:65600, 149800:150001]
    assert np.array_equal(cdf[sub], oracle_mod.logits_to_cdf(rows.cpu().numpy()[sub], lut_np))
    B, T = 70001, 3
    lut = torch.from_numpy(lut_np)
    lg = [(torch.randn(B, 256, generator=g, device="cuda") * 20).round().clamp(-128, 127).to(torch.int8)
          for _ in range(T)]
    sy = [torch.randint(0, 256, (B,), generator=g, device="cuda") for _ in range(T)]
    valid = torch.full((B,), T, dtype=torch.int64, device="cuda")
    valid[::1000] = 1
    enc = GpuRangeStepEncoder(B, T + 32, device="cuda")
    for t in range(T):
        enc.encode_step_int8(lg[t], lut, sy[t], valid, t)
    dec = GpuRangeDecoder(enc.get_compressed(), device="cuda")
    for t in range(T):
        got = dec.decode_step_int8(lg[t], lut, valid, t).clone()
        exp = torch.where(valid > t, sy[t], torch.full_like(sy[t], 256))
        assert torch.equal(got, exp), t
    dec.check()


def test_step_api_wide_batch_default_path_against_oracle(int_models, oracle_mod, monkeypatch):
    """A batch at the size from which the wide step kernels are chosen
    (2**18 streams + 1: 1,025 workgroups of 256 rows, the last with one),
    5 steps with stream lengths from 1 to 5: 64 streams' sealed words
    against the oracle, the decoder returns every coded symbol, and the
    narrow kernels give the same words."""
    monkeypatch.delenv("SC_HIP_STEP_WIDE", raising=False)
    from sigcomp_amd.gpu_entropy_coding import GpuRangeDecoder, GpuRangeStepEncoder
    lut_np = int_models["lossless"].exp_lut
    lut = torch.from_numpy(lut_np)
    B, T = (1 << 18) + 1, 5
    g = torch.Generator(device="cuda").manual_seed(8)
    lg = (torch.randn(T, B, 256, generator=g, device="cuda") * 20).round().clamp(-128, 127).to(torch.int8)
    sy = torch.randint(0, 256, (T, B), generator=g, device="cuda")
    valid = torch.randint(1, T + 1, (B,), generator=g, device="cuda")
    valid[-1] = T

    def encode():
        enc = GpuRangeStepEncoder(B, T + 32, device="cuda")
        for t in range(T):
            enc.encode_step_int8(lg[t], lut, sy[t], valid, t)
        return enc.get_compressed()

    words = encode()
    rng = np.random.default_rng(9)
    pick = np.r_[rng.choice(B - 1, 63, replace=False), B - 1]
    lg_h, sy_h, v_h = lg.cpu().numpy(), sy.cpu().numpy(), valid.cpu().numpy()
    for b in pick:
        n = int(v_h[b])
        ref = oracle_mod.encode_stream(lg_h[:n, b], sy_h[:n, b], lut_np)
        assert np.array_equal(np.frombuffer(words[b], "<u4"), ref), b
    dec = GpuRangeDecoder(words, device="cuda")
    for t in range(T):
        got = dec.decode_step_int8(lg[t], lut, valid, t).clone()
        assert torch.equal(got, torch.where(valid > t, sy[t], torch.full_like(sy[t], 256))), t
    dec.check()
    monkeypatch.setenv("SC_HIP_STEP_WIDE", "0")
    assert encode() == words


@pytest.mark.parametrize("wide", STEP_PATHS)
def test_step_encoder_capacity_per_stream(oracle_mod, int_models, wide, monkeypatch):
    """Streams that fit max_words, that overflow at their seal (oracle word
    count max_words + 1) and that overflow during a step, side by side:
    each overflowing stream, and only it, reports SC_STATUS_CAPACITY;
    every other stream's words equal the oracle's; get_compressed raises
    OverflowError naming the first overflowing stream."""
    monkeypatch.setenv("SC_HIP_STEP_WIDE", wide)
    from sigcomp_amd import _hip
    from sigcomp_amd.gpu_entropy_coding import GpuRangeStepEncoder
    rng = np.random.default_rng(21)
    lut_np = int_models["lossless"].exp_lut
    B = 48
    lens = rng.integers(1, 120, B)
    T = int(lens.max())
    lg = rng.normal(0, 20, (B, T, 256)).round().clip(-128, 127).astype(np.int8)
    sy = rng.integers(0, 256, (B, T)).astype(np.int64)
    totals = np.array([len(oracle_mod.encode_stream(lg[b, :lens[b]], sy[b, :lens[b]], lut_np)) for b in range(B)])
    j = int(np.argsort(totals, kind="stable")[B // 2])
    M = int(totals[j]) - 1                       # stream j's steps fit, its seal does not
    over = totals > M
    assert over.sum() >= 3 and (~over).sum() >= 3 and (totals >= M + 3).any()
    enc = GpuRangeStepEncoder(B, M, device="cuda")
    lg_d, sy_d = torch.from_numpy(lg).cuda(), torch.from_numpy(sy).cuda()
    v_d = torch.from_numpy(lens.astype(np.int64)).cuda()
    lut = torch.from_numpy(lut_np)
    for t in range(T):
        enc.encode_step_int8(lg_d[:, t], lut, sy_d[:, t], v_d, t)
    enc.seal()
    torch.cuda.synchronize()
    status = enc.status.cpu().numpy()
    assert np.array_equal(status != 0, over), (status, totals, M)
    assert (status[over] == _hip.SC_STATUS_CAPACITY).all()
    wp = enc.write_pos.cpu().numpy()
    ow = enc.output_words.cpu().numpy().view(np.uint32)
    for b in np.flatnonzero(~over):
        ref = oracle_mod.encode_stream(lg[b, :lens[b]], sy[b, :lens[b]], lut_np)
        assert np.array_equal(ow[b, :wp[b]], ref), b
    with pytest.raises(OverflowError, match=f"stream {int(np.flatnonzero(over)[0])};"):
        enc.get_compressed()


@pytest.mark.parametrize("wide", STEP_PATHS)
def test_step_decoder_invalid_stream_beside_valid_ones(oracle_mod, int_models, wide, monkeypatch):
    """A corrupt stream between valid ones: it returns 256 from the step
    that detects it on (its status stays set), check() raises, and its
    neighbours decode every symbol."""
    monkeypatch.setenv("SC_HIP_STEP_WIDE", wide)
    from sigcomp_amd.gpu_entropy_coding import GpuRangeDecoder
    rng = np.random.default_rng(22)
    lut_np = int_models["lossless"].exp_lut
    B, T = 5, 40
    lg = rng.normal(0, 20, (B, T, 256)).round().clip(-128, 127).astype(np.int8)
    sy = rng.integers(0, 256, (B, T)).astype(np.int64)
    streams = [oracle_mod.encode_stream(lg[b], sy[b], lut_np).tobytes() for b in range(B)]
    streams[2] = np.array([0xFFFFFFFF, 0xFFFFFFFF, 7], np.uint32).tobytes()
    dec = GpuRangeDecoder(streams, device="cuda")
    valid = torch.full((B,), T, dtype=torch.int64)
    lg_d = torch.from_numpy(lg).cuda()
    got = np.stack([dec.decode_step_int8(lg_d[:, t], lut_np, valid, t).cpu().numpy() for t in range(T)], axis=1)
    for b in (0, 1, 3, 4):
        assert np.array_equal(got[b], sy[b]), b
    assert (got[2] == 256).all()
    with pytest.raises(ValueError):
        dec.check()


@pytest.mark.parametrize("wide", STEP_PATHS)
def test_step_decoder_flags_invalid_stream(int_models, wide, monkeypatch):
    monkeypatch.setenv("SC_HIP_STEP_WIDE", wide)
    from sigcomp_amd.gpu_entropy_coding import GpuRangeDecoder
    bad = np.array([0xFFFFFFFF, 0xFFFFFFFF], np.uint32).tobytes()
    dec = GpuRangeDecoder([bad], device="cuda")
    lg = torch.zeros((1, 256), dtype=torch.int8, device="cuda")
    sym = dec.decode_step_int8(lg, int_models["lossless"].exp_lut, torch.tensor([4]), 0)
    assert int(sym[0]) == 256
    with pytest.raises(ValueError):
        dec.check()


def test_step_api_rejects_mis_shaped_arguments(int_models):
    """Per-stream arguments whose length is not the batch size (the kernels
    index them by stream) and logits of the wrong shape or dtype: ValueError
    before any launch, on the encoder and the decoder."""
    from sigcomp_amd.gpu_entropy_coding import GpuRangeDecoder, GpuRangeStepEncoder
    lut = int_models["lossless"].exp_lut
    B = 5
    lg = torch.zeros((B, 256), dtype=torch.int8, device="cuda")
    enc = GpuRangeStepEncoder(B, 8, device="cuda")
    sy = torch.zeros(B, dtype=torch.int64)
    ok = torch.full((B,), 3)
    for bad_sy, bad_valid in ((sy[:-1], ok), (sy, ok[:-1]), (sy, torch.full((B + 1,), 3))):
        with pytest.raises(ValueError):
            enc.encode_step_int8(lg, lut, bad_sy, bad_valid, 0)
    with pytest.raises(ValueError):
        enc.encode_step_int8(lg[:-1], lut, sy, ok, 0)
    with pytest.raises(ValueError):
        enc.encode_step_int8(lg.to(torch.int16), lut, sy, ok, 0)
    dec = GpuRangeDecoder([np.zeros(2, np.uint32).tobytes()] * B, device="cuda")
    for bad_valid in (ok[:-1], torch.full((B + 1,), 3), torch.full((B, 1), 3)):
        with pytest.raises(ValueError):
            dec.decode_step_int8(lg, lut, bad_valid, 0)
    with pytest.raises(ValueError):
        dec.decode_step_int8(lg[:-1], lut, ok, 0)
    assert dec.decode_step_int8(lg, lut, ok, 0).shape == (B,)


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_batch_inference_reads_matches_reference_e2e(codecs, name):
    from sigcomp_amd import signal
    z = np.load(GOLDEN / "e2e_reads.npz")
    lsb = int(z[f"{name}_lsb"])
    n = int(z[f"{name}_nreads"])
    small = [signal.split_signal(z[f"{name}_read{i}_signal"], lsb)[1]
             for i in range(n)]
    framed = codecs[name].batch_inference_reads(list_of_reads=small, batch_size=20480)
    for i in range(n):
        assert framed[i] == z[f"{name}_read{i}_sbytes"].tobytes(), i
    back = codecs[name].batch_inference_reads(list_of_compressed_reads=framed,
                                              list_of_lengths=[len(s) for s in small],
                                              batch_size=20480)
    for s, b in zip(small, back):
        assert np.array_equal(s, b)


@pytest.mark.parametrize("lengths", [[1], [2, 63, 64, 65], [127, 128, 129, 300, 2048, 1, 7],
                                     [2048] * 5 + [5, 1999]])
def test_compress_decompress_chunks_match_oracle(codecs, oracle_mod, oracle_models, lengths):
    rng = np.random.default_rng(sum(lengths))
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in lengths]
    chunks[0][: min(3, lengths[0])] = 255
    gpu = codecs["lossless"].compress_chunks(chunks, max_batch_size=4)
    ref = oracle_mod.compress_chunks(oracle_models["lossless"], chunks)
    assert gpu == ref
    back = codecs["lossless"].decompress_chunks(gpu, lengths)
    for c, b in zip(chunks, back):
        assert np.array_equal(c, b)


def test_compress_tile_table_with_empty_chunks(codecs, oracle_mod, oracle_models):
    """Compress finds each 128-step tile through a descriptor table built
    from the tile offsets of the chunks; empty chunks own no tiles and share
    their offset with the next chunk.  Empty chunks between, before and after
    chunks whose lengths end on and just past tile boundaries."""
    lengths = [0, 5, 0, 0, 128, 129, 0, 256, 1, 0]
    rng = np.random.default_rng(31)
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in lengths]
    gpu = codecs["lossless"].compress_chunks(chunks)
    assert gpu == oracle_mod.compress_chunks(oracle_models["lossless"], chunks)
    assert [len(b) == 0 for b in gpu] == [n == 0 for n in lengths]
    back = codecs["lossless"].decompress_chunks(gpu, lengths)
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))


def test_compress_abi_negative_length_owns_no_tiles(codecs, oracle_mod, oracle_models):
    """Through the C ABI (the Python layer rejects it), a negative chunk
    length counts as an empty chunk: it owns no compress tiles and no words,
    and the other chunks' tiles and bytes are unaffected."""
    from sigcomp_amd import _hip
    codec = codecs["lossless"]
    rng = np.random.default_rng(43)
    lengths = np.array([5, -300, 130, 0, 257], np.int32)
    used = np.maximum(lengths, 0)
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in used]
    n = len(lengths)
    n_tokens = int(used.sum())
    tok_off = np.zeros(n, np.int64)
    np.cumsum(used[:-1], out=tok_off[1:])
    cap = (used + 2).astype(np.int32)
    word_off = np.zeros(n, np.int64)
    np.cumsum(cap[:-1].astype(np.int64), out=word_off[1:])
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    t_tok, t_off, t_len, t_woff, t_cap = d(np.concatenate(chunks)), d(tok_off), d(lengths), d(word_off), d(cap)
    words, cnt, status, ws = codec._compress_buffers(n, n_tokens, int(cap.sum()))
    L, p = _hip.lib(), _hip.ptr
    _hip.check(L.sc_compress_chunks(codec.hip.handle, p(t_tok), p(t_off), p(t_len), n, n_tokens, p(words),
                                    p(t_woff), p(t_cap), p(cnt), p(status), p(ws), ws.numel(),
                                    torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ref = oracle_mod.compress_chunks(oracle_models["lossless"], chunks)
    w, c = words.cpu().numpy().view(np.uint32), cnt.cpu().numpy()
    assert not status.cpu().numpy().any() and c[1] == 0
    for i in range(n):
        assert w[word_off[i]:word_off[i] + c[i]].tobytes() == ref[i]


def test_compress_abi_word_capacity_per_chunk(codecs, oracle_mod, oracle_models):
    """Through the C ABI a caller sets each chunk's word capacity: chunks
    whose capacity is exactly their oracle word count, one word short (the
    seal does not fit) and half of it (a step does not fit), side by side.
    Each short chunk, and only it, reports SC_STATUS_CAPACITY; every other
    chunk's words equal the oracle's."""
    from sigcomp_amd import _hip
    codec = codecs["lossless"]
    rng = np.random.default_rng(44)
    lengths = np.array([300, 300, 300, 129, 129, 129, 2048, 2048, 1], np.int32)
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in lengths]
    ref = oracle_mod.compress_chunks(oracle_models["lossless"], chunks)
    need = np.array([len(r) // 4 for r in ref], np.int32)
    cap = need.copy()
    cap[[1, 4, 7]] -= 1                       # one word short
    cap[[2, 5]] //= 2                         # half
    short = cap < need
    n = len(lengths)
    n_tokens = int(lengths.sum())
    tok_off = np.zeros(n, np.int64)
    np.cumsum(lengths[:-1], out=tok_off[1:])
    word_off = np.zeros(n, np.int64)
    np.cumsum(cap[:-1].astype(np.int64), out=word_off[1:])
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    t_tok, t_off, t_len, t_woff, t_cap = d(np.concatenate(chunks)), d(tok_off), d(lengths), d(word_off), d(cap)
    words, cnt, status, ws = codec._compress_buffers(n, n_tokens, int(cap.sum()))
    L, p = _hip.lib(), _hip.ptr
    _hip.check(L.sc_compress_chunks(codec.hip.handle, p(t_tok), p(t_off), p(t_len), n, n_tokens, p(words),
                                    p(t_woff), p(t_cap), p(cnt), p(status), p(ws), ws.numel(),
                                    torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    st, c = status.cpu().numpy(), cnt.cpu().numpy()
    w = words.cpu().numpy().view(np.uint32)
    assert np.array_equal(st != 0, short), (st, cap, need)
    assert (st[short] == _hip.SC_STATUS_CAPACITY).all()
    for i in np.flatnonzero(~short):
        assert c[i] == need[i] and w[word_off[i]:word_off[i] + c[i]].tobytes() == ref[i], i


def test_long_chunk_len_matches_oracle(int_models, oracle_mod, oracle_models):
    """chunk_len 5000 (the reference lets the caller choose it): chunks span
    40 compress tiles and 20 decode launches of 256 steps, lengths not on
    tile or segment boundaries; then a read framed into such chunks."""
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    codec = QuantMLPCompression(chunk_len=5000, gpu=0, model=int_models["lossless"])
    rng = np.random.default_rng(41)
    lengths = [5000, 4999, 2049, 300]
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in lengths]
    gpu = codec.compress_chunks(chunks)
    assert gpu == oracle_mod.compress_chunks(oracle_models["lossless"], chunks)
    back = codec.decompress_chunks(gpu, lengths)
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))
    read = rng.integers(0, 60, 12345).astype(np.uint8)
    framed = codec.batch_inference_reads(list_of_reads=[read])
    out = codec.batch_inference_reads(list_of_compressed_reads=framed, list_of_lengths=[read.size])
    assert np.array_equal(out[0], read)


def test_decompress_many_chunks_round_trip(codecs):
    """More chunks than one workgroup row tile per CU; mixed lengths."""
    rng = np.random.default_rng(11)
    n = 3000
    lengths = rng.integers(1, 200, n)
    chunks = [rng.integers(0, 40, L).astype(np.uint8) for L in lengths]
    comp = codecs["lossy"].compress_chunks(chunks)
    back = codecs["lossy"].decompress_chunks(comp, list(lengths))
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))


def test_decompress_corrupt_chunk_raises(codecs):
    bad = [np.array([0xFFFFFFFF, 0xFFFFFFFF], np.uint32).tobytes()]
    with pytest.raises(ValueError):
        codecs["lossless"].decompress_chunks(bad, [10])


def test_decompress_flat_rejects_inconsistent_chunk_tables(codecs):
    """Word ranges outside the word array (negative offset or count, past
    its end), words for an empty chunk or none for a non-empty one, a length
    beyond chunk_len: ValueError before anything reaches the GPU."""
    codec = codecs["lossless"]
    words = np.arange(10, dtype=np.uint32)
    cases = [([0, -1], [4, 6], [5, 7], "Invalid range-coded"), ([0, 4], [4, -2], [5, 7], "Invalid range-coded"),
             ([0, 4], [4, 7], [5, 7], "Invalid range-coded"), ([0, 4], [4, 0], [5, 7], "Invalid range-coded"),
             ([0, 4], [4, 6], [5, 0], "Invalid range-coded"), ([0, 4], [4, 6], [5, codec.chunk_len + 1], "chunk_len"),
             ([0], [4, 6], [5, 7], "counts differ")]
    for woff, cnt, lengths, msg in cases:
        with pytest.raises(ValueError, match=msg):
            codec.decompress_flat(words, np.array(woff, np.int64), np.array(cnt, np.int32), np.array(lengths, np.int32))


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_full_symbol_range_against_oracle(codecs, oracle_mod, oracle_models, monkeypatch, name):
    """Tokens uniform over all 256 symbols (most of them rare under the
    model: frequencies at the floor of 1, ~3 bytes of stream per token), and
    chunks of only 255 or only 0: every chunk's bytes equal the oracle's and
    both the persistent and the split decode return the tokens."""
    codec = codecs[name]
    rng = np.random.default_rng(256 + (name == "lossy"))
    lengths = rng.integers(1, 301, 200).astype(np.int32)
    lengths[:4] = [1, 64, 300, 2048]
    chunks = [rng.integers(0, 256, n).astype(np.uint8) for n in lengths]
    chunks[0][:] = 255
    chunks[1][:] = 255
    chunks[2][:] = 0
    comp = codec.compress_chunks(chunks)
    assert comp == oracle_mod.compress_chunks(oracle_models[name], chunks)
    for split in ("0", None):
        if split is None:
            monkeypatch.delenv("SC_HIP_DEC_SPLIT", raising=False)
        else:
            monkeypatch.setenv("SC_HIP_DEC_SPLIT", split)
        back = codec.decompress_chunks(comp, list(lengths))
        assert all(np.array_equal(a, b) for a, b in zip(chunks, back)), split


def test_empty_inputs(codecs):
    assert codecs["lossless"].compress_chunks([]) == []
    assert codecs["lossless"].decompress_chunks([], []) == []
    assert codecs["lossless"].batch_inference_reads(list_of_reads=[np.zeros(0, np.uint8)]) == [b""]
    out = codecs["lossless"].batch_inference_reads(list_of_compressed_reads=[b""], list_of_lengths=[0])
    assert len(out) == 1 and out[0].size == 0


def _plain_and_generic_models():
    """Models that run the plain (non-pipelined) MLP core: the bundled lossless
    model with the core forced by SC_HIP_PLAIN_CORE, and a random model whose
    layer 3 needs the 64-bit requantisation (shift < 32 with m0 = 2**31, and
    m0 = 2**31 - 1), which the pipelined core does not take."""
    import dataclasses
    from sigcomp_amd.model_io import load_int_model, make_layer, random_int_model
    lossless = load_int_model()
    m = random_int_model(seed=21, per_channel=True)
    L = m.layers[3]
    n = L.n
    m0 = np.where(np.arange(n) % 2 == 0, 1 << 31, (1 << 31) - 1).astype(np.int64)
    shift = np.full(n, 41, np.int32)
    shift[::7] = 31
    w = (L.weight // 16).astype(np.int8)
    layers = list(m.layers)
    layers[3] = make_layer(w, L.bias // 64, m0, shift, True)
    return lossless, dataclasses.replace(m, layers=layers)


@pytest.mark.parametrize("which", ["plain_lossless", "generic_requant"])
def test_plain_core_matches_oracle(oracle_mod, monkeypatch, which):
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    lossless, generic = _plain_and_generic_models()
    if which == "plain_lossless":
        monkeypatch.setenv("SC_HIP_PLAIN_CORE", "1")
        model = lossless
    else:
        model = generic
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model=model)
    monkeypatch.delenv("SC_HIP_PLAIN_CORE", raising=False)
    assert not codec.hip.pipelined
    om = oracle_mod.OracleModel(model)
    rng = np.random.default_rng(5)
    ctx = rng.integers(0, 257, (300, 64))
    ctx[:50, :30] = 256
    exp = oracle_mod.mlp_forward(om, ctx)
    got = codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "logits").cpu().numpy()
    assert np.array_equal(got, exp)
    cdf = codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "cdf").cpu().numpy()
    assert np.array_equal(cdf.astype(np.int64), oracle_mod.logits_to_cdf(exp, model.exp_lut))
    lengths = [1, 64, 65, 300, 129]
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in lengths]
    gpu = codec.compress_chunks(chunks)
    assert gpu == oracle_mod.compress_chunks(om, chunks)
    back = codec.decompress_chunks(gpu, lengths)
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))


@pytest.mark.parametrize("core", ["pipelined", "plain"])
def test_fast_requant_clamp_bounds_match_oracle(oracle_mod, monkeypatch, core):
    """Fast-path layers (every shift >= 32, mulhi(acc, m0) >> (shift - 32))
    whose per-channel shifts span 32..63: shifts that saturate most values at
    127 and, on the output layer, at -128, shifts that leave 0 / -1, and the
    largest shifts (shift - 32 up to 31)."""
    from sigcomp_amd.model_io import make_layer, random_int_model
    from sigcomp_amd.quant_mlp_export import HipModel
    import dataclasses
    m = random_int_model(seed=13, per_channel=True)
    rng = np.random.default_rng(13)
    layers = list(m.layers)
    for li in (2, len(layers) - 1):
        L = layers[li]
        shift = np.full(L.n, 36, np.int32)
        for r, s in enumerate((32, 33, 56, 63, 55, 44)):
            shift[r::7] = s
        m0 = rng.integers(1 << 30, (1 << 31) - 1, L.n)
        layers[li] = make_layer(L.weight, L.bias, m0, shift, L.relu)
    model = dataclasses.replace(m, layers=layers)
    if core == "plain":
        monkeypatch.setenv("SC_HIP_PLAIN_CORE", "1")
    hm = HipModel(model, torch.device("cuda:0"))
    monkeypatch.delenv("SC_HIP_PLAIN_CORE", raising=False)
    assert hm.pipelined == (core == "pipelined")
    ctx = rng.integers(0, 257, (300, 64))
    ctx[:40, :25] = 256
    exp = oracle_mod.mlp_forward(oracle_mod.OracleModel(model), ctx)
    assert (exp == 127).any() and (exp == -128).any() and (exp == -1).any()
    got = hm.forward_windows(torch.from_numpy(ctx).cuda(), "logits").cpu().numpy()
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("layer,shift", [(2, 32), (2, 33), (2, 38), (2, 56), (2, 63),
                                         (-1, 32), (-1, 38), (-1, 56), (-1, 63)])
def test_per_tensor_requant_matches_oracle(oracle_mod, layer, shift):
    """Per-tensor constants (one m0 and shift per layer, as in the bundled
    checkpoints) select core 2, whose requantisation clamps before the shift
    against per-layer bounds and shifts into the packed byte.  Layer 2's
    shift: 32 (most values saturate at 127), 33, 38, 56 (the bound
    128 * 2**24 - 1 exceeds int32 and is capped) and 63; the output layer's
    (no ReLU, arithmetic shift): 32 (saturation at -128 and 127), 38, 56
    (both bounds capped) and 63.  Logits, CDFs, chunk bytes and the round
    trip are compared with the oracle."""
    import dataclasses
    from sigcomp_amd.model_io import make_layer, random_int_model
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    m = random_int_model(seed=17, per_channel=False)
    rng = np.random.default_rng(17)
    layers = list(m.layers)
    li = layer % len(layers)
    L = layers[li]
    m0 = int(rng.integers(1 << 30, 1 << 31))
    layers[li] = make_layer(L.weight, L.bias, np.full(L.n, m0), np.full(L.n, shift, np.int32), L.relu)
    model = dataclasses.replace(m, layers=layers)
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model=model)
    assert codec.hip.core == 2
    om = oracle_mod.OracleModel(model)
    ctx = rng.integers(0, 257, (300, 64))
    ctx[:40, :25] = 256
    exp = oracle_mod.mlp_forward(om, ctx)
    if li == len(layers) - 1 and shift == 32:
        assert (exp == 127).any() and (exp == -128).any()
    got = codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "logits").cpu().numpy()
    assert np.array_equal(got, exp)
    cdf = codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "cdf").cpu().numpy()
    assert np.array_equal(cdf.astype(np.int64), oracle_mod.logits_to_cdf(exp, model.exp_lut))
    lengths = [1, 64, 129, 700]
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in lengths]
    gpu = codec.compress_chunks(chunks)
    assert gpu == oracle_mod.compress_chunks(om, chunks)
    back = codec.decompress_chunks(gpu, lengths)
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))


def test_per_channel_model_runs_plain_core_in_codec(oracle_mod):
    """A pipelined-capable model with per-channel constants runs core 1: the
    pipelined core in the explicit-context kernels, the plain core in
    compress / decompress; chunk bytes still equal the oracle's."""
    from sigcomp_amd.model_io import random_int_model
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    model = random_int_model(seed=23, per_channel=True)
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model=model)
    assert codec.hip.core == 1
    rng = np.random.default_rng(23)
    lengths = [2, 65, 333]
    chunks = [rng.integers(0, 60, n).astype(np.uint8) for n in lengths]
    gpu = codec.compress_chunks(chunks)
    assert gpu == oracle_mod.compress_chunks(oracle_mod.OracleModel(model), chunks)
    back = codec.decompress_chunks(gpu, lengths)
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))


def test_pipelined_core_selected_for_bundled_models(codecs):
    assert codecs["lossless"].hip.core == 2 and codecs["lossy"].hip.core == 2


@pytest.mark.parametrize("pair", ["auto", "0"])
@pytest.mark.parametrize("units,extra", [(2, 7), (3, 0), (4, 31), (5, 1), (6, 500)])
def test_decompress_launch_plans(codecs, oracle_mod, oracle_models, monkeypatch, units, extra, pair):
    """Chunk counts that fill `units` full waves of 32-chunk row tiles per CU
    (split by the launch planner into 64/96/128-chunk workgroup launches)
    plus leftover chunks, paired with the last launch's rows (auto) or in a
    launch of their own (SC_HIP_DEC_PAIR=0); short random chunk lengths."""
    if pair == "0":
        monkeypatch.setenv("SC_HIP_DEC_PAIR", "0")
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    n = units * 32 * n_cu + extra
    rng = np.random.default_rng(units * 1000 + extra)
    lengths = rng.integers(1, 40, n).astype(np.int32)
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossless"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    back, tok_off = codec.decompress_flat(words, woff, wcnt, lengths)
    assert np.array_equal(back, tokens)
    sample = rng.choice(n, 16, replace=False)
    off = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    chunks = [tokens[off[i]:off[i] + lengths[i]] for i in sample]
    ref = oracle_mod.compress_chunks(oracle_models["lossless"], chunks)
    assert [words[woff[i]:woff[i] + wcnt[i]].tobytes() for i in sample] == ref


def test_decompress_greedy_plan_uses_160_chunk_workgroups(codecs, capfd, monkeypatch):
    """SC_HIP_DEC_PLAN=greedy with 6 units takes one launch of 160-chunk
    workgroups (the plain core's rt = 5 kernel) and one of 32, then the
    leftover chunks; every chunk round-trips."""
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    n = 6 * 32 * n_cu + 77
    rng = np.random.default_rng(66)
    lengths = rng.integers(1, 70, n).astype(np.int32)
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossless"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    capfd.readouterr()
    monkeypatch.setenv("SC_HIP_DEC_PLAN", "greedy")
    monkeypatch.setenv("SC_HIP_DEC_LOG", "1")
    back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
    log = capfd.readouterr().err
    assert "plan [5,1]" in log, log
    assert np.array_equal(back, tokens)


def test_decompress_one_million_chunks(codecs, capfd, monkeypatch):
    """1,000,003 chunks of 1..6 tokens: a plan of many full-wave launches,
    the decode state buffer grown to a million rows, and the length
    statistics over all of them."""
    rng = np.random.default_rng(7)
    n = 1_000_003
    lengths = rng.integers(1, 7, n).astype(np.int32)
    tokens = rng.integers(0, 60, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossy"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    capfd.readouterr()
    monkeypatch.setenv("SC_HIP_DEC_LOG", "1")
    back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
    assert "chunks 1000003" in capfd.readouterr().err
    assert np.array_equal(back, tokens)


def _decode_direct(codec, words, woff, wcnt, lengths, host_lengths=True, ws_fill=None):
    """sc_decompress_chunks on the chunks in the order given (the C ABI does
    not sort) -> (tokens of all chunks in chunk order, per-chunk status).
    Status starts at -1 so that a chunk whose status is never written shows.
    host_lengths: pass the host copy of the lengths (plan on the host) or
    NULL (plan statistics on the device); ws_fill: byte written over the
    workspace first (state left by an unrelated call)."""
    from sigcomp_amd import _hip
    n = len(lengths)
    tok_off = np.zeros(n, np.int64)
    np.cumsum(lengths[:-1], dtype=np.int64, out=tok_off[1:])
    n_tok = int(lengths.sum())
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    t_words, t_woff, t_cnt = d(words.view(np.int32)), d(woff.astype(np.int64)), d(wcnt.astype(np.int32))
    t_len, t_toff = d(lengths.astype(np.int32)), d(tok_off)
    tokens = torch.zeros(max(n_tok, 1), dtype=torch.uint8, device="cuda")
    status = torch.full((n,), -1, dtype=torch.int32, device="cuda")
    ws = codec._decompress_workspace(n)
    if ws_fill is not None:
        ws.fill_(ws_fill)
    len_host = np.ascontiguousarray(lengths, np.int32)   # referenced until the call returns
    _hip.check(_hip.lib().sc_decompress_chunks(
        codec.hip.handle, _hip.ptr(t_words), _hip.ptr(t_woff), _hip.ptr(t_cnt), _hip.ptr(t_len), n,
        _hip.ptr(tokens), _hip.ptr(t_toff), _hip.ptr(status),
        len_host.ctypes.data if host_lengths else None, _hip.ptr(ws), ws.numel(), _hip.stream_ptr()))
    torch.cuda.synchronize()
    return tokens.cpu().numpy()[:n_tok], status.cpu().numpy(), tok_off


def _set_dec_env(monkeypatch, seg):
    monkeypatch.setenv("SC_HIP_DEC_LOG", "1")
    if seg is None:
        monkeypatch.delenv("SC_HIP_DEC_SEG", raising=False)
    else:
        monkeypatch.setenv("SC_HIP_DEC_SEG", str(seg))


@pytest.mark.parametrize("seg", [None, 64, 0])
def test_decompress_pairs_leftover_chunks(codecs, capfd, monkeypatch, seg):
    """The chunks left over after the full waves (here 300, the shortest)
    are decoded by the last full-wave launch's shortest rows after their own
    chunk ends; default 256-step segments, 64-step segments, one launch."""
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    G, L = 2 * 32 * n_cu, 300
    rng = np.random.default_rng(31 + (seg or 0))
    lengths = np.concatenate([rng.integers(900, 1201, G - L), rng.integers(1, 701, 2 * L)]).astype(np.int32)
    rng.shuffle(lengths)
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossless"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    capfd.readouterr()
    _set_dec_env(monkeypatch, seg)
    back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
    log = capfd.readouterr().err
    assert "leftover 300 paired" in log, log
    assert np.array_equal(back, tokens)


def test_decompress_rejects_pairing_of_long_leftovers(codecs, capfd, monkeypatch):
    """Leftover chunks as long as the rest would stretch the last full-wave
    launch (64-chunk workgroups) by more than a separate leftover launch
    costs: no pairing."""
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    n = 2 * 32 * n_cu + 40
    rng = np.random.default_rng(8)
    lengths = rng.integers(550, 601, n).astype(np.int32)
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossless"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    capfd.readouterr()
    _set_dec_env(monkeypatch, None)
    back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
    log = capfd.readouterr().err
    assert "leftover 40 split launch" in log, log
    assert np.array_equal(back, tokens)


@pytest.mark.parametrize("seg", [None, 64])
def test_decompress_paired_rows_status_and_edges(codecs, capfd, monkeypatch, seg):
    """Pairing through the C ABI on unsorted chunks: first chunks that end on
    64- and 256-step edges, an empty first chunk, and corrupt first and
    second chunks.  Each corrupt chunk (and only it) reports an invalid
    stream; the other chunk of its row still decodes."""
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    G, L = 32 * n_cu, 120
    rng = np.random.default_rng(77 if seg is None else seg)
    lengths = np.concatenate([rng.integers(800, 1001, G - L), rng.integers(100, 401, L),
                              rng.integers(1, 301, L)]).astype(np.int32)
    # rows G-L .. G-1 are the paired first chunks; row c's second is 2G-1-c
    edge = [63, 64, 65, 127, 128, 255, 256, 257, 320, 383, 384, 385]
    lengths[G - L:G - L + len(edge)] = edge
    lengths[G - 1] = 0
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossless"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    bad = [G - L + 20, 2 * G - 1 - (G - L + 30), G - L + 6]   # a first, a second, an edge first chunk
    words = np.concatenate([words, np.full(2, 0xFFFFFFFF, np.uint32)])
    woff, wcnt = woff.copy(), wcnt.copy()
    woff[bad], wcnt[bad] = len(words) - 2, 2
    capfd.readouterr()
    _set_dec_env(monkeypatch, seg)
    back, status, tok_off = _decode_direct(codec, words, woff, wcnt, lengths)
    log = capfd.readouterr().err
    assert f"leftover {L} paired" in log, log
    expect = np.zeros(len(lengths), np.int32)
    expect[bad] = 2   # SC_STATUS_INVALID_STREAM
    assert np.array_equal(status, expect)
    for i in range(len(lengths)):
        if i not in bad:
            s = slice(tok_off[i], tok_off[i] + lengths[i])
            assert np.array_equal(back[s], tokens[s]), i


@pytest.mark.parametrize("seg, host", [(None, True), (64, True), (0, True), (64, False)])
def test_decompress_longest_row_is_a_pair_ending_on_a_segment_edge(codecs, capfd, monkeypatch, seg, host):
    """A paired row's second chunk starts one step after its first ends, so
    a pair of 24 + 1000 tokens takes 1025 steps: more than the longest
    single chunk (1000) and one past a 64- and 256-step segment edge.  The
    launch plan counts that step (its last token decodes) in 96-chunk
    workgroups, whose epilogue runs beside the next step's layer 0; with
    the plan's length statistics from the host copy of the lengths or from
    the device."""
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    G, L = 3 * 32 * n_cu, 50
    rng = np.random.default_rng(5 + (seg or 0))
    lengths = np.concatenate([rng.integers(900, 1001, G - L), rng.integers(100, 401, L),
                              rng.integers(1, 101, L)]).astype(np.int32)
    lengths[G - L] = 24                # first chunk of row G-L ...
    lengths[2 * G - 1 - (G - L)] = 1000   # ... and its second chunk
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossless"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    capfd.readouterr()
    _set_dec_env(monkeypatch, seg)
    back, status, tok_off = _decode_direct(codec, words, woff, wcnt, lengths, host_lengths=host)
    log = capfd.readouterr().err
    assert f"leftover {L} paired" in log and "steps 1025" in log, log
    assert not status.any()
    for i in range(len(lengths)):
        s = slice(tok_off[i], tok_off[i] + lengths[i])
        assert np.array_equal(back[s], tokens[s]), i


def test_decompress_status_survives_later_segments(codecs, monkeypatch):
    """A corrupt chunk in a workgroup whose rows all end in the first 64-step
    launch keeps its status through the later launches another workgroup's
    long chunk needs (those launches find nothing left to do there)."""
    rng = np.random.default_rng(4)
    lengths = np.full(64, 10, np.int32)
    lengths[0] = 300
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    codec = codecs["lossless"]
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    words = np.concatenate([words, np.full(2, 0xFFFFFFFF, np.uint32)])
    woff, wcnt = woff.copy(), wcnt.copy()
    woff[40], wcnt[40] = len(words) - 2, 2
    monkeypatch.setenv("SC_HIP_DEC_SEG", "64")
    # a workspace holding another call's state (every row's "current chunk"
    # field nonzero): launches past a workgroup's rows must not read it
    for host_lengths, fill in ((True, None), (False, 1), (True, 255)):
        back, status, tok_off = _decode_direct(codec, words, woff, wcnt, lengths, host_lengths, fill)
        expect = np.zeros(64, np.int32)
        expect[40] = 2
        assert np.array_equal(status, expect)
        keep = np.ones(len(back), bool)
        keep[tok_off[40]:tok_off[40] + 10] = False
        assert np.array_equal(back[keep], tokens[keep])


def _random_chunks(codec, n, hi, seed):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, hi + 1, n).astype(np.int32)
    tokens = rng.integers(0, 60, int(lengths.sum())).astype(np.uint8)
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    return tokens, lengths, words, woff, wcnt


@pytest.mark.parametrize("n,seg", [(1, None), (3, 64), (33, None), (675, None), (675, 64), (675, 0), (1024, None),
                                   (1025, None), (2048, None)])
def test_split_decode_matches_unsplit(codecs, capfd, monkeypatch, n, seg):
    """Launches of at most 64 groups of 32 chunks decode split (workgroups
    of a group share layer 0 and exchange its features every step): eight
    workgroups per group up to 32 groups, four up to 64 (and four when
    forced, SC_HIP_DEC_SPLIT=4).  One chunk, a partial group, two groups, 22
    groups (the c1 case) over 256-step and 64-step segments and one launch,
    32, 33 and 64 groups.  Tokens equal the input and the unsplit decode's
    (SC_HIP_DEC_SPLIT=0)."""
    codec = codecs["lossless"]
    tokens, lengths, words, woff, wcnt = _random_chunks(codec, n, 700, n)
    _set_dec_env(monkeypatch, seg)
    groups = (n + 31) // 32
    modes = [(None, "split launch p8" if groups <= 32 else "split launch p4")]
    if groups <= 32:
        modes.append(("4", "split launch p4"))
    modes.append(("0", "launch"))
    for env, expect in modes:
        if env is None:
            monkeypatch.delenv("SC_HIP_DEC_SPLIT", raising=False)
        else:
            monkeypatch.setenv("SC_HIP_DEC_SPLIT", env)
        capfd.readouterr()
        back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
        log = capfd.readouterr().err
        assert f"leftover {n} {expect} steps" in log, log
        assert np.array_equal(back, tokens), env


def test_split_decode_not_used_beyond_64_groups(codecs, capfd, monkeypatch):
    """2,049 chunks make 65 groups, more than a split launch holds: one
    unsplit launch of 32-chunk workgroups."""
    codec = codecs["lossless"]
    tokens, lengths, words, woff, wcnt = _random_chunks(codec, 2049, 200, 3)
    _set_dec_env(monkeypatch, None)
    capfd.readouterr()
    back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
    log = capfd.readouterr().err
    assert "leftover 2049 launch" in log, log
    assert np.array_equal(back, tokens)


@pytest.mark.parametrize("lossy", [False, True])
def test_split_decode_matches_oracle(codecs, oracle_mod, oracle_models, lossy):
    """Split decode of 40 chunks (two groups, the second partial) with the
    lossless and the lossy model: every chunk's tokens equal the oracle's
    decode of the same words."""
    name = "lossy" if lossy else "lossless"
    codec = codecs[name]
    tokens, lengths, words, woff, wcnt = _random_chunks(codec, 40, 300, 11 + lossy)
    back, status, tok_off = _decode_direct(codec, words, woff, wcnt, lengths)
    assert not status.any()
    enc = [words[woff[c]:woff[c] + wcnt[c]].astype("<u4").tobytes() for c in range(len(lengths))]
    ref = oracle_mod.decompress_chunks(oracle_models[name], enc, lengths)
    for c in range(len(lengths)):
        assert np.array_equal(back[tok_off[c]:tok_off[c] + lengths[c]], ref[c]), c


def test_split_decode_corrupt_chunks(codecs, monkeypatch):
    """Corrupt chunks in both groups of a split decode over 64-step
    segments: each reports an invalid stream, every other chunk decodes."""
    codec = codecs["lossless"]
    tokens, lengths, words, woff, wcnt = _random_chunks(codec, 70, 400, 5)
    bad = [0, 33, 69]
    words = np.concatenate([words, np.full(2, 0xFFFFFFFF, np.uint32)])
    woff, wcnt = woff.copy(), wcnt.copy()
    woff[bad], wcnt[bad] = len(words) - 2, 2
    monkeypatch.setenv("SC_HIP_DEC_SEG", "64")
    back, status, tok_off = _decode_direct(codec, words, woff, wcnt, lengths)
    expect = np.zeros(len(lengths), np.int32)
    expect[bad] = 2   # SC_STATUS_INVALID_STREAM
    assert np.array_equal(status, expect)
    for i in range(len(lengths)):
        if i not in bad:
            s = slice(tok_off[i], tok_off[i] + lengths[i])
            assert np.array_equal(back[s], tokens[s]), i


@pytest.mark.parametrize("split", ["0", None])
def test_decode_of_garbage_and_damaged_chunks_matches_oracle(codecs, oracle_mod, oracle_models, monkeypatch, split):
    """Arbitrary words are a range-coded stream too: the decoder either
    reaches a quantile outside the table (an invalid stream) or returns
    tokens.  Over 600 chunks (lengths 1-150) of three kinds side by side
    -- valid streams, 0 to 8 random words, and valid streams cut short or
    with one word changed -- plus five streams invalid at their first step,
    each chunk's status, and the tokens of every chunk that decodes, equal
    the C oracle's; with the persistent decode
    (split "0") and with the default plan, a split decode for this batch."""
    import ctypes
    codec = codecs["lossless"]
    rng = np.random.default_rng(600 if split is None else 601)
    n = 600
    lengths = rng.integers(1, 151, n).astype(np.int32)
    tokens = rng.integers(0, 60, int(lengths.sum())).astype(np.uint8)
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    streams = [words[woff[i]:woff[i] + wcnt[i]].copy() for i in range(n)]
    kind = rng.integers(0, 3, n)
    for i in np.flatnonzero(kind == 1):
        streams[i] = rng.integers(0, 1 << 32, rng.integers(0, 9), dtype=np.uint64).astype(np.uint32)
    for i in np.flatnonzero(kind == 2):
        s = streams[i]
        if len(s) > 1 and rng.random() < 0.5:
            streams[i] = s[:rng.integers(0, len(s))]
        else:
            s[rng.integers(0, len(s))] ^= np.uint32(1 << int(rng.integers(0, 32)))
    # (almost any words decode: a point outside the coder's range is rare)
    # five streams whose first step's quantile is outside the table
    bad = rng.choice(n, 5, replace=False)
    for i in bad:
        streams[i] = np.array([0xFFFFFFFF, 0xFFFFFFFF, 7], np.uint32)
    cnt = np.array([len(s) for s in streams], np.int32)
    off = np.zeros(n, np.int64)
    np.cumsum(cnt[:-1], dtype=np.int64, out=off[1:])
    flat = np.concatenate(streams + [np.zeros(1, np.uint32)])
    if split is None:
        monkeypatch.delenv("SC_HIP_DEC_SPLIT", raising=False)
    else:
        monkeypatch.setenv("SC_HIP_DEC_SPLIT", split)
    back, status, tok_off = _decode_direct(codec, flat, off, cnt, lengths)
    # the oracle, every chunk's status (its Python wrapper raises on the first)
    om = oracle_models["lossless"]
    ref_tok = np.zeros(int(lengths.sum()), np.uint8)
    ref_status = np.zeros(n, np.int32)
    oracle_mod.lib().sco_decompress_chunks(ctypes.byref(om.c), om.lut, flat, off, cnt, lengths, n, ref_tok,
                                           tok_off, ref_status)
    assert (status[bad] == 2).all()
    assert np.array_equal(status != 0, ref_status != 0), np.flatnonzero((status != 0) != (ref_status != 0))
    assert set(np.unique(status)) <= {0, 2}   # SC_STATUS_OK, SC_STATUS_INVALID_STREAM
    for i in np.flatnonzero(status == 0):
        s = slice(tok_off[i], tok_off[i] + lengths[i])
        assert np.array_equal(back[s], ref_tok[s]), i


def test_split_decode_timeout_reports_status_and_redecodes_unsplit(codecs, monkeypatch):
    """With a spin limit of 0 polls (SC_HIP_DEC_SPIN=0; the default is
    2**18) every wait of a split decode gives up at once: every chunk of
    every group reports SC_STATUS_SYNC_TIMEOUT through the C ABI, also
    through later step segments, and the kernels end normally.
    decompress_flat then decodes the timed-out chunks again with unsplit
    launches (SC_DEC_OPT_NO_SPLIT), which never wait, and returns the input;
    the next decode with the default limit is correct as well.  A corrupt
    chunk among them is still reported as such."""
    codec = codecs["lossless"]
    tokens, lengths, words, woff, wcnt = _random_chunks(codec, 40, 300, 9)
    monkeypatch.setenv("SC_HIP_DEC_SPIN", "0")
    monkeypatch.setenv("SC_HIP_DEC_SEG", "64")
    _, status, _ = _decode_direct(codec, words, woff, wcnt, lengths)
    assert (status == 4).all(), status   # SC_STATUS_SYNC_TIMEOUT
    back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
    assert np.array_equal(back, tokens)
    bad = words.copy()
    c = int(np.argmax(lengths))
    bad[woff[c]:woff[c] + wcnt[c]] = 0xFFFFFFFF
    with pytest.raises(ValueError, match="invalid range stream"):
        codec.decompress_flat(bad, woff, wcnt, lengths)
    monkeypatch.delenv("SC_HIP_DEC_SPIN")
    back, _ = codec.decompress_flat(words, woff, wcnt, lengths)
    assert np.array_equal(back, tokens)


def test_mfma_burn_hook_computes_its_products():
    """The power-limit measurement hook (sc_mfma_burn_i8) really issues the
    MFMAs it is timed for: its accumulator sums equal the int8 matrix
    products of its fragments, restated with numpy (fragment j of A holds
    A_j[m][k] at lane m + 32*(k // 16), byte k % 16; B likewise with column n;
    lane l, register v of the 32x32 result holds row 8*(v//4) + 4*(l//32) +
    v%4, column l % 32)."""
    from sigcomp_amd import _hip
    L = _hip.lib()
    rng = np.random.default_rng(8)
    ops = rng.integers(-128, 128, 8192).astype(np.int8)
    iters, groups = 2, 3
    out = torch.zeros(groups * 256 * 16, dtype=torch.int32, device="cuda")
    d_ops = torch.from_numpy(ops).cuda()
    _hip.check(L.sc_mfma_burn_i8(d_ops.data_ptr(), iters, groups, out.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream))
    got = out.cpu().numpy().reshape(groups, 4, 64, 16)
    frag = ops.reshape(512, 16).astype(np.int64)
    row = np.arange(32)[:, None]      # A: m, B: k
    col = np.arange(32)[None, :]      # A: k, B: n
    A = [frag[j * 64 + row + 32 * (col // 16), col % 16] for j in range(4)]          # A_j[m][k]
    B = [frag[256 + j * 64 + col + 32 * (row // 16), row % 16] for j in range(4)]    # B_j[k][n]
    D = np.zeros((32, 32), np.int64)
    for i2 in range(4):
        for j in range(8):
            D += A[j & 3] @ B[(j + i2) & 3] + A[(j + 1) & 3] @ B[(j + 2 + i2) & 3]
    D = (D * iters).astype(np.int64)
    lane = np.arange(64)[:, None]
    v = np.arange(16)[None, :]
    exp = D[8 * (v // 4) + 4 * (lane // 32) + v % 4, lane % 32].astype(np.int32)
    assert all(np.array_equal(got[g, w], exp) for g in range(groups) for w in range(4))


def test_pipelined_read_compression_matches_single_batch(codecs, oracle_mod, oracle_models, monkeypatch):
    """batch_inference_reads compresses reads in pipelined batches of whole
    reads (compress_reads_batches): with batches of ~8 chunks (many batches,
    reads of 0..9 chunks, empty reads at a batch edge) every payload equals
    the single-batch run's and the oracle's framing of its chunks, and the
    payloads decode back."""
    from framing_ref import chunk_views, frame
    from sigcomp_amd import quant_mlp_export
    rng = np.random.default_rng(21)
    lens = rng.integers(0, 9 * 2048, 40)
    lens[[3, 4, 17]] = 0
    reads = [rng.integers(0, 70, n).astype(np.uint8) for n in lens]
    codec = codecs["lossless"]
    one = codec.batch_inference_reads(list_of_reads=reads, batch_size=20480)
    monkeypatch.setattr(quant_mlp_export, "_MIN_PIPE_CHUNKS", 8)
    many = codec.batch_inference_reads(list_of_reads=reads, batch_size=1)
    assert many == one
    for r in (0, 3, 5, 39):
        assert many[r] == frame(oracle_mod.compress_chunks(oracle_models["lossless"], chunk_views(reads[r], 2048)))
    back = codec.batch_inference_reads(list_of_compressed_reads=many, list_of_lengths=[int(n) for n in lens])
    assert all(np.array_equal(a, b) for a, b in zip(reads, back))
