"""GPU parity at the benchmark configurations' full sizes, bit-exact.

* c2 shape: the explicit-context MLP kernel with several 128-row tiles per
  workgroup (its grid-stride tile loop, context reuse across tiles), both
  output modes, against the oracle on first and last tiles of several
  workgroups;
* c3 and c5: every chunk of the whole workload through compress_flat /
  decompress_flat (the decode plan's full-wave launches, every 256-step
  segment, the leftover chunks), lossless round trip of every chunk and the
  chunk bytes of >= 64 chunks against the oracle: the longest chunks, the
  last full-wave launch's last rows, the leftover chunks and random ones;
* GPUBitExactMLPDecoder.forward (teacher-forced windows padded with the
  first target, quant_mlp_export.py:122-130) against the oracle;
* the SIG2 record path: golden reads -> split -> GPU compress -> records ->
  archive bytes -> scan -> GPU decompress -> reassembly.
"""

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _n_cu():
    return torch.cuda.get_device_properties(0).multi_processor_count


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    return torch.device("cuda:0")


@pytest.mark.parametrize("mode", ["logits", "cdf"])
def test_mlp_context_several_tiles_per_workgroup(gpu, oracle_mod, mode):
    """2 x n_cu x 128 + 77 rows of the c2 model (per-channel constants): the
    grid is one workgroup per CU, so workgroup b runs tiles b, b + n_cu,
    b + 2 n_cu (the last one partial for b = 0)."""
    from sigcomp_amd import signal, synth
    from sigcomp_amd.model_io import random_int_model
    from sigcomp_amd.quant_mlp_export import HipModel
    n_cu = _n_cu()
    rows = 2 * n_cu * 128 + 77
    m = random_int_model(seed=2, per_channel=True)
    hm = HipModel(m, gpu)
    toks = np.concatenate([signal.split_signal(r)[1] for r in synth.synth_reads(8, 202, synth.DNA)]).astype(np.int64)
    starts = np.random.default_rng(3).integers(-63, len(toks) - 64, rows)
    idx = starts[:, None] + np.arange(64)[None, :]
    ctx = np.where(idx < 0, 256, toks[np.clip(idx, 0, None)])
    got = hm.forward_windows(torch.from_numpy(ctx).to(gpu), mode).cpu().numpy()
    n_tiles = -(-rows // 128)
    om = oracle_mod.OracleModel(m)
    checked = 0
    for b in (0, 1, n_cu // 2, n_cu - 1):
        for k in range(3):
            tile = b + k * n_cu
            if tile >= n_tiles:
                continue
            sl = slice(tile * 128, min(rows, tile * 128 + 128))
            ref = oracle_mod.mlp_forward(om, ctx[sl])
            if mode == "cdf":
                ref = oracle_mod.logits_to_cdf(ref, m.exp_lut)
            assert np.array_equal(got[sl].astype(np.int64), ref.astype(np.int64)), (b, k)
            checked += 1
    assert checked == 9   # workgroup 0 runs three tiles (its third one partial), the others two


def test_c2_full_launch_against_oracle(gpu, oracle_mod):
    """The c2 launch at its full size: 1,048,576 context rows of the c2 model
    (per-channel constants, the bench's rows) -> int32 CDF tables in one
    launch, one workgroup per CU, so workgroup b runs the 32 tiles b, b +
    n_cu, ..., b + 31 n_cu.  Its first, middle and last tiles (b, b + 16
    n_cu, b + 31 n_cu) of four workgroups against the oracle."""
    from sigcomp_amd import signal, synth
    from sigcomp_amd.model_io import random_int_model
    from sigcomp_amd.quant_mlp_export import HipModel
    n_cu = _n_cu()
    rows = 1 << 20
    m = random_int_model(seed=2, per_channel=True)
    hm = HipModel(m, gpu)
    toks = np.concatenate([signal.split_signal(r)[1] for r in synth.synth_reads(64, 202, synth.DNA)])
    toks = toks.astype(np.int64)
    starts = np.random.default_rng(3).integers(-63, len(toks) - 64, rows)
    idx = starts[:, None] + np.arange(64)[None, :]
    ctx = np.where(idx < 0, 256, toks[np.clip(idx, 0, None)])
    out = hm.forward_windows(torch.from_numpy(ctx).to(gpu), "cdf")
    n_tiles = rows // 128
    om = oracle_mod.OracleModel(m)
    tiles = sorted({b + k * n_cu for b in (0, 1, n_cu // 2, n_cu - 1) for k in (0, 16, 31) if b + k * n_cu < n_tiles})
    assert len(tiles) == 12
    for tile in tiles:
        sl = slice(tile * 128, tile * 128 + 128)
        ref = oracle_mod.logits_to_cdf(oracle_mod.mlp_forward(om, ctx[sl]), m.exp_lut)
        assert np.array_equal(out[sl].cpu().numpy().astype(np.int64), ref.astype(np.int64)), tile


def test_c1_full_config_split_decode_every_chunk_against_oracle(gpu, oracle_mod, capfd, monkeypatch):
    """Config c1 (BASELINE.json's CPU case, 64 reads, 675 chunks) through the
    HIP path: compress_flat, then decompress_flat, whose single launch of
    22 groups of 32 chunks runs split (8 workgroups per group sharing layer
    0, one exchange per step) over eight 256-step segments.  Every chunk's
    bytes equal the oracle's and every decoded chunk equals its input."""
    from sigcomp_amd import model_io, signal, synth
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    cfg = synth.CONFIGS["c1"]
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model_path=model_io.DEFAULT_QUANT_LOSSLESS_MODEL_PATH)
    small = signal.reads_tokens(signal.split_reads(synth.config_reads("c1"), cfg["lsb"]))
    chunks = [s[i:i + 2048] for s in small for i in range(0, len(s), 2048)]
    lengths = np.array([len(c) for c in chunks], np.int32)
    tokens = np.concatenate(chunks)
    print(f"[c1] {len(chunks)} chunks, {len(tokens)} tokens", flush=True)
    assert len(chunks) < 32 * _n_cu()
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    capfd.readouterr()
    monkeypatch.setenv("SC_HIP_DEC_LOG", "1")
    monkeypatch.delenv("SC_HIP_DEC_SEG", raising=False)
    monkeypatch.delenv("SC_HIP_DEC_SPLIT", raising=False)
    back, tok_off = codec.decompress_flat(words, woff, wcnt, lengths)
    log = capfd.readouterr().err
    assert "split launch p8" in log and "seg 256" in log, log
    assert int(lengths.max()) == 2048
    assert np.array_equal(back, tokens)
    ref = oracle_mod.compress_chunks(oracle_mod.OracleModel(codec.model), chunks)
    for i in range(len(chunks)):
        assert words[woff[i]:woff[i] + wcnt[i]].tobytes() == ref[i], i


def _oracle_pick(lengths, n_cu, rng):
    """Chunk indices (in the caller's order) to check against the oracle:
    with chunks sorted longest first (as decompress_flat sorts them), the 16
    longest, the 24 rows before the full-wave boundary (the last full-wave
    launch's last rows, which the leftover chunks follow), up to 24 leftover
    chunks and random ones (at least 16, 72 chunks in all)."""
    order = np.argsort(-lengths, kind="stable")
    full = (len(lengths) // (32 * n_cu)) * 32 * n_cu
    pos = set(range(16)) | set(range(max(0, full - 24), full)) | set(range(full, min(len(lengths), full + 24)))
    want = max(72, len(pos) + 16)              # random ones: at least 16, 72 chunks in all
    for p in rng.permutation(len(lengths)):
        if len(pos) >= want:
            break
        pos.add(int(p))
    return np.array(sorted(order[sorted(pos)]))


@pytest.mark.parametrize("cfg_name", ["c3", "c5"])
def test_full_config_round_trip_and_oracle_bytes(gpu, oracle_mod, capfd, monkeypatch, cfg_name):
    from sigcomp_amd import model_io, signal, synth
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    cfg = synth.CONFIGS[cfg_name]
    path = (model_io.DEFAULT_QUANT_LOSSY_MODEL_PATH if cfg["model"] == "lossy"
            else model_io.DEFAULT_QUANT_LOSSLESS_MODEL_PATH)
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model_path=path)
    small = signal.reads_tokens(signal.split_reads(synth.config_reads(cfg_name), cfg["lsb"]))
    chunks = [s[i:i + 2048] for s in small for i in range(0, len(s), 2048)]
    lengths = np.array([len(c) for c in chunks], np.int32)
    tokens = np.concatenate(chunks)
    print(f"[{cfg_name}] {len(chunks)} chunks, {len(tokens)} tokens", flush=True)
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    capfd.readouterr()
    monkeypatch.setenv("SC_HIP_DEC_LOG", "1")
    monkeypatch.delenv("SC_HIP_DEC_SEG", raising=False)
    back, tok_off = codec.decompress_flat(words, woff, wcnt, lengths)
    log = capfd.readouterr().err
    import re
    m = re.search(r"steps (\d+) seg 256", log)        # at least eight 256-step launches
    assert m and int(m.group(1)) >= 2048, log
    assert np.array_equal(back, tokens)
    pick = _oracle_pick(lengths, _n_cu(), np.random.default_rng(11))
    assert len(pick) >= 64 and int(lengths[pick].max()) == 2048
    ref = oracle_mod.compress_chunks(oracle_mod.OracleModel(codec.model), [chunks[i] for i in pick])
    for j, i in enumerate(pick):
        assert words[woff[i]:woff[i] + wcnt[i]].tobytes() == ref[j], i


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_decoder_forward_matches_oracle(gpu, oracle_mod, int_models, oracle_models, name):
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model=int_models[name])
    rng = np.random.default_rng(5)
    B, L, W = 3, 150, 64
    targets = rng.integers(0, 256, (B, L)).astype(np.int64)
    targets[1, 0] = 255
    got = codec.gpu_engine.forward(torch.from_numpy(targets).to(gpu)).cpu().numpy()
    assert got.shape == (B, L, 256) and got.dtype == np.int8
    for b in range(B):
        # window j = (W - 1 copies of the first target + targets)[j : j + W]
        padded = np.concatenate([np.full(W - 1, targets[b, 0]), targets[b]])
        windows = np.stack([padded[j:j + W] for j in range(L)])
        assert np.array_equal(got[b], oracle_mod.mlp_forward(oracle_models[name], windows)), b


@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_sig2_record_path_on_the_gpu(gpu, oracle_mod, int_models, name):
    """Golden reads -> split -> GPU compress (batch_inference_reads) -> SIG2
    records -> archive -> scan -> GPU decompress -> reassembly: the records'
    s-blobs are the reference's payloads and the samples come back (through
    the lossy transform for lsb > 0).  The large values and gaps are
    Rice-coded by sigcomp_amd.rice (this library's own blob format:
    fast-rice 0.1.0's is third-party)."""
    import signal_ref
    from sigcomp_amd import rice, sig2, signal
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    z = np.load(GOLDEN / "e2e_reads.npz")
    lsb = int(z[f"{name}_lsb"])
    reads = [z[f"{name}_read{i}_signal"] for i in range(int(z[f"{name}_nreads"]))]
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model=int_models[name])
    sp = signal.split_reads(reads, lsb)
    small = signal.reads_tokens(sp)
    s_bytes = codec.batch_inference_reads(list_of_reads=small, batch_size=20480)
    la, lg = rice.encode_split(sp)
    pod = np.zeros(len(reads), sig2.POD5_DTYPE)
    pod["read_id"] = (np.arange(len(reads))[:, None] * 7 + np.arange(16)[None, :]) % 256
    recs, _ = sig2.write_records(sig2.POD5, sp["sig0"], sp["len"], sp["n_small"], s_bytes, la, lg, pod5=pod)
    archive = sig2.header_bytes(b"header") + recs
    _, start = sig2.split_header(archive)
    sc = sig2.scan_records(archive, start, len(reads), sig2.POD5)
    blobs = [sig2.blob(sc, i, 0) for i in range(len(reads))]
    for i in range(len(reads)):
        assert blobs[i] == z[f"{name}_read{i}_sbytes"].tobytes(), i
    back = codec.batch_inference_reads(list_of_compressed_reads=blobs,
                                       list_of_lengths=[int(x) for x in sc["n_small"]], batch_size=20480)
    # c_large = N - 1 - c_small (main.py:562)
    n_large = sc["n_samples"].astype(np.int64) - 1 - sc["n_small"].astype(np.int64)
    assert np.array_equal(n_large, sp["n_large"])
    large_adj, large_gap, large_off = rice.decode_split([sig2.blob(sc, i, 1) for i in range(len(reads))],
                                                        [sig2.blob(sc, i, 2) for i in range(len(reads))], n_large)
    split = {"sig0": sc["sig0"], "len": sc["n_samples"].astype(np.int64), "small_off": sp["small_off"],
             "n_small": sc["n_small"].astype(np.int64), "large_adj": large_adj, "large_gap": large_gap,
             "large_off": large_off, "n_large": n_large}
    out = signal.reassemble_reads(split, small=np.concatenate(back), lsb=lsb)
    for r, o in zip(reads, out):
        want = signal_ref.lossy_decode(signal_ref.prepare_signal(r, lsb), lsb) if lsb else r
        assert np.array_equal(o, want)
