"""GPU parity of the generic path: model architectures other than the
bundled one (the reference's --dim / --num-dec-layers / --window-size,
main.py:1881-1885, read from an archive's header, main.py:1086-1094), run by
the padded-fragment kernels of sc_gen.hip, bit-exact against the oracle
(whose MLP, coder and drivers take any shape)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

# (window, emb_dim, hidden, n_hidden): widths that are not multiples of 32,
# a 16-token window with the bundled layer widths, a single linear layer
ARCHS = {"odd": (5, 24, 80, 3), "win16": (16, 128, 512, 2), "one_layer": (8, 16, 64, 0)}


@pytest.fixture(scope="module", params=sorted(ARCHS))
def arch(request):
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from sigcomp_amd.model_io import random_int_model
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    w, e, h, nh = ARCHS[request.param]
    m = random_int_model(seed=11 + nh, window=w, emb_dim=e, hidden=h, n_hidden=nh, per_channel=True)
    return request.param, m, QuantMLPCompression(chunk_len=300, gpu=0, model=m)


def test_generic_core_selected(arch):
    assert arch[2].hip.core == 3


@pytest.mark.parametrize("rows", [1, 77, 300])
def test_generic_forward_matches_oracle(arch, oracle_mod, rows):
    _, m, codec = arch
    rng = np.random.default_rng(rows)
    ctx = rng.integers(0, 257, (rows, m.window)).astype(np.int64)
    om = oracle_mod.OracleModel(m)
    ref = oracle_mod.mlp_forward(om, ctx)
    got = codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "logits").cpu().numpy()
    assert np.array_equal(got, ref)
    cdf = codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "cdf").cpu().numpy()
    assert np.array_equal(cdf.astype(np.int64), oracle_mod.logits_to_cdf(ref, m.exp_lut))


def test_generic_bad_token_raises(arch):
    _, m, codec = arch
    ctx = np.zeros((3, m.window), np.int64)
    ctx[1, 0] = 257
    with pytest.raises(ValueError):
        codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "logits")


def test_generic_compress_decompress_match_oracle(arch, oracle_mod):
    _, m, codec = arch
    rng = np.random.default_rng(5)
    lengths = [1, 5, 63, 64, 65, 129, 300, 0, 211]
    chunks = [rng.integers(0, 40, n).astype(np.uint8) for n in lengths]
    got = codec.compress_chunks(chunks)
    ref = oracle_mod.compress_chunks(oracle_mod.OracleModel(m), chunks)
    assert got == ref
    back = codec.decompress_chunks(got, lengths)
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))


def test_generic_abi_decode_without_host_lengths_and_corrupt_stream(arch):
    """sc_decompress_chunks on the generic path through the C ABI: plan from
    device lengths, a corrupt stream flagged (and only it)."""
    from test_gpu_parity import _decode_direct
    _, m, codec = arch
    rng = np.random.default_rng(9)
    lengths = rng.integers(1, 250, 40).astype(np.int32)
    tokens = rng.integers(0, 50, int(lengths.sum())).astype(np.uint8)
    words, woff, wcnt = codec.compress_flat(tokens, lengths)
    words = np.concatenate([words, np.full(2, 0xFFFFFFFF, np.uint32)])
    woff, wcnt = woff.copy(), wcnt.copy()
    woff[7], wcnt[7] = len(words) - 2, 2
    back, status, tok_off = _decode_direct(codec, words, woff, wcnt, lengths, host_lengths=False)
    expect = np.zeros(40, np.int32)
    expect[7] = 2
    assert np.array_equal(status, expect)
    for i in range(40):
        if i != 7:
            assert np.array_equal(back[tok_off[i]:tok_off[i] + lengths[i]], tokens[tok_off[i]:tok_off[i] + lengths[i]])


def test_generic_reads_round_trip(arch, oracle_mod):
    """batch_inference_reads (pipelined compression, framing, parse, decode)
    with chunk_len 300 and reads of 0 .. 4 chunks."""
    from framing_ref import chunk_views, frame
    _, m, codec = arch
    rng = np.random.default_rng(4)
    reads = [rng.integers(0, 60, n).astype(np.uint8) for n in (0, 1, 299, 300, 301, 1111)]
    framed = codec.batch_inference_reads(list_of_reads=reads, batch_size=16)
    om = oracle_mod.OracleModel(m)
    assert framed == [frame(oracle_mod.compress_chunks(om, chunk_views(r, 300))) for r in reads]
    back = codec.batch_inference_reads(list_of_compressed_reads=framed, list_of_lengths=[len(r) for r in reads])
    assert all(np.array_equal(a, b) for a, b in zip(reads, back))


def test_static_entry_rejects_generic_model(arch):
    from sigcomp_amd import _hip
    _, m, codec = arch
    L = _hip.lib()
    dummy = torch.zeros(8, dtype=torch.int64, device="cuda")
    p = dummy.data_ptr()
    rc = L.sc_decompress_chunks_static(codec.hip.handle, p, p, p, p, 1, p, p, p, None,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"bundled architecture" in L.sc_last_error()


def test_generic_model_loaded_by_dims(tmp_path, oracle_mod):
    """An integer export of another architecture loads through
    QuantMLPCompression's dim / num_dec_layers / window_size arguments (the
    reference's constructor, main.py:189-225) and codes like the oracle."""
    from sigcomp_amd import model_io
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    m = model_io.random_int_model(seed=4, window=12, emb_dim=32, hidden=128, n_hidden=2)   # dim 64
    f = tmp_path / "small.npz"
    model_io.export_npz(m, f)
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model_path=str(f), dim=64, num_dec_layers=2, window_size=12)
    assert codec.hip.core == 3 and codec.window_size == 12
    chunk = np.random.default_rng(1).integers(0, 30, 700).astype(np.uint8)
    assert codec.compress_chunks([chunk]) == oracle_mod.compress_chunks(oracle_mod.OracleModel(m), [chunk])


def test_generic_wide_model_batches_within_its_scratch_bound(oracle_mod):
    """A model 524,288 inputs wide (window 512 x 1,024-wide embedding): the
    generic path's scratch per call is bounded (1 GiB), so its batches
    shrink to 960 rows (forward, decode) and 7 tiles of 128 steps
    (compress) instead of 65,536 rows, which would need 64 GiB.  Forward on
    2,100 rows (three batches) and compress / decompress of chunks spanning
    two compress batches, bit-exact against the oracle."""
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from sigcomp_amd.model_io import random_int_model
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    m = random_int_model(seed=21, window=512, emb_dim=1024, hidden=64, n_hidden=1, per_channel=True)
    codec = QuantMLPCompression(chunk_len=1000, gpu=0, model=m)
    assert codec.hip.core == 3
    om = oracle_mod.OracleModel(m)
    rng = np.random.default_rng(3)
    ctx = rng.integers(0, 257, (2100, m.window)).astype(np.int64)
    got = codec.hip.forward_windows(torch.from_numpy(ctx).cuda(), "logits").cpu().numpy()
    assert np.array_equal(got, oracle_mod.mlp_forward(om, ctx))
    chunks = [rng.integers(0, 40, n).astype(np.uint8) for n in (130, 7, 1000)]
    comp = codec.compress_chunks(chunks)
    assert comp == oracle_mod.compress_chunks(om, chunks)
    back = codec.decompress_chunks(comp, [len(c) for c in chunks])
    assert all(np.array_equal(a, b) for a, b in zip(chunks, back))
