"""Pins the CPU oracle (oracle/sc_oracle.c) before anything is checked against it.

Golden fixtures come from the reference implementation itself
(tests/golden/make_golden.py); the remaining checks are closed forms,
invariants and brute force chosen so that a dropped term, wrong sign,
wrong rounding or wrong index fails.
"""

import json
import os
from fractions import Fraction

import numpy as np
import pytest

from conftest import GOLDEN, REFERENCE, REPO


# ---------------------------------------------------------------- requant / GEMM

def test_requantize_closed_form(oracle_mod):
    rq = oracle_mod.requantize
    # floor (not round) arithmetic shift on negative values
    assert rq(-1, 0, 1 << 30, 31, 0) == -1
    assert rq(-3, 0, 1 << 30, 31, 0) == -2
    assert rq(3, 0, 1 << 30, 31, 0) == 1
    # relu clamps at 0, non-relu at -128; both clamp at 127
    assert rq(-1000, 0, 1 << 31, 31, 1) == 0
    assert rq(-1000, 0, 1 << 31, 31, 0) == -128
    assert rq(1000, 0, 1 << 31, 31, 0) == 127
    # M0 == 2**31 is a legal multiplier (identity at shift 31)
    assert rq(77, 0, 1 << 31, 31, 0) == 77
    # the bias add wraps in int32 before the int64 product
    assert rq(2**31 - 1, 1, 1 << 31, 62, 0) == -1     # wraps to -2**31 -> -2**62 >> 62
    assert rq(5, 7, 3 << 29, 33, 0) == (12 * (3 << 29)) >> 33
    # shift 0 and 63
    assert rq(1, 0, 1, 0, 0) == 1
    assert rq(-5, 0, 1 << 31, 63, 0) == -1


def _int_mm_patterns():
    """Known-answer patterns of the reference's _int_mm conformance probe
    (cpu_int_inference.py:28-37)."""
    values = np.array([-128, 127, -127, 126, 0, 1, -1, 64], dtype=np.int8)
    for width in (64, 8192):
        x = np.resize(values, (33, width)).copy()
        x[0, :] = -128
        x[1, :] = 127
        w = np.resize(values[::-1], (64, width)).copy()
        w[0, :] = -128
        w[1, :] = 127
        w[1, 0] = 126
        yield x, w


def test_linear_int_mm_conformance_patterns(oracle_mod):
    from sigcomp_amd.model_io import make_layer
    for x, w in _int_mm_patterns():
        expected_acc = x.astype(np.int64) @ w.astype(np.int64).T
        # identity requant (M0=2**31, shift=31+s) exposes the accumulator's high bits
        for s in (0, 8, 16):
            layer = make_layer(w, np.zeros(64, np.int32), 1 << 31, 31 + s, False)
            got = oracle_mod.linear(x, layer)
            exp = np.clip(expected_acc >> s, -128, 127)
            for rows in (1, 17, 33):
                assert np.array_equal(got[:rows], exp[:rows])


def test_linear_matches_torch_int_mm(oracle_mod):
    torch = pytest.importorskip("torch")
    from sigcomp_amd.model_io import make_layer
    rng = np.random.default_rng(5)
    x = rng.integers(-128, 128, (37, 512)).astype(np.int8)
    w = rng.integers(-128, 128, (96, 512)).astype(np.int8)
    b = rng.integers(-50000, 50000, 96).astype(np.int32)
    m0 = rng.integers(1 << 30, 1 << 31, 96)
    sh = rng.integers(36, 42, 96).astype(np.int32)
    acc = torch._int_mm(torch.from_numpy(x), torch.from_numpy(w).t().contiguous()).numpy()
    biased = (acc.astype(np.int64) + b).astype(np.int32).astype(np.int64)
    exp = np.clip((biased * m0) >> sh, 0, 127).astype(np.int8)
    got = oracle_mod.linear(x, make_layer(w, b, m0, sh, True))
    assert np.array_equal(got, exp)


# ---------------------------------------------------------------- model loader

def test_loader_matches_reference_constants(int_models):
    from sigcomp_amd.model_io import build_integer_exp_lut
    import hashlib
    consts = json.loads((GOLDEN / "constants.json").read_text())
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    for name, model in int_models.items():
        c = consts[name]
        assert model.output_scale == c["output_scale"]
        assert sha(model.emb) == c["emb_sha256"]
        assert len(model.layers) == len(c["layers"])
        for layer, cl in zip(model.layers, c["layers"]):
            assert int(layer.m0[0]) == cl["m0"] and np.all(layer.m0 == cl["m0"])
            assert int(layer.shift[0]) == cl["shift"] and np.all(layer.shift == cl["shift"])
            assert layer.relu == cl["relu"]
            assert sha(layer.weight) == cl["weight_sha256"]
            assert sha(layer.bias) == cl["bias_sha256"]
        assert model.exp_lut.tolist() == c["exp_lut"]
        assert build_integer_exp_lut(model.output_scale).tolist() == c["exp_lut"]


def test_exp_lut_invariants(int_models):
    lossless, lossy = int_models["lossless"].exp_lut, int_models["lossy"].exp_lut
    assert lossless[0] == 1 << 38 and lossy[0] == 1 << 38
    assert lossless[255] == 429070 and (lossless > 0).sum() == 256
    assert (lossy > 0).sum() == 66 and lossy[255] == 0
    assert np.all(np.diff(lossless) <= 0)
    # float check of the closed form (the decimal evaluation is exact to 1 ulp of 2**38)
    s = int_models["lossless"].output_scale
    approx = np.exp(-np.arange(256) * s) * 2.0**38
    assert np.all(np.abs(approx - lossless) <= 2)


@pytest.mark.skipif(not (REFERENCE / "sigcomp" / "pretrained_models" / "lossless.pth").exists(),
                    reason="reference checkpoints not present")
def test_pth_and_npz_exports_agree(int_models):
    from sigcomp_amd.model_io import load_int_model
    m = load_int_model(REFERENCE / "sigcomp" / "pretrained_models" / "lossless.pth")
    n = int_models["lossless"]
    assert np.array_equal(m.emb, n.emb) and np.array_equal(m.exp_lut, n.exp_lut)
    for a, b in zip(m.layers, n.layers):
        assert np.array_equal(a.weight, b.weight) and np.array_equal(a.bias, b.bias)
        assert np.array_equal(a.m0, b.m0) and np.array_equal(a.shift, b.shift)


# ---------------------------------------------------------------- MLP

@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_mlp_matches_reference_logits(oracle_mod, oracle_models, name):
    z = np.load(GOLDEN / f"mlp_{name}.npz")
    got = oracle_mod.mlp_forward(oracle_models[name], z["ctx"])
    assert np.array_equal(got, z["logits"])


def test_vnni_and_portable_mlp_agree(oracle_mod, tmp_path):
    """The oracle's AVX-512 VNNI dot products (offset activations, row sums
    taken off) give the portable C path's logits, bit for bit, on both
    bundled models and a random per-channel model, with batches that leave
    partial 4-row groups and blocks."""
    import subprocess
    import sys
    if not oracle_mod.uses_vnni():
        pytest.skip("host CPU has no AVX-512 VNNI")
    script = tmp_path / "mlp.py"
    script.write_text(
        "import sys, numpy as np\n"
        f"sys.path[:0] = [{str(REPO)!r}, {str(REPO / 'oracle')!r}]\n"
        "import oracle\n"
        "from sigcomp_amd import model_io\n"
        "ms = [model_io.load_int_model(model_io.DEFAULT_QUANT_LOSSLESS_MODEL_PATH),\n"
        "      model_io.load_int_model(model_io.DEFAULT_QUANT_LOSSY_MODEL_PATH),\n"
        "      model_io.random_int_model(seed=9, per_channel=True)]\n"
        "rng = np.random.default_rng(2)\n"
        "out = []\n"
        "for m in ms:\n"
        "    for rows in (1, 6, 203):\n"
        "        ctx = rng.integers(0, 257, (rows, 64))\n"
        "        out.append(oracle.mlp_forward(oracle.OracleModel(m), ctx))\n"
        "np.savez(sys.argv[1], *out, vnni=oracle.uses_vnni())\n")
    res = {}
    for flag in ("0", "1"):
        f = tmp_path / f"out{flag}.npz"
        env = dict(os.environ, SCO_NO_VNNI=flag)
        subprocess.run([sys.executable, str(script), str(f)], check=True, env=env)
        res[flag] = np.load(f)
    assert bool(res["0"]["vnni"]) and not bool(res["1"]["vnni"])
    for k in res["0"].files:
        if k != "vnni":
            assert np.array_equal(res["0"][k], res["1"][k]), k


def test_mlp_rejects_out_of_range_tokens(oracle_mod, oracle_models):
    ctx = np.full((2, 64), 256, np.int32)
    ctx[1, 5] = 257
    with pytest.raises(ValueError):
        oracle_mod.mlp_forward(oracle_models["lossless"], ctx)


# ---------------------------------------------------------------- logits -> CDF

@pytest.mark.parametrize("name", ["lossless", "lossy"])
def test_cdf_matches_reference(oracle_mod, int_models, name):
    z = np.load(GOLDEN / f"cdf_{name}.npz")
    got = oracle_mod.logits_to_cdf(z["logits"], int_models[name].exp_lut)
    assert np.array_equal(got, z["cdf"])


def _cdf_by_fractions(logits, lut):
    """Independent exact-rational statement of the frequency rule."""
    m = int(logits.max())
    u = [int(lut[m - int(v)]) for v in logits]
    T = sum(u)
    f = [max(int(Fraction(x * (1 << 24), T)), 1) for x in u]   # floor for x >= 0
    i = f.index(max(f))
    f[i] -= sum(f) - (1 << 24)
    return np.concatenate([[0], np.cumsum(f)])


def test_cdf_invariants_and_special_cases(oracle_mod, int_models):
    rng = np.random.default_rng(1)
    for name in ("lossless", "lossy"):
        lut = int_models[name].exp_lut
        rows = rng.integers(-128, 128, (64, 256)).astype(np.int8)
        cdf = oracle_mod.logits_to_cdf(rows, lut)
        f = np.diff(cdf, axis=1)
        assert np.all(cdf[:, 0] == 0) and np.all(cdf[:, -1] == 1 << 24)
        assert np.all(f >= 1)
        for r in range(8):
            assert np.array_equal(cdf[r], _cdf_by_fractions(rows[r], lut))
        # all-equal logits: 2**24 / 256 each, no correction
        eq = oracle_mod.logits_to_cdf(np.zeros((1, 256), np.int8), lut)
        assert np.all(np.diff(eq[0]) == 65536)
    # single dominant logit under the lossy LUT: 255 entries clamp to 1
    one = np.full((1, 256), -128, np.int8)
    one[0, 9] = 127
    f = np.diff(oracle_mod.logits_to_cdf(one, int_models["lossy"].exp_lut)[0])
    assert f[9] == (1 << 24) - 255 and np.all(np.delete(f, 9) == 1)


def test_cdf_correction_goes_to_first_argmax(oracle_mod, int_models):
    lut = int_models["lossless"].exp_lut
    row = np.full((1, 256), -60, np.int8)
    row[0, 40] = row[0, 41] = 100          # tie between 40 and 41
    f = np.diff(oracle_mod.logits_to_cdf(row, lut)[0])
    m = int(row.max())
    u = lut[m - row[0].astype(np.int64)]
    raw = np.maximum((u * (1 << 24)) // u.sum(), 1)
    assert f[41] == raw[41] and f[40] == raw[40] - (raw.sum() - (1 << 24))


# ---------------------------------------------------------------- range coder

def _streams():
    z = np.load(GOLDEN / "coder_streams.npz")
    keys = sorted({k.rsplit("_", 1)[0] for k in z.files})
    return z, keys


def test_encoder_matches_reference_words(oracle_mod, int_models):
    z, keys = _streams()
    assert len(keys) == 12
    for key in keys:
        lut = int_models[key.split("_")[0]].exp_lut
        words = oracle_mod.encode_stream(z[f"{key}_logits"], z[f"{key}_symbols"], lut)
        assert np.array_equal(words, z[f"{key}_words"]), key


def test_decoder_matches_reference_symbols(oracle_mod, int_models):
    z, keys = _streams()
    for key in keys:
        lut = int_models[key.split("_")[0]].exp_lut
        sym = oracle_mod.decode_stream(z[f"{key}_words"], z[f"{key}_logits"], lut)
        assert np.array_equal(sym, z[f"{key}_decoded"]), key
        assert np.array_equal(sym, z[f"{key}_symbols"]), key


def _interval_check(words, cdfs, symbols):
    """The sealed code value must lie inside the final coding interval.

    Exact-rational model of the coder: each step narrows [low, low+rng) by
    scale = floor(rng / 2**24) (the coder's integer quantisation) with the
    renormalisation only changing the scale of representation.  The emitted
    words, read as a base-2**32 fraction, must fall in the final interval.
    """
    low, rng, bits = 0, (1 << 64) - 1, 64
    for cdf, s in zip(cdfs, symbols):
        scale = rng >> 24
        low += scale * int(cdf[s])
        rng = scale * int(cdf[s + 1] - cdf[s])
        if rng < (1 << 32):
            low <<= 32
            rng <<= 32
            bits += 32
    value = 0
    n = len(words)
    for w in words:
        value = (value << 32) | int(w)
    # align the code value to `bits` bits
    total = 32 * n
    value = value << (bits - total) if bits >= total else value >> (total - bits)
    return low <= value < low + rng


def test_encoder_interval_property(oracle_mod, int_models):
    rng = np.random.default_rng(7)
    for name in ("lossless", "lossy"):
        lut = int_models[name].exp_lut
        for length in (1, 2, 3, 17, 250):
            lg = rng.integers(-128, 128, (length, 256)).astype(np.int8)
            sym = rng.integers(0, 256, length)
            words = oracle_mod.encode_stream(lg, sym, lut)
            assert len(words) <= length + 2
            cdfs = oracle_mod.logits_to_cdf(lg, lut)
            assert _interval_check(words, cdfs, sym)


def test_round_trip_random_streams(oracle_mod, int_models):
    rng = np.random.default_rng(3)
    lut = int_models["lossy"].exp_lut
    for length in (1, 2, 5, 64, 500):
        lg = rng.integers(-128, 128, (length, 256)).astype(np.int8)
        sym = rng.integers(0, 256, length)
        words = oracle_mod.encode_stream(lg, sym, lut)
        assert np.array_equal(oracle_mod.decode_stream(words, lg, lut), sym)


def test_encoder_capacity_error(oracle_mod, int_models):
    rng = np.random.default_rng(4)
    lg = rng.integers(-128, 128, (50, 256)).astype(np.int8)
    sym = rng.integers(0, 256, 50)
    with pytest.raises(OverflowError):
        oracle_mod.encode_stream(lg, sym, int_models["lossless"].exp_lut, capacity=3)


def test_decoder_flags_invalid_stream(oracle_mod, int_models):
    lut = int_models["lossless"].exp_lut
    lg = np.zeros((4, 256), np.int8)
    # Initial state: lower = 0, scale = (2**64 - 1) >> 24, so a point of
    # 2**64 - 1 gives quantile >= 2**24, which no valid stream produces
    # (cpu_entropy_coding.py:240-248).
    bad = np.array([0xFFFFFFFF, 0xFFFFFFFF], np.uint32)
    with pytest.raises(ValueError):
        oracle_mod.decode_stream(bad, lg, lut)
    words = oracle_mod.encode_stream(np.zeros((3, 256), np.int8), [1, 2, 3], lut)
    assert np.array_equal(oracle_mod.decode_stream(words, np.zeros((3, 256), np.int8), lut),
                          [1, 2, 3])


# ---------------------------------------------------------------- end to end

def _e2e():
    z = np.load(GOLDEN / "e2e_reads.npz")
    return z


def test_compress_chunks_matches_reference_e2e(oracle_mod, oracle_models):
    from sigcomp_amd import signal
    from framing_ref import chunk_views as split_into_chunks, frame as frame_chunks, parse as parse_framed
    z = _e2e()
    for name in ("lossless", "lossy"):
        lsb = int(z[f"{name}_lsb"])
        for i in range(int(z[f"{name}_nreads"])):
            sig = z[f"{name}_read{i}_signal"]
            small = signal.split_signal(sig, lsb)[1]
            chunks = split_into_chunks(small, 2048)
            enc = oracle_mod.compress_chunks(oracle_models[name], chunks)
            framed = frame_chunks(enc)
            assert framed == z[f"{name}_read{i}_sbytes"].tobytes(), (name, i)
            # and back
            parts, lens = parse_framed(framed, len(small), 2048)
            dec = oracle_mod.decompress_chunks(oracle_models[name], parts, lens)
            back = np.concatenate(dec) if dec else np.zeros(0, np.uint8)
            assert np.array_equal(back, small)
