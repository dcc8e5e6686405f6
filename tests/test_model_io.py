"""Host-side model loading and the float CDF helper of the entropy-coding
module (CPU only)."""

import numpy as np
import pytest
import torch


def test_npz_loader_checks_the_requested_architecture(tmp_path):
    """An integer export must match dim / num_dec_layers / window_size, as
    load_cpu_decoder requires of a checkpoint (cpu_int_inference.py:395-445):
    a mismatched archive header fails at load, not as a corrupt stream."""
    from sigcomp_amd import model_io
    path = model_io.DEFAULT_QUANT_LOSSLESS_MODEL_PATH
    m = model_io.load_int_model(path, dim=256, num_dec_layers=8, window_size=64)
    assert len(m.layers) == 9 and m.emb.shape == (257, 128)
    for kw, msg in ((dict(dim=128), "--dim"), (dict(num_dec_layers=4), "--num-dec-layers"),
                    (dict(window_size=32), "--window-size")):
        with pytest.raises(ValueError, match=msg):
            model_io.load_int_model(path, **kw)
    # a smaller export loads when asked for its own architecture
    small = model_io.random_int_model(seed=1, window=8, emb_dim=16, hidden=64, n_hidden=2)
    f = tmp_path / "small.npz"
    model_io.export_npz(small, f)
    back = model_io.load_int_model(f, dim=32, num_dec_layers=2, window_size=8)
    assert all(np.array_equal(a.weight, b.weight) for a, b in zip(small.layers, back.layers))
    with pytest.raises(ValueError, match="--dim"):
        model_io.load_int_model(f, dim=256, num_dec_layers=2)


def _quantize_np(p, precision):
    """Restatement: floor(p * 2**precision) in p's float type, clamped to >= 1,
    the surplus taken from the first largest entry, exclusive cumsum."""
    total = 1 << precision
    f = np.maximum(np.floor(p * p.dtype.type(total)).astype(np.int64), 1)
    for row in f.reshape(-1, f.shape[-1]):
        row[int(np.argmax(row))] -= int(row.sum()) - total
    return np.concatenate([np.zeros(f.shape[:-1] + (1,), np.int64), np.cumsum(f, -1)], -1)


@pytest.mark.parametrize("precision", [16, 24])
def test_quantize_probs_to_cdf(precision):
    from sigcomp_amd.gpu_entropy_coding import quantize_probs_to_cdf
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(3, 7, 256, generator=g) * 4
    probs = torch.softmax(logits, -1)
    # ties for the largest frequency (first one takes the correction) and a
    # row whose floors undershoot a lot
    probs[0, 0] = 0.0
    probs[0, 0, [5, 9]] = 0.5
    probs[0, 1] = 1.0 / 256
    for det in (False, True):
        cdf = quantize_probs_to_cdf(probs, precision, deterministic=det)
        assert cdf.dtype == torch.int64 and cdf.shape == (3, 7, 257)
        assert np.array_equal(cdf.numpy(), _quantize_np(probs.numpy(), precision))
        f = torch.diff(cdf, dim=-1)
        assert bool((f >= 1).all()) and bool((cdf[..., -1] == 1 << precision).all())
    f0 = torch.diff(quantize_probs_to_cdf(probs, precision)[0, 0])
    assert int(f0[5]) < int(f0[9])   # index 5 (first of the tied maxima) absorbed the surplus
