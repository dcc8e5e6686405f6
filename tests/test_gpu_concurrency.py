"""One model shared by calls from two host threads, each on its own HIP
stream.  The model is read-only after sc_model_create and every call keeps
its mutable state in its own workspace, so concurrent calls must give what
the same calls give one after another: the oracle's bytes (on a sample) and
the input chunks back.  One thread's batch is large (the persistent decode
over many row tiles per CU), the other's small (at most 64 groups of 32
chunks: the split decode, a cooperative launch whose workgroups wait for
each other, running beside the other stream's kernels)."""

import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _chunk_sets(rng):
    big = [rng.integers(0, 60, n).astype(np.uint8) for n in rng.integers(1, 400, 2500)]
    small = [rng.integers(0, 60, n).astype(np.uint8) for n in rng.integers(200, 700, 96)]
    return big, small


def test_two_streams_share_one_model(int_models, oracle_mod, oracle_models, monkeypatch, capfd):
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression
    codec = QuantMLPCompression(chunk_len=2048, gpu=0, model=int_models["lossless"])
    rng = np.random.default_rng(2024)
    sets = _chunk_sets(rng)
    want = [codec.compress_chunks(s) for s in sets]
    for s, w in zip(sets, want):
        idx = sorted(rng.choice(len(s), 6, replace=False))
        assert [w[i] for i in idx] == oracle_mod.compress_chunks(oracle_models["lossless"], [s[i] for i in idx])
        back = codec.decompress_chunks(w, [len(c) for c in s])
        assert all(np.array_equal(a, b) for a, b in zip(s, back))

    capfd.readouterr()
    monkeypatch.setenv("SC_HIP_DEC_LOG", "1")
    monkeypatch.delenv("SC_HIP_DEC_SPLIT", raising=False)
    results, errors = [None, None], []
    start = threading.Barrier(2, timeout=60)

    def work(k):
        try:
            stream = torch.cuda.Stream()
            out = []
            with torch.cuda.stream(stream):
                start.wait()
                for _ in range(3):
                    comp = codec.compress_chunks(sets[k])
                    out.append((comp, codec.decompress_chunks(comp, [len(c) for c in sets[k]])))
            stream.synchronize()
            results[k] = out
        except BaseException as e:   # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=240)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    assert "split launch" in capfd.readouterr().err   # the small batch's decode ran split
    for k in range(2):
        for comp, back in results[k]:
            assert comp == want[k]
            assert all(np.array_equal(a, b) for a, b in zip(sets[k], back))
