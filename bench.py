"""SigComp codec benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all|c3|c5|c1|c2|ceiling|coder]

Default (--config all): every BASELINE configuration in one JSON line.

* headline = c3 + c4: 4,000 seeded synthetic R10.4.1-like reads (~82 M
  int16 samples), bundled lossless model, chunk_len 2048.  One step = one GPU
  compress of every chunk (teacher-forced MLP fused with the frequency step,
  then the range encoder; c3) followed by the GPU decompress of the resulting
  streams (persistent autoregressive decode of all chunks at once; c4).
  Inputs (token chunks / range-coded words) are resident in HBM before the
  timed region; host-side signal split and framing are outside it (the
  PCIe-inclusive read pipeline is reported separately as end_to_end).
  value = samples / (compress + decompress time), HIP events on the
  launching stream; the roofline of the dominant kernel (k_decompress, int8
  MFMA bound) and of k_compress_mlp; cpu_baseline = the C oracle (a
  restatement of the reference CPU backend) on a bounded sample, run the way
  the reference's CPU backend runs (all physical cores, 4,096-chunk decode
  batches), plus a 1-thread figure;
* configs.c1: the reference's CPU-runnable case (64 reads) on the GPU, and the
  CPU oracle over the whole workload with every chunk's bytes compared;
* configs.c2: MLP microbenchmark, 1,048,576 context rows -> int32 CDF tables,
  seeded random per-channel model with the checkpoints' layer dims;
* configs.c5: lossy (lsb 3, RNA-like reads, lossy model), same fields as the
  headline;
* power: socket power sampled every 20 ms by a separate process over each
  timed region (average W and J per Msample).

Single configurations (--config c3 / c5 / c1 / c2) are the runs the rocprofv3
summaries under profiles/ were made from; ceiling = the int8 MFMA rate the
GPU sustains at its power limit (profiles/mfma_ceiling.txt); coder = the
step-API coder kernels timed as their own launches against HBM bandwidth.
"""

from __future__ import annotations

import argparse
import glob
import json
import os
import subprocess
import sys
import threading
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

OPS_PER_ROW = 2 * (8192 * 512 + 7 * 512 * 512 + 512 * 256)   # 12,320,768 int8 ops
PEAK_INT8_TOPS = 5000.0                                       # MI355X dense int8
PEAK_HBM_GBS = 8000.0
CHUNK_LEN = 2048
METRIC = "compress/decompress Msamples/s on 1 MI355X; INT8 MFMA util; archive bits/sample"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ power

_SAMPLER = r"""
import sys, time
path, period = sys.argv[1], float(sys.argv[2])
f = open(path, "rb", buffering=0)
out = sys.stdout
while True:
    f.seek(0)
    v = f.read(64).strip()
    out.write(f"{time.monotonic()} {int(v)}\n")
    out.flush()
    time.sleep(period)
"""


class PowerSampler:
    """Socket power of GPU 0 sampled every `period` s by a separate process
    (hwmon power1_input in uW, what `amd-smi metric -p` reports as socket
    power); window(t0, t1) averages the samples of a time.monotonic()
    interval.  Inactive (None results) where the sysfs file is absent."""

    def __init__(self, period=0.02, files=None, scale=1e-6):
        if files is None:
            files = sorted(glob.glob("/sys/class/drm/card*/device/hwmon/hwmon*/power1_input") +
                           glob.glob("/sys/class/drm/card*/device/hwmon/hwmon*/power1_average"))
        self.path = files[0] if files else None
        self.scale = scale
        self.samples = []
        self.proc = None
        if self.path:
            self.proc = subprocess.Popen([sys.executable, "-c", _SAMPLER, self.path, str(period)],
                                         stdout=subprocess.PIPE, text=True)
            self.thread = threading.Thread(target=self._read, daemon=True)
            self.thread.start()

    def _read(self):
        for line in self.proc.stdout:
            t, p = line.split()
            self.samples.append((float(t), int(p) * self.scale))

    def window(self, t0, t1):
        if not self.proc:
            return None
        time.sleep(0.05)   # let the last samples arrive
        w = [p for t, p in list(self.samples) if t0 <= t <= t1]
        return {"avg_w": round(float(np.mean(w)), 1), "max_w": round(float(np.max(w)), 1),
                "samples": len(w)} if w else None

    def stop(self):
        if self.proc:
            self.proc.terminate()
            self.proc.wait(timeout=10)


def power_fields(pw, seconds, samples):
    """Average power over a timed region -> {avg_w, j_per_msample, ...}."""
    if not pw:
        return None
    return {**pw, "j_per_msample": round(pw["avg_w"] * seconds / (samples / 1e6), 3),
            "source": "hwmon power1_input of GPU 0 (socket power), sampled every 20 ms by a separate process "
                      "over the timed steps"}


# ---------------------------------------------------------- CPU hardware

def physical_cores():
    """Physical cores among the CPUs this process may run on: distinct
    thread-sibling sets (the reference's default thread count,
    cpu_runtime.py:37-80 / main.py:1763-1766)."""
    cpus = sorted(os.sched_getaffinity(0))
    sib = set()
    for c in cpus:
        try:
            sib.add(Path(f"/sys/devices/system/cpu/cpu{c}/topology/thread_siblings_list").read_text().strip())
        except OSError:
            return len(cpus)
    return len(sib) or len(cpus)


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_hardware():
    import oracle
    return {"cpu_model": cpu_model(), "logical_cpus": len(os.sched_getaffinity(0)),
            "physical_cores": physical_cores(), "int8_path": "AVX-512 VNNI" if oracle.uses_vnni() else "portable C"}


# ------------------------------------------------------------- workloads

def build_workload(cfg_name, n_reads):
    from sigcomp_amd import signal, synth
    cfg = synth.CONFIGS[cfg_name]
    reads = synth.synth_reads(n_reads or cfg["n_reads"], cfg["seed"], cfg["profile"])
    samples = int(sum(len(r) for r in reads))
    small = signal.reads_tokens(signal.split_reads(reads, cfg["lsb"]))
    chunks = [s[i:i + CHUNK_LEN] for s in small for i in range(0, len(s), CHUNK_LEN)]
    return cfg, reads, samples, small, chunks


def model_path(cfg):
    from sigcomp_amd.model_io import DEFAULT_QUANT_LOSSLESS_MODEL_PATH, DEFAULT_QUANT_LOSSY_MODEL_PATH
    return DEFAULT_QUANT_LOSSY_MODEL_PATH if cfg["model"] == "lossy" else DEFAULT_QUANT_LOSSLESS_MODEL_PATH


def roofline(kernel, tokens, seconds, config, direction):
    achieved = tokens * OPS_PER_ROW / seconds / 1e12
    return {"kernel": kernel, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_INT8_TOPS, 4),
            "traffic": pmc_traffic(config, kernel),
            "traffic_source": f"profiles/traffic_{config}.txt (rocprofv3 PMC, bytes per call)",
            "algorithmic": f"{OPS_PER_ROW} int8 ops per {direction} token x {tokens} tokens per call",
            **ceiling_fields(achieved, config), **pmc_mfma(config, kernel)}


PEAK_L1_GBS_PER_CU = 64 * 2.4   # vector L1 fill: 64 bytes per clock at the 2.4 GHz peak engine clock


def split_roofline(model, lengths, seconds, n_cu):
    """Bound of a decode that runs split (fewer than 32 x n_cu chunks in at
    most 64 groups of 32 that the CUs hold with 4 or 8 workgroups each, as
    sc_decompress_chunks plans it): each active CU streams its share of
    layer 0 plus every later layer's weights through its vector L1 once per
    step.  None when the decode does not run split."""
    n = len(lengths)
    groups = -(-n // 32)
    if n >= 32 * n_cu or groups > 64 or groups * 4 > n_cu:
        return None
    p = 8 if groups * 8 <= n_cu else 4
    per_cu = model.layers[0].n * model.layers[0].k // p + sum(L.n * L.k for L in model.layers[1:])
    steps = int(lengths.max())
    gbs = per_cu * steps / seconds / 1e9
    return {"kernel": f"k_decompress (split, {p} workgroups per 32-chunk group)", "bound": "vector L1 fill per CU",
            "achieved": round(gbs, 2), "peak": PEAK_L1_GBS_PER_CU, "unit": "GB/s per CU",
            "frac": round(gbs / PEAK_L1_GBS_PER_CU, 4),
            "algorithmic": f"{per_cu} weight bytes per CU per step x {steps} steps, {groups * p} CUs active"}


def calibration_copy(dev, copy_mib):
    """One plain elementwise kernel moving a known number of bytes (read
    copy_mib MiB, write copy_mib MiB), outside any timed region: the
    reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters."""
    if not copy_mib:
        return
    import torch
    src = torch.ones(copy_mib << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def run_codec(name, steps, warmup, sampler, n_reads=None, e2e=True, copy_mib=0):
    """One configuration's GPU compress + decompress, timed with HIP events on
    its own stream; every chunk round-trips, 24 random chunks' bytes are
    compared with the CPU oracle.  -> (result dict, raw data for the CPU legs)."""
    import torch
    from sigcomp_amd import _hip
    from sigcomp_amd.quant_mlp_export import QuantMLPCompression

    cfg, reads, samples, small, chunks = build_workload(name, n_reads)
    codec = QuantMLPCompression(chunk_len=CHUNK_LEN, gpu=0, model_path=model_path(cfg))
    n = len(chunks)
    lengths = np.array([len(c) for c in chunks], np.int32)
    n_tokens = int(lengths.sum())
    log(f"[bench] {name}: {len(reads)} reads, {samples} samples, {n_tokens} tokens, {n} chunks")
    tok_off = np.zeros(n, np.int64)
    np.cumsum(lengths[:-1], out=tok_off[1:])
    cap = (lengths + 2).astype(np.int32)
    word_off = np.zeros(n, np.int64)
    np.cumsum(cap[:-1].astype(np.int64), out=word_off[1:])
    dev = torch.device("cuda:0")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    t_tokens, t_tok_off, t_len, t_word_off, t_cap = d(np.concatenate(chunks)), d(tok_off), d(lengths), d(word_off), d(cap)
    words, cnt, status, ws = codec._compress_buffers(n, n_tokens, int(cap.sum()))
    order = np.argsort(-lengths, kind="stable")
    o_woff, o_len, o_toff = d(word_off[order]), d(lengths[order]), d(tok_off[order])
    o_idx = d(order.astype(np.int64))
    o_cnt = torch.empty(n, dtype=torch.int32, device=dev)
    out_tokens = torch.empty(n_tokens, dtype=torch.uint8, device=dev)
    dstatus = torch.empty(n, dtype=torch.int32, device=dev)
    o_len_host = np.ascontiguousarray(lengths[order])
    dws = codec._decompress_workspace(n)
    L = _hip.lib()
    stream = torch.cuda.Stream(device=dev)          # default priority
    h = codec.hip.handle

    def compress():
        _hip.check(L.sc_compress_chunks(h, _hip.ptr(t_tokens), _hip.ptr(t_tok_off), _hip.ptr(t_len), n,
                                        n_tokens, _hip.ptr(words), _hip.ptr(t_word_off), _hip.ptr(t_cap),
                                        _hip.ptr(cnt), _hip.ptr(status), _hip.ptr(ws), ws.numel(),
                                        stream.cuda_stream))

    def decompress():
        torch.index_select(cnt, 0, o_idx, out=o_cnt)
        _hip.check(L.sc_decompress_chunks(h, _hip.ptr(words), _hip.ptr(o_woff), _hip.ptr(o_cnt),
                                          _hip.ptr(o_len), n, _hip.ptr(out_tokens), _hip.ptr(o_toff),
                                          _hip.ptr(dstatus), o_len_host.ctypes.data, _hip.ptr(dws),
                                          dws.numel(), stream.cuda_stream))

    calibration_copy(dev, copy_mib)
    with torch.cuda.device(dev), torch.cuda.stream(stream):
        for w in range(warmup):
            compress(); decompress()
            stream.synchronize()
        log(f"[bench] {name}: {warmup} warmup steps done")
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        torch.cuda.synchronize()
        t0 = time.monotonic()
        for k in range(steps):
            ev[k][0].record(stream)
            compress()
            ev[k][1].record(stream)
            decompress()
            ev[k][2].record(stream)
        stream.synchronize()
        torch.cuda.synchronize()
        t1 = time.monotonic()
    wall = t1 - t0
    t_c = float(np.mean([e[0].elapsed_time(e[1]) for e in ev])) / 1e3
    t_d = float(np.mean([e[1].elapsed_time(e[2]) for e in ev])) / 1e3
    if int(status.sum().item()) or int(dstatus.sum().item()):
        raise RuntimeError("codec reported a stream error")
    back = out_tokens.cpu().numpy()
    if not np.array_equal(back, t_tokens.cpu().numpy()):
        raise RuntimeError("round trip mismatch")
    cnt_np = cnt.cpu().numpy()
    words_np = words.cpu().numpy().view(np.uint32)
    comp_bytes = int(cnt_np.sum()) * 4 + 2 * n
    parity = oracle_sample_check(codec.model, chunks, words_np, word_off, cnt_np)
    log(f"[bench] {name}: compress {t_c * 1e3:.1f} ms, decompress {t_d * 1e3:.1f} ms, oracle sample ok={parity}")
    res = {
        "workload": f"{name}: {len(reads)} reads, {samples} samples, {n} chunks of <= {CHUNK_LEN} tokens, "
                    f"model {cfg['model']}, lsb {cfg['lsb']}",
        "reads": len(reads), "samples": samples, "tokens": n_tokens, "chunks": n,
        "round_trip_msamples_s": round(samples / (t_c + t_d) / 1e6, 3),
        "ms_per_step": round((t_c + t_d) * 1e3, 3),
        "compress_msamples_s": round(samples / t_c / 1e6, 3),
        "decompress_msamples_s": round(samples / t_d / 1e6, 3),
        "compress_ms": round(t_c * 1e3, 3), "decompress_ms": round(t_d * 1e3, 3),
        "bits_per_sample_tokens": round(comp_bytes * 8 / samples, 4),
        "parity": {"round_trip_all_chunks": True, "oracle_sample_chunks": parity},
        "wall_s_timed": round(wall, 3),
        "power": power_fields(sampler.window(t0, t1), t_c + t_d, samples),
        "roofline": roofline("k_decompress", n_tokens, t_d, name, "decoded"),
        "roofline_compress": roofline("k_compress_mlp", n_tokens, t_c, name, "coded"),
    }
    rl1 = split_roofline(codec.model, lengths, t_d, torch.cuda.get_device_properties(0).multi_processor_count)
    if rl1:
        res["roofline_split"] = rl1
    if e2e:
        # the first pass also allocates the pinned staging buffers (torch keeps
        # them cached): report the second, as a process that compresses
        # batch after batch runs
        first = end_to_end(codec, reads, cfg["lsb"])
        res["end_to_end"] = end_to_end(codec, reads, cfg["lsb"])
        res["end_to_end"]["first_pass_msamples_s"] = first["msamples_s_round_trip"]
    return res, dict(model=codec.model, chunks=chunks, samples=samples, words=words_np, word_off=word_off,
                     word_cnt=cnt_np)


def end_to_end(codec, reads, lsb):
    """One pass of the whole read pipeline as main.py drives it: int16 reads
    in host memory -> split (host library) -> batch_inference_reads (host ->
    device copy, GPU compress, framing) -> batch_inference_reads back
    (parsing, GPU decompress, device -> host) -> reassembly.  Reports the
    PCIe-inclusive rate and the stage times (not the headline value)."""
    from sigcomp_amd import signal
    t = {}
    t0 = time.perf_counter()
    sp = signal.split_reads(reads, lsb)
    small = signal.reads_tokens(sp)
    t["split"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    framed = codec.batch_inference_reads(list_of_reads=small, batch_size=20480)
    t["compress_reads"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    back = codec.batch_inference_reads(list_of_compressed_reads=framed, list_of_lengths=[len(x) for x in small],
                                       batch_size=20480)
    t["decompress_reads"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    out = signal.reassemble_reads(sp, small=np.concatenate(back) if back else None, lsb=lsb)
    t["reassemble"] = time.perf_counter() - t0
    if not all(np.array_equal(a, b) for a, b in zip(small, back)):
        raise RuntimeError("end-to-end token round trip mismatch")
    if lsb == 0 and not all(np.array_equal(a, b) for a, b in zip(reads, out)):
        raise RuntimeError("end-to-end sample round trip mismatch")
    total = sum(t.values())
    samples = sum(len(r) for r in reads)
    return {"msamples_s_round_trip": round(samples / total / 1e6, 3),
            "seconds": {k: round(v, 4) for k, v in t.items()},
            "payload_bytes": int(sum(len(f) for f in framed)),
            "note": "int16 reads in host memory -> SIG2 chunk payloads -> int16 reads, incl. host stages "
                    "and PCIe copies; not the headline value"}


def pmc_traffic(config, kernel):
    """HBM-side bytes per call of `kernel` from the committed rocprofv3 PMC
    summary of this workload (profiles/traffic_<config>.txt: FETCH_SIZE +
    WRITE_SIZE passes, calibrated against a copy kernel), or None."""
    path = REPO / "profiles" / f"traffic_{config}.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes" and f[1] == kernel:
            return int(f[2])
    return None


def pmc_mfma(config, kernel):
    """Counter-measured MFMA utilisation of `kernel` on this workload from the
    committed rocprofv3 PMC summary (profiles/mfma_util.txt: fraction of
    SIMD cycles the matrix cores are busy, and the clock), or {}."""
    path = REPO / "profiles" / "mfma_util.txt"
    if not path.exists():
        return {}
    out = {}
    for line in path.read_text().splitlines():
        f = line.split()
        if len(f) == 4 and f[1] == kernel and f[2] == config:
            if f[0] == "mfma_busy":
                out["mfma_busy_counters"] = float(f[3])
            elif f[0] == "mfma_clock_ghz":
                out["mfma_clock_ghz_counters"] = float(f[3])
    if out:
        out["mfma_counters_source"] = ("profiles/mfma_util.txt (rocprofv3 PMC SQ_VALU_MFMA_BUSY_CYCLES / "
                                       "GRBM_GUI_ACTIVE, SQ_INSTS_VALU_MFMA_MOPS_I8)")
    return out


def oracle_sample_check(model, chunks, words_np, word_off, cnt_np, k=24):
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle
    rng = np.random.default_rng(0)
    idx = np.sort(rng.choice(len(chunks), size=min(k, len(chunks)), replace=False))
    ref = oracle.compress_chunks(oracle.OracleModel(model), [chunks[i] for i in idx])
    for j, i in enumerate(idx):
        got = words_np[word_off[i]:word_off[i] + cnt_np[i]].tobytes()
        if got != ref[j]:
            raise RuntimeError(f"chunk {i} differs from the CPU oracle")
    return int(len(idx))


# ------------------------------------------------------------ CPU legs

def _cpu_leg(om, chunks, words, word_off, word_cnt, threads, n_compress, n_decode, prefix, rng):
    """Compress n_compress random whole chunks; decode the first `prefix`
    tokens of n_decode random chunks in one batch (autoregressive, batched
    across chunks); check the decode against the tokens.  -> token counts
    and seconds."""
    import oracle
    oracle.set_num_threads(threads)
    pick = rng.choice(len(chunks), size=min(len(chunks), n_compress), replace=False)
    sample = [chunks[i] for i in pick]
    t0 = time.perf_counter()
    oracle.compress_chunks(om, sample)
    tc = time.perf_counter() - t0
    dpick = rng.choice(len(chunks), size=min(len(chunks), n_decode), replace=False)
    streams = [words[word_off[i]:word_off[i] + word_cnt[i]].tobytes() for i in dpick]
    lens = [min(prefix, len(chunks[i])) for i in dpick]
    t0 = time.perf_counter()
    dec = oracle.decompress_chunks(om, streams, lens)
    td = time.perf_counter() - t0
    for i, dd in zip(dpick, dec):
        if not np.array_equal(dd, chunks[i][:len(dd)]):
            raise RuntimeError("CPU oracle decode disagrees with the GPU stream")
    return sum(len(c) for c in sample), tc, sum(lens), td


def cpu_baseline(raw, hw):
    """The C oracle (restatement of the reference CPU backend) on a bounded
    sample of the workload, as the reference's CPU backend runs: one thread
    per physical core (main.py:1763-1766), chunks compressed independently,
    decode batched over 4,096 chunks (the reference's --cpu-batch-size
    default for decompress, main.py:1958-1961), int8 dot products with
    AVX-512 VNNI where the host has it (the reference's int_mm backend,
    cpu_int_inference.py:24-82).  Also one thread on a smaller sample.
    Rates are converted to samples with the workload's samples per token."""
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle
    om = oracle.OracleModel(raw["model"])
    spt = raw["samples"] / sum(len(c) for c in raw["chunks"])
    threads = hw["physical_cores"]
    rng = np.random.default_rng(1)
    args = (om, raw["chunks"], raw["words"], raw["word_off"], raw["word_cnt"])
    ct, tc, dt, td = _cpu_leg(*args, threads, 64 * threads, 4096, 384, rng)
    ct1, tc1, dt1, td1 = _cpu_leg(*args, 1, 12, 256, 96, rng)
    oracle.set_num_threads(threads)
    c_rate, d_rate = ct * spt / tc, dt * spt / td
    c1r, d1r = ct1 * spt / tc1, dt1 * spt / td1
    rt = lambda c, d: 1.0 / (1.0 / c + 1.0 / d)
    return {"value": round(rt(c_rate, d_rate) / 1e6, 5), "unit": "Msamples/s (round trip)", "cores": threads,
            "kind": "port",
            "compress_msamples_s": round(c_rate / 1e6, 5), "decompress_msamples_s": round(d_rate / 1e6, 5),
            "one_thread": {"value": round(rt(c1r, d1r) / 1e6, 6), "compress_msamples_s": round(c1r / 1e6, 6),
                           "decompress_msamples_s": round(d1r / 1e6, 6)},
            **hw,
            "sample": f"{threads} threads: compress {64 * threads} random whole chunks ({ct} tokens, {tc:.1f} s); "
                      f"decompress the first 384 tokens of 4096 random chunks decoded together ({dt} tokens, "
                      f"{td:.1f} s); 1 thread: 12 whole chunks ({tc1:.1f} s), first 96 tokens of 256 chunks "
                      f"({td1:.1f} s); C oracle, the GPU's streams decoded and checked"}


def cpu_full(raw, hw):
    """Config c1 (the reference's CPU-runnable case): the CPU oracle over the
    whole workload, one thread per physical core, every chunk checked:
    compress every chunk (bytes compared with the GPU's), decode every GPU
    stream in one batch (all 675 chunks fit the reference's 4,096-chunk
    batch), tokens compared with the originals."""
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle
    threads = hw["physical_cores"]
    oracle.set_num_threads(threads)
    om = oracle.OracleModel(raw["model"])
    chunks, samples = raw["chunks"], raw["samples"]
    t0 = time.perf_counter()
    ref = oracle.compress_chunks(om, chunks)
    tc = time.perf_counter() - t0
    w, wo, wc = raw["words"], raw["word_off"], raw["word_cnt"]
    streams = [w[wo[i]:wo[i] + wc[i]].tobytes() for i in range(len(chunks))]
    bad = [i for i in range(len(chunks)) if streams[i] != ref[i]]
    if bad:
        raise RuntimeError(f"{len(bad)} chunks differ from the CPU oracle (first {bad[0]})")
    t0 = time.perf_counter()
    dec = oracle.decompress_chunks(om, streams, [len(c) for c in chunks])
    td = time.perf_counter() - t0
    if not all(np.array_equal(d, c) for d, c in zip(dec, chunks)):
        raise RuntimeError("CPU oracle decode disagrees with the GPU streams")
    return {"value": round(samples / (tc + td) / 1e6, 5), "unit": "Msamples/s (round trip)", "cores": threads,
            "kind": "port",
            "compress_msamples_s": round(samples / tc / 1e6, 5),
            "decompress_msamples_s": round(samples / td / 1e6, 5), **hw,
            "sample": f"the whole workload: {len(chunks)} chunks compressed ({tc:.1f} s) and decoded in one batch "
                      f"({td:.1f} s) by the C oracle on {threads} threads; all {len(chunks)} chunk byte strings "
                      f"equal the GPU's"}


# ----------------------------------------------------------------- c2

def _time_mlp(hm, ctx_d, steps, warmup, sampler):
    """HIP-event time per forward_windows(ctx, "cdf") launch and the power
    window of the timed launches -> (seconds, power dict or None, output)."""
    import torch
    for _ in range(warmup):
        hm.forward_windows(ctx_d, "cdf")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.monotonic()
    e0.record()
    for _ in range(steps):
        out = hm.forward_windows(ctx_d, "cdf")
    e1.record()
    torch.cuda.synchronize()
    t1 = time.monotonic()
    return e0.elapsed_time(e1) / 1e3 / steps, (sampler.window(t0, t1) if sampler else None), out


def run_mlp(rows, steps, warmup, sampler, copy_mib=0):
    """Config c2: `rows` context rows -> int32 CDF tables, seeded random
    per-channel model with the bundled checkpoints' layer dims; 256 random
    rows checked against the oracle.  Beside it, the same rows through the
    same kernel with a random per-tensor model and with the bundled lossless
    checkpoint (what per-channel constants and uniform random weights cost;
    each checked on 64 rows)."""
    import torch
    from sigcomp_amd import signal, synth
    from sigcomp_amd.model_io import DEFAULT_QUANT_LOSSLESS_MODEL_PATH, load_int_model, random_int_model
    from sigcomp_amd.quant_mlp_export import HipModel
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle
    m = random_int_model(seed=2, per_channel=True)
    hm = HipModel(m, torch.device("cuda:0"))
    toks = np.concatenate([signal.split_signal(r)[1] for r in synth.synth_reads(64, 202, synth.DNA)])
    toks = toks.astype(np.int64)
    starts = np.random.default_rng(3).integers(-63, len(toks) - 64, rows)
    idx = starts[:, None] + np.arange(64)[None, :]
    ctx = np.where(idx < 0, 256, toks[np.clip(idx, 0, None)])
    ctx_d = torch.from_numpy(ctx).cuda()
    calibration_copy(ctx_d.device, copy_mib)

    def check(model, out, n, seed):
        sub = np.random.default_rng(seed).choice(rows, n, replace=False)
        ref = oracle.logits_to_cdf(oracle.mlp_forward(oracle.OracleModel(model), ctx[sub]), model.exp_lut)
        if not np.array_equal(out[torch.from_numpy(sub).cuda()].cpu().numpy().astype(np.int64), ref):
            raise RuntimeError("c2 CDF mismatch vs oracle")

    t, pw, out = _time_mlp(hm, ctx_d, steps, warmup, sampler)
    check(m, out, 256, 4)
    achieved = rows * OPS_PER_ROW / t / 1e12
    side = {}
    for name, model in (("random_per_tensor", random_int_model(seed=2, per_channel=False)),
                        ("lossless_checkpoint", load_int_model(DEFAULT_QUANT_LOSSLESS_MODEL_PATH))):
        h2 = HipModel(model, torch.device("cuda:0"))
        t2, pw2, out2 = _time_mlp(h2, ctx_d, min(steps, 200), warmup, sampler)
        check(model, out2, 64, 5)
        side[name] = {"mrows_s": round(rows / t2 / 1e6, 3), "achieved_tops": round(rows * OPS_PER_ROW / t2 / 1e12, 2),
                      "core": h2.core, "mean_abs_weight": round(float(np.mean(
                          [np.abs(L.weight.astype(np.int32)).mean() for L in model.layers])), 2),
                      "avg_w": pw2["avg_w"] if pw2 else None}
        del h2, out2
    return {"workload": f"c2: {rows} context rows -> int32 CDF tables, random per-channel int8 model with the "
                        "checkpoints' layer dims",
            "mrows_s": round(rows / t / 1e6, 3), "ms_per_step": round(t * 1e3, 3), "steps": steps,
            "parity": {"oracle_rows": 256},
            "power": ({**pw, "j_per_mrow": round(pw["avg_w"] * t / (rows / 1e6), 3)} if pw else None),
            "roofline": {"kernel": "k_mlp_context<cdf>", "bound": "mfma", "achieved": round(achieved, 2),
                         "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_INT8_TOPS, 4),
                         "traffic": pmc_traffic("c2", "k_mlp_context"),
                         "traffic_source": "profiles/traffic_c2.txt (rocprofv3 PMC, bytes per launch)",
                         "algorithmic": f"{OPS_PER_ROW} int8 ops per row x {rows} rows per launch",
                         **ceiling_fields(achieved, "c2"), **pmc_mfma("c2", "k_mlp_context")},
            "same_rows_other_models": {**side, "note": "the same rows and kernel with a random per-tensor model "
                                                       "and with the bundled lossless checkpoint; not the c2 figure"}}


def bench_mlp(args):
    r = run_mlp(args.rows, args.steps, args.warmup, None, copy_mib=args.copy_mib)
    return {"metric": "INT8 MLP rows/s -> int32 CDF (c2 microbench)", "value": r["mrows_s"], "unit": "Mrows/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
            "data": "synthetic", "config": {"workload": r["workload"]}, "roofline": r["roofline"],
            "same_rows_other_models": r["same_rows_other_models"]}


# ------------------------------------------------------- ceiling, coder

# Share of a token's int8 MACs in layer 0 (8192 -> 512); the rest are the
# hidden and output layers (512-wide inputs).
LAYER0_MAC_SHARE = 8192 * 512 / (OPS_PER_ROW // 2)


def _a_frag(m):
    """32 x 32 int8 block M[m][k] -> one A fragment of v_mfma_i32_32x32x32_i8
    (lane l holds M[l % 32][16 (l // 32) .. +15])."""
    return np.ascontiguousarray(m.reshape(32, 2, 16).transpose(1, 0, 2).reshape(64, 16))


def _b_frag(m):
    """32 x 32 int8 block M[k][n] -> one B fragment (lane l holds
    M[16 (l // 32) .. +15][l % 32])."""
    return np.ascontiguousarray(m.reshape(2, 16, 32).transpose(0, 2, 1).reshape(64, 16))


def _requant(acc, layer):
    """(acc + bias) * M0 >> shift, clamped to int8 (ReLU layers at 0): the
    integer linear layer's epilogue, in int64."""
    y = (acc + layer.bias.astype(np.int64)) * layer.m0.astype(np.int64) >> layer.shift.astype(np.int64)
    return np.clip(y, 0 if layer.relu else -128, 127).astype(np.int8)


def checkpoint_operands(model, cfg_name, seed=7):
    """MFMA operand sets of a bundled checkpoint as the codec feeds them:
    {"layer0": 4 A fragments of layer-0 weights and 4 B fragments of 32
    embedded context rows (tokens of the config's synthetic reads),
    "hidden": 4 A fragments of hidden-layer weights and 4 B fragments of the
    same rows' layer-0 outputs (ReLU activations)} as 8192-byte arrays."""
    from sigcomp_amd import signal, synth
    cfg = synth.CONFIGS[cfg_name]
    rng = np.random.default_rng(seed)
    toks = np.concatenate([signal.split_signal(r, cfg["lsb"])[1]
                           for r in synth.synth_reads(8, cfg["seed"], cfg["profile"])]).astype(np.int64)
    starts = rng.integers(0, len(toks) - 64, 32)
    ctx = toks[starts[:, None] + np.arange(64)[None, :]]
    x0 = model.emb[ctx].reshape(32, 64 * model.emb.shape[1]).astype(np.int64)   # [rows, 8192]
    L0 = model.layers[0]
    x1 = _requant((x0.astype(np.float64) @ L0.weight.astype(np.float64).T).astype(np.int64), L0)  # exact
    sets = {}
    for name, w_layers, act in (("layer0", [L0], x0), ("hidden", model.layers[1:-1], x1.astype(np.int64))):
        frags_a, frags_b = [], []
        for j in range(4):
            W = w_layers[j % len(w_layers)].weight
            nt, kt = rng.integers(0, W.shape[0] // 32), rng.integers(0, W.shape[1] // 32)
            frags_a.append(_a_frag(W[nt * 32:nt * 32 + 32, kt * 32:kt * 32 + 32]))
            kb = rng.integers(0, act.shape[1] // 32)
            frags_b.append(_b_frag(act[:, kb * 32:kb * 32 + 32].T.astype(np.int8)))
        sets[name] = np.concatenate(frags_a + frags_b).reshape(-1).astype(np.int8)
    return sets


def bench_ceiling(args):
    """The int8 MFMA rate the GPU sustains at its power limit, per operand
    data: every CU runs register-operand v_mfma_i32_32x32x32_i8 chains
    (sc_mfma_burn_i8) for about 6 s per operand set (long enough for the
    power controller to settle), with uniform random int8 operands, with
    zeros (no toggling: close to the clock-limited 5.0 POP/s), and with the
    operands the codec's MFMAs see for each bundled checkpoint: layer-0
    weight fragments against embedded context rows of the config's
    synthetic reads, and hidden-layer weight fragments against those rows'
    ReLU activations.  A checkpoint's ceiling weights the two by their share
    of a token's MACs (layer 0: 68.1%).  Socket power and, where hwmon has
    it, the GFX clock are sampled over each set."""
    import torch
    from sigcomp_amd import _hip
    from sigcomp_amd.model_io import (DEFAULT_QUANT_LOSSLESS_MODEL_PATH, DEFAULT_QUANT_LOSSY_MODEL_PATH,
                                      load_int_model)
    L = _hip.lib()
    n_groups = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 5000
    ops_per_launch = n_groups * 4 * iters * 64 * 65536
    out = torch.empty(n_groups * 256 * 16, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(1)
    sets = {"random": torch.randint(-128, 128, (8192,), dtype=torch.int8, generator=g).numpy(),
            "zero": np.zeros(8192, np.int8)}
    for tag, path, cfg in (("lossless", DEFAULT_QUANT_LOSSLESS_MODEL_PATH, "c3"),
                           ("lossy", DEFAULT_QUANT_LOSSY_MODEL_PATH, "c5")):
        for k, v in checkpoint_operands(load_int_model(path), cfg).items():
            sets[f"{tag}_{k}"] = v
    power = PowerSampler()
    clk_files = sorted(glob.glob("/sys/class/drm/card*/device/hwmon/hwmon*/freq1_input"))
    clock = PowerSampler(period=0.05, files=clk_files, scale=1e-6) if clk_files else None   # Hz -> MHz
    res = {}
    try:
        for name, arr in sets.items():
            ops = torch.from_numpy(arr.copy()).cuda()
            rc = L.sc_mfma_burn_i8(ops.data_ptr(), 10, n_groups, out.data_ptr(), stream)
            if rc:
                raise RuntimeError(L.sc_last_error().decode())
            torch.cuda.synchronize()
            rates = []
            t_end = time.time() + 6.0
            while time.time() < t_end:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                L.sc_mfma_burn_i8(ops.data_ptr(), iters, n_groups, out.data_ptr(), stream)
                e1.record()
                torch.cuda.synchronize()
                rates.append((time.monotonic(), ops_per_launch / (e0.elapsed_time(e1) / 1e3) / 1e12))
            # the last second: the steady state under the power limit
            tail = rates[-max(1, len(rates) // 6):]
            t0 = tail[0][0] - (tail[1][0] - tail[0][0] if len(tail) > 1 else 0.2)
            pw = power.window(t0, tail[-1][0])
            ck = clock.window(t0, tail[-1][0]) if clock else None
            res[name] = {"tops": round(float(np.median([r for _, r in tail])), 1),
                         "socket_w": pw["avg_w"] if pw else None, "gfx_mhz": ck["avg_w"] if ck else None,
                         "mean_abs_operand": round(float(np.abs(arr.astype(np.int32)).mean()), 2)}
            log(f"[bench] MFMA burn, {name} operands: {res[name]}")
    finally:
        power.stop()
        if clock:
            clock.stop()
    for tag in ("lossless", "lossy"):
        r0, rh = res[f"{tag}_layer0"]["tops"], res[f"{tag}_hidden"]["tops"]
        res[f"{tag}_checkpoint"] = {"tops": round(1.0 / (LAYER0_MAC_SHARE / r0 + (1 - LAYER0_MAC_SHARE) / rh), 1),
                                    "note": "layer-0 and hidden-layer operand rates weighted by their share of "
                                            "a token's MACs (time-weighted harmonic mean)"}
    return {"metric": "sustained int8 MFMA rate (register operands, all CUs)",
            "value": res["lossless_checkpoint"]["tops"], "unit": "TOP/s", "n_gpus": 1, "steps": 1, "warmup": 1,
            "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8", "data": "synthetic operands and the bundled checkpoints' own",
            "config": {"workload": f"{n_groups} workgroups x 4 waves x {iters * 64} v_mfma_i32_32x32x32_i8 per "
                                   "launch, ~6 s per operand set"},
            "operand_sets": res, "peak": PEAK_INT8_TOPS,
            "frac_of_peak": {k: round(v["tops"] / PEAK_INT8_TOPS, 4) for k, v in res.items()}}


# Algorithmic HBM bytes per stream and step of the coder step kernels
# (device arrays as GpuRangeStepEncoder / GpuRangeDecoder keep them), words
# excluded (added from the measured word count):
#   k_logits_to_cdf: 256 B logits in, 257 x int64 CDF out
#   k_encode_step:   logits 256, symbol 8, valid 8, status 4, state read and
#                    written (lower 8, range 8, inverted 4, first 4, pos 4)
#   k_decode_step:   logits 256, valid 8, status 4, state read (lower, range,
#                    point, read_pos, end_pos: 40) and written (32), symbol 8
# from this many streams the library runs the encode / decode steps as its
# wide kernels (64 rows per wave), below as the narrow ones
STEP_WIDE_MIN_ROWS = 1 << 18
CODER_BYTES = {"k_logits_to_cdf": 256 + 257 * 8, "k_encode_step": 256 + 8 + 8 + 4 + 2 * 28,
               "k_decode_step": 256 + 8 + 4 + 40 + 32 + 8}


def bench_coder(args):
    """The reference's step-API coder kernels (logits -> CDF, encode step,
    decode step) timed as their own launches, HIP events on the launching
    stream: B streams of synthetic int8 logits per step (normal, sd 20; the
    coded symbol is the argmax of the logits plus uniform noise), `steps`
    steps, called through the C ABI.  At B = 1,048,576 one step's logits
    (268 MB) exceed the 256 MB MALL, so the launches stream from HBM;
    B = 20,480 (the reference's batch) shows the launch-bound regime.  The
    decoder, fed the encoder's sealed words, must return every coded symbol."""
    import torch
    from sigcomp_amd import _hip
    from sigcomp_amd.gpu_entropy_coding import GpuRangeDecoder, GpuRangeStepEncoder
    from sigcomp_amd.model_io import load_int_model
    dev = torch.device("cuda:0")
    L = _hip.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    lut = torch.from_numpy(load_int_model().exp_lut.astype(np.int64)).to(dev)
    calibration_copy(dev, args.copy_mib)
    T = max(2, args.steps)
    out = {}
    for B in (args.rows, 20480):
        g = torch.Generator(device=dev).manual_seed(5)
        logits = [(torch.randn(B, 256, generator=g, device=dev) * 20).round().clamp(-128, 127).to(torch.int8)
                  for _ in range(T)]
        syms = [torch.argmax(lg.float() + torch.rand(B, 256, generator=g, device=dev) * 40, dim=1)
                for lg in logits]
        valid = torch.full((B,), T, dtype=torch.int64, device=dev)
        cdf = torch.empty((B, 257), dtype=torch.int64, device=dev)
        enc = GpuRangeStepEncoder(B, T + 32, device=dev)

        def timed(fn):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for t in range(T):
                _hip.check(fn(t))
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / 1e3 / T

        p = _hip.ptr
        # first launches load the kernels' code object: untimed, and at
        # t = T every stream is inactive (no coder state changes)
        scratch = torch.empty(B, dtype=torch.int64, device=dev)
        _hip.check(L.sc_logits_to_cdf(p(logits[0]), B, p(lut), p(cdf), stream))
        _hip.check(L.sc_encode_step(p(logits[0]), p(lut), p(syms[0]), p(valid), T, B, enc._state,
                                    p(enc.output_words), enc.max_words, stream))
        t_cdf = timed(lambda t: L.sc_logits_to_cdf(p(logits[t]), B, p(lut), p(cdf), stream))
        t_enc = timed(lambda t: L.sc_encode_step(p(logits[t]), p(lut), p(syms[t]), p(valid), t, B, enc._state,
                                                 p(enc.output_words), enc.max_words, stream))
        words = enc.get_compressed()
        wpt = sum(len(w) for w in words) / 4 / (B * T)     # words per stream-step, seal included
        dec = GpuRangeDecoder(words, device=dev)
        got = torch.empty((T, B), dtype=torch.int64, device=dev)
        _hip.check(L.sc_decode_step(p(logits[0]), p(lut), p(valid), T, B, dec._state, p(dec.comp_words),
                                    p(scratch), stream))
        t_dec = timed(lambda t: L.sc_decode_step(p(logits[t]), p(lut), p(valid), t, B, dec._state,
                                                 p(dec.comp_words), p(got[t]), stream))
        dec.check()
        if not all(torch.equal(got[t], syms[t]) for t in range(T)):
            raise RuntimeError("coder round trip mismatch")
        res = {}
        for k, tk, extra in (("k_logits_to_cdf", t_cdf, 0.0), ("k_encode_step", t_enc, 4 * wpt),
                             ("k_decode_step", t_dec, 4 * wpt)):
            gbs = B * (CODER_BYTES[k] + extra) / tk / 1e9
            res[k] = {"us_per_launch": round(tk * 1e6, 2), "gb_s": round(gbs, 1),
                      "frac_of_hbm": round(gbs / PEAK_HBM_GBS, 4),
                      "bytes_per_stream": round(CODER_BYTES[k] + extra, 2)}
        res["words_per_stream_step"] = round(wpt, 4)
        out[B] = res
        log(f"[bench] coder B={B}: " + ", ".join(f"{k} {v['us_per_launch']} us {v['gb_s']} GB/s"
                                                for k, v in res.items() if k.startswith("k_")))
        del logits, syms, enc, dec, got, cdf, scratch
    big = out[args.rows]
    d = big["k_decode_step"]
    return {"metric": "range-coder step kernels (logits->CDF, encode step, decode step), HBM GB/s",
            "value": d["gb_s"], "unit": "GB/s (k_decode_step)", "n_gpus": 1, "steps": T, "warmup": 0,
            "ms_per_step": round(d["us_per_launch"] / 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u64", "data": "synthetic",
            "config": {"workload": f"coder: {args.rows} streams x {T} steps of synthetic int8 logits "
                                   f"(and {20480} streams, the reference's batch)"},
            "roofline": {"kernel": "k_decode_step_wide" if args.rows >= STEP_WIDE_MIN_ROWS else "k_decode_step", "bound": "hbm", "achieved": d["gb_s"], "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": d["frac_of_hbm"], "traffic": None,
                         "algorithmic": f"{d['bytes_per_stream']} B per stream and step x {args.rows} streams"},
            "kernels": {str(B): v for B, v in out.items()}}


# Operand data each configuration's MFMAs see -> the ceiling it is read
# against: the bundled checkpoints' own (c1, c3/c4 lossless; c5 lossy) and
# uniform random for c2's random model.
CEILING_OPERANDS = {"c1": "lossless_checkpoint", "c3": "lossless_checkpoint", "c4": "lossless_checkpoint",
                    "c5": "lossy_checkpoint", "c2": "random_operands"}


def power_capped_peak(operands="lossless_checkpoint"):
    """Sustained int8 MFMA rate for the given operand data, measured by
    `bench.py --config ceiling` and recorded in profiles/mfma_ceiling.txt."""
    f = REPO / "profiles" / "mfma_ceiling.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith(operands + "_tops"):
            return float(line.split()[1])
    return None


def ceiling_fields(achieved, config):
    operands = CEILING_OPERANDS.get(config, "lossless_checkpoint")
    cap = power_capped_peak(operands)
    if cap is None:
        return {}
    return {"power_capped_peak": cap, "frac_of_power_capped_peak": round(achieved / cap, 4),
            "power_capped_peak_operands": operands,
            "power_capped_peak_source": "profiles/mfma_ceiling.txt (bench.py --config ceiling)"}


# ----------------------------------------------------------------- main

def headline(res, steps, warmup):
    """The contract's fields for one codec configuration's result."""
    return {"metric": METRIC, "value": res["round_trip_msamples_s"], "unit": "Msamples/s (round trip)",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
            "data": "synthetic",
            "config": {"workload": res["workload"], "reads": res["reads"], "samples": res["samples"],
                       "tokens": res["tokens"], "chunks": res["chunks"]}}


def run_all(args):
    """Every BASELINE configuration, one JSON line (headline = c3 + c4)."""
    sys.path.insert(0, str(REPO / "oracle"))
    sampler = PowerSampler()
    try:
        hw = cpu_hardware()
        c3, raw3 = run_codec("c3", args.steps, args.warmup, sampler, copy_mib=args.copy_mib)
        out = headline(c3, args.steps, args.warmup)
        out.update({k: c3[k] for k in ("compress_msamples_s", "decompress_msamples_s", "bits_per_sample_tokens",
                                        "parity", "wall_s_timed", "power", "end_to_end", "roofline",
                                        "roofline_compress")})
        c5, raw5 = run_codec("c5", args.steps, args.warmup, sampler, e2e=False)
        c1, raw1 = run_codec("c1", args.steps, args.warmup, sampler, e2e=False)
        # c2 steps are ~5 ms: enough of them for a power reading of ~2 s
        c2 = run_mlp(args.rows, max(args.steps, 400), args.warmup, sampler)
        if not args.no_cpu_baseline:
            log("[bench] cpu baselines ...")
            out["cpu_baseline"] = cpu_baseline(raw3, hw)
            c5["cpu_baseline"] = cpu_baseline(raw5, hw)
            c1["cpu_baseline"] = cpu_full(raw1, hw)
            c1["parity"]["oracle_all_chunks"] = len(raw1["chunks"])
        keep = ("workload", "samples", "tokens", "chunks", "bits_per_sample_tokens", "power")
        out["configs"] = {
            "c1": c1,
            "c2": c2,
            "c3": {**{k: c3[k] for k in keep}, "compress_msamples_s": c3["compress_msamples_s"],
                   "compress_ms": c3["compress_ms"], "roofline": c3["roofline_compress"],
                   "note": "the headline's compress half"},
            "c4": {**{k: c3[k] for k in keep}, "decompress_msamples_s": c3["decompress_msamples_s"],
                   "decompress_ms": c3["decompress_ms"], "roofline": c3["roofline"],
                   "note": "the headline's decompress half (the c3 archive's streams)"},
            "c5": c5,
        }
        return out
    finally:
        sampler.stop()


def run_one(args):
    """One codec configuration (profiling runs)."""
    sys.path.insert(0, str(REPO / "oracle"))
    sampler = PowerSampler()
    try:
        res, raw = run_codec(args.config, args.steps, args.warmup, sampler, n_reads=args.n_reads,
                             e2e=args.config == "c3" and not args.no_end_to_end, copy_mib=args.copy_mib)
    finally:
        sampler.stop()
    out = headline(res, args.steps, args.warmup)
    out.update({k: v for k, v in res.items() if k not in out and k not in ("workload", "reads", "samples",
                                                                             "tokens", "chunks")})
    if not args.no_cpu_baseline:
        hw = cpu_hardware()
        if args.config == "c1":
            out["cpu_baseline"] = cpu_full(raw, hw)
        else:
            out["cpu_baseline"] = cpu_baseline(raw, hw)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="all", choices=["all", "c3", "c5", "c1", "c2", "ceiling", "coder"])
    ap.add_argument("--n-reads", type=int, default=None)
    ap.add_argument("--rows", type=int, default=1 << 20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-end-to-end", action="store_true",
                    help="single configurations: skip the PCIe-inclusive read pipeline pass (profiling runs)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="run one elementwise copy of this many MiB first (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the codec shards by independent reads with no "
              "collective, so multi-GPU runs are out of scope for this build", file=sys.stderr)
        sys.exit(2)
    runners = {"all": run_all, "c2": bench_mlp, "ceiling": bench_ceiling, "coder": bench_coder}
    print(json.dumps(runners.get(args.config, run_one)(args)), flush=True)
    # release every model handle and device buffer, and let the device
    # finish, while the interpreter and the HIP runtime are still whole
    # (rather than from finalisers during interpreter shutdown)
    import gc
    import torch
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.synchronize()


if __name__ == "__main__":
    main()
