"""CPU oracle for SigComp's integer codec path -- TEST INFRASTRUCTURE ONLY.

Python side of ``oracle/sc_oracle.c`` (a C restatement of the reference CPU
backend).  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or the
timed CPU baseline.  The product (``sigcomp_amd``) never imports it.

Functions and what pins them
----------------------------
=========================  ==================================  =============================================
oracle function            reference it restates               pinned by
=========================  ==================================  =============================================
``requantize``             cpu_int_kernels.py:5-14             golden MLP logits (reference ``_ar_step``);
                                                               closed-form edge cases (M0 = 2**31, shift 63,
                                                               int32 wrap of the bias add) in test_oracle
``linear``                 cpu_int_kernels.py:143-156,         reference ``_int_mm`` conformance patterns
                           cpu_int_inference.py:125-256        (cpu_int_inference.py:28-37) vs int64 numpy
                                                               matmul; ``torch._int_mm`` cross-check
``mlp_forward``            cpu_int_inference.py:270-347,       golden logits from the reference decoder on
                           quant_mlp_export.py:113-141         both bundled checkpoints (tests/golden)
``logits_to_cdf``          cpu_entropy_coding.py:73-110        golden CDFs from the reference; invariants
                                                               (sum 2**24, f >= 1, first-argmax correction)
``encode_stream``          cpu_entropy_coding.py:121-227       golden word streams from the reference
                                                               CpuRangeStepEncoder (python backend)
``decode_stream``          cpu_entropy_coding.py:230-266,      golden symbols from the reference
                           :451-497                            CpuRangeDecoder; decode(encode(x)) == x
``compress_chunks``        cpu_compression.py:178-257          golden end-to-end chunk bytes written by
                                                               composing the reference's own functions
``decompress_chunks``      cpu_compression.py:259-332          round trip against ``compress_chunks``
=========================  ==================================  =============================================
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libsc_oracle.so"
MAX_LAYERS = 16

_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")


class _Layer(ctypes.Structure):
    _fields_ = [("n", ctypes.c_int32), ("k", ctypes.c_int32),
                ("w", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("m0", ctypes.c_void_p), ("shift", ctypes.c_void_p),
                ("relu", ctypes.c_int32)]


class _Model(ctypes.Structure):
    _fields_ = [("n_layers", ctypes.c_int32), ("window", ctypes.c_int32),
                ("emb_rows", ctypes.c_int32), ("emb_dim", ctypes.c_int32),
                ("emb", ctypes.c_void_p), ("layers", _Layer * MAX_LAYERS)]


def build() -> Path:
    """Compile the oracle with its Makefile (no-op when up to date)."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB_PATH


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.sco_requantize.restype = ctypes.c_int8
        L.sco_requantize.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                                     ctypes.c_int32, ctypes.c_int32]
        L.sco_linear.argtypes = [_i8p, ctypes.c_int64, ctypes.c_int32, _i8p, ctypes.c_int32,
                                 _i32p, _i64p, _i32p, ctypes.c_int32, _i8p]
        L.sco_mlp_forward.argtypes = [ctypes.POINTER(_Model), _i32p, ctypes.c_int64, _i8p]
        L.sco_logits_to_cdf.argtypes = [_i8p, ctypes.c_int64, _i64p, _i64p]
        L.sco_frequencies.argtypes = [_i8p, _i64p, _i64p]
        L.sco_encode_stream.argtypes = [_i8p, _i32p, ctypes.c_int64, _i64p, _u32p,
                                        ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]
        L.sco_decode_stream.argtypes = [_u32p, ctypes.c_int64, _i8p, ctypes.c_int64,
                                        _i64p, _i32p]
        L.sco_compress_chunks.argtypes = [ctypes.POINTER(_Model), _i64p, _u8p, _i64p, _i32p,
                                          ctypes.c_int64, _u32p, _i64p, _i64p, _i32p, _i32p]
        L.sco_decompress_chunks.argtypes = [ctypes.POINTER(_Model), _i64p, _u32p, _i64p,
                                            _i32p, _i32p, ctypes.c_int64, _u8p, _i64p, _i32p]
        L.sco_num_threads.restype = ctypes.c_int
        L.sco_uses_vnni.restype = ctypes.c_int
        L.sco_set_num_threads.argtypes = [ctypes.c_int]
        _LIB = L
    return _LIB


def set_num_threads(n: int) -> None:
    lib().sco_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().sco_num_threads())


def uses_vnni() -> bool:
    """True when the MLP runs its AVX-512 VNNI dot products (the int_mm
    backend's instructions); SCO_NO_VNNI=1 in the environment before the
    first call selects the portable C path."""
    return bool(lib().sco_uses_vnni())


class OracleModel:
    """Holds the C view of an ``IntModel`` (arrays kept alive here)."""

    def __init__(self, model):
        if len(model.layers) > MAX_LAYERS:
            raise ValueError("too many layers for the oracle")
        self.model = model
        self._keep = []
        c = _Model()
        c.n_layers = len(model.layers)
        c.window = int(model.window)
        emb = np.ascontiguousarray(model.emb, dtype=np.int8)
        c.emb_rows, c.emb_dim = emb.shape
        c.emb = emb.ctypes.data
        self._keep.append(emb)
        for i, layer in enumerate(model.layers):
            arrs = [np.ascontiguousarray(layer.weight, np.int8),
                    np.ascontiguousarray(layer.bias, np.int32),
                    np.ascontiguousarray(layer.m0, np.int64),
                    np.ascontiguousarray(layer.shift, np.int32)]
            self._keep.extend(arrs)
            c.layers[i] = _Layer(layer.n, layer.k, arrs[0].ctypes.data, arrs[1].ctypes.data,
                                 arrs[2].ctypes.data, arrs[3].ctypes.data, int(layer.relu))
        self.c = c
        self.lut = np.ascontiguousarray(model.exp_lut, dtype=np.int64)
        self.window = int(model.window)


def requantize(acc, bias, m0, shift, relu) -> int:
    return int(lib().sco_requantize(int(acc), int(bias), int(m0), int(shift), int(relu)))


def linear(x, layer) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.int8)
    out = np.empty((x.shape[0], layer.n), dtype=np.int8)
    lib().sco_linear(x, x.shape[0], layer.k, np.ascontiguousarray(layer.weight, np.int8),
                     layer.n, np.ascontiguousarray(layer.bias, np.int32),
                     np.ascontiguousarray(layer.m0, np.int64),
                     np.ascontiguousarray(layer.shift, np.int32), int(layer.relu), out)
    return out


def mlp_forward(om: OracleModel, ctx) -> np.ndarray:
    """int8 logits [rows, 256] for explicit token windows ``ctx`` [rows, window]."""
    ctx = np.ascontiguousarray(ctx, dtype=np.int32)
    if ctx.ndim != 2 or ctx.shape[1] != om.window:
        raise ValueError("context must be [rows, window]")
    out = np.empty((ctx.shape[0], 256), dtype=np.int8)
    st = lib().sco_mlp_forward(ctypes.byref(om.c), ctx, ctx.shape[0], out)
    if st:
        raise ValueError(f"oracle MLP failed with status {st}")
    return out


def frequencies(logits_row, lut) -> np.ndarray:
    out = np.empty(256, dtype=np.int64)
    lib().sco_frequencies(np.ascontiguousarray(logits_row, np.int8),
                          np.ascontiguousarray(lut, np.int64), out)
    return out


def logits_to_cdf(logits, lut) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.int8)
    out = np.empty((logits.shape[0], 257), dtype=np.int64)
    lib().sco_logits_to_cdf(logits, logits.shape[0], np.ascontiguousarray(lut, np.int64), out)
    return out


def encode_stream(logits, symbols, lut, capacity=None) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.int8)
    symbols = np.ascontiguousarray(symbols, dtype=np.int32)
    n = symbols.shape[0]
    cap = n + 32 if capacity is None else int(capacity)
    out = np.zeros(max(cap, 1), dtype=np.uint32)
    nw = ctypes.c_int64(0)
    st = lib().sco_encode_stream(logits, symbols, n, np.ascontiguousarray(lut, np.int64),
                                 out, cap, ctypes.byref(nw))
    if st == 1:
        raise OverflowError("range-coder output capacity exceeded")
    if st:
        raise ValueError(f"oracle encoder failed with status {st}")
    return out[:nw.value].copy()


def decode_stream(words, logits, lut) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.uint32)
    logits = np.ascontiguousarray(logits, dtype=np.int8)
    out = np.zeros(logits.shape[0], dtype=np.int32)
    st = lib().sco_decode_stream(words if words.size else np.zeros(1, np.uint32), words.size,
                                 logits, logits.shape[0], np.ascontiguousarray(lut, np.int64), out)
    if st:
        raise ValueError("invalid range stream or mismatching entropy model")
    return out


def compress_chunks(om: OracleModel, chunks) -> list:
    """list of uint8 token chunks -> list of range-coded chunk bytes."""
    chunks = [np.ascontiguousarray(c, dtype=np.uint8) for c in chunks]
    n = len(chunks)
    if n == 0:
        return []
    lengths = np.array([len(c) for c in chunks], dtype=np.int32)
    tok_off = np.zeros(n, dtype=np.int64)
    tok_off[1:] = np.cumsum(lengths[:-1], dtype=np.int64)
    tokens = np.concatenate(chunks) if lengths.sum() else np.zeros(1, np.uint8)
    cap = lengths.astype(np.int64) + 2
    word_off = np.zeros(n, dtype=np.int64)
    word_off[1:] = np.cumsum(cap[:-1])
    words = np.zeros(int(cap.sum()), dtype=np.uint32)
    cnt = np.zeros(n, dtype=np.int32)
    status = np.zeros(n, dtype=np.int32)
    st = lib().sco_compress_chunks(ctypes.byref(om.c), om.lut, tokens, tok_off, lengths, n,
                                   words, word_off, cap, cnt, status)
    if st:
        raise ValueError(f"oracle compress failed with status {st}")
    return [words[word_off[i]:word_off[i] + cnt[i]].astype("<u4").tobytes() for i in range(n)]


def decompress_chunks(om: OracleModel, chunk_bytes, lengths) -> list:
    n = len(chunk_bytes)
    if n == 0:
        return []
    lengths = np.asarray(lengths, dtype=np.int32)
    streams = [np.frombuffer(b, dtype="<u4").astype(np.uint32) for b in chunk_bytes]
    cnt = np.array([len(s) for s in streams], dtype=np.int32)
    word_off = np.zeros(n, dtype=np.int64)
    word_off[1:] = np.cumsum(cnt[:-1], dtype=np.int64)
    words = np.concatenate(streams) if cnt.sum() else np.zeros(1, np.uint32)
    tok_off = np.zeros(n, dtype=np.int64)
    tok_off[1:] = np.cumsum(lengths[:-1], dtype=np.int64)
    tokens = np.zeros(max(int(lengths.sum()), 1), dtype=np.uint8)
    status = np.zeros(n, dtype=np.int32)
    st = lib().sco_decompress_chunks(ctypes.byref(om.c), om.lut, words, word_off, cnt, lengths,
                                     n, tokens, tok_off, status)
    if st:
        raise ValueError(f"invalid range stream in chunk {int(np.flatnonzero(status)[0])}")
    return [tokens[tok_off[i]:tok_off[i] + lengths[i]].copy() for i in range(n)]


def cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1
