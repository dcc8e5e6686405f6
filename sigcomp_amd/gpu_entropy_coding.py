"""GPU entropy coding: drop-in for the reference's ``gpu_entropy_coding`` module.

Same names and call contracts as ``gpu_entropy_coding.py`` of the reference
(``build_integer_exp_lut`` :8-22, ``int8_logits_to_cdf`` :25-51,
``GpuRangeStepEncoder`` :255-303, ``GpuRangeDecoder`` :400-454), executed by
the gfx950 kernels of ``libsigcomp_hip.so``.  Differences, all toward the
reference CPU backend's stricter behaviour (``cpu_entropy_coding.py``):
encoding after ``seal()`` raises, sealing twice emits nothing, and capacity
overflows / invalid streams / out-of-range symbols are flagged per stream and
raised as ``OverflowError`` / ``ValueError`` at the next host sync point
(``get_compressed()``, ``check()``).
"""

from __future__ import annotations

import numpy as np
import torch

from . import _hip
from .model_io import build_integer_exp_lut as _build_lut_np

PRECISION = 24
VOCAB_SIZE = 256


def build_integer_exp_lut(output_scale, lut_precision_bits=38):
    """int64 [256] CPU tensor ``max(int(exp(-i*s) * 2**38), 0)`` (decimal, 50 digits)."""
    return torch.from_numpy(_build_lut_np(output_scale, lut_precision_bits))


def quantize_probs_to_cdf(probs, precision=PRECISION, deterministic=False):
    """Float probabilities [..., V] -> int64 CDF [..., V + 1] summing to
    2**precision (``gpu_entropy_coding.py:54-75``; no caller on the codec
    path, kept for the module's interface).  Each frequency is
    floor(p * 2**precision) in the tensor's own float type, at least 1; the
    surplus or deficit against 2**precision is taken from the first largest
    frequency (``deterministic`` selects that index explicitly in the
    reference; torch's argmax already returns the first maximum, so both
    settings give the same table).  Runs where `probs` lives."""
    total = 1 << int(precision)
    freqs = torch.floor(probs * total).to(torch.int64).clamp_min(1)
    excess = freqs.sum(dim=-1, keepdim=True) - total
    freqs.scatter_add_(-1, freqs.argmax(dim=-1, keepdim=True), -excess)
    cdf = torch.zeros(*freqs.shape[:-1], freqs.shape[-1] + 1, dtype=torch.int64, device=freqs.device)
    torch.cumsum(freqs, dim=-1, out=cdf[..., 1:])
    return cdf


def _device_of(t: torch.Tensor) -> torch.device:
    if not t.is_cuda:
        raise ValueError("GPU entropy coding needs CUDA (HIP) tensors")
    return t.device


def _lut_on(exp_lut, device) -> torch.Tensor:
    lut = torch.as_tensor(exp_lut, dtype=torch.int64)
    if lut.shape != (VOCAB_SIZE,):
        raise ValueError("exp_lut must have shape (256,)")
    return lut.to(device).contiguous()


def int8_logits_to_cdf(int8_logits, exp_lut, precision=PRECISION):
    """int8 logits [B, 256] (device) -> int64 CDF [B, 257] (``gpu_entropy_coding.py:25-51``)."""
    if precision != PRECISION:
        raise ValueError("the SigComp stream format requires 24-bit precision")
    if int8_logits.dtype != torch.int8 or int8_logits.ndim != 2 or int8_logits.shape[1] != VOCAB_SIZE:
        raise ValueError("int8_logits must be an int8 tensor of shape (batch, 256)")
    dev = _device_of(int8_logits)
    logits = int8_logits.contiguous()
    lut = _lut_on(exp_lut, dev)
    out = torch.empty((logits.shape[0], VOCAB_SIZE + 1), dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        _hip.check(_hip.lib().sc_logits_to_cdf(_hip.ptr(logits), logits.shape[0], _hip.ptr(lut),
                                               _hip.ptr(out), _hip.stream_ptr()))
    return out


class GpuRangeStepEncoder:
    """Per-stream range encoders advanced one time step per call."""

    def __init__(self, B, max_words, device="cuda"):
        if B < 0 or max_words < 2:
            raise ValueError("B must be nonnegative and max_words must be at least two")
        self.B = int(B)
        self.max_words = int(max_words)
        self.device = torch.device(device)
        kw = dict(device=self.device)
        self.state_lower = torch.zeros(self.B, dtype=torch.int64, **kw)
        self.state_range = torch.full((self.B,), -1, dtype=torch.int64, **kw)
        self.num_inverted = torch.zeros(self.B, dtype=torch.int32, **kw)
        self.first_inv_word = torch.zeros(self.B, dtype=torch.int32, **kw)
        self.output_words = torch.zeros((self.B, self.max_words), dtype=torch.int32, **kw)
        self.write_pos = torch.zeros(self.B, dtype=torch.int32, **kw)
        self.status = torch.zeros(self.B, dtype=torch.int32, **kw)
        self._state = _hip.EncoderState(
            _hip.ptr(self.state_lower), _hip.ptr(self.state_range), _hip.ptr(self.num_inverted),
            _hip.ptr(self.first_inv_word), _hip.ptr(self.write_pos), _hip.ptr(self.status))
        self._sealed = False

    def encode_step_int8(self, int8_logits, exp_lut, symbols, valid_lens_tensor, t):
        if self._sealed:
            raise ValueError("cannot encode after seal()")
        if t < 0:
            raise ValueError("t must be nonnegative")
        if int8_logits.dtype != torch.int8 or tuple(int8_logits.shape) != (self.B, VOCAB_SIZE):
            raise ValueError("int8_logits must have shape (batch, 256)")
        logits = int8_logits.to(self.device).contiguous()
        syms = torch.as_tensor(symbols).to(self.device, torch.int64).contiguous()
        valid = torch.as_tensor(valid_lens_tensor).to(self.device, torch.int64).contiguous()
        if syms.shape != (self.B,) or valid.shape != (self.B,):
            raise ValueError("symbols and valid_lens must have shape (batch,)")
        lut = _lut_on(exp_lut, self.device)
        with torch.cuda.device(self.device):
            _hip.check(_hip.lib().sc_encode_step(
                _hip.ptr(logits), _hip.ptr(lut), _hip.ptr(syms), _hip.ptr(valid), int(t), self.B,
                self._state, _hip.ptr(self.output_words), self.max_words, _hip.stream_ptr()))

    def seal(self):
        if self._sealed:
            return
        with torch.cuda.device(self.device):
            _hip.check(_hip.lib().sc_encode_seal(self.B, self._state, _hip.ptr(self.output_words),
                                                 self.max_words, _hip.stream_ptr()))
        self._sealed = True

    def check(self):
        status = self.status.cpu().numpy()
        bad = np.flatnonzero(status)
        if bad.size:
            b = int(bad[0])
            if status[b] == _hip.SC_STATUS_CAPACITY:
                raise OverflowError(f"range-coder output capacity exceeded in stream {b}; "
                                    "increase max_words")
            raise ValueError(f"active symbols must be in [0, 255] (stream {b})")

    def get_compressed(self):
        """Seal if needed, then one ``bytes`` (little-endian u32 words) per stream."""
        self.seal()
        torch.cuda.synchronize(self.device)
        self.check()
        pos = self.write_pos.cpu().numpy()
        words = self.output_words.cpu().numpy().view(np.uint32)
        return [words[b, :int(pos[b])].astype("<u4", copy=False).tobytes() for b in range(self.B)]


class GpuRangeDecoder:
    """Per-stream range decoders over a flat word array."""

    def __init__(self, compressed_bytes_list, device="cuda"):
        self.B = len(compressed_bytes_list)
        self.device = torch.device(device)
        points = np.zeros(self.B, dtype=np.uint64)
        read_pos = np.zeros(self.B, dtype=np.int64)
        end_pos = np.zeros(self.B, dtype=np.int64)
        streams = []
        offset = 0
        for b, data in enumerate(compressed_bytes_list):
            if len(data) % 4:
                raise ValueError("compressed range stream length must be a multiple of four bytes")
            words = np.frombuffer(data, dtype="<u4").astype(np.uint32)
            point = 0
            for i in range(min(2, len(words))):
                point = (point << 32) | int(words[i])
            if len(words) == 1:
                point <<= 32
            points[b] = point
            read_pos[b] = offset + min(2, len(words))
            offset += len(words)
            end_pos[b] = offset
            streams.append(words)
        flat = np.concatenate(streams) if streams and offset else np.zeros(1, dtype=np.uint32)
        kw = dict(device=self.device)
        self.comp_words = torch.from_numpy(flat.view(np.int32)).to(**kw)
        self.read_pos = torch.from_numpy(read_pos).to(**kw)
        self.end_pos = torch.from_numpy(end_pos).to(**kw)
        self.point = torch.from_numpy(points.view(np.int64)).to(**kw)
        self.state_lower = torch.zeros(self.B, dtype=torch.int64, **kw)
        self.state_range = torch.full((self.B,), -1, dtype=torch.int64, **kw)
        self.symbols_out = torch.zeros(self.B, dtype=torch.int64, **kw)
        self.status = torch.zeros(self.B, dtype=torch.int32, **kw)
        self._state = _hip.DecoderState(
            _hip.ptr(self.state_lower), _hip.ptr(self.state_range), _hip.ptr(self.point),
            _hip.ptr(self.read_pos), _hip.ptr(self.end_pos), _hip.ptr(self.status))

    def decode_step_int8(self, int8_logits, exp_lut, valid_lens_tensor, t):
        """Decoded symbols of step ``t`` (int64 [B]; 256 for inactive streams).

        The returned tensor is reused by the next call, as in the reference.
        """
        if int8_logits.dtype != torch.int8 or tuple(int8_logits.shape) != (self.B, VOCAB_SIZE):
            raise ValueError("int8_logits must have shape (batch, 256)")
        if t < 0:
            raise ValueError("t must be nonnegative")
        logits = int8_logits.to(self.device).contiguous()
        valid = torch.as_tensor(valid_lens_tensor).to(self.device, torch.int64).contiguous()
        if valid.shape != (self.B,):
            raise ValueError("valid_lens must have shape (batch,)")
        lut = _lut_on(exp_lut, self.device)
        with torch.cuda.device(self.device):
            _hip.check(_hip.lib().sc_decode_step(
                _hip.ptr(logits), _hip.ptr(lut), _hip.ptr(valid), int(t), self.B, self._state,
                _hip.ptr(self.comp_words), _hip.ptr(self.symbols_out), _hip.stream_ptr()))
        return self.symbols_out

    def check(self):
        status = self.status.cpu().numpy()
        bad = np.flatnonzero(status)
        if bad.size:
            raise ValueError(f"invalid range stream or mismatching entropy model in stream {int(bad[0])}")
