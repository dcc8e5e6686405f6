"""GPU codec: drop-in for the reference's ``QuantMLPCompression``.

Mirrors ``quant_mlp_export.py`` of the reference (``QuantMLPCompression``
:210-377, ``GPUBitExactMLPDecoder`` :113-141): constructed with
``(chunk_len, gpu, model_path, dim, num_dec_layers, window_size)``, exposing
``compress_chunks`` / ``decompress_chunks`` and, through
``ReadFramingMixin``, ``batch_inference_reads``.  The work runs in the gfx950
kernels of ``libsigcomp_hip.so``:

* compress: one persistent kernel runs the teacher-forced MLP over every
  step of every chunk (all tokens are known) fused with the logits ->
  frequency step, then one thread per chunk runs the range encoder and seal;
* decompress: one persistent kernel in which each workgroup owns a tile of
  chunks and runs the whole autoregressive loop for them on chip.

Chunk bytes equal ``CPUQuantMLPCompression``'s (``cpu_compression.py:178-332``).
``max_batch_size`` bounds host staging only: chunks are independent, so the
batch split does not change any output byte.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _hip
from .framing import ReadFramingMixin, token_array
from .model_io import (DEFAULT_QUANT_LOSSLESS_MODEL_PATH, DEFAULT_QUANT_LOSSY_MODEL_PATH,  # noqa: F401
                       DEFAULT_QUANT_MODEL_PATH, DEFAULT_LSB_SETTING_FOR_LOSSY_MODEL, IntModel,
                       SOS_TOKEN, VOCAB_SIZE, load_int_model)

# Chunks staged per kernel launch (bounds host/device staging memory only).
_MIN_LAUNCH_CHUNKS = 1 << 16
# Chunks per batch of the pipelined read compression (compress_reads_batches):
# enough for every compress workgroup to run hundreds of 128-token tiles.
_MIN_PIPE_CHUNKS = 1 << 13


def _progress(it, use_tqdm, desc):
    """`it`, wrapped in a tqdm progress bar when asked for (and installed)."""
    if not use_tqdm:
        return it
    try:
        from tqdm import tqdm
    except ImportError:
        return it
    return tqdm(it, desc=desc)


def _h2d(a, dev):
    """Host array -> device tensor through pinned memory, without waiting
    (stream-ordered on the current stream; torch keeps the pinned block
    until the copy is done)."""
    a = np.ascontiguousarray(a)
    pin = torch.empty(a.shape, dtype=_TORCH_DTYPE[a.dtype], pin_memory=True)
    pin.numpy()[...] = a
    return pin.to(dev, non_blocking=True)


_TORCH_DTYPE = {np.dtype(k): v for k, v in ((np.uint8, torch.uint8), (np.int8, torch.int8), (np.int16, torch.int16),
                                              (np.int32, torch.int32), (np.int64, torch.int64),
                                              (np.uint16, torch.uint16), (np.uint32, torch.uint32))}


def _to_device(a, dev):
    """Host array -> device tensor (read-only arrays, e.g. views of a bytes
    object, are copied first: torch only wraps writable memory)."""
    a = np.ascontiguousarray(a)
    if not a.flags.writeable:
        a = a.copy()
    return torch.from_numpy(a).to(dev)


class HipModel:
    """An ``IntModel`` uploaded to one GPU (owns the ``sc_model`` handle)."""

    def __init__(self, model: IntModel, device: torch.device):
        self.model = model
        self.device = torch.device(device)
        self.window = int(model.window)
        layers = (_hip.LayerDesc * len(model.layers))()
        keep = []
        for i, L in enumerate(model.layers):
            arrs = [np.ascontiguousarray(L.weight, np.int8), np.ascontiguousarray(L.bias, np.int32),
                    np.ascontiguousarray(L.m0, np.int64), np.ascontiguousarray(L.shift, np.int32)]
            keep.extend(arrs)
            layers[i] = _hip.LayerDesc(L.n, L.k, arrs[0].ctypes.data, arrs[1].ctypes.data,
                                       arrs[2].ctypes.data, arrs[3].ctypes.data, int(L.relu))
        emb = np.ascontiguousarray(model.emb, np.int8)
        lut = np.ascontiguousarray(model.exp_lut, np.int64)
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _hip.check(_hip.lib().sc_model_create(emb.ctypes.data, emb.shape[0], emb.shape[1],
                                                  self.window, layers, len(model.layers),
                                                  lut.ctypes.data, self.device.index or 0,
                                                  ctypes.byref(handle)))
        self.handle = handle
        self.exp_lut = torch.from_numpy(lut.copy()).to(self.device)
        # MLP core of the kernels (sc_model_core): 2 = pipelined with per-tensor
        # requant constants (every kernel), 1 = pipelined for the explicit-context
        # kernels only, 0 = plain, 3 = generic (an architecture other than the
        # bundled one)
        self.core = int(_hip.lib().sc_model_core(handle))
        self.pipelined = self.core in (1, 2)

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                _hip.lib().sc_model_destroy(h)
            except Exception:
                pass
            self.handle = None

    # ---- explicit windows -------------------------------------------------

    def forward_windows(self, ctx: torch.Tensor, out: str = "logits") -> torch.Tensor:
        """ctx int64 [rows, window] (device) -> int8 logits [rows, 256] or int32 CDF [rows, 257]."""
        if ctx.ndim != 2 or ctx.shape[1] != self.window:
            raise ValueError("context windows must be a [rows, window_size] tensor")
        ctx = ctx.to(self.device, torch.int64).contiguous()
        rows = ctx.shape[0]
        status = torch.zeros(1, dtype=torch.int32, device=self.device)
        with torch.cuda.device(self.device):
            if out == "logits":
                res = torch.empty((rows, VOCAB_SIZE), dtype=torch.int8, device=self.device)
                fn = _hip.lib().sc_mlp_forward
            else:
                res = torch.empty((rows, VOCAB_SIZE + 1), dtype=torch.int32, device=self.device)
                fn = _hip.lib().sc_mlp_forward_cdf
            _hip.check(fn(self.handle, _hip.ptr(ctx), rows, _hip.ptr(res), _hip.ptr(status),
                          _hip.stream_ptr()))
        if int(status.item()) != 0:
            raise ValueError("context tokens must be in [0, 256]")
        return res


class GPUBitExactMLPDecoder:
    """``quant_mlp_export.py:113-141``: the integer MLP on explicit windows."""

    def __init__(self, hip_model: HipModel, output_scale: float):
        self.hip = hip_model
        self.window_size = hip_model.window
        self.vocab_size = SOS_TOKEN + 1
        self.output_scale = torch.tensor(float(output_scale), dtype=torch.float32)

    def eval(self):
        return self

    def _ar_step(self, context_window: torch.Tensor) -> torch.Tensor:
        """context int64 [B, 64] -> int8 logits [B, 1, 256]."""
        return self.hip.forward_windows(context_window, "logits").unsqueeze(1)

    def forward(self, targets: torch.Tensor) -> torch.Tensor:
        """Teacher-forced logits [B, L, 256]; windows pad with the first target
        token repeated, as ``quant_mlp_export.py:122-130`` does."""
        B, L = targets.shape
        targets = targets.to(self.hip.device, torch.int64)
        pad = targets[:, :1].expand(-1, self.window_size - 1)
        windows = torch.cat([pad, targets], dim=1).unfold(1, self.window_size, 1)
        out = self.hip.forward_windows(windows.reshape(-1, self.window_size), "logits")
        return out.view(B, L, VOCAB_SIZE)

    def dequantize_logits(self, int8_logits):
        return int8_logits.float() * self.output_scale.to(int8_logits.device)


class QuantMLPCompression(ReadFramingMixin):
    DEFAULT_DIM = 256
    DEFAULT_NUM_DEC_LAYERS = 8
    DEFAULT_WINDOW_SIZE = 64

    def __init__(self, chunk_len=1024, gpu=0, model_path=None, dim=None, num_dec_layers=None,
                 window_size=None, *, model: IntModel | None = None):
        if chunk_len < 1:
            raise ValueError("chunk_len must be positive")
        dim = dim or self.DEFAULT_DIM
        num_dec_layers = num_dec_layers or self.DEFAULT_NUM_DEC_LAYERS
        window_size = window_size or self.DEFAULT_WINDOW_SIZE
        if model is None:
            model = load_int_model(model_path or DEFAULT_QUANT_MODEL_PATH, dim, num_dec_layers,
                                   window_size)
        self.gpu = int(gpu)
        self.device = f"cuda:{self.gpu}"
        self.SOS_token = SOS_TOKEN
        self.window_size = int(model.window)
        self.chunk_len = int(chunk_len)
        self.model = model
        self.hip = HipModel(model, torch.device(self.device))
        self.gpu_engine = GPUBitExactMLPDecoder(self.hip, model.output_scale)
        self._exp_lut = self.hip.exp_lut
        self.last_timing = {}

    # ------------------------------------------------------------ compress

    def compress_chunks(self, chunks, max_batch_size=64, use_perfect=False, use_tqdm=False):
        if max_batch_size < 1:
            raise ValueError("max_batch_size must be positive")
        chunks = [token_array(c) for c in chunks]
        if any(len(c) > self.chunk_len for c in chunks):
            raise ValueError("A token chunk exceeds chunk_len")
        n = len(chunks)
        if n == 0:
            return []
        lengths = np.fromiter((len(c) for c in chunks), dtype=np.int32, count=n)
        tokens = np.concatenate(chunks)
        words, word_off, word_cnt = self.compress_flat(tokens, lengths, max_batch_size, use_tqdm=use_tqdm)
        return [words[word_off[i]:word_off[i] + word_cnt[i]].tobytes() for i in range(n)]

    def compress_flat(self, tokens, lengths, max_batch_size=64, use_tqdm=False):
        """Compress chunks given as concatenated uint8 tokens and int32 chunk
        lengths -> (uint32 words of all chunks, densely packed, per-chunk
        word offsets, per-chunk word counts).  Each chunk is coded
        independently; launches cover up to max(max_batch_size, 65536)
        chunks (use_tqdm: a progress bar over them, as the reference shows
        one over its batches)."""
        tokens = np.ascontiguousarray(tokens, np.uint8)
        lengths = np.ascontiguousarray(lengths, np.int32)
        if np.any(lengths < 0) or np.any(lengths > self.chunk_len):
            raise ValueError("Chunk lengths must be in [0, chunk_len]")
        if int(lengths.sum()) != len(tokens):
            raise ValueError("Chunk lengths do not add up to the token count")
        if len(lengths) == 0:
            return np.zeros(0, np.uint32), np.zeros(0, np.int64), np.zeros(0, np.int32)
        per = max(int(max_batch_size), _MIN_LAUNCH_CHUNKS)
        parts, tok0 = [], 0
        for s in _progress(range(0, len(lengths), per), use_tqdm, "Compressing chunks (GPU)"):
            ln = lengths[s:s + per]
            nt = int(ln.sum())
            rec = self._compress_enqueue([tokens[tok0:tok0 + nt]], ln)
            self._compress_gather(rec)
            parts.append(self._compress_collect(rec))
            tok0 += nt
        if len(parts) == 1:
            return parts[0]
        words = np.concatenate([p[0] for p in parts])
        base = np.cumsum([0] + [len(p[0]) for p in parts[:-1]])
        word_off = np.concatenate([p[1] + b for p, b in zip(parts, base)])
        return words, word_off, np.concatenate([p[2] for p in parts])

    def compress_reads_batches(self, reads, max_batch_size=64, use_tqdm=False):
        """Compress every chunk of `reads` (uint8 token arrays, cut into
        chunk_len chunks), pipelined over batches of whole reads of at least
        max(max_batch_size, 8192) chunks: yields (r0, r1, words, word_off,
        word_cnt) for reads r0 .. r1-1 (dense words of their chunks in order)
        as soon as they are on the host.  All GPU work is on the current
        stream; while the caller frames batch k, the GPU compresses batch
        k + 2 (the word gather and copy of batch k + 1 queue behind it)."""
        from .framing import chunk_layout
        cl = int(self.chunk_len)
        n_tok = np.fromiter((len(r) for r in reads), np.int64, count=len(reads))
        first, sizes = chunk_layout(n_tok, cl)
        target = max(int(max_batch_size), _MIN_PIPE_CHUNKS)
        bounds = [0]
        while bounds[-1] < len(reads):
            r0 = bounds[-1]
            r1 = int(np.searchsorted(first, first[r0] + target, side="left"))
            bounds.append(min(len(reads), max(r1, r0 + 1)))
        parts = list(zip(bounds[:-1], bounds[1:]))
        recs = []
        for k, (r0, r1) in enumerate(_progress(parts, use_tqdm, "Compressing reads (GPU)")):
            recs.append(self._compress_enqueue(reads[r0:r1], sizes[first[r0]:first[r1]]))
            if k >= 1:
                self._compress_gather(recs[k - 1])
            if k >= 2:
                yield (*parts[k - 2], *self._compress_collect(recs[k - 2]))
                recs[k - 2] = None
        for k in range(max(0, len(parts) - 2), len(parts)):
            if k == len(parts) - 1:
                self._compress_gather(recs[k])
            yield (*parts[k], *self._compress_collect(recs[k]))
            recs[k] = None

    def _compress_enqueue(self, pieces, lengths):
        """Stage the concatenated token arrays `pieces` (chunks of `lengths`)
        in pinned memory, enqueue the copy and sc_compress_chunks on the
        current stream, then the copy of the word counts and status back
        (pinned); returns the batch record."""
        lengths = np.ascontiguousarray(lengths, np.int32)
        n = len(lengths)
        n_tokens = int(lengths.sum())
        dev = self.hip.device
        pin = torch.empty(max(n_tokens, 1), dtype=torch.uint8, pin_memory=True)
        if n_tokens:
            np.concatenate(pieces, out=pin.numpy()[:n_tokens]) if len(pieces) > 1 else \
                np.copyto(pin.numpy()[:n_tokens], pieces[0])
        tok_off = np.zeros(n, dtype=np.int64)
        np.cumsum(lengths[:-1], out=tok_off[1:])
        cap = lengths + 2
        word_off = np.zeros(n, dtype=np.int64)
        np.cumsum(cap[:-1], dtype=np.int64, out=word_off[1:])
        rec = {"n": n, "dev": dev}
        with torch.cuda.device(dev):
            t_tokens = pin.to(dev, non_blocking=True)
            d = lambda a: _h2d(a, dev)
            t_tok_off, t_len, t_word_off, t_cap = d(tok_off), d(lengths), d(word_off), d(cap.astype(np.int32))
            words, cnt, status, ws = self._compress_buffers(n, n_tokens, int(cap.sum()))
            _hip.check(_hip.lib().sc_compress_chunks(
                self.hip.handle, _hip.ptr(t_tokens), _hip.ptr(t_tok_off), _hip.ptr(t_len), n,
                n_tokens, _hip.ptr(words), _hip.ptr(t_word_off), _hip.ptr(t_cap), _hip.ptr(cnt),
                _hip.ptr(status), _hip.ptr(ws), ws.numel(), _hip.stream_ptr()))
            h_cnt = torch.empty(n, dtype=torch.int32, pin_memory=True)
            h_status = torch.empty(n, dtype=torch.int32, pin_memory=True)
            h_cnt.copy_(cnt, non_blocking=True)
            h_status.copy_(status, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
        rec.update(keep=(pin, t_tokens, t_tok_off, t_len, t_cap, ws), words=words, cnt=cnt, t_word_off=t_word_off,
                   h_cnt=h_cnt, h_status=h_status, ev_cnt=ev)
        return rec

    def _compress_gather(self, rec):
        """Wait for a batch's word counts, then enqueue the dense word
        gather and its copy into pinned memory."""
        rec["ev_cnt"].synchronize()
        st = rec["h_status"].numpy()
        if st.any():
            b = int(np.flatnonzero(st)[0])
            raise OverflowError(f"range-coder output capacity exceeded in stream {b}")
        n, dev = rec["n"], rec["dev"]
        cnt_np = rec["h_cnt"].numpy().copy()
        dense_off = np.zeros(n, dtype=np.int64)
        np.cumsum(cnt_np[:-1], dtype=np.int64, out=dense_off[1:])
        total = max(int(cnt_np.sum()), 1)
        with torch.cuda.device(dev):
            dense = torch.empty(total, dtype=torch.int32, device=dev)
            t_dense_off = _h2d(dense_off, dev)
            _hip.check(_hip.lib().sc_gather_words(_hip.ptr(rec["words"]), _hip.ptr(rec["t_word_off"]),
                                                  _hip.ptr(rec["cnt"]), n, _hip.ptr(dense), _hip.ptr(t_dense_off),
                                                  _hip.stream_ptr()))
            h_words = torch.empty(total, dtype=torch.int32, pin_memory=True)
            h_words.copy_(dense, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
        rec.update(keep2=(dense, t_dense_off), h_words=h_words, ev_words=ev, dense_off=dense_off, cnt_np=cnt_np)

    @staticmethod
    def _compress_collect(rec):
        """A gathered batch's (dense words, offsets, counts) on the host."""
        rec["ev_words"].synchronize()
        return rec["h_words"].numpy().view(np.uint32), rec["dense_off"], rec["cnt_np"]

    def _compress_buffers(self, n, n_tokens, n_words):
        dev = self.hip.device
        ws_bytes = int(_hip.lib().sc_compress_workspace_bytes(n_tokens, n))
        words = torch.empty(max(n_words, 1), dtype=torch.int32, device=dev)
        cnt = torch.empty(n, dtype=torch.int32, device=dev)
        status = torch.empty(n, dtype=torch.int32, device=dev)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        return words, cnt, status, ws

    # ---------------------------------------------------------- decompress

    @staticmethod
    def pinned_words(n_words):
        """A pinned int32 host tensor for n_words range-coder words (parse
        target, copied to the device without staging)."""
        return torch.empty(max(int(n_words), 1), dtype=torch.int32, pin_memory=True)

    def _decompress_workspace(self, n):
        """Per-call decode state (sc_decompress_workspace_bytes): a tensor
        from torch's stream-ordered allocator, so calls never share it."""
        nbytes = int(_hip.lib().sc_decompress_workspace_bytes(n))
        return torch.empty(nbytes, dtype=torch.uint8, device=self.hip.device)

    def decompress_chunks(self, compressed_bytes_list, valid_lengths, max_batch_size=64,
                          use_perfect=False, use_tqdm=False):
        if max_batch_size < 1:
            raise ValueError("max_batch_size must be positive")
        if len(compressed_bytes_list) != len(valid_lengths):
            raise ValueError("Compressed chunk and length counts differ")
        if any(int(n) != n or n < 0 or n > self.chunk_len for n in valid_lengths):
            raise ValueError("Chunk lengths must be integers in [0, chunk_len]")
        for data, length in zip(compressed_bytes_list, valid_lengths):
            if (length and (not data or len(data) % 4)) or (not length and data):
                raise ValueError("Invalid range-coded chunk for its token length")
        per = max(int(max_batch_size), _MIN_LAUNCH_CHUNKS)
        out = []
        for s in _progress(range(0, len(compressed_bytes_list), per), use_tqdm, "Decompressing chunks (GPU)"):
            out.extend(self._decompress_batch(compressed_bytes_list[s:s + per],
                                              valid_lengths[s:s + per]))
        return out

    def _decompress_batch(self, chunk_bytes, valid_lengths):
        n = len(chunk_bytes)
        if n == 0:
            return []
        lengths = np.asarray(valid_lengths, dtype=np.int32)
        cnt = np.fromiter((len(b) // 4 for b in chunk_bytes), dtype=np.int32, count=n)
        word_off = np.zeros(n, dtype=np.int64)
        np.cumsum(cnt[:-1], dtype=np.int64, out=word_off[1:])
        flat = (np.frombuffer(b"".join(chunk_bytes), dtype="<u4").astype(np.uint32, copy=False)
                if cnt.sum() else np.zeros(1, np.uint32))
        tok, tok_off = self.decompress_flat(flat, word_off, cnt, lengths)
        return [tok[tok_off[i]:tok_off[i] + lengths[i]].copy() for i in range(n)]

    def decompress_flat(self, words, word_off, word_cnt, lengths, use_tqdm=False, words_pinned=None):
        """Decompress chunks given as one uint32 word array with per-chunk
        word offsets / counts and token lengths -> (uint8 tokens of all
        chunks concatenated in chunk order, per-chunk token offsets).  One
        persistent-kernel call for all chunks; raises ValueError on a corrupt
        stream."""
        words = np.ascontiguousarray(words, np.uint32)
        word_off = np.ascontiguousarray(word_off, np.int64)
        cnt = np.ascontiguousarray(word_cnt, np.int32)
        lengths = np.ascontiguousarray(lengths, np.int32)
        n = len(lengths)
        if len(word_off) != n or len(cnt) != n:
            raise ValueError("Compressed chunk and length counts differ")
        if n and (np.any(lengths < 0) or np.any(lengths > self.chunk_len)):
            raise ValueError("Chunk lengths must be integers in [0, chunk_len]")
        if n and (np.any(word_off < 0) or np.any(cnt < 0) or np.any(word_off + cnt > len(words))
                  or np.any((lengths > 0) & (cnt == 0)) or np.any((lengths == 0) & (cnt > 0))):
            raise ValueError("Invalid range-coded chunk for its token length")
        tok_off = np.zeros(n, dtype=np.int64)
        if n > 1:
            np.cumsum(lengths[:-1], dtype=np.int64, out=tok_off[1:])
        n_tokens = int(lengths.sum())
        if n == 0:
            return np.zeros(0, np.uint8), tok_off
        if len(words) == 0:
            words = np.zeros(1, np.uint32)
        # longest chunks first: every workgroup then holds chunks of similar
        # length and stops at its own longest one
        order = np.argsort(-lengths, kind="stable")
        dev = self.hip.device
        len_host = np.ascontiguousarray(lengths[order])
        with torch.cuda.device(dev):
            # every copy through pinned memory, stream-ordered: the call
            # waits once, for the tokens
            if words_pinned is not None and words_pinned.data_ptr() == words.ctypes.data:
                t_words = words_pinned.to(dev, non_blocking=True)
            else:
                t_words = _h2d(words.view(np.int32), dev)
            d = lambda a: _h2d(a, dev)
            t_woff, t_cnt, t_len, t_toff = d(word_off[order]), d(cnt[order]), d(len_host), d(tok_off[order])
            tokens = torch.empty(max(n_tokens, 1), dtype=torch.uint8, device=dev)
            status = torch.empty(n, dtype=torch.int32, device=dev)
            ws = self._decompress_workspace(n)
            _hip.check(_hip.lib().sc_decompress_chunks(
                self.hip.handle, _hip.ptr(t_words), _hip.ptr(t_woff), _hip.ptr(t_cnt),
                _hip.ptr(t_len), n, _hip.ptr(tokens), _hip.ptr(t_toff), _hip.ptr(status),
                len_host.ctypes.data, _hip.ptr(ws), ws.numel(), _hip.stream_ptr()))
            h_tokens = torch.empty(max(n_tokens, 1), dtype=torch.uint8, pin_memory=True)
            h_status = torch.empty(n, dtype=torch.int32, pin_memory=True)
            h_tokens.copy_(tokens, non_blocking=True)
            h_status.copy_(status, non_blocking=True)
            torch.cuda.current_stream().synchronize()
            st = h_status.numpy()
            late = np.flatnonzero(st == _hip.SC_STATUS_SYNC_TIMEOUT)
            if len(late):
                # a split launch whose workgroups timed out waiting for each
                # other (one of them was not scheduled in time): its chunks
                # are decoded again, each an independent stream, by unsplit
                # launches that never wait between workgroups
                self._redecode_unsplit(late, word_off[order], cnt[order], len_host, tok_off[order], t_words,
                                       tokens, h_tokens, st)
        if st.any():
            bad = np.flatnonzero(st)
            if (st[bad] == _hip.SC_STATUS_SYNC_TIMEOUT).any():
                raise RuntimeError("GPU decode: the workgroups sharing a decode step timed out waiting for each other")
            raise ValueError("invalid range stream or mismatching entropy model in chunk "
                             f"{int(order[bad[0]])}")
        return h_tokens.numpy()[:n_tokens], tok_off

    def _redecode_unsplit(self, rows, woff, cnt, lens, toff, t_words, tokens, h_tokens, st):
        """Decode the chunks `rows` (indices into the sorted arrays) again with
        SC_DEC_OPT_NO_SPLIT into the same device token buffer, refresh the
        host copy and their entries of `st` (the host status array)."""
        dev = self.hip.device
        m = len(rows)
        sub_len = np.ascontiguousarray(lens[rows], np.int32)
        d = lambda a: _h2d(np.ascontiguousarray(a), dev)
        t_woff, t_cnt, t_len, t_toff = d(woff[rows]), d(cnt[rows]), d(sub_len), d(toff[rows])
        status = torch.empty(m, dtype=torch.int32, device=dev)
        ws = self._decompress_workspace(m)
        _hip.check(_hip.lib().sc_decompress_chunks_opts(
            self.hip.handle, _hip.ptr(t_words), _hip.ptr(t_woff), _hip.ptr(t_cnt), _hip.ptr(t_len), m,
            _hip.ptr(tokens), _hip.ptr(t_toff), _hip.ptr(status), sub_len.ctypes.data, _hip.ptr(ws), ws.numel(),
            _hip.SC_DEC_OPT_NO_SPLIT, _hip.stream_ptr()))
        h_tokens.copy_(tokens, non_blocking=True)
        h_sub = torch.empty(m, dtype=torch.int32, pin_memory=True)
        h_sub.copy_(status, non_blocking=True)
        torch.cuda.current_stream().synchronize()
        st[rows] = h_sub.numpy()
