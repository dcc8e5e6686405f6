"""Per-read chunking and ``<H``-length framing of range-coded chunks.

Restates ``ReadFramingMixin.batch_inference_reads``
(``cpu_compression.py:28-84``), which the reference GPU codec inherits
through its MRO (``main.py:215``): each read's tokens are cut into
``chunk_len`` chunks; a read's payload is the concatenation, per chunk, of
a little-endian uint16 byte length and the chunk's little-endian u32 words.
An empty read has an empty payload.  Decoding validates nonzero sizes that
are multiples of four, no truncation and no trailing bytes.
"""

from __future__ import annotations

import struct

import numpy as np

_CHUNK_LENGTH = struct.Struct("<H")


def as_symbols(values) -> np.ndarray:
    """``cpu_compression.py:18-25``: one-dimensional integer tokens in [0, 255]."""
    values = np.asarray(values)
    if values.ndim != 1:
        raise ValueError("Each token sequence must be one-dimensional")
    if values.size and (values.dtype.kind not in "iu" or np.any(values < 0) or np.any(values > 255)):
        raise ValueError("Signal tokens must be integers in [0, 255]")
    return np.ascontiguousarray(values, dtype=np.uint8)


def split_into_chunks(tokens, chunk_len: int) -> list:
    tokens = as_symbols(tokens)
    return [tokens[i:i + chunk_len] for i in range(0, len(tokens), chunk_len)]


def frame_chunks(encoded_chunks) -> bytes:
    framed = bytearray()
    for chunk in encoded_chunks:
        if len(chunk) > 65535:
            raise ValueError("Compressed chunk exceeds the SIG2 uint16 frame; "
                             "compress with a smaller --chunk-len")
        framed.extend(_CHUNK_LENGTH.pack(len(chunk)))
        framed.extend(chunk)
    return bytes(framed)


def parse_framed(data: bytes, length: int, chunk_len: int):
    """-> (list of chunk byte strings, list of chunk token counts)."""
    if int(length) != length or length < 0:
        raise ValueError("Token lengths must be nonnegative integers")
    chunks, lengths = [], []
    remaining, pos = int(length), 0
    while remaining:
        if pos + _CHUNK_LENGTH.size > len(data):
            raise ValueError("Truncated SIG2 chunk length")
        size, = _CHUNK_LENGTH.unpack_from(data, pos)
        pos += _CHUNK_LENGTH.size
        if size == 0 or size % 4 or pos + size > len(data):
            raise ValueError("Invalid or truncated SIG2 range-coded chunk")
        count = min(chunk_len, remaining)
        chunks.append(data[pos:pos + size])
        lengths.append(count)
        pos += size
        remaining -= count
    if pos != len(data):
        raise ValueError("Trailing SIG2 chunk data disagrees with token length")
    return chunks, lengths


class ReadFramingMixin:
    """Drop-in for the reference mixin: ``batch_inference_reads`` on top of
    ``self.compress_chunks`` / ``self.decompress_chunks`` and ``self.chunk_len``.

    Codecs that also provide ``compress_flat`` / ``decompress_flat`` (the GPU
    codec does) take the batched path: chunking, framing and parsing of all
    reads in one call each to the host library (``sigcomp_amd._host``), with
    the same bytes and the same errors."""

    def batch_inference_reads(self, list_of_reads=None, list_of_compressed_reads=None,
                              list_of_lengths=None, batch_size=64, use_tqdm=False, prob_quant=0):
        if batch_size < 1:
            raise ValueError("batch_size must be positive")
        flat = hasattr(self, "compress_flat") and hasattr(self, "decompress_flat")
        chunks, lengths, mapping = [], [], []
        if list_of_reads is not None:
            if flat:
                return self._compress_reads_flat(list_of_reads, batch_size)
            for read in list_of_reads:
                begin = len(chunks)
                chunks.extend(split_into_chunks(read, self.chunk_len))
                mapping.append((begin, len(chunks)))
            encoded = self.compress_chunks(chunks, max_batch_size=batch_size, use_tqdm=use_tqdm)
            return [frame_chunks(encoded[b:e]) for b, e in mapping]

        if list_of_compressed_reads is None or list_of_lengths is None:
            raise ValueError("Compressed reads and token lengths are required")
        if len(list_of_compressed_reads) != len(list_of_lengths):
            raise ValueError("Compressed read and token length counts differ")
        if flat:
            return self._decompress_reads_flat(list_of_compressed_reads, list_of_lengths)
        for data, length in zip(list_of_compressed_reads, list_of_lengths):
            begin = len(chunks)
            parts, counts = parse_framed(data, length, self.chunk_len)
            chunks.extend(parts)
            lengths.extend(counts)
            mapping.append((begin, len(chunks)))
        decoded = self.decompress_chunks(chunks, lengths, max_batch_size=batch_size,
                                         use_tqdm=use_tqdm)
        return [np.concatenate(decoded[b:e]) if e > b else np.empty(0, dtype=np.uint8)
                for b, e in mapping]

    def _compress_reads_flat(self, list_of_reads, batch_size):
        from . import _host
        reads = [as_symbols(r) for r in list_of_reads]
        cl = int(self.chunk_len)
        lens = np.fromiter((len(r) for r in reads), np.int64, count=len(reads))
        nch = (lens + cl - 1) // cl
        chunk_begin = np.zeros(len(reads) + 1, np.int64)
        np.cumsum(nch, out=chunk_begin[1:])
        n_chunks = int(chunk_begin[-1])
        chunk_len = np.full(n_chunks, cl, np.int32)
        last = chunk_begin[1:][nch > 0] - 1
        chunk_len[last] = (lens[nch > 0] - (nch[nch > 0] - 1) * cl).astype(np.int32)
        tokens = np.concatenate(reads) if reads else np.zeros(0, np.uint8)
        words, word_off, word_cnt = self.compress_flat(tokens, chunk_len, batch_size)
        buf, bounds = _host.frame(words, word_off, word_cnt)
        return [buf[bounds[chunk_begin[r]]:bounds[chunk_begin[r + 1]]].tobytes() for r in range(len(reads))]

    def _decompress_reads_flat(self, payloads, list_of_lengths):
        from . import _host
        bad_len = next((i for i, x in enumerate(list_of_lengths) if int(x) != x or x < 0), None)
        if bad_len is not None:
            # the reference checks reads in order: a framing error of an
            # earlier read is raised first
            _host.parse(payloads[:bad_len], [int(x) for x in list_of_lengths[:bad_len]], int(self.chunk_len))
            raise ValueError("Token lengths must be nonnegative integers")
        tokens = np.fromiter((int(x) for x in list_of_lengths), np.int64, count=len(list_of_lengths))
        pr = _host.parse(payloads, tokens, int(self.chunk_len))
        tok, tok_off = self.decompress_flat(pr["words"], pr["word_off"], pr["word_cnt"], pr["tok_cnt"])
        out = []
        for r, n in enumerate(tokens):
            c = pr["chunk_begin"][r]
            start = tok_off[c] if pr["frames"][r] else 0
            out.append(tok[start:start + n] if n else np.empty(0, dtype=np.uint8))
        return out
