"""Per-read chunking and SIG2 chunk framing around the GPU codec.

``ReadFramingMixin.batch_inference_reads`` has the contract of the
reference's mixin (``cpu_compression.py:28-84``, inherited by the reference
GPU codec through ``main.py:215``): a read's tokens are cut into
``chunk_len``-token chunks, every chunk is range coded independently, and a
read's payload is, per chunk, a little-endian uint16 byte count followed by
the chunk's little-endian u32 words (an empty read has an empty payload).
Decoding checks every frame and the read's token count.

All reads of a call are handled together: the chunk layout is computed with
numpy, framing and parsing run in the multithreaded host library
(``sigcomp_amd._host``: ``sc_host_frame`` / ``sc_host_parse``), and the codec
sees every chunk of the call at once (``compress_flat`` / ``decompress_flat``
when it has them, else ``compress_chunks`` / ``decompress_chunks``).
"""

from __future__ import annotations

import numpy as np

from . import _host


def token_array(values) -> np.ndarray:
    """One read's or chunk's tokens as a contiguous uint8 array; raises
    ValueError unless they are a 1-D integer sequence in [0, 255]."""
    a = np.asarray(values)
    if a.ndim != 1:
        raise ValueError(f"token sequences are one-dimensional, got shape {a.shape}")
    if a.size:
        if a.dtype.kind not in "iu":
            raise ValueError(f"tokens must be integers, got dtype {a.dtype}")
        if a.dtype != np.uint8 and (int(a.min()) < 0 or int(a.max()) > 255):
            raise ValueError("tokens must lie in [0, 255]")
    return np.ascontiguousarray(a, dtype=np.uint8)


def chunk_layout(read_lengths: np.ndarray, chunk_len: int):
    """Chunks of every read in read order -> (first chunk of each read
    [n_reads + 1], token count of each chunk [n_chunks] int32)."""
    read_lengths = np.asarray(read_lengths, np.int64)
    per_read = -(-read_lengths // chunk_len)
    first = np.zeros(len(read_lengths) + 1, np.int64)
    np.cumsum(per_read, out=first[1:])
    sizes = np.full(int(first[-1]), chunk_len, np.int32)
    nonempty = per_read > 0
    # a read's last chunk holds what the full ones leave
    sizes[first[1:][nonempty] - 1] = (read_lengths[nonempty] - (per_read[nonempty] - 1) * chunk_len)
    return first, sizes


def _words_of(encoded) -> tuple:
    """Encoded chunk byte strings -> (u32 words, offsets, counts)."""
    cnt = np.fromiter((len(e) // 4 for e in encoded), np.int32, count=len(encoded))
    off = np.zeros(len(encoded), np.int64)
    np.cumsum(cnt[:-1], out=off[1:])
    words = np.frombuffer(b"".join(encoded), "<u4").astype(np.uint32) if cnt.sum() else np.zeros(0, np.uint32)
    return words, off, cnt


class ReadFramingMixin:
    """Drop-in for the reference mixin: ``batch_inference_reads`` on top of
    the codec's chunk calls and ``self.chunk_len``."""

    def batch_inference_reads(self, list_of_reads=None, list_of_compressed_reads=None,
                              list_of_lengths=None, batch_size=64, use_tqdm=False, prob_quant=0):
        if batch_size < 1:
            raise ValueError("batch_size must be positive")
        if list_of_reads is not None:
            return self._compress_reads(list_of_reads, batch_size, use_tqdm)
        if list_of_compressed_reads is None or list_of_lengths is None:
            raise ValueError("Compressed reads and token lengths are required")
        if len(list_of_compressed_reads) != len(list_of_lengths):
            raise ValueError("Compressed read and token length counts differ")
        return self._decompress_reads(list_of_compressed_reads, list_of_lengths, batch_size, use_tqdm)

    def _compress_reads(self, list_of_reads, batch_size, use_tqdm):
        reads = [token_array(r) for r in list_of_reads]
        cl = int(self.chunk_len)
        first, sizes = chunk_layout([r.size for r in reads], cl)
        if hasattr(self, "compress_reads_batches"):
            # batches of whole reads, each framed while the codec works on later ones
            out = []
            for r0, r1, words, word_off, word_cnt in self.compress_reads_batches(reads, batch_size, use_tqdm):
                buf, bounds = _host.frame(words, word_off, word_cnt)
                cf = first[r0:r1 + 1] - first[r0]
                out.extend(buf[bounds[cf[i]]:bounds[cf[i + 1]]].tobytes() for i in range(r1 - r0))
            return out
        tokens = np.concatenate(reads) if reads else np.zeros(0, np.uint8)
        if hasattr(self, "compress_flat"):
            words, word_off, word_cnt = self.compress_flat(tokens, sizes, batch_size, use_tqdm=use_tqdm)
        else:
            starts = np.zeros(len(sizes), np.int64)
            np.cumsum(sizes[:-1], out=starts[1:])
            encoded = self.compress_chunks([tokens[s:s + n] for s, n in zip(starts, sizes)],
                                           max_batch_size=batch_size, use_tqdm=use_tqdm)
            words, word_off, word_cnt = _words_of(encoded)
        buf, bounds = _host.frame(words, word_off, word_cnt)
        return [buf[bounds[first[r]]:bounds[first[r + 1]]].tobytes() for r in range(len(reads))]

    def _decompress_reads(self, payloads, list_of_lengths, batch_size, use_tqdm):
        bad_len = next((i for i, x in enumerate(list_of_lengths) if int(x) != x or x < 0), None)
        if bad_len is not None:
            # reads are checked in order: a framing error of an earlier read
            # is raised first
            _host.parse(payloads[:bad_len], [int(x) for x in list_of_lengths[:bad_len]], int(self.chunk_len))
            raise ValueError("Token lengths must be nonnegative integers")
        n_tok = np.fromiter((int(x) for x in list_of_lengths), np.int64, count=len(list_of_lengths))
        staging = getattr(self, "pinned_words", None)
        pinned = staging(_host.parse_word_count(payloads)) if staging else None
        pr = _host.parse(payloads, n_tok, int(self.chunk_len),
                         words_out=pinned.numpy().view(np.uint32) if pinned is not None else None)
        if hasattr(self, "decompress_flat"):
            kw = {"words_pinned": pinned} if pinned is not None else {}
            tok, tok_off = self.decompress_flat(pr["words"], pr["word_off"], pr["word_cnt"], pr["tok_cnt"],
                                                use_tqdm=use_tqdm, **kw)
        else:
            w = pr["words"]
            encoded = [w[o:o + c].tobytes() for o, c in zip(pr["word_off"], pr["word_cnt"])]
            dec = self.decompress_chunks(encoded, [int(x) for x in pr["tok_cnt"]], max_batch_size=batch_size,
                                         use_tqdm=use_tqdm)
            tok = np.concatenate(dec) if dec else np.zeros(0, np.uint8)
            tok_off = np.zeros(len(dec), np.int64)
            np.cumsum(pr["tok_cnt"][:-1], out=tok_off[1:])
        out = []
        for r, n in enumerate(n_tok):
            start = tok_off[pr["chunk_begin"][r]] if pr["frames"][r] else 0
            out.append(tok[start:start + n] if n else np.empty(0, dtype=np.uint8))
        return out
