"""TEST INFRASTRUCTURE ONLY -- never imported by the product (sigcomp_amd/).

Python restatement of the SIG2 per-read chunk framing of the reference's
``ReadFramingMixin.batch_inference_reads`` (``cpu_compression.py:28-84``),
the checker for the host library's ``sc_host_frame`` / ``sc_host_parse``
(``tests/test_host.py``).  The format: a read's payload is, for each chunk
of ``chunk_len`` tokens in order, the chunk's byte length as little-endian
uint16 followed by its little-endian u32 words; an empty read has an empty
payload.  Parsing rejects a missing or truncated length, a length that is
zero, not a multiple of four or past the end, and bytes left over once the
read's tokens are covered.  Error messages carry the reference's wording
(``cpu_compression.py:50-52,67-79``) so the host library's can be compared.

Pinned by the reference-written payloads in ``tests/golden/e2e_reads.npz``
(``tests/test_oracle.py``).
"""

from __future__ import annotations

import numpy as np

MAX_FRAME = 0xFFFF


def chunk_views(tokens, chunk_len: int) -> list:
    """Consecutive slices of at most chunk_len tokens (none for an empty read)."""
    tokens = np.ascontiguousarray(tokens, np.uint8)
    starts = range(0, tokens.size, chunk_len)
    return [tokens[s:s + chunk_len] for s in starts]


def frame(encoded_chunks) -> bytes:
    """Concatenate <H byte length + bytes for each encoded chunk."""
    sizes = [len(e) for e in encoded_chunks]
    if any(s > MAX_FRAME for s in sizes):
        raise ValueError("Compressed chunk exceeds the SIG2 uint16 frame; "
                         "compress with a smaller --chunk-len")
    out = bytearray(sum(sizes) + 2 * len(sizes))
    at = 0
    for e, s in zip(encoded_chunks, sizes):
        out[at:at + 2] = s.to_bytes(2, "little")
        out[at + 2:at + 2 + s] = e
        at += 2 + s
    return bytes(out)


def parse(data: bytes, n_tokens: int, chunk_len: int):
    """-> (encoded chunk byte strings, token count of each) of one read."""
    if int(n_tokens) != n_tokens or n_tokens < 0:
        raise ValueError("Token lengths must be nonnegative integers")
    data = bytes(data)
    n_chunks = -(-int(n_tokens) // chunk_len)
    counts = [min(chunk_len, int(n_tokens) - k * chunk_len) for k in range(n_chunks)]
    parts, at = [], 0
    for _ in counts:
        if len(data) - at < 2:
            raise ValueError("Truncated SIG2 chunk length")
        size = int.from_bytes(data[at:at + 2], "little")
        body = at + 2
        if size == 0 or size % 4 or body + size > len(data):
            raise ValueError("Invalid or truncated SIG2 range-coded chunk")
        parts.append(data[body:body + size])
        at = body + size
    if at != len(data):
        raise ValueError("Trailing SIG2 chunk data disagrees with token length")
    return parts, counts
