"""Caller-side signal transforms around the codec (host C++, multithreaded).

These produce the 8-bit token streams that the GPU codec compresses and
restore int16 samples from them, as ``main.py:129-171`` (delta / zigzag /
lossy LSB transforms) and ``main.py:504-546`` (small/large split and
reassembly) do with numpy, here through libsigcomp_host.so
(include/sigcomp_host.h):

* ``np.diff`` on int16 wraps modulo 2**16; zigzag maps the int16 deltas to
  uint16; values < 256 are the "small" tokens, the rest are "large"
  (stored as ``value - 256``) with gap-coded uint32 positions;
* with ``lsb > 0`` the samples are first rounded to a multiple of ``2**lsb``
  and shifted right by ``lsb`` (``_lossy_encode(_reduce_lsb(...))``,
  ``main.py:862-864``), and shifted back after reassembly (``main.py:1164``).

The large values and positions are returned uncoded; ``sigcomp_amd.rice``
Rice-codes them for the archive (the reference uses the third-party
``fast-rice==0.1.0`` package there, ``main.py:174-186``).
"""

from __future__ import annotations

import numpy as np

from . import _host


def split_reads(reads, lsb: int = 0, n_threads: int = 0) -> dict:
    """Split a list of int16 reads.  Returns concatenated arrays with
    per-read offsets/counts: ``sig0``, ``len``, ``small`` (uint8 tokens),
    ``small_off``, ``n_small``, ``large_adj`` (uint16, value - 256),
    ``large_gap`` (uint32 gap-coded positions), ``large_off``, ``n_large``."""
    return _host.split(reads, lsb, n_threads)


def reads_tokens(split: dict):
    """Per-read views of the small tokens of a ``split_reads`` result."""
    s, o, n = split["small"], split["small_off"], split["n_small"]
    return [s[o[i]:o[i] + n[i]] for i in range(len(n))]


def split_signal(sig: np.ndarray, lsb: int = 0):
    """``_split_signal`` (main.py:504-521) of one read, after the lossy
    transform when ``lsb > 0`` -> (sig0, small uint8 tokens, large - 256
    uint16, gap-coded uint32 positions)."""
    r = split_reads([np.asarray(sig, np.int16)], lsb, n_threads=1)
    return int(r["sig0"][0]), r["small"], r["large_adj"], r["large_gap"]


def reassemble_reads(split: dict, small=None, lsb: int = 0, n_threads: int = 0):
    """Inverse of ``split_reads`` (optionally with the small tokens replaced,
    e.g. by decoded ones, concatenated in read order) -> list of int16 reads."""
    sm = split["small"] if small is None else np.ascontiguousarray(small, np.uint8)
    out, out_off = _host.reassemble(split["sig0"], split["len"], sm, split["small_off"], split["n_small"],
                                    split["large_adj"], split["large_gap"], split["large_off"],
                                    split["n_large"], lsb, n_threads)
    lens = split["len"]
    return [out[out_off[i]:out_off[i] + lens[i]] for i in range(len(lens))]


def reassemble_signal(sig0: int, n: int, small_vals, large_adj, large_pos_deltas, lsb: int = 0) -> np.ndarray:
    """``_reassemble_signal`` (main.py:524-546) of one read with the
    Rice-decoded large values and gaps given, then ``_lossy_decode`` when
    ``lsb > 0``."""
    small_vals = np.ascontiguousarray(small_vals, np.uint8)
    large_adj = np.ascontiguousarray(large_adj, np.uint16)
    large_pos_deltas = np.ascontiguousarray(large_pos_deltas, np.uint32)
    if len(large_adj) != len(large_pos_deltas):
        raise ValueError("large values and positions differ in count")
    split = {"sig0": np.array([sig0], np.int16), "len": np.array([n], np.int64),
             "small": small_vals, "small_off": np.zeros(1, np.int64),
             "n_small": np.array([len(small_vals)], np.int64), "large_adj": large_adj,
             "large_gap": large_pos_deltas, "large_off": np.zeros(1, np.int64),
             "n_large": np.array([len(large_adj)], np.int64)}
    return reassemble_reads(split, lsb=lsb, n_threads=1)[0]
