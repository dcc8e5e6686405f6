"""Seeded synthetic nanopore-like reads for the benchmark configurations.

The reference ships no data generator; this one follows the configurations
it is benchmarked on:

* DNA (R10.4.1-like, configs 1-4): log-normal read lengths with median
  20,000 samples (sigma 0.25); piecewise-constant current with geometric
  dwell (mean 10 samples at 5 kHz), levels ~ N(90, 15) pA, Gaussian noise
  sd 2 pA.
* RNA (RNA004-like, config 5): median 40,000 samples at 4 kHz, dwell mean
  40, levels ~ N(85, 18) pA, noise sd 2.5 pA.

Current is mapped to int16 ADC units by ``adc = round(pA / scale - offset)``
with the fixed calibration below.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

ADC_SCALE = 0.1825      # pA per ADC unit
ADC_OFFSET = -240.0     # ADC offset


@dataclass(frozen=True)
class ReadProfile:
    median_len: float
    sigma_len: float
    dwell_mean: float
    level_mean: float
    level_sd: float
    noise_sd: float


DNA = ReadProfile(20000.0, 0.25, 10.0, 90.0, 15.0, 2.0)
RNA = ReadProfile(40000.0, 0.25, 40.0, 85.0, 18.0, 2.5)


def synth_read(rng: np.random.Generator, n: int, profile: ReadProfile) -> np.ndarray:
    """One read of ``n`` int16 ADC samples."""
    n = int(n)
    if n <= 0:
        return np.zeros(0, dtype=np.int16)
    p = 1.0 / profile.dwell_mean
    # enough dwells to cover n samples
    n_events = max(8, int(n * p * 1.5) + 16)
    dwells = rng.geometric(p, size=n_events)
    while dwells.sum() < n:
        dwells = np.concatenate([dwells, rng.geometric(p, size=n_events)])
    levels = rng.normal(profile.level_mean, profile.level_sd, size=len(dwells))
    current = np.repeat(levels, dwells)[:n]
    current = current + rng.normal(0.0, profile.noise_sd, size=n)
    adc = np.rint(current / ADC_SCALE - ADC_OFFSET)
    return np.clip(adc, -32768, 32767).astype(np.int16)


def synth_reads(n_reads: int, seed: int, profile: ReadProfile = DNA,
                lengths=None) -> list:
    """``n_reads`` seeded reads (PCG64); ``lengths`` overrides the length draw."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if lengths is None:
        lengths = np.maximum(2, np.rint(profile.median_len *
                                        np.exp(rng.normal(0.0, profile.sigma_len, n_reads))))
    return [synth_read(rng, int(n), profile) for n in lengths]


# Benchmark configurations (seeds are part of the definition).
CONFIGS = {
    "c1": dict(n_reads=64, seed=101, profile=DNA, lsb=0, model="lossless"),
    "c3": dict(n_reads=4000, seed=303, profile=DNA, lsb=0, model="lossless"),
    "c5": dict(n_reads=2000, seed=505, profile=RNA, lsb=3, model="lossy"),
}


def config_reads(name: str, n_reads=None):
    cfg = CONFIGS[name]
    return synth_reads(cfg["n_reads"] if n_reads is None else n_reads, cfg["seed"], cfg["profile"])
