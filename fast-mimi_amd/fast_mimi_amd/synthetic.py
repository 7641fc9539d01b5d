"""Seeded synthetic 24 kHz test audio (numpy only, platform independent).

Each clip is a sum of three sinusoids (frequencies log-uniform in
[80, 4000] Hz, phases uniform in [0, 2*pi)) plus pink noise at -20 dB RMS
relative to the sinusoid sum, peak-normalised to ``peak``.  Pink noise is
PCG64 white noise shaped by 1/sqrt(f) in the rfft domain with the DC bin
zeroed.  Clip ``i`` of a batch uses seed ``base_seed + i``.
"""

from __future__ import annotations

import numpy as np

SAMPLE_RATE = 24_000


def clip(num_samples: int, seed: int, peak: float = 0.5,
         sample_rate: int = SAMPLE_RATE) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    freqs = np.exp(rng.uniform(np.log(80.0), np.log(4000.0), size=3))
    phases = rng.uniform(0.0, 2.0 * np.pi, size=3)
    t = np.arange(num_samples, dtype=np.float64) / sample_rate
    tone = np.zeros(num_samples, dtype=np.float64)
    for f, p in zip(freqs, phases):
        tone += np.sin(2.0 * np.pi * f * t + p)
    white = rng.standard_normal(num_samples)
    spectrum = np.fft.rfft(white)
    bins = np.arange(spectrum.shape[0], dtype=np.float64)
    shape = np.zeros_like(bins)
    shape[1:] = 1.0 / np.sqrt(bins[1:])
    pink = np.fft.irfft(spectrum * shape, n=num_samples)
    tone_rms = np.sqrt(np.mean(tone ** 2)) if num_samples else 0.0
    pink_rms = np.sqrt(np.mean(pink ** 2)) if num_samples else 0.0
    if pink_rms > 0:
        pink *= (tone_rms * 10.0 ** (-20.0 / 20.0)) / pink_rms
    wave = tone + pink
    top = np.max(np.abs(wave)) if num_samples else 0.0
    if top > 0:
        wave *= peak / top
    return wave.astype(np.float32)


def batch(batch_size: int, num_samples: int, base_seed: int = 0,
          peak: float | None = 0.5, padded_tail: int = 0,
          padded_length: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Audio ``[B, 1, S]`` float32 and padding mask ``[B, 1, S]`` bool.

    ``peak=None`` draws each clip's peak from U[0.1, 0.9] (seeded by the clip).
    The last ``padded_tail`` clips are generated at ``padded_length`` samples
    and zero-padded to ``num_samples`` with the mask False on the padding.
    """
    audio = np.zeros((batch_size, 1, num_samples), dtype=np.float32)
    mask = np.ones((batch_size, 1, num_samples), dtype=bool)
    for i in range(batch_size):
        seed = base_seed + i
        amp = peak
        if amp is None:
            amp = float(np.random.Generator(np.random.PCG64(10_000 + seed)).uniform(0.1, 0.9))
        length = num_samples
        if padded_tail and i >= batch_size - padded_tail:
            length = int(padded_length)
            mask[i, 0, length:] = False
        audio[i, 0, :length] = clip(length, seed, amp)
    return audio, mask


def config_inputs(name: str) -> tuple[np.ndarray, np.ndarray, int]:
    """Inputs of the benchmark configurations: ``(audio, mask, num_quantizers)``.

    c1: B1 x 5 s; c2: B1 x 10 s; c3: B16 x 10 s, last 4 padded from 6 s with
    per-clip peak U[0.1, 0.9]; c4: B1 x 100 s; c5: B64 x 10 s, 32 codebooks.
    """
    if name == "c1":
        a, m = batch(1, 120_000)
        return a, m, 8
    if name == "c2":
        a, m = batch(1, 240_000)
        return a, m, 8
    if name == "c3":
        a, m = batch(16, 240_000, peak=None, padded_tail=4, padded_length=144_000)
        return a, m, 8
    if name == "c4":
        a, m = batch(1, 2_400_000)
        return a, m, 8
    if name == "c5":
        a, m = batch(64, 240_000)
        return a, m, 32
    raise ValueError(f"unknown configuration {name!r}")
