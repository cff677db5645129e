"""Seeded synthetic inputs for the BASELINE workloads (no audio files ship here).

All randomness comes from the same SplitMix64 streams as the weights, so the
arrays do not depend on numpy's RNG version.
"""
from __future__ import annotations

import math

import numpy as np

from .weights import stream_normal, stream_u01

SAMPLE_RATE = 44100


def gaussian_segments(seed: int, batch: int, length: int, std: float = 0.1, channels: int = 2) -> np.ndarray:
    """(batch, channels, length) Gaussian white noise N(0, std^2)."""
    return stream_normal(f"mix.gaussian.{batch}x{channels}x{length}", seed, (batch, channels, length), std)


def synthetic_mix(seed: int, seconds: float, sr: int = SAMPLE_RATE) -> np.ndarray:
    """(2, samples) mix: 16 sinusoids (55-8000 Hz log-uniform, amplitude
    U(0.01, 0.1), random phase), pink noise at -30 dBFS RMS, and white-noise
    bursts with a 50 ms exponential decay (peak 0.1) every 0.5 s."""
    n = int(round(seconds * sr))
    t = np.arange(n, dtype=np.float64) / sr
    u = stream_u01("mix.sines", seed, 16 * 3 + 2 * 16)
    mix = np.zeros((2, n), dtype=np.float64)
    for i in range(16):
        freq = 55.0 * (8000.0 / 55.0) ** u[3 * i]
        amp = 0.01 + 0.09 * u[3 * i + 1]
        phase = 2 * math.pi * u[3 * i + 2]
        tone = amp * np.sin(2 * math.pi * freq * t + phase)
        for c in range(2):
            mix[c] += tone * (0.75 + 0.5 * u[48 + 2 * i + c])  # mild per-channel panning
    # Pink noise: white noise shaped by 1/sqrt(f) in the frequency domain.
    white = stream_normal("mix.pink", seed, (2, n)).astype(np.float64)
    spec = np.fft.rfft(white, axis=1)
    f = np.fft.rfftfreq(n, 1.0 / sr)
    shape = np.ones_like(f)
    shape[1:] = 1.0 / np.sqrt(f[1:] / f[1])
    shape[0] = 0.0
    pink = np.fft.irfft(spec * shape, n=n, axis=1)
    pink *= 10 ** (-30 / 20) / max(np.sqrt(np.mean(pink ** 2)), 1e-12)
    mix += pink
    # Decaying bursts every 0.5 s.
    period = int(0.5 * sr)
    env_len = min(period, n)
    env = 0.1 * np.exp(-np.arange(env_len) / (0.05 * sr))
    burst = stream_normal("mix.bursts", seed, (2, n)).astype(np.float64)
    burst /= max(np.max(np.abs(burst)), 1e-12)
    for start in range(0, n, period):
        end = min(n, start + env_len)
        mix[:, start:end] += burst[:, start:end] * env[: end - start]
    return mix.astype(np.float32)
