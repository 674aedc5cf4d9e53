"""CPU restatement of the reference's Euler Discrete scheduler (scheduler.js).

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: imported by tests/ as
the checker of ``drawinstant.scheduler`` and of the device kernels behind
``di_noise_latent`` / ``di_euler_scale`` / ``di_euler_step``.

The reference keeps every array in a Float32Array and does the arithmetic in
JavaScript doubles, so each stored value is a double expression rounded once
to fp32.  The restatement follows that literally: Python floats are IEEE
doubles, ``np.float32(x)`` is the Float32Array store.
"""
from __future__ import annotations

import math

import numpy as np

# scheduler.js:21-23
NUM_TRAIN_TIMESTEPS = 1000
BETA_START = 0.00085
BETA_END = 0.012


def scaled_linear_betas(n: int, start: float, end: float) -> np.ndarray:
    """scheduler.js:25-35: ((sqrt(start) + (sqrt(end) - sqrt(start)) * i / (n - 1))^2."""
    out = np.zeros(n, np.float32)
    s, e = math.sqrt(start), math.sqrt(end)
    for i in range(n):
        t = i / (n - 1)
        v = s + (e - s) * t
        out[i] = v * v
    return out


def cumulative_alphas(betas: np.ndarray) -> np.ndarray:
    """scheduler.js:37-45: running product of (1 - beta) in double, stored fp32."""
    out = np.zeros(len(betas), np.float32)
    acc = 1.0
    for i, b in enumerate(betas):
        acc *= 1.0 - float(b)
        out[i] = acc
    return out


def sigmas_from_alphas(alphas: np.ndarray) -> np.ndarray:
    """scheduler.js:48-54: sigma = sqrt((1 - a) / a)."""
    out = np.zeros(len(alphas), np.float32)
    for i, a in enumerate(alphas):
        a = float(a)
        out[i] = math.sqrt((1.0 - a) / a)
    return out


def interp(sigmas: np.ndarray, t: float) -> float:
    """scheduler.js:57-63: linear interpolation at a fractional timestep."""
    if t <= 0:
        return float(sigmas[0])
    if t >= len(sigmas) - 1:
        return float(sigmas[-1])
    i = math.floor(t)
    f = t - i
    return float(sigmas[i]) * (1 - f) + float(sigmas[i + 1]) * f


def _js_round(x: float) -> float:
    """Math.round: nearest integer, halves toward +infinity."""
    return float(math.floor(x + 0.5))


def trailing_timesteps(n: int) -> np.ndarray:
    """scheduler.js:67-75: round(T - (i + 1) * step + step) - 1, step = T / n."""
    step = NUM_TRAIN_TIMESTEPS / n
    out = np.zeros(n, np.float32)
    for i in range(n):
        out[i] = _js_round(NUM_TRAIN_TIMESTEPS - (i + 1) * step + step) - 1
    return out


class EulerRef:
    """makeEulerScheduler (scheduler.js:77-112)."""

    def __init__(self, num_inference: int = 4):
        betas = scaled_linear_betas(NUM_TRAIN_TIMESTEPS, BETA_START, BETA_END)
        self.betas = betas
        self.alphas = cumulative_alphas(betas)
        self.sigmas_full = sigmas_from_alphas(self.alphas)
        self.timesteps = trailing_timesteps(num_inference)
        self.sigmas = np.zeros(num_inference + 1, np.float32)
        for i in range(num_inference):
            self.sigmas[i] = interp(self.sigmas_full, float(self.timesteps[i]))
        self.sigmas[num_inference] = 0
        self.num_inference = num_inference
        self.init_noise_sigma = float(self.sigmas[0])

    def scale_model_input(self, latent: np.ndarray, i: int) -> np.ndarray:
        """scheduler.js:95-101: latent * (1 / sqrt(sigma_i^2 + 1))."""
        s = float(self.sigmas[i])
        inv = 1.0 / math.sqrt(s * s + 1.0)
        return (latent.astype(np.float64) * inv).astype(np.float32)

    def step(self, latent: np.ndarray, pred: np.ndarray, i: int) -> np.ndarray:
        """scheduler.js:105-110: latent + (sigma_{i+1} - sigma_i) * pred."""
        dt = float(self.sigmas[i + 1]) - float(self.sigmas[i])
        return (latent.astype(np.float64) + dt * pred.astype(np.float64)).astype(np.float32)


def lcg_states(seed: int, count: int) -> np.ndarray:
    """The generator of sampleNoiseLatent (scheduler.js:122-126): s = (s * 1664525
    + 1013904223) | 0 starting from (seed | 0) || 1; returns the unsigned states
    s_1 .. s_count (each rand() is s >>> 0 over 2^32)."""
    s = int(np.int32(np.int64(seed) & 0xFFFFFFFF)) or 1
    out = np.zeros(count, np.uint64)
    for k in range(count):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[k] = s
    return out


def sample_noise_latent(B: int = 1, H: int = 64, W: int = 64, seed: int = 0,
                        init_sigma: float = 1.0) -> np.ndarray:
    """sampleNoiseLatent (scheduler.js:117-134): Box-Muller pairs from the LCG,
    element i = r * cos(2 pi u2) * sigma, element i + 1 = r * sin(2 pi u2) * sigma,
    r = sqrt(-2 log max(u1, 1e-9)); [B, 4, H, W] fp32."""
    n = B * 4 * H * W
    st = lcg_states(seed, 2 * ((n + 1) // 2))
    out = np.zeros(n, np.float32)
    for p in range((n + 1) // 2):
        u1 = max(float(st[2 * p]) / 4294967296.0, 1e-9)
        u2 = float(st[2 * p + 1]) / 4294967296.0
        r = math.sqrt(-2 * math.log(u1))
        out[2 * p] = r * math.cos(2 * math.pi * u2) * init_sigma
        if 2 * p + 1 < n:
            out[2 * p + 1] = r * math.sin(2 * math.pi * u2) * init_sigma
    return out.reshape(B, 4, H, W)
