"""Euler Discrete scheduler for SD-Turbo (reference scheduler.js) on
libdrawinstant_hip.

``make_euler_scheduler`` mirrors makeEulerScheduler (scheduler.js:77-112):
the schedule constants (scaled-linear betas, cumulative alphas, sigmas,
trailing timesteps) are host scalars computed exactly as the reference does
(double arithmetic, each Float32Array element rounded once to fp32).  The
per-element work - the noise latent (sampleNoiseLatent, :117-134),
scaleModelInput (:95-101) and the Euler update (:105-110) - runs on the
device through ``di_noise_latent`` / ``di_euler_scale`` / ``di_euler_step``,
so ``denoise`` keeps an N-step loop on the GPU: the reference reads the latent
back after every step (pipeline.js:274-288).
"""
from __future__ import annotations

import math

import numpy as np

from .device import Buffer, call

NUM_TRAIN_TIMESTEPS = 1000  # scheduler.js:21-23
BETA_START = 0.00085
BETA_END = 0.012


def _scaled_linear_betas(n: int) -> np.ndarray:
    s, e = math.sqrt(BETA_START), math.sqrt(BETA_END)
    t = np.arange(n, dtype=np.float64) / (n - 1)
    v = s + (e - s) * t
    return (v * v).astype(np.float32)


def _cumulative_alphas(betas: np.ndarray) -> np.ndarray:
    # the running product is a double, stored rounded after every factor
    return np.cumprod(1.0 - betas.astype(np.float64)).astype(np.float32)


def _sigmas(alphas: np.ndarray) -> np.ndarray:
    a = alphas.astype(np.float64)
    return np.sqrt((1.0 - a) / a).astype(np.float32)


def _interp(sig: np.ndarray, t: float) -> float:
    if t <= 0:
        return float(sig[0])
    if t >= len(sig) - 1:
        return float(sig[-1])
    i = int(math.floor(t))
    f = t - i
    return float(sig[i]) * (1 - f) + float(sig[i + 1]) * f


def _trailing(n: int) -> np.ndarray:
    step = NUM_TRAIN_TIMESTEPS / n
    # Math.round: halves go up
    return np.array([math.floor(NUM_TRAIN_TIMESTEPS - (i + 1) * step + step + 0.5) - 1
                     for i in range(n)], np.float32)


class EulerScheduler:
    """The object makeEulerScheduler returns: timesteps, sigmas (with the final
    0), num_inference, init_noise_sigma, and the two per-step operations on
    device buffers."""

    def __init__(self, num_inference: int = 4):
        if num_inference < 1:
            raise ValueError("num_inference must be >= 1")
        sig_full = _sigmas(_cumulative_alphas(_scaled_linear_betas(NUM_TRAIN_TIMESTEPS)))
        self.timesteps = _trailing(num_inference)
        self.sigmas = np.zeros(num_inference + 1, np.float32)
        for i in range(num_inference):
            self.sigmas[i] = _interp(sig_full, float(self.timesteps[i]))
        self.num_inference = num_inference
        self.init_noise_sigma = float(self.sigmas[0])

    def inv_scale(self, i: int) -> float:
        """1 / sqrt(sigma_i^2 + 1) in double (scheduler.js:97)."""
        s = float(self.sigmas[i])
        return 1.0 / math.sqrt(s * s + 1.0)

    def dt(self, i: int) -> float:
        """sigma_{i+1} - sigma_i in double (scheduler.js:106)."""
        return float(self.sigmas[i + 1]) - float(self.sigmas[i])

    def scale_model_input(self, device, latent: Buffer, out: Buffer, n: int, i: int) -> None:
        call("di_euler_scale", device.ctx, latent.handle, out.handle, n, self.inv_scale(i))

    def step(self, device, latent: Buffer, pred: Buffer, out: Buffer, n: int, i: int,
             next_in: Buffer | None = None) -> None:
        """out = latent + dt_i * pred; with next_in, also the scaled input of
        step i + 1 (requires i + 1 < num_inference)."""
        inv_next = 0.0
        if next_in is not None:
            if i + 1 >= self.num_inference:
                raise ValueError("next_in given for the last step")
            inv_next = self.inv_scale(i + 1)
        call("di_euler_step", device.ctx, latent.handle, pred.handle, out.handle,
             next_in.handle if next_in is not None else 0, n, self.dt(i), inv_next)


def make_euler_scheduler(num_inference: int = 4) -> EulerScheduler:
    """makeEulerScheduler (scheduler.js:77-112)."""
    return EulerScheduler(num_inference)


def sample_noise_latent(device, out: Buffer, B: int = 1, H: int = 64, W: int = 64, seed: int = 0,
                        init_sigma: float = 1.0) -> None:
    """sampleNoiseLatent (scheduler.js:117-134) into the fp32 [B,4,H,W] buffer
    ``out``, on the device."""
    s = int(np.int64(seed) & 0xFFFFFFFF)
    call("di_noise_latent", device.ctx, out.handle, B * 4 * H * W,
         int(np.uint32(s).astype(np.int32)), float(init_sigma))


class Denoiser:
    """The reference's denoise loop (pipeline.js:274-288) with nothing leaving
    the GPU: noise latent, then per step scaleModelInput -> U-Net -> Euler
    update, the update fused with the next step's input scaling.  The work
    buffers live as long as the object, so repeated runs replay the U-Net's
    captured graph instead of capturing a new one."""

    def __init__(self, unet, B: int = 1, H: int = 64, W: int = 64, Sctx: int = 77,
                 steps: int = 4):
        self.unet, self.B, self.H, self.W, self.Sctx = unet, B, H, W, Sctx
        self.sched = make_euler_scheduler(steps)
        dev = unet.device
        self.n = B * 4 * H * W
        self.model_in = dev.create_buffer(self.n * 4)
        self.pred = dev.create_buffer(self.n * 4)
        self.tbuf = dev.create_buffer(B * 4)
        # every step's timestep, resident; the U-Net reads the current one from tbuf
        self.tall = dev.storage(np.repeat(self.sched.timesteps, B).astype(np.float32))

    def run(self, context: Buffer, latent: Buffer, seed: int = 0, graph: bool = True) -> None:
        """Enqueue the loop: ``latent`` (fp32 [B,4,H,W]) receives the final
        latent; ``context`` is fp32 [B,Sctx,cross_dim]."""
        dev, sc, n, B = self.unet.device, self.sched, self.n, self.B
        sample_noise_latent(dev, latent, B, self.H, self.W, seed, sc.init_noise_sigma)
        sc.scale_model_input(dev, latent, self.model_in, n, 0)
        for i in range(sc.num_inference):
            dev.copy(self.tbuf, self.tall, B * 4, 0, i * B * 4)
            self.unet.forward(self.model_in, self.tbuf, context, self.pred, B, self.H, self.W,
                              self.Sctx, graph)
            last = i + 1 == sc.num_inference
            sc.step(dev, latent, self.pred, latent, n, i, None if last else self.model_in)

    def destroy(self) -> None:
        self.unet.device.sync()
        for b in (self.model_in, self.pred, self.tbuf, self.tall):
            b.destroy()


def denoise(unet, context: Buffer, latent: Buffer, B: int = 1, H: int = 64, W: int = 64,
            Sctx: int = 77, steps: int = 4, seed: int = 0, graph: bool = True) -> EulerScheduler:
    """One run of a temporary Denoiser; returns its schedule once the device
    is done."""
    d = Denoiser(unet, B, H, W, Sctx, steps)
    try:
        d.run(context, latent, seed, graph)
    finally:
        d.destroy()
    return d.sched
