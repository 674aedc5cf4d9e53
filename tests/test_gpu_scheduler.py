"""GPU tests of the Euler scheduler kernels (di_noise_latent, di_euler_scale,
di_euler_step) and the on-device denoise loop, against the oracle
restatement of scheduler.js (oracle/scheduler_ref.py).

* scale / step: every element is a double expression rounded once to fp32 on
  both sides, so they must agree bit for bit;
* noise: the LCG states are integer-exact; log / cos / sin are the device's
  and the host's libm in double, so an element may differ by one fp32 ulp when
  a double result sits on a rounding boundary (required: >= 99.9 % identical,
  none off by more than 1 ulp);
* denoise: two steps of the narrow U-Net against the oracle composition
  (EulerRef + unet_ref), rel-L2 <= 1e-2; graph replay equals eager.
"""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import scheduler_ref as R
from oracle import unet_ref

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    ai = a.view(np.int32).astype(np.int64)
    bi = b.view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


@pytest.mark.parametrize("B,H,W,seed,sigma", [(1, 64, 64, 0, 14.614641), (2, 16, 24, -7, 1.0),
                                              (1, 8, 8, 2**31 - 1, 3.5)])
def test_noise_latent_matches_oracle(dev, B, H, W, seed, sigma):
    from drawinstant import scheduler as S
    out = dev.create_buffer(B * 4 * H * W * 4)
    S.sample_noise_latent(dev, out, B, H, W, seed, sigma)
    got = dev.download(out, np.float32, (B, 4, H, W))
    ref = R.sample_noise_latent(B, H, W, seed, sigma)
    d = _ulps(got.ravel(), ref.ravel())
    print(f"[noise] B={B} {H}x{W} seed={seed}: identical {np.mean(d == 0):.5f}, max ulp {d.max()}",
          flush=True)
    assert d.max() <= 1 and np.mean(d == 0) >= 0.999
    out.destroy()


def test_noise_latent_odd_count(dev):
    from drawinstant.device import call
    out = dev.create_buffer(8 * 4)
    dev.upload(out, np.full(8, 123.0, np.float32))
    call("di_noise_latent", dev.ctx, out.handle, 7, 5, 1.0)
    got = dev.download(out, np.float32)
    ref = R.sample_noise_latent(1, 2, 1, 5, 1.0).ravel()  # 8 values; the first 7 are written
    assert np.all(_ulps(got[:7], ref[:7]) <= 1) and got[7] == 123.0


@pytest.mark.parametrize("steps", [1, 2, 4])
def test_scale_and_step_bit_exact(dev, rng, steps):
    from drawinstant import scheduler as S
    e, m = R.EulerRef(steps), S.make_euler_scheduler(steps)
    n = 4 * 17 * 9
    x = (rng.standard_normal(n) * 5).astype(np.float32)
    p = rng.standard_normal(n).astype(np.float32)
    bx, bp = dev.storage(x), dev.storage(p)
    by, bn = dev.create_buffer(n * 4), dev.create_buffer(n * 4)
    for i in range(steps):
        m.scale_model_input(dev, bx, by, n, i)
        assert np.array_equal(dev.download(by, np.float32), e.scale_model_input(x, i))
        nxt = bn if i + 1 < steps else None
        m.step(dev, bx, bp, by, n, i, nxt)
        want = e.step(x, p, i)
        assert np.array_equal(dev.download(by, np.float32), want)
        if nxt is not None:
            assert np.array_equal(dev.download(bn, np.float32), e.scale_model_input(want, i + 1))
    # in place: out aliases latent
    m.step(dev, bx, bp, bx, n, 0)
    assert np.array_equal(dev.download(bx, np.float32), e.step(x, p, 0))
    for b in (bx, bp, by, bn):
        b.destroy()


def test_step_rejects_aliasing(dev):
    from drawinstant.device import DiError, call
    a, b = dev.create_buffer(64), dev.create_buffer(64)
    with pytest.raises(DiError):
        call("di_euler_step", dev.ctx, a.handle, b.handle, b.handle, 0, 16, 0.5, 0.0)
    with pytest.raises(DiError):
        call("di_euler_step", dev.ctx, a.handle, b.handle, a.handle, a.handle, 16, 0.5, 0.5)
    a.destroy()
    b.destroy()


def test_denoise_two_steps_vs_oracle(dev, rng):
    """pipeline.js:274-288 with the narrow U-Net: noise -> (scale -> U-Net ->
    Euler) x 2, all on the device, against the same loop on the oracle."""
    from drawinstant import scheduler as S
    from drawinstant.unet import UNet, UNetConfig
    cfg = UNetConfig.small()
    u = UNet(dev, cfg, seed=13)
    try:
        B, H, W, T = 1, 16, 16, 77
        ctx = rng.standard_normal((B, T, cfg.cross_dim)).astype(np.float32)
        bc = dev.storage(ctx)
        lat = dev.create_buffer(B * 4 * H * W * 4)
        S.denoise(u, bc, lat, B, H, W, T, steps=2, seed=11, graph=False)
        got = dev.download(lat, np.float32, (B, 4, H, W))
        S.denoise(u, bc, lat, B, H, W, T, steps=2, seed=11, graph=True)
        np.testing.assert_array_equal(dev.download(lat, np.float32, (B, 4, H, W)), got)
        e = R.EulerRef(2)
        sd = u.state_dict()
        x = R.sample_noise_latent(B, H, W, 11, e.init_noise_sigma)
        for i in range(2):
            mi = e.scale_model_input(x, i)
            pred = unet_ref.unet_forward(unet_ref.OracleOps(), sd, cfg.as_dict(), mi,
                                         np.full(B, e.timesteps[i], np.float32), ctx)
            x = e.step(x, np.asarray(pred, np.float32), i)
        err = rel_l2(got, x)
        print(f"[denoise 2 steps] rel-L2 {err:.2e}", flush=True)
        assert np.isfinite(got).all() and err <= 1e-2
        for b in (bc, lat):
            b.destroy()
    finally:
        u.destroy()
