"""Euler Discrete scheduler (scheduler.js): the oracle restatement pinned by
closed forms and published values, and the host mirror
(``drawinstant.scheduler``) against it.  CPU only: the device kernels are
checked in test_gpu_scheduler.py."""
import math

import numpy as np
import pytest

from oracle import scheduler_ref as R


def test_trailing_timesteps_known_lists():
    # scheduler.js:4 ([999, 749, 499, 249] for 4 steps); diffusers "trailing":
    # round(arange(1000, 0, -1000 / n)) - 1
    assert R.trailing_timesteps(4).tolist() == [999, 749, 499, 249]
    assert R.trailing_timesteps(1).tolist() == [999]
    assert R.trailing_timesteps(2).tolist() == [999, 499]
    for n in (3, 5, 8):
        ref = [int(np.floor(x + 0.5)) - 1 for x in np.arange(1000, 0, -1000 / n)][:n]
        assert R.trailing_timesteps(n).tolist() == ref


def test_betas_alphas_sigmas_closed_forms():
    b = R.scaled_linear_betas(1000, R.BETA_START, R.BETA_END)
    assert abs(float(b[0]) - 0.00085) < 1e-9 and abs(float(b[-1]) - 0.012) < 1e-9
    # midpoint of the sqrt-linear ramp
    mid = ((math.sqrt(0.00085) + math.sqrt(0.012)) / 2) ** 2
    assert abs(float(R.scaled_linear_betas(3, 0.00085, 0.012)[1]) - mid) < 1e-9
    a = R.cumulative_alphas(b)
    assert float(a[0]) == np.float32(1 - float(b[0]))
    assert np.all(np.diff(a.astype(np.float64)) < 0)
    s = R.sigmas_from_alphas(a)
    assert abs(float(s[0]) - math.sqrt(float(b[0]) / (1 - float(b[0])))) < 1e-6
    # published init_noise_sigma of this schedule at t = 999 (SD 2.x Euler): 14.6146
    assert abs(float(s[999]) - 14.6146) < 1e-3


def test_interp_and_schedule():
    sig = np.array([0.0, 10.0, 20.0], np.float32)
    assert R.interp(sig, 0.25) == 2.5 and R.interp(sig, 1.5) == 15.0
    assert R.interp(sig, -1) == 0.0 and R.interp(sig, 7) == 20.0
    e = R.EulerRef(4)
    assert e.sigmas[-1] == 0 and np.all(np.diff(e.sigmas) < 0)
    assert e.init_noise_sigma == float(e.sigmas[0]) == float(e.sigmas_full[999])


def test_euler_update_closed_form():
    e = R.EulerRef(2)
    x = np.array([1.0, -2.0, 0.5], np.float32)
    p = np.array([0.25, 4.0, -1.0], np.float32)
    # step i: x + (sigma_{i+1} - sigma_i) * pred; the last step lands at sigma 0
    got = e.step(x, p, 1)
    want = np.float32(x.astype(np.float64) - float(e.sigmas[1]) * p.astype(np.float64))
    assert np.array_equal(got, want)
    s0 = float(e.sigmas[0])
    assert np.array_equal(e.scale_model_input(x, 0),
                          (x.astype(np.float64) / math.sqrt(s0 * s0 + 1)).astype(np.float32))


def test_lcg_against_jump_ahead():
    # the oracle's sequential generator against an independent closed form:
    # s_k = a^k s_0 + c (a^k - 1) / (a - 1) mod 2^32
    a, c, m = 1664525, 1013904223, 1 << 32
    for seed in (0, 1, 42, -7, 2**31 - 1):
        s0 = (seed & 0xFFFFFFFF) or 1
        st = R.lcg_states(seed, 40)
        for k in (1, 2, 17, 40):
            ak = pow(a, k, m * (a - 1))
            want = (pow(a, k, m) * s0 + c * ((ak - 1) // (a - 1))) % m
            assert int(st[k - 1]) == want
    assert int(R.lcg_states(0, 1)[0]) == 1015568748  # 1664525 + 1013904223


def test_noise_latent_statistics():
    z = R.sample_noise_latent(1, 16, 16, seed=3, init_sigma=2.0)
    assert z.shape == (1, 4, 16, 16) and z.dtype == np.float32
    assert abs(float(z.mean())) < 0.2 and abs(float(z.std()) - 2.0) < 0.2
    assert not np.array_equal(z, R.sample_noise_latent(1, 16, 16, seed=4, init_sigma=2.0))


@pytest.mark.parametrize("n", [1, 2, 3, 4, 6, 8])
def test_host_mirror_matches_oracle(n):
    # the mirror's schedule constants are host scalars (no device needed)
    from drawinstant import scheduler as S
    e, m = R.EulerRef(n), S.make_euler_scheduler(n)
    assert np.array_equal(m.timesteps, e.timesteps)
    assert np.array_equal(m.sigmas, e.sigmas)
    assert m.init_noise_sigma == e.init_noise_sigma
    for i in range(n):
        s = float(e.sigmas[i])
        assert m.inv_scale(i) == 1.0 / math.sqrt(s * s + 1.0)
        assert m.dt(i) == float(e.sigmas[i + 1]) - float(e.sigmas[i])
