"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the parity
checker of the HIP kernels.

Inputs are the closed-form known-answer generators of the reference's kernel
tests (wgsl-ops-test.js:38-435); expected values come from what the
mathematics fixes independently of the oracle's code: library routines
(torch CPU in float64, numpy, math.erf), published error bounds, invariants
and brute-force special cases.  A dropped term, wrong sign, swapped index or
transposed operand in the oracle fails at least one of these.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

T64 = lambda a: torch.from_numpy(np.asarray(a, np.float64))


# ---------------- element-wise (wgsl-ops-test.js:38-98) ----------------

def _kat_unary_x():
    n = 1024
    return np.array([(i - n / 2) / (n / 4) for i in range(n)], np.float32)  # :40


@pytest.mark.parametrize("op,ref", [
    ("Sigmoid", lambda x: torch.sigmoid(x)),
    ("Sqrt", lambda x: torch.sqrt(torch.clamp(x, min=0))),
    ("SiLU", lambda x: F.silu(x)),
    ("Abs", lambda x: torch.abs(x)),
    ("Neg", lambda x: -x),
    ("Exp", lambda x: torch.exp(x)),
    ("Sin", lambda x: torch.sin(x)),
    ("Cos", lambda x: torch.cos(x)),
    ("GELU_TANH", lambda x: F.gelu(x, approximate="tanh")),
])
def test_unary_exact_ops(op, ref):
    x = _kat_unary_x()
    got = oracle.unary(op, x)
    exp = ref(T64(x)).numpy()
    np.testing.assert_allclose(got, exp, rtol=2e-7, atol=2e-7)


def test_erf_within_abramowitz_stegun_bound():
    # A&S 7.1.26 guarantees |err| <= 1.5e-7; fp32 output rounding adds ~6e-8.
    x = np.linspace(-4, 4, 4001).astype(np.float32)
    got = oracle.unary("Erf", x)
    exp = np.array([math.erf(float(v)) for v in x])
    assert np.max(np.abs(got - exp)) < 1.5e-7 + 1.2e-7
    assert abs(got[2000]) < 1.5e-7                      # A&S gives 1e-9 at 0, not 0
    np.testing.assert_array_equal(got[:2000], -got[2001:][::-1])  # odd function


def test_gelu_matches_exact_erf_gelu():
    x = _kat_unary_x()
    got = oracle.unary("GELU", x)
    exp = F.gelu(T64(x), approximate="none").numpy()
    # erf error 1.5e-7 scaled by |x|/2 <= 1 on [-2, 2]
    assert np.max(np.abs(got - exp)) < 3e-7


def test_log_clamps_at_1e_minus_12():
    x = np.array([0.0, -1.0, 1.0, math.e], np.float32)
    got = oracle.unary("Log", x)
    np.testing.assert_allclose(got, [math.log(1e-12), math.log(1e-12), 0.0, 1.0], rtol=1e-6)


def _kat_binary():
    n = 512
    a = np.array([(i + 1) * 0.1 for i in range(n)], np.float32)            # :80
    b = np.array([math.sin(i * 0.1) + 1.5 for i in range(n)], np.float32)  # :80
    return a, b


@pytest.mark.parametrize("op,ref", [
    ("Add", np.add), ("Sub", np.subtract), ("Mul", np.multiply), ("Div", np.divide),
    ("Max", np.maximum), ("Min", np.minimum),
])
def test_binary_ops(op, ref):
    a, b = _kat_binary()
    got = oracle.binary(op, a, b)
    exp = ref(a.astype(np.float64), b.astype(np.float64))
    np.testing.assert_allclose(got, exp, rtol=1e-7)


def test_pow_is_sign_aware_for_integer_exponents():
    a = np.array([-2.0, -2.0, -2.0, 3.0, 0.5, -4.0], np.float32)
    b = np.array([2.0, 3.0, 0.5, 2.0, 3.0, 1.0], np.float32)
    got = oracle.binary("Pow", a, b)
    # odd integer exponent keeps the sign; non-integer uses |a|
    np.testing.assert_allclose(got, [4.0, -8.0, math.sqrt(2.0), 9.0, 0.125, -4.0], rtol=1e-6)


@pytest.mark.parametrize("e", [2, 3, 0.5])
def test_pow_scalar_kat(e):
    n = 256
    x = np.array([(i - n / 2) / (n / 8) for i in range(n)], np.float32)  # :418
    got = oracle.pow_scalar(x, e)
    xd = x.astype(np.float64)
    if float(e).is_integer():
        exp = np.power(xd, e)
    else:
        exp = np.where(xd < 0, 0.0, np.power(np.abs(xd), e))
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-6)


def test_binary_bcast_matches_numpy_broadcasting(rng):
    a = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    b = rng.standard_normal((1, 3, 1, 5)).astype(np.float32)
    # row-major strides, 0 on broadcast dims (wgsl-executor.js:647-657)
    got = oracle.binary_bcast("Mul", a, b, (2, 3, 4, 5), (60, 20, 5, 1), (0, 5, 0, 1))
    np.testing.assert_allclose(got, a.astype(np.float64) * b, rtol=1e-7)


# ---------------- softmax / reductions ----------------

def test_softmax_kat():
    x = np.array([math.sin(i * 0.1) * 2 for i in range(4 * 64)], np.float32).reshape(4, 64)  # :105
    got = oracle.softmax(x)
    exp = torch.softmax(T64(x), -1).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-6)


def test_softmax_shift_invariance(rng):
    x = rng.standard_normal((8, 77)).astype(np.float32)
    np.testing.assert_allclose(oracle.softmax(x), oracle.softmax(x + 100.0), atol=1e-6)


def test_reduce_mean(rng):
    x = rng.standard_normal((6, 320)).astype(np.float32)
    np.testing.assert_allclose(oracle.reduce_mean(x)[:, 0], x.astype(np.float64).mean(-1),
                               rtol=1e-6, atol=1e-8)


# ---------------- normalisation ----------------

def test_instance_norm_kat():
    n, c, h, w = 2, 4, 8, 8                                                   # :132
    x = np.array([math.sin(i * 0.07) * 3 + 1 for i in range(n * c * h * w)],
                 np.float32).reshape(n, c, h, w)
    g = np.full(c, 1.2, np.float32)
    b = np.full(c, -0.3, np.float32)
    got = oracle.instance_norm(x, g, b, eps=1e-5)
    exp = F.instance_norm(T64(x), weight=T64(g), bias=T64(b), eps=1e-5).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("shape,G,eps,silu", [
    ((1, 320, 16, 16), 32, 1e-5, True),
    ((2, 64, 8, 8), 32, 1e-6, False),
    ((1, 96, 5, 7), 4, 1e-5, True),
])
def test_group_norm_vs_torch(shape, G, eps, silu, rng):
    x = rng.standard_normal(shape).astype(np.float32) * 2 + 0.5
    g = (1 + 0.02 * rng.standard_normal(shape[1])).astype(np.float32)
    b = (0.02 * rng.standard_normal(shape[1])).astype(np.float32)
    got = oracle.group_norm(x, g, b, G, eps=eps, silu=silu)
    exp = F.group_norm(T64(x), G, T64(g), T64(b), eps=eps)
    if silu:
        exp = F.silu(exp)
    np.testing.assert_allclose(got, exp.numpy(), rtol=2e-6, atol=2e-6)


def test_group_norm_invariant_unit_affine(rng):
    # gamma=1, beta=0: each (n,g) block has mean 0, variance var/(var+eps).
    x = (3.0 * rng.standard_normal((1, 64, 16, 16))).astype(np.float32)
    y = oracle.group_norm(x, np.ones(64, np.float32), np.zeros(64, np.float32), 8, eps=1e-2)
    blocks = y.reshape(8, -1).astype(np.float64)
    xv = x.reshape(8, -1).astype(np.float64).var(-1)
    np.testing.assert_allclose(blocks.mean(-1), 0.0, atol=1e-6)
    np.testing.assert_allclose(blocks.var(-1), xv / (xv + 1e-2), rtol=1e-5)


def test_layer_norm_kat():
    rows, inner = 8, 128                                                      # :308
    x = np.array([math.sin(i * 0.05) * 2 + 1 for i in range(rows * inner)],
                 np.float32).reshape(rows, inner)
    g = np.array([0.9 + i * 0.01 for i in range(inner)], np.float32)
    b = np.array([-0.1 + i * 0.005 for i in range(inner)], np.float32)
    got = oracle.layer_norm(x, g, b, eps=1e-5)
    exp = F.layer_norm(T64(x), (inner,), T64(g), T64(b), eps=1e-5).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-6)


# ---------------- contractions ----------------

def test_matmul_kat():
    M, N, K = 32, 48, 24                                                      # :165
    a = np.array([math.sin(i * 0.3) for i in range(M * K)], np.float32).reshape(M, K)
    b = np.array([math.cos(i * 0.17) for i in range(K * N)], np.float32).reshape(K, N)
    np.testing.assert_allclose(oracle.matmul(a, b), a.astype(np.float64) @ b, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("batched_b", [False, True])
def test_matmul_batched_kat(batched_b):
    Bt, M, N, K = 2, 20, 24, 12                                               # :189, :213
    a = np.array([math.sin(i * 0.21) for i in range(Bt * M * K)], np.float32).reshape(Bt, M, K)
    nb = Bt * K * N if batched_b else K * N
    b = np.array([math.cos(i * 0.13) for i in range(nb)], np.float32)
    b = b.reshape((Bt, K, N) if batched_b else (K, N))
    exp = a.astype(np.float64) @ b.astype(np.float64)
    np.testing.assert_allclose(oracle.matmul(a, b), exp, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("trans_b", [False, True])
def test_gemm_kat(trans_b):
    M, N, K = 16, 24, 12                                                      # :341, :367
    a = np.array([math.sin(i * 0.1) for i in range(M * K)], np.float32).reshape(M, K)
    b = np.array([math.cos(i * 0.15) for i in range(K * N)], np.float32)
    b = b.reshape((N, K) if trans_b else (K, N))
    c = np.array([0.01 * i for i in range(N)], np.float32)
    bm = b.astype(np.float64).T if trans_b else b.astype(np.float64)
    np.testing.assert_allclose(oracle.gemm(a, b, c, trans_b), a.astype(np.float64) @ bm + c,
                               rtol=1e-6, atol=1e-6)


def test_linear_matches_torch(rng):
    x = rng.standard_normal((7, 40)).astype(np.float32)
    w = rng.standard_normal((24, 40)).astype(np.float32)
    b = rng.standard_normal(24).astype(np.float32)
    np.testing.assert_allclose(oracle.linear(x, w, b), F.linear(T64(x), T64(w), T64(b)).numpy(),
                               rtol=1e-6, atol=1e-6)


def test_conv3x3_kat():
    cin, cout, h, w = 3, 4, 8, 8                                              # :239
    x = np.array([math.sin(i * 0.2) for i in range(cin * h * w)], np.float32).reshape(1, cin, h, w)
    wt = np.array([math.cos(i * 0.13) * 0.5 for i in range(cout * cin * 9)],
                  np.float32).reshape(cout, cin, 3, 3)
    bias = np.array([0.1 * i for i in range(cout)], np.float32)
    exp = F.conv2d(T64(x), T64(wt), T64(bias), padding=1).numpy()
    np.testing.assert_allclose(oracle.conv2d(x, wt, bias), exp, rtol=1e-6, atol=1e-6)


def test_conv1x1_kat():
    cin, cout, h, w = 8, 6, 4, 4                                              # :275
    x = np.array([math.sin(i * 0.1) for i in range(cin * h * w)], np.float32).reshape(1, cin, h, w)
    wt = np.array([math.cos(i * 0.2) * 0.3 for i in range(cout * cin)],
                  np.float32).reshape(cout, cin, 1, 1)
    bias = np.array([0.05 * i for i in range(cout)], np.float32)
    exp = F.conv2d(T64(x), T64(wt), T64(bias)).numpy()
    np.testing.assert_allclose(oracle.conv2d(x, wt, bias), exp, rtol=1e-6, atol=1e-6)


def test_conv_stride2_batched_matches_torch(rng):
    x = rng.standard_normal((2, 5, 9, 10)).astype(np.float32)
    wt = rng.standard_normal((7, 5, 3, 3)).astype(np.float32)
    bias = rng.standard_normal(7).astype(np.float32)
    exp = F.conv2d(T64(x), T64(wt), T64(bias), stride=2, padding=1).numpy()
    np.testing.assert_allclose(oracle.conv2d(x, wt, bias, stride=2), exp, rtol=1e-6, atol=1e-6)


def test_conv_delta_kernel_is_a_shift(rng):
    # A kernel with a single 1 at (ky, kx) = (0, 2) reads x[y-1, x+1].
    x = rng.standard_normal((1, 1, 6, 6)).astype(np.float32)
    wt = np.zeros((1, 1, 3, 3), np.float32)
    wt[0, 0, 0, 2] = 1.0
    y = oracle.conv2d(x, wt)
    exp = np.zeros_like(x)
    exp[0, 0, 1:, :-1] = x[0, 0, :-1, 1:]
    np.testing.assert_array_equal(y, exp)


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
def test_attention_vs_torch_sdpa(layout, rng):
    B, H, Sq, Skv, d = 2, 3, 17, 11, 8
    shp = (lambda s: (B, H, s, d)) if layout == "bhsd" else (lambda s: (B, s, H, d))
    q = rng.standard_normal(shp(Sq)).astype(np.float32)
    k = rng.standard_normal(shp(Skv)).astype(np.float32)
    v = rng.standard_normal(shp(Skv)).astype(np.float32)
    got = oracle.attention(q, k, v, layout=layout)
    tq, tk, tv = T64(q), T64(k), T64(v)
    if layout == "bshd":
        tq, tk, tv = (t.transpose(1, 2) for t in (tq, tk, tv))
    exp = F.scaled_dot_product_attention(tq, tk, tv)
    if layout == "bshd":
        exp = exp.transpose(1, 2)
    np.testing.assert_allclose(got, exp.numpy(), rtol=1e-6, atol=1e-6)


def test_attention_single_key_returns_value(rng):
    q = rng.standard_normal((1, 2, 5, 4)).astype(np.float32)
    k = rng.standard_normal((1, 2, 1, 4)).astype(np.float32)
    v = rng.standard_normal((1, 2, 1, 4)).astype(np.float32)
    got = oracle.attention(q, k, v)
    np.testing.assert_allclose(got, np.broadcast_to(v, got.shape), rtol=1e-7)


def test_resize_nearest_kat():
    c, h, w = 3, 4, 4                                                         # :394
    x = np.array([math.sin(i * 0.3) for i in range(c * h * w)], np.float32).reshape(c, h, w)
    got = oracle.resize_nearest(x, 8, 8)
    np.testing.assert_array_equal(got, x.repeat(2, axis=1).repeat(2, axis=2))


# ---------------- timestep embedding ----------------

def test_tembed_matches_diffusers_definition(rng):
    # diffusers Timesteps(320, flip_sin_to_cos=True, downscale_freq_shift=0)
    # -> TimestepEmbedding(320, 1280): linear_1, SiLU, linear_2.
    emb_dim, hid = 320, 64
    w1 = (0.05 * rng.standard_normal((hid, emb_dim))).astype(np.float32)
    b1 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    w2 = (0.05 * rng.standard_normal((hid, hid))).astype(np.float32)
    b2 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    for t in (0.0, 500.0, 999.0):
        half = emb_dim // 2
        exponent = -math.log(10000) * torch.arange(half, dtype=torch.float64) / half
        e = t * torch.exp(exponent)
        emb = torch.cat([torch.sin(e), torch.cos(e)])
        emb = torch.cat([emb[half:], emb[:half]])  # flip_sin_to_cos
        h = F.silu(F.linear(emb, T64(w1), T64(b1)))
        exp = F.linear(h, T64(w2), T64(b2)).numpy()
        np.testing.assert_allclose(oracle.tembed(t, w1, b1, w2, b2), exp, rtol=1e-5, atol=1e-6)


# ---------------- seeded generator ----------------

def test_splitmix64_reference_stream():
    # Published SplitMix64 outputs for seed 1234567 (Vigna's splitmix64.c).
    exp = [6457827717110365317, 3203168211198807973, 9817491932198370423,
           4593380528125082431, 16408922859458223821]
    assert [oracle.splitmix_at(1234567, j) for j in range(5)] == exp


def test_fill_normal_moments():
    x = oracle.fill_normal(1_000_001, seed=42).astype(np.float64)
    assert abs(x.mean()) < 4e-3 and abs(x.std() - 1.0) < 4e-3
    y = oracle.fill_normal(1000, seed=42, mean=2.0, std=0.5)
    np.testing.assert_allclose(y, 2.0 + 0.5 * x[:1000].astype(np.float32), rtol=1e-6)


def test_fp32_accumulation_build_matches_fp64():
    """liboracle_f32.so (the CPU baseline's build) runs the same loops in fp32:
    within fp32 rounding of the fp64 checker on a conv, a GroupNorm+SiLU, a
    linear and an attention; a dropped term or a changed loop would not be."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 64, 16, 16)).astype(np.float32)
    w = (rng.standard_normal((32, 64, 3, 3)) / 24).astype(np.float32)
    b = rng.standard_normal(32).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    bt = (0.1 * rng.standard_normal(64)).astype(np.float32)
    xl = rng.standard_normal((40, 96)).astype(np.float32)
    wl = (rng.standard_normal((48, 96)) / 10).astype(np.float32)
    q, k, v = (rng.standard_normal((1, 2, 33, 64)).astype(np.float32) for _ in range(3))

    def run():
        return [oracle.conv2d(x, w, b, stride=1, pad=1),
                oracle.group_norm(x, g, bt, 32, eps=1e-5, silu=True),
                oracle.linear(xl, wl, None),
                oracle.attention(q, k, v, layout="bhsd")]
    ref = run()
    with oracle.accumulation("fp32"):
        got = run()
    after = run()
    for r, a, z in zip(ref, got, after):
        assert np.array_equal(r, z)  # the context restores the fp64 build
        rel = np.linalg.norm(a.astype(np.float64) - r) / np.linalg.norm(r)
        assert 0 < rel < 1e-5 or np.array_equal(a, r)
        assert np.max(np.abs(a - r)) <= 1e-4 * max(1.0, float(np.max(np.abs(r))))
