"""GPU parity of the MFMA contraction kernels (di_matmul / di_gemm /
di_linear / di_conv2d) against the CPU oracle on identical inputs.

Tolerances: fp32 paths (exact fp32 MFMA products, fp32 accumulation) use the
reference KAT gate max-rel <= 1e-4.  fp16 paths are compared with the oracle
run on the same fp16-rounded inputs, so only fp32 summation order and the
fp16 rounding of the output differ: rel-L2 <= 2e-3 asserted (the north-star
bar for MFMA contractions is rel-L2 <= 1e-2); max-abs is printed.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from conftest import max_rel, rel_l2

pytestmark = pytest.mark.gpu

F32, F16, NCHW, NHWC = 0, 1, 0, 1
ACT = {"none": 0, "gelu": 1, "geglu": 2, "silu": 3}


def _call(dev, fn, *a):
    import drawinstant
    drawinstant.call(fn, dev.ctx, *a)


def _h(b):
    return 0 if b is None else b.handle


# ---------------- fp32 executor ops: reference KATs ----------------

def test_matmul_kat(dev):
    M, N, K = 32, 48, 24  # wgsl-ops-test.js:165-167
    a = np.array([math.sin(i * 0.3) for i in range(M * K)], np.float32).reshape(M, K)
    b = np.array([math.cos(i * 0.17) for i in range(K * N)], np.float32).reshape(K, N)
    ba, bb, y = dev.storage(a), dev.storage(b), dev.create_buffer(M * N * 4)
    _call(dev, "di_matmul", ba.handle, bb.handle, y.handle, M, N, K, 1, 0, F32)
    assert max_rel(dev.download(y).reshape(M, N), oracle.matmul(a, b)) <= 1e-4


@pytest.mark.parametrize("batched", [0, 1])
def test_matmul_batched_kat(dev, batched):
    Bt, M, N, K = 2, 20, 24, 12  # wgsl-ops-test.js:189-191, :213-215
    a = np.array([math.sin(i * 0.21) for i in range(Bt * M * K)], np.float32).reshape(Bt, M, K)
    nb = Bt * K * N if batched else K * N
    b = np.array([math.cos(i * 0.13) for i in range(nb)], np.float32)
    b = b.reshape((Bt, K, N) if batched else (K, N))
    y = dev.create_buffer(Bt * M * N * 4)
    _call(dev, "di_matmul", dev.storage(a).handle, dev.storage(b).handle, y.handle, M, N, K, Bt,
          batched, F32)
    assert max_rel(dev.download(y).reshape(Bt, M, N), oracle.matmul(a, b, bool(batched))) <= 1e-4


@pytest.mark.parametrize("trans_b", [0, 1])
def test_gemm_kat(dev, trans_b):
    M, N, K = 16, 24, 12  # wgsl-ops-test.js:341-343, :367-369
    a = np.array([math.sin(i * 0.1) for i in range(M * K)], np.float32).reshape(M, K)
    b = np.array([math.cos(i * 0.15) for i in range(K * N)], np.float32)
    b = b.reshape((N, K) if trans_b else (K, N))
    c = np.array([0.01 * i for i in range(N)], np.float32)
    y = dev.create_buffer(M * N * 4)
    _call(dev, "di_gemm", dev.storage(a).handle, dev.storage(b).handle, dev.storage(c).handle,
          y.handle, M, N, K, trans_b, F32)
    assert max_rel(dev.download(y).reshape(M, N), oracle.gemm(a, b, c, bool(trans_b))) <= 1e-4


def test_gemm_fp32_large_ragged(dev, rng):
    M, N, K = 333, 1281, 77
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((N, K)).astype(np.float32)
    c = rng.standard_normal(N).astype(np.float32)
    y = dev.create_buffer(M * N * 4)
    _call(dev, "di_gemm", dev.storage(a).handle, dev.storage(b).handle, dev.storage(c).handle,
          y.handle, M, N, K, 1, F32)
    assert max_rel(dev.download(y).reshape(M, N), oracle.gemm(a, b, c, True)) <= 1e-4


def test_conv3x3_kat(dev):
    cin, cout, h, w = 3, 4, 8, 8  # wgsl-ops-test.js:239-243
    x = np.array([math.sin(i * 0.2) for i in range(cin * h * w)], np.float32).reshape(1, cin, h, w)
    wt = np.array([math.cos(i * 0.13) * 0.5 for i in range(cout * cin * 9)],
                  np.float32).reshape(cout, cin, 3, 3)
    bias = np.array([0.1 * i for i in range(cout)], np.float32)
    y = dev.create_buffer(cout * h * w * 4)
    _call(dev, "di_conv2d", dev.storage(x).handle, dev.storage(wt).handle, dev.storage(bias).handle,
          0, y.handle, 1, cin, cout, h, w, 3, 1, 1, 0, F32, NCHW)
    assert max_rel(dev.download(y).reshape(1, cout, h, w), oracle.conv2d(x, wt, bias)) <= 1e-4


def test_conv1x1_kat(dev):
    cin, cout, h, w = 8, 6, 4, 4  # wgsl-ops-test.js:275-279
    x = np.array([math.sin(i * 0.1) for i in range(cin * h * w)], np.float32).reshape(1, cin, h, w)
    wt = np.array([math.cos(i * 0.2) * 0.3 for i in range(cout * cin)],
                  np.float32).reshape(cout, cin, 1, 1)
    bias = np.array([0.05 * i for i in range(cout)], np.float32)
    y = dev.create_buffer(cout * h * w * 4)
    _call(dev, "di_conv2d", dev.storage(x).handle, dev.storage(wt).handle, dev.storage(bias).handle,
          0, y.handle, 1, cin, cout, h, w, 1, 1, 0, 0, F32, NCHW)
    assert max_rel(dev.download(y).reshape(1, cout, h, w), oracle.conv2d(x, wt, bias)) <= 1e-4


def test_conv_fp32_stride2_batched_residual(dev, rng):
    x = rng.standard_normal((2, 5, 9, 10)).astype(np.float32)
    wt = rng.standard_normal((7, 5, 3, 3)).astype(np.float32)
    bias = rng.standard_normal(7).astype(np.float32)
    ref = oracle.conv2d(x, wt, bias, stride=2)
    r = rng.standard_normal(ref.shape).astype(np.float32)
    y = dev.create_buffer(ref.nbytes)
    _call(dev, "di_conv2d", dev.storage(x).handle, dev.storage(wt).handle, dev.storage(bias).handle,
          dev.storage(r).handle, y.handle, 2, 5, 7, 9, 10, 3, 2, 1, 0, F32, NCHW)
    assert max_rel(dev.download(y).reshape(ref.shape), ref + r) <= 1e-4


def _silu_res_ref(x, wt, bias, r):
    """fused-conv.js:206 evaluated by the oracle: conv (+bias) -> SiLU -> + r."""
    conv = oracle.conv2d(x, wt, bias)
    return oracle.unary("SiLU", conv.ravel()).reshape(conv.shape) + r


@pytest.mark.parametrize("n,c,h,w", [
    (1, 1280, 16, 16),   # fused-conv.js SHAPE
    (1, 37, 11, 13),     # ragged: channels and both spatial dims off every tile
    (2, 45, 7, 9),       # ragged, two images
])
def test_conv_silu_residual_epilogue_vs_oracle(dev, rng, n, c, h, w):
    """di_conv2d with DI_CONV_SILU and a residual (the runConvBench fused
    path, fp32 NCHW, exact fp32 MFMA) against oracle conv2d -> SiLU -> + r."""
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((c, c, 3, 3)) * math.sqrt(2.0 / (9 * c))).astype(np.float32)
    bias = (rng.standard_normal(c) * 0.1).astype(np.float32)
    r = rng.standard_normal((n, c, h, w)).astype(np.float32)
    ref = _silu_res_ref(x, wt, bias, r)
    y = dev.create_buffer(ref.nbytes)
    _call(dev, "di_conv2d", dev.storage(x).handle, dev.storage(wt).handle, dev.storage(bias).handle,
          dev.storage(r).handle, y.handle, n, c, c, h, w, 3, 1, 1, 4, F32, NCHW)  # 4 = DI_CONV_SILU
    got = dev.download(y).reshape(ref.shape)
    err = max_rel(got, ref)
    print(f"[conv silu+res {n}x{c}x{h}x{w}] max-rel {err:.2e}", flush=True)
    assert err <= 1e-4
    # the epilogue is SiLU *then* the residual: a plain conv + r is far off
    assert max_rel(oracle.conv2d(x, wt, bias) + r, ref) > 1e-2


def test_run_conv_bench_output_vs_oracle(dev):
    """The runConvBench entry point's own fused output (its seeded inputs at
    the reference SHAPE [1,1280,16,16]) against the oracle composition."""
    from drawinstant import fused
    res = fused.run_conv_bench(dev, repeats=1, warm_ms=20.0, return_tensors=True)
    t = res["tensors"]
    ref = _silu_res_ref(t["x"], t["w"], t["bias"], t["r"])
    err = max_rel(t["y"], ref)
    print(f"[run_conv_bench] max-rel {err:.2e}", flush=True)
    assert t["y"].shape == (1, 1280, 16, 16)
    assert err <= 1e-4


# ---------------- fp16 MFMA paths ----------------

def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


@pytest.mark.parametrize("M,N,K,act,res", [
    (4096, 320, 320, "none", True),     # proj_in / to_out + residual
    (4096, 960, 320, "none", False),    # fused QKV
    (4096, 2560, 320, "geglu", False),  # GEGLU proj (64x64 level)
    (4096, 320, 1280, "none", True),    # FF out + residual
    (77, 640, 1024, "none", False),     # cross-attn K/V from context
    (64, 1280, 5120, "none", True),     # 8x8 level FF out (split-K)
    (256, 10240, 1280, "geglu", False), # 16x16 level GEGLU
    (100, 96, 40, "gelu", False),       # ragged M, N, K % 8 == 0
    (1, 1280, 1280, "silu", False),     # GEMV-shaped
])
def test_linear_fp16(dev, rng, M, N, K, act, res):
    print(f"[linear f16] M={M} N={N} K={K} act={act}", flush=True)
    x = _f16(rng.standard_normal((M, K)))
    w = _f16(rng.standard_normal((N, K)) * math.sqrt(1.0 / K))
    b = (0.01 * rng.standard_normal(N)).astype(np.float32)
    nout = N // 2 if act == "geglu" else N
    r = _f16(rng.standard_normal((M, nout))) if res else None
    y = dev.create_buffer(M * nout * 2)
    br = dev.storage(r) if res else None
    _call(dev, "di_linear", dev.storage(x).handle, dev.storage(w).handle, dev.storage(b).handle,
          _h(br), y.handle, M, N, K, ACT[act], F16)
    got = dev.download(y, np.float16).astype(np.float32).reshape(M, nout)
    full = oracle.linear(x.astype(np.float32), w.astype(np.float32), b)
    if act == "geglu":
        grp = full.reshape(M, N // 32, 2, 16)
        ref = grp[:, :, 0, :].reshape(M, nout) * oracle.unary("GELU", grp[:, :, 1, :].reshape(M, nout))
    elif act == "gelu":
        ref = oracle.unary("GELU", full)
    elif act == "silu":
        ref = oracle.unary("SiLU", full)
    else:
        ref = full
    if res:
        ref = ref + r.astype(np.float32)
    err = rel_l2(got, ref)
    print(f"   rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e}", flush=True)
    assert err <= 2e-3


@pytest.mark.parametrize("M,N,K,act,res", [
    (300, 640, 512, "none", True),    # ragged M, residual
    (256, 1280, 512, "geglu", False),  # GEGLU pairs
    (200, 104, 192, "gelu", False),   # N % 32 != 0, ragged tiles
])
def test_linear_fp16_every_plan(dev, rng, monkeypatch, M, N, K, act, res):
    """Every tile shape x split-K factor (planner overridden) gives the same
    result: covers the LDS-staged vector epilogue, split-K partial stores and
    the vector reducer with bias / residual / activation / GEGLU."""
    import drawinstant
    x = _f16(rng.standard_normal((M, K)))
    w = _f16(rng.standard_normal((N, K)) * math.sqrt(1.0 / K))
    b = (0.01 * rng.standard_normal(N)).astype(np.float32)
    nout = N // 2 if act == "geglu" else N
    r = _f16(rng.standard_normal((M, nout))) if res else None
    bx, bw, bb = dev.storage(x), dev.storage(w), dev.storage(b)
    br = dev.storage(r) if res else None
    y = dev.create_buffer(M * nout * 2)
    full = oracle.linear(x.astype(np.float32), w.astype(np.float32), b)
    if act == "geglu":
        grp = full.reshape(M, N // 32, 2, 16)
        ref = grp[:, :, 0, :].reshape(M, nout) * oracle.unary("GELU", grp[:, :, 1, :].reshape(M, nout))
    elif act == "gelu":
        ref = oracle.unary("GELU", full)
    else:
        ref = full
    if res:
        ref = ref + r.astype(np.float32)
    for tile in (0, 1, 2, 3, 5, 6, 7, 8, 9, 10, 11, 12, 14):
        for splits in (1, 2, 3):
            monkeypatch.setenv("DI_GEMM_TILE", str(tile))
            monkeypatch.setenv("DI_GEMM_SPLITS", str(splits))
            dev.fill_normal(y, M * nout, 3, dtype=F16)  # stale output must be overwritten
            _call(dev, "di_linear", bx.handle, bw.handle, bb.handle, _h(br), y.handle, M, N, K,
                  ACT[act], F16)
            got = dev.download(y, np.float16).astype(np.float32).reshape(M, nout)
            err = rel_l2(got, ref)
            print(f"[plan] M={M} N={N} K={K} {act} tile={tile} splits={splits} rel-L2 {err:.2e}",
                  flush=True)
            assert err <= 2e-3


def _conv_case(dev, rng, n, cin, cout, h, w, k, s, pad, up=1, res=False, cin_pad=None):
    """NHWC fp16 conv vs the oracle's NCHW conv on the same fp16 values."""
    x = _f16(rng.standard_normal((n, h, w, cin)))
    wt = _f16(rng.standard_normal((cout, k, k, cin)) * math.sqrt(2.0 / (cin * k * k)))
    bias = (0.01 * rng.standard_normal(cout)).astype(np.float32)
    hi, wi = h * up, w * up
    ho, wo = (hi + 2 * pad - k) // s + 1, (wi + 2 * pad - k) // s + 1
    r = _f16(rng.standard_normal((n, ho, wo, cout))) if res else None
    y = dev.create_buffer(n * ho * wo * cout * 2)
    flags = 2 if up == 2 else 0
    _call(dev, "di_conv2d", dev.storage(x).handle, dev.storage(wt).handle, dev.storage(bias).handle,
          _h(dev.storage(r) if res else None), y.handle, n, cin, cout, h, w, k, s, pad, flags, F16,
          NHWC)
    got = dev.download(y, np.float16).astype(np.float32).reshape(n, ho, wo, cout)
    xin = x.astype(np.float32).transpose(0, 3, 1, 2)
    if up == 2:
        xin = xin.repeat(2, axis=2).repeat(2, axis=3)
    ref = oracle.conv2d(xin, wt.astype(np.float32).transpose(0, 3, 1, 2), bias, stride=s, pad=pad)
    ref = ref.transpose(0, 2, 3, 1)
    if res:
        ref = ref + r.astype(np.float32)
    err = rel_l2(got, ref)
    print(f"   rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e}", flush=True)
    return err


@pytest.mark.parametrize("n,cin,cout,h,w,k,s,pad,up,res", [
    (1, 320, 320, 64, 64, 3, 1, 1, 1, False),   # cfg2 shape
    (1, 320, 640, 32, 32, 3, 1, 1, 1, False),   # cfg3 conv1
    (1, 640, 640, 32, 32, 3, 1, 1, 1, True),    # cfg3 conv2 + skip residual
    (1, 320, 640, 32, 32, 1, 1, 0, 1, False),   # cfg3 1x1 skip
    (1, 320, 320, 64, 64, 3, 2, 1, 1, False),   # Downsample2D
    (1, 1280, 1280, 8, 8, 3, 1, 1, 2, False),   # Upsample2D conv (fused 2x nearest)
    (1, 2560, 1280, 8, 8, 3, 1, 1, 1, False),   # up0 resnet conv1 (8x8, split-K)
    (2, 64, 48, 7, 9, 3, 1, 1, 1, True),        # batch 2, ragged
    # the halo kernel (k_conv3.hip): 2x upsample fused, channel-chunk split-K,
    # batch 2, six chunks, a 256-wide image in 128-pixel row runs
    (1, 640, 640, 16, 16, 3, 1, 1, 2, True),
    (1, 1280, 1280, 16, 16, 3, 1, 1, 1, True),
    (2, 320, 320, 32, 32, 3, 1, 1, 1, True),
    (1, 384, 128, 64, 64, 3, 1, 1, 1, False),
    (1, 320, 64, 256, 256, 3, 1, 1, 1, False),
    (1, 8, 320, 64, 64, 3, 1, 1, 1, False),     # conv_in (channels padded to 8)
    (1, 320, 8, 64, 64, 3, 1, 1, 1, False),     # conv_out (padded to 8)
])
def test_conv_nhwc_fp16(dev, rng, n, cin, cout, h, w, k, s, pad, up, res):
    print(f"[conv f16] n={n} cin={cin} cout={cout} {h}x{w} k={k} s={s} up={up}", flush=True)
    assert _conv_case(dev, rng, n, cin, cout, h, w, k, s, pad, up, res) <= 2e-3


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 5, 6, 7, 8, 9, 10, 11, 12, 14])
def test_conv_nhwc_fp16_every_tile(dev, rng, monkeypatch, tile):
    """conv3x3 (implicit GEMM, buffer-load path) with every tile shape forced,
    including the eight-wavefront k-half variants, split-K 1 and 2."""
    for splits in (1, 2):
        monkeypatch.setenv("DI_GEMM_TILE", str(tile))
        monkeypatch.setenv("DI_GEMM_SPLITS", str(splits))
        print(f"[conv tile] tile={tile} splits={splits}", flush=True)
        assert _conv_case(dev, rng, 1, 128, 192, 12, 12, 3, 1, 1, res=True) <= 2e-3


def test_conv_nchw_f32_via_f16_compute_cfg2(dev, rng):
    """cfg2: fp32 NCHW tensors, fp16-in / fp32-acc MFMA (DI_CONV_F16_COMPUTE);
    compared with the fp32 oracle on the unrounded fp32 inputs: rel-L2 <= 1e-2."""
    x = rng.standard_normal((1, 320, 64, 64)).astype(np.float32)
    wt = (rng.standard_normal((320, 320, 3, 3)) * math.sqrt(2.0 / 2880)).astype(np.float32)
    bias = (0.01 * rng.standard_normal(320)).astype(np.float32)
    y = dev.create_buffer(x.nbytes)
    _call(dev, "di_conv2d", dev.storage(x).handle, dev.storage(wt).handle, dev.storage(bias).handle,
          0, y.handle, 1, 320, 320, 64, 64, 3, 1, 1, 1, F32, NCHW)
    got = dev.download(y).reshape(x.shape)
    ref = oracle.conv2d(x, wt, bias)
    err = rel_l2(got, ref)
    print(f"   cfg2 rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e}", flush=True)
    assert err <= 1e-2


# ---------------- fp32 with fp16-resident weights (DI_F32W16) ----------------
F32W16 = 2


def _run_pair(dev, fn, make_args, w16):
    """Run `fn` with the weight operand fp16 (DI_F32W16) and, on the same
    fp16 values widened on the host, with DI_F32; both outputs."""
    w32 = w16.astype(np.float32)
    outs = []
    for dt, w in ((F32W16, w16), (F32, w32)):
        y, n, args = make_args(dev.storage(w))
        _call(dev, fn, *args(dt))
        outs.append(dev.download(y, np.float32, (n,)))
    return outs


@pytest.mark.parametrize("M,N,K,bb", [(77, 1280, 1024, 0), (4096, 320, 320, 0), (33, 45, 27, 0),
                                      (64, 96, 64, 1), (1, 1280, 320, 0)])
def test_matmul_w16_equals_widened(dev, rng, M, N, K, bb):
    """Same plan and summation order: bit-identical to DI_F32 on the widened
    weights, aligned and ragged (per-element B loads) shapes, shared and
    batched B."""
    batch = 3 if bb else 1
    a = rng.standard_normal((batch, M, K)).astype(np.float32)
    w = (rng.standard_normal(((batch if bb else 1), K, N)) / math.sqrt(K)).astype(np.float16)
    ba = dev.storage(a)

    def make(bw):
        y = dev.create_buffer(batch * M * N * 4)
        return y, batch * M * N, lambda dt: (ba.handle, bw.handle, y.handle, M, N, K, batch, bb,
                                             dt)
    w16, w32 = _run_pair(dev, "di_matmul", make, w)
    assert np.array_equal(w16, w32)
    ref = oracle.matmul(a, w.astype(np.float32), batched_b=bool(bb))
    assert max_rel(w16.reshape(ref.shape), ref) <= 1e-4


@pytest.mark.parametrize("trans_b", [0, 1])
def test_gemm_w16_equals_widened(dev, rng, trans_b):
    M, N, K = 2, 1280, 320  # the time-embedding linear
    a = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K) if trans_b else (K, N)) * 0.05).astype(np.float16)
    c = rng.standard_normal(N).astype(np.float32)
    ba, bc = dev.storage(a), dev.storage(c)

    def make(bw):
        y = dev.create_buffer(M * N * 4)
        return y, M * N, lambda dt: (ba.handle, bw.handle, bc.handle, y.handle, M, N, K, trans_b,
                                     dt)
    w16, w32 = _run_pair(dev, "di_gemm", make, w)
    assert np.array_equal(w16, w32)


@pytest.mark.parametrize("cin,cout,h,k,s", [(320, 320, 16, 3, 1), (4, 320, 16, 3, 1),
                                            (64, 128, 8, 1, 1), (128, 128, 16, 3, 2)])
def test_conv_nchw_w16_equals_widened(dev, rng, cin, cout, h, k, s):
    x = rng.standard_normal((1, cin, h, h)).astype(np.float32)
    w = (rng.standard_normal((cout, cin, k, k)) / math.sqrt(cin * k * k)).astype(np.float16)
    bias = rng.standard_normal(cout).astype(np.float32) * 0.1
    pad = k // 2
    ho = (h + 2 * pad - k) // s + 1
    bx, bbias = dev.storage(x), dev.storage(bias)

    def make(bw):
        y = dev.create_buffer(cout * ho * ho * 4)
        return y, cout * ho * ho, lambda dt: (bx.handle, bw.handle, bbias.handle, 0, y.handle, 1,
                                              cin, cout, h, h, k, s, pad, 0, dt, NCHW)
    w16, w32 = _run_pair(dev, "di_conv2d", make, w)
    assert np.array_equal(w16, w32)
    ref = oracle.conv2d(x, w.astype(np.float32), bias, stride=s, pad=pad)
    assert max_rel(w16.reshape(ref.shape), ref) <= 1e-4


def test_w16_rejected_outside_contractions(dev):
    import drawinstant
    x = dev.create_buffer(64)
    with pytest.raises(drawinstant.DiError):
        _call(dev, "di_unary", 0, x.handle, x.handle, 16, F32W16)
    with pytest.raises(drawinstant.DiError):  # NHWC conv is fp16 already
        _call(dev, "di_conv2d", x.handle, x.handle, 0, 0, x.handle, 1, 8, 8, 1, 1, 1, 1, 0, 0,
              F32W16, NHWC)
