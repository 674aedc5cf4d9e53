"""Fused-block entry points: the ``run*Bench`` functions of draw-instant's
fused-*.js, on libdrawinstant_hip.

Each function builds seeded inputs at the reference's SHAPE, runs a *naive*
path (the unfused op-by-op composition, one executor dispatch per op, fp32
NCHW as the reference's executor) and the *fused* library entry point, checks
them against each other and times both with the interleaved slope method
(``timing.measure_pair``).  The return value has the reference's schema:

    {shape, naive, fused, speedup, correctness: {maxAbsDiff, l2},
     dispatchesNaive, dispatchesFused, ...}

(``naive`` / ``fused`` in ms per iteration, median of the repeats; ``l2`` is
the RMS difference, as the reference computes it.)  The reference fills its
inputs with unseeded Math.random; here every tensor is drawn from a seeded
numpy generator so results are reproducible.

| function | reference |
|---|---|
| run_group_norm_bench | fused-groupnorm.js:280-383 |
| run_conv_bench | fused-conv.js:174-284 |
| run_resnet_bench | fused-resnet.js:267-420 |
| run_attn_bench | fused-attn.js:364-476 |
| run_cross_attn_bench | fused-cross-attn.js:220-318 |
| run_ffn_bench | fused-block.js:219-342 |
| run_block_bench | fused-block-full.js:456-686 |
| run_tembed_bench | fused-tembed.js:175-267 |
"""
from __future__ import annotations

import math
from typing import Callable, Optional

import numpy as np

from .device import F16, F32, NCHW, NHWC, Device, call
from .executor import create_dispatchers, row_major_strides
from .timing import REPEATS, WARM_MS, measure_pair, median

GN_SHAPE = {"B": 1, "C": 1280, "G": 32, "H": 16, "W": 16}
CONV_SHAPE = {"B": 1, "C": 1280, "H": 16, "W": 16, "K": 3}
RESNET_SHAPE = {"B": 1, "C": 1280, "G": 32, "H": 16, "W": 16, "K": 3}
ATTN_SHAPE = {"B": 2, "H": 20, "S": 256, "HEAD_DIM": 64}
CROSS_ATTN_SHAPE = {"B": 2, "HEADS": 20, "S_Q": 256, "S_KV": 77, "HEAD_DIM": 64}
FFN_SHAPE = {"B": 2, "S": 1024, "D": 1280, "D_FFN": 5120}
BLOCK_SHAPE = {"B": 2, "S": 256, "D": 1280, "D_FFN": 5120, "H": 20, "HEAD_DIM": 64}
TEMBED_SHAPE = {"T": 500.0, "EMB": 320, "HID": 1280}

UN_SILU, UN_COS, UN_SIN, UN_GELU_TANH = 8, 5, 4, 11
DI_CONV_SILU = 4
DI_ACT_GELU_TANH = 4


class _Bench:
    """Buffer bookkeeping + the common result assembly."""

    def __init__(self, device: Optional[Device], seed: int):
        self.own = device is None
        self.dev = device or Device(0)
        self.rng = np.random.default_rng(seed)
        self.bufs = []
        self.d = create_dispatchers(self.dev)

    def up(self, a):
        b = self.dev.storage(np.ascontiguousarray(a))
        self.bufs.append(b)
        return b

    def out(self, nbytes):
        b = self.dev.create_buffer(max(int(nbytes), 4))
        self.bufs.append(b)
        return b

    def rand(self, shape, s=0.3):
        """Uniform (-s, s), the reference's (Math.random() - 0.5) * 2 * s."""
        return ((self.rng.random(shape) - 0.5) * 2.0 * s).astype(np.float32)

    def read(self, b, shape, dt=np.float32):
        return self.dev.download(b, dt, shape)

    def finish(self, shape, run_naive: Callable, run_fused: Callable, y_naive, y_fused,
               n_naive: int, n_fused: int, repeats: int, warm_ms: float, **extra):
        run_naive()
        run_fused()
        self.dev.sync()
        yn, yf = y_naive(), y_fused()
        d = np.abs(yn.astype(np.float64) - yf.astype(np.float64))
        corr = {"maxAbsDiff": float(d.max()), "l2": float(np.sqrt(np.mean(d * d)))}
        t = measure_pair(self.dev, run_naive, run_fused, repeats, warm_ms)
        naive, fused = median(t["a"]), median(t["b"])
        for b in self.bufs:
            b.destroy()
        if self.own:
            self.dev.destroy()
        res = {"shape": dict(shape), "naive": naive, "fused": fused,
               "speedup": naive / fused if fused > 0 else float("inf"), "correctness": corr,
               "dispatchesNaive": n_naive, "dispatchesFused": n_fused}
        res.update(extra)
        return res


def _bstr(t_dims, dims):
    st, out = 1, [0] * len(dims)
    pad = len(dims) - len(t_dims)
    for i in range(len(t_dims) - 1, -1, -1):
        out[pad + i] = 0 if (t_dims[i] == 1 and dims[pad + i] != 1) else st
        st *= t_dims[i]
    return out


def _mul_bcast(d, a, b, y, a_dims, b_dims):
    dims = [max(x, z) for x, z in zip(a_dims, b_dims)]
    n = int(np.prod(dims))
    d.binary_bcast["Mul"](a, b, y, len(dims), dims, _bstr(a_dims, dims), _bstr(b_dims, dims), n)


def _add_bcast(d, a, b, y, a_dims, b_dims):
    dims = [max(x, z) for x, z in zip(a_dims, b_dims)]
    n = int(np.prod(dims))
    d.binary_bcast["Add"](a, b, y, len(dims), dims, _bstr(a_dims, dims), _bstr(b_dims, dims), n)


def _transpose(d, x, y, dims, perm):
    new = [dims[i] for i in perm]
    r = len(dims)
    d.transpose(x, y, r, new + [1] * (4 - r), row_major_strides(dims) + [0] * (4 - r),
                list(perm) + [0] * (4 - r), int(np.prod(dims)))


# ------------------------------------------------------------- GroupNorm --
def run_group_norm_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                         repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 1):
    """GroupNorm (no SiLU).  naive: the executor's unfused ONNX export of
    GroupNorm (InstanceNorm over [N, G, cpg*HW] -> Mul gamma -> Add beta, 3
    dispatches); fused: di_group_norm."""
    S = dict(shape or GN_SHAPE)
    B, C, G, H, W = S["B"], S["C"], S["G"], S["H"], S["W"]
    bn = _Bench(device, seed)
    n, cpg, hw = B * C * H * W, C // G, H * W
    x = bn.up(bn.rand(n))
    g = bn.up(np.ones(C, np.float32))
    be = bn.up(np.zeros(C, np.float32))
    ones_g, zeros_g = bn.up(np.ones(G, np.float32)), bn.up(np.zeros(G, np.float32))
    t1, t2, yn, yf = bn.out(n * 4), bn.out(n * 4), bn.out(n * 4), bn.out(n * 4)
    d = bn.d

    def naive():
        d.instance_norm(x, ones_g, zeros_g, t1, B, G, cpg * hw, 1e-5)
        _mul_bcast(d, t1, g, t2, [B, C, H, W], [1, C, 1, 1])
        _add_bcast(d, t2, be, yn, [B, C, H, W], [1, C, 1, 1])

    def fused():
        d.group_norm(x, g, be, yf, B, G, cpg, hw, 1e-5)

    return bn.finish(S, naive, fused, lambda: bn.read(yn, (n,)), lambda: bn.read(yf, (n,)), 3, 1,
                     repeats, warm_ms, bytesSaved=2 * n * 4 * 2)


# ------------------------------------------------------------------ Conv --
def run_conv_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                   repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 2,
                   return_tensors: bool = False):
    """conv3x3 with the WGSL_CONV epilogue silu(conv + bias) + residual.
    naive: conv -> SiLU -> Add (3 dispatches); fused: one di_conv2d with
    DI_CONV_SILU and the residual.  fp32 NCHW, exact fp32 MFMA.

    ``return_tensors`` adds ``tensors``: the host inputs (x, w, bias, r in
    NCHW / OIHW) and the fused output y, for a parity check of the fused
    epilogue against an independent evaluation."""
    S = dict(shape or CONV_SHAPE)
    B, C, H, W, K = S["B"], S["C"], S["H"], S["W"], S["K"]
    bn = _Bench(device, seed)
    n = B * C * H * W
    xs, rs = bn.rand(n), bn.rand(n)
    ws = bn.rand(C * C * K * K, math.sqrt(3.0 / (C * K * K)))
    bs = bn.rand(C, 0.05)
    x, r, w, bias = bn.up(xs), bn.up(rs), bn.up(ws), bn.up(bs)
    t1, t2, yn, yf = bn.out(n * 4), bn.out(n * 4), bn.out(n * 4), bn.out(n * 4)
    d = bn.d

    def naive():
        d.conv_mm(x, w, bias, t1, B, C, C, H, W, K, 1, K // 2)
        d.unary["SiLU"](t1, t2, n)
        d.binary["Add"](t2, r, yn, n)

    def fused():
        call("di_conv2d", bn.dev.ctx, x.handle, w.handle, bias.handle, r.handle, yf.handle, B, C,
             C, H, W, K, 1, K // 2, DI_CONV_SILU, F32, NCHW)

    kept = {}

    def read_fused():
        y = bn.read(yf, (n,))
        if return_tensors:
            kept["tensors"] = {"x": xs.reshape(B, C, H, W), "w": ws.reshape(C, C, K, K),
                               "bias": bs, "r": rs.reshape(B, C, H, W),
                               "y": y.reshape(B, C, H, W)}
        return y

    res = bn.finish(S, naive, fused, lambda: bn.read(yn, (n,)), read_fused, 3, 1,
                    repeats, warm_ms, flops=2.0 * B * H * W * C * C * K * K)
    res.update(kept)
    return res


# ---------------------------------------------------------------- ResNet --
def run_resnet_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                     repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 3):
    """GN+SiLU -> conv -> GN+SiLU -> conv + x (C_in = C_out, no temb).
    naive: 7 fp32 NCHW dispatches (GN, SiLU, conv, GN, SiLU, conv, Add);
    fused: di_resnet_block on NHWC fp16 (input converted once, outside the
    timed region; the comparison converts the output back)."""
    from .blocks import resnet_block, upload_resnet
    S = dict(shape or RESNET_SHAPE)
    B, C, G, H, W, K = S["B"], S["C"], S["G"], S["H"], S["W"], S["K"]
    bn = _Bench(device, seed)
    n, hw = B * C * H * W, H * W
    xs = bn.rand(n, 1.0)
    sd = {}
    p = "res"
    for i in (1, 2):
        sd[f"{p}.norm{i}.weight"] = (1 + 0.02 * bn.rng.standard_normal(C)).astype(np.float32)
        sd[f"{p}.norm{i}.bias"] = (0.02 * bn.rng.standard_normal(C)).astype(np.float32)
        sd[f"{p}.conv{i}.weight"] = (bn.rng.standard_normal((C, C, K, K)) *
                                     math.sqrt(2.0 / (C * K * K))).astype(np.float32)
        sd[f"{p}.conv{i}.bias"] = (0.01 * bn.rng.standard_normal(C)).astype(np.float32)
    x = bn.up(xs)
    g1, b1 = bn.up(sd[p + ".norm1.weight"]), bn.up(sd[p + ".norm1.bias"])
    g2, b2 = bn.up(sd[p + ".norm2.weight"]), bn.up(sd[p + ".norm2.bias"])
    w1, c1 = bn.up(sd[p + ".conv1.weight"]), bn.up(sd[p + ".conv1.bias"])
    w2, c2 = bn.up(sd[p + ".conv2.weight"]), bn.up(sd[p + ".conv2.bias"])
    t = [bn.out(n * 4) for _ in range(6)]
    yn = bn.out(n * 4)
    rw = upload_resnet(bn.dev, sd, p)
    xh, yh, yf = bn.out(n * 2), bn.out(n * 2), bn.out(n * 4)
    call("di_layout_convert", bn.dev.ctx, x.handle, F32, NCHW, xh.handle, F16, NHWC, B, C, H, W)
    d = bn.d

    def naive():
        d.group_norm(x, g1, b1, t[0], B, G, C // G, hw, 1e-5)
        d.unary["SiLU"](t[0], t[1], n)
        d.conv_mm(t[1], w1, c1, t[2], B, C, C, H, W, K, 1, K // 2)
        d.group_norm(t[2], g2, b2, t[3], B, G, C // G, hw, 1e-5)
        d.unary["SiLU"](t[3], t[4], n)
        d.conv_mm(t[4], w2, c2, t[5], B, C, C, H, W, K, 1, K // 2)
        d.binary["Add"](t[5], x, yn, n)

    def fused():
        resnet_block(bn.dev, rw, xh, None, yh, B, C, C, H, W, groups=G)

    def y_fused():
        call("di_layout_convert", bn.dev.ctx, yh.handle, F16, NHWC, yf.handle, F32, NCHW, B, C,
             H, W)
        return bn.read(yf, (n,))

    try:
        return bn.finish(S, naive, fused, lambda: bn.read(yn, (n,)), y_fused, 7, 1, repeats,
                         warm_ms, flops=2 * 2.0 * B * hw * C * C * K * K,
                         fusedPrecision="fp16 NHWC activations and weights, fp32 accumulation")
    finally:
        rw.destroy()


# ------------------------------------------------------------- attention --
def _naive_attention(bn, d, q, k, v, o, B, H, Sq, Skv, dh, scale, layout_bshd):
    """Materialised scores: (transpose to BHSD) -> K^T -> Q.K^T -> *scale ->
    softmax -> P.V (-> transpose back).  Returns a closure and its dispatch
    count."""
    bh = B * H
    qh, kh, vh = (bn.out(B * H * s * dh * 4) for s in (Sq, Skv, Skv))
    kt = bn.out(bh * dh * Skv * 4)
    sc, sc2, p_ = bn.out(bh * Sq * Skv * 4), bn.out(bh * Sq * Skv * 4), bn.out(bh * Sq * Skv * 4)
    ob = bn.out(bh * Sq * dh * 4)
    scal = bn.up(np.array([scale], np.float32))

    def run():
        if layout_bshd:
            _transpose(d, q, qh, [B, Sq, H, dh], [0, 2, 1, 3])
            _transpose(d, k, kh, [B, Skv, H, dh], [0, 2, 1, 3])
            _transpose(d, v, vh, [B, Skv, H, dh], [0, 2, 1, 3])
            qq, kk, vv = qh, kh, vh
        else:
            qq, kk, vv = q, k, v
        _transpose(d, kk, kt, [bh, Skv, dh], [0, 2, 1])
        d.matmul(qq, kt, sc, Sq, Skv, dh, bh, 1)
        _mul_bcast(d, sc, scal, sc2, [bh, Sq, Skv], [1, 1, 1])
        d.softmax(sc2, p_, Skv, bh * Sq)
        if layout_bshd:
            d.matmul(p_, vv, ob, Sq, dh, Skv, bh, 1)
            _transpose(d, ob, o, [B, H, Sq, dh], [0, 2, 1, 3])
        else:
            d.matmul(p_, vv, o, Sq, dh, Skv, bh, 1)
    return run, (9 if layout_bshd else 5)


def run_attn_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                   repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 4):
    """softmax(Q K^T / sqrt(d)) V, [B, S, H, d] (fused-attn.js:69-70).
    naive: materialised scores (9 dispatches); fused: di_attn_self."""
    S = dict(shape or ATTN_SHAPE)
    B, H, Sq, dh = S["B"], S["H"], S["S"], S["HEAD_DIM"]
    bn = _Bench(device, seed)
    n = B * Sq * H * dh
    q, k, v = bn.up(bn.rand(n, 1.0)), bn.up(bn.rand(n, 1.0)), bn.up(bn.rand(n, 1.0))
    yn, yf = bn.out(n * 4), bn.out(n * 4)
    scale = 1.0 / math.sqrt(dh)
    naive, nd = _naive_attention(bn, bn.d, q, k, v, yn, B, H, Sq, Sq, dh, scale, True)

    def fused():
        call("di_attn_self", bn.dev.ctx, q.handle, k.handle, v.handle, yf.handle, B, H, Sq, dh,
             0, scale, F32)

    return bn.finish(S, naive, fused, lambda: bn.read(yn, (n,)), lambda: bn.read(yf, (n,)), nd, 1,
                     repeats, warm_ms, flops=4.0 * B * H * Sq * Sq * dh,
                     fusedPrecision="fp16 operands (staged from fp32), fp32 softmax/accumulation")


def run_cross_attn_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                         repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 5):
    """Cross attention over S_KV keys, [B, H, S, d] (fused-cross-attn.js:51-52).
    naive: K^T, Q.K^T, scale, softmax, P.V (5 dispatches); fused:
    di_attn_cross."""
    S = dict(shape or CROSS_ATTN_SHAPE)
    B, H, Sq, Skv, dh = S["B"], S["HEADS"], S["S_Q"], S["S_KV"], S["HEAD_DIM"]
    bn = _Bench(device, seed)
    nq, nk = B * H * Sq * dh, B * H * Skv * dh
    q, k, v = bn.up(bn.rand(nq, 1.0)), bn.up(bn.rand(nk, 1.0)), bn.up(bn.rand(nk, 1.0))
    yn, yf = bn.out(nq * 4), bn.out(nq * 4)
    scale = 1.0 / math.sqrt(dh)
    naive, nd = _naive_attention(bn, bn.d, q, k, v, yn, B, H, Sq, Skv, dh, scale, False)

    def fused():
        call("di_attn_cross", bn.dev.ctx, q.handle, k.handle, v.handle, yf.handle, B, H, Sq, Skv,
             dh, 1, scale, F32)

    return bn.finish(S, naive, fused, lambda: bn.read(yn, (nq,)), lambda: bn.read(yf, (nq,)), nd,
                     1, repeats, warm_ms, flops=4.0 * B * H * Sq * Skv * dh,
                     fusedPrecision="fp16 operands (staged from fp32), fp32 softmax/accumulation")


# ------------------------------------------------------------------- FFN --
def _ffn_weights(bn, D, F):
    w1 = bn.up(bn.rand(F * D, math.sqrt(3.0 / D)))
    b1 = bn.up(bn.rand(F, 0.02))
    w2 = bn.up(bn.rand(D * F, math.sqrt(3.0 / F)))
    b2 = bn.up(bn.rand(D, 0.02))
    return w1, b1, w2, b2


def run_ffn_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                  repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 6):
    """Y = X + W2 GELU_tanh(W1 X + b1) + b2 (fused-block.js WGSL_MATMUL
    epilogues :54-115).  naive: gemm, GELU, gemm, Add (4 dispatches); fused:
    di_ffn (2 MFMA GEMMs with the GELU and residual in their epilogues).
    fp32 operands."""
    S = dict(shape or FFN_SHAPE)
    B, Sx, D, F = S["B"], S["S"], S["D"], S["D_FFN"]
    rows = B * Sx
    bn = _Bench(device, seed)
    x = bn.up(bn.rand(rows * D, 1.0))
    w1, b1, w2, b2 = _ffn_weights(bn, D, F)
    h1, h2, h3, yn, yf = (bn.out(rows * F * 4), bn.out(rows * F * 4), bn.out(rows * D * 4),
                          bn.out(rows * D * 4), bn.out(rows * D * 4))
    d = bn.d

    def naive():
        d.gemm(x, w1, b1, h1, rows, F, D, 1)
        call("di_unary", bn.dev.ctx, UN_GELU_TANH, h1.handle, h2.handle, rows * F, F32)
        d.gemm(h2, w2, b2, h3, rows, D, F, 1)
        d.binary["Add"](h3, x, yn, rows * D)

    def fused():
        call("di_ffn", bn.dev.ctx, x.handle, w1.handle, b1.handle, w2.handle, b2.handle, yf.handle,
             rows, D, F, DI_ACT_GELU_TANH, F32)

    return bn.finish(S, naive, fused, lambda: bn.read(yn, (rows * D,)),
                     lambda: bn.read(yf, (rows * D,)), 4, 2, repeats, warm_ms,
                     flops=4.0 * rows * D * F)


# -------------------------------------------------------- transformer block --
def run_block_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                    repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 7):
    """Pre-LN transformer block (fused-block-full.js:456-686): LN -> Q, K, V
    -> attention -> out proj + residual -> LN -> FFN (GELU_tanh) + residual.
    naive: materialised attention and unfused epilogues (one dispatch per op);
    fused (9 dispatches, as the reference's fused chain): di_layer_norm, three
    di_linear, di_attn_self, di_linear + residual, di_layer_norm, di_linear
    with the GELU epilogue, di_linear + residual.  fp32 operands."""
    S = dict(shape or BLOCK_SHAPE)
    B, Sx, D, F, H, dh = S["B"], S["S"], S["D"], S["D_FFN"], S["H"], S["HEAD_DIM"]
    rows = B * Sx
    bn = _Bench(device, seed)
    d, ctx = bn.d, bn.dev.ctx
    x = bn.up(bn.rand(rows * D, 1.0))
    ln1g, ln1b = bn.up((1 + 0.02 * bn.rng.standard_normal(D)).astype(np.float32)), \
        bn.up((0.02 * bn.rng.standard_normal(D)).astype(np.float32))
    ln2g, ln2b = bn.up((1 + 0.02 * bn.rng.standard_normal(D)).astype(np.float32)), \
        bn.up((0.02 * bn.rng.standard_normal(D)).astype(np.float32))
    wq, wk, wv, wo = (bn.up(bn.rand(D * D, math.sqrt(3.0 / D))) for _ in range(4))
    bq, bk, bv, bo = (bn.up(bn.rand(D, 0.02)) for _ in range(4))
    w1, b1, w2, b2 = _ffn_weights(bn, D, F)
    scale = 1.0 / math.sqrt(dh)
    nrd = rows * D
    # naive temporaries
    ln_a, q_, k_, v_, at, o1, h1r, ln_b, f3, yn = (bn.out(nrd * 4) for _ in range(10))
    f1, f2 = bn.out(rows * F * 4), bn.out(rows * F * 4)
    attn_naive, nd_attn = _naive_attention(bn, d, q_, k_, v_, at, B, H, Sx, Sx, dh, scale, True)
    # fused temporaries
    fl, fq, fk, fv, fa, fh, fl2, yf = (bn.out(nrd * 4) for _ in range(8))
    ff = bn.out(rows * F * 4)

    def naive():
        d.layer_norm(x, ln1g, ln1b, ln_a, rows, D, 1e-5)
        d.gemm(ln_a, wq, bq, q_, rows, D, D, 1)
        d.gemm(ln_a, wk, bk, k_, rows, D, D, 1)
        d.gemm(ln_a, wv, bv, v_, rows, D, D, 1)
        attn_naive()
        d.gemm(at, wo, bo, o1, rows, D, D, 1)
        d.binary["Add"](o1, x, h1r, nrd)
        d.layer_norm(h1r, ln2g, ln2b, ln_b, rows, D, 1e-5)
        d.gemm(ln_b, w1, b1, f1, rows, F, D, 1)
        call("di_unary", ctx, UN_GELU_TANH, f1.handle, f2.handle, rows * F, F32)
        d.gemm(f2, w2, b2, f3, rows, D, F, 1)
        d.binary["Add"](f3, h1r, yn, nrd)

    def fused():
        call("di_layer_norm", ctx, x.handle, ln1g.handle, ln1b.handle, fl.handle, rows, D, 1e-5,
             F32)
        for w, b, o in ((wq, bq, fq), (wk, bk, fk), (wv, bv, fv)):
            call("di_linear", ctx, fl.handle, w.handle, b.handle, 0, o.handle, rows, D, D, 0, F32)
        call("di_attn_self", ctx, fq.handle, fk.handle, fv.handle, fa.handle, B, H, Sx, dh, 0,
             scale, F32)
        call("di_linear", ctx, fa.handle, wo.handle, bo.handle, x.handle, fh.handle, rows, D, D, 0,
             F32)
        call("di_layer_norm", ctx, fh.handle, ln2g.handle, ln2b.handle, fl2.handle, rows, D, 1e-5,
             F32)
        # FFN: GELU in the first GEMM's epilogue, the pre-LN residual fh in the
        # second's (di_ffn would add its own, normalised, input instead)
        call("di_linear", ctx, fl2.handle, w1.handle, b1.handle, 0, ff.handle, rows, F, D,
             DI_ACT_GELU_TANH, F32)
        call("di_linear", ctx, ff.handle, w2.handle, b2.handle, fh.handle, yf.handle, rows, D, F, 0,
             F32)

    return bn.finish(S, naive, fused, lambda: bn.read(yn, (nrd,)), lambda: bn.read(yf, (nrd,)),
                     11 + nd_attn, 9, repeats, warm_ms,
                     flops=2.0 * rows * D * D * 4 + 4.0 * B * H * Sx * Sx * dh + 4.0 * rows * D * F,
                     fusedPrecision="attention fp16 operands (staged), GEMMs fp32 MFMA")


# --------------------------------------------------------- timestep embed --
def run_tembed_bench(device: Optional[Device] = None, shape=None, on_progress=None,
                     repeats: int = REPEATS, warm_ms: float = WARM_MS, seed: int = 8):
    """Timestep embedding (fused-tembed.js): [cos(t f) || sin(t f)],
    f_i = exp(-ln(1e4) i / (EMB/2)) -> Linear -> SiLU -> Linear.
    naive: t*f, cos, sin, 2 concat copies, gemm, SiLU, gemm (8 dispatches);
    fused: di_tembed (one GEMV pair).  fp32 weights."""
    S = dict(shape or TEMBED_SHAPE)
    T, E, Hd = S["T"], S["EMB"], S["HID"]
    half = E // 2
    bn = _Bench(device, seed)
    d, ctx = bn.d, bn.dev.ctx
    t = bn.up(np.array([T], np.float32))
    freqs = bn.up(np.exp(-math.log(10000.0) * np.arange(half, dtype=np.float64) / half)
                  .astype(np.float32))
    w1 = bn.up(bn.rand(Hd * E, math.sqrt(3.0 / E)))
    b1 = bn.up(bn.rand(Hd, 0.02))
    w2 = bn.up(bn.rand(Hd * Hd, math.sqrt(3.0 / Hd)))
    b2 = bn.up(bn.rand(Hd, 0.02))
    arg, c_, s_, emb, h1, h2, yn, yf = (bn.out(half * 4), bn.out(half * 4), bn.out(half * 4),
                                        bn.out(E * 4), bn.out(Hd * 4), bn.out(Hd * 4),
                                        bn.out(Hd * 4), bn.out(Hd * 4))

    def naive():
        _mul_bcast(d, t, freqs, arg, [1], [half])
        d.unary["Cos"](arg, c_, half)
        d.unary["Sin"](arg, s_, half)
        d.concat_copy(c_, emb, half, E, 0, half)
        d.concat_copy(s_, emb, half, E, half, half)
        d.gemm(emb, w1, b1, h1, 1, Hd, E, 1)
        d.unary["SiLU"](h1, h2, Hd)
        d.gemm(h2, w2, b2, yn, 1, Hd, Hd, 1)

    def fused():
        call("di_tembed", ctx, t.handle, w1.handle, b1.handle, w2.handle, b2.handle, yf.handle, 1,
             E, Hd, F32)

    return bn.finish(S, naive, fused, lambda: bn.read(yn, (Hd,)), lambda: bn.read(yf, (Hd,)), 8, 1,
                     repeats, warm_ms, weightBytes=4 * (Hd * E + Hd * Hd))


ALL_BENCHES = {
    "groupnorm": run_group_norm_bench,
    "conv": run_conv_bench,
    "resnet": run_resnet_bench,
    "attn": run_attn_bench,
    "cross_attn": run_cross_attn_bench,
    "ffn": run_ffn_bench,
    "block": run_block_bench,
    "tembed": run_tembed_bench,
}
