"""CPU oracle for the SD-Turbo U-Net op / fused-block path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by bench.py's ``cpu_baseline`` leg, always as the checker (or the timed
CPU baseline), never as the thing measured or shipped.  The product path
(``drawinstant``) must not import this package.

The arithmetic lives in ``oracle.c`` (a plain-C restatement of the reference
WGSL kernels with fp64 accumulation, built to ``_build/liboracle.so``, and
once more with fp32 accumulation for the CPU baseline only); this
module wraps it for numpy arrays and composes the block-level references
(ResNet block, transformer block, full SD2.1 U-Net) in ``blocks.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
# the same loops accumulating in fp32 (-DOR_ACC=float): bench.py's CPU
# baseline only; every check uses the fp64 build
_SO32 = os.path.join(_HERE, "_build", "liboracle_f32.so")
_lib = None
_libs: dict = {}
_use_f32 = False

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float
_dbl = ctypes.c_double


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc -O3 -fopenmp)."""
    args = ["make", "-C", _HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _SO


class accumulation:
    """``with oracle.accumulation("fp32"):`` routes the wrappers to the fp32
    build (the CPU baseline's precision); fp64 otherwise."""

    def __init__(self, kind: str):
        assert kind in ("fp32", "fp64")
        self.kind = kind

    def __enter__(self):
        global _use_f32, _lib
        self.prev = _use_f32
        _use_f32 = self.kind == "fp32"
        _lib = None
        return self

    def __exit__(self, *exc):
        global _use_f32, _lib
        _use_f32 = self.prev
        _lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    so = _SO32 if _use_f32 else _SO
    if so in _libs:
        _lib = _libs[so]
        return _lib
    if not os.path.exists(so):
        build()
    L = ctypes.CDLL(so)
    sig = {
        "or_threads": ([], _int),
        "or_unary": ([_int, _f32p, _f32p, _i64], None),
        "or_binary": ([_int, _f32p, _f32p, _f32p, _i64], None),
        "or_binary_bcast": ([_int, _f32p, _f32p, _f32p, _int, _u32p, _u32p, _u32p, _i64], None),
        "or_pow_scalar": ([_f32p, _f32p, _i64, _flt], None),
        "or_softmax": ([_f32p, _f32p, _i64, _i64], None),
        "or_reduce_mean": ([_f32p, _f32p, _i64, _i64], None),
        "or_group_norm": ([_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _flt, _int], None),
        "or_layer_norm": ([_f32p, _f32p, _f32p, _f32p, _i64, _i64, _flt], None),
        "or_conv2d": ([_f32p, _f32p, ctypes.c_void_p, _f32p] + [_i64] * 8, None),
        "or_matmul": ([_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _int], None),
        "or_gemm": ([_f32p, _f32p, ctypes.c_void_p, _f32p, _i64, _i64, _i64, _int], None),
        "or_linear": ([_f32p, _f32p, ctypes.c_void_p, _f32p, _i64, _i64, _i64], None),
        "or_attention": ([_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _dbl]
                         + [_i64] * 12, None),
        "or_tembed": ([_flt, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64], None),
        "or_resize_nearest": ([_f32p, _f32p, _i64, _i64, _i64, _i64, _i64], None),
        "or_splitmix_at": ([ctypes.c_uint64, ctypes.c_uint64], ctypes.c_uint64),
        "or_fill_normal": ([_f32p, _i64, ctypes.c_uint64, _flt, _flt], None),
    }
    for name, (argt, rest) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = argt
        fn.restype = rest
    _libs[so] = L
    _lib = L
    return L


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr_or_none(a):
    return None if a is None else _f32(a).ctypes.data_as(ctypes.c_void_p)


def threads() -> int:
    return lib().or_threads()


# ---------------- element-wise ----------------

UNARY = {"Sigmoid": 0, "Sqrt": 1, "Neg": 2, "Abs": 3, "Sin": 4, "Cos": 5, "Exp": 6, "Log": 7,
         "SiLU": 8, "GELU": 9, "Erf": 10, "GELU_TANH": 11}
BINARY = {"Add": 0, "Sub": 1, "Mul": 2, "Div": 3, "Pow": 4, "Max": 5, "Min": 6}


def unary(op: str, x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_unary(UNARY[op], x.ravel(), y.ravel(), x.size)
    return y


def binary(op: str, a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    y = np.empty_like(a)
    lib().or_binary(BINARY[op], a.ravel(), b.ravel(), y.ravel(), a.size)
    return y


def binary_bcast(op: str, a, b, out_dims, a_strides, b_strides) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    n = int(np.prod(out_dims))
    y = np.empty(n, np.float32)
    u = lambda v: np.ascontiguousarray(list(v) + [0] * (4 - len(v)), np.uint32)
    lib().or_binary_bcast(BINARY[op], a.ravel(), b.ravel(), y, len(out_dims), u(out_dims),
                          u(a_strides), u(b_strides), n)
    return y.reshape(out_dims)


def pow_scalar(x, e: float) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_pow_scalar(x.ravel(), y.ravel(), x.size, e)
    return y


def softmax(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    inner = x.shape[-1]
    lib().or_softmax(x.ravel(), y.ravel(), x.size // inner, inner)
    return y


def reduce_mean(x) -> np.ndarray:
    x = _f32(x)
    inner = x.shape[-1]
    y = np.empty(x.shape[:-1] + (1,), np.float32)
    lib().or_reduce_mean(x.ravel(), y.ravel(), x.size // inner, inner)
    return y


def resize_nearest(x, h_out: int, w_out: int) -> np.ndarray:
    x = _f32(x)
    *lead, h, w = x.shape
    planes = int(np.prod(lead)) if lead else 1
    y = np.empty(tuple(lead) + (h_out, w_out), np.float32)
    lib().or_resize_nearest(x.ravel(), y.ravel(), planes, h, w, h_out, w_out)
    return y


# ---------------- normalisation ----------------

def group_norm(x, gamma, beta, groups: int, eps: float = 1e-5, silu: bool = False) -> np.ndarray:
    """NCHW GroupNorm (+SiLU), x shape [N, C, *spatial]."""
    x = _f32(x)
    n, c = x.shape[0], x.shape[1]
    hw = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    y = np.empty_like(x)
    lib().or_group_norm(x.ravel(), _f32(gamma), _f32(beta), y.ravel(), n, groups, c // groups,
                        hw, eps, int(silu))
    return y


def instance_norm(x, gamma, beta, eps: float = 1e-5) -> np.ndarray:
    return group_norm(x, gamma, beta, groups=x.shape[1], eps=eps)


def layer_norm(x, gamma, beta, eps: float = 1e-5) -> np.ndarray:
    x = _f32(x)
    inner = x.shape[-1]
    y = np.empty_like(x)
    lib().or_layer_norm(x.ravel(), _f32(gamma), _f32(beta), y.ravel(), x.size // inner, inner, eps)
    return y


# ---------------- contractions ----------------

def conv2d(x, w, bias=None, stride: int = 1, pad: int | None = None) -> np.ndarray:
    """NCHW x, OIHW w (square kernel), symmetric pad (default (K-1)//2)."""
    x, w = _f32(x), _f32(w)
    n, cin, h, wd = x.shape
    cout, cin2, k, k2 = w.shape
    assert cin == cin2 and k == k2
    if pad is None:
        pad = (k - 1) // 2
    ho = (h + 2 * pad - k) // stride + 1
    wo = (wd + 2 * pad - k) // stride + 1
    y = np.empty((n, cout, ho, wo), np.float32)
    b = None if bias is None else _f32(bias)
    lib().or_conv2d(x.ravel(), w.ravel(), _ptr_or_none(b), y.ravel(), n, cin, cout, h, wd, k,
                    stride, pad)
    return y


def matmul(a, b, batched_b: bool | None = None) -> np.ndarray:
    """Reference MatMul: a [..., M, K] . b [K, N] or [..., K, N]."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape[-2:]
    n = b.shape[-1]
    batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    if batched_b is None:
        batched_b = b.ndim > 2 and int(np.prod(b.shape[:-2])) > 1
    y = np.empty(a.shape[:-2] + (m, n), np.float32)
    lib().or_matmul(a.ravel(), b.ravel(), y.ravel(), m, n, k, batch, int(batched_b))
    return y


def gemm(a, b, c=None, trans_b: bool = False) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    y = np.empty((m, n), np.float32)
    cc = None if c is None else _f32(c)
    lib().or_gemm(a.ravel(), b.ravel(), _ptr_or_none(cc), y.ravel(), m, n, k, int(trans_b))
    return y


def linear(x, w, bias=None) -> np.ndarray:
    """torch-layout linear: x [..., K], w [N, K] -> [..., N]."""
    x, w = _f32(x), _f32(w)
    k = x.shape[-1]
    n = w.shape[0]
    m = x.size // k
    y = np.empty(x.shape[:-1] + (n,), np.float32)
    bb = None if bias is None else _f32(bias)
    lib().or_linear(x.ravel(), w.ravel(), _ptr_or_none(bb), y.ravel(), m, n, k)
    return y


def attention(q, k, v, scale: float | None = None, layout: str = "bhsd") -> np.ndarray:
    """softmax(q k^T * scale) v.  layout 'bhsd' ([B,H,S,d], fused-cross-attn.js)
    or 'bshd' ([B,S,H,d], fused-attn.js)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    if layout == "bshd":
        b, sq, h, d = q.shape
        skv = k.shape[1]
        st = lambda s: (s * h * d, d, h * d)
        qs, ks, vs = st(sq), st(skv), st(skv)
        os_ = st(sq)
    else:
        b, h, sq, d = q.shape
        skv = k.shape[2]
        st = lambda s: (h * s * d, s * d, d)
        qs, ks, vs, os_ = st(sq), st(skv), st(skv), st(sq)
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    o = np.empty_like(q)
    lib().or_attention(q.ravel(), k.ravel(), v.ravel(), o.ravel(), b, h, sq, skv, d, float(scale),
                       *qs, *ks, *vs, *os_)
    return o


def tembed(t: float, w1, b1, w2, b2) -> np.ndarray:
    w1, w2 = _f32(w1), _f32(w2)
    hid, emb = w1.shape
    y = np.empty(hid, np.float32)
    lib().or_tembed(float(t), w1.ravel(), _f32(b1), w2.ravel(), _f32(b2), y, emb, hid)
    return y


def fill_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    y = np.empty(n, np.float32)
    lib().or_fill_normal(y, n, seed, mean, std)
    return y


def splitmix_at(seed: int, j: int) -> int:
    return int(lib().or_splitmix_at(seed, j))
