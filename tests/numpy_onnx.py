"""A small numpy interpreter for the executor's Graph objects (test
infrastructure): ONNX semantics for the op types torch's opset-14 export of
the SD blocks uses, and the oracle's kernels for the ops the fusing rewrites
insert (GroupNorm[+SiLU], LayerNormalization, Gelu, FusedAttention).  Used
to check that a rewrite leaves a graph's outputs unchanged, on the CPU."""
from __future__ import annotations

import numpy as np

import oracle
from drawinstant.executor import (Graph, get_attr_float, get_attr_int, get_attr_ints,
                                  get_attr_string)

_NP = {1: np.float32, 6: np.int32, 7: np.int64, 9: np.bool_, 10: np.float16, 11: np.float64}


def _bin(f):
    return lambda n, i: f(i[0], i[1])


def _slice(n, i):
    x = i[0]
    starts, ends = list(i[1]), list(i[2])
    axes = list(i[3]) if len(i) > 3 and i[3] is not None else list(range(len(starts)))
    steps = list(i[4]) if len(i) > 4 and i[4] is not None else [1] * len(starts)
    sl = [slice(None)] * x.ndim
    for s, e, a, st in zip(starts, ends, axes, steps):
        dim = x.shape[a]
        s = int(max(min(s, dim), -dim)) if abs(s) < 2 ** 62 else (dim if s > 0 else 0)
        e = int(max(min(e, dim), -dim - 1)) if abs(e) < 2 ** 62 else (dim if e > 0 else -dim - 1)
        sl[a] = slice(s, e if e != -dim - 1 else None, int(st))
    return x[tuple(sl)]


def _reshape(n, i):
    x, shape = i[0], [int(v) for v in i[1]]
    shape = [x.shape[k] if v == 0 else v for k, v in enumerate(shape)]
    return x.reshape(shape)


def _instance_norm(n, i):
    x, g, b = i
    eps = get_attr_float(n, "epsilon", 1e-5)
    ax = tuple(range(2, x.ndim))
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=ax, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=ax, keepdims=True)
    shp = (1, -1) + (1,) * (x.ndim - 2)
    y = (x64 - mu) / np.sqrt(var + eps) * g.reshape(shp) + b.reshape(shp)
    return y.astype(np.float32)


def _conv(n, i):
    x, w = i[0], i[1]
    b = i[2] if len(i) > 2 else None
    pads = get_attr_ints(n, "pads", [0, 0, 0, 0])
    st = get_attr_ints(n, "strides", [1, 1])
    return oracle.conv2d(x, w, b, stride=st[0], pad=pads[0])


def _gemm(n, i):
    a, b = i[0].astype(np.float64), i[1].astype(np.float64)
    if get_attr_int(n, "transA", 0):
        a = a.T
    if get_attr_int(n, "transB", 0):
        b = b.T
    y = get_attr_float(n, "alpha", 1.0) * (a @ b)
    if len(i) > 2 and i[2] is not None:
        y = y + get_attr_float(n, "beta", 1.0) * i[2]
    return y.astype(np.float32)


def _softmax(n, i):
    x = i[0]
    return oracle.softmax(x.reshape(-1, x.shape[-1])).reshape(x.shape)


def _shape(n, i):
    dims = list(i[0].shape)
    perm = get_attr_ints(n, "perm", None)
    if perm:
        dims = [dims[j] for j in perm]
    r = len(dims)
    s, e = get_attr_int(n, "start", 0), get_attr_int(n, "end", r)
    s = min(max(s + r if s < 0 else s, 0), r)
    e = min(max(e + r if e < 0 else e, 0), r)
    return np.array(dims[s:e], np.int64)


def _layer_norm(n, i):
    x = i[0]
    d = x.shape[-1]
    g = i[1].reshape(-1) if len(i) > 1 and i[1] is not None else np.ones(d, np.float32)
    b = i[2].reshape(-1) if len(i) > 2 and i[2] is not None else np.zeros(d, np.float32)
    return oracle.layer_norm(x.reshape(-1, d), g, b, get_attr_float(n, "epsilon", 1e-5)) \
        .reshape(x.shape)


def _fused_attention(n, i):
    q, k, v = i[:3]
    scale = get_attr_float(n, "scale", 1.0)
    for f in i[3:5]:
        if f is not None:
            scale *= float(np.asarray(f).reshape(-1)[0])
    if get_attr_string(n, "layout", "bhsd") == "bshd":
        return oracle.attention(q, k, v, scale=scale, layout="bshd")
    if get_attr_int(n, "k_transposed", 1):
        k = np.swapaxes(k, -1, -2)
    lead = q.shape[:-2]
    h = int(np.prod(lead)) if lead else 1
    o = oracle.attention(q.reshape(1, h, *q.shape[-2:]), k.reshape(1, h, *k.shape[-2:]),
                         v.reshape(1, h, *v.shape[-2:]), scale=scale)
    return o.reshape(q.shape[:-1] + (v.shape[-1],))


def _resize_nearest(n, i):
    """Resize, mode nearest with asymmetric coordinates and floor rounding:
    out[o] = in[floor(o / scale)] on each axis."""
    assert get_attr_string(n, "mode", "nearest") == "nearest"
    x, scales = i[0], np.asarray(i[2], np.float64)
    idx = [np.minimum(np.floor(np.arange(int(np.floor(d * sc))) / sc).astype(np.int64), d - 1)
           for d, sc in zip(x.shape, scales)]
    return x[np.ix_(*idx)]


def _constant(n, i):
    t = next(a for a in n.attributes if a.name == "value").t
    return t.array().reshape(t.dims) if t.dims else t.array().reshape(())


def _constant_of_shape(n, i):
    v = next((a for a in n.attributes if a.name == "value"), None)
    fill = v.t.array().reshape(-1)[:1] if v is not None and v.t is not None else \
        np.zeros(1, np.float32)
    return np.full([int(d) for d in i[0]], fill[0], fill.dtype)


def _expand(n, i):
    """Numpy-style broadcast of x against the shape operand (ONNX Expand)."""
    shape = [int(d) for d in i[1]]
    full = np.broadcast_shapes(i[0].shape, tuple(shape))
    return np.ascontiguousarray(np.broadcast_to(i[0], full))


OPS = {
    "Add": _bin(np.add), "Sub": _bin(np.subtract), "Mul": _bin(np.multiply),
    "Div": lambda n, i: (i[0] / i[1]) if i[0].dtype.kind == "f" else
    np.trunc(i[0] / i[1]).astype(i[0].dtype),
    "Pow": _bin(np.power),
    "Sqrt": lambda n, i: np.sqrt(i[0]),
    "Sin": lambda n, i: np.sin(i[0].astype(np.float64)).astype(i[0].dtype),
    "Cos": lambda n, i: np.cos(i[0].astype(np.float64)).astype(i[0].dtype),
    "Equal": lambda n, i: np.equal(i[0], i[1]),
    "Where": lambda n, i: np.where(i[0], i[1], i[2]),
    "Expand": _expand, "ConstantOfShape": _constant_of_shape,
    "Erf": lambda n, i: oracle.unary("Erf", i[0]),
    "Sigmoid": lambda n, i: oracle.unary("Sigmoid", i[0]),
    "Silu": lambda n, i: oracle.unary("SiLU", i[0]),
    "Gelu": lambda n, i: oracle.unary("GELU" if get_attr_string(n, "approximate", "none") ==
                                      "none" else "GELU_TANH", i[0]),
    "ReduceMean": lambda n, i: i[0].astype(np.float64).mean(
        axis=tuple(get_attr_ints(n, "axes", [-1])),
        keepdims=bool(get_attr_int(n, "keepdims", 1))).astype(np.float32),
    "Transpose": lambda n, i: np.ascontiguousarray(i[0].transpose(get_attr_ints(n, "perm", None))),
    "MatMul": lambda n, i: np.matmul(i[0].astype(np.float64), i[1].astype(np.float64))
    .astype(np.float32),
    "Softmax": _softmax, "Reshape": _reshape, "Shape": _shape, "Slice": _slice,
    "Cast": lambda n, i: i[0].astype(_NP[get_attr_int(n, "to", 1)]),
    "Constant": _constant,
    "Unsqueeze": lambda n, i: np.expand_dims(i[0], tuple(
        int(a) for a in (i[1] if len(i) > 1 and i[1] is not None else
                         get_attr_ints(n, "axes", None)))),
    "Squeeze": lambda n, i: np.squeeze(i[0], tuple(
        int(a) for a in (i[1] if len(i) > 1 and i[1] is not None else
                         get_attr_ints(n, "axes", None)))),
    "Resize": lambda n, i: _resize_nearest(n, i),
    "Gather": lambda n, i: np.take(i[0], i[1], axis=get_attr_int(n, "axis", 0)),
    "Concat": lambda n, i: np.concatenate(i, axis=get_attr_int(n, "axis", 0)),
    "InstanceNormalization": _instance_norm, "Conv": _conv, "Gemm": _gemm,
    "AffineBcast": lambda n, i: (i[0] * i[1] + i[2]).astype(np.float32),
    "GroupNorm": lambda n, i: oracle.group_norm(
        i[0], i[1].reshape(-1), i[2].reshape(-1), get_attr_int(n, "num_groups", 32),
        get_attr_float(n, "epsilon", 1e-5), silu=get_attr_string(n, "activation", "") == "silu"),
    "LayerNormalization": _layer_norm, "FusedAttention": _fused_attention,
}


def run(g: Graph, feeds: dict) -> dict:
    """Evaluate ``g`` on ``feeds`` (input name -> array); returns every graph
    output."""
    env = dict(feeds)
    for name, t in g.tensors.items():
        a = t.array()
        if t.dtype == "float16":
            a = a.astype(np.float32)
        env[name] = a.reshape(t.dims) if t.dims else a.reshape(())
    for n in g.nodes:
        ins = [env[x] if x else None for x in n.inputs]
        env[n.outputs[0]] = OPS[n.op_type](n, ins)
    return {o["name"]: env[o["name"]] for o in g.outputs}
