"""Graph executor: the op-dispatch API of draw-instant's wgsl-executor.js,
driving libdrawinstant_hip.so.

Mirrors, name for name (snake_case), the reference's executor contract:

* ``Tensor`` (wgsl-executor.js:45-55): device buffer + dims + dtype; CPU-side
  metadata tensors (shape vectors, int64 timesteps, scalar constants) are
  ``CpuTensor`` objects with ``cpu_data`` and no buffer, as the reference's
  ``{isShape, cpuData, dims, dtype}`` objects.
* ``BufferPool`` (:62-94): acquire/release by 4 KiB-rounded size with
  live / peak / allocs statistics, over ``di_alloc`` / ``di_free``.
* ``OPS`` (:96-1114): ``OPS[op_type](ctx, node, inputs) -> tensor`` for the
  37 op types of the reference (plus the three ops the fusing rewrites
  insert), each GPU op one C-ABI call (shapes as scalars instead of uniform
  buffers).  Activations are fp32 NCHW, as in the reference.
* graph rewrites ``fuse_silu_pattern`` (:799-839), ``fuse_mul_add_pattern``
  (:845-898), ``fuse_group_norm_pattern`` (:905-1008), and four that map
  exported subgraphs onto the library's fused kernels, which the reference
  runs op by op: ``fuse_group_norm_silu_pattern`` (GroupNorm -> SiLU, one
  dispatch), ``fuse_layer_norm_pattern`` (the 8-9 op LayerNorm decomposition
  -> ``LayerNormalization``), ``fuse_gelu_pattern`` (Div/Erf/Add/Mul/Mul ->
  ``Gelu``) and ``fuse_attention_pattern`` (MatMul -> scale -> Softmax ->
  MatMul, with its head-split Transposes, -> ``FusedAttention``, flash
  attention without the score matrix); ``optimize_graph`` runs them all.
* ``plan_execution`` (:1157-1170), ``create_dispatchers`` (:1174-1197),
  ``infer_graph_io`` (:1205-1221), ``Executor.run`` (:1223-1466) with the
  same input-seeding, CPU promotion, consumer counting, output snapshot and
  error convention (``op @<i> <op> (<name>) failed: <msg>``).

Differences by design: the in-order HIP stream replaces the command encoder
(``run`` synchronises once at the end, as the reference's single submit);
``Conv`` accepts batch N >= 1 (the reference's kernel computes batch 0 only,
so it rejects N != 1); buffers created by CPU-to-device promotion and the
graph outputs' pool buffers are returned to the pool at the end of ``run``
(the reference never releases them, so its pool grows by a few buffers per
run).
"""
from __future__ import annotations

import ctypes
import math
import time
import weakref
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional

import numpy as np

from .device import BHSD, BSHD, F16, F32, F32W16, NCHW, Buffer, Device, call

# ---------------------------------------------------------------- logging --
LOG = {"verbose": False, "node_count": 0, "op_hist": {}, "t0": 0.0, "profile": False,
       "profile_data": None, "traffic": False, "traffic_data": None}


def set_verbose(v: bool) -> None:
    LOG["verbose"] = bool(v)


def _dlog(*a) -> None:
    if LOG["verbose"]:
        print("[hip-exec]", *a, flush=True)


# ------------------------------------------------------------ graph types --
@dataclass
class TensorProto:
    """An initializer / Constant payload: dims, ONNX dtype name, raw data."""
    dims: List[int]
    dtype: str = "float32"
    data: Any = None  # bytes-like or numpy array
    name: str = ""

    def array(self) -> np.ndarray:
        dt = {"float32": np.float32, "float16": np.float16, "int64": np.int64,
              "int32": np.int32, "bool": np.uint8, "float64": np.float64, "uint8": np.uint8,
              "int8": np.int8, "int16": np.int16, "uint16": np.uint16}[self.dtype]
        if isinstance(self.data, np.ndarray):
            return np.ascontiguousarray(self.data, dt).reshape(-1)
        return np.frombuffer(bytes(self.data or b""), dt).copy()


@dataclass
class Attr:
    name: str
    i: Optional[int] = None
    f: Optional[float] = None
    ints: Optional[List[int]] = None
    floats: Optional[List[float]] = None
    s: Optional[Any] = None
    t: Optional[TensorProto] = None
    strings: Optional[List[str]] = None


@dataclass
class Node:
    op_type: str
    name: str = ""
    inputs: List[str] = field(default_factory=list)
    outputs: List[str] = field(default_factory=list)
    attributes: List[Attr] = field(default_factory=list)
    domain: str = ""


@dataclass
class Graph:
    nodes: List[Node]
    inputs: List[dict] = field(default_factory=list)   # [{"name": ...}]
    outputs: List[dict] = field(default_factory=list)
    tensors: Dict[str, TensorProto] = field(default_factory=dict)  # initializers


# ----------------------------------------------------------------- tensors --
class Tensor:
    """Device tensor (wgsl-executor.js:45-55): fp32, byte_length = numel * 4."""

    def __init__(self, buf: Optional[Buffer], dims, dtype: str = "float32", consumers: int = 0,
                 cpu_data: Optional[np.ndarray] = None):
        self.buf = buf
        self.dims = [int(d) for d in dims]
        self.dtype = dtype
        self.consumers = consumers
        self.cpu_data = cpu_data  # CPU mirror for scalar fast paths (Pow exponent, scales)
        self.numel = int(np.prod(self.dims)) if self.dims else 1
        self.byte_length = self.numel * (2 if dtype == "float16" else 4)
        self.is_shape = False

    def __repr__(self):
        return f"Tensor(GPU{self.dims}{':f16' if self.dtype == 'float16' else ''})"


class CpuTensor:
    """CPU-only metadata tensor: ``{isShape, cpuData, dims, dtype}``."""
    buf = None

    def __init__(self, cpu_data, dims, dtype: str, is_shape: bool = True):
        self.cpu_data = np.asarray(cpu_data)
        self.dims = [int(d) for d in dims]
        self.dtype = dtype
        self.is_shape = is_shape

    @property
    def numel(self) -> int:
        return int(self.cpu_data.size)

    def __repr__(self):
        return f"CpuTensor({self.dims}:{self.dtype})"


def _is_cpu(t) -> bool:
    return t is not None and getattr(t, "buf", None) is None and getattr(t, "cpu_data", None) is not None


def _dtype_of(a: np.ndarray) -> str:
    if a.dtype == np.int64:
        return "int64"
    if a.dtype == np.int32:
        return "int32"
    if a.dtype == np.uint8 or a.dtype == np.bool_:
        return "bool"
    return "float32"


# ------------------------------------------------------------ buffer pool --
class BufferPool:
    """Allocate once, reuse (wgsl-executor.js:62-94): free lists keyed by the
    byte size rounded up to 4 KiB."""

    def __init__(self, device: Device):
        self.device = device
        self.free: Dict[int, List[Buffer]] = {}
        self.owned = weakref.WeakSet()  # pool-allocated buffers (ours to recycle)
        self.live = 0
        self.peak = 0
        self.allocs = 0
        self.live_bytes = 0  # bucket bytes handed out and not yet released
        self.peak_bytes = 0

    @staticmethod
    def key(nbytes: int) -> int:
        return int(math.ceil(nbytes / 4096)) * 4096

    def acquire(self, nbytes: int) -> Buffer:
        k = self.key(nbytes)
        lst = self.free.get(k)
        self.live += 1
        self.peak = max(self.peak, self.live)
        self.live_bytes += k
        self.peak_bytes = max(self.peak_bytes, self.live_bytes)
        if lst:
            return lst.pop()
        self.allocs += 1
        buf = self.device.create_buffer(k)
        self.owned.add(buf)
        return buf

    def release(self, buf: Buffer, _nbytes: int = 0) -> None:
        """Release by the buffer's bucket capacity (an aliased reshape's
        logical size differs from it)."""
        if buf not in self.owned:
            return
        self.free.setdefault(buf.size, []).append(buf)
        self.live -= 1
        self.live_bytes -= buf.size

    def owns(self, buf: Buffer) -> bool:
        return buf in self.owned

    def destroy(self) -> None:
        for lst in self.free.values():
            for b in lst:
                b.destroy()
        self.free.clear()


# ------------------------------------------------------------ weight cache --
class WeightCache:
    """Initializers uploaded once on first use (wgsl-unet.js:55-104): floats
    (fp16 widened to fp32) on the device, int64/int32/bool kept on the CPU as
    shape tensors; scalar floats also expose ``cpu_data``.

    ``keep_f16``: fp16 initializers of rank >= 2 (the MatMul / Gemm / Conv
    weights of an fp16 ONNX file) stay fp16 on the device, half the bytes;
    the contractions read them through DI_F32W16 (widened exactly as they
    load, so results are unchanged) and any other consumer gets an fp32 copy
    for the run."""

    def __init__(self, device: Device, tensors: Dict[str, TensorProto], keep_f16: bool = False):
        self.device = device
        self.tensors = tensors
        self.keep_f16 = keep_f16
        self.gpu: Dict[str, Any] = {}

    @property
    def device_bytes(self) -> int:
        """Bytes of the initializers uploaded so far."""
        return sum(v.byte_length for v in self.gpu.values() if isinstance(v, Tensor))

    def get(self, name: str):
        if name in self.gpu:
            return self.gpu[name]
        t = self.tensors.get(name)
        if t is None:
            raise KeyError(f"weight not found: {name}")
        a = t.array()
        if t.dtype in ("int64", "int32", "bool"):
            entry = CpuTensor(a, t.dims, t.dtype, is_shape=t.dtype != "bool")
        elif self.keep_f16 and t.dtype == "float16" and len(t.dims) >= 2:
            entry = Tensor(self.device.storage(a), t.dims, "float16")
        else:
            f = a.astype(np.float32)
            entry = Tensor(self.device.storage(f if f.size else np.zeros(1, np.float32)), t.dims,
                           cpu_data=f if f.size == 1 else None)
        self.gpu[name] = entry
        return entry

    def has(self, name: str) -> bool:
        return name in self.tensors

    def names(self, prefix: str = "") -> List[str]:
        return [k for k in self.tensors if k.startswith(prefix)]

    def destroy(self) -> None:
        for v in self.gpu.values():
            if isinstance(v, Tensor) and v.buf is not None:
                v.buf.destroy()
        self.gpu.clear()


# ------------------------------------------------------------- dispatchers --
UNARY_CODE = {"Sigmoid": 0, "Sqrt": 1, "Neg": 2, "Abs": 3, "Sin": 4, "Cos": 5, "Exp": 6, "Log": 7,
              "SiLU": 8, "GELU": 9, "Erf": 10, "GELU_TANH": 11}
BINARY_CODE = {"Add": 0, "Sub": 1, "Mul": 2, "Div": 3, "Pow": 4, "Max": 5, "Min": 6}


def _u32x4(vals) -> ctypes.Array:
    v = list(vals) + [0] * (4 - len(vals))
    return (ctypes.c_uint32 * 4)(*[int(x) for x in v])


class Dispatchers:
    """Kernel closures built once per device (createDispatchers,
    wgsl-executor.js:1174-1197); each is one C-ABI call on the device stream."""

    def __init__(self, device: Device):
        ctx = device.ctx
        self.device = device
        self.unary: Dict[str, Callable] = {}
        self.binary: Dict[str, Callable] = {}
        self.binary_bcast: Dict[str, Callable] = {}
        for op, code in UNARY_CODE.items():
            self.unary[op] = (lambda c: lambda x, y, n: call("di_unary", ctx, c, x.handle, y.handle,
                                                                  n, F32))(code)
        for op in ("Add", "Sub", "Mul", "Div", "Max", "Min"):
            code = BINARY_CODE[op]
            self.binary[op] = (lambda c: lambda a, b, y, n: call(
                "di_binary", ctx, c, a.handle, b.handle, y.handle, n, F32))(code)
            self.binary_bcast[op] = (lambda c: lambda a, b, y, rank, dims, sa, sb, n: call(
                "di_binary_bcast", ctx, c, a.handle, b.handle, y.handle, rank, _u32x4(dims),
                _u32x4(sa), _u32x4(sb), n, F32))(code)
        self.softmax = lambda x, y, inner, rows: call("di_softmax", ctx, x.handle, y.handle, inner,
                                                      rows, F32)
        self.instance_norm = lambda x, g, b, y, n, c, hw, eps: call(
            "di_instance_norm", ctx, x.handle, g.handle, b.handle, y.handle, n, c, hw, eps, F32)
        self.group_norm = lambda x, g, b, y, n, G, cpg, hw, eps, flags=0: call(
            "di_group_norm", ctx, x.handle, g.handle, b.handle, y.handle, n, G, cpg, hw, eps, flags,
            F32, NCHW)
        self.layer_norm = lambda x, g, b, y, rows, inner, eps: call(
            "di_layer_norm", ctx, x.handle, g.handle, b.handle, y.handle, rows, inner, eps, F32)
        # dt F32W16: the weight operand (b / w) is fp16-resident
        self.matmul = lambda a, b, y, M, N, K, batch, bb, dt=F32: call(
            "di_matmul", ctx, a.handle, b.handle, y.handle, M, N, K, batch, bb, dt)
        self.gemm = lambda a, b, c, y, M, N, K, tb, dt=F32: call(
            "di_gemm", ctx, a.handle, b.handle, c.handle if c is not None else 0, y.handle, M, N,
            K, tb, dt)
        self.conv_mm = lambda x, w, bias, y, n, cin, cout, h, wd, k, s, pad, flags=0, dt=F32: call(
            "di_conv2d", ctx, x.handle, w.handle, bias.handle if bias is not None else 0, 0,
            y.handle, n, cin, cout, h, wd, k, s, pad, flags, dt, NCHW)
        self.convert = lambda x, sdt, y, ddt, n: call("di_convert", ctx, x.handle, sdt, y.handle,
                                                      ddt, n)
        self.resize_nearest = lambda x, y, planes, hi, wi, ho, wo: call(
            "di_resize_nearest", ctx, x.handle, y.handle, planes, hi, wi, ho, wo, F32)
        self.reduce_mean = lambda x, y, inner, rows: call("di_reduce_mean", ctx, x.handle, y.handle,
                                                          inner, rows, F32)
        self.concat_copy = lambda x, y, si, so, off, n: call(
            "di_concat_copy", ctx, x.handle, y.handle, si, so, off, n, F32)
        self.transpose = lambda x, y, rank, dims, strides, perm, n: call(
            "di_transpose", ctx, x.handle, y.handle, rank, _u32x4(dims), _u32x4(strides),
            _u32x4(perm), n, F32)
        self.pow_scalar = lambda x, y, n, e: call("di_pow_scalar", ctx, x.handle, y.handle, n, e,
                                                  F32)
        self.slice = lambda x, y, rank, dims, strides, start, n: call(
            "di_slice", ctx, x.handle, y.handle, rank, _u32x4(dims), _u32x4(strides),
            _u32x4(start), n, F32)
        self.attention = lambda q, k, v, o, b, h, sq, skv, d, layout, scale: call(
            "di_attn_cross", ctx, q.handle, k.handle, v.handle, o.handle, b, h, sq, skv, d,
            layout, scale, F32)
        self.affine_bcast = lambda x, g, b, y, rank, dims, sx, sg, n: call(
            "di_affine_bcast", ctx, x.handle, g.handle, b.handle, y.handle, rank, _u32x4(dims),
            _u32x4(sx), _u32x4(sg), n, F32)


def create_dispatchers(device: Device) -> Dispatchers:
    return Dispatchers(device)


# ----------------------------------------------------------------- helpers --
def _attr(node: Node, name: str) -> Optional[Attr]:
    for a in node.attributes:
        if a.name == name:
            return a
    return None


def get_attr_int(node: Node, name: str, dflt):
    a = _attr(node, name)
    return a.i if a is not None and a.i is not None else dflt


def get_attr_ints(node: Node, name: str, dflt):
    a = _attr(node, name)
    return list(a.ints) if a is not None and a.ints is not None else dflt


def get_attr_float(node: Node, name: str, dflt):
    a = _attr(node, name)
    return float(a.f) if a is not None and a.f is not None else dflt


def get_attr_string(node: Node, name: str, dflt):
    a = _attr(node, name)
    if a is None or not a.s:
        return dflt
    return a.s if isinstance(a.s, str) else bytes(a.s).decode()


def row_major_strides(dims: List[int]) -> List[int]:
    s = [1] * len(dims)
    for i in range(len(dims) - 2, -1, -1):
        s[i] = s[i + 1] * dims[i + 1]
    return s


def broadcast_shape(a: List[int], b: List[int]) -> List[int]:
    n = max(len(a), len(b))
    out = [0] * n
    for i in range(n):
        aa = a[len(a) - 1 - i] if i < len(a) else 1
        bb = b[len(b) - 1 - i] if i < len(b) else 1
        if aa == bb or bb == 1:
            out[n - 1 - i] = aa
        elif aa == 1:
            out[n - 1 - i] = bb
        else:
            raise ValueError(f"cannot broadcast {a} vs {b}")
    return out


def _bcast_strides(t_dims: List[int], dims: List[int]) -> List[int]:
    """Right-aligned element strides of an operand, 0 on broadcast dims
    (wgsl-executor.js:646-657)."""
    strides = [0] * len(dims)
    st = 1
    pad = len(dims) - len(t_dims)
    for i in range(len(t_dims) - 1, -1, -1):
        od, td = dims[pad + i], t_dims[i]
        strides[pad + i] = 0 if (td == 1 and od != 1) else st
        st *= td
    return strides


def _passthrough_with_dims(x, new_dims):
    """Relabel dims; CPU tensors stay CPU when their data covers the new shape."""
    if _is_cpu(x):
        n = int(np.prod(new_dims)) if new_dims else 1
        if x.cpu_data.size == n or (not new_dims and x.cpu_data.size == 1):
            dtype = x.dtype or _dtype_of(x.cpu_data)
            is_shape = x.is_shape if x.is_shape is not None else dtype in ("int64", "int32")
            return CpuTensor(x.cpu_data, new_dims, dtype, is_shape)
    return Tensor(x.buf, new_dims, getattr(x, "dtype", "float32"))


def _trunc_div(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """BigInt division semantics: truncate toward zero."""
    q = np.abs(a) // np.abs(b)
    return np.where((a < 0) ^ (b < 0), -q, q)


def _erf_as(v: np.ndarray) -> np.ndarray:
    """Abramowitz-Stegun 7.1.26, the device erf (wgsl-executor.js:687-691)."""
    t = 1.0 / (1.0 + 0.3275911 * np.abs(v))
    y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t
               + 0.254829592) * t * np.exp(-v * v)
    return np.where(v >= 0, y, -y)


UNARY_CPU = {
    "Sigmoid": lambda v: 1.0 / (1.0 + np.exp(-v)),
    "Sqrt": lambda v: np.sqrt(np.maximum(v, 0.0)),
    "Abs": np.abs,
    "Neg": lambda v: -v,
    "Erf": _erf_as,
}

# -------------------------------------------------------------------- OPS --
OPS: Dict[str, Callable] = {}


def _op(name):
    def deco(fn):
        OPS[name] = fn
        return fn
    return deco


@_op("Identity")
def _identity(ctx, node, inputs):
    x = inputs[0]
    return _passthrough_with_dims(x, list(x.dims))


@_op("Reshape")
def _reshape(ctx, node, inputs):
    x, shape = inputs[0], inputs[1] if len(inputs) > 1 else None
    raw = [int(v) for v in shape.cpu_data.reshape(-1)] if shape is not None and _is_cpu(shape) \
        else list(x.dims)
    new = list(raw)
    xn = int(np.prod(x.dims)) if x.dims else 1
    for i in range(len(new)):
        if new[i] == 0:
            new[i] = x.dims[i]  # allowzero = 0: copy from the input
    known = int(np.prod([d for d in new if d > 0])) if any(d > 0 for d in new) else 1
    for i in range(len(new)):
        if new[i] == -1:
            new[i] = xn // known
    return _passthrough_with_dims(x, new)


@_op("Shape")
def _shape(ctx, node, inputs):
    """Dims as an int64 host tensor, with opset-15 start / end; a ``perm``
    attribute (set by fuse_attention_pattern on Shape nodes whose Transpose
    input it removed) permutes the dims first."""
    dims = list(inputs[0].dims or [])
    perm = get_attr_ints(node, "perm", None)
    if perm:
        dims = [dims[j] for j in perm]
    r = len(dims)
    start = get_attr_int(node, "start", 0)
    end = get_attr_int(node, "end", r)
    start = min(max(start + r if start < 0 else start, 0), r)
    end = min(max(end + r if end < 0 else end, 0), r)
    dims = dims[start:end] if end > start else []
    return CpuTensor(np.array(dims, np.int64), [len(dims)], "int64", True)


@_op("Unsqueeze")
def _unsqueeze(ctx, node, inputs):
    x = inputs[0]
    axes = inputs[1] if len(inputs) > 1 else None
    ax = [int(v) for v in axes.cpu_data.reshape(-1)] if axes is not None and _is_cpu(axes) \
        else get_attr_ints(node, "axes", [0])
    dims = list(x.dims) if x.dims is not None else [x.cpu_data.size]
    for a in ax:
        dims.insert(len(dims) + 1 + a if a < 0 else a, 1)
    if _is_cpu(x):
        return CpuTensor(x.cpu_data, dims, x.dtype or "int64", x.is_shape is not False)
    return Tensor(x.buf, dims)


@_op("Squeeze")
def _squeeze(ctx, node, inputs):
    x = inputs[0]
    axes = inputs[1] if len(inputs) > 1 else None
    ax = [int(v) for v in axes.cpu_data.reshape(-1)] if axes is not None and _is_cpu(axes) \
        else get_attr_ints(node, "axes", None)
    dims = list(x.dims)
    if ax:
        rm = {a + len(dims) if a < 0 else a for a in ax}
    else:
        rm = {i for i, d in enumerate(dims) if d == 1}
    return _passthrough_with_dims(x, [d for i, d in enumerate(dims) if i not in rm])


@_op("Constant")
def _constant(ctx, node, inputs):
    a_t, a_ints, a_int = _attr(node, "value"), _attr(node, "value_ints"), _attr(node, "value_int")
    a_floats, a_float = _attr(node, "value_floats"), _attr(node, "value_float")
    if a_t is not None and a_t.t is not None:
        t = a_t.t
        arr = t.array()
        if t.dtype in ("int64", "int32"):
            return CpuTensor(arr, t.dims, t.dtype, True)
        if t.dtype in ("float32", "float16", "float64"):  # every float lives as fp32
            f = arr.astype(np.float32)
            buf = ctx.pool.acquire(max(f.nbytes, 4))
            ctx.device.upload(buf, f)
            return Tensor(buf, list(t.dims), cpu_data=f)
        return CpuTensor(arr, t.dims, t.dtype, True)
    if a_ints is not None and a_ints.ints is not None:
        return CpuTensor(np.array(a_ints.ints, np.int64), [len(a_ints.ints)], "int64", True)
    if a_int is not None and a_int.i is not None:
        return CpuTensor(np.array([a_int.i], np.int64), [], "int64", True)

    def upload(vals, dims):
        f = np.asarray(vals, np.float32).reshape(-1)
        buf = ctx.pool.acquire(max(f.nbytes, 4))
        ctx.device.upload(buf, f)
        return Tensor(buf, dims, cpu_data=f)
    if a_floats is not None and a_floats.floats is not None:
        return upload(a_floats.floats, [len(a_floats.floats)])
    if a_float is not None and a_float.f is not None:
        return upload([a_float.f], [])
    raise ValueError(f"Constant {node.name}: no recognised value attribute")


@_op("ConstantOfShape")
def _constant_of_shape(ctx, node, inputs):
    dims = [int(v) for v in inputs[0].cpu_data.reshape(-1)]
    numel = int(np.prod(dims)) if dims else 1
    v = _attr(node, "value")
    fill, vdt = 0.0, None
    if v is not None and v.t is not None and v.t.data is not None and len(v.t.array()):
        vdt = v.t.dtype
        fill = v.t.array()[0]
    if vdt in ("int64", "int32"):
        dt = np.int64 if vdt == "int64" else np.int32
        return CpuTensor(np.full(max(numel, 0), fill, dt), dims, vdt, True)
    buf = ctx.pool.acquire(max(numel * 4, 4))
    ctx.device.upload(buf, np.full(max(numel, 1), float(fill), np.float32))
    return Tensor(buf, dims)


@_op("Cast")
def _cast(ctx, node, inputs):
    x = inputs[0]
    to = get_attr_int(node, "to", 1)
    if _is_cpu(x):
        d = x.cpu_data
        if to == 7 and d.dtype != np.int64:
            return CpuTensor(np.trunc(d.astype(np.float64)).astype(np.int64), x.dims, "int64",
                             x.is_shape is not False)
        if to == 6 and d.dtype != np.int32:
            return CpuTensor(np.trunc(d.astype(np.float64)).astype(np.int32), x.dims, "int32",
                             x.is_shape is not False)
        if to == 1 and d.dtype != np.float32:
            return CpuTensor(d.astype(np.float32), x.dims, "float32", False)
        return CpuTensor(d, x.dims, x.dtype, x.is_shape is not False)
    return Tensor(x.buf, list(x.dims))  # fp16 <-> fp32 on device: stored fp32 either way


@_op("Slice")
def _slice(ctx, node, inputs):
    x = inputs[0]
    get = lambda i: inputs[i] if len(inputs) > i and inputs[i] is not None else None
    starts_t, ends_t, axes_t, steps_t = get(1), get(2), get(3), get(4)
    vals = lambda t: [int(v) for v in t.cpu_data.reshape(-1)] if t is not None and \
        getattr(t, "cpu_data", None) is not None else None
    if _is_cpu(x):
        data = x.cpu_data.reshape(-1)
        n = data.size
        s = (vals(starts_t) or [0])[0]
        e = (vals(ends_t) or [n])[0]
        st = (vals(steps_t) or [1])[0] or 1
        if s < 0:
            s += n
        if e < 0:
            e += n
        s, e = max(0, min(n, s)), max(0, min(n, e))
        out = np.array([data[i] for i in range(s, e, st)] if st > 0 else
                       [data[i] for i in range(s, e, st)], data.dtype)
        return CpuTensor(out, [out.size], x.dtype or "int64", x.is_shape is not False)
    rank = len(x.dims)
    if rank > 4:
        raise ValueError(f"Slice: rank {rank} > 4 not supported")
    s_arr, e_arr = vals(starts_t) or [], vals(ends_t) or []
    a_arr = vals(axes_t) or list(range(len(s_arr)))
    step_arr = vals(steps_t) or [1] * len(s_arr)
    if any(v != 1 for v in step_arr):
        raise ValueError("Slice: step != 1 not supported")
    out_dim, start = list(x.dims), [0] * rank
    for i, ax in enumerate(a_arr):
        ax = ax + rank if ax < 0 else ax
        ss, ee = s_arr[i], e_arr[i]
        if ss < 0:
            ss += x.dims[ax]
        if ee < 0:
            ee += x.dims[ax]
        ss = max(0, min(x.dims[ax], ss))
        ee = max(0, min(x.dims[ax], ee))
        start[ax] = ss
        out_dim[ax] = max(0, ee - ss)
    numel = int(np.prod(out_dim))
    out = ctx.pool.acquire(max(numel * 4, 4))
    if numel:
        ctx.dispatchers.slice(x.buf, out, rank, out_dim, row_major_strides(x.dims), start, numel)
    return Tensor(out, out_dim)


@_op("Gather")
def _gather(ctx, node, inputs):
    data, indices = inputs[0], inputs[1]
    if getattr(data, "is_shape", False) and _is_cpu(data):
        d = data.cpu_data.reshape(-1)
        n = d.size
        idx = [int(i) + n if int(i) < 0 else int(i) for i in
               (indices.cpu_data.reshape(-1) if indices is not None else [0])]
        out = np.array([d[i] if 0 <= i < n else 0 for i in idx], np.int64)
        return CpuTensor(out, list(indices.dims) if indices is not None else [], "int64", True)
    raise ValueError(f"Gather {node.name}: GPU-tensor path not implemented")


@_op("Transpose")
def _transpose(ctx, node, inputs):
    x = inputs[0]
    dims = list(x.dims or [])
    perm = get_attr_ints(node, "perm", list(range(len(dims) - 1, -1, -1)))
    new = [dims[i] for i in perm]
    if _is_cpu(x):
        return _passthrough_with_dims(x, new)
    if len(dims) > 4:
        raise ValueError(f"Transpose: rank {len(dims)} > 4 not supported")
    rank = len(dims)
    numel = int(np.prod(new))
    out = ctx.pool.acquire(max(numel * 4, 4))
    ctx.dispatchers.transpose(x.buf, out, rank, new + [1] * (4 - rank),
                              row_major_strides(dims) + [0] * (4 - rank), perm + [0] * (4 - rank),
                              numel)
    return Tensor(out, new)


@_op("Concat")
def _concat(ctx, node, inputs):
    axis = get_attr_int(node, "axis", 0)
    ref = next((t for t in inputs if t is not None and (t.dims is not None)), None)
    rank = len(ref.dims) if ref is not None else 1
    if axis < 0:
        axis += rank
    all_cpu = all(_is_cpu(t) for t in inputs)
    if not all_cpu and any(_is_cpu(t) for t in inputs):
        inputs = [ctx.promote(t) if _is_cpu(t) else t for t in inputs]
    if all_cpu:
        first = inputs[0]
        big = any(t.cpu_data.dtype == np.int64 for t in inputs)
        out = np.concatenate([t.cpu_data.reshape(-1) for t in inputs]).astype(
            np.int64 if big else np.float32)
        return CpuTensor(out, [out.size], first.dtype or "int64", first.is_shape is not False)
    dims = list(inputs[0].dims)
    dims[axis] = sum(t.dims[axis] for t in inputs)
    numel = int(np.prod(dims))
    out = ctx.pool.acquire(max(numel * 4, 4))
    stripe_out = int(np.prod(dims[axis:]))
    off = 0
    for t in inputs:
        stripe_in = int(np.prod(t.dims[axis:]))
        if t.numel:
            ctx.dispatchers.concat_copy(t.buf, out, stripe_in, stripe_out, off, t.numel)
        off += stripe_in
    return Tensor(out, dims)


@_op("ReduceMean")
def _reduce_mean(ctx, node, inputs):
    x = inputs[0]
    axes = get_attr_ints(node, "axes", [len(x.dims) - 1])
    keep = get_attr_int(node, "keepdims", 1)
    if len(axes) != 1 or (axes[0] != -1 and axes[0] != len(x.dims) - 1):
        raise ValueError(f"ReduceMean: only last-dim reduction supported, got axes {axes}")
    inner = x.dims[-1]
    rows = x.numel // inner
    out = ctx.pool.acquire(rows * 4)
    ctx.dispatchers.reduce_mean(x.buf, out, inner, rows)
    return Tensor(out, x.dims[:-1] + [1] if keep else x.dims[:-1])


def _unary_gpu(op):
    def fn(ctx, node, inputs):
        x = inputs[0]
        if _is_cpu(x) and op in UNARY_CPU:
            out = UNARY_CPU[op](x.cpu_data.astype(np.float64)).astype(np.float32)
            return CpuTensor(out, list(x.dims or []), "float32", True)
        out = ctx.pool.acquire(x.byte_length)
        ctx.dispatchers.unary["SiLU" if op == "Silu" else op](x.buf, out, x.numel)
        return Tensor(out, list(x.dims))
    return fn


for _u in ("Sigmoid", "Sqrt", "Erf", "Abs", "Neg", "Sin", "Cos", "Silu"):
    OPS[_u] = _unary_gpu(_u)


@_op("Pow")
def _pow(ctx, node, inputs):
    a, b = inputs[0], inputs[1]
    exponent = None
    if b is not None and getattr(b, "cpu_data", None) is not None and b.cpu_data.size >= 1 and \
            (b.cpu_data.size == 1 or all(d == 1 for d in (b.dims or []))):
        exponent = float(b.cpu_data.reshape(-1)[0])
    if exponent is None:
        raise ValueError(f"Pow: non-scalar exponent not yet supported (b.dims={getattr(b, 'dims', None)})")
    ag = a if a.buf is not None else ctx.promote(a)
    out = ctx.pool.acquire(ag.numel * 4)
    ctx.dispatchers.pow_scalar(ag.buf, out, ag.numel, exponent)
    return Tensor(out, list(ag.dims))


@_op("Expand")
def _expand(ctx, node, inputs):
    x, shape = inputs[0], inputs[1]
    new = [int(v) for v in shape.cpu_data.reshape(-1)] if shape is not None else list(x.dims)
    if int(np.prod(new)) != int(np.prod(x.dims or [1])):
        raise ValueError(f"Expand {node.name}: real broadcast {x.dims} -> {new} not implemented")
    return _passthrough_with_dims(x, new)


@_op("Equal")
def _equal(ctx, node, inputs):
    a, b = inputs
    if _is_cpu(a) and _is_cpu(b):
        av, bv = a.cpu_data.reshape(-1), b.cpu_data.reshape(-1)
        out = (av.astype(np.float64) == bv.astype(np.float64)).astype(np.uint8)
        dims = (a.dims if av.size >= bv.size else b.dims) or [out.size]
        return CpuTensor(out, list(dims), "bool", True)
    raise ValueError(f"Equal {node.name}: GPU path not implemented")


@_op("Where")
def _where(ctx, node, inputs):
    c, a, b = inputs
    if _is_cpu(c) and _is_cpu(a) and _is_cpu(b):
        cv, av, bv = (t.cpu_data.reshape(-1) for t in (c, a, b))
        n = max(cv.size, av.size, bv.size)
        dt = av.dtype if av.size >= bv.size else bv.dtype
        pick = lambda v, i: v[0] if v.size == 1 else v[i]
        out = np.array([pick(av, i) if pick(cv, i) else pick(bv, i) for i in range(n)], dt)
        return CpuTensor(out, [n], a.dtype or b.dtype or "int64",
                         a.is_shape is not False or b.is_shape is not False)
    raise ValueError(f"Where {node.name}: GPU path not implemented")


def _host_small(t) -> bool:
    """A tensor whose values are also on the host and few (scalars, shape
    vectors): binary ops between two of them run on the host."""
    d = getattr(t, "cpu_data", None) if t is not None else None
    return d is not None and np.asarray(d).size <= 16 and \
        int(np.prod(t.dims or [1])) == np.asarray(d).size


def _binary(op):
    def fn(ctx, node, inputs):
        a, b = inputs
        if (_is_cpu(a) and _is_cpu(b)) or (_host_small(a) and _host_small(b)):
            dims = broadcast_shape(list(a.dims), list(b.dims))
            big = a.cpu_data.dtype == np.int64 or b.cpu_data.dtype == np.int64
            av = a.cpu_data.reshape(a.dims) if a.dims else a.cpu_data.reshape(())
            bv = b.cpu_data.reshape(b.dims) if b.dims else b.cpu_data.reshape(())
            if big:
                av, bv = av.astype(np.int64), bv.astype(np.int64)
                out = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply,
                       "Div": _trunc_div}[op](av, bv)
            else:
                av, bv = av.astype(np.float32), bv.astype(np.float32)
                out = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply,
                       "Div": np.divide}[op](av, bv).astype(np.float32)
            out = np.broadcast_to(out, dims).reshape(-1).copy()
            return CpuTensor(out, dims, "int64" if big else "float32",
                             bool(a.is_shape or b.is_shape))
        if _is_cpu(a):
            a = ctx.promote(a)
        if _is_cpu(b):
            b = ctx.promote(b)
        dims = broadcast_shape(list(a.dims), list(b.dims))
        numel = int(np.prod(dims)) if dims else 1
        out = ctx.pool.acquire(max(numel * 4, 4))
        if list(a.dims) == dims and list(b.dims) == dims:
            ctx.dispatchers.binary[op](a.buf, b.buf, out, numel)
        else:
            if len(dims) > 4:
                raise ValueError(f"{op} broadcast: rank {len(dims)} > 4 not supported")
            ctx.dispatchers.binary_bcast[op](a.buf, b.buf, out, len(dims), dims,
                                             _bcast_strides(list(a.dims), dims),
                                             _bcast_strides(list(b.dims), dims), numel)
        return Tensor(out, dims)
    return fn


for _b in ("Add", "Sub", "Mul", "Div"):
    OPS[_b] = _binary(_b)


@_op("GroupNorm")
def _group_norm(ctx, node, inputs):
    x, g, b = (t if t is None or t.buf is not None else ctx.promote(t) for t in inputs[:3])
    if not x.dims or len(x.dims) < 2:
        raise ValueError(f"GroupNorm {node.name}: expected rank>=2 input, got dims={x.dims}")
    N, C = x.dims[0], x.dims[1]
    HW = int(np.prod(x.dims[2:])) if len(x.dims) > 2 else 1
    G = int(get_attr_int(node, "num_groups", 32))
    if C % G:
        raise ValueError(f"GroupNorm: C={C} not divisible by G={G}")
    eps = get_attr_float(node, "epsilon", 1e-5)
    act = get_attr_string(node, "activation", "")
    if act not in ("", "silu"):
        raise ValueError(f"GroupNorm {node.name}: activation {act!r}")
    out = ctx.pool.acquire(N * C * HW * 4)
    ctx.dispatchers.group_norm(x.buf, g.buf, b.buf, out, N, G, C // G, HW, eps,
                               1 if act == "silu" else 0)
    return Tensor(out, list(x.dims))


@_op("AffineBcast")
def _affine_bcast(ctx, node, inputs):
    x, g, b = (t if t.buf is not None else ctx.promote(t) for t in inputs[:3])
    dims = list(x.dims)
    if len(dims) > 4:
        raise ValueError(f"AffineBcast: rank {len(dims)} > 4")
    numel = int(np.prod(dims))
    out = ctx.pool.acquire(numel * 4)
    ctx.dispatchers.affine_bcast(x.buf, g.buf, b.buf, out, len(dims), dims,
                                 _bcast_strides(dims, dims), _bcast_strides(list(g.dims), dims),
                                 numel)
    return Tensor(out, dims)


@_op("InstanceNormalization")
def _instance_norm(ctx, node, inputs):
    """eps 1e-5 regardless of the node attribute, as the reference kernel
    hard-codes it (wgsl-executor.js:1020; GroupNorm carries the real eps)."""
    x, g, b = inputs[:3]
    if len(x.dims) == 4:
        N, C, HW = x.dims[0], x.dims[1], x.dims[2] * x.dims[3]
    elif len(x.dims) == 3:
        N, C, HW = x.dims
    else:
        raise ValueError(f"InstanceNorm needs 3D or 4D input, got {len(x.dims)}D")
    g = g if g.buf is not None else ctx.promote(g)
    b = b if b.buf is not None else ctx.promote(b)
    out = ctx.pool.acquire(x.byte_length)
    ctx.dispatchers.instance_norm(x.buf, g.buf, b.buf, out, N, C, HW, 1e-5)
    return Tensor(out, list(x.dims))


@_op("Softmax")
def _softmax(ctx, node, inputs):
    x = inputs[0]
    axis = get_attr_int(node, "axis", -1)
    ax = axis + len(x.dims) if axis < 0 else axis
    if ax != len(x.dims) - 1:
        raise ValueError(f"Softmax: only last-axis supported, got axis={axis} dims={x.dims}")
    inner = x.dims[ax]
    out = ctx.pool.acquire(x.byte_length)
    ctx.dispatchers.softmax(x.buf, out, inner, x.numel // inner)
    return Tensor(out, list(x.dims))


@_op("MatMul")
def _matmul(ctx, node, inputs):
    a, b = inputs
    M, K, N = a.dims[-2], a.dims[-1], b.dims[-1]
    batch = int(np.prod(a.dims[:-2])) if len(a.dims) > 2 else 1
    b_batch = int(np.prod(b.dims[:-2])) if len(b.dims) > 2 else 1
    if b_batch != 1 and b_batch != batch:
        raise ValueError(f"MatMul: batch mismatch a={a.dims} b={b.dims}")
    if batch == 1 and b_batch > 1:
        raise ValueError("MatMul: batched B with unbatched A not supported")
    out = ctx.pool.acquire(batch * M * N * 4)
    ctx.dispatchers.matmul(a.buf, b.buf, out, M, N, K, batch, 1 if b_batch > 1 else 0,
                           F32W16 if b.dtype == "float16" else F32)
    return Tensor(out, list(a.dims[:-2]) + [M, N])


@_op("Gemm")
def _gemm(ctx, node, inputs):
    a, b = inputs[0], inputs[1]
    c = inputs[2] if len(inputs) > 2 else None
    tb = get_attr_int(node, "transB", 0)
    M, K = a.dims
    N = b.dims[0] if tb else b.dims[1]
    out = ctx.pool.acquire(M * N * 4)
    ctx.dispatchers.gemm(a.buf, b.buf, c.buf if c is not None else None, out, M, N, K, tb,
                         F32W16 if b.dtype == "float16" else F32)
    return Tensor(out, [M, N])


@_op("Conv")
def _conv(ctx, node, inputs):
    x, w = inputs[0], inputs[1]
    bias = inputs[2] if len(inputs) > 2 else None
    ks = get_attr_ints(node, "kernel_shape", [3, 3])
    if ks[0] != ks[1]:
        raise ValueError(f"Conv: non-square kernel {ks} not supported")
    K = ks[0]
    st = get_attr_ints(node, "strides", [1, 1])
    if st[0] != st[1]:
        raise ValueError(f"Conv: non-square stride {st} not supported")
    S = st[0]
    pads = get_attr_ints(node, "pads", [(K - 1) >> 1] * 4)
    if not (pads[0] == pads[1] == pads[2] == pads[3]):
        raise ValueError(f"Conv: asymmetric pads {pads} not supported")
    P = pads[0]
    N, Cin, H, W = x.dims
    Cout = w.dims[0]
    Ho, Wo = (H + 2 * P - K) // S + 1, (W + 2 * P - K) // S + 1
    out = ctx.pool.acquire(N * Cout * Ho * Wo * 4)
    ctx.dispatchers.conv_mm(x.buf, w.buf, bias.buf if bias is not None else None, out, N, Cin,
                            Cout, H, W, K, S, P, CONV_F16_COMPUTE if ctx.conv_f16 else 0,
                            F32W16 if w.dtype == "float16" else F32)
    return Tensor(out, [N, Cout, Ho, Wo])


@_op("Resize")
def _resize(ctx, node, inputs):
    x = inputs[0]
    if get_attr_string(node, "mode", "nearest") != "nearest":
        raise ValueError(f"Resize mode {get_attr_string(node, 'mode', '')} not yet supported")
    sc = inputs[2] if len(inputs) > 2 else None
    scales = sc.cpu_data.reshape(-1) if sc is not None and getattr(sc, "cpu_data", None) is not None \
        else None
    sh = float(scales[2]) if scales is not None else 2.0
    sw = float(scales[3]) if scales is not None else 2.0
    N, C, H, W = x.dims
    Ho, Wo = int(round(H * sh)), int(round(W * sw))
    out = ctx.pool.acquire(N * C * Ho * Wo * 4)
    ctx.dispatchers.resize_nearest(x.buf, out, N * C, H, W, Ho, Wo)
    return Tensor(out, [N, C, Ho, Wo])


# --------------------------------------------- ops inserted by the rewrites --
def _on_device(ctx, t):
    return t if t is None or getattr(t, "buf", None) is not None else ctx.promote(t)


@_op("Gelu")
def _gelu(ctx, node, inputs):
    """ONNX Gelu (inserted by fuse_gelu_pattern): the erf form through the
    same Abramowitz-Stegun erf as OPS.Erf, or approximate="tanh"."""
    x = _on_device(ctx, inputs[0])
    approx = get_attr_string(node, "approximate", "none")
    if approx not in ("none", "tanh"):
        raise ValueError(f"Gelu: approximate={approx!r}")
    out = ctx.pool.acquire(x.byte_length)
    ctx.dispatchers.unary["GELU" if approx == "none" else "GELU_TANH"](x.buf, out, x.numel)
    return Tensor(out, list(x.dims))


@_op("LayerNormalization")
def _layer_norm(ctx, node, inputs):
    """ONNX LayerNormalization over the last axis (inserted by
    fuse_layer_norm_pattern): one di_layer_norm dispatch (layerNorm,
    wgsl-ops.js:772-812).  Absent gamma / beta mean 1 / 0."""
    x = _on_device(ctx, inputs[0])
    g = _on_device(ctx, inputs[1]) if len(inputs) > 1 else None
    b = _on_device(ctx, inputs[2]) if len(inputs) > 2 else None
    rank = len(x.dims)
    axis = get_attr_int(node, "axis", -1)
    if rank < 1 or (axis + rank if axis < 0 else axis) != rank - 1:
        raise ValueError(f"LayerNormalization: only the last axis is supported, got axis={axis} "
                         f"dims={x.dims}")
    inner = x.dims[-1]
    if g is None:
        g = ctx.promote(CpuTensor(np.ones(inner, np.float32), [inner], "float32", False))
    if b is None:
        b = ctx.promote(CpuTensor(np.zeros(inner, np.float32), [inner], "float32", False))
    if g.numel != inner or b.numel != inner:
        raise ValueError(f"LayerNormalization: gamma {g.dims} / beta {b.dims} do not match the "
                         f"normalised dim {inner}")
    out = ctx.pool.acquire(x.byte_length)
    ctx.dispatchers.layer_norm(x.buf, g.buf, b.buf, out, x.numel // inner, inner,
                               get_attr_float(node, "epsilon", 1e-5))
    return Tensor(out, list(x.dims))


ATTN_HEAD_DIM = 64  # the flash kernel's head dim


def _host_scalar(t) -> Optional[float]:
    """The value of a one-element tensor known on the host, else None."""
    d = getattr(t, "cpu_data", None) if t is not None else None
    if d is None or np.asarray(d).size != 1:
        return None
    return float(np.asarray(d, np.float64).reshape(-1)[0])


def _attention_unfused(ctx, q, k, v, scale, k_transposed, axis, q_fac=None, k_fac=None):
    """The chain the rewrite replaced, op by op: [Q * q_fac], MatMul(Q, K^T
    [* k_fac]) -> * scale -> Softmax -> MatMul(., V)."""
    tmp = []
    if q_fac is not None:
        q = OPS["Mul"](ctx, Node("Mul"), [q, q_fac])
        tmp.append(q)
    if not k_transposed:
        perm = list(range(len(k.dims)))
        perm[-2], perm[-1] = perm[-1], perm[-2]
        k = OPS["Transpose"](ctx, Node("Transpose", "", [], [], [Attr("perm", ints=perm)]), [k])
        tmp.append(k)
    if k_fac is not None:
        k = OPS["Mul"](ctx, Node("Mul"), [k, k_fac])
        tmp.append(k)
    s = OPS["MatMul"](ctx, Node("MatMul"), [q, k])
    tmp.append(s)
    if scale != 1.0:
        s = OPS["Mul"](ctx, Node("Mul"), [s, CpuTensor(np.array([scale], np.float32), [1],
                                                          "float32", False)])
        tmp.append(s)
    p = OPS["Softmax"](ctx, Node("Softmax", "", [], [], [Attr("axis", i=axis)]), [s])
    tmp.append(p)
    o = OPS["MatMul"](ctx, Node("MatMul"), [p, v])
    for t in tmp:  # the stream is in order: later work may reuse these at once
        ctx.pool.release(t.buf)
    return o


@_op("FusedAttention")
def _fused_attention(ctx, node, inputs):
    """softmax(Q K^T * scale) V (inserted by fuse_attention_pattern) through
    di_attn_cross (WGSL_FUSED_ATTN fused-attn.js:199-307, WGSL_FUSED
    fused-cross-attn.js:112-173).  layout "bhsd": Q [.., Sq, 64], K
    [.., Skv, 64] (K^T [.., 64, Skv] with k_transposed), V [.., Skv, 64] with
    equal leading dims, which run as heads; layout "bshd": Q [B, Sq, H, 64],
    K / V [B, Skv, H, 64].  Optional inputs 3 / 4 are factors on Q and on
    K^T, folded into the scale when they are host scalars.  Other shapes or
    factors run the unfused chain."""
    q, k, v = (_on_device(ctx, t) for t in inputs[:3])
    q_fac = inputs[3] if len(inputs) > 3 and inputs[3] is not None else None
    k_fac = inputs[4] if len(inputs) > 4 and inputs[4] is not None else None
    scale = get_attr_float(node, "scale", 1.0)
    kt = get_attr_int(node, "k_transposed", 1)
    axis = get_attr_int(node, "softmax_axis", -1)
    facs_ok = True
    for f in (q_fac, k_fac):
        if f is not None:
            hv = _host_scalar(f)
            facs_ok = facs_ok and hv is not None and hv > 0
            scale *= hv if hv is not None else 1.0
    if not facs_ok:
        scale = get_attr_float(node, "scale", 1.0)
    rank = len(q.dims)
    last_axis = (axis + rank if axis < 0 else axis) == rank - 1
    d = q.dims[-1] if rank else 0
    if get_attr_string(node, "layout", "bhsd") == "bshd":
        ok = facs_ok and kt == 0 and rank == 4 and len(k.dims) == 4 and len(v.dims) == 4 and \
            last_axis and q.dims[0] == k.dims[0] == v.dims[0] and \
            q.dims[2] == k.dims[2] == v.dims[2] and k.dims[1] == v.dims[1] and \
            d == k.dims[3] == v.dims[3] == ATTN_HEAD_DIM and q.dims[1] > 0 and k.dims[1] > 0
        if not ok:
            heads = Node("Transpose", "", [], [], [Attr("perm", ints=[0, 2, 1, 3])])
            qh, kh, vh = (OPS["Transpose"](ctx, heads, [t]) for t in (q, k, v))
            oh = _attention_unfused(ctx, qh, kh, vh, scale, kt, axis,
                                    None if facs_ok else q_fac, None if facs_ok else k_fac)
            out = OPS["Transpose"](ctx, heads, [oh])
            for t in (qh, kh, vh, oh):
                ctx.pool.release(t.buf)
            return out
        B, Sq, H, _ = q.dims
        out = ctx.pool.acquire(q.numel * 4)
        ctx.dispatchers.attention(q.buf, k.buf, v.buf, out, B, H, Sq, k.dims[1], d, BSHD, scale)
        return Tensor(out, list(q.dims))
    ok = facs_ok and rank >= 2 and len(k.dims) == rank and len(v.dims) == rank and \
        q.dims[:-2] == k.dims[:-2] == v.dims[:-2] and last_axis
    if ok:
        Skv = k.dims[-1] if kt else k.dims[-2]
        ok = d == ATTN_HEAD_DIM and (k.dims[-2] if kt else k.dims[-1]) == d and \
            v.dims[-2] == Skv and v.dims[-1] == ATTN_HEAD_DIM and q.dims[-2] > 0 and Skv > 0
    if not ok:
        return _attention_unfused(ctx, q, k, v, scale, kt, axis, None if facs_ok else q_fac,
                                  None if facs_ok else k_fac)
    heads = int(np.prod(q.dims[:-2])) if rank > 2 else 1
    Sq = q.dims[-2]
    k_buf, tmp = k.buf, None
    if kt:
        tmp = ctx.pool.acquire(heads * Skv * d * 4)
        ctx.dispatchers.transpose(k.buf, tmp, 3, [heads, Skv, d, 1], [d * Skv, Skv, 1, 0],
                                  [0, 2, 1, 0], heads * Skv * d)
        k_buf = tmp
    out = ctx.pool.acquire(heads * Sq * d * 4)
    ctx.dispatchers.attention(q.buf, k_buf, v.buf, out, 1, heads, Sq, Skv, d, BHSD, scale)
    if tmp is not None:
        ctx.pool.release(tmp)
    return Tensor(out, list(q.dims))


# ---------------------------------------------------------- graph rewrites --
def _consumers_and_producers(graph: Graph):
    consumers: Dict[str, int] = {}
    for n in graph.nodes:
        for i in n.inputs:
            if i:
                consumers[i] = consumers.get(i, 0) + 1
    for o in graph.outputs or []:
        consumers[o["name"]] = consumers.get(o["name"], 0) + 1
    producer = {}
    for idx, n in enumerate(graph.nodes):
        for o in n.outputs:
            producer[o] = idx
    return consumers, producer


def fuse_silu_pattern(graph: Graph) -> dict:
    """Sigmoid(X) -> Mul(X, sig) => Silu(X) when the Sigmoid output has the
    Mul as its only consumer (wgsl-executor.js:799-839)."""
    nodes = graph.nodes
    consumers, producer = _consumers_and_producers(graph)
    drop, fused = set(), 0
    for i, mul in enumerate(nodes):
        if mul.op_type != "Mul":
            continue
        a, b = (mul.inputs + [None, None])[:2]

        def try_fuse(sig_out, other):
            nonlocal fused
            if not sig_out or not other or consumers.get(sig_out, 0) != 1:
                return False
            pi = producer.get(sig_out)
            if pi is None:
                return False
            sig = nodes[pi]
            if sig.op_type != "Sigmoid" or sig.inputs[0] != other:
                return False
            nodes[i] = Node("Silu", (mul.name or "") + "_fused", [other], list(mul.outputs), [])
            drop.add(pi)
            fused += 1
            return True
        if not try_fuse(a, b):
            try_fuse(b, a)
    if fused:
        graph.nodes = [n for k, n in enumerate(nodes) if k not in drop]
    return {"fused": fused}


def fuse_mul_add_pattern(graph: Graph, tensor_shapes: Optional[dict] = None) -> dict:
    """Mul(X, gamma) -> Add(., beta) => AffineBcast(X, gamma, beta) when gamma
    and beta have identical shapes and the Mul output has one consumer
    (wgsl-executor.js:845-898)."""
    nodes = graph.nodes
    consumers, producer = _consumers_and_producers(graph)
    drop, fused = set(), 0

    def shape_of(name):
        if tensor_shapes and name in tensor_shapes:
            return list(tensor_shapes[name])
        t = graph.tensors.get(name) if graph.tensors else None
        return list(t.dims) if t is not None else None

    for i, add in enumerate(nodes):
        if add.op_type != "Add":
            continue
        a, b = (add.inputs + [None, None])[:2]

        def try_fuse(mul_out, beta):
            nonlocal fused
            if consumers.get(mul_out, 0) != 1:
                return False
            pi = producer.get(mul_out)
            if pi is None or nodes[pi].op_type != "Mul":
                return False
            mul = nodes[pi]
            ma, mb = mul.inputs[:2]
            sa, sb, sbeta = shape_of(ma), shape_of(mb), shape_of(beta)
            if not sbeta:
                return False
            if sa is not None and sa == sbeta:
                x, gamma = mb, ma
            elif sb is not None and sb == sbeta:
                x, gamma = ma, mb
            else:
                return False
            nodes[i] = Node("AffineBcast", (mul.name or "") + "_affinefused", [x, gamma, beta],
                            list(add.outputs), [])
            drop.add(pi)
            fused += 1
            return True
        if not try_fuse(a, b):
            try_fuse(b, a)
    if fused:
        graph.nodes = [n for k, n in enumerate(nodes) if k not in drop]
    return {"fused": fused}


def _uniform_value(t: TensorProto):
    if t.dtype not in ("float32", "float16", "float64") or t.data is None:
        return None
    f = t.array().astype(np.float32)
    if f.size == 0:
        return None
    return float(f[0]) if np.all(f == f[0]) else None


def fuse_group_norm_pattern(graph: Graph) -> dict:
    """Reshape(X,[N,G,-1]) -> InstanceNorm(., ones, zeros) -> Reshape(., shape)
    -> AffineBcast(., gamma, beta) => GroupNorm(X, gamma, beta)
    (wgsl-executor.js:905-1008).  Scale/bias constants resolve from Constant
    nodes or initializers; G is read from a Constant-node reshape shape (index
    1), default 32, as in the reference.  Run after fuse_mul_add_pattern."""
    nodes = graph.nodes
    consumers, producer = _consumers_and_producers(graph)

    def const_val(name):
        init = graph.tensors.get(name) if graph.tensors else None
        if init is not None and init.data is not None:
            return _uniform_value(init)
        pi = producer.get(name)
        if pi is None or nodes[pi].op_type != "Constant":
            return None
        a = _attr(nodes[pi], "value")
        return _uniform_value(a.t) if a is not None and a.t is not None and a.t.data is not None \
            else None

    drop, fused = set(), 0
    for i, aff in enumerate(nodes):
        if aff.op_type != "AffineBcast":
            continue
        aff_x, gamma, beta = aff.inputs[:3]
        if consumers.get(aff_x, 0) != 1:
            continue
        r1 = producer.get(aff_x)
        if r1 is None or nodes[r1].op_type != "Reshape":
            continue
        in_out = nodes[r1].inputs[0]
        if consumers.get(in_out, 0) != 1:
            continue
        ii = producer.get(in_out)
        if ii is None or nodes[ii].op_type != "InstanceNormalization":
            continue
        in_node = nodes[ii]
        resh_out, scale, bias = in_node.inputs[:3]
        if const_val(scale) != 1 or const_val(bias) != 0:
            continue
        if consumers.get(resh_out, 0) != 1:
            continue
        r0 = producer.get(resh_out)
        if r0 is None or nodes[r0].op_type != "Reshape":
            continue
        x_name, shape0 = nodes[r0].inputs[:2]
        G = 32
        rsp = producer.get(shape0)
        if rsp is not None and nodes[rsp].op_type == "Constant":
            a = _attr(nodes[rsp], "value")
            if a is not None and a.t is not None and a.t.dtype == "int64" and a.t.data is not None:
                v = a.t.array()
                if v.size >= 2:
                    G = int(v[1])
        eps = get_attr_float(in_node, "epsilon", 1e-5)
        nodes[i] = Node("GroupNorm", (aff.name or "") + "_gn", [x_name, gamma, beta],
                        list(aff.outputs), [Attr("num_groups", i=G), Attr("epsilon", f=eps)])
        drop.update((r1, ii, r0))
        fused += 1
    if fused:
        graph.nodes = [n for k, n in enumerate(nodes) if k not in drop]
    return {"fused": fused}


def _const_value(graph: Graph, producer: dict, name: str) -> Optional[float]:
    """The value of a one-element initializer or Constant-node output of rank
    <= 1 (an exported scalar; larger constants could broadcast the result to
    a bigger shape, which the fused ops do not reproduce)."""
    init = graph.tensors.get(name) if graph.tensors else None
    if init is None or init.data is None:
        pi = producer.get(name)
        if pi is None or graph.nodes[pi].op_type != "Constant":
            return None
        a = _attr(graph.nodes[pi], "value")
        init = a.t if a is not None else None
        if init is None or init.data is None:
            return None
    if len(init.dims) > 1 or int(np.prod(init.dims or [1])) != 1:
        return None
    v = _uniform_value(init)
    return None if v is None else _Const(v, init.dtype)


class _Const(float):
    """A scalar constant that remembers its storage type: an fp16 graph
    stores sqrt(2) as 1.4140625, which must still read as sqrt(2)."""

    def __new__(cls, v, dtype):
        o = super().__new__(cls, v)
        o.dtype = dtype
        return o


def _scalar_operand(graph: Graph, producer: dict, node: Node):
    """(other input, constant) when one of a binary node's two inputs is a
    uniform constant; for Div only the divisor may be the constant."""
    a, b = (node.inputs + [None, None])[:2]
    if not a or not b:
        return None
    cb = _const_value(graph, producer, b)
    if cb is not None:
        return a, cb
    if node.op_type in ("Add", "Mul"):
        ca = _const_value(graph, producer, a)
        if ca is not None:
            return b, ca
    return None


# relative half-ulp of the storage types a constant may come in
_CONST_TOL = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}


def _near(v: Optional[float], want: float, tol: Optional[float] = None) -> bool:
    """v equals ``want`` up to ``tol`` (relative), by default up to the
    rounding of v's storage type (1e-6 for fp32 / fp64 constants)."""
    if v is None:
        return False
    if tol is None:
        tol = _CONST_TOL.get(getattr(v, "dtype", None), 1e-6)
    return abs(v - want) <= tol * max(1.0, abs(want))


def fuse_gelu_pattern(graph: Graph) -> dict:
    """Div(X, sqrt 2) -> Erf -> Add(., 1) -> Mul(X, .) -> Mul(., 0.5) => Gelu(X),
    the erf GELU as torch.onnx exports it and as the decomposition the
    reference's executor runs op by op (OPS.Div/Erf/Add/Mul, wgsl-executor.js
    :587-706; GELU = x * 0.5 * (1 + erf(x / sqrt 2)), wgsl-ops.js:77-81).  A
    Mul by 1/sqrt 2 stands for the Div, and the 0.5 may instead scale X first
    (Mul(Mul(X, 0.5), 1 + erf)).  Every intermediate must have the chain as its
    only consumer."""
    nodes = graph.nodes
    consumers, producer = _consumers_and_producers(graph)

    def only(name, op):
        if consumers.get(name, 0) != 1:
            return None
        pi = producer.get(name)
        return pi if pi is not None and nodes[pi].op_type == op else None

    drop, fused = set(), 0
    for i, last in enumerate(nodes):
        if last.op_type != "Mul" or i in drop:
            continue
        cands = []  # (x, name of 1 + erf(...), index of the other Mul)
        so = _scalar_operand(graph, producer, last)
        if so is not None:
            mi = only(so[0], "Mul") if _near(so[1], 0.5) else None
            if mi is not None:
                ma, mb = nodes[mi].inputs[:2]
                cands = [(ma, mb, mi), (mb, ma, mi)]
        else:
            la, lb = last.inputs[:2]
            for h, a_out in ((la, lb), (lb, la)):
                hi = only(h, "Mul")
                ho = _scalar_operand(graph, producer, nodes[hi]) if hi is not None else None
                if ho is not None and _near(ho[1], 0.5):
                    cands.append((ho[0], a_out, hi))
        for x, a_out, mi in cands:
            ai = only(a_out, "Add")
            ao = _scalar_operand(graph, producer, nodes[ai]) if ai is not None else None
            if ao is None or not _near(ao[1], 1.0):
                continue
            ei = only(ao[0], "Erf")
            if ei is None:
                continue
            d_out = nodes[ei].inputs[0]
            di = producer.get(d_out)
            if di is None or consumers.get(d_out, 0) != 1:
                continue
            dn = nodes[di]
            do = _scalar_operand(graph, producer, dn) if dn.op_type in ("Div", "Mul") else None
            if do is None or do[0] != x:
                continue
            if not ((dn.op_type == "Div" and _near(do[1], math.sqrt(2.0))) or
                    (dn.op_type == "Mul" and _near(do[1], 1.0 / math.sqrt(2.0)))):
                continue
            nodes[i] = Node("Gelu", (last.name or "") + "_gelu", [x], list(last.outputs),
                            [Attr("approximate", s="none")])
            drop.update((mi, ai, ei, di))
            fused += 1
            break
    if fused:
        graph.nodes = [n for k, n in enumerate(nodes) if k not in drop]
    return {"fused": fused}


# ONNX TensorProto types FLOAT, FLOAT16, DOUBLE, BFLOAT16
_FLOAT_TYPES = (1, 10, 11, 16)


def _last_axis_attr(node: Node) -> Optional[int]:
    axes = get_attr_ints(node, "axes", None)
    if axes is None or len(axes) != 1 or get_attr_int(node, "keepdims", 1) != 1:
        return None
    return int(axes[0])


def fuse_layer_norm_pattern(graph: Graph) -> dict:
    """The exported LayerNorm decomposition ReduceMean(X) -> Sub(X, mean) ->
    Pow(., 2) -> ReduceMean -> Add(., eps) -> Sqrt -> Div(X - mean, .) [->
    Mul(., gamma) -> Add(., beta) | AffineBcast(., gamma, beta)] =>
    LayerNormalization(X, gamma, beta) over the last axis, one di_layer_norm
    dispatch instead of the 8-9 the reference's executor issues
    (OPS.ReduceMean/Sub/Pow/Add/Sqrt/Div, wgsl-executor.js:491-706; the
    fused form is layerNorm, wgsl-ops.js:772-812).  Both ReduceMeans reduce
    the same single axis with keepdims; gamma / beta must be initializers
    whose dims are 1 except the last."""
    nodes = graph.nodes
    consumers, producer = _consumers_and_producers(graph)

    def prod(name, op, uses=1):
        if consumers.get(name, 0) != uses:
            return None
        pi = producer.get(name)
        return pi if pi is not None and nodes[pi].op_type == op else None

    def vec_param(name):
        t = graph.tensors.get(name) if graph.tensors else None
        return t is not None and t.data is not None and len(t.dims) >= 1 and \
            all(d == 1 for d in t.dims[:-1])

    def float_cast(name, uses=1):
        """Index of the float->float Cast that produces ``name`` (the fp16
        export widens X - mean before the variance and narrows the result)."""
        if consumers.get(name, 0) != uses:
            return None
        pi = producer.get(name)
        if pi is None or nodes[pi].op_type != "Cast" or \
                get_attr_int(nodes[pi], "to", 0) not in _FLOAT_TYPES:
            return None
        return pi

    drop, fused = set(), 0
    for i, dv in enumerate(nodes):
        if dv.op_type != "Div" or i in drop or len(dv.inputs) < 2:
            continue
        xc, sd = dv.inputs[:2]
        casts = []
        si = prod(sd, "Sqrt")
        if si is None:
            continue
        ai = prod(nodes[si].inputs[0], "Add")
        if ai is None:
            continue
        ao = _scalar_operand(graph, producer, nodes[ai])
        if ao is None or ao[1] < 0:
            continue
        v_out, eps = ao
        r2 = prod(v_out, "ReduceMean")
        if r2 is None:
            continue
        pw = prod(nodes[r2].inputs[0], "Pow")
        if pw is None or nodes[pw].inputs[0] != xc:
            continue
        if not _near(_const_value(graph, producer, nodes[pw].inputs[1]), 2.0, 0.0):
            continue
        ci = float_cast(xc, uses=2)
        if ci is not None:
            casts.append(ci)
            sb = prod(nodes[ci].inputs[0], "Sub")
        else:
            sb = prod(xc, "Sub", uses=2)
        if sb is None:
            continue
        x, mu = nodes[sb].inputs[:2]
        r1 = prod(mu, "ReduceMean")
        if r1 is None or nodes[r1].inputs[0] != x:
            continue
        ax1, ax2 = _last_axis_attr(nodes[r1]), _last_axis_attr(nodes[r2])
        if ax1 is None or ax1 != ax2:
            continue
        # optional affine tail
        xn = dv.outputs[0]
        if consumers.get(xn, 0) == 1:
            ci = next((k for k, n in enumerate(nodes) if xn in n.inputs), None)
            if ci is not None and nodes[ci].op_type == "Cast" and \
                    get_attr_int(nodes[ci], "to", 0) in _FLOAT_TYPES:
                casts.append(ci)
                xn = nodes[ci].outputs[0]
        tail, gamma, beta, out = [], None, None, xn
        if consumers.get(xn, 0) == 1:
            ci = next((k for k, n in enumerate(nodes) if xn in n.inputs), None)
            cn = nodes[ci] if ci is not None else None
            if cn is not None and cn.op_type == "AffineBcast" and cn.inputs[0] == xn and \
                    vec_param(cn.inputs[1]) and vec_param(cn.inputs[2]):
                tail, gamma, beta, out = [ci], cn.inputs[1], cn.inputs[2], cn.outputs[0]
            elif cn is not None and cn.op_type == "Mul":
                g = cn.inputs[1] if cn.inputs[0] == xn else cn.inputs[0]
                mo = cn.outputs[0]
                ad = next((k for k, n in enumerate(nodes) if mo in n.inputs), None) \
                    if consumers.get(mo, 0) == 1 else None
                if vec_param(g) and ad is not None and nodes[ad].op_type == "Add":
                    an = nodes[ad]
                    b = an.inputs[1] if an.inputs[0] == mo else an.inputs[0]
                    if vec_param(b):
                        tail, gamma, beta, out = [ci, ad], g, b, an.outputs[0]
        ins = [x, gamma or "", beta or ""]
        fused_node = Node("LayerNormalization", (dv.name or "") + "_ln", ins, [out],
                          [Attr("axis", i=ax1), Attr("epsilon", f=float(eps))])
        keep = tail[-1] if tail else (casts[-1] if len(casts) and
                                          nodes[casts[-1]].outputs[0] == out else i)
        nodes[keep] = fused_node
        drop.update(k for k in (r1, sb, pw, r2, ai, si, i, *casts, *tail) if k != keep)
        fused += 1
    if fused:
        graph.nodes = [n for k, n in enumerate(nodes) if k not in drop]
    return {"fused": fused}


def fuse_group_norm_silu_pattern(graph: Graph) -> dict:
    """GroupNorm -> Silu => GroupNorm with the SiLU epilogue (the
    WGSL_FUSED_GN_SILU kernel, fused-resnet.js:121-166, one dispatch instead
    of two).  Run after fuse_silu_pattern and fuse_group_norm_pattern."""
    nodes = graph.nodes
    consumers, producer = _consumers_and_producers(graph)
    drop, fused = set(), 0
    for i, sl in enumerate(nodes):
        if sl.op_type != "Silu":
            continue
        g_out = sl.inputs[0]
        gi = producer.get(g_out)
        if gi is None or consumers.get(g_out, 0) != 1 or nodes[gi].op_type != "GroupNorm" or \
                get_attr_string(nodes[gi], "activation", "") == "silu":
            continue
        gn = nodes[gi]
        nodes[i] = Node("GroupNorm", (gn.name or "") + "_silu", list(gn.inputs), list(sl.outputs),
                        list(gn.attributes) + [Attr("activation", s="silu")])
        drop.add(gi)
        fused += 1
    if fused:
        graph.nodes = [n for k, n in enumerate(nodes) if k not in drop]
    return {"fused": fused}


def fuse_attention_pattern(graph: Graph) -> dict:
    """MatMul(Q, K^T) [-> Mul / Div by a constant] -> Softmax(last axis) ->
    MatMul(., V) => FusedAttention(Q, K, V): flash attention through
    di_attn_cross, so the [.., Sq, Skv] score matrix the reference's executor
    materialises (OPS.MatMul + OPS.Softmax, wgsl-executor.js:1027-1054) is
    never written.

    * Muls on Q or on K^T (torch's scaled_dot_product_attention export
      splits the scale as sqrt(scale) over both) fold away: by constants into
      the scale attribute; by a computed factor (SDPA derives it from
      Shape(Q)) as extra inputs 3 / 4, multiplied into the scale at run time
      when they are one-element host values.
    * A single-use Transpose producing K^T gets its last two perm entries
      swapped so it yields K directly.
    * When Q, K and V come from [B, S, H, d] through head-split Transposes
      (perm 0,2,1,3; for K^T composed with the last-axes swap) and the output
      goes through the inverse one, those Transposes go too and the node
      reads and writes [B, S, H, d] (layout="bshd", the fused-attn.js
      layout).  Shape nodes reading a dropped Transpose read its source with
      a ``perm`` attribute instead.

    The fused node runs head dim 64 with fp16 MFMA operands (fp32 softmax
    state and accumulation), so its outputs agree with the fp32 chain to
    about 1e-3 relative RMS, not bit for bit; other shapes (or scale inputs
    that are not host scalars) run the unfused chain inside the node."""
    nodes = graph.nodes
    consumers, producer = _consumers_and_producers(graph)
    shape_readers: Dict[str, List[int]] = {}
    for k, n in enumerate(nodes):
        if n.op_type == "Shape" and n.inputs:
            shape_readers.setdefault(n.inputs[0], []).append(k)

    def single(name, ops):
        if consumers.get(name, 0) != 1:
            return None
        pi = producer.get(name)
        return pi if pi is not None and nodes[pi].op_type in ops else None

    def trace_transposes(name):
        """(source, composed perm from the source or None, Transpose
        indices, Shape fix-ups) of the chain of rank-4 Transposes producing
        `name` whose outputs are read by nothing else but Shape nodes."""
        chain = []
        while True:
            ti = producer.get(name)
            if ti is None or nodes[ti].op_type != "Transpose" or \
                    consumers.get(name, 0) - len(shape_readers.get(name, [])) != 1:
                break
            p = get_attr_ints(nodes[ti], "perm", None)
            if not p or len(p) != 4:
                break
            chain.append(ti)
            name = nodes[ti].inputs[0]
        perm, fix = None, []
        for ti in reversed(chain):  # forward from the source
            p = get_attr_ints(nodes[ti], "perm", None)
            perm = list(p) if perm is None else [perm[j] for j in p]
            fix += [(si, list(perm)) for si in shape_readers.get(nodes[ti].outputs[0], [])]
        return name, perm, chain, fix

    def consumer_of(name):
        if consumers.get(name, 0) != 1:
            return None
        return next((k for k, n in enumerate(nodes) if name in n.inputs), None)

    HEADS = [0, 2, 1, 3]
    drop, fused = set(), 0
    for i, sm in enumerate(nodes):
        if sm.op_type != "Softmax" or i in drop:
            continue
        p = sm.outputs[0]
        if consumers.get(p, 0) != 1:
            continue
        pv = next((k for k, n in enumerate(nodes) if n.op_type == "MatMul" and n.inputs and
                   n.inputs[0] == p), None)
        if pv is None:
            continue
        scale, s_in, used = 1.0, sm.inputs[0], [i]
        si = single(s_in, ("Mul", "Div"))
        if si is not None:
            so = _scalar_operand(graph, producer, nodes[si])
            if so is None or so[1] == 0:
                continue
            scale *= so[1] if nodes[si].op_type == "Mul" else 1.0 / so[1]
            s_in = so[0]
            used.append(si)
        qk = single(s_in, ("MatMul",))
        if qk is None:
            continue
        used.append(qk)
        q, kt = nodes[qk].inputs[:2]
        extra = ["", ""]  # computed factors on Q and on K^T
        for which in (0, 1):
            name = q if which == 0 else kt
            mi = single(name, ("Mul",))
            if mi is None:
                continue
            so = _scalar_operand(graph, producer, nodes[mi])
            if so is not None:
                scale *= so[1]
                data = so[0]
            else:
                a, b = nodes[mi].inputs[:2]
                # the factor is the operand that is not the head-split data
                data, fac = (b, a) if trace_transposes(b)[2] and not trace_transposes(a)[2] \
                    else (a, b)
                if not fac or fac in (q, kt):
                    continue
                extra[which] = fac
            used.append(mi)
            if which == 0:
                q = data
            else:
                kt = data
        if not scale > 0:
            continue
        v = nodes[pv].inputs[1]
        attrs = [Attr("scale", f=float(scale)),
                 Attr("softmax_axis", i=get_attr_int(sm, "axis", -1))]
        tail = extra if any(extra) else []
        o_name = nodes[pv].outputs[0]
        # [B,S,H,d] in and out: every head split / merge Transpose goes
        qs, cq, tq, fq = trace_transposes(q)
        ks, ck, tk, fk = trace_transposes(kt)
        vs, cv, tv, fv = trace_transposes(v)
        oc = consumer_of(o_name)
        if cq == HEADS and ck is not None and ck[:2] + [ck[3], ck[2]] == HEADS and \
                cv == HEADS and oc is not None and nodes[oc].op_type == "Transpose" and \
                get_attr_ints(nodes[oc], "perm", None) == HEADS and \
                not shape_readers.get(o_name):
            nodes[oc] = Node("FusedAttention", (nodes[pv].name or "") + "_attn",
                             [qs, ks, vs] + tail, list(nodes[oc].outputs),
                             attrs + [Attr("k_transposed", i=0), Attr("layout", s="bshd")])
            used += tq + tk + tv + [pv]
            for sidx, perm in fq + fk + fv:
                sn = nodes[sidx]
                src = qs if (sidx, perm) in fq else ks if (sidx, perm) in fk else vs
                old = get_attr_ints(sn, "perm", None)
                if old:
                    perm = [perm[j] for j in old]
                nodes[sidx] = Node("Shape", sn.name, [src], list(sn.outputs),
                                   [a for a in sn.attributes if a.name != "perm"] +
                                   [Attr("perm", ints=perm)])
        else:
            k_transposed = 1
            ti = single(kt, ("Transpose",))
            if ti is not None:
                perm = get_attr_ints(nodes[ti], "perm", None)
                if perm and len(perm) >= 2:
                    perm = list(perm[:-2]) + [perm[-1], perm[-2]]
                    tn = nodes[ti]
                    nodes[ti] = Node("Transpose", tn.name, list(tn.inputs), list(tn.outputs),
                                     [Attr("perm", ints=perm)])
                    k_transposed = 0
            nodes[pv] = Node("FusedAttention", (nodes[pv].name or "") + "_attn",
                             [q, kt, v] + tail, [o_name],
                             attrs + [Attr("k_transposed", i=k_transposed)])
        drop.update(used)
        fused += 1
    if fused:
        graph.nodes = [n for k, n in enumerate(nodes) if k not in drop]
    return {"fused": fused}


def optimize_graph(graph: Graph, attention: bool = True) -> dict:
    """Every rewrite, in dependency order: the reference's three
    (unet-wgsl.js:103-107) and then GN+SiLU, LayerNorm, GELU and (unless
    ``attention`` is False) flash attention.  Returns the per-rewrite
    counts."""
    stats = {"silu": fuse_silu_pattern(graph)["fused"],
             "mul_add": fuse_mul_add_pattern(graph)["fused"],
             "group_norm": fuse_group_norm_pattern(graph)["fused"],
             "group_norm_silu": fuse_group_norm_silu_pattern(graph)["fused"],
             "layer_norm": fuse_layer_norm_pattern(graph)["fused"],
             "gelu": fuse_gelu_pattern(graph)["fused"]}
    if attention:
        stats["attention"] = fuse_attention_pattern(graph)["fused"]
    return stats


# ---------------------------------------------------------------- planning --
def plan_execution(graph: Graph) -> dict:
    unsupported: Dict[str, int] = {}
    supported = 0
    for n in graph.nodes:
        if n.op_type in OPS:
            supported += 1
        else:
            unsupported[n.op_type] = unsupported.get(n.op_type, 0) + 1
    total = len(graph.nodes)
    return {"total": total, "supported_count": supported,
            "coverage": supported / total if total else 1.0,
            "unsupported_ops": sorted(unsupported.items(), key=lambda kv: -kv[1])}


def infer_graph_io(nodes: List[Node], weight_names) -> dict:
    """Graph inputs = consumed but never produced and not weights; outputs =
    produced but never consumed (wgsl-executor.js:1205-1221)."""
    produced, consumed = [], []
    ps, cs = set(), set()
    for n in nodes:
        for i in n.inputs:
            if i and i not in cs:
                cs.add(i)
                consumed.append(i)
        for o in n.outputs:
            if o not in ps:
                ps.add(o)
                produced.append(o)
    return {"inputs": [{"name": c} for c in consumed if c not in ps and c not in weight_names],
            "outputs": [{"name": p} for p in produced if p not in cs]}


# ---------------------------------------------------------------- executor --
METADATA_OPS = {"Reshape", "Shape", "Unsqueeze", "Squeeze", "Gather", "Slice", "Concat", "Constant",
                "ConstantOfShape", "Cast", "Expand", "Equal", "Where", "Identity", "Transpose"}
# fp16-resident weights: (op, input index) pairs that read them as they are;
# relabelling ops pass the dtype on; every other consumer gets an fp32 copy
F16_WEIGHT_INPUTS = {("MatMul", 1), ("Gemm", 1), ("Conv", 1)}
CONV_F16_COMPUTE = 1  # DI_CONV_F16_COMPUTE
F16_PASSTHROUGH = {"Reshape", "Unsqueeze", "Squeeze", "Identity", "Expand", "Shape"}
BINARY_SHAPE_AWARE = {"Add", "Sub", "Mul", "Div"}


class ExecutorError(RuntimeError):
    pass


class _Ctx:
    def __init__(self, device, pool, dispatchers, weights, promote, conv_f16=False):
        self.device = device
        self.pool = pool
        self.dispatchers = dispatchers
        self.weights = weights
        self.promote = promote
        self.conv_f16 = conv_f16


class Executor:
    """Walks a topologically sorted graph, one C-ABI dispatch per GPU node
    (wgsl-executor.js:1223-1466)."""

    def __init__(self, device: Device, graph: Graph, weight_cache: WeightCache,
                 conv_f16: bool = False):
        """``conv_f16`` (opt-in): Conv nodes run on the fp16 MFMA path
        (DI_CONV_F16_COMPUTE: fp32 tensors staged to fp16 operands, fp32
        accumulation and output) instead of the exact fp32 MFMA path the
        reference's fp32 semantics call for."""
        self.device = device
        self.graph = graph
        self.weights = weight_cache
        self.conv_f16 = conv_f16
        self.pool = BufferPool(device)
        self.dispatchers = create_dispatchers(device)
        if not graph.inputs or not graph.outputs:
            io = infer_graph_io(graph.nodes, set(weight_cache.tensors.keys()))
            if not graph.inputs:
                graph.inputs = io["inputs"]
            if not graph.outputs:
                graph.outputs = io["outputs"]
        self.consumers: Dict[str, int] = {}
        for n in graph.nodes:
            for i in n.inputs:
                if i:
                    self.consumers[i] = self.consumers.get(i, 0) + 1
        for o in graph.outputs:
            self.consumers[o["name"]] = self.consumers.get(o["name"], 0) + 1
        self.graph_input_names = {i["name"] for i in graph.inputs}
        self._temps: List[Buffer] = []

    def _promote(self, t):
        """CPU-only tensor -> device fp32 tensor (a pool buffer released at the
        end of the run)."""
        if t is None or getattr(t, "buf", None) is not None:
            return t
        f = np.asarray(t.cpu_data).astype(np.float32).reshape(-1)
        buf = self.pool.acquire(max(f.nbytes, 4))
        self.device.upload(buf, f)
        self._temps.append(buf)
        return Tensor(buf, list(t.dims) if t.dims is not None else [f.size])

    def _widen(self, t):
        """fp16 device tensor -> fp32 copy (a pool buffer released at the end
        of the run)."""
        buf = self.pool.acquire(max(t.numel * 4, 4))
        self.dispatchers.convert(t.buf, F16, buf, F32, t.numel)
        self._temps.append(buf)
        return Tensor(buf, list(t.dims))

    def run(self, inputs: Dict[str, Any]) -> Dict[str, Tensor]:
        """One forward pass.  ``inputs``: name -> Tensor | CpuTensor | numpy
        array (uploaded as fp32; float arrays keep their shape, int arrays
        stay on the CPU as shape tensors)."""
        consumers = dict(self.consumers)
        env: Dict[str, Any] = {}
        self._temps = []
        for name, val in inputs.items():
            if isinstance(val, (Tensor, CpuTensor)):
                env[name] = val
            elif isinstance(val, np.ndarray):
                if val.dtype.kind in "iu":
                    env[name] = CpuTensor(val.reshape(-1), list(val.shape), _dtype_of(val), True)
                else:
                    # a pool buffer, returned with the run's other temporaries
                    f = np.ascontiguousarray(val, np.float32)
                    buf = self.pool.acquire(max(f.nbytes, 4))
                    self.device.upload(buf, f)
                    self._temps.append(buf)
                    env[name] = Tensor(buf, list(f.shape))
            else:
                raise ExecutorError(f'unsupported input seed for "{name}": {type(val).__name__}')
        ctx = _Ctx(self.device, self.pool, self.dispatchers, self.weights, self._promote,
                   self.conv_f16)
        LOG["t0"] = time.perf_counter()
        LOG["node_count"] = len(self.graph.nodes)
        LOG["op_hist"] = {}
        if LOG["profile"]:
            LOG["profile_data"] = []
        # Live env names per device buffer (a Reshape / Cast / Expand output
        # aliases its input's buffer): a pool buffer goes back to the free
        # list as soon as no live name refers to it, i.e. right after the
        # last consumer of its last alias is enqueued.  Every kernel and copy
        # runs in order on the one library stream, so a later kernel that
        # receives the recycled buffer runs after every earlier reader.
        refs: Dict[int, int] = {}
        for t in env.values():
            b = getattr(t, "buf", None)
            if b is not None:
                refs[id(b)] = refs.get(id(b), 0) + 1
        protected = set(self.graph_input_names) | {o["name"] for o in self.graph.outputs}

        def drop(name):
            t = env.pop(name)
            b = getattr(t, "buf", None)
            if b is None:
                return
            refs[id(b)] -= 1
            if refs[id(b)] == 0 and self.pool.owns(b) and b not in self._temps:
                self.pool.release(b)
        for ni, node in enumerate(self.graph.nodes):
            op = OPS.get(node.op_type)
            if op is None:
                raise ExecutorError(f"unsupported op @{ni}: {node.op_type} ({node.name})")
            LOG["op_hist"][node.op_type] = LOG["op_hist"].get(node.op_type, 0) + 1
            ins = []
            for name in node.inputs:
                if not name:
                    ins.append(None)
                elif name in env:
                    ins.append(env[name])
                elif self.weights.has(name):
                    ins.append(self.weights.get(name))
                else:
                    raise ExecutorError(f"tensor not found @{ni} {node.op_type}: {name}")
            if node.op_type not in F16_PASSTHROUGH:
                ins = [self._widen(t) if getattr(t, "dtype", None) == "float16" and
                       getattr(t, "buf", None) is not None and
                       (node.op_type, k) not in F16_WEIGHT_INPUTS else t
                       for k, t in enumerate(ins)]
            if node.op_type not in METADATA_OPS:
                keep_int = node.op_type in BINARY_SHAPE_AWARE
                promoted = []
                for t in ins:
                    if t is None or getattr(t, "buf", None) is not None:
                        promoted.append(t)
                    elif keep_int and t.cpu_data.dtype in (np.int64, np.int32):
                        promoted.append(t)
                    elif t.cpu_data.size == 1:
                        promoted.append(t)  # scalar CPU constants feed CPU fast paths
                    else:
                        promoted.append(self._promote(t))
                ins = promoted
            t_prof = time.perf_counter()
            try:
                out = op(ctx, node, ins)
            except Exception as e:  # noqa: BLE001 - re-raised with the node context
                descs = ",".join("null" if t is None else (f"GPU{t.dims}" if getattr(t, "buf", None)
                                 is not None else f"CPU{t.dims}:{t.dtype}") for t in ins)
                _dlog(f"FAIL @{ni} {node.op_type} ({node.name}): {e} ins={descs}")
                raise ExecutorError(f"op @{ni} {node.op_type} ({node.name}) failed: {e}") from e
            if len(node.outputs) > 1:
                raise ExecutorError(f"multi-output op not supported yet: {node.op_type}")
            _dlog(f"@{ni} {node.op_type:<18} {node.name} -> {out!r} pool.live={self.pool.live}")
            if LOG["traffic"] and node.op_type not in METADATA_OPS:
                td = LOG["traffic_data"] = LOG["traffic_data"] or {"weights": 0, "acts": 0,
                                                                   "out": 0, "by_op": {}}
                nb = 0
                for name, t in zip(node.inputs, ins):
                    if t is None or getattr(t, "buf", None) is None:
                        continue
                    nb += t.byte_length
                    td["weights" if self.weights.has(name) else "acts"] += t.byte_length
                if getattr(out, "buf", None) is not None:
                    td["out"] += out.byte_length
                    nb += out.byte_length
                td["by_op"][node.op_type] = td["by_op"].get(node.op_type, 0) + nb
            oname = node.outputs[0]
            if oname in env:  # a name produced twice: the old value is dead
                drop(oname)
            env[oname] = out
            if getattr(out, "buf", None) is not None:
                refs[id(out.buf)] = refs.get(id(out.buf), 0) + 1
            if LOG["profile"] and getattr(out, "buf", None) is not None:
                self.device.sync()
                LOG["profile_data"].append({"ni": ni, "op": node.op_type, "name": node.name,
                                            "dims": out.dims,
                                            "ms": (time.perf_counter() - t_prof) * 1e3})
            for name in node.inputs:
                if not name or name not in env:
                    continue
                consumers[name] = consumers.get(name, 0) - 1
                if consumers[name] <= 0 and name not in protected:
                    drop(name)
            if consumers.get(oname, 0) <= 0 and oname not in protected:
                drop(oname)  # produced but never read
        # snapshot graph outputs into fresh buffers owned by the caller
        snaps: Dict[str, Tensor] = {}
        for o in self.graph.outputs:
            t = env.get(o["name"])
            if getattr(t, "buf", None) is None:
                continue
            stable = self.device.create_buffer(max(t.numel * 4, 4))
            self.device.copy(stable, t.buf, t.numel * 4)
            snaps[o["name"]] = Tensor(stable, list(t.dims))
        self.device.sync()
        # Everything pool-owned goes back once the device is done: deferred
        # intermediates, alias-held env entries, CPU promotions and the graph
        # outputs' own buffers (the caller holds the snapshots).  The reference
        # keeps the last two live forever, so its pool grows on every run.
        released = set()
        for buf in self._temps:
            if id(buf) in released:
                continue
            released.add(id(buf))
            self.pool.release(buf)
        for name, t in env.items():
            b = getattr(t, "buf", None)
            if b is None or id(b) in released or self.weights.has(name) or \
                    name in self.graph_input_names or not self.pool.owns(b):
                continue
            released.add(id(b))
            self.pool.release(b)
        self._temps = []
        _dlog(f"run: done in {(time.perf_counter() - LOG['t0']) * 1e3:.1f} ms "
              f"pool.allocs={self.pool.allocs} peak={self.pool.peak} "
              f"peak_bytes={self.pool.peak_bytes}")
        return {o["name"]: snaps.get(o["name"], env.get(o["name"])) for o in self.graph.outputs}

    def destroy(self) -> None:
        self.pool.destroy()
