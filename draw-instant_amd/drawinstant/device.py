"""Device, buffers and errors: the host-side objects around libdrawinstant_hip.so.

``Device`` plays the role of the WebGPU ``GPUDevice`` the reference passes to
every kernel factory (wgsl-ops.js:25-42) and ``Buffer`` the role of a
``GPUBuffer``: an opaque device allocation, here a u64 library handle.  The
library's one in-order stream replaces the command encoder + queue.submit
pairs, so ops run in call order without any explicit submit.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

F32 = 0
F16 = 1
F32W16 = 2  # fp32 activations, fp16-resident weights (matmul / gemm / conv2d)
NCHW = 0
NHWC = 1
BSHD = 0  # attention layouts
BHSD = 1

_NP_DT = {F32: np.float32, F16: np.float16}
_DT_OF = {np.dtype(np.float32): F32, np.dtype(np.float16): F16}

STATUS = {0: "DI_OK", 1: "DI_EINVAL", 2: "DI_ENOMEM", 3: "DI_EHIP", 4: "DI_EUNSUPPORTED",
          5: "DI_EHANDLE"}


class DiError(RuntimeError):
    """A failing libdrawinstant_hip call: status code + the library's message."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn}: {STATUS.get(code, code)}: {msg}")
        self.code = code
        self.fn = fn


def lib():
    return _lib.load()


def call(fn: str, *args):
    """Call a di_* entry point and raise DiError on a non-zero status."""
    rc = getattr(lib(), fn)(*args)
    if rc != 0:
        raise DiError(fn, rc, lib().di_last_error().decode(errors="replace"))
    return rc


def dtype_code(dt) -> int:
    if isinstance(dt, int):
        return dt
    return _DT_OF[np.dtype(dt)]


def np_dtype(code: int):
    return _NP_DT[code]


class Buffer:
    """A device allocation (the GPUBuffer of the reference)."""

    __slots__ = ("device", "handle", "size", "__weakref__")

    def __init__(self, device: "Device", handle: int, size: int):
        self.device = device
        self.handle = handle
        self.size = size

    def destroy(self):
        if self.handle:
            call("di_free", self.device.ctx, self.handle)
            self.handle = 0

    def __repr__(self):
        return f"Buffer(handle={self.handle}, size={self.size})"


class Device:
    """One HIP device + in-order stream (a di_ctx)."""

    def __init__(self, index: int = 0):
        ctx = ctypes.c_void_p()
        call("di_create", index, ctypes.byref(ctx))
        self.ctx = ctx
        self.index = index
        n_cu, clk, hbm = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_uint64()
        call("di_device_info", self.ctx, ctypes.byref(n_cu), ctypes.byref(clk), ctypes.byref(hbm))
        self.num_cus, self.clock_khz, self.hbm_bytes = n_cu.value, clk.value, hbm.value

    # ---- lifecycle ----
    def destroy(self):
        if self.ctx:
            call("di_destroy", self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()

    def sync(self):
        """Wait for all enqueued work; raises on asynchronous kernel faults."""
        call("di_sync", self.ctx)

    # ---- memory ----
    def create_buffer(self, nbytes: int) -> Buffer:
        h = ctypes.c_uint64()
        call("di_alloc", self.ctx, int(nbytes), ctypes.byref(h))
        return Buffer(self, h.value, int(nbytes))

    def storage(self, array) -> Buffer:
        """createStorage (wgsl-ops.js:1172-1180): allocate + upload."""
        a = np.ascontiguousarray(array)
        b = self.create_buffer(max(a.nbytes, 1))
        self.upload(b, a)
        return b

    def upload(self, buf: Buffer, array, offset: int = 0):
        a = np.ascontiguousarray(array)
        call("di_upload", self.ctx, buf.handle, offset, a.ctypes.data_as(ctypes.c_void_p), a.nbytes)

    def download(self, buf: Buffer, dtype=np.float32, shape=None, offset: int = 0) -> np.ndarray:
        """readBack (wgsl-ops.js:1195-1210)."""
        dt = np.dtype(dtype)
        if shape is None:
            shape = ((buf.size - offset) // dt.itemsize,)
        out = np.empty(shape, dt)
        call("di_download", self.ctx, buf.handle, offset, out.ctypes.data_as(ctypes.c_void_p),
             out.nbytes)
        return out

    def copy(self, dst: Buffer, src: Buffer, nbytes: int, dst_offset: int = 0, src_offset: int = 0):
        call("di_copy", self.ctx, dst.handle, dst_offset, src.handle, src_offset, nbytes)

    def pool_stats(self) -> dict:
        v = [ctypes.c_uint64() for _ in range(4)]
        call("di_pool_stats", self.ctx, *[ctypes.byref(x) for x in v])
        return dict(zip(("live", "peak", "allocs", "reserved"), (x.value for x in v)))

    def workspace_stats(self) -> dict:
        b, pinned, retired = ctypes.c_uint64(), ctypes.c_uint32(), ctypes.c_uint32()
        call("di_workspace_stats", self.ctx, ctypes.byref(b), ctypes.byref(pinned),
             ctypes.byref(retired))
        return {"bytes": b.value, "pinned": pinned.value, "retired": retired.value}

    def fill_normal(self, buf: Buffer, n: int, seed: int, mean: float = 0.0, std: float = 1.0,
                    dtype=F32):
        call("di_fill_normal", self.ctx, buf.handle, dtype_code(dtype), n, seed, mean, std)

    # ---- timers ----
    def timer_begin(self, slot: int = 0):
        call("di_timer_begin", self.ctx, slot)

    def timer_end(self, slot: int = 0):
        call("di_timer_end", self.ctx, slot)

    def timer_ms(self, slot: int = 0) -> float:
        ms = ctypes.c_float()
        call("di_timer_ms", self.ctx, slot, ctypes.byref(ms))
        return ms.value
