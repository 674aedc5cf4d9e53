"""drawinstant — MI355X-native SD-Turbo U-Net op / fused-block layer.

Python host mirror of draw-instant's wgsl-executor op-dispatch API and
fused-*.js block entry points, driving the hand-written gfx950 HIP kernels of
libdrawinstant_hip.so through its C ABI (include/drawinstant.h).
"""
from .device import (F16, F32, NCHW, NHWC, Buffer, DiError, Device, call, dtype_code,  # noqa: F401
                     np_dtype)

__all__ = ["Device", "Buffer", "DiError", "call", "F32", "F16", "NCHW", "NHWC", "dtype_code",
           "np_dtype"]
