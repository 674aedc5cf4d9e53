"""SD-Turbo (SD2.1 UNet2DConditionModel) denoise step on libdrawinstant_hip.

Host mirror of the reference's WGSL U-Net driver (unet-wgsl.js):
``load_unet`` plays loadUNetWGSL (:40-114) - except that weights are seeded
random (the reference downloads a 1.73 GB ONNX, impossible offline) or come
from ``load_state_dict`` - and ``UNet.forward`` plays unetForwardWGSL
(:145-195): sample [B,4,H,W], one timestep per sample, encoder hidden states
[B,77,1024] -> out_sample [B,4,H,W], with device-resident buffers and no
per-op readback.

``state_dict`` / ``load_state_dict`` translate between the library's physical
parameter layouts and diffusers' logical ones (OIHW convs, separate
to_q/to_k/to_v, GEGLU proj as [hidden; gate] rows).
"""
from __future__ import annotations

import ctypes
import re

import numpy as np

from .device import Buffer, Device, call

PARAM_VECTOR, PARAM_LINEAR, PARAM_CONV_OHWI, PARAM_LINEAR_STACKED, PARAM_GEGLU_ROWS = range(5)
UNET_GRAPH = 1


class UNetConfig(ctypes.Structure):
    """Mirror of di_unet_config (include/drawinstant.h)."""
    _fields_ = [
        ("in_channels", ctypes.c_uint32), ("out_channels", ctypes.c_uint32),
        ("block_channels", ctypes.c_uint32 * 4), ("cross_attn", ctypes.c_uint32 * 4),
        ("layers_per_block", ctypes.c_uint32), ("cross_dim", ctypes.c_uint32),
        ("time_dim", ctypes.c_uint32), ("groups", ctypes.c_uint32),
        ("resnet_eps", ctypes.c_float), ("transformer_gn_eps", ctypes.c_float),
        ("ln_eps", ctypes.c_float),
    ]

    @classmethod
    def sd21(cls) -> "UNetConfig":
        c = cls()
        call("di_unet_default_config", ctypes.byref(c))
        return c

    @classmethod
    def small(cls, channels=(64, 128, 256, 256), cross_dim=256, time_dim=256) -> "UNetConfig":
        """Same architecture, narrow channels: the CPU-oracle-sized U-Net."""
        c = cls.sd21()
        for i, ch in enumerate(channels):
            c.block_channels[i] = ch
        c.cross_dim = cross_dim
        c.time_dim = time_dim
        return c

    def as_dict(self) -> dict:
        return {
            "in_channels": self.in_channels, "out_channels": self.out_channels,
            "block_channels": list(self.block_channels), "cross_attn": list(self.cross_attn),
            "layers_per_block": self.layers_per_block, "cross_dim": self.cross_dim,
            "time_dim": self.time_dim, "groups": self.groups, "resnet_eps": self.resnet_eps,
            "transformer_gn_eps": self.transformer_gn_eps, "ln_eps": self.ln_eps,
        }


def _geglu_split(rows: np.ndarray):
    """Physical [16 hidden | 16 gate] row groups -> (hidden, gate)."""
    g = rows.reshape((rows.shape[0] // 32, 2, 16) + rows.shape[1:])
    hid = g[:, 0].reshape((rows.shape[0] // 2,) + rows.shape[1:])
    gate = g[:, 1].reshape((rows.shape[0] // 2,) + rows.shape[1:])
    return hid, gate


def _geglu_join(hid: np.ndarray, gate: np.ndarray) -> np.ndarray:
    n = hid.shape[0]
    h = hid.reshape((n // 16, 1, 16) + hid.shape[1:])
    g = gate.reshape((n // 16, 1, 16) + gate.shape[1:])
    return np.concatenate([h, g], axis=1).reshape((2 * n,) + hid.shape[1:])


class UNet:
    """A di_unet on one Device."""

    def __init__(self, device: Device, config: UNetConfig | None = None, seed: int = 0):
        self.device = device
        self.config = config if config is not None else UNetConfig.sd21()
        h = ctypes.c_void_p()
        call("di_unet_create", device.ctx, ctypes.byref(self.config), seed, ctypes.byref(h))
        self.handle = h
        n_t, n_e = ctypes.c_uint32(), ctypes.c_uint64()
        call("di_unet_num_params", device.ctx, self.handle, ctypes.byref(n_t), ctypes.byref(n_e))
        self.params = [self._info(i) for i in range(n_t.value)]
        self.num_physical_elements = n_e.value

    def _info(self, i: int) -> dict:
        name = ctypes.create_string_buffer(256)
        dims = (ctypes.c_uint32 * 8)()
        nd, dt, lay = ctypes.c_uint32(), ctypes.c_int32(), ctypes.c_int32()
        call("di_unet_param_info", self.device.ctx, self.handle, i, name, 256, dims,
             ctypes.byref(nd), ctypes.byref(dt), ctypes.byref(lay))
        return {"index": i, "name": name.value.decode(), "shape": tuple(dims[:nd.value]),
                "dtype": np.float32 if dt.value == 0 else np.float16, "layout": lay.value}

    def destroy(self):
        if self.handle:
            call("di_unet_destroy", self.device.ctx, self.handle)
            self.handle = None

    # ---- parameters ----
    def download_param(self, p: dict) -> np.ndarray:
        out = np.empty(p["shape"], p["dtype"])
        call("di_unet_param_download", self.device.ctx, self.handle, p["index"],
             out.ctypes.data_as(ctypes.c_void_p), out.nbytes)
        return out

    def upload_param(self, p: dict, arr: np.ndarray):
        a = np.ascontiguousarray(arr, p["dtype"]).reshape(p["shape"])
        call("di_unet_param_upload", self.device.ctx, self.handle, p["index"],
             a.ctypes.data_as(ctypes.c_void_p), a.nbytes)

    def state_dict(self, dtype=np.float32) -> dict:
        """diffusers-named, diffusers-layout tensors (float32 by default)."""
        sd = {}
        for p in self.params:
            a = self.download_param(p).astype(dtype)
            name, lay = p["name"], p["layout"]
            if lay == PARAM_CONV_OHWI:
                a = a.transpose(0, 3, 1, 2)
                if name == "conv_in.weight":
                    a = a[:, : self.config.in_channels]
                sd[name] = np.ascontiguousarray(a)
            elif lay == PARAM_LINEAR_STACKED:
                base = name[: -len(".to_qkv.weight")] if name.endswith("to_qkv.weight") else \
                    name[: -len(".to_kv.weight")]
                parts = ("to_q", "to_k", "to_v") if name.endswith("to_qkv.weight") else ("to_k", "to_v")
                for j, nm in enumerate(np.split(a, len(parts), axis=0)):
                    sd[f"{base}.{parts[j]}.weight"] = np.ascontiguousarray(nm)
            elif lay == PARAM_GEGLU_ROWS:
                hid, gate = _geglu_split(a)
                sd[name] = np.ascontiguousarray(np.concatenate([hid, gate], axis=0))
            else:
                sd[name] = a
        return sd

    def load_state_dict(self, sd: dict):
        """Upload diffusers-layout tensors (the inverse of state_dict)."""
        for p in self.params:
            name, lay = p["name"], p["layout"]
            if lay == PARAM_CONV_OHWI:
                w = np.asarray(sd[name], np.float32)
                if name == "conv_in.weight":
                    pad = p["shape"][3] - w.shape[1]
                    w = np.concatenate([w, np.zeros((w.shape[0], pad) + w.shape[2:], w.dtype)], 1)
                a = w.transpose(0, 2, 3, 1)
            elif lay == PARAM_LINEAR_STACKED:
                qkv = name.endswith("to_qkv.weight")
                base = re.sub(r"\.to_q?kv\.weight$", "", name)
                parts = ("to_q", "to_k", "to_v") if qkv else ("to_k", "to_v")
                a = np.concatenate([np.asarray(sd[f"{base}.{x}.weight"]) for x in parts], 0)
            elif lay == PARAM_GEGLU_ROWS:
                full = np.asarray(sd[name])
                hid, gate = np.split(full, 2, axis=0)
                a = _geglu_join(hid, gate)
            else:
                a = sd[name]
            self.upload_param(p, a)

    def num_logical_params(self) -> int:
        return int(sum(v.size for v in self.state_dict(np.float16).values()))

    # ---- forward ----
    def forward(self, sample: Buffer, timesteps: Buffer, context: Buffer, out: Buffer, B: int = 1,
                H: int = 64, W: int = 64, Sctx: int = 77, graph: bool = False):
        """Enqueue one denoise step (unetForwardWGSL, unet-wgsl.js:145)."""
        call("di_unet_forward", self.device.ctx, self.handle, sample.handle, timesteps.handle,
             context.handle, out.handle, B, H, W, Sctx, UNET_GRAPH if graph else 0)

    def __call__(self, sample: np.ndarray, timestep, context: np.ndarray, graph: bool = False):
        """Host arrays in, host array out (uploads, one step, one readback)."""
        dev = self.device
        sample = np.ascontiguousarray(sample, np.float32)
        context = np.ascontiguousarray(context, np.float32)
        B, _, H, W = sample.shape
        ts = np.broadcast_to(np.asarray(timestep, np.float32), (B,)).copy()
        bs, bt, bc = dev.storage(sample), dev.storage(ts), dev.storage(context)
        bo = dev.create_buffer(B * self.config.out_channels * H * W * 4)
        try:
            self.forward(bs, bt, bc, bo, B, H, W, context.shape[1], graph)
            return dev.download(bo, np.float32, (B, self.config.out_channels, H, W))
        finally:
            for b in (bs, bt, bc, bo):
                b.destroy()


def load_unet(device: Device, config: UNetConfig | None = None, seed: int = 0) -> UNet:
    """loadUNetWGSL counterpart: build the model on the device."""
    return UNet(device, config, seed)


_state: dict = {}


def unet_forward_hip(sample: np.ndarray, timestep, cond: np.ndarray, B: int = 1, H: int = 64,
                     W: int = 64, tokens: int = 77, dim: int = 1024, seed: int = 0,
                     graph: bool = True) -> dict:
    """unetForwardWGSL (unet-wgsl.js:145-195): sample [B,4,H,W] fp32, one
    scheduler timestep, cond [B,tokens,dim] -> {"out": [B,4,H,W] fp32,
    "dims", "ms"}.  The timestep is rounded to an integer, as the reference
    passes it to its int64 graph input; the model is built once per process
    (the reference's ``_state``) from seeded weights."""
    st = _state.get("unet")
    if st is None:
        dev = Device(0)
        st = _state["unet"] = (dev, UNet(dev, seed=seed))
    dev, u = st
    sample = np.ascontiguousarray(sample, np.float32).reshape(B, 4, H, W)
    cond = np.ascontiguousarray(cond, np.float32).reshape(B, tokens, dim)
    ts_val = timestep if np.isscalar(timestep) else np.asarray(timestep).reshape(-1)[0]
    ts = np.full(B, float(round(float(ts_val))), np.float32)
    bs, bt, bc = dev.storage(sample), dev.storage(ts), dev.storage(cond)
    bo = dev.create_buffer(sample.nbytes)
    try:
        import time
        t0 = time.perf_counter()
        u.forward(bs, bt, bc, bo, B, H, W, tokens, graph)
        out = dev.download(bo, np.float32, (B, 4, H, W))  # implicit sync; raises on faults
        ms = (time.perf_counter() - t0) * 1e3
    finally:
        for b in (bs, bt, bc, bo):
            b.destroy()
    return {"out": out, "dims": [B, 4, H, W], "ms": ms}
