"""SD VAE decoder on libdrawinstant_hip: the decode of the reference's
vae-wgsl.js / vae.js without the executor.

``VAE`` plays loadVAEWGSL (vae-wgsl.js:28-72) - with seeded weights or
``load_state_dict`` instead of the downloaded vae_decoder ONNX - and
``VAE.decode`` plays vaeDecodeWGSL (:94-140): latent [B,4,H,W] fp32 scaled by
1 / 0.18215 -> image [B,3,8H,8W] fp32 in [-1, 1]-ish units (the reference
maps it to pixels afterwards), device-resident, no per-op readback.

``state_dict`` / ``load_state_dict`` translate between the library's physical
layouts and diffusers' (AutoencoderKL names under ``post_quant_conv.`` and
``decoder.``; OIHW convs; separate to_q / to_k / to_v with biases).
"""
from __future__ import annotations

import ctypes
import re

import numpy as np

from .device import Buffer, Device, call

PARAM_VECTOR, PARAM_LINEAR, PARAM_CONV_OHWI, PARAM_LINEAR_STACKED = range(4)
VAE_GRAPH = 1
SCALING_FACTOR = 0.18215  # vae-wgsl.js:26


class VAEConfig(ctypes.Structure):
    """Mirror of di_vae_config (include/drawinstant.h)."""
    _fields_ = [
        ("latent_channels", ctypes.c_uint32), ("out_channels", ctypes.c_uint32),
        ("block_channels", ctypes.c_uint32 * 4), ("layers_per_block", ctypes.c_uint32),
        ("groups", ctypes.c_uint32), ("eps", ctypes.c_float),
    ]

    @classmethod
    def sd(cls) -> "VAEConfig":
        c = cls()
        call("di_vae_default_config", ctypes.byref(c))
        return c

    @classmethod
    def small(cls, channels=(32, 32, 64, 64)) -> "VAEConfig":
        """Same architecture, narrow channels: the CPU-oracle-sized decoder."""
        c = cls.sd()
        for i, ch in enumerate(channels):
            c.block_channels[i] = ch
        return c

    def as_dict(self) -> dict:
        return {"latent_channels": self.latent_channels, "out_channels": self.out_channels,
                "block_channels": list(self.block_channels),
                "layers_per_block": self.layers_per_block, "groups": self.groups,
                "eps": self.eps}


class VAE:
    """A di_vae on one Device."""

    def __init__(self, device: Device, config: VAEConfig | None = None, seed: int = 0):
        self.device = device
        self.config = config if config is not None else VAEConfig.sd()
        h = ctypes.c_void_p()
        call("di_vae_create", device.ctx, ctypes.byref(self.config), seed, ctypes.byref(h))
        self.handle = h
        n_t, n_e = ctypes.c_uint32(), ctypes.c_uint64()
        call("di_vae_num_params", device.ctx, self.handle, ctypes.byref(n_t), ctypes.byref(n_e))
        self.params = [self._info(i) for i in range(n_t.value)]
        self.num_physical_elements = n_e.value

    def _info(self, i: int) -> dict:
        name = ctypes.create_string_buffer(256)
        dims = (ctypes.c_uint32 * 8)()
        nd, dt, lay = ctypes.c_uint32(), ctypes.c_int32(), ctypes.c_int32()
        call("di_vae_param_info", self.device.ctx, self.handle, i, name, 256, dims,
             ctypes.byref(nd), ctypes.byref(dt), ctypes.byref(lay))
        return {"index": i, "name": name.value.decode(), "shape": tuple(dims[:nd.value]),
                "dtype": np.float32 if dt.value == 0 else np.float16, "layout": lay.value}

    def destroy(self):
        if self.handle:
            call("di_vae_destroy", self.device.ctx, self.handle)
            self.handle = None

    # ---- parameters ----
    def download_param(self, p: dict) -> np.ndarray:
        out = np.empty(p["shape"], p["dtype"])
        call("di_vae_param_download", self.device.ctx, self.handle, p["index"],
             out.ctypes.data_as(ctypes.c_void_p), out.nbytes)
        return out

    def upload_param(self, p: dict, arr: np.ndarray):
        a = np.ascontiguousarray(arr, p["dtype"]).reshape(p["shape"])
        call("di_vae_param_upload", self.device.ctx, self.handle, p["index"],
             a.ctypes.data_as(ctypes.c_void_p), a.nbytes)

    def state_dict(self, dtype=np.float32) -> dict:
        """diffusers-named, diffusers-layout tensors."""
        sd = {}
        L = self.config.latent_channels
        for p in self.params:
            a = self.download_param(p).astype(dtype)
            name, lay = p["name"], p["layout"]
            if lay == PARAM_CONV_OHWI:
                a = a.transpose(0, 3, 1, 2)
                if name == "decoder.conv_in.weight":
                    a = a[:, :L]
                sd[name] = np.ascontiguousarray(a)
            elif lay == PARAM_LINEAR_STACKED:
                base = re.sub(r"\.to_qkv\.(weight|bias)$", "", name)
                kind = name.rsplit(".", 1)[1]
                for part, t in zip(("to_q", "to_k", "to_v"), np.split(a, 3, axis=0)):
                    sd[f"{base}.{part}.{kind}"] = np.ascontiguousarray(t)
            elif name == "post_quant_conv.weight":
                sd[name] = a.reshape(L, L, 1, 1)
            else:
                sd[name] = a
        return sd

    def load_state_dict(self, sd: dict):
        """Upload diffusers-layout tensors (the inverse of state_dict)."""
        for p in self.params:
            name, lay = p["name"], p["layout"]
            if lay == PARAM_CONV_OHWI:
                w = np.asarray(sd[name], np.float32)
                if name == "decoder.conv_in.weight":
                    pad = p["shape"][3] - w.shape[1]
                    w = np.concatenate([w, np.zeros((w.shape[0], pad) + w.shape[2:], w.dtype)], 1)
                a = w.transpose(0, 2, 3, 1)
            elif lay == PARAM_LINEAR_STACKED:
                base = re.sub(r"\.to_qkv\.(weight|bias)$", "", name)
                kind = name.rsplit(".", 1)[1]
                a = np.concatenate([np.asarray(sd[f"{base}.{x}.{kind}"])
                                    for x in ("to_q", "to_k", "to_v")], 0)
            else:
                a = np.asarray(sd[name]).reshape(p["shape"])
            self.upload_param(p, a)

    # ---- decode ----
    def decode(self, latent: Buffer, image: Buffer, B: int = 1, H: int = 64, W: int = 64,
               scale: float = 1.0 / SCALING_FACTOR, graph: bool = False):
        """Enqueue one decode (vaeDecodeWGSL, vae-wgsl.js:94)."""
        call("di_vae_decode", self.device.ctx, self.handle, latent.handle, image.handle, B, H, W,
             scale, VAE_GRAPH if graph else 0)

    def __call__(self, latent: np.ndarray, scale: float = 1.0 / SCALING_FACTOR,
                 graph: bool = False) -> np.ndarray:
        """Host latent in, host image out."""
        dev = self.device
        z = np.ascontiguousarray(latent, np.float32)
        B, _, H, W = z.shape
        bz = dev.storage(z)
        bi = dev.create_buffer(B * self.config.out_channels * 64 * H * W * 4)
        try:
            self.decode(bz, bi, B, H, W, scale, graph)
            return dev.download(bi, np.float32, (B, self.config.out_channels, 8 * H, 8 * W))
        finally:
            bz.destroy()
            bi.destroy()


def load_vae(device: Device, config: VAEConfig | None = None, seed: int = 0) -> VAE:
    """loadVAEWGSL counterpart: build the decoder on the device."""
    return VAE(device, config, seed)


_state: dict = {}


def vae_decode_hip(latent: np.ndarray, B: int = 1, lH: int = 64, lW: int = 64,
                   seed: int = 0) -> dict:
    """vaeDecodeWGSL (vae-wgsl.js:94-140): latent [B,4,lH,lW] fp32 ->
    {"image": [B,3,8lH,8lW] fp32, "dims", "decodeMs"}; the decoder is built
    once per process from seeded weights."""
    import time
    st = _state.get("vae")
    if st is None:
        dev = Device(0)
        st = _state["vae"] = (dev, VAE(dev, seed=seed))
    dev, v = st
    z = np.ascontiguousarray(latent, np.float32).reshape(B, 4, lH, lW)
    t0 = time.perf_counter()
    img = v(z)
    ms = (time.perf_counter() - t0) * 1e3
    return {"image": img, "dims": list(img.shape), "decodeMs": ms}
