"""Fused-block entry points of libdrawinstant_hip (ResNet block, SD
transformer block, FFN) with diffusers-layout weight upload.

These are the kernels behind the reference's fused-resnet.js
(runResNetBench :267), fused-block-full.js (runBlockBench :456) and
fused-block.js (runFFNBench :219) block chains, as callable ops on
device-resident NHWC fp16 activations.
"""
from __future__ import annotations

import ctypes

import numpy as np

from .device import Buffer, Device, call
from .unet import _geglu_join

_RES_FIELDS = ["norm1_gamma", "norm1_beta", "conv1_w", "conv1_b", "temb_w", "temb_b",
               "norm2_gamma", "norm2_beta", "conv2_w", "conv2_b", "skip_w", "skip_b"]
_TF_FIELDS = ["norm_gamma", "norm_beta", "proj_in_w", "proj_in_b", "ln1_gamma", "ln1_beta",
              "attn1_qkv_w", "attn1_out_w", "attn1_out_b", "ln2_gamma", "ln2_beta", "attn2_q_w",
              "attn2_kv_w", "attn2_out_w", "attn2_out_b", "ln3_gamma", "ln3_beta", "ff_in_w",
              "ff_in_b", "ff_out_w", "ff_out_b", "proj_out_w", "proj_out_b"]


class ResnetWeights(ctypes.Structure):
    """di_resnet_weights."""
    _fields_ = [(n, ctypes.c_uint64) for n in _RES_FIELDS]


class TransformerWeights(ctypes.Structure):
    """di_transformer_weights."""
    _fields_ = [(n, ctypes.c_uint64) for n in _TF_FIELDS]


class _Owned:
    """Keeps the uploaded weight buffers alive with their struct."""

    def __init__(self, struct, bufs):
        self.struct = struct
        self.bufs = bufs

    def destroy(self):
        for b in self.bufs:
            b.destroy()
        self.bufs = []


def _f16(a):
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16))


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def conv_ohwi(w):
    """OIHW -> OHWI fp16 (the implicit-GEMM weight layout)."""
    return _f16(np.asarray(w).transpose(0, 2, 3, 1))


def upload_resnet(dev: Device, sd: dict, p: str) -> _Owned:
    """Upload diffusers ResnetBlock2D weights `p.*` in the library layout."""
    bufs = []

    def put(a):
        b = dev.storage(a)
        bufs.append(b)
        return b.handle

    w = ResnetWeights()
    w.norm1_gamma, w.norm1_beta = put(_f32(sd[p + ".norm1.weight"])), put(_f32(sd[p + ".norm1.bias"]))
    w.conv1_w, w.conv1_b = put(conv_ohwi(sd[p + ".conv1.weight"])), put(_f32(sd[p + ".conv1.bias"]))
    if (p + ".time_emb_proj.weight") in sd:
        w.temb_w = put(_f16(sd[p + ".time_emb_proj.weight"]))
        w.temb_b = put(_f32(sd[p + ".time_emb_proj.bias"]))
    w.norm2_gamma, w.norm2_beta = put(_f32(sd[p + ".norm2.weight"])), put(_f32(sd[p + ".norm2.bias"]))
    w.conv2_w, w.conv2_b = put(conv_ohwi(sd[p + ".conv2.weight"])), put(_f32(sd[p + ".conv2.bias"]))
    if (p + ".conv_shortcut.weight") in sd:
        w.skip_w = put(_f16(np.asarray(sd[p + ".conv_shortcut.weight"])[:, :, 0, 0]))
        w.skip_b = put(_f32(sd[p + ".conv_shortcut.bias"]))
    return _Owned(w, bufs)


def upload_transformer(dev: Device, sd: dict, p: str) -> _Owned:
    """Upload diffusers Transformer2DModel weights `p.*` in the library layout."""
    bufs = []
    tb = p + ".transformer_blocks.0"

    def put(a):
        b = dev.storage(a)
        bufs.append(b)
        return b.handle

    w = TransformerWeights()
    w.norm_gamma, w.norm_beta = put(_f32(sd[p + ".norm.weight"])), put(_f32(sd[p + ".norm.bias"]))
    w.proj_in_w, w.proj_in_b = put(_f16(sd[p + ".proj_in.weight"])), put(_f32(sd[p + ".proj_in.bias"]))
    for k, (g, b) in {1: ("ln1_gamma", "ln1_beta"), 2: ("ln2_gamma", "ln2_beta"),
                      3: ("ln3_gamma", "ln3_beta")}.items():
        setattr(w, g, put(_f32(sd[f"{tb}.norm{k}.weight"])))
        setattr(w, b, put(_f32(sd[f"{tb}.norm{k}.bias"])))
    w.attn1_qkv_w = put(_f16(np.concatenate([sd[f"{tb}.attn1.to_{x}.weight"] for x in "qkv"], 0)))
    w.attn1_out_w = put(_f16(sd[tb + ".attn1.to_out.0.weight"]))
    w.attn1_out_b = put(_f32(sd[tb + ".attn1.to_out.0.bias"]))
    w.attn2_q_w = put(_f16(sd[tb + ".attn2.to_q.weight"]))
    w.attn2_kv_w = put(_f16(np.concatenate([sd[f"{tb}.attn2.to_{x}.weight"] for x in "kv"], 0)))
    w.attn2_out_w = put(_f16(sd[tb + ".attn2.to_out.0.weight"]))
    w.attn2_out_b = put(_f32(sd[tb + ".attn2.to_out.0.bias"]))
    ffw = np.asarray(sd[tb + ".ff.net.0.proj.weight"])
    ffb = np.asarray(sd[tb + ".ff.net.0.proj.bias"])
    w.ff_in_w = put(_f16(_geglu_join(*np.split(ffw, 2, axis=0))))
    w.ff_in_b = put(_f32(_geglu_join(*np.split(ffb, 2, axis=0))))
    w.ff_out_w = put(_f16(sd[tb + ".ff.net.2.weight"]))
    w.ff_out_b = put(_f32(sd[tb + ".ff.net.2.bias"]))
    w.proj_out_w = put(_f16(sd[p + ".proj_out.weight"]))
    w.proj_out_b = put(_f32(sd[p + ".proj_out.bias"]))
    return _Owned(w, bufs)


def resnet_block(dev: Device, w: _Owned, X: Buffer, temb: Buffer | None, Y: Buffer, B: int,
                 Cin: int, Cout: int, H: int, W: int, temb_dim: int = 1280, groups: int = 32,
                 eps: float = 1e-5):
    call("di_resnet_block", dev.ctx, ctypes.byref(w.struct), X.handle,
         temb.handle if temb is not None else 0, Y.handle, B, Cin, Cout, H, W, temb_dim, groups,
         eps)


def transformer_block(dev: Device, w: _Owned, X: Buffer, context: Buffer, Y: Buffer, B: int,
                      C: int, H: int, W: int, Sctx: int = 77, cross_dim: int = 1024,
                      groups: int = 32, gn_eps: float = 1e-6, ln_eps: float = 1e-5):
    call("di_transformer_block", dev.ctx, ctypes.byref(w.struct), X.handle, context.handle,
         Y.handle, B, C, H, W, Sctx, cross_dim, groups, gn_eps, ln_eps)
