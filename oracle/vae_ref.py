"""Reference composition of SD's VAE decoder (TEST INFRASTRUCTURE ONLY).

AutoencoderKL's decode path as the reference runs it from
vae_decoder/model.onnx (vae-wgsl.js:94-140): latent * scale ->
post_quant_conv (1x1) -> Decoder (conv_in; mid block ResNet, one-head
attention over all channels with a GroupNorm in front and a residual,
ResNet; four up blocks of layers_per_block + 1 ResNets, the first three
followed by nearest x2 upsampling and a conv3x3; GroupNorm + SiLU; conv_out).
Every GroupNorm uses eps 1e-6 and 32 groups; ResNets carry no time
embedding.  Written against the op interface of ``unet_ref`` so it runs on
the C oracle (``OracleOps``) or torch (``TorchOps``); parameters are
diffusers-named, diffusers-layout float32 arrays
(``drawinstant.vae.VAE.state_dict``).
"""
from __future__ import annotations

import math

import numpy as np

from .unet_ref import resnet


def attention(ops, sd, p, x, groups, eps):
    """diffusers Attention of the VAE mid block (heads 1, biases on q/k/v)."""
    b, c, h, w = x.shape
    t = ops.to_tokens(ops.gn(x, sd[p + ".group_norm.weight"], sd[p + ".group_norm.bias"], groups,
                             eps, False))
    q, k, v = (ops.linear(t, sd[f"{p}.{n}.weight"], sd[f"{p}.{n}.bias"])[:, None]
               for n in ("to_q", "to_k", "to_v"))
    o = ops.attn(q, k, v)[:, 0]
    o = ops.linear(o, sd[p + ".to_out.0.weight"], sd[p + ".to_out.0.bias"])
    return ops.from_tokens(o, h, w) + x


def vae_decode(ops, sd, cfg: dict, z, scale: float):
    """latent [B, C, H, W] -> image [B, out, 8H, 8W]."""
    g, eps, L = cfg["groups"], cfg["eps"], cfg["layers_per_block"]
    h = ops.conv(z * scale, sd["post_quant_conv.weight"], sd["post_quant_conv.bias"], pad=0)
    h = ops.conv(h, sd["decoder.conv_in.weight"], sd["decoder.conv_in.bias"])
    m = "decoder.mid_block"
    h = resnet(ops, sd, m + ".resnets.0", h, None, eps, g)
    h = attention(ops, sd, m + ".attentions.0", h, g, eps)
    h = resnet(ops, sd, m + ".resnets.1", h, None, eps, g)
    for i in range(4):
        for j in range(L + 1):
            h = resnet(ops, sd, f"decoder.up_blocks.{i}.resnets.{j}", h, None, eps, g)
        if i < 3:
            p = f"decoder.up_blocks.{i}.upsamplers.0.conv"
            h = ops.conv(ops.up2(h), sd[p + ".weight"], sd[p + ".bias"])
    h = ops.gn(h, sd["decoder.conv_norm_out.weight"], sd["decoder.conv_norm_out.bias"], g, eps,
               True)
    return ops.conv(h, sd["decoder.conv_out.weight"], sd["decoder.conv_out.bias"])


def vae_param_shapes(cfg: dict) -> dict:
    L, lat, out = cfg["layers_per_block"], cfg["latent_channels"], cfg["out_channels"]
    rev = list(reversed(cfg["block_channels"]))
    s = {"post_quant_conv.weight": (lat, lat, 1, 1), "post_quant_conv.bias": (lat,)}

    def conv(p, ci, co, k):
        s[p + ".weight"] = (co, ci, k, k)
        s[p + ".bias"] = (co,)

    def norm(p, c):
        s[p + ".weight"] = (c,)
        s[p + ".bias"] = (c,)

    def res(p, ci, co):
        norm(p + ".norm1", ci)
        conv(p + ".conv1", ci, co, 3)
        norm(p + ".norm2", co)
        conv(p + ".conv2", co, co, 3)
        if ci != co:
            conv(p + ".conv_shortcut", ci, co, 1)

    conv("decoder.conv_in", lat, rev[0], 3)
    m = "decoder.mid_block"
    res(m + ".resnets.0", rev[0], rev[0])
    a = m + ".attentions.0"
    norm(a + ".group_norm", rev[0])
    for n in ("to_q", "to_k", "to_v", "to_out.0"):
        s[f"{a}.{n}.weight"] = (rev[0], rev[0])
        s[f"{a}.{n}.bias"] = (rev[0],)
    res(m + ".resnets.1", rev[0], rev[0])
    prev = rev[0]
    for i, c in enumerate(rev):
        for j in range(L + 1):
            res(f"decoder.up_blocks.{i}.resnets.{j}", prev if j == 0 else c, c)
        if i < 3:
            conv(f"decoder.up_blocks.{i}.upsamplers.0.conv", c, c, 3)
        prev = c
    norm("decoder.conv_norm_out", rev[-1])
    conv("decoder.conv_out", rev[-1], out, 3)
    return s


def random_state_dict(cfg: dict, seed: int = 0) -> dict:
    """Seeded weights (Kaiming convs, 1/sqrt(fan_in) linears, N(1, .02) /
    N(0, .02) norms, N(0, .01) biases), rounded through fp16 so the library's
    fp16 weights hold them exactly."""
    rng = np.random.default_rng(seed)
    sd = {}
    for name, shp in vae_param_shapes(cfg).items():
        if len(shp) == 4:
            a = rng.standard_normal(shp) * math.sqrt(2.0 / (shp[1] * shp[2] * shp[3]))
        elif len(shp) == 2:
            a = rng.standard_normal(shp) / math.sqrt(shp[1])
        elif "norm" in name and name.endswith(".weight"):
            a = 1.0 + 0.02 * rng.standard_normal(shp)
        elif "norm" in name:
            a = 0.02 * rng.standard_normal(shp)
        else:
            a = 0.01 * rng.standard_normal(shp)
        sd[name] = a.astype(np.float16).astype(np.float32)
    return sd


def small_config() -> dict:
    return {"latent_channels": 4, "out_channels": 3, "block_channels": [32, 32, 64, 64],
            "layers_per_block": 2, "groups": 32, "eps": 1e-6}


def sd_config() -> dict:
    c = small_config()
    c["block_channels"] = [128, 256, 512, 512]
    return c
