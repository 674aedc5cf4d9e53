"""Reference compositions of the SD2.1 U-Net blocks (TEST INFRASTRUCTURE ONLY).

ResnetBlock2D, Transformer2DModel (linear projection, one
BasicTransformerBlock with GEGLU), Down/Upsample2D, the timestep embedding
and the full UNet2DConditionModel forward, written once against a small op
interface and run on one of two backends:

  * ``OracleOps`` - the plain-C oracle (oracle.c, fp64 accumulation, NCHW):
    the CPU parity checker for block- and small-U-Net-sized cases;
  * ``TorchOps`` - torch.nn.functional in float32 on any device: the
    reference for the full-size SD2.1 step on the GPU box (a floating-point
    path, checked with rel-L2), whose primitives are the same library
    routines test_oracle.py pins the C oracle against.

Semantics follow diffusers' UNet2DConditionModel as the reference executor
runs it from the SD-Turbo ONNX graph (unet-wgsl.js:145-195): GN eps 1e-5 in
ResNets, 1e-6 in transformers, LN eps 1e-5, attention scale 1/sqrt(64),
timestep sinusoid [cos || sin] (fused-tembed.js:36-42), GEGLU
h * GELU(gate) on a last-dim chunk.  Parameters are diffusers-named,
diffusers-layout float32 arrays (``drawinstant.unet.UNet.state_dict``).

Pinned (tests/test_unet_composition.py) against an independent module-form
UNet2DConditionModel with diffusers' module tree and names
(tests/golden/unet_module.py) in float64 on the same weights: rel-L2 < 1e-5
for the whole step on both backends' configs, < 1e-6 per ResNet and
transformer block; planted wiring mistakes (skip concat order, an unflipped
[sin || cos] sinusoid, moved cross-attention levels) fail that comparison.
"""
from __future__ import annotations

import math

import numpy as np

import oracle


class OracleOps:
    """NCHW numpy arrays through the C oracle."""

    def conv(self, x, w, b, stride=1, pad=None):
        return oracle.conv2d(x, w, b, stride=stride, pad=pad)

    def gn(self, x, g, b, groups, eps, silu):
        return oracle.group_norm(x, g, b, groups, eps=eps, silu=silu)

    def ln(self, x, g, b, eps):
        return oracle.layer_norm(x, g, b, eps=eps)

    def linear(self, x, w, b=None):
        return oracle.linear(x, w, b)

    def silu(self, x):
        return oracle.unary("SiLU", x)

    def gelu(self, x):
        return oracle.unary("GELU", x)

    def attn(self, q, k, v):  # [B, H, S, d]
        return oracle.attention(q, k, v, layout="bhsd")

    def up2(self, x):
        return x.repeat(2, axis=2).repeat(2, axis=3)

    def cat(self, xs, axis):
        return np.concatenate(xs, axis=axis)

    def sinusoid(self, t, dim):
        half = dim // 2
        f = np.exp(-math.log(10000.0) * np.arange(half, dtype=np.float64) / half)
        a = np.asarray(t, np.float64)[:, None] * f[None, :]
        return np.concatenate([np.cos(a), np.sin(a)], axis=1).astype(np.float32)

    def to_tokens(self, x):  # [B,C,H,W] -> [B,HW,C]
        b, c, h, w = x.shape
        return np.ascontiguousarray(x.reshape(b, c, h * w).transpose(0, 2, 1))

    def from_tokens(self, t, h, w):
        b, s, c = t.shape
        return np.ascontiguousarray(t.transpose(0, 2, 1).reshape(b, c, h, w))

    def heads(self, t, n):  # [B,S,C] -> [B,n,S,C/n]
        b, s, c = t.shape
        return np.ascontiguousarray(t.reshape(b, s, n, c // n).transpose(0, 2, 1, 3))

    def merge(self, t):  # [B,n,S,d] -> [B,S,n*d]
        b, n, s, d = t.shape
        return np.ascontiguousarray(t.transpose(0, 2, 1, 3).reshape(b, s, n * d))

    def chunk2(self, t):
        a, b = np.split(t, 2, axis=-1)
        return np.ascontiguousarray(a), np.ascontiguousarray(b)

    def asarray(self, a):
        return np.ascontiguousarray(a, np.float32)


class TorchOps:
    """float32 torch.nn.functional on `device` (reference for full-size runs)."""

    def __init__(self, device="cuda"):
        import torch
        import torch.nn.functional as F
        self.t, self.F, self.device = torch, F, device

    def asarray(self, a):
        return self.t.as_tensor(np.asarray(a, np.float32), device=self.device)

    def conv(self, x, w, b, stride=1, pad=None):
        k = w.shape[-1]
        return self.F.conv2d(x, w, b, stride=stride, padding=(k - 1) // 2 if pad is None else pad)

    def gn(self, x, g, b, groups, eps, silu):
        y = self.F.group_norm(x, groups, g, b, eps)
        return self.F.silu(y) if silu else y

    def ln(self, x, g, b, eps):
        return self.F.layer_norm(x, (x.shape[-1],), g, b, eps)

    def linear(self, x, w, b=None):
        return self.F.linear(x, w, b)

    def silu(self, x):
        return self.F.silu(x)

    def gelu(self, x):
        return self.F.gelu(x)

    def attn(self, q, k, v):
        # float32 attention (math path), contiguous operands
        return self.F.scaled_dot_product_attention(q.contiguous(), k.contiguous(), v.contiguous())

    def up2(self, x):
        return self.F.interpolate(x, scale_factor=2.0, mode="nearest")

    def cat(self, xs, axis):
        return self.t.cat(xs, dim=axis)

    def sinusoid(self, t, dim):
        half = dim // 2
        f = np.exp(-math.log(10000.0) * np.arange(half, dtype=np.float64) / half)
        a = np.asarray(t, np.float64)[:, None] * f[None, :]
        return self.asarray(np.concatenate([np.cos(a), np.sin(a)], axis=1))

    def to_tokens(self, x):
        b, c, h, w = x.shape
        return x.reshape(b, c, h * w).transpose(1, 2).contiguous()

    def from_tokens(self, t, h, w):
        b, s, c = t.shape
        return t.transpose(1, 2).reshape(b, c, h, w).contiguous()

    def heads(self, t, n):
        b, s, c = t.shape
        return t.reshape(b, s, n, c // n).transpose(1, 2).contiguous()

    def merge(self, t):
        b, n, s, d = t.shape
        return t.transpose(1, 2).reshape(b, s, n * d).contiguous()

    def chunk2(self, t):
        a, b = t.chunk(2, dim=-1)
        return a.contiguous(), b.contiguous()


def resnet(ops, sd, p, x, temb_silu, eps=1e-5, groups=32):
    """diffusers ResnetBlock2D (output_scale_factor 1)."""
    h = ops.gn(x, sd[p + ".norm1.weight"], sd[p + ".norm1.bias"], groups, eps, True)
    h = ops.conv(h, sd[p + ".conv1.weight"], sd[p + ".conv1.bias"])
    if temb_silu is not None:
        t = ops.linear(temb_silu, sd[p + ".time_emb_proj.weight"], sd[p + ".time_emb_proj.bias"])
        h = h + t[:, :, None, None]
    h = ops.gn(h, sd[p + ".norm2.weight"], sd[p + ".norm2.bias"], groups, eps, True)
    h = ops.conv(h, sd[p + ".conv2.weight"], sd[p + ".conv2.bias"])
    if (p + ".conv_shortcut.weight") in sd:
        x = ops.conv(x, sd[p + ".conv_shortcut.weight"], sd[p + ".conv_shortcut.bias"], pad=0)
    return x + h


def attention(ops, sd, p, x, ctx, heads):
    """diffusers Attention (no q/k/v bias, to_out.0 with bias)."""
    kv = x if ctx is None else ctx
    q = ops.heads(ops.linear(x, sd[p + ".to_q.weight"]), heads)
    k = ops.heads(ops.linear(kv, sd[p + ".to_k.weight"]), heads)
    v = ops.heads(ops.linear(kv, sd[p + ".to_v.weight"]), heads)
    o = ops.merge(ops.attn(q, k, v))
    return ops.linear(o, sd[p + ".to_out.0.weight"], sd[p + ".to_out.0.bias"])


def transformer(ops, sd, p, x, ctx, gn_eps=1e-6, ln_eps=1e-5, groups=32, head_dim=64):
    """diffusers Transformer2DModel, use_linear_projection=True, 1 block."""
    b, c, h, w = x.shape
    heads = c // head_dim
    t = ops.gn(x, sd[p + ".norm.weight"], sd[p + ".norm.bias"], groups, gn_eps, False)
    t = ops.linear(ops.to_tokens(t), sd[p + ".proj_in.weight"], sd[p + ".proj_in.bias"])
    tb = p + ".transformer_blocks.0"
    n = ops.ln(t, sd[tb + ".norm1.weight"], sd[tb + ".norm1.bias"], ln_eps)
    t = attention(ops, sd, tb + ".attn1", n, None, heads) + t
    n = ops.ln(t, sd[tb + ".norm2.weight"], sd[tb + ".norm2.bias"], ln_eps)
    t = attention(ops, sd, tb + ".attn2", n, ctx, heads) + t
    n = ops.ln(t, sd[tb + ".norm3.weight"], sd[tb + ".norm3.bias"], ln_eps)
    hg = ops.linear(n, sd[tb + ".ff.net.0.proj.weight"], sd[tb + ".ff.net.0.proj.bias"])
    hid, gate = ops.chunk2(hg)
    t = ops.linear(hid * ops.gelu(gate), sd[tb + ".ff.net.2.weight"], sd[tb + ".ff.net.2.bias"]) + t
    t = ops.linear(t, sd[p + ".proj_out.weight"], sd[p + ".proj_out.bias"])
    return ops.from_tokens(t, h, w) + x


def time_embedding(ops, sd, t, dim):
    e = ops.sinusoid(t, dim)
    e = ops.silu(ops.linear(e, sd["time_embedding.linear_1.weight"], sd["time_embedding.linear_1.bias"]))
    return ops.linear(e, sd["time_embedding.linear_2.weight"], sd["time_embedding.linear_2.bias"])


def unet_forward(ops, sd, cfg: dict, sample, t, ctx):
    """UNet2DConditionModel.forward -> out_sample (NCHW)."""
    sd = {k: ops.asarray(v) for k, v in sd.items()}
    sample, ctx = ops.asarray(sample), ops.asarray(ctx)
    G, L = cfg["groups"], cfg["layers_per_block"]
    ch, xattn = cfg["block_channels"], cfg["cross_attn"]
    temb = time_embedding(ops, sd, t, ch[0])
    ts = ops.silu(temb)
    h = ops.conv(sample, sd["conv_in.weight"], sd["conv_in.bias"])
    skips = [h]
    for i in range(4):
        for j in range(L):
            h = resnet(ops, sd, f"down_blocks.{i}.resnets.{j}", h, ts, cfg["resnet_eps"], G)
            if xattn[i]:
                h = transformer(ops, sd, f"down_blocks.{i}.attentions.{j}", h, ctx,
                                cfg["transformer_gn_eps"], cfg["ln_eps"], G)
            skips.append(h)
        if i < 3:
            h = ops.conv(h, sd[f"down_blocks.{i}.downsamplers.0.conv.weight"],
                         sd[f"down_blocks.{i}.downsamplers.0.conv.bias"], stride=2, pad=1)
            skips.append(h)
    h = resnet(ops, sd, "mid_block.resnets.0", h, ts, cfg["resnet_eps"], G)
    h = transformer(ops, sd, "mid_block.attentions.0", h, ctx, cfg["transformer_gn_eps"],
                    cfg["ln_eps"], G)
    h = resnet(ops, sd, "mid_block.resnets.1", h, ts, cfg["resnet_eps"], G)
    for i in range(4):
        for j in range(L + 1):
            h = ops.cat([h, skips.pop()], 1)
            h = resnet(ops, sd, f"up_blocks.{i}.resnets.{j}", h, ts, cfg["resnet_eps"], G)
            if xattn[3 - i]:
                h = transformer(ops, sd, f"up_blocks.{i}.attentions.{j}", h, ctx,
                                cfg["transformer_gn_eps"], cfg["ln_eps"], G)
        if i < 3:
            h = ops.conv(ops.up2(h), sd[f"up_blocks.{i}.upsamplers.0.conv.weight"],
                         sd[f"up_blocks.{i}.upsamplers.0.conv.bias"])
    h = ops.gn(h, sd["conv_norm_out.weight"], sd["conv_norm_out.bias"], G, cfg["resnet_eps"], True)
    return ops.conv(h, sd["conv_out.weight"], sd["conv_out.bias"])


def sd21_param_count() -> int:
    """Closed-form parameter count of diffusers' SD2.1 UNet2DConditionModel,
    summed module by module (independent of the library's registry)."""
    def conv(ci, co, k):
        return co * ci * k * k + co

    def lin(i, o, bias=True):
        return i * o + (o if bias else 0)

    def norm(c):
        return 2 * c

    def res(ci, co, temb=1280):
        n = norm(ci) + conv(ci, co, 3) + lin(temb, co) + norm(co) + conv(co, co, 3)
        return n + (conv(ci, co, 1) if ci != co else 0)

    def tf(c, cross=1024):
        attn1 = 3 * lin(c, c, False) + lin(c, c)
        attn2 = lin(c, c, False) + 2 * lin(cross, c, False) + lin(c, c)
        ff = lin(c, 8 * c) + lin(4 * c, c)
        return norm(c) + lin(c, c) + 3 * norm(c) + attn1 + attn2 + ff + lin(c, c)

    ch = [320, 640, 1280, 1280]
    n = conv(4, 320, 3) + lin(320, 1280) + lin(1280, 1280)
    cin = 320
    for i in range(4):
        for j in range(2):
            n += res(cin if j == 0 else ch[i], ch[i])
            if i < 3:
                n += tf(ch[i])
        cin = ch[i]
        if i < 3:
            n += conv(ch[i], ch[i], 3)
    n += 2 * res(1280, 1280) + tf(1280)
    rev = ch[::-1]
    prev = 1280
    for i in range(4):
        out, inp = rev[i], rev[min(i + 1, 3)]
        for j in range(3):
            skip = inp if j == 2 else out
            n += res((prev if j == 0 else out) + skip, out)
            if i > 0:
                n += tf(out)
        prev = out
        if i < 3:
            n += conv(out, out, 3)
    return n + norm(320) + conv(320, 4, 3)


def unet_param_shapes(cfg: dict) -> dict:
    """diffusers parameter names -> logical shapes for a UNet2DConditionModel
    config (SD2.1 layout family), derived from the module definitions."""
    S = {}
    ch, xattn, L = cfg["block_channels"], cfg["cross_attn"], cfg["layers_per_block"]
    X, T = cfg["cross_dim"], cfg["time_dim"]

    def conv(p, ci, co, k):
        S[p + ".weight"] = (co, ci, k, k)
        S[p + ".bias"] = (co,)

    def lin(p, i, o, bias=True):
        S[p + ".weight"] = (o, i)
        if bias:
            S[p + ".bias"] = (o,)

    def norm(p, c):
        S[p + ".weight"] = (c,)
        S[p + ".bias"] = (c,)

    def res(p, ci, co):
        norm(p + ".norm1", ci)
        conv(p + ".conv1", ci, co, 3)
        lin(p + ".time_emb_proj", T, co)
        norm(p + ".norm2", co)
        conv(p + ".conv2", co, co, 3)
        if ci != co:
            conv(p + ".conv_shortcut", ci, co, 1)

    def tf(p, c):
        tb = p + ".transformer_blocks.0"
        norm(p + ".norm", c)
        lin(p + ".proj_in", c, c)
        for k in (1, 2, 3):
            norm(f"{tb}.norm{k}", c)
        for a, kv in (("attn1", c), ("attn2", X)):
            lin(f"{tb}.{a}.to_q", c, c, False)
            lin(f"{tb}.{a}.to_k", kv, c, False)
            lin(f"{tb}.{a}.to_v", kv, c, False)
            lin(f"{tb}.{a}.to_out.0", c, c)
        lin(tb + ".ff.net.0.proj", c, 8 * c)
        lin(tb + ".ff.net.2", 4 * c, c)
        lin(p + ".proj_out", c, c)

    conv("conv_in", cfg["in_channels"], ch[0], 3)
    lin("time_embedding.linear_1", ch[0], T)
    lin("time_embedding.linear_2", T, T)
    cin = ch[0]
    for i in range(4):
        for j in range(L):
            res(f"down_blocks.{i}.resnets.{j}", cin if j == 0 else ch[i], ch[i])
            if xattn[i]:
                tf(f"down_blocks.{i}.attentions.{j}", ch[i])
        cin = ch[i]
        if i < 3:
            conv(f"down_blocks.{i}.downsamplers.0.conv", ch[i], ch[i], 3)
    res("mid_block.resnets.0", ch[3], ch[3])
    tf("mid_block.attentions.0", ch[3])
    res("mid_block.resnets.1", ch[3], ch[3])
    rev = ch[::-1]
    prev = ch[3]
    for i in range(4):
        out, inp = rev[i], rev[min(i + 1, 3)]
        for j in range(L + 1):
            skip = inp if j == L else out
            res(f"up_blocks.{i}.resnets.{j}", (prev if j == 0 else out) + skip, out)
            if xattn[3 - i]:
                tf(f"up_blocks.{i}.attentions.{j}", out)
        prev = out
        if i < 3:
            conv(f"up_blocks.{i}.upsamplers.0.conv", out, out, 3)
    norm("conv_norm_out", ch[0])
    conv("conv_out", ch[0], cfg["out_channels"], 3)
    return S


def random_state_dict(cfg: dict, seed: int = 0) -> dict:
    """Seeded random weights with the library's init families (Kaiming convs,
    Xavier linears, N(1, .02) / N(0, .02) norms, N(0, .01) biases)."""
    rng = np.random.default_rng(seed)
    sd = {}
    for name, shp in unet_param_shapes(cfg).items():
        if len(shp) == 4:
            std = math.sqrt(2.0 / (shp[1] * shp[2] * shp[3]))
            a = rng.standard_normal(shp) * std
        elif len(shp) == 2:
            a = rng.standard_normal(shp) * math.sqrt(2.0 / (shp[0] + shp[1]))
        elif "norm" in name and name.endswith(".weight"):
            a = 1.0 + 0.02 * rng.standard_normal(shp)
        elif "norm" in name:
            a = 0.02 * rng.standard_normal(shp)
        else:
            a = 0.01 * rng.standard_normal(shp)
        sd[name] = a.astype(np.float16).astype(np.float32)
    return sd


def small_config() -> dict:
    return {"in_channels": 4, "out_channels": 4, "block_channels": [64, 128, 256, 256],
            "cross_attn": [1, 1, 1, 0], "layers_per_block": 2, "cross_dim": 256,
            "time_dim": 256, "groups": 32, "resnet_eps": 1e-5, "transformer_gn_eps": 1e-6,
            "ln_eps": 1e-5}


def sd21_config() -> dict:
    c = small_config()
    c.update(block_channels=[320, 640, 1280, 1280], cross_dim=1024, time_dim=1280)
    return c
