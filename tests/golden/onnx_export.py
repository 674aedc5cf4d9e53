"""Real ONNX graphs for the executor tests, exported from torch modules with
torch's TorchScript exporter (opset 14, the opset whose LayerNorm, GELU and
attention exports are the decomposed chains the reference's executor runs).

The modules restate the SD2.1 U-Net's blocks as diffusers defines them
(ResnetBlock2D; Transformer2DModel with linear projection around a
BasicTransformerBlock: self-attention via scaled_dot_product_attention,
cross-attention, GEGLU feed-forward whose chunk is written as two slices, as
the SD-Turbo graph has it).  Weights are seeded; the expected outputs are the
same modules run in float64.

The ``onnx`` Python package is not installed in this image.  torch's exporter
needs it only to splice onnxscript functions into the finished proto, which
these graphs do not use, so that one step is replaced by the identity; the
proto bytes are torch's own C++ serialisation.
"""
from __future__ import annotations

import io
import math

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn


class Attention(nn.Module):
    """diffusers Attention with AttnProcessor2_0: no q/k/v bias, to_out bias."""

    def __init__(self, dim, ctx_dim, heads, head_dim):
        super().__init__()
        self.h, self.d = heads, head_dim
        inner = heads * head_dim
        self.to_q = nn.Linear(dim, inner, bias=False)
        self.to_k = nn.Linear(ctx_dim, inner, bias=False)
        self.to_v = nn.Linear(ctx_dim, inner, bias=False)
        self.to_out = nn.Linear(inner, dim)

    def forward(self, x, ctx=None):
        kv = x if ctx is None else ctx
        b = x.shape[0]
        q = self.to_q(x).reshape(b, -1, self.h, self.d).transpose(1, 2)
        k = self.to_k(kv).reshape(b, -1, self.h, self.d).transpose(1, 2)
        v = self.to_v(kv).reshape(b, -1, self.h, self.d).transpose(1, 2)
        o = F.scaled_dot_product_attention(q, k, v)
        return self.to_out(o.transpose(1, 2).reshape(b, -1, self.h * self.d))


class EagerAttention(Attention):
    """The same attention written out (MatMul, scale, Softmax, MatMul)."""

    def forward(self, x, ctx=None):
        kv = x if ctx is None else ctx
        b = x.shape[0]
        q = self.to_q(x).reshape(b, -1, self.h, self.d).transpose(1, 2)
        k = self.to_k(kv).reshape(b, -1, self.h, self.d).permute(0, 2, 3, 1)
        v = self.to_v(kv).reshape(b, -1, self.h, self.d).transpose(1, 2)
        p = torch.softmax(torch.matmul(q, k) * (1.0 / math.sqrt(self.d)), dim=-1)
        return self.to_out(torch.matmul(p, v).transpose(1, 2).reshape(b, -1, self.h * self.d))


class FeedForward(nn.Module):
    """GEGLU (dim -> 2 * inner, h * gelu(gate)) then inner -> dim."""

    def __init__(self, dim, mult=4):
        super().__init__()
        self.inner = dim * mult
        self.proj = nn.Linear(dim, 2 * self.inner)
        self.out = nn.Linear(self.inner, dim)

    def forward(self, x):
        p = self.proj(x)
        h, gate = p[..., :self.inner], p[..., self.inner:]
        return self.out(h * F.gelu(gate))


class Transformer2D(nn.Module):
    """Transformer2DModel, linear projection, one BasicTransformerBlock."""

    def __init__(self, C, ctx_dim, heads, head_dim, attn=Attention):
        super().__init__()
        self.norm = nn.GroupNorm(32, C, eps=1e-6)
        self.proj_in = nn.Linear(C, C)
        self.norm1, self.norm2, self.norm3 = nn.LayerNorm(C), nn.LayerNorm(C), nn.LayerNorm(C)
        self.attn1 = attn(C, C, heads, head_dim)
        self.attn2 = attn(C, ctx_dim, heads, head_dim)
        self.ff = FeedForward(C)
        self.proj_out = nn.Linear(C, C)

    def forward(self, x, ctx):
        b, c, h, w = x.shape
        r = x
        x = self.norm(x).permute(0, 2, 3, 1).reshape(b, h * w, c)
        x = self.proj_in(x)
        x = x + self.attn1(self.norm1(x))
        x = x + self.attn2(self.norm2(x), ctx)
        x = x + self.ff(self.norm3(x))
        x = self.proj_out(x).reshape(b, h, w, c).permute(0, 3, 1, 2)
        return x + r


class ResnetBlock2D(nn.Module):
    """GN -> SiLU -> conv3x3 -> + Linear(SiLU(temb)) -> GN -> SiLU -> conv3x3
    -> + conv1x1 shortcut (Cin != Cout)."""

    def __init__(self, cin, cout, temb_dim):
        super().__init__()
        self.norm1 = nn.GroupNorm(32, cin, eps=1e-5)
        self.conv1 = nn.Conv2d(cin, cout, 3, padding=1)
        self.time_emb_proj = nn.Linear(temb_dim, cout)
        self.norm2 = nn.GroupNorm(32, cout, eps=1e-5)
        self.conv2 = nn.Conv2d(cout, cout, 3, padding=1)
        self.conv_shortcut = nn.Conv2d(cin, cout, 1)

    def forward(self, x, temb):
        h = self.conv1(F.silu(self.norm1(x)))
        h = h + self.time_emb_proj(F.silu(temb))[:, :, None, None]
        h = self.conv2(F.silu(self.norm2(h)))
        return self.conv_shortcut(x) + h


class VAEResnet(nn.Module):
    """The VAE decoder's ResnetBlock2D: no time embedding, eps 1e-6."""

    def __init__(self, cin, cout):
        super().__init__()
        self.norm1 = nn.GroupNorm(32, cin, eps=1e-6)
        self.conv1 = nn.Conv2d(cin, cout, 3, padding=1)
        self.norm2 = nn.GroupNorm(32, cout, eps=1e-6)
        self.conv2 = nn.Conv2d(cout, cout, 3, padding=1)
        self.conv_shortcut = nn.Conv2d(cin, cout, 1) if cin != cout else None

    def forward(self, x):
        h = self.conv1(F.silu(self.norm1(x)))
        h = self.conv2(F.silu(self.norm2(h)))
        return (x if self.conv_shortcut is None else self.conv_shortcut(x)) + h


class VAEAttention(nn.Module):
    """The mid-block attention: GroupNorm, one head over all channels,
    residual."""

    def __init__(self, C):
        super().__init__()
        self.group_norm = nn.GroupNorm(32, C, eps=1e-6)
        self.to_q, self.to_k, self.to_v = nn.Linear(C, C), nn.Linear(C, C), nn.Linear(C, C)
        self.to_out = nn.Linear(C, C)

    def forward(self, x):
        b, c, h, w = x.shape
        t = self.group_norm(x).reshape(b, c, h * w).transpose(1, 2)
        q, k, v = (f(t).unsqueeze(1) for f in (self.to_q, self.to_k, self.to_v))
        o = F.scaled_dot_product_attention(q, k, v).squeeze(1)
        return self.to_out(o).transpose(1, 2).reshape(b, c, h, w) + x


class VAEDecoder(nn.Module):
    """AutoencoderKL's post_quant_conv + Decoder as SD uses them: conv_in,
    mid (ResNet, attention, ResNet), four up blocks of three ResNets with a
    nearest-x2 + conv3x3 upsampler on all but the last, GroupNorm, SiLU,
    conv_out to RGB.  channels = block_out_channels (SD: 128, 256, 512,
    512)."""

    def __init__(self, channels=(128, 256, 512, 512), latent=4):
        super().__init__()
        rev = list(reversed(channels))
        self.post_quant_conv = nn.Conv2d(latent, latent, 1)
        self.conv_in = nn.Conv2d(latent, rev[0], 3, padding=1)
        self.mid = nn.ModuleList([VAEResnet(rev[0], rev[0]), VAEAttention(rev[0]),
                                  VAEResnet(rev[0], rev[0])])
        self.ups = nn.ModuleList()
        self.upconvs = nn.ModuleList()
        prev = rev[0]
        for i, c in enumerate(rev):
            self.ups.append(nn.ModuleList([VAEResnet(prev if j == 0 else c, c) for j in range(3)]))
            self.upconvs.append(nn.Conv2d(c, c, 3, padding=1) if i < len(rev) - 1 else
                                nn.Identity())
            prev = c
        self.norm_out = nn.GroupNorm(32, rev[-1], eps=1e-6)
        self.conv_out = nn.Conv2d(rev[-1], 3, 3, padding=1)

    def forward(self, z):
        h = self.conv_in(self.post_quant_conv(z))
        for m in self.mid:
            h = m(h)
        for i, blocks in enumerate(self.ups):
            for m in blocks:
                h = m(h)
            if i < len(self.ups) - 1:
                h = self.upconvs[i](F.interpolate(h, scale_factor=2.0, mode="nearest"))
        return self.conv_out(F.silu(self.norm_out(h)))


def _seeded(module: nn.Module, seed: int) -> nn.Module:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.endswith("bias"):
                p.copy_(0.02 * torch.randn(p.shape, generator=g))
            elif p.dim() == 1:  # norm scales
                p.copy_(1 + 0.05 * torch.randn(p.shape, generator=g))
            else:
                fan_in = int(np.prod(p.shape[1:]))
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(fan_in))
    return module.eval()


def export(module: nn.Module, args, input_names, output_name="y", opset: int = 14) -> bytes:
    from torch.onnx._internal.torchscript_exporter import onnx_proto_utils, utils
    keep = onnx_proto_utils._add_onnxscript_fn
    onnx_proto_utils._add_onnxscript_fn = lambda proto, custom_opsets: proto
    try:
        f = io.BytesIO()
        with torch.no_grad():
            utils.export(module, args, f, opset_version=opset, do_constant_folding=True,
                         input_names=list(input_names), output_names=[output_name])
        return f.getvalue()
    finally:
        onnx_proto_utils._add_onnxscript_fn = keep


def _expected(module: nn.Module, args):
    m64 = module.double()
    with torch.no_grad():
        y = m64(*[a.double() for a in args])
    module.float()
    return y.numpy().astype(np.float32)


def transformer_case(C=128, heads=2, head_dim=64, H=8, W=8, Sctx=77, ctx_dim=96, seed=0,
                     eager=False):
    """(onnx bytes, {input name: array}, expected output) for Transformer2D."""
    m = _seeded(Transformer2D(C, ctx_dim, heads, head_dim,
                              EagerAttention if eager else Attention), seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(1, C, H, W, generator=g)
    ctx = torch.randn(1, Sctx, ctx_dim, generator=g)
    data = export(m, (x, ctx), ("x", "ctx"))
    return data, {"x": x.numpy(), "ctx": ctx.numpy()}, _expected(m, (x, ctx))


def resnet_case(cin=64, cout=128, H=8, W=8, temb_dim=256, seed=0):
    """(onnx bytes, {input name: array}, expected output) for ResnetBlock2D."""
    m = _seeded(ResnetBlock2D(cin, cout, temb_dim), seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(1, cin, H, W, generator=g)
    t = torch.randn(1, temb_dim, generator=g)
    data = export(m, (x, t), ("x", "temb"))
    return data, {"x": x.numpy(), "temb": t.numpy()}, _expected(m, (x, t))


def vae_case(channels=(32, 32, 64, 64), latent_hw=8, seed=0, expected=True):
    """(onnx bytes, {"latent": array}, expected image or None) for the VAE
    decoder; SD's decoder is channels (128, 256, 512, 512) at latent 64x64."""
    m = _seeded(VAEDecoder(channels), seed)
    g = torch.Generator().manual_seed(seed + 1)
    z = torch.randn(1, 4, latent_hw, latent_hw, generator=g)
    data = export(m, (z,), ("latent",), output_name="sample")
    return data, {"latent": z.numpy()}, (_expected(m, (z,)) if expected else None)
