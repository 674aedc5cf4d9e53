"""Module-form SD2.1 UNet2DConditionModel (TEST INFRASTRUCTURE ONLY).

An independent restatement of diffusers' UNet2DConditionModel as SD2.1 /
SD-Turbo configure it, written as torch modules with diffusers' own module
tree, so its ``state_dict()`` keys are diffusers' parameter names:

* ``Timesteps(320, flip_sin_to_cos=True, downscale_freq_shift=0)``: the
  sinusoid is built as [sin || cos] and then flipped, as diffusers'
  ``get_timestep_embedding`` does, not written directly as [cos || sin];
* ``TimestepEmbedding``: linear_1 -> SiLU -> linear_2;
* down blocks ``CrossAttnDownBlock2D`` x 3 + ``DownBlock2D``, each returning
  its per-layer outputs as a tuple that the U-Net concatenates onto
  ``down_block_res_samples`` (which starts with conv_in's output);
* ``UNetMidBlock2DCrossAttn``: resnet, then (attention, resnet) pairs;
* up blocks ``UpBlock2D`` + ``CrossAttnUpBlock2D`` x 3, each taking the last
  ``len(resnets)`` entries of the skip tuple and consuming them from the end;
  channel bookkeeping (prev_output_channel / in_channels / res_skip_channels)
  as diffusers' constructors compute it;
* ``ResnetBlock2D`` (groups 32, eps 1e-5, 1x1 ``conv_shortcut`` only when
  channels change, output scale 1), ``Downsample2D`` (3x3 stride 2 pad 1) and
  ``Upsample2D`` (nearest x2 then 3x3);
* ``Transformer2DModel`` with linear projection (GroupNorm eps 1e-6) around
  one ``BasicTransformerBlock`` (LayerNorm eps 1e-5; self-attention,
  cross-attention, GEGLU ``FeedForward`` whose ``net`` is
  [GEGLU, Dropout, Linear] and ``to_out`` is [Linear, Dropout]).

The library's U-Net and the oracle's composition (oracle/unet_ref.py) are
pinned against this module on the same weights; it shares no code with
either.  ``forward`` takes the timestep as an int64 tensor, as the SD-Turbo
ONNX graph does (unet.js:13-19), and ``half_io`` wraps it in the fp32-in /
fp16-inside / fp32-out form of that graph for ONNX export.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn


def get_timestep_embedding(timesteps, dim, flip_sin_to_cos=True, downscale_freq_shift=0.0,
                           max_period=10000.0):
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(half, dtype=torch.float32,
                                                    device=timesteps.device)
    exponent = exponent / (half - downscale_freq_shift)
    emb = timesteps[:, None].float() * torch.exp(exponent)[None, :]
    emb = torch.cat([torch.sin(emb), torch.cos(emb)], dim=-1)
    if flip_sin_to_cos:
        emb = torch.cat([emb[:, half:], emb[:, :half]], dim=-1)
    return emb


class TimestepEmbedding(nn.Module):
    def __init__(self, in_channels, time_embed_dim):
        super().__init__()
        self.linear_1 = nn.Linear(in_channels, time_embed_dim)
        self.act = nn.SiLU()
        self.linear_2 = nn.Linear(time_embed_dim, time_embed_dim)

    def forward(self, sample):
        return self.linear_2(self.act(self.linear_1(sample)))


class ResnetBlock2D(nn.Module):
    def __init__(self, in_channels, out_channels, temb_channels, groups=32, eps=1e-5):
        super().__init__()
        self.norm1 = nn.GroupNorm(groups, in_channels, eps=eps, affine=True)
        self.conv1 = nn.Conv2d(in_channels, out_channels, 3, stride=1, padding=1)
        self.time_emb_proj = nn.Linear(temb_channels, out_channels)
        self.norm2 = nn.GroupNorm(groups, out_channels, eps=eps, affine=True)
        self.dropout = nn.Dropout(0.0)
        self.conv2 = nn.Conv2d(out_channels, out_channels, 3, stride=1, padding=1)
        self.nonlinearity = nn.SiLU()
        self.use_in_shortcut = in_channels != out_channels
        self.conv_shortcut = (nn.Conv2d(in_channels, out_channels, 1, stride=1, padding=0)
                              if self.use_in_shortcut else None)

    def forward(self, input_tensor, temb):
        hidden = self.nonlinearity(self.norm1(input_tensor))
        hidden = self.conv1(hidden)
        temb = self.time_emb_proj(self.nonlinearity(temb))[:, :, None, None]
        hidden = hidden + temb
        hidden = self.nonlinearity(self.norm2(hidden))
        hidden = self.conv2(self.dropout(hidden))
        if self.conv_shortcut is not None:
            input_tensor = self.conv_shortcut(input_tensor)
        return input_tensor + hidden


class Downsample2D(nn.Module):
    def __init__(self, channels):
        super().__init__()
        self.conv = nn.Conv2d(channels, channels, 3, stride=2, padding=1)

    def forward(self, hidden):
        return self.conv(hidden)


class Upsample2D(nn.Module):
    def __init__(self, channels):
        super().__init__()
        self.conv = nn.Conv2d(channels, channels, 3, padding=1)

    def forward(self, hidden):
        return self.conv(F.interpolate(hidden, scale_factor=2.0, mode="nearest"))


class Attention(nn.Module):
    def __init__(self, query_dim, cross_attention_dim=None, heads=8, dim_head=64):
        super().__init__()
        inner = heads * dim_head
        kv_dim = query_dim if cross_attention_dim is None else cross_attention_dim
        self.heads, self.dim_head = heads, dim_head
        self.to_q = nn.Linear(query_dim, inner, bias=False)
        self.to_k = nn.Linear(kv_dim, inner, bias=False)
        self.to_v = nn.Linear(kv_dim, inner, bias=False)
        self.to_out = nn.ModuleList([nn.Linear(inner, query_dim, bias=True), nn.Dropout(0.0)])

    def forward(self, hidden, encoder_hidden_states=None):
        ctx = hidden if encoder_hidden_states is None else encoder_hidden_states
        b = hidden.shape[0]
        q = self.to_q(hidden).view(b, -1, self.heads, self.dim_head).transpose(1, 2)
        k = self.to_k(ctx).view(b, -1, self.heads, self.dim_head).transpose(1, 2)
        v = self.to_v(ctx).view(b, -1, self.heads, self.dim_head).transpose(1, 2)
        o = F.scaled_dot_product_attention(q, k, v)
        o = o.transpose(1, 2).reshape(b, -1, self.heads * self.dim_head)
        for m in self.to_out:
            o = m(o)
        return o


class GEGLU(nn.Module):
    def __init__(self, dim_in, dim_out):
        super().__init__()
        self.proj = nn.Linear(dim_in, dim_out * 2)

    def forward(self, hidden):
        hidden, gate = self.proj(hidden).chunk(2, dim=-1)
        return hidden * F.gelu(gate)


class FeedForward(nn.Module):
    def __init__(self, dim, mult=4):
        super().__init__()
        inner = dim * mult
        self.net = nn.ModuleList([GEGLU(dim, inner), nn.Dropout(0.0), nn.Linear(inner, dim)])

    def forward(self, hidden):
        for m in self.net:
            hidden = m(hidden)
        return hidden


class BasicTransformerBlock(nn.Module):
    def __init__(self, dim, heads, dim_head, cross_attention_dim):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim, eps=1e-5)
        self.attn1 = Attention(dim, None, heads, dim_head)
        self.norm2 = nn.LayerNorm(dim, eps=1e-5)
        self.attn2 = Attention(dim, cross_attention_dim, heads, dim_head)
        self.norm3 = nn.LayerNorm(dim, eps=1e-5)
        self.ff = FeedForward(dim)

    def forward(self, hidden, encoder_hidden_states):
        hidden = self.attn1(self.norm1(hidden)) + hidden
        hidden = self.attn2(self.norm2(hidden), encoder_hidden_states) + hidden
        return self.ff(self.norm3(hidden)) + hidden


class Transformer2DModel(nn.Module):
    def __init__(self, heads, dim_head, in_channels, cross_attention_dim, groups=32):
        super().__init__()
        inner = heads * dim_head
        self.norm = nn.GroupNorm(groups, in_channels, eps=1e-6, affine=True)
        self.proj_in = nn.Linear(in_channels, inner)
        self.transformer_blocks = nn.ModuleList(
            [BasicTransformerBlock(inner, heads, dim_head, cross_attention_dim)])
        self.proj_out = nn.Linear(inner, in_channels)

    def forward(self, hidden, encoder_hidden_states):
        b, _, h, w = hidden.shape
        residual = hidden
        hidden = self.norm(hidden)
        inner = hidden.shape[1]
        hidden = hidden.permute(0, 2, 3, 1).reshape(b, h * w, inner)
        hidden = self.proj_in(hidden)
        for blk in self.transformer_blocks:
            hidden = blk(hidden, encoder_hidden_states)
        hidden = self.proj_out(hidden)
        hidden = hidden.reshape(b, h, w, inner).permute(0, 3, 1, 2).contiguous()
        return hidden + residual


class CrossAttnDownBlock2D(nn.Module):
    def __init__(self, in_channels, out_channels, temb_channels, num_layers, heads, cross_dim,
                 add_downsample):
        super().__init__()
        self.resnets = nn.ModuleList()
        self.attentions = nn.ModuleList()
        for i in range(num_layers):
            self.resnets.append(ResnetBlock2D(in_channels if i == 0 else out_channels,
                                              out_channels, temb_channels))
            self.attentions.append(Transformer2DModel(heads, out_channels // heads, out_channels,
                                                      cross_dim))
        self.downsamplers = (nn.ModuleList([Downsample2D(out_channels)]) if add_downsample
                             else None)

    def forward(self, hidden, temb, encoder_hidden_states):
        output_states = ()
        for resnet, attn in zip(self.resnets, self.attentions):
            hidden = resnet(hidden, temb)
            hidden = attn(hidden, encoder_hidden_states)
            output_states = output_states + (hidden,)
        if self.downsamplers is not None:
            for d in self.downsamplers:
                hidden = d(hidden)
            output_states = output_states + (hidden,)
        return hidden, output_states


class DownBlock2D(nn.Module):
    def __init__(self, in_channels, out_channels, temb_channels, num_layers, add_downsample):
        super().__init__()
        self.resnets = nn.ModuleList([ResnetBlock2D(in_channels if i == 0 else out_channels,
                                                    out_channels, temb_channels)
                                      for i in range(num_layers)])
        self.downsamplers = (nn.ModuleList([Downsample2D(out_channels)]) if add_downsample
                             else None)

    def forward(self, hidden, temb, encoder_hidden_states=None):
        output_states = ()
        for resnet in self.resnets:
            hidden = resnet(hidden, temb)
            output_states = output_states + (hidden,)
        if self.downsamplers is not None:
            for d in self.downsamplers:
                hidden = d(hidden)
            output_states = output_states + (hidden,)
        return hidden, output_states


class UNetMidBlock2DCrossAttn(nn.Module):
    def __init__(self, channels, temb_channels, heads, cross_dim):
        super().__init__()
        self.attentions = nn.ModuleList([Transformer2DModel(heads, channels // heads, channels,
                                                            cross_dim)])
        self.resnets = nn.ModuleList([ResnetBlock2D(channels, channels, temb_channels)
                                      for _ in range(2)])

    def forward(self, hidden, temb, encoder_hidden_states):
        hidden = self.resnets[0](hidden, temb)
        for attn, resnet in zip(self.attentions, self.resnets[1:]):
            hidden = attn(hidden, encoder_hidden_states)
            hidden = resnet(hidden, temb)
        return hidden


class UpBlock2D(nn.Module):
    def __init__(self, in_channels, prev_output_channel, out_channels, temb_channels, num_layers,
                 add_upsample):
        super().__init__()
        self.resnets = nn.ModuleList()
        for i in range(num_layers):
            res_skip = in_channels if i == num_layers - 1 else out_channels
            res_in = prev_output_channel if i == 0 else out_channels
            self.resnets.append(ResnetBlock2D(res_in + res_skip, out_channels, temb_channels))
        self.upsamplers = nn.ModuleList([Upsample2D(out_channels)]) if add_upsample else None

    def forward(self, hidden, res_hidden_states_tuple, temb, encoder_hidden_states=None):
        for resnet in self.resnets:
            res = res_hidden_states_tuple[-1]
            res_hidden_states_tuple = res_hidden_states_tuple[:-1]
            hidden = torch.cat([hidden, res], dim=1)
            hidden = resnet(hidden, temb)
        if self.upsamplers is not None:
            for u in self.upsamplers:
                hidden = u(hidden)
        return hidden


class CrossAttnUpBlock2D(nn.Module):
    def __init__(self, in_channels, prev_output_channel, out_channels, temb_channels, num_layers,
                 heads, cross_dim, add_upsample):
        super().__init__()
        self.resnets = nn.ModuleList()
        self.attentions = nn.ModuleList()
        for i in range(num_layers):
            res_skip = in_channels if i == num_layers - 1 else out_channels
            res_in = prev_output_channel if i == 0 else out_channels
            self.resnets.append(ResnetBlock2D(res_in + res_skip, out_channels, temb_channels))
            self.attentions.append(Transformer2DModel(heads, out_channels // heads, out_channels,
                                                      cross_dim))
        self.upsamplers = nn.ModuleList([Upsample2D(out_channels)]) if add_upsample else None

    def forward(self, hidden, res_hidden_states_tuple, temb, encoder_hidden_states):
        for resnet, attn in zip(self.resnets, self.attentions):
            res = res_hidden_states_tuple[-1]
            res_hidden_states_tuple = res_hidden_states_tuple[:-1]
            hidden = torch.cat([hidden, res], dim=1)
            hidden = resnet(hidden, temb)
            hidden = attn(hidden, encoder_hidden_states)
        if self.upsamplers is not None:
            for u in self.upsamplers:
                hidden = u(hidden)
        return hidden


class UNet2DConditionModel(nn.Module):
    """SD2.1 family: down types (CrossAttnDown x 3, Down) unless ``cross_attn``
    says otherwise, up types mirrored, head dim 64."""

    def __init__(self, in_channels=4, out_channels=4, block_out_channels=(320, 640, 1280, 1280),
                 cross_attn=(1, 1, 1, 0), layers_per_block=2, cross_attention_dim=1024,
                 head_dim=64):
        super().__init__()
        ch = list(block_out_channels)
        time_embed_dim = ch[0] * 4
        self.time_proj_dim = ch[0]
        self.conv_in = nn.Conv2d(in_channels, ch[0], 3, padding=1)
        self.time_embedding = TimestepEmbedding(ch[0], time_embed_dim)
        self.down_blocks = nn.ModuleList()
        output_channel = ch[0]
        for i in range(len(ch)):
            input_channel, output_channel = output_channel, ch[i]
            final = i == len(ch) - 1
            if cross_attn[i]:
                blk = CrossAttnDownBlock2D(input_channel, output_channel, time_embed_dim,
                                           layers_per_block, output_channel // head_dim,
                                           cross_attention_dim, not final)
            else:
                blk = DownBlock2D(input_channel, output_channel, time_embed_dim,
                                  layers_per_block, not final)
            self.down_blocks.append(blk)
        self.mid_block = UNetMidBlock2DCrossAttn(ch[-1], time_embed_dim, ch[-1] // head_dim,
                                                 cross_attention_dim)
        self.up_blocks = nn.ModuleList()
        rev = list(reversed(ch))
        rev_xattn = list(reversed(cross_attn))
        output_channel = rev[0]
        for i in range(len(ch)):
            prev_output_channel = output_channel
            output_channel = rev[i]
            input_channel = rev[min(i + 1, len(ch) - 1)]
            final = i == len(ch) - 1
            if rev_xattn[i]:
                blk = CrossAttnUpBlock2D(input_channel, prev_output_channel, output_channel,
                                         time_embed_dim, layers_per_block + 1,
                                         output_channel // head_dim, cross_attention_dim,
                                         not final)
            else:
                blk = UpBlock2D(input_channel, prev_output_channel, output_channel,
                                time_embed_dim, layers_per_block + 1, not final)
            self.up_blocks.append(blk)
        self.conv_norm_out = nn.GroupNorm(32, ch[0], eps=1e-5)
        self.conv_act = nn.SiLU()
        self.conv_out = nn.Conv2d(ch[0], out_channels, 3, padding=1)

    def forward(self, sample, timestep, encoder_hidden_states):
        timesteps = timestep.reshape(-1).expand(sample.shape[0])
        t_emb = get_timestep_embedding(timesteps, self.time_proj_dim).to(sample.dtype)
        emb = self.time_embedding(t_emb)
        sample = self.conv_in(sample)
        down_block_res_samples = (sample,)
        for blk in self.down_blocks:
            sample, res = blk(sample, emb, encoder_hidden_states)
            down_block_res_samples += res
        sample = self.mid_block(sample, emb, encoder_hidden_states)
        for blk in self.up_blocks:
            res = down_block_res_samples[-len(blk.resnets):]
            down_block_res_samples = down_block_res_samples[:-len(blk.resnets)]
            sample = blk(sample, res, emb, encoder_hidden_states)
        sample = self.conv_act(self.conv_norm_out(sample))
        return self.conv_out(sample)


class HalfIO(nn.Module):
    """fp32 sample / context in, fp16 U-Net inside, fp32 out: the I/O form of
    the SD-Turbo ONNX graph (fp16 initializers, unet.js:13-19)."""

    def __init__(self, unet: UNet2DConditionModel):
        super().__init__()
        self.unet = unet.half()

    def forward(self, sample, timestep, encoder_hidden_states):
        out = self.unet(sample.half(), timestep, encoder_hidden_states.half())
        return out.float()


def from_config(cfg: dict) -> UNet2DConditionModel:
    """Module for a config dict with the keys of the library's U-Net config
    (block_channels, cross_attn, layers_per_block, cross_dim, in/out
    channels); time_dim must be 4 x block_channels[0] as in diffusers."""
    assert cfg["time_dim"] == 4 * cfg["block_channels"][0]
    assert cfg["groups"] == 32
    return UNet2DConditionModel(cfg["in_channels"], cfg["out_channels"], cfg["block_channels"],
                                cfg["cross_attn"], cfg["layers_per_block"], cfg["cross_dim"])


def load(module: nn.Module, sd: dict, dtype=torch.float64) -> nn.Module:
    """Strict load of a {diffusers name: array} dict (every name must match)."""
    module.load_state_dict({k: torch.as_tensor(v) for k, v in sd.items()}, strict=True)
    return module.to(dtype).eval()


def export_case(cfg: dict, sd: dict, H: int, W: int, S: int = 77, seed: int = 0,
                device: str = "cpu"):
    """The SD-Turbo-form ONNX graph of this module for a config and weights:
    (onnx bytes, feeds, fp16-rounded state dict).

    The graph has the I/O of the SD-Turbo U-Net file (unet.js:13-19): fp32
    ``sample`` [1,4,H,W], int64 ``timestep`` [1], fp32
    ``encoder_hidden_states`` [1,S,cross_dim], fp16 initializers inside,
    fp32 ``out_sample``; exported by torch's TorchScript exporter at opset
    14.  The weights are rounded to fp16 first, so the returned state dict
    is exactly what the file holds.  ``device`` is where the export trace
    runs (a full-size fp16 trace is quick on the GPU)."""
    from golden import onnx_export
    import numpy as np
    sd16 = {k: np.asarray(v, np.float32).astype(np.float16).astype(np.float32)
            for k, v in sd.items()}
    m = HalfIO(load(from_config(cfg), sd16, dtype=torch.float32)).to(device)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, cfg["in_channels"], H, W, generator=g)
    ctx = torch.randn(1, S, cfg["cross_dim"], generator=g)
    t = torch.tensor([999], dtype=torch.int64)
    data = onnx_export.export(m, (x.to(device), t.to(device), ctx.to(device)),
                              ("sample", "timestep", "encoder_hidden_states"),
                              output_name="out_sample")
    del m
    feeds = {"sample": x.numpy(), "timestep": t.numpy(), "encoder_hidden_states": ctx.numpy()}
    return data, feeds, sd16
