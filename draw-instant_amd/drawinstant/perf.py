"""Algorithmic work of the SD2.1 U-Net step and its blocks (dense FLOPs of
every contraction, minimum HBM bytes of the bandwidth-bound ops), used for
roofline figures.  Counts follow the module shapes of UNet2DConditionModel;
nothing here touches the GPU."""
from __future__ import annotations

from dataclasses import dataclass, field

# MI355X published peaks (dense)
PEAK_FP16_FLOPS = 2.5e15
PEAK_HBM_BYTES = 8.0e12


@dataclass
class Work:
    flops: dict = field(default_factory=dict)  # category -> FLOPs

    def add(self, cat: str, f: float):
        self.flops[cat] = self.flops.get(cat, 0.0) + f

    @property
    def total(self) -> float:
        return sum(self.flops.values())


def conv_flops(B, cin, cout, ho, wo, k):
    return 2.0 * B * ho * wo * cout * cin * k * k


def resnet_flops(w: Work, B, cin, cout, h, wd, temb_dim=1280):
    w.add("resnet_conv", conv_flops(B, cin, cout, h, wd, 3) + conv_flops(B, cout, cout, h, wd, 3))
    if cin != cout:
        w.add("resnet_conv", conv_flops(B, cin, cout, h, wd, 1))
    w.add("temb", 2.0 * B * temb_dim * cout)


def transformer_flops(w: Work, B, c, h, wd, sctx=77, cross=1024):
    s = h * wd
    lin = lambda m, n, k: 2.0 * B * m * n * k
    w.add("tf_linear", lin(s, c, c) * 2)            # proj_in, proj_out
    w.add("tf_linear", lin(s, 3 * c, c) + lin(s, c, c))  # qkv, to_out
    w.add("tf_linear", lin(s, c, c) + lin(s, c, c))  # to_q, to_out (cross)
    w.add("tf_linear", lin(sctx, 2 * c, cross))      # context K/V
    w.add("tf_linear", lin(s, 8 * c, c) + lin(s, c, 4 * c))  # GEGLU, ff out
    w.add("self_attn", 4.0 * B * s * s * c)         # QK^T + PV over all heads
    w.add("cross_attn", 4.0 * B * s * sctx * c)


def unet_work(B=1, H=64, W=64, ch=(320, 640, 1280, 1280), xattn=(1, 1, 1, 0), L=2,
              sctx=77, cross=1024, time_dim=1280, in_ch=4, out_ch=4) -> Work:
    w = Work()
    w.add("conv_io", conv_flops(B, in_ch, ch[0], H, W, 3))
    w.add("temb", 2.0 * B * (ch[0] * time_dim + time_dim * time_dim))
    h, wd, cin = H, W, ch[0]
    for i in range(4):
        for j in range(L):
            resnet_flops(w, B, cin if j == 0 else ch[i], ch[i], h, wd, time_dim)
            if xattn[i]:
                transformer_flops(w, B, ch[i], h, wd, sctx, cross)
        cin = ch[i]
        if i < 3:
            h, wd = (h + 1) // 2, (wd + 1) // 2
            w.add("sample_conv", conv_flops(B, ch[i], ch[i], h, wd, 3))
    resnet_flops(w, B, ch[3], ch[3], h, wd, time_dim)
    transformer_flops(w, B, ch[3], h, wd, sctx, cross)
    resnet_flops(w, B, ch[3], ch[3], h, wd, time_dim)
    rev = ch[::-1]
    prev = ch[3]
    for i in range(4):
        out, inp = rev[i], rev[min(i + 1, 3)]
        for j in range(L + 1):
            skip = inp if j == L else out
            resnet_flops(w, B, (prev if j == 0 else out) + skip, out, h, wd, time_dim)
            if xattn[3 - i]:
                transformer_flops(w, B, out, h, wd, sctx, cross)
        prev = out
        if i < 3:
            h, wd = h * 2, wd * 2
            w.add("sample_conv", conv_flops(B, out, out, h, wd, 3))
    w.add("conv_io", conv_flops(B, ch[0], out_ch, h, wd, 3))
    return w


def gn_silu_bytes(N, C, HW, elem=4):
    """cfg1 algorithmic traffic: read x, write y, read gamma/beta."""
    return 2 * N * C * HW * elem + 2 * C * 4


def vae_work(B=1, H=64, W=64, ch=(128, 256, 512, 512), L=2, latent=4, out=3) -> Work:
    """Dense FLOPs of SD's VAE decode (post_quant_conv + Decoder) for a
    [B, latent, H, W] latent: convs, the mid attention (QKV, scores, PV,
    out projection); norms and element-wise work are not counted."""
    w = Work()
    rev = list(reversed(ch))
    w.add("conv", conv_flops(B, latent, latent, H, W, 1) + conv_flops(B, latent, rev[0], H, W, 3))
    hh, ww = H, W
    for _ in range(2):
        resnet_flops(w, B, rev[0], rev[0], hh, ww, temb_dim=0)
    S, C = hh * ww, rev[0]
    w.add("attention", 2.0 * B * S * C * 3 * C + 4.0 * B * S * S * C + 2.0 * B * S * C * C)
    prev = rev[0]
    for i, c in enumerate(rev):
        for j in range(L + 1):
            resnet_flops(w, B, prev if j == 0 else c, c, hh, ww, temb_dim=0)
        prev = c
        if i < 3:
            hh, ww = hh * 2, ww * 2
            w.add("upsample_conv", conv_flops(B, c, c, hh, ww, 3))
    w.add("conv", conv_flops(B, rev[-1], out, hh, ww, 3))
    return w
