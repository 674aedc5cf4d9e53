"""GPU parity of the fused blocks (di_resnet_block, di_transformer_block,
di_ffn) against the oracle compositions (oracle/unet_ref.py on the C oracle)
on the same fp16-representable weights and inputs.

Block outputs chain several fp16-stored intermediates, so the bar is the
north-star rel-L2 <= 1e-2 for MFMA paths; measured values are printed."""
import math

import numpy as np
import pytest

import oracle
from conftest import rel_l2
from oracle import unet_ref

pytestmark = pytest.mark.gpu

F16 = 1


def _q(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _res_sd(rng, p, cin, cout, temb_dim):
    sd = {}
    k = lambda ci: math.sqrt(2.0 / (ci * 9))
    sd[p + ".norm1.weight"] = _q(1 + 0.02 * rng.standard_normal(cin))
    sd[p + ".norm1.bias"] = _q(0.02 * rng.standard_normal(cin))
    sd[p + ".conv1.weight"] = _q(rng.standard_normal((cout, cin, 3, 3)) * k(cin))
    sd[p + ".conv1.bias"] = _q(0.01 * rng.standard_normal(cout))
    if temb_dim:
        sd[p + ".time_emb_proj.weight"] = _q(rng.standard_normal((cout, temb_dim)) * math.sqrt(2 / (temb_dim + cout)))
        sd[p + ".time_emb_proj.bias"] = _q(0.01 * rng.standard_normal(cout))
    sd[p + ".norm2.weight"] = _q(1 + 0.02 * rng.standard_normal(cout))
    sd[p + ".norm2.bias"] = _q(0.02 * rng.standard_normal(cout))
    sd[p + ".conv2.weight"] = _q(rng.standard_normal((cout, cout, 3, 3)) * k(cout))
    sd[p + ".conv2.bias"] = _q(0.01 * rng.standard_normal(cout))
    if cin != cout:
        sd[p + ".conv_shortcut.weight"] = _q(rng.standard_normal((cout, cin, 1, 1)) * math.sqrt(2.0 / cin))
        sd[p + ".conv_shortcut.bias"] = _q(0.01 * rng.standard_normal(cout))
    return sd


def _tf_sd(rng, p, c, cross):
    shapes = {}
    for k, v in unet_ref.unet_param_shapes(unet_ref.sd21_config()).items():
        if k.startswith("mid_block.attentions.0."):
            shapes[p + k[len("mid_block.attentions.0"):]] = v
    sd = {}
    for name, shp in shapes.items():
        shp = tuple(c * (s // 1280) if s % 1280 == 0 and s >= 1280 else s for s in shp)
        if name.endswith(("to_k.weight", "to_v.weight")) and ".attn2." in name:
            shp = (c, cross)
        if len(shp) == 2:
            a = rng.standard_normal(shp) * math.sqrt(2.0 / (shp[0] + shp[1]))
        elif "norm" in name and name.endswith("weight"):
            a = 1 + 0.02 * rng.standard_normal(shp)
        else:
            a = 0.02 * rng.standard_normal(shp)
        sd[name] = _q(a)
    return sd


@pytest.mark.parametrize("B,cin,cout,H,W,temb", [
    (1, 320, 640, 32, 32, True),    # cfg3: SD2.1 ResNet 320->640 @32x32 with temb + 1x1 skip
    (1, 1280, 1280, 16, 16, False), # fused-resnet.js SHAPE (no temb, identity skip)
    (2, 640, 640, 16, 16, True),    # batch 2
    (1, 1280, 1280, 8, 8, True),    # 8x8: split-K conv1 with GroupNorm in the reducer
    (2, 1280, 1280, 8, 8, True),    # the same, two images (one reducer workgroup row each)
    (1, 1280, 1280, 16, 16, True),  # 16x16: conv1 split 5, GN2 + SiLU applied by its reducer
])
def test_resnet_block(dev, rng, B, cin, cout, H, W, temb):
    from drawinstant import blocks
    print(f"[resnet] B={B} {cin}->{cout} {H}x{W} temb={temb}", flush=True)
    sd = _res_sd(rng, "r", cin, cout, 1280 if temb else 0)
    x = _q(rng.standard_normal((B, cin, H, W)))
    t = rng.standard_normal((B, 1280)).astype(np.float32)
    w = blocks.upload_resnet(dev, sd, "r")
    bx = dev.storage(x.transpose(0, 2, 3, 1).astype(np.float16))
    bt = dev.storage(t) if temb else None
    y = dev.create_buffer(B * H * W * cout * 2)
    blocks.resnet_block(dev, w, bx, bt, y, B, cin, cout, H, W, 1280)
    got = dev.download(y, np.float16).astype(np.float32).reshape(B, H, W, cout).transpose(0, 3, 1, 2)
    ts = oracle.unary("SiLU", t) if temb else None
    ref = unet_ref.resnet(unet_ref.OracleOps(), sd, "r", x, ts)
    err = rel_l2(got, ref)
    print(f"   rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e}", flush=True)
    assert err <= 1e-2
    w.destroy()


@pytest.mark.parametrize("B,cin,cout,H,W", [
    (1, 1280, 1280, 8, 8),    # conv1 split 12: one row-step of 64 pixels per thread
    (2, 1280, 1280, 16, 16),  # split 5, two images: four 64-row slices exchanging
    (1, 640, 640, 32, 32),    # 20 channels per group, split 2: eight 128-row slices exchanging
    (1, 2560, 1280, 8, 8),    # up-block input width (K = 23040)
])
def test_resnet_gn_reducer_matches_apply(dev, rng, monkeypatch, B, cin, cout, H, W):
    """conv1's GroupNorm2 + SiLU applied by its split-K reducer against the
    same block with the separate statistics + apply launches
    (DI_GN_REDUCE_FUSE=0): the fp16 conv1 values are the same, only the
    order of the statistics' fp32 sums differs, so the block outputs agree
    to fp16 rounding."""
    from drawinstant import blocks
    print(f"[resnet gn reducer] B={B} {cin}->{cout} {H}x{W}", flush=True)
    sd = _res_sd(rng, "r", cin, cout, 1280)
    x = _q(rng.standard_normal((B, cin, H, W)))
    t = rng.standard_normal((B, 1280)).astype(np.float32)
    w = blocks.upload_resnet(dev, sd, "r")
    bx = dev.storage(x.transpose(0, 2, 3, 1).astype(np.float16))
    bt = dev.storage(t)
    def run():
        y = dev.create_buffer(B * H * W * cout * 2)
        blocks.resnet_block(dev, w, bx, bt, y, B, cin, cout, H, W, 1280)
        return dev.download(y, np.float16).astype(np.float32)

    monkeypatch.setenv("DI_GN_REDUCE_FUSE", "1")
    fused = run()
    if H * W >= 256:
        # four (16 x 16) or eight (32 x 32) workgroups per (group, image)
        # exchanging their statistics:
        # the recomputing path (no slice awaited) gives the same bits, one
        # workgroup per group the same values up to the order of the sums
        monkeypatch.setenv("DI_GN_XCHG_SPIN", "0")
        np.testing.assert_array_equal(run(), fused)
        monkeypatch.delenv("DI_GN_XCHG_SPIN")
        monkeypatch.setenv("DI_GN_REDUCE_XCHG", "0")
        one = run()
        monkeypatch.delenv("DI_GN_REDUCE_XCHG")
        print(f"   exchange vs one workgroup per group: rel-L2 {rel_l2(fused, one):.2e}",
              flush=True)
        assert rel_l2(fused, one) <= 1e-3
    monkeypatch.setenv("DI_GN_REDUCE_FUSE", "0")
    sep = run()
    err = rel_l2(fused, sep)
    scale = float(np.max(np.abs(sep)))
    print(f"   rel-L2 {err:.2e} max-abs {np.max(np.abs(fused - sep)):.2e} (max |y| {scale:.2f})",
          flush=True)
    assert np.all(np.isfinite(fused))
    assert err <= 1e-3
    assert np.max(np.abs(fused - sep)) <= 4e-3 * max(scale, 1.0)
    w.destroy()


@pytest.mark.parametrize("B,C,H,W", [
    (1, 320, 64, 64),   # cfg4: 4096 tokens x 320, 5 heads, context 77x1024
    (1, 1280, 8, 8),    # mid block (20 heads)
    (2, 640, 16, 16),   # batch 2, 10 heads
])
def test_transformer_block(dev, rng, B, C, H, W):
    from drawinstant import blocks
    print(f"[transformer] B={B} C={C} {H}x{W}", flush=True)
    sd = _tf_sd(rng, "t", C, 1024)
    x = _q(rng.standard_normal((B, C, H, W)))
    ctx = _q(rng.standard_normal((B, 77, 1024)))
    w = blocks.upload_transformer(dev, sd, "t")
    bx = dev.storage(x.transpose(0, 2, 3, 1).astype(np.float16))
    bc = dev.storage(ctx.astype(np.float16))
    y = dev.create_buffer(B * H * W * C * 2)
    blocks.transformer_block(dev, w, bx, bc, y, B, C, H, W)
    got = dev.download(y, np.float16).astype(np.float32).reshape(B, H, W, C).transpose(0, 3, 1, 2)
    ref = unet_ref.transformer(unet_ref.OracleOps(), sd, "t", x, ctx)
    err = rel_l2(got, ref)
    print(f"   rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e}", flush=True)
    assert err <= 1e-2
    w.destroy()


@pytest.mark.parametrize("rows,D,F,act", [(2048, 1280, 5120, 4), (4096, 320, 1280, 2)])
def test_ffn(dev, rng, rows, D, F, act):
    """runFFNBench shape [2*1024, 1280 -> 5120] with the bench's tanh GELU, and the
    SD GEGLU FFN at 64x64 (320 -> 2x1280 -> 320)."""
    import drawinstant
    n1 = 2 * F if act == 2 else F
    x = _q(rng.standard_normal((rows, D)))
    w1 = _q(rng.standard_normal((n1, D)) * math.sqrt(2 / (D + n1)))
    b1 = _q(0.01 * rng.standard_normal(n1))
    w2 = _q(rng.standard_normal((D, F)) * math.sqrt(2 / (D + F)))
    b2 = _q(0.01 * rng.standard_normal(D))
    y = dev.create_buffer(rows * D * 2)
    drawinstant.call("di_ffn", dev.ctx, dev.storage(x.astype(np.float16)).handle,
                     dev.storage(w1.astype(np.float16)).handle, dev.storage(b1).handle,
                     dev.storage(w2.astype(np.float16)).handle, dev.storage(b2).handle, y.handle,
                     rows, D, F, act, F16)
    got = dev.download(y, np.float16).astype(np.float32).reshape(rows, D)
    hpre = oracle.linear(x, w1, b1)
    if act == 2:  # rows interleaved in 16-row [hidden | gate] groups
        g = hpre.reshape(rows, n1 // 32, 2, 16)
        h = g[:, :, 0].reshape(rows, F) * oracle.unary("GELU", g[:, :, 1].reshape(rows, F))
    else:
        h = oracle.unary("GELU_TANH", hpre)
    ref = oracle.linear(_q(h), w2, b2) + x
    err = rel_l2(got, ref)
    print(f"   ffn rel-L2 {err:.2e}", flush=True)
    assert err <= 1e-2
