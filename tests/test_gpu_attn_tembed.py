"""GPU parity of flash attention (di_attn_self / di_attn_cross) and the
timestep embedding (di_tembed) against the CPU oracle.

Attention runs fp16 MFMA with fp32 accumulation; the oracle runs in fp64 on
the same fp16-rounded Q/K/V, so the error is P's fp16 rounding plus the
output rounding: rel-L2 <= 2e-3 asserted (north-star bar 1e-2), max-abs
printed.  di_tembed with fp32 weights is an fp32 path: max-rel <= 1e-4.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import max_rel, rel_l2

pytestmark = pytest.mark.gpu

F32, F16, BSHD, BHSD = 0, 1, 0, 1


def _call(dev, fn, *a):
    import drawinstant
    drawinstant.call(fn, dev.ctx, *a)


def _attn_case(dev, rng, B, H, Sq, Skv, layout, dt, fn, scale=0.0, qkv=None):
    shp = (lambda s: (B, s, H, 64)) if layout == BSHD else (lambda s: (B, H, s, 64))
    if qkv is None:
        q = rng.standard_normal(shp(Sq)).astype(np.float16)
        k = rng.standard_normal(shp(Skv)).astype(np.float16)
        v = rng.standard_normal(shp(Skv)).astype(np.float16)
    else:
        q, k, v = (a.astype(np.float16) for a in qkv)
    npdt = np.float16 if dt == F16 else np.float32
    bq, bk, bv = (dev.storage(a.astype(npdt)) for a in (q, k, v))
    o = dev.create_buffer(q.size * (2 if dt == F16 else 4))
    if fn == "di_attn_self":
        _call(dev, fn, bq.handle, bk.handle, bv.handle, o.handle, B, H, Sq, 64, layout, scale, dt)
    else:
        _call(dev, fn, bq.handle, bk.handle, bv.handle, o.handle, B, H, Sq, Skv, 64, layout, scale,
              dt)
    got = dev.download(o, npdt).astype(np.float32).reshape(q.shape)
    ref = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                           scale=scale if scale > 0 else None,
                           layout="bshd" if layout == BSHD else "bhsd")
    err = rel_l2(got, ref)
    print(f"   rel-L2 {err:.2e} max-abs {np.max(np.abs(got - ref)):.2e}", flush=True)
    return err


@pytest.mark.parametrize("B,H,S,layout", [
    (1, 5, 4096, BSHD),    # cfg4 self-attention (64x64 latent, 5 heads)
    (2, 20, 256, BSHD),    # fused-attn.js SHAPE [2,20,256,64]
    (1, 10, 1024, BHSD),   # 32x32 level
    (1, 20, 64, BHSD),     # 8x8 level
    (1, 3, 100, BSHD),     # ragged: partial query and key tiles
])
def test_attn_self_fp16(dev, rng, B, H, S, layout):
    print(f"[attn self] B={B} H={H} S={S} layout={layout}", flush=True)
    assert _attn_case(dev, rng, B, H, S, S, layout, F16, "di_attn_self") <= 2e-3


@pytest.mark.parametrize("B,H,Sq,Skv,layout", [
    (1, 5, 4096, 77, BSHD),   # cfg4 cross-attention
    (2, 20, 256, 77, BHSD),   # fused-cross-attn.js SHAPE
    (1, 4, 130, 1, BHSD),     # single key: output = V
    (1, 2, 64, 65, BSHD),     # one key past a tile boundary
    (1, 2, 130, 2113, BHSD),  # key-range split: 34 tiles in 2 ranges, last tile 1 key
    (2, 3, 200, 3100, BSHD),  # key-range split (3 ranges of 17/17/15 tiles) with batch 2
])
def test_attn_cross_fp16(dev, rng, B, H, Sq, Skv, layout):
    print(f"[attn cross] B={B} H={H} Sq={Sq} Skv={Skv}", flush=True)
    assert _attn_case(dev, rng, B, H, Sq, Skv, layout, F16, "di_attn_cross") <= 2e-3


@pytest.mark.parametrize("B,H,Sq,Skv,growth", [
    (1, 2, 256, 4096, 6.0),   # one key range: the max rises over 64 tiles
    (1, 3, 130, 2113, 4.0),   # key-range split, ragged last tile
    (2, 2, 64, 77, 12.0),     # cross-attention length, steep rise within two tiles
])
def test_attn_rising_scores_fp16(dev, rng, B, H, Sq, Skv, growth):
    """Key norms grow along the sequence (x1 -> x(1+growth)), so later key
    tiles hold scores up to ~20 log2 units above the first tile's max: the
    kernel's running max must be raised mid-range (the lane-sum overflow
    check and the tile redo) without losing the earlier tiles' weight."""
    print(f"[attn rising] B={B} H={H} Sq={Sq} Skv={Skv} growth={growth}", flush=True)
    q = rng.standard_normal((B, Sq, H, 64))
    ramp = 1.0 + growth * (np.arange(Skv) / max(1, Skv - 1))
    k = rng.standard_normal((B, Skv, H, 64)) * ramp[None, :, None, None]
    v = rng.standard_normal((B, Skv, H, 64))
    assert _attn_case(dev, rng, B, H, Sq, Skv, BSHD, F16, "di_attn_cross", qkv=(q, k, v)) <= 2e-3


@pytest.mark.parametrize("B,H,Sq,Skv,layout", [
    (1, 3, 128, 499, BSHD),    # 8 key tiles over 2 key groups (4/4), last tile 51 keys
    (2, 2, 96, 571, BHSD),     # 9 tiles: groups of 5 and 4, partial query block, batch 2
    (1, 4, 64, 1983, BSHD),    # 31 tiles (16/15), last tile 63 keys
    (1, 10, 1024, 1024, BSHD), # the 32x32 level in the U-Net's token-major layout: 2 x 8 tiles
])
def test_attn_key_groups_fp16(dev, rng, B, H, Sq, Skv, layout):
    """Small grids with 8 - 31 key tiles split each workgroup's keys over
    two groups of four wavefronts, merged in LDS: odd tile counts give the
    groups unequal runs, and the shorter one idles through barriers."""
    print(f"[attn key groups] B={B} H={H} Sq={Sq} Skv={Skv} layout={layout}", flush=True)
    assert _attn_case(dev, rng, B, H, Sq, Skv, layout, F16, "di_attn_cross") <= 2e-3


@pytest.mark.parametrize("Skv,growth", [(900, 6.0), (571, 12.0)])
def test_attn_key_groups_rising_scores_fp16(dev, rng, Skv, growth):
    """Rising key norms inside key groups: each group raises its own running
    max, and the LDS merge rescales the groups' parts to the largest."""
    B, H, Sq = 1, 2, 128
    print(f"[attn key groups rising] Skv={Skv} growth={growth}", flush=True)
    q = rng.standard_normal((B, Sq, H, 64))
    ramp = 1.0 + growth * (np.arange(Skv) / max(1, Skv - 1))
    k = rng.standard_normal((B, Skv, H, 64)) * ramp[None, :, None, None]
    v = rng.standard_normal((B, Skv, H, 64))
    assert _attn_case(dev, rng, B, H, Sq, Skv, BSHD, F16, "di_attn_cross", qkv=(q, k, v)) <= 2e-3


def test_attn_fp32_tensors_and_explicit_scale(dev, rng):
    assert _attn_case(dev, rng, 1, 4, 200, 200, BHSD, F32, "di_attn_self", scale=0.05) <= 2e-3


def test_attn_rejects_other_head_dims(dev):
    import drawinstant
    b = dev.create_buffer(1 << 16)
    with pytest.raises(drawinstant.DiError) as e:
        drawinstant.call("di_attn_self", dev.ctx, b.handle, b.handle, b.handle, b.handle, 1, 1, 8,
                         32, BHSD, 0.0, F16)
    assert e.value.code == 4


@pytest.mark.parametrize("t", [0.0, 500.0, 999.0])
def test_tembed_fp32_reference_shape(dev, rng, t):
    """fused-tembed.js shape 320 -> 1280 -> 1280, fp32 weights."""
    emb, hid = 320, 1280
    w1 = (rng.standard_normal((hid, emb)) * 0.03).astype(np.float32)
    b1 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    w2 = (rng.standard_normal((hid, hid)) * 0.03).astype(np.float32)
    b2 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    y = dev.create_buffer(hid * 4)
    _call(dev, "di_tembed", dev.storage(np.array([t], np.float32)).handle, dev.storage(w1).handle,
          dev.storage(b1).handle, dev.storage(w2).handle, dev.storage(b2).handle, y.handle, 1, emb,
          hid, F32)
    assert max_rel(dev.download(y), oracle.tembed(t, w1, b1, w2, b2)) <= 1e-4


@pytest.mark.parametrize("B,emb,hid,dt", [
    (1, 1280, 1280, F16),  # K = 1280: the last vector slot of half the lanes is empty
    (2, 96, 1000, F16),    # rows not a multiple of 4 per workgroup
    (3, 320, 1280, F32),   # B > 2: one row per wavefront
    (8, 64, 200, F32),     # the largest batch
    (2, 100, 1277, F16),   # K % 8 != 0: the scalar path
])
def test_tembed_gemv_shapes(dev, rng, B, emb, hid, dt):
    """Both GEMV paths (vector loads issued before the input is staged, and
    the scalar fallback) across batch sizes, ragged row counts and K."""
    ts = np.linspace(999.0, 0.0, B).astype(np.float32)
    wt = np.float16 if dt == F16 else np.float32
    w1 = (rng.standard_normal((hid, emb)) * math.sqrt(1 / emb)).astype(wt)
    b1 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    w2 = (rng.standard_normal((hid, hid)) * math.sqrt(1 / hid)).astype(wt)
    b2 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    y = dev.create_buffer(B * hid * 4)
    _call(dev, "di_tembed", dev.storage(ts).handle, dev.storage(w1).handle, dev.storage(b1).handle,
          dev.storage(w2).handle, dev.storage(b2).handle, y.handle, B, emb, hid, dt)
    got = dev.download(y).reshape(B, hid)
    for i, t in enumerate(ts):
        ref = oracle.tembed(float(t), w1.astype(np.float32), b1, w2.astype(np.float32), b2)
        err = max_rel(got[i], ref)
        print(f"[tembed] B={B} emb={emb} hid={hid} dt={dt} t={t:.0f} max-rel {err:.2e}", flush=True)
        assert err <= 1e-4


def test_tembed_fp16_weights_batched(dev, rng):
    emb, hid, B = 320, 1280, 4
    ts = np.array([999.0, 750.0, 1.0, 0.0], np.float32)
    w1 = (rng.standard_normal((hid, emb)) * math.sqrt(1 / emb)).astype(np.float16)
    b1 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    w2 = (rng.standard_normal((hid, hid)) * math.sqrt(1 / hid)).astype(np.float16)
    b2 = (0.01 * rng.standard_normal(hid)).astype(np.float32)
    y = dev.create_buffer(B * hid * 4)
    _call(dev, "di_tembed", dev.storage(ts).handle, dev.storage(w1).handle, dev.storage(b1).handle,
          dev.storage(w2).handle, dev.storage(b2).handle, y.handle, B, emb, hid, F16)
    got = dev.download(y).reshape(B, hid)
    for i, t in enumerate(ts):
        ref = oracle.tembed(float(t), w1.astype(np.float32), b1, w2.astype(np.float32), b2)
        assert max_rel(got[i], ref) <= 1e-4
