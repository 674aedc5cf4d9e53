"""GPU: the native VAE decoder (di_vae_*) against the reference composition
oracle/vae_ref.py, which is pinned against torch modules on the CPU.

Tolerances: activations are fp16 with fp32 accumulation, so the image is
compared by rel-L2 <= 1e-2 (the north-star bar for MFMA paths) against the
C oracle (small decoder, fp64 accumulation) and against torch float32 on the
GPU (SD's decoder at a 64x64 latent, 512x512 image); graph replay must be
bit-identical to the eager decode.
"""
import numpy as np
import pytest

from conftest import rel_l2
from drawinstant.vae import SCALING_FACTOR, VAE, VAEConfig
from oracle import unet_ref, vae_ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(dev):
    cfg = vae_ref.small_config()
    v = VAE(dev, VAEConfig.small(tuple(cfg["block_channels"])))
    sd = vae_ref.random_state_dict(cfg, seed=5)
    v.load_state_dict(sd)
    yield v, sd, cfg
    v.destroy()


def test_state_dict_round_trip(small):
    v, sd, _ = small
    back = v.state_dict()
    assert set(back) == set(sd)
    for k in sd:
        assert np.array_equal(back[k], sd[k]), k


# (2, 32): 256x256 images, whose GroupNorm statistics are pre-folded
# (more than 256 chunks per image), two images per launch
@pytest.mark.parametrize("B,h", [(1, 8), (2, 8), (1, 5), (2, 32)])
def test_small_decoder_vs_oracle(small, B, h):
    v, sd, cfg = small
    z = np.random.default_rng(6 + B).standard_normal((B, 4, h, h)).astype(np.float32)
    got = v(z)
    ref = vae_ref.vae_decode(unet_ref.OracleOps(), sd, cfg, z, 1 / SCALING_FACTOR)
    e = rel_l2(got, ref)
    print(f"[vae] small B={B} latent {h}x{h} rel_l2={e:.2e}", flush=True)
    assert got.shape == (B, 3, 8 * h, 8 * h) and e <= 1e-2


@pytest.mark.parametrize("check", [False, True])
def test_graph_replay_is_bit_identical(dev, small, monkeypatch, check):
    """Replays equal the eager decode; with DI_GRAPH_CHECK=1 the captured
    graph's nodes and, before each replay, its buffers are validated too."""
    v, _, _ = small
    if check:
        monkeypatch.setenv("DI_GRAPH_CHECK", "1")
    z = np.random.default_rng(9).standard_normal((1, 4, 8, 8)).astype(np.float32)
    bz = dev.storage(z)
    bi = dev.create_buffer(3 * 64 * 64 * 4)
    try:
        v.decode(bz, bi, 1, 8, 8)
        eager = dev.download(bi, np.float32, (1, 3, 64, 64))
        outs = []
        for _ in range(3):
            dev.fill_normal(bi, 3 * 64 * 64, 1)  # stale output must be overwritten
            v.decode(bz, bi, 1, 8, 8, graph=True)
            outs.append(dev.download(bi, np.float32, (1, 3, 64, 64)))
        for o in outs:
            assert np.array_equal(o, eager)
    finally:
        bz.destroy()
        bi.destroy()


def test_sd_decoder_512_vs_torch(dev):
    """SD's decoder (128/256/512/512), latent 64x64 -> 512x512."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("torch reference needs the GPU")
    cfg = vae_ref.sd_config()
    sd = vae_ref.random_state_dict(cfg, seed=7)
    v = VAE(dev)
    try:
        v.load_state_dict(sd)
        z = np.random.default_rng(8).standard_normal((1, 4, 64, 64)).astype(np.float32)
        got = v(z, graph=True)
    finally:
        v.destroy()
    ops = unet_ref.TorchOps("cuda")
    tsd = {k: ops.asarray(a) for k, a in sd.items()}
    with torch.no_grad():
        ref = vae_ref.vae_decode(ops, tsd, cfg, ops.asarray(z), 1 / SCALING_FACTOR).cpu().numpy()
    e = rel_l2(got, ref)
    print(f"[vae] SD decoder 512x512 rel_l2={e:.2e}", flush=True)
    assert got.shape == (1, 3, 512, 512) and np.isfinite(got).all() and e <= 1e-2
