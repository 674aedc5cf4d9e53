"""CPU checks of the U-Net reference composition (oracle/unet_ref.py): the
architecture table reproduces SD2.1's published parameter count, and the
composition run on the C oracle agrees with the same composition on torch's
library ops (float32 CPU) on a small seeded U-Net."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import unet_ref


def test_sd21_parameter_count():
    # diffusers' SD2.1 UNet2DConditionModel has 865,910,724 parameters
    assert unet_ref.sd21_param_count() == 865_910_724
    shapes = unet_ref.unet_param_shapes(unet_ref.sd21_config())
    assert sum(int(np.prod(s)) for s in shapes.values()) == 865_910_724
    assert len(shapes) == 686


def test_oracle_composition_matches_torch_composition():
    torch = pytest.importorskip("torch")
    cfg = unet_ref.small_config()
    cfg["block_channels"] = [64, 64, 128, 128]
    cfg["cross_dim"] = 64
    cfg["time_dim"] = 128
    sd = unet_ref.random_state_dict(cfg, seed=3)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 4, 16, 16)).astype(np.float32)
    ctx = rng.standard_normal((1, 7, 64)).astype(np.float32)
    t = np.array([999.0], np.float32)
    got = unet_ref.unet_forward(unet_ref.OracleOps(), sd, cfg, x, t, ctx)
    ref = unet_ref.unet_forward(unet_ref.TorchOps("cpu"), sd, cfg, x, t, ctx).numpy()
    assert np.isfinite(got).all() and got.shape == (1, 4, 16, 16)
    assert rel_l2(got, ref) < 1e-4
