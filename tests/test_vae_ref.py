"""CPU: the VAE decoder reference composition (oracle/vae_ref.py) pinned
against an independent implementation, torch's nn.Conv2d / GroupNorm /
scaled_dot_product_attention modules of tests/golden/onnx_export.VAEDecoder
run in float64 on the same weights, and the parameter inventory of SD's
decoder (49.49 M parameters)."""
import numpy as np
import pytest
import torch

from conftest import max_rel
from golden import onnx_export
from oracle import unet_ref, vae_ref


def module_name(name: str) -> str:
    """diffusers VAE-decoder name -> the torch test module's name."""
    n = name.replace("decoder.mid_block.resnets.0.", "mid.0.")
    n = n.replace("decoder.mid_block.attentions.0.", "mid.1.")
    n = n.replace("decoder.mid_block.resnets.1.", "mid.2.")
    n = n.replace("to_out.0.", "to_out.")
    for i in range(4):
        n = n.replace(f"decoder.up_blocks.{i}.upsamplers.0.conv.", f"upconvs.{i}.")
        for j in range(8):
            n = n.replace(f"decoder.up_blocks.{i}.resnets.{j}.", f"ups.{i}.{j}.")
    n = n.replace("decoder.conv_norm_out.", "norm_out.").replace("decoder.", "")
    return n


def test_sd_decoder_parameter_count():
    shapes = vae_ref.vae_param_shapes(vae_ref.sd_config())
    assert sum(int(np.prod(s)) for s in shapes.values()) == 49_490_199


@pytest.mark.parametrize("scale", [1.0, 1 / 0.18215])
def test_vae_ref_matches_torch_module(scale):
    cfg = vae_ref.small_config()
    sd = vae_ref.random_state_dict(cfg, seed=3)
    m = onnx_export.VAEDecoder(tuple(cfg["block_channels"])).double().eval()
    msd = m.state_dict()
    assert len(msd) == len(sd)
    with torch.no_grad():
        for k, v in sd.items():
            msd[module_name(k)].copy_(torch.from_numpy(v.astype(np.float64)))
    z = np.random.default_rng(4).standard_normal((2, 4, 8, 8)).astype(np.float32)
    with torch.no_grad():
        want = m(torch.from_numpy(z.astype(np.float64) * scale)).numpy()
    got = vae_ref.vae_decode(unet_ref.OracleOps(), sd, cfg, z, scale)
    assert got.shape == (2, 3, 64, 64)
    assert max_rel(got, want) <= 1e-4
