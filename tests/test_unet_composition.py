"""CPU pins of the U-Net composition (oracle/unet_ref.py) against independent
torch modules in float64.

* blocks: ``unet_ref.resnet`` / ``unet_ref.transformer`` against
  tests/golden/onnx_export.py's ResnetBlock2D / Transformer2D (names mapped)
  and against tests/golden/unet_module.py's diffusers-named blocks;
* whole step: ``unet_ref.unet_forward`` (C oracle and torch-op backends)
  against the module-form UNet2DConditionModel of tests/golden/unet_module.py
  on the same weights, which also fixes the parameter names (strict load)
  and the SD2.1 parameter count;
* sensitivity: plausible wiring mistakes planted in the oracle's composition
  (skip concat order, [sin || cos] timestep sinusoid, swapped cross-attention
  flags) are caught by the same comparison.
"""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import unet_ref

torch = pytest.importorskip("torch")

from golden import onnx_export, unet_module  # noqa: E402


def _tiny_cfg():
    cfg = unet_ref.small_config()
    cfg.update(block_channels=[64, 64, 128, 128], cross_dim=64, time_dim=256)
    return cfg


def _inputs(cfg, B=1, H=16, W=16, S=7, seed=5):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, cfg["in_channels"], H, W)).astype(np.float32)
    ctx = rng.standard_normal((B, S, cfg["cross_dim"])).astype(np.float32)
    return x, ctx


def _module_out(cfg, sd, x, t, ctx):
    m = unet_module.load(unet_module.from_config(cfg), sd)
    with torch.no_grad():
        y = m(torch.as_tensor(x, dtype=torch.float64), torch.tensor([int(t)], dtype=torch.int64),
              torch.as_tensor(ctx, dtype=torch.float64))
    return y.numpy()


def test_module_names_and_sd21_parameter_count():
    with torch.device("meta"):
        m = unet_module.UNet2DConditionModel()
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    ref = unet_ref.unet_param_shapes(unet_ref.sd21_config())
    assert shapes == {k: tuple(v) for k, v in ref.items()}
    assert sum(int(np.prod(s)) for s in shapes.values()) == 865_910_724


def test_resnet_block_vs_modules():
    rng = np.random.default_rng(0)
    cin, cout, temb = 64, 128, 256
    sd = {k: v for k, v in unet_ref.random_state_dict(_tiny_cfg(), 1).items()
          if k.startswith("down_blocks.2.resnets.0.")}
    p = "down_blocks.2.resnets.0"
    x = rng.standard_normal((2, cin, 8, 8)).astype(np.float32)
    t = rng.standard_normal((2, temb)).astype(np.float32)
    ops = unet_ref.OracleOps()
    got = unet_ref.resnet(ops, {k: ops.asarray(v) for k, v in sd.items()}, p, x,
                          ops.silu(t), 1e-5, 32)
    local = {k[len(p) + 1:]: torch.as_tensor(v) for k, v in sd.items()}
    for mod in (onnx_export.ResnetBlock2D(cin, cout, temb),
                unet_module.ResnetBlock2D(cin, cout, temb)):
        mod.load_state_dict(local, strict=True)
        mod = mod.double().eval()
        with torch.no_grad():
            ref = mod(torch.as_tensor(x, dtype=torch.float64),
                      torch.as_tensor(t, dtype=torch.float64)).numpy()
        assert rel_l2(got, ref) < 1e-6, type(mod).__module__


def test_transformer_block_vs_modules():
    rng = np.random.default_rng(1)
    cfg = _tiny_cfg()
    C, X = 128, cfg["cross_dim"]
    p = "down_blocks.2.attentions.0"
    sd = {k: v for k, v in unet_ref.random_state_dict(cfg, 2).items() if k.startswith(p + ".")}
    x = rng.standard_normal((1, C, 8, 8)).astype(np.float32)
    ctx = rng.standard_normal((1, 11, X)).astype(np.float32)
    ops = unet_ref.OracleOps()
    got = unet_ref.transformer(ops, {k: ops.asarray(v) for k, v in sd.items()}, p, x, ctx)
    local = {k[len(p) + 1:]: torch.as_tensor(v) for k, v in sd.items()}
    # onnx_export's blocks hold the same tensors under shorter names
    renamed = {}
    for k, v in local.items():
        k2 = k.replace("transformer_blocks.0.", "").replace("ff.net.0.proj", "ff.proj")
        k2 = k2.replace("ff.net.2", "ff.out").replace("to_out.0", "to_out")
        renamed[k2] = v
    mods = ((onnx_export.Transformer2D(C, X, C // 64, 64), renamed),
            (unet_module.Transformer2DModel(C // 64, 64, C, X), local))
    for mod, state in mods:
        mod.load_state_dict(state, strict=True)
        mod = mod.double().eval()
        with torch.no_grad():
            ref = mod(torch.as_tensor(x, dtype=torch.float64),
                      torch.as_tensor(ctx, dtype=torch.float64)).numpy()
        assert rel_l2(got, ref) < 1e-6, type(mod).__module__


@pytest.mark.parametrize("cfg_name", ["tiny", "small"])
def test_unet_forward_vs_module(cfg_name):
    cfg = _tiny_cfg() if cfg_name == "tiny" else unet_ref.small_config()
    sd = unet_ref.random_state_dict(cfg, seed=3)
    x, ctx = _inputs(cfg, B=2 if cfg_name == "tiny" else 1)
    t = 999
    ref = _module_out(cfg, sd, x, t, ctx)
    got = unet_ref.unet_forward(unet_ref.OracleOps(), sd, cfg, x,
                                np.full(x.shape[0], t, np.float32), ctx)
    err = rel_l2(got, ref)
    print(f"[{cfg_name}] oracle composition vs module: rel-L2 {err:.2e}")
    assert err < 1e-5
    got_t = unet_ref.unet_forward(unet_ref.TorchOps("cpu"), sd, cfg, x,
                                  np.full(x.shape[0], t, np.float32), ctx).numpy()
    assert rel_l2(got_t, ref) < 1e-4


class _CatSwapped(unet_ref.OracleOps):
    def cat(self, xs, axis):  # skip first, then the running activation
        return np.concatenate(xs[::-1], axis=axis)


class _SinCos(unet_ref.OracleOps):
    def sinusoid(self, t, dim):  # [sin || cos]: flip_sin_to_cos forgotten
        e = super().sinusoid(t, dim)
        h = dim // 2
        return np.ascontiguousarray(np.concatenate([e[:, h:], e[:, :h]], axis=1))


@pytest.mark.parametrize("mistake", ["cat_order", "sin_cos", "cross_attn_flags"])
def test_planted_composition_mistakes_are_caught(mistake):
    cfg = _tiny_cfg()
    sd = unet_ref.random_state_dict(cfg, seed=4)
    x, ctx = _inputs(cfg)
    t = np.array([999.0], np.float32)
    ref = _module_out(cfg, sd, x, 999, ctx)
    ops, run_cfg = unet_ref.OracleOps(), dict(cfg)
    if mistake == "cat_order":
        ops = _CatSwapped()
        # concatenation order changes which input channels meet which
        # weights; shapes still agree when skip and running widths match
    elif mistake == "sin_cos":
        ops = _SinCos()
    else:
        run_cfg["cross_attn"] = [0, 1, 1, 1]
        # the flag swap needs transformer weights at the level that gains
        # one: add only the names the module's weights lack
        extra = unet_ref.random_state_dict(dict(cfg, cross_attn=[1, 1, 1, 1]), seed=9)
        sd = dict(sd, **{k: v for k, v in extra.items() if k not in sd})
    got = unet_ref.unet_forward(ops, sd, run_cfg, x, t, ctx)
    err = rel_l2(got, ref)
    print(f"[planted {mistake}] rel-L2 {err:.2e}")
    assert err > 1e-2, mistake
