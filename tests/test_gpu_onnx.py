"""GPU: real ONNX graphs through the parser and the executor.

torch.onnx exports (opset 14) of a diffusers-style Transformer2D block
(scaled_dot_product_attention and eager attention), a ResnetBlock2D and a
reduced-width VAE decoder (channels 32/32/64/64, latent 8x8) are
parsed by drawinstant.onnx_parser and run by Executor, op by op as the
reference's executor would and after optimize_graph, against the modules'
float64 outputs.  Tolerances: the op-by-op fp32 path rel-L2 <= 1e-5 (1e-4
for the 35-convolution VAE) and max-rel <= 1e-4; the optimized graph the same except where flash attention
(fp16 MFMA operands) is in the path: rel-L2 <= 2e-3.
"""
import copy

import numpy as np
import pytest

from conftest import max_rel, rel_l2
from drawinstant.executor import Executor, WeightCache, optimize_graph
from drawinstant.onnx_parser import parse_onnx_graph
from golden import onnx_export

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cases():
    return {"sdpa": onnx_export.transformer_case(), "eager": onnx_export.transformer_case(eager=True),
            "resnet": onnx_export.resnet_case(), "vae": onnx_export.vae_case()}


def run(dev, g, feeds, reps=1):
    wc = WeightCache(dev, g.tensors)
    ex = Executor(dev, g, wc)
    try:
        res = []
        for _ in range(reps):
            outs = ex.run(feeds)
            t = outs["sample" if "sample" in outs else "y"]
            res.append(dev.download(t.buf, np.float32, tuple(t.dims)))
            t.buf.destroy()
        return res
    finally:
        ex.destroy()
        wc.destroy()


@pytest.mark.parametrize("key", ["sdpa", "eager", "resnet", "vae"])
@pytest.mark.parametrize("fused", [False, True])
def test_exported_block(dev, cases, key, fused):
    data, feeds, y = cases[key]
    g = parse_onnx_graph(data)
    if fused:
        g = copy.deepcopy(g)
        optimize_graph(g)
    out = run(dev, g, feeds, reps=2)
    print(f"[onnx] {key} fused={fused} nodes={len(g.nodes)} rel_l2={rel_l2(out[0], y):.2e} "
          f"max_rel={max_rel(out[0], y):.2e}", flush=True)
    assert np.array_equal(out[0], out[1])  # a second run through the reused pool
    if fused and key != "resnet":
        assert rel_l2(out[0], y) <= 2e-3
    else:
        # the VAE chains 35 fp32 convolutions and 30 GroupNorms (variance as
        # E[x^2] - E[x]^2, the reference's formula): rel-L2 1e-4 there
        assert rel_l2(out[0], y) <= (1e-4 if key == "vae" else 1e-5)
        assert max_rel(out[0], y) <= 1e-4


def as_fp16_file(g):
    """The same graph as an fp16 ONNX file would carry it (float initializers
    in fp16), like the SD-Turbo U-Net's."""
    g = copy.deepcopy(g)
    for t in g.tensors.values():
        if t.dtype == "float32":
            t.data = t.array().astype(np.float16).tobytes()
            t.dtype = "float16"
    return g


@pytest.mark.parametrize("key", ["sdpa", "resnet", "vae"])
@pytest.mark.parametrize("fused", [False, True])
def test_fp16_resident_weights(dev, cases, key, fused):
    """WeightCache(keep_f16=True): MatMul / Gemm / Conv weights stay fp16 on
    the device (DI_F32W16) and the run is bit-identical to the reference's
    widen-on-upload path, with the weight bytes nearly halved."""
    data, feeds, y = cases[key]
    g = as_fp16_file(parse_onnx_graph(data))
    if fused:
        optimize_graph(g)
    outs, nbytes = [], []
    for keep in (False, True):
        wc = WeightCache(dev, g.tensors, keep_f16=keep)
        ex = Executor(dev, g, wc)
        try:
            outs_run = ex.run(feeds)
            t = outs_run["sample" if "sample" in outs_run else "y"]
            outs.append(dev.download(t.buf, np.float32, tuple(t.dims)))
            t.buf.destroy()
            nbytes.append(wc.device_bytes)
        finally:
            ex.destroy()
            wc.destroy()
    print(f"[onnx-f16] {key} fused={fused} weight bytes {nbytes[0]} -> {nbytes[1]} "
          f"rel_l2 vs fp64 {rel_l2(outs[1], y):.2e}", flush=True)
    assert np.array_equal(outs[0], outs[1])
    assert nbytes[1] < 0.56 * nbytes[0]
    assert rel_l2(outs[1], y) <= 5e-3  # fp16-rounded weights


@pytest.mark.parametrize("key", ["resnet", "vae"])
@pytest.mark.parametrize("f16_weights", [False, True])
def test_conv_f16_compute_option(dev, cases, key, f16_weights):
    """Executor(conv_f16=True): Conv nodes on the fp16 MFMA path (operands
    rounded to fp16, fp32 accumulation), with fp32 or fp16-resident weights:
    rel-L2 <= 5e-3 against the modules' float64 output."""
    data, feeds, y = cases[key]
    g = parse_onnx_graph(data)
    optimize_graph(g)
    if f16_weights:
        g = as_fp16_file(g)
    wc = WeightCache(dev, g.tensors, keep_f16=f16_weights)
    ex = Executor(dev, g, wc, conv_f16=True)
    try:
        outs = ex.run(feeds)
        t = outs["sample" if "sample" in outs else "y"]
        got = dev.download(t.buf, np.float32, tuple(t.dims))
        t.buf.destroy()
    finally:
        ex.destroy()
        wc.destroy()
    e = rel_l2(got, y)
    print(f"[onnx-conv16] {key} f16_weights={f16_weights} rel_l2={e:.2e}", flush=True)
    assert e <= 5e-3
