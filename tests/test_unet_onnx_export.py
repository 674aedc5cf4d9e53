"""CPU: the whole SD2.1-architecture U-Net as an SD-Turbo-form ONNX graph
(fp32 I/O, int64 timestep, fp16 initializers; torch.onnx opset 14 export of
tests/golden/unet_module.py) parsed by drawinstant.onnx_parser and
evaluated by the numpy interpreter of tests/numpy_onnx.py, before and after
optimize_graph, against the module in float64 on the same (fp16-rounded)
weights.

This is the reference's target route (loadUNetWGSL -> rewrites ->
Executor.run over the U-Net graph, unet-wgsl.js:96-114, :145-195) checked
for graph semantics on the CPU: the numpy interpreter applies the graph's
fp16 Casts, so the bound is 1e-3 (fp16 rounding of the inputs and of the
LayerNorm / timestep-embedding outputs), and every rewrite must fire once
per block of the architecture: 48 LayerNorms (3 per transformer), 16 erf
GELUs, 32 attentions, 61 GroupNorms (2 per ResNet, 1 per transformer,
conv_norm_out), 45 of them with SiLU.
"""
import copy

import numpy as np
import pytest

from conftest import rel_l2
from oracle import unet_ref

torch = pytest.importorskip("torch")

import numpy_onnx  # noqa: E402
from drawinstant.executor import optimize_graph  # noqa: E402
from drawinstant.onnx_parser import parse_onnx_graph  # noqa: E402
from golden import unet_module  # noqa: E402


@pytest.fixture(scope="module")
def small_graph():
    cfg = unet_ref.small_config()
    data, feeds, sd16 = unet_module.export_case(cfg, unet_ref.random_state_dict(cfg, 3), 16, 16)
    m = unet_module.load(unet_module.from_config(cfg), sd16)
    with torch.no_grad():
        ref = m(torch.as_tensor(feeds["sample"], dtype=torch.float64),
                torch.as_tensor(feeds["timestep"]),
                torch.as_tensor(feeds["encoder_hidden_states"], dtype=torch.float64)).numpy()
    return data, feeds, ref


def test_graph_io_and_ops(small_graph):
    data, feeds, _ = small_graph
    g = parse_onnx_graph(data)
    assert [i["name"] for i in g.inputs] == ["sample", "timestep", "encoder_hidden_states"]
    assert [o["name"] for o in g.outputs] == ["out_sample"]
    ops = {n.op_type for n in g.nodes}
    # the timestep path (int64 input, Expand to the batch, sinusoid) and the
    # nearest upsampling are in the graph
    assert {"Cast", "Expand", "Sin", "Cos", "Resize", "Concat", "Conv", "MatMul",
            "Softmax", "InstanceNormalization", "Erf"} <= ops
    f16 = [t for t in g.tensors.values() if t.dtype == "float16"]
    assert len(f16) > 300


def test_whole_unet_graph_numpy(small_graph):
    data, feeds, ref = small_graph
    g = parse_onnx_graph(data)
    out = numpy_onnx.run(g, feeds)["out_sample"]
    e0 = rel_l2(out, ref)
    g2 = copy.deepcopy(g)
    stats = optimize_graph(g2)
    out2 = numpy_onnx.run(g2, feeds)["out_sample"]
    e1 = rel_l2(out2, ref)
    print(f"[unet-onnx] nodes {len(g.nodes)} -> {len(g2.nodes)} {stats} rel-L2 {e0:.2e} / {e1:.2e}")
    assert stats == {"silu": 47, "mul_add": 109, "group_norm": 61, "group_norm_silu": 45,
                     "layer_norm": 48, "gelu": 16, "attention": 32}
    assert e0 <= 1e-3 and e1 <= 1e-3
    assert rel_l2(out2, out) <= 1e-3
