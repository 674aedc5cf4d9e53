"""GPU: the whole SD2.1-architecture U-Net graph through the reference's
route — SD-Turbo-form ONNX file (fp32 I/O, int64 timestep, fp16
initializers; torch.onnx opset-14 export of tests/golden/unet_module.py)
-> drawinstant.onnx_parser -> optimize_graph -> Executor.run
(loadUNetWGSL + unetForwardWGSL, unet-wgsl.js:96-114, :145-195;
wgsl-executor.js:1248-1466).

* small config (channels 64/128/256/256, 16x16 latent, 3,284 nodes): op by
  op against the float64 module on the file's weights, rel-L2 <= 1e-4 (fp32
  executor; the graph's fp16 Casts are identities on the device, as in the
  reference's executor); after optimize_graph (2,148 nodes; flash attention
  with fp16 operands) rel-L2 <= 5e-3; fp16-resident weights bit-identical to
  widen-on-upload; a second run bit-identical, allocating nothing new, with
  the library's live-buffer count back where it started; and the native
  fp16 U-Net (di_unet) on the same weights within 1e-2 of the same module.
* SD2.1 at 64x64 (512x512 image): the same route against the module in
  float32 on the GPU, op by op rel-L2 <= 1e-4, optimized <= 5e-3.
"""
import copy
import time

import numpy as np
import pytest

from conftest import max_rel, rel_l2
from oracle import unet_ref

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from drawinstant.executor import Executor, WeightCache, optimize_graph  # noqa: E402
from drawinstant.onnx_parser import parse_onnx_graph  # noqa: E402
from golden import unet_module  # noqa: E402


def _run(dev, g, feeds, keep_f16=False, reps=1):
    """Outputs of ``reps`` runs, the executor's pool counters and the
    library's live-buffer count after each run."""
    wc = WeightCache(dev, g.tensors, keep_f16=keep_f16)
    ex = Executor(dev, g, wc)
    outs, allocs, live, ms = [], [], [], []
    try:
        for _ in range(reps):
            t0 = time.perf_counter()
            res = ex.run(feeds)["out_sample"]
            dev.sync()
            ms.append(round((time.perf_counter() - t0) * 1e3, 1))
            outs.append(dev.download(res.buf, np.float32, tuple(res.dims)))
            res.buf.destroy()
            allocs.append(ex.pool.allocs)
            live.append(dev.pool_stats()["live"])
        info = {"allocs": allocs, "live": live, "peak_bytes": ex.pool.peak_bytes,
                "weight_bytes": wc.device_bytes, "ms": ms}
    finally:
        ex.destroy()
        wc.destroy()
    return outs, info


@pytest.fixture(scope="module")
def small():
    cfg = unet_ref.small_config()
    data, feeds, sd16 = unet_module.export_case(cfg, unet_ref.random_state_dict(cfg, 3), 16, 16)
    m = unet_module.load(unet_module.from_config(cfg), sd16)
    with torch.no_grad():
        ref = m(torch.as_tensor(feeds["sample"], dtype=torch.float64),
                torch.as_tensor(feeds["timestep"]),
                torch.as_tensor(feeds["encoder_hidden_states"], dtype=torch.float64)).numpy()
    return cfg, data, feeds, sd16, ref


def test_small_unet_graph_op_by_op(dev, small):
    _, data, feeds, _, ref = small
    g = parse_onnx_graph(data)
    outs, info = _run(dev, g, feeds, reps=2)
    e = rel_l2(outs[0], ref)
    print(f"[unet-onnx] small op-by-op nodes={len(g.nodes)} rel_l2={e:.2e} "
          f"max_rel={max_rel(outs[0], ref):.2e} {info}", flush=True)
    assert e <= 1e-4
    assert np.array_equal(outs[0], outs[1])
    assert info["allocs"][1] == info["allocs"][0]  # the second run reuses the pool
    assert info["live"][1] == info["live"][0]  # nothing leaks per run


def test_small_unet_graph_optimized(dev, small):
    _, data, feeds, _, ref = small
    g = parse_onnx_graph(data)
    stats = optimize_graph(g)
    outs = {}
    for keep in (False, True):
        o, info = _run(dev, g, feeds, keep_f16=keep)
        outs[keep] = (o[0], info)
    e = rel_l2(outs[False][0], ref)
    print(f"[unet-onnx] small optimized nodes={len(g.nodes)} {stats} rel_l2={e:.2e} "
          f"weights {outs[False][1]['weight_bytes']} -> {outs[True][1]['weight_bytes']} "
          f"peak pool bytes {outs[False][1]['peak_bytes']}", flush=True)
    assert len(g.nodes) == 2148 and stats["attention"] == 32 and stats["layer_norm"] == 48
    assert e <= 5e-3
    assert np.array_equal(outs[False][0], outs[True][0])
    assert outs[True][1]["weight_bytes"] < 0.56 * outs[False][1]["weight_bytes"]


def test_native_unet_on_the_file_weights(dev, small):
    """The product path (di_unet, fp16 NHWC) loaded with the ONNX file's
    weights against the same float64 module."""
    from drawinstant.unet import UNet, UNetConfig
    cfg, _, feeds, sd16, ref = small
    u = UNet(dev, UNetConfig.small(), seed=0)
    try:
        u.load_state_dict(sd16)
        got = u(feeds["sample"], float(feeds["timestep"][0]), feeds["encoder_hidden_states"])
    finally:
        u.destroy()
    e = rel_l2(got, ref)
    print(f"[unet-onnx] native di_unet on the file weights rel_l2={e:.2e}", flush=True)
    assert e <= 1e-2


@pytest.mark.timeout(600)
def test_sd21_unet_graph(dev):
    """Full SD2.1 (865.9 M parameters, a 1.73 GB fp16 ONNX file) at a 64x64
    latent through parser + Executor, op by op and optimized, against the
    module in float32 on the GPU."""
    cfg = unet_ref.sd21_config()
    t0 = time.perf_counter()
    data, feeds, sd16 = unet_module.export_case(cfg, unet_ref.random_state_dict(cfg, 21), 64, 64,
                                                device="cuda")
    t_export = time.perf_counter() - t0
    m = unet_module.load(unet_module.from_config(cfg), sd16, dtype=torch.float32).cuda()
    del sd16
    with torch.no_grad():
        ref = m(torch.as_tensor(feeds["sample"]).cuda(), torch.as_tensor(feeds["timestep"]).cuda(),
                torch.as_tensor(feeds["encoder_hidden_states"]).cuda()).cpu().numpy()
    del m
    torch.cuda.empty_cache()
    g = parse_onnx_graph(data)
    del data
    n0 = len(g.nodes)
    o, info = _run(dev, g, feeds, reps=2)
    e0 = rel_l2(o[1], ref)
    print(f"[unet-onnx] sd21 export {t_export:.1f}s nodes={n0} op-by-op rel_l2={e0:.2e} "
          f"{info}", flush=True)
    stats = optimize_graph(g)
    o2, info2 = _run(dev, g, feeds, reps=2)
    e1 = rel_l2(o2[1], ref)
    print(f"[unet-onnx] sd21 optimized nodes={len(g.nodes)} {stats} rel_l2={e1:.2e} {info2}",
          flush=True)
    assert e0 <= 1e-4 and e1 <= 5e-3
