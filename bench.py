#!/usr/bin/env python3
"""Headline benchmark: one SD-Turbo (SD2.1) U-Net denoise step at 512x512
(latent [1,4,64,64]), batch 1, on one MI355X - BASELINE.json's metric
"U-Net step ms @512^2 b1 (1 GPU); per-block MFMA util % / HBM GB/s".

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Prints ONE JSON line.  `value` = ms per step (lower is better), timed with
HIP events on the library's stream over exactly K graph-replayed steps
(bracketed by device synchronisation), inputs resident in HBM.

* `roofline`: the dominant conv shape, conv3x3 320->320 on 64x64 NHWC fp16
  (seven launches per step; also BASELINE cfg2), which the plan routes to the
  halo conv kernel (k_conv3_halo), timed live with HIP events on the stream
  it is launched on.  achieved = 2*HW*Cout*Cin*9 FLOP per launch / average
  launch time; `traffic` = HBM bytes per launch from the committed rocprofv3
  FETCH_SIZE / WRITE_SIZE summary (null without it).
* `cpu_baseline`: one whole step of the repo's C restatement of the
  reference kernels (oracle/, OpenMP, fp32 accumulation build) composed as
  the same U-Net with the same weights, on the host cores.  Skipped with
  --no-cpu.
* `blocks` (unless --no-blocks): per-config figures (cfg1 GN+SiLU HBM GB/s,
  cfg2 conv / cfg3 ResNet / cfg4 transformer / self-attention / GEGLU FFN
  MFMA %).  `--blocks-only` prints just these (the leg the per-block
  rocprofv3 counter passes run).
* `denoise_loop`: the 4-step SD-Turbo loop (noise, scaleModelInput, U-Net,
  Euler update) entirely on the device, host wall time including the final
  wait.  `batch4`: the same step at B=4 (cfg5's other batch), ms per step
  and per sample.
* `executor_rewrites` (unless --no-blocks): the op-by-op executor over the
  exported cfg4 attention and LayerNorm + GELU subgraphs, unfused and after
  optimize_graph, wall ms per run.
* `executor_onnx_cfg4` (unless --no-blocks): the same for a real ONNX file,
  torch.onnx's export of the cfg4 transformer block, through the parser.
* `vae_decode_512` (unless --no-blocks): SD's VAE decoder as the native
  di_vae object, [1,4,64,64] -> [1,3,512,512], graph replay, TFLOP/s over
  the decode's 2.51 TFLOP; `executor_vae_decode_512`: the same decode the
  way vae-wgsl.js runs it, the exported decoder through parser + executor.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "draw-instant_amd"))

import numpy as np  # noqa: E402

METRIC = "U-Net step ms @512² b1 (1 GPU); per-block MFMA util % / HBM GB/s"
TIMER = 0


def timed(dev, fn, iters):
    """Average ms of `fn` over `iters` back-to-back calls (HIP events on the
    library stream, device synchronised on both sides)."""
    dev.sync()
    dev.timer_begin(TIMER)
    for i in range(iters):
        fn(i)
    dev.timer_end(TIMER)
    ms = dev.timer_ms(TIMER)
    dev.sync()
    return ms / iters


def step_spread(dev, step, batch=10, batches=9, slope_reps=7):
    """Spread of the graph-replayed step, measured after the headline's K
    steps: (a) `batches` batches of `batch` back-to-back replays, each
    bracketed by HIP events (ms per step: median and interquartile range);
    (b) the reference's slope method (bench-timing.js:49-97): interleaved
    batches of N and 2N replays, (t2N - tN) / N, median and IQR of
    `slope_reps` pairs, which cancels the per-batch fixed cost."""
    per = [timed(dev, step, batch) for _ in range(batches)]
    slopes = []
    for _ in range(slope_reps):
        t1 = timed(dev, step, batch) * batch
        t2 = timed(dev, step, 2 * batch) * 2 * batch
        slopes.append((t2 - t1) / batch)
    q = np.percentile(per, [25, 50, 75])
    qs = np.percentile(slopes, [25, 50, 75])
    return {"batches": {"n": batches, "steps_each": batch, "median_ms": round(float(q[1]), 4),
                        "iqr_ms": [round(float(q[0]), 4), round(float(q[2]), 4)],
                        "min_ms": round(float(min(per)), 4), "max_ms": round(float(max(per)), 4)},
            "slope": {"n": slope_reps, "N": batch, "median_ms": round(float(qs[1]), 4),
                      "iqr_ms": [round(float(qs[0]), 4), round(float(qs[2]), 4)]}}


def bench_unet(dev, args):
    from drawinstant.unet import UNet
    u = UNet(dev, seed=501)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 4, 64, 64)).astype(np.float32)
    ctx = rng.standard_normal((1, 77, 1024)).astype(np.float32)
    bs, bc = dev.storage(x), dev.storage(ctx)
    bt = dev.storage(np.array([999.0], np.float32))
    bo = dev.create_buffer(x.nbytes)
    step = lambda i, g=True: u.forward(bs, bt, bc, bo, 1, 64, 64, 77, graph=g)
    for i in range(max(args.warmup, 1)):
        step(i)
    dev.sync()
    try:
        import torch
        torch.cuda.synchronize()
    except Exception:
        pass
    t0 = time.perf_counter()
    ms = timed(dev, step, args.steps)
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    spread = step_spread(dev, step)
    eager = timed(dev, lambda i: step(i, False), max(2, args.steps // 4))
    out = dev.download(bo, np.float32, x.shape)
    finite = bool(np.isfinite(out).all())
    return u, ms, wall, eager, finite, (x, ctx), spread


def bench_unet_batch(dev, u, B=4, iters=20):
    """The same step at batch B (cfg5's B=4): ms per step and per sample."""
    rng = np.random.default_rng(4)
    x = dev.storage(rng.standard_normal((B, 4, 64, 64)).astype(np.float32))
    c = dev.storage(rng.standard_normal((B, 77, 1024)).astype(np.float32))
    t = dev.storage(np.full(B, 999.0, np.float32))
    o = dev.create_buffer(B * 4 * 64 * 64 * 4)
    try:
        step = lambda i: u.forward(x, t, c, o, B, 64, 64, 77, graph=True)
        for i in range(5):
            step(i)
        ms = timed(dev, step, iters)
        out = dev.download(o, np.float32, (B * 4 * 64 * 64,))
        return {"batch": B, "ms_per_step": round(ms, 4), "ms_per_sample": round(ms / B, 4),
                "output_finite": bool(np.isfinite(out).all())}
    finally:
        for b in (x, c, t, o):
            b.destroy()


def bench_denoise(dev, u, ctx, steps=4, reps=21):
    """The SD-Turbo denoise loop (pipeline.js:274-288) on the device: noise,
    then per step scaleModelInput -> U-Net (graph) -> Euler update (scheduler
    kernels, no host round trip).  Interleaved A/B: each rep times the whole
    loop (A) and, right after, the same `steps` graph replays on the same
    buffers without the scheduler kernels (B), each bracketed by HIP events;
    `scheduler_us_per_step` is the median of (A - B) / steps with its
    interquartile range."""
    from drawinstant import scheduler as S
    bc = dev.storage(ctx)
    lat = dev.create_buffer(4 * 64 * 64 * 4)
    d = S.Denoiser(u, steps=steps)
    d.run(bc, lat, seed=0)  # capture with these buffers
    dev.sync()

    def bare(i):
        for _ in range(steps):
            u.forward(d.model_in, d.tbuf, bc, d.pred, 1, 64, 64, 77, graph=True)
    loop, diff = [], []
    for _ in range(reps):
        a = timed(dev, lambda i: d.run(bc, lat, seed=0), 1)
        b = timed(dev, bare, 1)
        loop.append(a)
        diff.append((a - b) / steps * 1e3)
    d.run(bc, lat, seed=0)
    out = dev.download(lat, np.float32)
    d.destroy()
    for b in (bc, lat):
        b.destroy()
    ms = float(np.median(loop))
    q = np.percentile(diff, [25, 50, 75])
    return {"steps": steps, "ms": round(ms, 4), "ms_per_step": round(ms / steps, 4),
            "scheduler_us_per_step": round(float(q[1]), 2),
            "scheduler_us_per_step_iqr": [round(float(q[0]), 2), round(float(q[2]), 2)],
            "method": f"median of {reps} interleaved A/B pairs (loop vs {steps} bare replays)",
            "final_latent_finite": bool(np.isfinite(out).all())}


def bench_blocks(dev, num_rot=64):
    """cfg1..cfg4 micro-benchmarks, live HIP-event timing."""
    import drawinstant
    from drawinstant import blocks, perf
    from drawinstant.device import call
    res = {}
    rng = np.random.default_rng(1)
    # cfg1: GN32+SiLU fp32 NCHW [1,320,64,64]; rotate 64 x 10.5 MB buffer pairs
    # (> 2 x 256 MB Infinity Cache) so every launch reads HBM
    N, C, HW = 1, 320, 4096
    xs = [dev.create_buffer(N * C * HW * 4) for _ in range(num_rot)]
    ys = [dev.create_buffer(N * C * HW * 4) for _ in range(num_rot)]
    for i, b in enumerate(xs):
        dev.fill_normal(b, N * C * HW, 101 + i)
    g = dev.storage((1 + 0.02 * rng.standard_normal(C)).astype(np.float32))
    bb = dev.storage((0.02 * rng.standard_normal(C)).astype(np.float32))
    gn = lambda i: call("di_gn_silu", dev.ctx, xs[i % num_rot].handle, g.handle, bb.handle,
                        ys[i % num_rot].handle, N, C, 32, HW, 1e-5, 0, 0)
    for i in range(num_rot):
        gn(i)
    ms = timed(dev, gn, 4 * num_rot)
    nbytes = perf.gn_silu_bytes(N, C, HW)
    res["cfg1_gn_silu"] = {"us": ms * 1e3, "GBps": nbytes / (ms * 1e-3) / 1e9,
                           "hbm_frac": nbytes / (ms * 1e-3) / perf.PEAK_HBM_BYTES,
                           "bytes": nbytes}
    for b in xs + ys:
        b.destroy()
    # cfg2: conv3x3 320->320 @64x64, fp16 NHWC implicit GEMM
    x = dev.storage(rng.standard_normal((1, 64, 64, 320)).astype(np.float16))
    w = dev.storage((rng.standard_normal((320, 3, 3, 320)) * 0.026).astype(np.float16))
    bias = dev.storage(np.zeros(320, np.float32))
    y = dev.create_buffer(64 * 64 * 320 * 2)
    conv = lambda i: call("di_conv2d", dev.ctx, x.handle, w.handle, bias.handle, 0, y.handle, 1,
                          320, 320, 64, 64, 3, 1, 1, 0, 1, 1)
    conv(0)
    ms = timed(dev, conv, 50)
    fl = perf.conv_flops(1, 320, 320, 64, 64, 3)
    res["cfg2_conv3x3"] = {"us": ms * 1e3, "TFLOPs": fl / (ms * 1e-3) / 1e12,
                           "mfma_frac": fl / (ms * 1e-3) / perf.PEAK_FP16_FLOPS, "flops": fl}
    # self-attention at 64x64: 5 heads x 4096 tokens x 64
    q = dev.storage(rng.standard_normal((1, 4096, 5, 64)).astype(np.float16))
    o = dev.create_buffer(4096 * 320 * 2)
    att = lambda i: call("di_attn_self", dev.ctx, q.handle, q.handle, q.handle, o.handle, 1, 5,
                         4096, 64, 0, 0.0, 1)
    att(0)
    ms = timed(dev, att, 50)
    fl = 4.0 * 4096 * 4096 * 320
    res["self_attn_64x64"] = {"us": ms * 1e3, "TFLOPs": fl / (ms * 1e-3) / 1e12,
                              "mfma_frac": fl / (ms * 1e-3) / perf.PEAK_FP16_FLOPS, "flops": fl}
    # GEGLU FFN at 64x64 (down_blocks.0 transformer): 4096 x 320 -> 2x1280
    # (GELU-gated) -> 320, plus the residual, two GEMM launches (di_ffn)
    rows, D, F = 4096, 320, 1280
    fx = dev.storage(rng.standard_normal((rows, D)).astype(np.float16))
    w1 = dev.storage((rng.standard_normal((2 * F, D)) * 0.04).astype(np.float16))
    b1 = dev.storage(np.zeros(2 * F, np.float32))
    w2 = dev.storage((rng.standard_normal((D, F)) * 0.025).astype(np.float16))
    b2 = dev.storage(np.zeros(D, np.float32))
    fy = dev.create_buffer(rows * D * 2)
    ffn = lambda i: call("di_ffn", dev.ctx, fx.handle, w1.handle, b1.handle, w2.handle, b2.handle,
                         fy.handle, rows, D, F, 2, 1)
    ffn(0)
    ms = timed(dev, ffn, 50)
    fl = 2.0 * rows * D * 2 * F + 2.0 * rows * F * D
    res["ffn_geglu_64x64"] = {"us": ms * 1e3, "TFLOPs": fl / (ms * 1e-3) / 1e12,
                              "mfma_frac": fl / (ms * 1e-3) / perf.PEAK_FP16_FLOPS, "flops": fl}
    # cfg4 cross-attention (fused-cross-attn.js:112-173): 4096 queries x 5
    # heads x 64 against the 77 context tokens, fp16 [B,S,H,d]
    cq = dev.storage(rng.standard_normal((1, 4096, 5, 64)).astype(np.float16))
    ck = dev.storage(rng.standard_normal((1, 77, 5, 64)).astype(np.float16))
    cv = dev.storage(rng.standard_normal((1, 77, 5, 64)).astype(np.float16))
    co = dev.create_buffer(4096 * 320 * 2)
    xatt = lambda i: call("di_attn_cross", dev.ctx, cq.handle, ck.handle, cv.handle, co.handle, 1,
                          5, 4096, 77, 64, 0, 0.0, 1)
    xatt(0)
    ms = timed(dev, xatt, 100)
    fl = 4.0 * 4096 * 77 * 320
    res["cross_attn_64x64"] = {"us": ms * 1e3, "TFLOPs": fl / (ms * 1e-3) / 1e12,
                               "mfma_frac": fl / (ms * 1e-3) / perf.PEAK_FP16_FLOPS, "flops": fl}
    # timestep embedding (fused-tembed.js:73-130): sinusoid(t) -> Linear
    # 320->1280 + SiLU -> Linear 1280->1280, fp16 weights, B = 1; the weights
    # rotate over 96 copies (> 256 MB Infinity Cache), as a step reads them cold
    E, Hd, nrot = 320, 1280, 96
    tt = dev.storage(np.array([999.0], np.float32))
    tw1 = [dev.create_buffer(Hd * E * 2) for _ in range(nrot)]
    tw2 = [dev.create_buffer(Hd * Hd * 2) for _ in range(nrot)]
    for i in range(nrot):
        dev.fill_normal(tw1[i], Hd * E, 7000 + i, 0.0, 0.05, dtype=np.float16)
        dev.fill_normal(tw2[i], Hd * Hd, 8000 + i, 0.0, 0.03, dtype=np.float16)
    tb1 = dev.storage((0.02 * rng.standard_normal(Hd)).astype(np.float32))
    tb2 = dev.storage((0.02 * rng.standard_normal(Hd)).astype(np.float32))
    ty = dev.create_buffer(Hd * 4)
    temb = lambda i: call("di_tembed", dev.ctx, tt.handle, tw1[i % nrot].handle, tb1.handle,
                          tw2[i % nrot].handle, tb2.handle, ty.handle, 1, E, Hd, 1)
    for i in range(nrot):
        temb(i)
    ms = timed(dev, temb, 2 * nrot)
    nbytes = 2 * (Hd * E + Hd * Hd) + 4 * (2 * Hd + 1 + Hd)
    res["tembed_1280"] = {"us": ms * 1e3, "GBps": nbytes / (ms * 1e-3) / 1e9,
                          "hbm_frac": nbytes / (ms * 1e-3) / perf.PEAK_HBM_BYTES, "bytes": nbytes,
                          "launches": 2}
    for b in tw1 + tw2 + [tt, tb1, tb2, ty, cq, ck, cv, co]:
        b.destroy()
    return res


def bench_block_chains(dev, u):
    """cfg3 / cfg4 through the fused-block entry points, with the SD2.1
    U-Net's own weights of those blocks (down_blocks.1.resnets.0 is the
    320->640 @32x32 ResNet, down_blocks.0.attentions.0 the 320-channel
    64x64 transformer)."""
    from drawinstant import blocks, perf
    res = {}
    rng = np.random.default_rng(2)
    sd = u.state_dict(np.float32)
    rw = blocks.upload_resnet(dev, sd, "down_blocks.1.resnets.0")
    x = dev.storage(rng.standard_normal((1, 32, 32, 320)).astype(np.float16))
    t = dev.storage(rng.standard_normal((1, 1280)).astype(np.float32))
    y = dev.create_buffer(32 * 32 * 640 * 2)
    run = lambda i: blocks.resnet_block(dev, rw, x, t, y, 1, 320, 640, 32, 32)
    run(0)
    ms = timed(dev, run, 30)
    w = perf.Work()
    perf.resnet_flops(w, 1, 320, 640, 32, 32)
    res["cfg3_resnet"] = {"us": ms * 1e3, "TFLOPs": w.total / (ms * 1e-3) / 1e12,
                          "mfma_frac": w.total / (ms * 1e-3) / perf.PEAK_FP16_FLOPS,
                          "flops": w.total}
    tw = blocks.upload_transformer(dev, sd, "down_blocks.0.attentions.0")
    x2 = dev.storage(rng.standard_normal((1, 64, 64, 320)).astype(np.float16))
    c2 = dev.storage(rng.standard_normal((1, 77, 1024)).astype(np.float16))
    y2 = dev.create_buffer(64 * 64 * 320 * 2)
    run2 = lambda i: blocks.transformer_block(dev, tw, x2, c2, y2, 1, 320, 64, 64)
    run2(0)
    ms = timed(dev, run2, 20)
    w = perf.Work()
    perf.transformer_flops(w, 1, 320, 64, 64)
    res["cfg4_transformer"] = {"us": ms * 1e3, "TFLOPs": w.total / (ms * 1e-3) / 1e12,
                               "mfma_frac": w.total / (ms * 1e-3) / perf.PEAK_FP16_FLOPS,
                               "flops": w.total}
    rw.destroy()
    tw.destroy()
    return res


def _export_subgraphs(S=4096, H=5, d=64, D=320, F=1280):
    """The cfg4 (64x64 level) attention and LayerNorm + GELU chains as
    torch.onnx exports them, for the executor-rewrite leg."""
    from drawinstant.executor import Attr, Graph, Node, TensorProto

    def tp(a):
        a = np.ascontiguousarray(a, np.float32)
        return TensorProto(list(a.shape), "float32", a.tobytes())

    perm = [Attr("perm", ints=[0, 2, 1, 3])]
    attn = Graph([
        Node("Transpose", "tq", ["q"], ["qh"], perm),
        Node("Transpose", "tk", ["k"], ["kh"], [Attr("perm", ints=[0, 2, 3, 1])]),
        Node("Transpose", "tv", ["v"], ["vh"], perm), Node("MatMul", "qk", ["qh", "kh"], ["s"]),
        Node("Mul", "sc", ["s", "scale"], ["ss"]),
        Node("Softmax", "sm", ["ss"], ["p"], [Attr("axis", i=-1)]),
        Node("MatMul", "pv", ["p", "vh"], ["o"]), Node("Transpose", "to", ["o"], ["y"], perm)],
        outputs=[{"name": "y"}], tensors={"scale": tp(np.array([d ** -0.5]))})
    rng = np.random.default_rng(3)
    rm = [Attr("axes", ints=[-1])]
    t = {"two": tp([2.0]), "eps": tp([1e-5]), "g": tp(1 + 0.02 * rng.standard_normal(D)),
         "b": tp(0.02 * rng.standard_normal(D)), "sq2": tp([2 ** 0.5]), "one": tp([1.0]),
         "half": tp([0.5]), "w": tp(0.03 * rng.standard_normal((D, F)))}
    ln_gelu = Graph([
        Node("ReduceMean", "rm1", ["x"], ["mu"], rm), Node("Sub", "sub", ["x", "mu"], ["xc"]),
        Node("Pow", "pw", ["xc", "two"], ["x2"]), Node("ReduceMean", "rm2", ["x2"], ["var"], rm),
        Node("Add", "ae", ["var", "eps"], ["ve"]), Node("Sqrt", "sq", ["ve"], ["sd"]),
        Node("Div", "dv", ["xc", "sd"], ["xn"]), Node("Mul", "mg", ["xn", "g"], ["xg"]),
        Node("Add", "ab", ["xg", "b"], ["ln"]), Node("MatMul", "ff", ["ln", "w"], ["h"]),
        Node("Div", "d2", ["h", "sq2"], ["u"]), Node("Erf", "erf", ["u"], ["e"]),
        Node("Add", "a1", ["e", "one"], ["e1"]), Node("Mul", "mx", ["h", "e1"], ["pg"]),
        Node("Mul", "mh", ["pg", "half"], ["y"])], outputs=[{"name": "y"}], tensors=t)
    feeds_attn = {n: rng.standard_normal((1, S, H, d)).astype(np.float32) for n in "qkv"}
    feeds_ln = {"x": rng.standard_normal((1, S, D)).astype(np.float32)}
    return (attn, feeds_attn), (ln_gelu, feeds_ln)


def bench_executor_rewrites(dev, reps=7):
    """The executor over exported subgraphs at the cfg4 shapes, op by op
    (as the reference's executor dispatches them) and after optimize_graph:
    wall ms per Executor.run (median of `reps`, device-synchronised)."""
    import copy
    from drawinstant.executor import Executor, Tensor, WeightCache, optimize_graph
    res = {}
    for key, (graph, feeds) in zip(("attention_64x64", "layer_norm_gelu_64x64"),
                                   _export_subgraphs()):
        inputs = {k: dev.storage(v) for k, v in feeds.items()}
        seeds = {k: Tensor(b, list(feeds[k].shape)) for k, b in inputs.items()}
        row = {}
        for fused in (False, True):
            g = copy.deepcopy(graph)
            if fused:
                row["rewrites"] = {k: v for k, v in optimize_graph(g).items() if v}
            wc = WeightCache(dev, g.tensors)
            ex = Executor(dev, g, wc)
            ts = []
            for r in range(reps + 1):
                t0 = time.perf_counter()
                outs = ex.run(seeds)
                dt = (time.perf_counter() - t0) * 1e3
                for o in outs.values():
                    o.buf.destroy()
                if r:
                    ts.append(dt)
            ts.sort()
            row["fused_ms" if fused else "unfused_ms"] = round(ts[len(ts) // 2], 4)
            row["fused_nodes" if fused else "unfused_nodes"] = len(g.nodes)
            ex.destroy()
            wc.destroy()
        row["speedup"] = round(row["unfused_ms"] / row["fused_ms"], 2)
        res[key] = row
        for b in inputs.values():
            b.destroy()
    return res


def bench_executor_onnx(dev, reps=5):
    """A real ONNX graph: torch.onnx's opset-14 export of the cfg4 block (the
    SD2.1 64x64 Transformer2D: C 320, 5 heads x 64, context [1,77,1024],
    scaled_dot_product_attention), written by the test fixture generator,
    parsed by drawinstant.onnx_parser and run by Executor op by op and after
    optimize_graph; wall ms per run (median of `reps`)."""
    import copy
    sys.path.insert(0, os.path.join(REPO, "tests"))
    from golden import onnx_export
    from drawinstant.executor import Executor, Tensor, WeightCache, optimize_graph
    from drawinstant.onnx_parser import parse_onnx_graph
    data, feeds, _ = onnx_export.transformer_case(C=320, heads=5, head_dim=64, H=64, W=64,
                                                  Sctx=77, ctx_dim=1024)
    graph = parse_onnx_graph(data)
    inputs = {k: dev.storage(v) for k, v in feeds.items()}
    seeds = {k: Tensor(b, list(feeds[k].shape)) for k, b in inputs.items()}
    row = {"onnx_bytes": len(data), "exported_nodes": len(graph.nodes)}
    # unfused / fused as exported (fp32 initializers); then fused with the
    # initializers in fp16 as the SD-Turbo file carries them, widened on
    # upload (the reference's WeightCache) or kept fp16 on the device
    for key in ("unfused", "fused", "fused_f16file_widened", "fused_f16_resident"):
        g = copy.deepcopy(graph)
        if key != "unfused":
            st = {k: v for k, v in optimize_graph(g).items() if v}
            row.setdefault("rewrites", st)
        if "f16" in key:
            for t in g.tensors.values():
                if t.dtype == "float32":
                    t.data, t.dtype = t.array().astype(np.float16).tobytes(), "float16"
        wc = WeightCache(dev, g.tensors, keep_f16=key == "fused_f16_resident")
        ex = Executor(dev, g, wc)
        ts = []
        for r in range(reps + 1):
            t0 = time.perf_counter()
            outs = ex.run(seeds)
            dt = (time.perf_counter() - t0) * 1e3
            for o in outs.values():
                o.buf.destroy()
            if r:
                ts.append(dt)
        ts.sort()
        row[key] = {"ms": round(ts[len(ts) // 2], 3), "nodes": len(g.nodes),
                    "weight_bytes_on_device": wc.device_bytes}
        ex.destroy()
        wc.destroy()
    row["speedup_fused"] = round(row["unfused"]["ms"] / row["fused"]["ms"], 2)
    for b in inputs.values():
        b.destroy()
    return row


def bench_vae(dev, iters=10, graph=True):
    """SD's VAE decoder as one native object (di_vae_decode): latent
    [1,4,64,64] -> image [1,3,512,512], seeded weights, graph replay (or
    eager launches); HIP events on the library stream."""
    from drawinstant import perf
    from drawinstant.vae import VAE
    v = VAE(dev, seed=0)
    z = dev.create_buffer(4 * 64 * 64 * 4)
    dev.fill_normal(z, 4 * 64 * 64, 11)
    img = dev.create_buffer(3 * 512 * 512 * 4)
    try:
        run = lambda i: v.decode(z, img, 1, 64, 64, graph=graph)
        run(0)
        run(0)
        ms = timed(dev, run, iters)
        out = dev.download(img, np.float32, (3 * 512 * 512,))
        fl = perf.vae_work().total
        return {"ms": round(ms, 3), "gflop": round(fl / 1e9, 1),
                "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                "mfma_frac": round(fl / (ms * 1e-3) / perf.PEAK_FP16_FLOPS, 4),
                "image_finite": bool(np.isfinite(out).all())}
    finally:
        z.destroy()
        img.destroy()
        v.destroy()


def bench_executor_vae(dev, reps=3):
    """The VAE decode of vae-wgsl.js: torch.onnx's export of SD's VAE decoder
    (post_quant_conv + Decoder, channels 128/256/512/512, seeded weights,
    latent [1,4,64,64] -> image [1,3,512,512]) parsed and run by Executor op
    by op, after optimize_graph, and with fp16-resident weights; wall ms per
    decode (median of `reps`)."""
    import copy
    sys.path.insert(0, os.path.join(REPO, "tests"))
    from golden import onnx_export
    from drawinstant.executor import Executor, Tensor, WeightCache, optimize_graph
    from drawinstant.onnx_parser import parse_onnx_graph
    data, feeds, _ = onnx_export.vae_case(channels=(128, 256, 512, 512), latent_hw=64,
                                          expected=False)
    graph = parse_onnx_graph(data)
    del data
    z = dev.storage(feeds["latent"] / 0.18215)  # vae-wgsl.js scaling
    seeds = {"latent": Tensor(z, [1, 4, 64, 64])}
    row = {"exported_nodes": len(graph.nodes), "weights_mb": round(graph.bytes / 2 ** 20, 1)}
    for key in ("unfused", "fused", "fused_f16_resident", "fused_conv_f16"):
        g = copy.deepcopy(graph)
        if key != "unfused":
            row.setdefault("rewrites", {k: v for k, v in optimize_graph(g).items() if v})
        if "f16_resident" in key:
            for t in g.tensors.values():
                if t.dtype == "float32":
                    t.data, t.dtype = t.array().astype(np.float16).tobytes(), "float16"
        wc = WeightCache(dev, g.tensors, keep_f16="f16_resident" in key)
        ex = Executor(dev, g, wc, conv_f16=key == "fused_conv_f16")
        ts = []
        for r in range(reps + 1):
            t0 = time.perf_counter()
            outs = ex.run(seeds)
            dt = (time.perf_counter() - t0) * 1e3
            for o in outs.values():
                if o.buf is not None:
                    o.buf.destroy()
            if r:
                ts.append(dt)
        ts.sort()
        row[key] = {"ms": round(ts[len(ts) // 2], 2), "nodes": len(g.nodes),
                    "pool_peak_buffers": ex.pool.peak}
        ex.destroy()
        wc.destroy()
    z.destroy()
    return row


ROOFLINE_PMC = os.path.join(REPO, "profiles", "k_conv3_halo_conv3x3_64x64x320_pmc.md")


def roofline_conv(dev, iters=200, cold=True):
    """Live roofline of the dominant kernel at its U-Net shape (warm: the
    same weights every launch; `cold`: also with the weights from HBM)."""
    from drawinstant import perf
    from drawinstant.device import call
    rng = np.random.default_rng(3)
    x = dev.storage(rng.standard_normal((1, 64, 64, 320)).astype(np.float16))
    w = dev.storage((rng.standard_normal((320, 3, 3, 320)) * 0.026).astype(np.float16))
    bias = dev.storage((0.01 * rng.standard_normal(320)).astype(np.float32))
    y = dev.create_buffer(64 * 64 * 320 * 2)
    conv = lambda i: call("di_conv2d", dev.ctx, x.handle, w.handle, bias.handle, 0, y.handle, 1,
                          320, 320, 64, 64, 3, 1, 1, 0, 1, 1)
    for i in range(20):
        conv(i)
    ms = timed(dev, conv, iters)
    fl = perf.conv_flops(1, 320, 320, 64, 64, 3)
    achieved = fl / (ms * 1e-3) / 1e12
    peak = perf.PEAK_FP16_FLOPS / 1e12
    # the same launches with the weights read cold, as in the U-Net step:
    # 160 weight copies (295 MB > the 256 MB Infinity Cache) in rotation
    nrot = 160 if cold else 0
    ws = [dev.create_buffer(320 * 9 * 320 * 2) for _ in range(nrot)]
    for i, b in enumerate(ws):
        dev.fill_normal(b, 320 * 9 * 320, 9000 + i, 0.0, 0.026, dtype=np.float16)
    conv_cold = lambda i: call("di_conv2d", dev.ctx, x.handle, ws[i % nrot].handle, bias.handle, 0,
                          y.handle, 1, 320, 320, 64, 64, 3, 1, 1, 0, 1, 1)
    ms_cold = None
    if nrot:
        for i in range(nrot):
            conv_cold(i)
        ms_cold = timed(dev, conv_cold, nrot)
    for b in ws:
        b.destroy()
    traffic = None
    if os.path.exists(ROOFLINE_PMC):
        for line in open(ROOFLINE_PMC):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(float(line.split(":", 1)[1]))
    for b in (x, w, bias, y):
        b.destroy()
    return {"kernel": "k_conv3_halo<64> conv3x3 320->320 @64x64 NHWC fp16 (fp32 acc), input "
                      "halo staged per channel chunk",
            "bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": traffic,
            "flop_per_launch": fl, "us_per_launch": round(ms * 1e3, 3),
            "cold_weights": None if ms_cold is None else {
                "us_per_launch": round(ms_cold * 1e3, 3),
                "achieved": round(fl / (ms_cold * 1e-3) / 1e12, 2),
                "frac": round(fl / (ms_cold * 1e-3) / 1e12 / peak, 4),
                "note": "weights from HBM (160 copies in rotation), as in the step"}}


def cpu_baseline(u):
    """One whole SD2.1 denoise step (same weights, latent, context and
    timestep as the headline) on the fp32 CPU restatement, timed end to end."""
    import oracle
    from oracle import unet_ref
    from drawinstant import perf
    sd = u.state_dict(np.float32)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 4, 64, 64)).astype(np.float32)
    ctx = rng.standard_normal((1, 77, 1024)).astype(np.float32)
    with oracle.accumulation("fp32"):
        ops = unet_ref.OracleOps()
        t0 = time.perf_counter()
        out = unet_ref.unet_forward(ops, sd, u.config.as_dict(), x,
                                    np.array([999.0], np.float32), ctx)
        sec = time.perf_counter() - t0
        cores = int(oracle.lib().or_threads())
    step = perf.unet_work().total
    return {"value": round(sec * 1e3, 1), "unit": "ms", "cores": cores, "kind": "port",
            "finite": bool(np.isfinite(out).all()),
            "sample": f"CPU restatement, not the reference's WGSL (no Deno / Vulkan ICD on the "
                      f"box): one whole SD2.1 U-Net step ({step / 1e9:.1f} GFLOP, the headline's "
                      f"weights and inputs) on oracle/oracle.c built with fp32 accumulation in "
                      f"the reference kernels' loop order (liboracle_f32.so, gcc -O3 -fopenmp, "
                      f"{cores} threads)"}


def cpu_configs():
    """The fp32 CPU restatement (liboracle_f32.so) on BASELINE cfg1-cfg4 at
    full size, ms per call (one call each after a warm-up of cfg1)."""
    import oracle
    from oracle import unet_ref
    rng = np.random.default_rng(7)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    out = {}
    with oracle.accumulation("fp32"):
        x = f(1, 320, 64, 64)
        g, b = 1 + 0.02 * f(320), 0.02 * f(320)
        oracle.group_norm(x, g, b, 32, eps=1e-5, silu=True)
        t0 = time.perf_counter()
        oracle.group_norm(x, g, b, 32, eps=1e-5, silu=True)
        out["cfg1_gn_silu"] = (time.perf_counter() - t0) * 1e3
        w = f(320, 320, 3, 3) * 0.026
        t0 = time.perf_counter()
        oracle.conv2d(x, w, 0.01 * f(320), stride=1, pad=1)
        out["cfg2_conv3x3"] = (time.perf_counter() - t0) * 1e3
        cfg = unet_ref.sd21_config()
        sd = {k: (0.02 * rng.standard_normal(v)).astype(np.float32)
              for k, v in unet_ref.unet_param_shapes(cfg).items()
              if k.startswith("down_blocks.1.resnets.0.") or k.startswith("down_blocks.0.attentions.0.")}
        ops = unet_ref.OracleOps()
        t0 = time.perf_counter()
        unet_ref.resnet(ops, sd, "down_blocks.1.resnets.0", f(1, 320, 32, 32), f(1, 1280))
        out["cfg3_resnet"] = (time.perf_counter() - t0) * 1e3
        t0 = time.perf_counter()
        unet_ref.transformer(ops, sd, "down_blocks.0.attentions.0", x, f(1, 77, 1024))
        out["cfg4_transformer"] = (time.perf_counter() - t0) * 1e3
        cores = int(oracle.lib().or_threads())
    return {"ms": {k: round(v, 2) for k, v in out.items()}, "cores": cores,
            "kind": "port (fp32 CPU restatement, oracle/oracle.c -DOR_ACC=float)"}


def pcie_inclusive(u, inputs, iters=5):
    """Host-buffer boundary: upload latent+context, eager step, download (ms)."""
    x, ctx = inputs
    u(x, 999.0, ctx)
    t0 = time.perf_counter()
    for _ in range(iters):
        u(x, 999.0, ctx)
    return (time.perf_counter() - t0) * 1e3 / iters


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # 50 timed steps after 20 warm-up replays: ~0.2 s of GPU time, and the
    # median-of-batches figure of longer runs to within 1 us (20 / 5 read
    # 10-25 us high: the clocks and caches are still settling)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-blocks", action="store_true", help="skip the per-block figures")
    ap.add_argument("--cpu-configs", action="store_true",
                    help="also time the fp32 CPU restatement on cfg1-cfg4 (one call each)")
    ap.add_argument("--vae-only", action="store_true",
                    help="only the native VAE decode leg (for rocprofv3 kernel summaries)")
    ap.add_argument("--eager-only", type=int, default=0, metavar="K",
                    help="only K eager (non-graph) U-Net steps after the warm-up, for rocprofv3 "
                         "kernel summaries (with --vae-only: eager decodes)")
    ap.add_argument("--blocks-only", action="store_true",
                    help="only the per-block figures (cfg1 GN+SiLU, cfg2 conv, self-attention, "
                         "GEGLU FFN), for rocprofv3 counter passes")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the roofline kernel and a 256 MiB copy (for rocprofv3 --pmc runs "
                         "that calibrate FETCH_SIZE / WRITE_SIZE against a known byte count)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the U-Net step is data-parallel over batch and is not sharded here", file=sys.stderr)
        sys.exit(2)
    import drawinstant
    from drawinstant import perf
    dev = drawinstant.Device(0)
    if args.roofline_only:
        rl = roofline_conv(dev, cold=False)
        # calibration: a streaming kernel of known traffic (di_unary NEG over
        # 64 Mi floats reads 256 MiB and writes 256 MiB)
        from drawinstant.device import call
        n = 64 << 20
        a, b = dev.create_buffer(n * 4), dev.create_buffer(n * 4)
        call("di_unary", dev.ctx, 2, a.handle, b.handle, n, 0)
        dev.sync()
        print(json.dumps({"roofline": rl, "calibration_read_bytes": n * 4,
                          "calibration_write_bytes": n * 4}), flush=True)
        return
    if args.blocks_only:
        blk = bench_blocks(dev)
        print(json.dumps({"blocks": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                                         for kk, vv in v.items()} for k, v in blk.items()}}),
              flush=True)
        return
    if args.vae_only:
        print(json.dumps({"vae_decode_512": bench_vae(dev, graph=not args.eager_only)}), flush=True)
        return
    if args.eager_only:
        from drawinstant.unet import UNet
        u = UNet(dev, seed=501)
        rng = np.random.default_rng(0)
        bs = dev.storage(rng.standard_normal((1, 4, 64, 64)).astype(np.float32))
        bc = dev.storage(rng.standard_normal((1, 77, 1024)).astype(np.float32))
        bt = dev.storage(np.array([999.0], np.float32))
        bo = dev.create_buffer(4 * 64 * 64 * 4)
        step = lambda i: u.forward(bs, bt, bc, bo, 1, 64, 64, 77, graph=False)
        for i in range(args.warmup):
            step(i)
        ms = timed(dev, step, args.eager_only)
        print(json.dumps({"eager_steps": args.eager_only, "eager_ms_per_step": round(ms, 4)}),
              flush=True)
        return
    u, ms, wall, eager, finite, inputs, spread = bench_unet(dev, args)
    work = perf.unet_work()
    line = {
        "metric": METRIC, "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "cfg5: SD2.1 UNet2DConditionModel (SD-Turbo) denoise step, "
                               "latent [1,4,64,64] (512x512), context [1,77,1024], timestep 999, "
                               "random-init fp16 weights (865.9M params), HIP-graph replay",
                   "batch": 1, "latent": [64, 64], "gflop_per_step": round(work.total / 1e9, 2),
                   "parallelism": "single GPU"},
        "step_spread": spread,
        "eager_ms_per_step": round(eager, 4),
        "wall_ms_per_step": round(wall, 4),
        "step_tflops": round(work.total / (ms * 1e-3) / 1e12, 1),
        "step_mfma_frac": round(work.total / (ms * 1e-3) / perf.PEAK_FP16_FLOPS, 4),
        "output_finite": finite,
        "pcie_inclusive_eager_ms_per_step": round(pcie_inclusive(u, inputs), 3),
        "roofline": roofline_conv(dev),
        "denoise_loop": bench_denoise(dev, u, inputs[1]),
        "batch4": bench_unet_batch(dev, u, 4),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(u)
    if args.cpu_configs:
        line["cpu_configs"] = cpu_configs()
    if not args.no_blocks:
        blk = bench_blocks(dev)
        blk.update(bench_block_chains(dev, u))
        line["blocks"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                              for kk, vv in v.items()} for k, v in blk.items()}
        # secondary legs: a failure is reported in the line, never lost with it
        for key, fn in (("executor_rewrites", bench_executor_rewrites),
                        ("executor_onnx_cfg4", bench_executor_onnx), ("vae_decode_512", bench_vae),
                        ("executor_vae_decode_512", bench_executor_vae)):
            try:
                line[key] = fn(dev)
            except Exception as e:  # noqa: BLE001 - recorded, the headline still prints
                line[key] = {"error": f"{type(e).__name__}: {e}"}
                print(f"bench.py: {key} failed: {e}", file=sys.stderr, flush=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
