"""GPU parity of the executor mirror: ONNX-exported subgraphs of the SD U-Net
run through Executor (one C-ABI dispatch per node, fp32 NCHW as the
reference's executor) against the CPU oracle, fused and unfused, and the
reference's fused-block entry points (run*Bench) end to end.

Tolerances: fp32 executor paths use the reference KAT gate max-rel <= 1e-4 (or
1e-3 where an fp32 reduction order differs over >= 1e4 terms); paths whose
fused side computes in fp16 (ResNet block, flash attention) are bounded in
RMS relative to the output's RMS.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import max_rel, rel_l2
from drawinstant.executor import (Attr, Executor, Graph, Node, TensorProto, WeightCache,
                                  fuse_attention_pattern, fuse_gelu_pattern,
                                  fuse_group_norm_pattern, fuse_layer_norm_pattern,
                                  fuse_mul_add_pattern, fuse_silu_pattern, get_attr_int,
                                  get_attr_string, optimize_graph)

pytestmark = pytest.mark.gpu


def tp(a, dtype="float32"):
    a = np.asarray(a)
    return TensorProto(list(a.shape), dtype, np.ascontiguousarray(a).tobytes())


def mk(op, name, ins, outs, attrs=None):
    return Node(op, name, list(ins), list(outs), list(attrs or []))


def run_graph(dev, g, inputs, fuse=()):
    for f in fuse:
        f(g)
    wc = WeightCache(dev, g.tensors)
    ex = Executor(dev, g, wc)
    try:
        outs = ex.run(inputs)
        res = {}
        for k, t in outs.items():
            if t.buf is not None:
                res[k] = dev.download(t.buf, np.float32, tuple(t.dims))
                t.buf.destroy()
            else:
                res[k] = t.cpu_data
        return res, ex
    finally:
        ex.destroy()
        wc.destroy()


def gn_export_graph(N, C, H, W, G, eps):
    """torch.onnx's GroupNorm: Reshape [N,G,-1] -> InstanceNorm(1, 0) ->
    Reshape back -> Mul gamma -> Add beta."""
    rng = np.random.default_rng(11)
    gamma = (1 + 0.1 * rng.standard_normal((C, 1, 1))).astype(np.float32)
    beta = (0.1 * rng.standard_normal((C, 1, 1))).astype(np.float32)
    tensors = {"sc": tp(np.ones(G, np.float32)), "bi": tp(np.zeros(G, np.float32)),
               "shape1": tp(np.array([N, C, H, W], np.int64), "int64"),
               "gamma": tp(gamma), "beta": tp(beta)}
    nodes = [mk("Constant", "s0", [], ["shape0"],
                [Attr("value", t=tp(np.array([0, G, -1], np.int64), "int64"))]),
             mk("Reshape", "r0", ["x", "shape0"], ["r0"]),
             mk("InstanceNormalization", "in", ["r0", "sc", "bi"], ["i0"],
                [Attr("epsilon", f=eps)]),
             mk("Reshape", "r1", ["i0", "shape1"], ["r1"]),
             mk("Mul", "m", ["r1", "gamma"], ["m0"]),
             mk("Add", "a", ["m0", "beta"], ["y"])]
    return Graph(nodes, outputs=[{"name": "y"}], tensors=tensors), gamma, beta


@pytest.mark.parametrize("fused", [False, True])
def test_groupnorm_export_subgraph(dev, fused):
    N, C, H, W, G = 1, 320, 16, 16, 32
    g, gamma, beta = gn_export_graph(N, C, H, W, G, 1e-5)
    x = np.random.default_rng(12).standard_normal((N, C, H, W)).astype(np.float32)
    fz = (fuse_mul_add_pattern, fuse_group_norm_pattern) if fused else ()
    out, ex = run_graph(dev, g, {"x": x}, fz)
    if fused:
        assert [n.op_type for n in g.nodes] == ["Constant", "GroupNorm"]
    ref = oracle.group_norm(x, gamma.reshape(-1), beta.reshape(-1), G, eps=1e-5)
    assert max_rel(out["y"], ref) <= 1e-4


@pytest.mark.parametrize("fused", [False, True])
def test_silu_subgraph(dev, fused):
    g = Graph([mk("Sigmoid", "s", ["x"], ["sg"]), mk("Mul", "m", ["x", "sg"], ["y"])],
              outputs=[{"name": "y"}])
    x = np.linspace(-6, 6, 4096, dtype=np.float32).reshape(1, 4, 32, 32)
    out, _ = run_graph(dev, g, {"x": x}, (fuse_silu_pattern,) if fused else ())
    assert max_rel(out["y"], oracle.unary("SiLU", x)) <= 1e-5


@pytest.mark.parametrize("fused", [False, True])
def test_decomposed_layernorm_and_gelu_subgraphs(dev, fused):
    """LN as exported (ReduceMean, Sub, Pow 2, ReduceMean, Add eps, Sqrt, Div,
    Mul, Add) and erf-GELU (Div sqrt2, Erf, Add 1, Mul x, Mul 0.5), op by op
    and after fuse_layer_norm_pattern + fuse_gelu_pattern (two dispatches)."""
    rng = np.random.default_rng(13)
    S, D = 256, 320
    x = rng.standard_normal((1, S, D)).astype(np.float32)
    gam = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    bet = (0.1 * rng.standard_normal(D)).astype(np.float32)
    t = {"two": tp(np.array([2.0], np.float32)), "eps": tp(np.array([1e-5], np.float32)),
         "g": tp(gam), "b": tp(bet), "sq2": tp(np.array([math.sqrt(2.0)], np.float32)),
         "one": tp(np.array([1.0], np.float32)), "half": tp(np.array([0.5], np.float32))}
    rm = [Attr("axes", ints=[-1])]
    nodes = [mk("ReduceMean", "rm1", ["x"], ["mu"], rm), mk("Sub", "sub", ["x", "mu"], ["xc"]),
             mk("Pow", "pw", ["xc", "two"], ["x2"]), mk("ReduceMean", "rm2", ["x2"], ["var"], rm),
             mk("Add", "ae", ["var", "eps"], ["ve"]), mk("Sqrt", "sq", ["ve"], ["sd"]),
             mk("Div", "dv", ["xc", "sd"], ["xn"]), mk("Mul", "mg", ["xn", "g"], ["xg"]),
             mk("Add", "ab", ["xg", "b"], ["ln"]),
             mk("Div", "d2", ["ln", "sq2"], ["u"]), mk("Erf", "erf", ["u"], ["e"]),
             mk("Add", "a1", ["e", "one"], ["e1"]), mk("Mul", "mx", ["ln", "e1"], ["p"]),
             mk("Mul", "mh", ["p", "half"], ["y"])]
    g = Graph(nodes, outputs=[{"name": "ln"}, {"name": "y"}], tensors=t)
    fuse = (fuse_layer_norm_pattern, fuse_gelu_pattern) if fused else ()
    out, ex = run_graph(dev, g, {"x": x}, fuse)
    if fused:
        assert [n.op_type for n in g.nodes] == ["LayerNormalization", "Gelu"]
    ln_ref = oracle.layer_norm(x.reshape(S, D), gam, bet, eps=1e-5).reshape(1, S, D)
    assert max_rel(out["ln"], ln_ref) <= 1e-4
    assert max_rel(out["y"], oracle.unary("GELU", ln_ref)) <= 1e-4


def attention_graph(scale_op="Mul", shared_kt=False, merge=True):
    """Exported attention: Transpose heads, MatMul Q.K^T, scale, Softmax,
    MatMul P.V, Transpose back (the materialised-score path flash attention
    replaces).  shared_kt also outputs K^T, so its Transpose cannot be
    folded; merge=False leaves the output in [B, H, S, d]."""
    t = {"scale": tp(np.array([1 / 8 if scale_op == "Mul" else 8.0], np.float32))}
    perm = [Attr("perm", ints=[0, 2, 1, 3])]
    nodes = [mk("Transpose", "tq", ["q"], ["qh"], perm), mk("Transpose", "tk", ["k"], ["kh"],
                                                            [Attr("perm", ints=[0, 2, 3, 1])]),
             mk("Transpose", "tv", ["v"], ["vh"], perm), mk("MatMul", "qk", ["qh", "kh"], ["s"]),
             mk(scale_op, "sc", ["s", "scale"], ["ss"]), mk("Softmax", "sm", ["ss"], ["p"],
                                                            [Attr("axis", i=-1)]),
             mk("MatMul", "pv", ["p", "vh"], ["o" if merge else "y"])]
    if merge:
        nodes.append(mk("Transpose", "to", ["o"], ["y"], perm))
    outs = [{"name": "y"}] + ([{"name": "kh"}] if shared_kt else [])
    return Graph(nodes, outputs=outs, tensors=t)


@pytest.mark.parametrize("fused,Sq,Skv,d,scale_op,shared_kt,merge", [
    (False, 256, 256, 64, "Mul", False, True),
    (True, 256, 256, 64, "Mul", False, True),   # self, [B,S,H,d] in and out (BSHD)
    (True, 256, 77, 64, "Div", False, True),    # cross: 77 keys, Div scale
    (True, 256, 77, 64, "Mul", False, False),   # [B,H,S,d] out: BHSD, K transpose turned
    (True, 200, 77, 64, "Mul", True, True),     # shared K^T: transposed on the device
    (True, 96, 40, 32, "Mul", False, True),     # head dim 32: unfused chain inside the node
    (True, 96, 40, 32, "Mul", False, False),    # same, BHSD with the turned K transpose
])
def test_attention_subgraph(dev, fused, Sq, Skv, d, scale_op, shared_kt, merge):
    """The exported attention chain, op by op and after fuse_attention_pattern.
    The flash path computes with fp16 MFMA operands: rel-L2 <= 2e-3 against
    the fp64-accumulated oracle; the unfused fp32 chains keep max-rel 1e-4."""
    rng = np.random.default_rng(14)
    B, H = 1, 5
    q = rng.standard_normal((B, Sq, H, d)).astype(np.float32)
    k, v = (rng.standard_normal((B, Skv, H, d)).astype(np.float32) for _ in range(2))
    g = attention_graph(scale_op, shared_kt, merge)
    out, _ = run_graph(dev, g, {"q": q, "k": k, "v": v}, (fuse_attention_pattern,) if fused else ())
    ref = oracle.attention(q.transpose(0, 2, 1, 3).copy(), k.transpose(0, 2, 1, 3).copy(),
                           v.transpose(0, 2, 1, 3).copy(), scale=1 / 8)
    if merge:
        ref = ref.transpose(0, 2, 1, 3)
    if fused:
        fa = [n for n in g.nodes if n.op_type == "FusedAttention"]
        assert len(fa) == 1 and "Softmax" not in [n.op_type for n in g.nodes]
        assert get_attr_int(fa[0], "k_transposed", -1) == (1 if shared_kt else 0)
        assert get_attr_string(fa[0], "layout", "bhsd") == \
            ("bshd" if merge and not shared_kt else "bhsd")
    if fused and d == 64:
        assert rel_l2(out["y"], ref) <= 2e-3
    else:
        assert max_rel(out["y"], ref) <= 1e-4
    if shared_kt:
        assert max_rel(out["kh"], k.transpose(0, 2, 3, 1)) == 0


def test_optimized_gn_silu_subgraph(dev):
    """torch.onnx GroupNorm + Sigmoid*x SiLU through optimize_graph: one
    GroupNorm dispatch with the SiLU epilogue (DI_NORM_SILU)."""
    N, C, H, W, G, eps = 1, 64, 16, 16, 32, 1e-6
    g, gamma, beta = gn_export_graph(N, C, H, W, G, eps)
    g.nodes[-1].outputs = ["h"]
    g.nodes += [mk("Sigmoid", "sg", ["h"], ["s"]), mk("Mul", "ms", ["h", "s"], ["y"])]
    x = np.random.default_rng(15).standard_normal((N, C, H, W)).astype(np.float32)
    out, _ = run_graph(dev, g, {"x": x}, (optimize_graph,))
    assert [n.op_type for n in g.nodes if n.op_type != "Constant"] == ["GroupNorm"]
    ref = oracle.group_norm(x, gamma.reshape(-1), beta.reshape(-1), G, eps, silu=True)
    assert max_rel(out["y"], ref) <= 1e-4


def test_conv_resize_concat_slice_gemm_subgraph(dev):
    """Upsample block shapes: Resize x2 -> Conv3x3 -> Concat skip -> Slice;
    plus a Gemm(transB) time-embedding linear."""
    rng = np.random.default_rng(15)
    x = rng.standard_normal((1, 8, 8, 8)).astype(np.float32)
    skip = rng.standard_normal((1, 4, 16, 16)).astype(np.float32)
    w = (rng.standard_normal((16, 8, 3, 3)) * 0.1).astype(np.float32)
    b = (0.01 * rng.standard_normal(16)).astype(np.float32)
    a = rng.standard_normal((1, 320)).astype(np.float32)
    wl = (rng.standard_normal((1280, 320)) * 0.05).astype(np.float32)
    bl = (0.01 * rng.standard_normal(1280)).astype(np.float32)
    t = {"w": tp(w), "b": tp(b), "scales": tp(np.array([1, 1, 2, 2], np.float32)),
         "st": tp(np.array([2], np.int64), "int64"), "en": tp(np.array([14], np.int64), "int64"),
         "ax": tp(np.array([1], np.int64), "int64"), "wl": tp(wl), "bl": tp(bl)}
    nodes = [mk("Resize", "rs", ["x", "", "scales"], ["xu"], [Attr("mode", s="nearest")]),
             mk("Conv", "cv", ["xu", "w", "b"], ["h"], [Attr("kernel_shape", ints=[3, 3]),
                                                        Attr("pads", ints=[1, 1, 1, 1])]),
             mk("Concat", "cc", ["h", "skip"], ["hc"], [Attr("axis", i=1)]),
             mk("Slice", "sl", ["hc", "st", "en", "ax"], ["y"]),
             mk("Gemm", "gm", ["a", "wl", "bl"], ["z"], [Attr("transB", i=1)])]
    out, _ = run_graph(dev, Graph(nodes, outputs=[{"name": "y"}, {"name": "z"}], tensors=t),
                       {"x": x, "skip": skip, "a": a})
    xu = x.repeat(2, axis=2).repeat(2, axis=3)
    h = oracle.conv2d(xu, w, b, stride=1, pad=1)
    ref = np.concatenate([h, skip], 1)[:, 2:14]
    assert max_rel(out["y"], ref) <= 1e-4
    assert max_rel(out["z"], oracle.linear(a, wl, bl)) <= 1e-4


def test_timestep_path_and_rerun_pool_reuse(dev):
    """int64 timestep seed stays on the CPU through Cast -> Unsqueeze, then
    Mul by the frequency initializer, Cos / Sin, Concat (flip_sin_to_cos
    order) on the device.  A second run reuses the pool (no new allocations)
    and returns an independent snapshot."""
    half = 160
    freqs = np.exp(-math.log(10000.0) * np.arange(half) / half).astype(np.float32)
    t = {"f": tp(freqs.reshape(1, half)), "ax": tp(np.array([1], np.int64), "int64")}
    nodes = [mk("Cast", "c", ["ts"], ["tf"], [Attr("to", i=1)]),
             mk("Unsqueeze", "u", ["tf", "ax"], ["t2"]),
             mk("Mul", "m", ["t2", "f"], ["arg"]),
             mk("Cos", "cs", ["arg"], ["c0"]), mk("Sin", "sn", ["arg"], ["s0"]),
             mk("Concat", "cat", ["c0", "s0"], ["y"], [Attr("axis", i=-1)])]
    g = Graph(nodes, outputs=[{"name": "y"}], tensors=t)
    wc = WeightCache(dev, t)
    ex = Executor(dev, g, wc)
    try:
        outs = []
        for ts in (999, 1):
            o = ex.run({"ts": np.array([ts], np.int64)})["y"]
            outs.append(dev.download(o.buf, np.float32, tuple(o.dims)))
            o.buf.destroy()
            if ts == 999:
                allocs = ex.pool.allocs
        assert ex.pool.allocs == allocs
        for ts, y in zip((999, 1), outs):
            arg = np.float32(ts) * freqs
            ref = np.concatenate([np.cos(arg.astype(np.float64)), np.sin(arg.astype(np.float64))])
            assert y.shape == (1, 2 * half)
            assert np.max(np.abs(y.reshape(-1) - ref)) <= 2e-4  # |arg| <= 999: fp32 ulp ~6e-5
    finally:
        ex.destroy()
        wc.destroy()


# ------------------------------------------------------- block entry points --
def _check(res, key, max_rms_rel):
    print(f"[{key}] naive {res['naive']:.3f} ms fused {res['fused']:.3f} ms "
          f"speedup {res['speedup']:.2f}x maxAbsDiff {res['correctness']['maxAbsDiff']:.2e} "
          f"l2 {res['correctness']['l2']:.2e}", flush=True)
    for k in ("shape", "naive", "fused", "speedup", "correctness", "dispatchesNaive",
              "dispatchesFused"):
        assert k in res
    assert res["naive"] > 0 and res["fused"] > 0
    assert res["correctness"]["l2"] <= max_rms_rel * res.get("_rms", 1.0)


@pytest.mark.parametrize("key,tol", [
    ("groupnorm", 1e-5), ("conv", 1e-5), ("resnet", 3e-2), ("attn", 1e-3), ("cross_attn", 1e-3),
    ("ffn", 2e-4), ("block", 2e-3), ("tembed", 1e-3),
])
def test_fused_entry_points(dev, key, tol):
    """Each run*Bench at the reference's SHAPE: schema, both paths timed, and
    naive vs fused agreement (RMS difference; fp16-computing fused paths get
    the wider bound)."""
    from drawinstant import fused
    print(f"[bench] {key}", flush=True)
    res = fused.ALL_BENCHES[key](dev, repeats=1, warm_ms=20.0)
    _check(res, key, tol)
