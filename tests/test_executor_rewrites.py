"""CPU tests of the executor's fusing rewrites (no GPU): fuse_gelu_pattern,
fuse_layer_norm_pattern, fuse_group_norm_silu_pattern, fuse_attention_pattern
and optimize_graph.

Each rewrite is checked two ways: structurally (which nodes remain, their
inputs and attributes, and the guards that must stop a rewrite), and
semantically, by evaluating the graph before and after the rewrite with a
small numpy interpreter whose fused ops are the CPU oracle's (GELU,
LayerNorm, GroupNorm+SiLU, attention).  A wrong scale fold, a transposed K or
a dropped affine changes the evaluated output and fails the second check.
The exported subgraphs follow torch.onnx's decompositions of nn.GELU,
nn.LayerNorm and attention (eager and scaled_dot_product_attention)."""
import math

import numpy as np
import pytest

import oracle
from drawinstant.executor import (Attr, Graph, Node, TensorProto, fuse_attention_pattern,
                                  fuse_gelu_pattern, fuse_group_norm_silu_pattern,
                                  fuse_layer_norm_pattern, fuse_mul_add_pattern, get_attr_float,
                                  get_attr_int, get_attr_ints, get_attr_string, optimize_graph)


def tp(a, dtype="float32"):
    a = np.asarray(a)
    return TensorProto(list(a.shape), dtype, np.ascontiguousarray(a).tobytes())


def mk(op, name, ins, outs, attrs=None):
    return Node(op, name, list(ins), list(outs), list(attrs or []))


def ops_of(g):
    return [n.op_type for n in g.nodes]


# ------------------------------------------------------ numpy interpreter --
def _eval_node(n, ins):
    op = n.op_type
    if op == "ReduceMean":
        ax = get_attr_ints(n, "axes", [-1])[0]
        return ins[0].mean(axis=ax, keepdims=True, dtype=np.float64).astype(np.float32)
    if op in ("Add", "Sub", "Mul", "Div"):
        f = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide}[op]
        return f(ins[0], ins[1]).astype(np.float32)
    if op == "Pow":
        return np.power(ins[0], ins[1]).astype(np.float32)
    if op == "Sqrt":
        return np.sqrt(ins[0])
    if op == "Erf":
        return oracle.unary("Erf", ins[0])
    if op == "Sigmoid":
        return oracle.unary("Sigmoid", ins[0])
    if op == "Silu":
        return oracle.unary("SiLU", ins[0])
    if op == "Gelu":
        assert get_attr_string(n, "approximate", "none") == "none"
        return oracle.unary("GELU", ins[0])
    if op == "Transpose":
        return np.ascontiguousarray(ins[0].transpose(get_attr_ints(n, "perm", None)))
    if op == "MatMul":
        return np.matmul(ins[0].astype(np.float64), ins[1].astype(np.float64)).astype(np.float32)
    if op == "Softmax":
        x = ins[0]
        return oracle.softmax(x.reshape(-1, x.shape[-1])).reshape(x.shape)
    if op == "AffineBcast":
        return (ins[0] * ins[1] + ins[2]).astype(np.float32)
    if op == "LayerNormalization":
        x = ins[0]
        d = x.shape[-1]
        g = ins[1].reshape(-1) if len(ins) > 1 and ins[1] is not None else np.ones(d, np.float32)
        b = ins[2].reshape(-1) if len(ins) > 2 and ins[2] is not None else np.zeros(d, np.float32)
        return oracle.layer_norm(x.reshape(-1, d), g, b, get_attr_float(n, "epsilon", 1e-5)) \
            .reshape(x.shape)
    if op == "GroupNorm":
        return oracle.group_norm(ins[0], ins[1].reshape(-1), ins[2].reshape(-1),
                                 get_attr_int(n, "num_groups", 32),
                                 get_attr_float(n, "epsilon", 1e-5),
                                 silu=get_attr_string(n, "activation", "") == "silu")
    if op == "FusedAttention" and get_attr_string(n, "layout", "bhsd") == "bshd":
        return oracle.attention(*ins, scale=get_attr_float(n, "scale", 1.0), layout="bshd")
    if op == "FusedAttention":
        q, k, v = ins
        if get_attr_int(n, "k_transposed", 1):
            k = np.swapaxes(k, -1, -2)
        lead = q.shape[:-2]
        h = int(np.prod(lead)) if lead else 1
        o = oracle.attention(q.reshape(1, h, *q.shape[-2:]), k.reshape(1, h, *k.shape[-2:]),
                             v.reshape(1, h, *v.shape[-2:]), scale=get_attr_float(n, "scale", 1.0))
        return o.reshape(q.shape[:-1] + (v.shape[-1],))
    raise AssertionError(f"interpreter: no {op}")


def evaluate(g, feeds):
    env = dict(feeds)
    for name, t in g.tensors.items():
        env[name] = t.array().reshape(t.dims) if t.dims else t.array().reshape(())
    for n in g.nodes:
        ins = [env[i] if i else None for i in n.inputs]
        env[n.outputs[0]] = _eval_node(n, ins)
    return {o["name"]: env[o["name"]] for o in g.outputs}


def rewrite_keeps_outputs(build, rewrite, feeds, rtol):
    before = evaluate(build(), feeds)
    g = build()
    stats = rewrite(g)
    after = evaluate(g, feeds)
    for k, v in before.items():
        np.testing.assert_allclose(after[k], v, rtol=rtol, atol=rtol)
    return g, stats


# ------------------------------------------------------------------ GELU --
def gelu_graph(variant="div", half_first=False, swap=False, sq2=math.sqrt(2.0), one=1.0,
               extra_out=None):
    t = {"c": tp(np.float32(sq2 if variant == "div" else 1 / sq2)), "one": tp(np.float32(one)),
         "half": tp(np.float32(0.5))}
    first = mk("Div" if variant == "div" else "Mul", "d", ["x", "c"], ["u"])
    nodes = [first, mk("Erf", "erf", ["u"], ["e"]),
             mk("Add", "a1", ["one", "e"] if swap else ["e", "one"], ["e1"])]
    if half_first:
        nodes += [mk("Mul", "h", ["x", "half"], ["xh"]),
                  mk("Mul", "m", ["e1", "xh"] if swap else ["xh", "e1"], ["y"])]
    else:
        nodes += [mk("Mul", "m", ["e1", "x"] if swap else ["x", "e1"], ["p"]),
                  mk("Mul", "h", ["half", "p"] if swap else ["p", "half"], ["y"])]
    outs = [{"name": "y"}] + ([{"name": extra_out}] if extra_out else [])
    return Graph(nodes, outputs=outs, tensors=t)


@pytest.mark.parametrize("variant,half_first,swap", [
    ("div", False, False), ("div", False, True), ("mul", False, False), ("div", True, False),
    ("mul", True, True)])
def test_fuse_gelu_variants(variant, half_first, swap):
    x = np.linspace(-4, 4, 96, dtype=np.float32).reshape(2, 48)
    g, st = rewrite_keeps_outputs(lambda: gelu_graph(variant, half_first, swap), fuse_gelu_pattern,
                                  {"x": x}, 1e-6)
    assert st == {"fused": 1} and ops_of(g) == ["Gelu"]
    assert g.nodes[0].inputs == ["x"] and g.nodes[0].outputs == ["y"]


@pytest.mark.parametrize("kw", [{"sq2": 2.0}, {"one": 2.0}, {"extra_out": "e"},
                                {"extra_out": "u"}], ids=["div2", "add2", "erf-used", "div-used"])
def test_fuse_gelu_guards(kw):
    g = gelu_graph(**kw)
    assert fuse_gelu_pattern(g) == {"fused": 0} and len(g.nodes) == 5


# ------------------------------------------------------------- LayerNorm --
def ln_graph(affine="muladd", pow_e=2.0, axes2=(-1,), mean_of="x", eps=1e-5):
    rng = np.random.default_rng(3)
    D = 32
    t = {"two": tp(np.float32(pow_e)), "eps": tp(np.float32(eps)),
         "g": tp((1 + 0.1 * rng.standard_normal(D)).astype(np.float32)),
         "b": tp((0.1 * rng.standard_normal(D)).astype(np.float32))}
    rm = [Attr("axes", ints=[-1])]
    nodes = [mk("ReduceMean", "rm1", [mean_of], ["mu"], rm), mk("Sub", "sub", ["x", "mu"], ["xc"]),
             mk("Pow", "pw", ["xc", "two"], ["x2"]),
             mk("ReduceMean", "rm2", ["x2"], ["var"], [Attr("axes", ints=list(axes2))]),
             mk("Add", "ae", ["var", "eps"], ["ve"]), mk("Sqrt", "sq", ["ve"], ["sd"]),
             mk("Div", "dv", ["xc", "sd"], ["xn"])]
    out = "xn"
    if affine == "muladd":
        nodes += [mk("Mul", "mg", ["g", "xn"], ["xg"]), mk("Add", "ab", ["xg", "b"], ["ln"])]
        out = "ln"
    elif affine == "bcast":
        nodes += [mk("AffineBcast", "af", ["xn", "g", "b"], ["ln"])]
        out = "ln"
    nodes.append(mk("Sigmoid", "after", [out], ["y"]))
    return Graph(nodes, outputs=[{"name": "y"}], tensors=t)


@pytest.mark.parametrize("affine", ["muladd", "bcast", "none"])
def test_fuse_layer_norm(affine):
    x = np.random.default_rng(4).standard_normal((3, 5, 32)).astype(np.float32) * 2 + 0.5
    g, st = rewrite_keeps_outputs(lambda: ln_graph(affine), fuse_layer_norm_pattern, {"x": x}, 2e-5)
    assert st == {"fused": 1} and ops_of(g) == ["LayerNormalization", "Sigmoid"]
    ln = g.nodes[0]
    want = ["x", "g", "b"] if affine != "none" else ["x", "", ""]
    assert ln.inputs == want and ln.outputs == (["xn"] if affine == "none" else ["ln"])
    assert get_attr_float(ln, "epsilon", 0) == pytest.approx(1e-5)
    assert get_attr_int(ln, "axis", 0) == -1


def test_fuse_layer_norm_after_mul_add_rewrite():
    """The reference's own order runs fuse_mul_add first, leaving AffineBcast."""
    g = ln_graph("muladd")
    assert fuse_mul_add_pattern(g, {"g": [32], "b": [32]})["fused"] == 1
    assert "AffineBcast" in ops_of(g)
    assert fuse_layer_norm_pattern(g) == {"fused": 1}
    assert ops_of(g) == ["LayerNormalization", "Sigmoid"] and g.nodes[0].inputs == ["x", "g", "b"]


@pytest.mark.parametrize("kw", [{"pow_e": 3.0}, {"axes2": (1,)}, {"mean_of": "x_other"}],
                         ids=["pow3", "axes-differ", "mean-of-other"])
def test_fuse_layer_norm_guards(kw):
    g = ln_graph(**kw)
    n = len(g.nodes)
    assert fuse_layer_norm_pattern(g) == {"fused": 0} and len(g.nodes) == n


# ------------------------------------------------------------ GroupNorm+SiLU --
def test_fuse_group_norm_silu():
    rng = np.random.default_rng(5)
    C = 8
    gam = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    bet = (0.1 * rng.standard_normal(C)).astype(np.float32)

    def build(extra=False):
        t = {"g": tp(gam), "b": tp(bet)}
        nodes = [mk("GroupNorm", "gn", ["x", "g", "b"], ["h"],
                    [Attr("num_groups", i=4), Attr("epsilon", f=1e-6)]),
                 mk("Silu", "s", ["h"], ["y"])]
        return Graph(nodes, outputs=[{"name": "y"}] + ([{"name": "h"}] if extra else []),
                     tensors=t)

    x = rng.standard_normal((1, C, 4, 4)).astype(np.float32)
    g0 = build()
    ref = evaluate(g0, {"x": x})["y"]
    assert fuse_group_norm_silu_pattern(g0) == {"fused": 1} and ops_of(g0) == ["GroupNorm"]
    n = g0.nodes[0]
    assert get_attr_string(n, "activation", "") == "silu" and get_attr_int(n, "num_groups", 0) == 4
    assert get_attr_float(n, "epsilon", 0) == pytest.approx(1e-6) and n.outputs == ["y"]
    np.testing.assert_allclose(evaluate(g0, {"x": x})["y"], ref, rtol=1e-6, atol=1e-6)
    g1 = build(extra=True)  # the GroupNorm output is also a graph output
    assert fuse_group_norm_silu_pattern(g1) == {"fused": 0}


# ------------------------------------------------------------- attention --
def attn_graph(style="eager", scale_op="Mul", k_extra_use=False, sm_extra_use=False, axis=-1,
               merge=True):
    """eager: Transpose q/k/v heads, MatMul(q, k^T), scale, Softmax, MatMul,
    Transpose back.  sdpa: torch's scaled_dot_product_attention export, the
    scale split as sqrt(scale) over q and k^T, K^T by Transpose(0,1,3,2).
    merge=False leaves the output in [B, H, S, d]."""
    s = 1 / 8
    t = {"scale": tp(np.float32(s if scale_op == "Mul" else 1 / s)),
         "rs": tp(np.float32(math.sqrt(s)))}
    perm = [Attr("perm", ints=[0, 2, 1, 3])]
    nodes = [mk("Transpose", "tq", ["q"], ["qh"], perm), mk("Transpose", "tv", ["v"], ["vh"], perm)]
    if style == "eager":
        nodes += [mk("Transpose", "tk", ["k"], ["kh"], [Attr("perm", ints=[0, 2, 3, 1])]),
                  mk("MatMul", "qk", ["qh", "kh"], ["sc"])]
        if scale_op:
            nodes.append(mk(scale_op, "scl", ["sc", "scale"], ["ss"]))
        last = "ss" if scale_op else "sc"
    else:
        nodes += [mk("Transpose", "tk0", ["k"], ["kb"], perm),
                  mk("Transpose", "tk", ["kb"], ["kh"], [Attr("perm", ints=[0, 1, 3, 2])]),
                  mk("Mul", "mq", ["qh", "rs"], ["qs"]), mk("Mul", "mk", ["rs", "kh"], ["ks"]),
                  mk("MatMul", "qk", ["qs", "ks"], ["ss"])]
        last = "ss"
    nodes += [mk("Softmax", "sm", [last], ["p"], [Attr("axis", i=axis)]),
              mk("MatMul", "pv", ["p", "vh"], ["o" if merge else "y"])]
    if merge:
        nodes.append(mk("Transpose", "to", ["o"], ["y"], perm))
    outs = [{"name": "y"}]
    if k_extra_use:
        outs.append({"name": "kh"})
    if sm_extra_use:
        outs.append({"name": "p"})
    return Graph(nodes, outputs=outs, tensors=t)


def attn_feeds():
    rng = np.random.default_rng(6)
    B, S, H, d = 2, 24, 3, 64
    return {n: rng.standard_normal((B, S, H, d)).astype(np.float32) for n in "qkv"}


@pytest.mark.parametrize("style,scale_op", [("eager", "Mul"), ("eager", "Div"), ("eager", None),
                                            ("sdpa", None)])
def test_fuse_attention_bshd(style, scale_op):
    """Head split / merge Transposes around the chain fold into the node:
    one FusedAttention reading and writing [B, S, H, d]."""
    g, st = rewrite_keeps_outputs(lambda: attn_graph(style, scale_op), fuse_attention_pattern,
                                  attn_feeds(), 2e-5)
    assert st == {"fused": 1} and ops_of(g) == ["FusedAttention"]
    fa = g.nodes[0]
    assert fa.inputs == ["q", "k", "v"] and fa.outputs == ["y"]
    assert get_attr_string(fa, "layout", "") == "bshd"
    want = 1.0 if (style == "eager" and scale_op is None) else 1 / 8
    assert get_attr_float(fa, "scale", 0) == pytest.approx(want, rel=1e-6)


@pytest.mark.parametrize("style", ["eager", "sdpa"])
def test_fuse_attention_bhsd_output(style):
    """Output left in [B, H, S, d]: the node keeps the head-split inputs and
    the single-use Transpose into K^T is turned to yield K."""
    g, st = rewrite_keeps_outputs(lambda: attn_graph(style, merge=False), fuse_attention_pattern,
                                  attn_feeds(), 2e-5)
    assert st == {"fused": 1} and "Softmax" not in ops_of(g) and "MatMul" not in ops_of(g)
    fa = next(n for n in g.nodes if n.op_type == "FusedAttention")
    assert get_attr_string(fa, "layout", "bhsd") == "bhsd" and fa.outputs == ["y"]
    assert get_attr_int(fa, "k_transposed", 1) == 0 and fa.inputs[0] == "qh"
    tk = next(n for n in g.nodes if n.name == "tk")
    assert get_attr_ints(tk, "perm", None) == ([0, 2, 1, 3] if style == "eager" else [0, 1, 2, 3])
    if style == "sdpa":
        assert "Mul" not in ops_of(g)


def test_fuse_attention_keeps_shared_transpose():
    """K^T read elsewhere too: its Transpose stays and the node takes K^T."""
    g, st = rewrite_keeps_outputs(lambda: attn_graph(k_extra_use=True), fuse_attention_pattern,
                                  attn_feeds(), 2e-5)
    fa = next(n for n in g.nodes if n.op_type == "FusedAttention")
    assert st == {"fused": 1} and get_attr_int(fa, "k_transposed", 0) == 1
    assert get_attr_string(fa, "layout", "bhsd") == "bhsd"
    assert get_attr_ints(next(n for n in g.nodes if n.name == "tk"), "perm", None) == [0, 2, 3, 1]


def test_fuse_attention_guards():
    g = attn_graph(sm_extra_use=True)  # probabilities are a graph output
    assert fuse_attention_pattern(g) == {"fused": 0} and "Softmax" in ops_of(g)


def test_optimize_graph_counts():
    g = attn_graph()
    st = optimize_graph(g)
    assert st["attention"] == 1 and st["layer_norm"] == 0 and st["gelu"] == 0
    g2 = gelu_graph()
    assert optimize_graph(g2, attention=False) == {
        "silu": 0, "mul_add": 0, "group_norm": 0, "group_norm_silu": 0, "layer_norm": 0,
        "gelu": 1}
