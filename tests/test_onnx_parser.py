"""CPU tests of the ONNX parser (drawinstant.onnx_parser) and of the fusing
rewrites on real exported graphs.

* The reference's own parser fixture (onnx-parser-test.mjs:1-93: a ModelProto
  with one MatMul node, one [2,3] float initializer whose raw data starts
  1.5, -2.25, input "a", output "y", opset 17) is rebuilt byte for byte with
  the same encoder and must give the same answers.
* Wire-format cases the reference's walk handles (packed and unpacked dims,
  float_data, negative int64 attributes as 10-byte varints) and its
  recovery paths (a garbage prefix, a truncated file).
* torch.onnx exports of a diffusers-style Transformer2D block (SDPA and eager
  attention), ResnetBlock2D and a reduced-width VAE decoder: parsed initializers equal the module's
  parameters, the graph evaluated by the numpy interpreter equals torch's
  float64 output, and so does the graph after optimize_graph, whose rewrite
  counts are checked.
"""
import copy
import struct

import numpy as np
import pytest

import numpy_onnx
from golden import onnx_export
from drawinstant.executor import get_attr_int, get_attr_ints, get_attr_string, optimize_graph
from drawinstant.onnx_parser import (ProtoError, _Reader, load_onnx, parse_onnx_graph,
                                     parse_onnx_weights)


# ---------------------------------------------- the reference's encoder --
def varint(n):
    out = []
    n &= (1 << 64) - 1
    while n > 0x7F:
        out.append((n & 0x7F) | 0x80)
        n >>= 7
    out.append(n)
    return out


def tag(field, wire):
    return varint((field << 3) | wire)


def len_delim(field, data):
    return tag(field, 2) + varint(len(data)) + list(data)


def text(field, s):
    return len_delim(field, s.encode())


def vint(field, n):
    return tag(field, 0) + varint(n)


def tensor(name, dims, dtype, raw, packed_dims=False, float_data=None):
    out = len_delim(1, sum((varint(d) for d in dims), [])) if packed_dims else \
        sum((vint(1, d) for d in dims), [])
    out += vint(2, dtype) + text(8, name)
    if float_data is not None:
        out += len_delim(4, struct.pack(f"<{len(float_data)}f", *float_data))
    else:
        out += len_delim(9, raw)
    return out


def node(inputs, outputs, op, attrs=()):
    out = sum((text(1, i) for i in inputs), []) + sum((text(2, o) for o in outputs), [])
    out += text(4, op)
    for a in attrs:
        out += len_delim(5, a)
    return out


def model(graph_bytes):
    return bytes(vint(1, 8) + text(2, "draw.instant.test") + len_delim(7, graph_bytes) +
                 len_delim(8, vint(2, 17)))


def reference_fixture():
    """onnx-parser-test.mjs:48-72."""
    raw = bytearray(24)
    struct.pack_into("<f", raw, 0, 1.5)
    struct.pack_into("<f", raw, 4, -2.25)
    g = len_delim(1, node(["a", "w1"], ["y"], "MatMul"))
    g += len_delim(5, tensor("w1", [2, 3], 1, raw))
    g += len_delim(11, text(1, "a")) + len_delim(12, text(1, "y"))
    return model(g)


def test_reference_fixture():
    buf = reference_fixture()
    g = parse_onnx_graph(buf)
    assert len(g.tensors) == 1 and len(g.nodes) == 1
    assert g.nodes[0].op_type == "MatMul" and g.nodes[0].inputs == ["a", "w1"]
    assert g.nodes[0].outputs == ["y"]
    w1 = g.tensors["w1"]
    assert w1.dims == [2, 3] and w1.dtype == "float32" and len(w1.data) == 24
    assert list(w1.array()[:3]) == [1.5, -2.25, 0.0]
    assert [i["name"] for i in g.inputs] == ["a"] and [o["name"] for o in g.outputs] == ["y"]
    assert g.op_hist == {"MatMul": 1} and g.bytes == 24
    w = parse_onnx_weights(buf)
    assert w["count"] == 1 and w["bytes"] == 24


def test_wire_variants():
    # packed dims, float_data, a negative int64 attribute and a strings list
    attr_axes = text(1, "axes") + vint(20, 7) + vint(8, -1)
    attr_perm = text(1, "perm") + len_delim(8, varint(0) + varint(2) + varint(1))
    attr_eps = text(1, "epsilon") + vint(20, 1) + tag(2, 5) + list(struct.pack("<f", 1e-6))
    attr_strs = text(1, "names") + text(9, "ab") + text(9, "c")
    g = len_delim(1, node(["x"], ["m"], "ReduceMean", [attr_axes, attr_eps]))
    g += len_delim(1, node(["m"], ["t"], "Transpose", [attr_perm, attr_strs]))
    g += len_delim(5, tensor("p", [3, 2], 1, b"", packed_dims=True,
                             float_data=[1, 2, 3, 4, 5, -6]))
    vi = text(1, "x") + len_delim(2, len_delim(1, vint(1, 1) + len_delim(
        2, len_delim(1, vint(1, 2)) + len_delim(1, text(2, "batch")))))
    g += len_delim(11, vi)
    gr = parse_onnx_graph(model(g))
    rm, tr = gr.nodes
    assert get_attr_ints(rm, "axes", None) == [-1]
    assert next(a for a in rm.attributes if a.name == "epsilon").f == pytest.approx(1e-6)
    assert get_attr_ints(tr, "perm", None) == [0, 2, 1]
    assert next(a for a in tr.attributes if a.name == "names").strings == ["ab", "c"]
    p = gr.tensors["p"]
    assert p.dims == [3, 2] and list(p.array()) == [1, 2, 3, 4, 5, -6]
    assert gr.inputs == [{"name": "x", "dtype": 1, "dims": [2, -1]}]


def test_reader_rejects_overruns():
    r = _Reader(bytes([0x80, 0x80]))
    with pytest.raises(ProtoError):
        r.varint()
    r = _Reader(bytes(tag(1, 2) + varint(50) + [1, 2]))
    r.tag()
    with pytest.raises(ProtoError):
        r.span()


def test_recovery_paths():
    buf = reference_fixture()
    # junk before the model: the top-level walk desyncs, the graph-tag scan
    # finds the graph (onnx-parser.js:443-509)
    g = parse_onnx_graph(bytes([0x07, 0xFF]) + buf)
    assert len(g.nodes) == 1 and "w1" in g.tensors and g.warnings
    # truncated inside the graph: a warning and no exception
    g = parse_onnx_graph(buf[:len(buf) - 30])
    assert isinstance(g.nodes, list)


# -------------------------------------------------- real exported graphs --
@pytest.fixture(scope="module")
def cases():
    return {"sdpa": onnx_export.transformer_case(), "eager": onnx_export.transformer_case(eager=True),
            "resnet": onnx_export.resnet_case(), "vae": onnx_export.vae_case()}


def max_rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b) / np.maximum(1.0, np.abs(b))))


def test_exported_transformer_parses(cases, tmp_path):
    data, feeds, _ = cases["sdpa"]
    p = tmp_path / "tf.onnx"
    p.write_bytes(data)
    g = load_onnx(str(p))  # memory-mapped path
    assert [i["name"] for i in g.inputs] == ["x", "ctx"] and g.outputs[0]["name"] == "y"
    assert g.inputs[0]["dims"] == [1, 128, 8, 8] and g.inputs[1]["dims"] == [1, 77, 96]
    assert g.op_hist["Softmax"] == 2 and g.op_hist["InstanceNormalization"] == 1
    assert g.op_hist["ReduceMean"] == 6 and g.op_hist["Erf"] == 1
    # initializers are the module's parameters (Linear weights stored
    # transposed, as the exporter feeds them to MatMul)
    m = onnx_export._seeded(onnx_export.Transformer2D(128, 96, 2, 64), 0)
    np.testing.assert_array_equal(g.tensors["attn1.to_out.bias"].array(),
                                  m.attn1.to_out.bias.detach().numpy())
    proj = m.ff.proj.weight.detach().numpy().T
    assert sum(np.array_equal(t.array().reshape(t.dims), proj) for t in g.tensors.values()
               if t.dims == list(proj.shape)) == 1
    assert g.bytes == sum(p.numel() * 4 for p in m.parameters())


@pytest.mark.parametrize("key,want", [
    ("sdpa", {"mul_add": 4, "group_norm": 1, "layer_norm": 3, "gelu": 1, "attention": 2}),
    ("eager", {"mul_add": 4, "group_norm": 1, "layer_norm": 3, "gelu": 1, "attention": 2}),
    ("resnet", {"silu": 3, "mul_add": 2, "group_norm": 2, "group_norm_silu": 2}),
    ("vae", {"silu": 29, "mul_add": 30, "group_norm": 30, "group_norm_silu": 29, "attention": 1}),
])
def test_exported_graphs_rewrite_and_evaluate(cases, key, want):
    """torch's float64 output = the parsed graph's = the rewritten graph's."""
    data, feeds, y = cases[key]
    out = "sample" if key == "vae" else "y"
    g = parse_onnx_graph(data)
    assert max_rel(numpy_onnx.run(g, feeds)[out], y) <= 1e-5
    g2 = copy.deepcopy(g)
    st = optimize_graph(g2)
    assert {k: v for k, v in st.items() if v} == want
    assert max_rel(numpy_onnx.run(g2, feeds)[out], y) <= 1e-5
    ops = [n.op_type for n in g2.nodes]
    assert "Softmax" not in ops and "Erf" not in ops and "InstanceNormalization" not in ops
    if key in ("sdpa", "eager"):
        fa = [n for n in g2.nodes if n.op_type == "FusedAttention"]
        # head split / merge Transposes folded: [B, S, H, d] in and out
        assert all(get_attr_string(n, "layout", "") == "bshd" for n in fa)
        assert all(get_attr_int(n, "k_transposed", 1) == 0 for n in fa)
        assert ops.count("Transpose") == 2  # only the NCHW <-> tokens pair remains
        if key == "sdpa":  # the computed sqrt(scale) factors ride along as inputs
            assert all(len(n.inputs) == 5 for n in fa)


# ------------------------------------------------ randomised round trips --
from hypothesis import given, settings, strategies as st  # noqa: E402

_names = st.text(alphabet="abcdefghijklmnopqrstuvwxyz_/.0123456789", min_size=1, max_size=12)
_ints = st.lists(st.integers(min_value=-(1 << 62), max_value=(1 << 62)), max_size=6)
_floats = st.lists(st.floats(width=32, allow_nan=False, allow_infinity=False), max_size=5)


@st.composite
def _graphs(draw):
    nodes = []
    for _ in range(draw(st.integers(1, 5))):
        ins = draw(st.lists(_names, max_size=3))
        outs = draw(st.lists(_names, min_size=1, max_size=2))
        op = draw(st.sampled_from(["MatMul", "Add", "Reshape", "Transpose", "Softmax", "Conv"]))
        ints, floats, name_i = draw(_ints), draw(_floats), draw(st.integers(-5, 5))
        nodes.append((ins, outs, op, ints, floats, name_i))
    dims = draw(st.lists(st.integers(1, 4), min_size=1, max_size=3))
    data = np.random.default_rng(draw(st.integers(0, 99))).standard_normal(
        int(np.prod(dims))).astype(np.float32)
    packed = draw(st.booleans())
    return nodes, dims, data, packed


@settings(max_examples=60, deadline=None)
@given(_graphs())
def test_random_graph_round_trip(case):
    """Whatever the encoder writes, the parser reads back: node inputs /
    outputs / op types, int64 attribute lists (negative values as 10-byte
    varints, packed), float lists, a scalar int attribute and an
    initializer's dims and bytes."""
    nodes, dims, data, packed = case
    gl = []
    for ins, outs, op, ints, floats, name_i in nodes:
        attrs = [text(1, "i") + vint(20, 2) + vint(3, name_i)]
        if ints:
            body = sum((varint(v) for v in ints), [])
            attrs.append(text(1, "ints") + (len_delim(8, body) if packed else
                                            sum((vint(8, v) for v in ints), [])))
        if floats:
            attrs.append(text(1, "floats") + len_delim(7, struct.pack(f"<{len(floats)}f", *floats)))
        gl += len_delim(1, node(ins, outs, op, attrs))
    gl += len_delim(5, tensor("w", dims, 1, data.tobytes(), packed_dims=packed))
    parsed = parse_onnx_graph(model(gl))
    assert len(parsed.nodes) == len(nodes)
    for n, (ins, outs, op, ints, floats, name_i) in zip(parsed.nodes, nodes):
        assert n.inputs == ins and n.outputs == outs and n.op_type == op
        assert get_attr_int(n, "i", None) == name_i
        assert (get_attr_ints(n, "ints", None) or []) == ints
        got_f = next((a.floats for a in n.attributes if a.name == "floats"), None) or []
        assert np.array_equal(np.float32(got_f), np.float32(floats))
    w = parsed.tensors["w"]
    assert w.dims == dims and np.array_equal(w.array(), data)
