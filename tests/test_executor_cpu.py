"""CPU tests of the executor mirror (no GPU): graph rewrites, buffer-pool
bucketing, planning / IO inference, and the CPU shape path of Executor.run.

The GroupNorm-fusion fixtures are the two graphs of the reference's
fusion-test.mjs:21-41 (Constant-node style, as in the VAE; initializer style,
as in the U-Net), with the same expectation: one fused site each.
"""
import numpy as np
import pytest

from drawinstant.executor import (OPS, Attr, BufferPool, CpuTensor, Executor, ExecutorError, Graph,
                                  Node, TensorProto, WeightCache, fuse_group_norm_pattern,
                                  fuse_mul_add_pattern, fuse_silu_pattern, infer_graph_io,
                                  plan_execution)


def f32(vals):
    return TensorProto([len(vals)], "float32", np.asarray(vals, np.float32).tobytes())


def i64(vals):
    return TensorProto([len(vals)], "int64", np.asarray(vals, np.int64).tobytes())


def mk(op, name, ins, outs, attrs=None):
    return Node(op, name, list(ins), list(outs), list(attrs or []))


def gn_fixture(const_as_initializer: bool, scale=(1, 1)):
    """fusion-test.mjs:21-41."""
    tensors = {"shape0": TensorProto([3], "int64", bytes(24)),
               "shape1": TensorProto([4], "int64", bytes(32)),
               "gamma": f32([1, 1]), "beta": f32([0, 0])}
    nodes = [mk("Reshape", "/r0", ["X", "shape0"], ["r0"]),
             mk("InstanceNormalization", "/in", ["r0", "sc", "bi"], ["inout"],
                [Attr("epsilon", f=1e-5)]),
             mk("Reshape", "/r1", ["inout", "shape1"], ["r1"]),
             mk("AffineBcast", "/aff", ["r1", "gamma", "beta"], ["Y"])]
    if const_as_initializer:
        tensors["sc"], tensors["bi"] = f32(list(scale)), f32([0, 0])
    else:
        nodes = [mk("Constant", "/c_sc", [], ["sc"], [Attr("value", t=f32(list(scale)))]),
                 mk("Constant", "/c_bi", [], ["bi"], [Attr("value", t=f32([0, 0]))])] + nodes
    return Graph(nodes, outputs=[{"name": "Y"}], tensors=tensors)


@pytest.mark.parametrize("as_init", [False, True], ids=["constant-nodes", "initializers"])
def test_fuse_group_norm_reference_fixtures(as_init):
    g = gn_fixture(as_init)
    before = len(g.nodes)
    assert fuse_group_norm_pattern(g) == {"fused": 1}
    assert len(g.nodes) == before - 3
    gn = [n for n in g.nodes if n.op_type == "GroupNorm"]
    assert len(gn) == 1 and gn[0].inputs == ["X", "gamma", "beta"] and gn[0].outputs == ["Y"]
    attrs = {a.name: a for a in gn[0].attributes}
    assert attrs["num_groups"].i == 32 and attrs["epsilon"].f == pytest.approx(1e-5)


def test_fuse_group_norm_rejects_non_identity_scale():
    g = gn_fixture(True, scale=(1, 2))
    assert fuse_group_norm_pattern(g) == {"fused": 0}
    assert len(g.nodes) == 4


def test_mul_add_then_group_norm_chain_reads_groups_and_eps():
    """Mul/Add tail -> AffineBcast -> GroupNorm; G from a Constant-node reshape
    shape [N, G, -1] (index 1), eps from the InstanceNorm attribute."""
    tensors = {"gamma": TensorProto([1, 64, 1, 1], "float32", np.ones(64, np.float32).tobytes()),
               "beta": TensorProto([1, 64, 1, 1], "float32", np.zeros(64, np.float32).tobytes()),
               "sc": f32([1] * 16), "bi": f32([0] * 16), "shape1": i64([1, 64, 8, 8])}
    nodes = [mk("Constant", "/s0", [], ["shape0"], [Attr("value", t=i64([0, 16, -1]))]),
             mk("Reshape", "/r0", ["X", "shape0"], ["r0"]),
             mk("InstanceNormalization", "/in", ["r0", "sc", "bi"], ["inout"],
                [Attr("epsilon", f=1e-6)]),
             mk("Reshape", "/r1", ["inout", "shape1"], ["r1"]),
             mk("Mul", "/mul", ["r1", "gamma"], ["m"]),
             mk("Add", "/add", ["m", "beta"], ["Y"])]
    g = Graph(nodes, outputs=[{"name": "Y"}], tensors=tensors)
    assert fuse_mul_add_pattern(g) == {"fused": 1}
    assert [n.op_type for n in g.nodes][-1] == "AffineBcast"
    assert fuse_group_norm_pattern(g) == {"fused": 1}
    gn = g.nodes[-1]
    attrs = {a.name: a for a in gn.attributes}
    assert gn.op_type == "GroupNorm" and attrs["num_groups"].i == 16
    assert attrs["epsilon"].f == pytest.approx(1e-6)


def test_fuse_mul_add_requires_matching_shapes():
    tensors = {"gamma": TensorProto([4], "float32", np.ones(4, np.float32).tobytes()),
               "beta": TensorProto([1, 4], "float32", np.zeros(4, np.float32).tobytes())}
    g = Graph([mk("Mul", "m", ["X", "gamma"], ["t"]), mk("Add", "a", ["t", "beta"], ["Y"])],
              outputs=[{"name": "Y"}], tensors=tensors)
    assert fuse_mul_add_pattern(g) == {"fused": 0}
    assert fuse_mul_add_pattern(g, {"gamma": [1, 4]}) == {"fused": 1}


def test_fuse_silu_pattern_and_guards():
    g = Graph([mk("Sigmoid", "s", ["X"], ["sg"]), mk("Mul", "m", ["sg", "X"], ["Y"])],
              outputs=[{"name": "Y"}])
    assert fuse_silu_pattern(g) == {"fused": 1}
    assert [(n.op_type, n.inputs) for n in g.nodes] == [("Silu", ["X"])]
    # the sigmoid output has a second consumer: not fusable
    g = Graph([mk("Sigmoid", "s", ["X"], ["sg"]), mk("Mul", "m", ["X", "sg"], ["Y"]),
               mk("Neg", "n", ["sg"], ["Z"])], outputs=[{"name": "Y"}, {"name": "Z"}])
    assert fuse_silu_pattern(g) == {"fused": 0}
    # Mul's other input is not the sigmoid's input
    g = Graph([mk("Sigmoid", "s", ["X"], ["sg"]), mk("Mul", "m", ["sg", "W"], ["Y"])],
              outputs=[{"name": "Y"}])
    assert fuse_silu_pattern(g) == {"fused": 0}


def test_plan_and_infer_io():
    nodes = [mk("Conv", "c", ["x", "w", "b"], ["h"]), mk("FancyOp", "f", ["h"], ["y"]),
             mk("FancyOp", "f2", ["y"], ["z"])]
    p = plan_execution(Graph(nodes))
    assert p["total"] == 3 and p["supported_count"] == 1
    assert p["unsupported_ops"] == [("FancyOp", 2)]
    io = infer_graph_io(nodes, {"w", "b"})
    assert io == {"inputs": [{"name": "x"}], "outputs": [{"name": "z"}]}
    # the reference's 37 op types plus the three the fusing rewrites insert
    assert len(OPS) == 40
    assert {"Gelu", "LayerNormalization", "FusedAttention"} <= set(OPS)


class _FakeBuf:
    def __init__(self, size):
        self.size = size
        self.handle = 0


class _FakeDevice:
    """Stands in for Device where no GPU call may happen."""
    ctx = None

    def __init__(self):
        self.created = []

    def create_buffer(self, n):
        b = _FakeBuf(n)
        self.created.append(b)
        return b

    def sync(self):
        pass

    def upload(self, *a):
        raise AssertionError("CPU-only test must not upload")

    def storage(self, *a):
        raise AssertionError("CPU-only test must not upload")


def test_buffer_pool_buckets_and_stats():
    pool = BufferPool(_FakeDevice())
    a = pool.acquire(1)
    assert a.size == 4096 and pool.allocs == 1 and pool.live == 1
    b = pool.acquire(4097)
    assert b.size == 8192 and pool.peak == 2
    pool.release(a)
    assert pool.live == 1
    c = pool.acquire(4000)  # same 4 KiB bucket: reused
    assert c is a and pool.allocs == 2
    pool.release(_FakeBuf(4096))  # not ours: ignored
    assert pool.live == 2 and pool.owns(b) and not pool.owns(_FakeBuf(8192))


def test_executor_cpu_shape_path():
    """Shape arithmetic stays on the CPU (int64 semantics: BigInt division
    truncates toward zero), as the reference's METADATA_OPS / shape-aware
    binary fast paths; nothing touches the device."""
    tensors = {"one": i64([1]), "two": i64([2]), "neg7": i64([-7]), "zero": i64([0]),
               "axes0": i64([0])}
    nodes = [
        mk("Shape", "sh", ["ids"], ["s"]),                       # [2, 3]
        mk("Gather", "g", ["s", "one"], ["d1"]),                 # [3]
        mk("Mul", "m", ["d1", "two"], ["d2"]),                   # [6]
        mk("Div", "dv", ["neg7", "two"], ["q"]),                 # [-3] (trunc)
        mk("Concat", "c", ["d2", "q"], ["cat"], [Attr("axis", i=0)]),   # [6, -3]
        mk("Cast", "cf", ["cat"], ["catf"], [Attr("to", i=1)]),   # float32
        mk("Equal", "eq", ["q", "neg7"], ["e"]),                  # [False]
        mk("Where", "w", ["e", "one", "two"], ["wv"]),            # [2]
        mk("Slice", "sl", ["s", "zero", "one"], ["s0"]),          # [2]
        mk("Unsqueeze", "u", ["wv", "axes0"], ["wu"]),            # dims [1, 1]
        mk("ConstantOfShape", "cos", ["s"], ["filled"],
           [Attr("value", t=TensorProto([1], "int64", np.array([5], np.int64).tobytes()))]),
        mk("Cast", "c6", ["d2"], ["d2f"], [Attr("to", i=1)]),
        mk("Sqrt", "sq", ["d2f"], ["rt"]),  # 1-element shape value: CPU fast path (attention scale)
    ]
    g = Graph(nodes, outputs=[{"name": n} for n in ("cat", "catf", "wv", "s0", "wu", "filled",
                                                     "rt")], tensors=tensors)
    dev = _FakeDevice()
    ex = Executor(dev, g, WeightCache(dev, tensors))
    out = ex.run({"ids": CpuTensor(np.arange(6, dtype=np.int64), [2, 3], "int64")})
    assert out["cat"].cpu_data.tolist() == [6, -3] and out["cat"].dtype == "int64"
    assert out["catf"].cpu_data.dtype == np.float32
    assert out["wv"].cpu_data.tolist() == [2]
    assert out["s0"].cpu_data.tolist() == [2]
    assert out["wu"].dims == [1, 1]
    assert out["filled"].cpu_data.tolist() == [5] * 6 and out["filled"].dims == [2, 3]
    np.testing.assert_allclose(out["rt"].cpu_data, [np.sqrt(6.0)], rtol=1e-6)
    assert dev.created == []


def test_executor_error_convention():
    g = Graph([mk("Gather", "bad_gather", ["x", "i"], ["y"])], outputs=[{"name": "y"}],
              tensors={"i": i64([0])})
    dev = _FakeDevice()
    ex = Executor(dev, g, WeightCache(dev, g.tensors))
    with pytest.raises(ExecutorError, match=r"op @0 Gather \(bad_gather\) failed: .*GPU-tensor path"):
        ex.run({"x": CpuTensor(np.zeros(4, np.float32), [4], "float32", is_shape=False)})
    g2 = Graph([mk("NoSuchOp", "n", ["x"], ["y"])], outputs=[{"name": "y"}])
    with pytest.raises(ExecutorError, match="unsupported op @0: NoSuchOp"):
        Executor(dev, g2, WeightCache(dev, {})).run({"x": CpuTensor(np.zeros(1), [1], "float32")})
