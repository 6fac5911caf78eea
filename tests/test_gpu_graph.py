"""GPU parity of graph execution (mfh_graph_call): graphs built, optimised and
lowered by the graph layer, then run on the device and checked against the
oracle.

A fused node must give what CPUKernel.Run (codegen/cpu.go:59-214) gives for
its FusionAST; an unfused elementwise node what the same evaluator gives for
that one node; every node output is stored in its dtype with the reference's
rounding.  Kernels are attached with MFH_FUSION_PRECISE (transcendentals in
f64 as the reference writes them), so results agree to the bit except at f64
rounding ties: the bound is 1 ulp in the storage dtype.
"""
import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd import graph as G
from manifesto_amd.graph import Graph, GraphNode
import oracle as O

from gpu_util import compare_storage, empty_dev, log, stream, to_dev, to_host

pytestmark = pytest.mark.gpu

SIZE = {O.FLOAT32: 4, O.BFLOAT16: 2, O.FLOAT16: 2}
NP = {O.FLOAT32: np.float32, O.BFLOAT16: np.uint16, O.FLOAT16: np.uint16}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def normal(rng, n, dt, sigma=1.0):
    return O.encode(rng.normal(0.0, sigma, n).astype(np.float32), dt)


class Bufs:
    """Device copies of storage arrays and output buffers for one call."""

    def __init__(self):
        self.keep = []

    def input(self, a, dt):
        t, p = to_dev(a)
        self.keep.append(t)
        return (p, dt, a.size)

    def output(self, n, dt):
        t, p = empty_dev(n * SIZE[dt])
        self.keep.append(t)
        return t, (p, dt, n)


def fused_ast(node):
    fusion = node.attributes[G.FUSE_ATTRIBUTE_AST]
    return [(n.type, n.input_index, n.value) for n in fusion.root.preorder()], fusion.input_ports


def test_graph_call_swiglu():
    n = (1 << 20) + 13
    log(f"graph swiglu n={n}")
    rng = np.random.default_rng(0x5EED + 3)
    graph = Graph(inputs=["gate", "up"], outputs={"y": "h"}, execution_dtype=O.BFLOAT16, nodes=[
        GraphNode("act", "activation.swish", ["gate"], input_types=[O.BFLOAT16], output_type=O.BFLOAT16),
        GraphNode("h", "math.mul", ["act", "up"], input_types=[O.BFLOAT16, O.BFLOAT16], output_type=O.BFLOAT16)])
    assert G.run(graph).fusion.clusters == 1
    assert G.attach_kernels(graph, flags=M.FUSION_PRECISE) == 1
    gate, up = normal(rng, n, O.BFLOAT16), normal(rng, n, O.BFLOAT16)
    b = Bufs()
    out, ov = b.output(n, O.BFLOAT16)
    graph.call({"gate": b.input(gate, O.BFLOAT16), "up": b.input(up, O.BFLOAT16)}, {"y": ov}, stream())
    got = to_host(out, np.uint16)
    nodes, ports = fused_ast(graph.nodes[0])
    want = O.encode(O.run(nodes, [O.decode(gate, O.BFLOAT16), O.decode(up, O.BFLOAT16)], n), O.BFLOAT16)
    compare_storage(got, want, O.BFLOAT16, 1, "graph swiglu")
    assert np.mean(got == want) > 0.9999
    # the output was written in place: the workspace holds nothing
    assert graph.workspace_bytes() == 0


def test_graph_call_gelu_chain_with_broadcasts():
    rows, d = 96, 4096
    n = rows * d
    log(f"graph gelu chain n={n}")
    rng = np.random.default_rng(0x5EED + 4)
    graph = Graph(inputs=["x", "bias", "residual"], outputs={"out": "y"}, execution_dtype=O.FLOAT16, nodes=[
        GraphNode("s", "math.constant", [], attributes={"value": 1.1}),
        GraphNode("a", "math.add", ["x", "bias"], input_types=[O.FLOAT16, O.FLOAT16], output_type=O.FLOAT16),
        GraphNode("m", "math.mul", ["a", "s"], input_types=[O.FLOAT16, O.FLOAT32], output_type=O.FLOAT16),
        GraphNode("g", "activation.gelu", ["m"], input_types=[O.FLOAT16], output_type=O.FLOAT16),
        GraphNode("y", "math.add", ["g", "residual"], input_types=[O.FLOAT16, O.FLOAT16], output_type=O.FLOAT16)])
    G.run(graph)
    assert G.attach_kernels(graph, flags=M.FUSION_PRECISE) == 1
    x, res = normal(rng, n, O.FLOAT16), normal(rng, n, O.FLOAT16)
    bias = normal(rng, d, O.FLOAT16, 0.02)
    b = Bufs()
    out, ov = b.output(n, O.FLOAT16)
    graph.call({"x": b.input(x, O.FLOAT16), "bias": b.input(bias, O.FLOAT16),
                "residual": b.input(res, O.FLOAT16)}, {"out": ov}, stream())
    got = to_host(out, np.uint16)
    nodes, ports = fused_ast(graph.nodes[1])
    assert ports == ["x", "bias", "s", "residual"]
    s = np.array([1.1], np.float32)  # the constant node, fl32(Value)
    want = O.encode(O.run(nodes, [O.decode(x, O.FLOAT16), O.decode(bias, O.FLOAT16), s,
                                  O.decode(res, O.FLOAT16)], n, periods=[0, d, 1, 0]), O.FLOAT16)
    compare_storage(got, want, O.FLOAT16, 1, "graph gelu chain")
    assert np.mean(got == want) > 0.9999
    # only the constant lives in the workspace
    assert graph.workspace_bytes() == 256


def eval_node(op, args, out_dt, count):
    """One unfused node with the oracle: f32 evaluation, then the node's
    storage rounding."""
    t, _ = G.is_elementwise_op(op)
    full = [np.broadcast_to(a, (count // a.size, a.size)).reshape(-1) if a.size != count else a for a in args]
    v = O.eval_unary(t, full[0]) if len(full) == 1 else O.eval_binary(t, *full)
    return O.encode(v, out_dt)


def test_graph_call_mixed_nodes_workspace_and_outputs():
    # n1 = exp(x)          f32   (shared: read by n2 and n4 -> not absorbed)
    # n2 = n1 * y          bf16  \ fused with n3
    # n3 = relu(n2)        bf16  /
    # n4 = max(n1, k)      f16   (k: constant, a scalar operand; a graph output,
    #                            so not absorbed: a one-node kernel)
    # n5 = n4 - row        f32   (row: a [64] periodic input) fused with n6
    # n6 = neg(n5)         f32
    # outputs: a = n3, b = n6, c = n1 (an intermediate also read later), d = x, e = n4
    rows, d = 300, 64
    n = rows * d
    log(f"graph mixed n={n}")
    rng = np.random.default_rng(7)
    graph = Graph(inputs=["x", "y", "row"], execution_dtype=O.FLOAT32,
                  outputs={"a": "n3", "b": "n6", "c": "n1", "d": "x", "e": "n4"}, nodes=[
        GraphNode("k", "math.constant", [], attributes={"value": 0.75}),
        GraphNode("n1", "math.exp", ["x"], output_type=O.FLOAT32),
        GraphNode("n2", "math.mul", ["n1", "y"], output_type=O.BFLOAT16),
        GraphNode("n3", "activation.relu", ["n2"], output_type=O.BFLOAT16),
        GraphNode("n4", "math.max", ["n1", "k"], output_type=O.FLOAT16),
        GraphNode("n5", "math.sub", ["n4", "row"], output_type=O.FLOAT32),
        GraphNode("n6", "math.neg", ["n5"], output_type=O.FLOAT32)])
    stats = G.run(graph)
    assert stats.fusion.clusters == 2
    assert [nd.op for nd in graph.nodes] == ["math.constant", "math.exp", G.FUSE_OP, "math.max", G.FUSE_OP]
    assert G.attach_kernels(graph, flags=M.FUSION_PRECISE) == 2

    x = rng.normal(0, 1.5, n).astype(np.float32)
    y = normal(rng, n, O.BFLOAT16)
    row = normal(rng, d, O.FLOAT16)
    b = Bufs()
    outs = {}
    views = {}
    for key, dt in (("a", O.BFLOAT16), ("b", O.FLOAT32), ("c", O.FLOAT32), ("d", O.FLOAT32), ("e", O.FLOAT16)):
        outs[key], views[key] = b.output(n, dt)
    inputs = {"x": b.input(x, O.FLOAT32), "y": b.input(y, O.BFLOAT16), "row": b.input(row, O.FLOAT16)}
    graph.call(inputs, views, stream())

    # reference: CPUKernel of each fused AST, single-node evaluation otherwise;
    # a node downstream of a checked output is evaluated from the device's value
    compare_storage(to_host(outs["c"], np.float32), eval_node("math.exp", [x], O.FLOAT32, n), O.FLOAT32, 1,
                    "output c (exp node)")
    n1 = to_host(outs["c"], np.float32).copy()
    fused = graph.nodes[2]
    nodes, ports = fused_ast(fused)
    assert ports == ["n1", "y"]
    n3 = O.encode(O.run(nodes, [n1, O.decode(y, O.BFLOAT16)], n), O.BFLOAT16)
    n4 = eval_node("math.max", [n1, np.array([0.75], np.float32)], O.FLOAT16, n)
    compare_storage(to_host(outs["e"], np.uint16), n4, O.FLOAT16, 0, "output e (one-node max with a constant)")
    nodes, ports = fused_ast(graph.nodes[4])
    assert ports == ["n4", "row"]
    n6 = O.encode(O.run(nodes, [O.decode(n4, O.FLOAT16), O.decode(row, O.FLOAT16)], n, periods=[0, d]), O.FLOAT32)
    compare_storage(to_host(outs["a"], np.uint16), n3, O.BFLOAT16, 1, "output a (fused bf16)")
    compare_storage(to_host(outs["b"], np.float32), n6, O.FLOAT32, 0, "output b (fused f32)")
    np.testing.assert_array_equal(to_host(outs["d"], np.float32), x)  # an input passed through
    ws = graph.workspace_bytes()
    assert 0 < ws < 4 * n * 4

    # a second call reuses the workspace; a larger one grows it
    graph.call(inputs, views, stream())
    assert graph.workspace_bytes() == ws
    compare_storage(to_host(outs["b"], np.float32), n6, O.FLOAT32, 0, "output b (second call)")
    n2_ = 2 * n
    x2 = rng.normal(0, 1.0, n2_).astype(np.float32)
    y2 = normal(rng, n2_, O.BFLOAT16)
    b2 = Bufs()
    out_b, vb = b2.output(n2_, O.FLOAT32)
    out_c, vc = b2.output(n2_, O.FLOAT32)
    graph.call({"x": b2.input(x2, O.FLOAT32), "y": b2.input(y2, O.BFLOAT16), "row": b2.input(row, O.FLOAT16)},
               {"b": vb, "c": vc}, stream())
    assert graph.workspace_bytes() > ws
    n1b = to_host(out_c, np.float32).copy()
    compare_storage(n1b, eval_node("math.exp", [x2], O.FLOAT32, n2_), O.FLOAT32, 1, "output c (grown)")
    n4b = eval_node("math.max", [n1b, np.array([0.75], np.float32)], O.FLOAT16, n2_)
    n6b = O.encode(O.run(nodes, [O.decode(n4b, O.FLOAT16), O.decode(row, O.FLOAT16)], n2_, periods=[0, d]),
                   O.FLOAT32)
    compare_storage(to_host(out_b, np.float32), n6b, O.FLOAT32, 0, "output b (grown workspace)")


def test_graph_call_errors():
    graph = Graph(inputs=["x", "y"], outputs={"o": "r"}, nodes=[
        GraphNode("m", "math.mul", ["x", "y"]), GraphNode("r", "activation.relu", ["m"])])
    G.run(graph)
    b = Bufs()
    x = b.input(np.ones(10, np.float32), O.FLOAT32)
    y3 = b.input(np.ones(3, np.float32), O.FLOAT32)
    _, o10 = b.output(10, O.FLOAT32)
    with pytest.raises(M.MFHError, match="has no HIP kernel attached"):
        graph.call({"x": x, "y": x}, {"o": o10})
    G.attach_kernels(graph)
    with pytest.raises(M.MFHError, match="operand \"y\" has 3 elements, the node 10") as e:
        graph.call({"x": x, "y": y3}, {"o": o10})
    assert e.value.code == -3
    with pytest.raises(M.MFHError, match="unknown input \"z\""):
        graph.call({"x": x, "y": x, "z": x}, {"o": o10})
    with pytest.raises(M.MFHError, match="reads \"y\", which is neither"):
        graph.call({"x": x}, {"o": o10})
    _, o10h = b.output(10, O.FLOAT16)
    with pytest.raises(M.MFHError, match="output \"o\" holds f16") as e:
        graph.call({"x": x, "y": x}, {"o": o10h})
    assert e.value.code == -2
    with pytest.raises(M.MFHError, match="unknown output"):
        graph.call({"x": x, "y": x}, {"zz": o10})
    opaque = Graph(inputs=["x"], outputs={"o": "p"}, nodes=[GraphNode("p", "projection.linear", ["x"])])
    with pytest.raises(M.MFHError, match="has no HIP lowering"):
        opaque.call({"x": x}, {"o": o10})
    # a good call still works after the failures
    graph.call({"x": x, "y": x}, {"o": o10})
