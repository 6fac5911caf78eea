"""CPU tests of the graph layer: the elementwise table, Fuse, ConstantFold and
AttachKernels with the HIP target (include/mfh_graph.h).

The first tests restate the reference's own cases (optimizer/optimizer_test.go,
optimizer/constant_fold_test.go, codegen/codegen_test.go) with the HIP target
in place of CPU/Metal.  The rest pin the quirks the Go code has and check that
Fuse preserves what a graph computes, with the oracle evaluating both forms.
No kernel is launched here.
"""
import math
import struct

import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd import graph as G
from manifesto_amd.graph import ASTNode, FusionAST, Graph, GraphNode
import oracle as O


def node_types(root):
    return [n.type for n in root.preorder()]


# ---- optimizer/optimizer_test.go -------------------------------------------------

def test_fuse_straight_chain():
    # TestFuseStraightChain (optimizer/optimizer_test.go:10-49)
    graph = Graph(inputs=["x", "y"], outputs={"result": "relu_out"}, nodes=[
        GraphNode("add_out", "math.add", ["x", "y"]),
        GraphNode("sigmoid_out", "activation.sigmoid", ["add_out"]),
        GraphNode("relu_out", "activation.relu", ["sigmoid_out"]),
    ])
    stats = G.fuse(graph)
    assert (stats.clusters, stats.nodes_fused, stats.nodes_removed) == (1, 3, 2)
    nodes = graph.nodes
    assert len(nodes) == 1
    assert nodes[0].op == G.FUSE_OP
    assert nodes[0].inputs == ["x", "y"]
    fusion = nodes[0].attributes[G.FUSE_ATTRIBUTE_AST]
    assert fusion.root.type == G.NODE_RELU
    assert fusion.root.children[0].type == G.NODE_SIGMOID
    assert fusion.root.children[0].children[0].type == G.NODE_ADD
    assert sorted(fusion.contained_node_ids) == ["add_out", "relu_out", "sigmoid_out"]
    assert nodes[0].metadata["fused_node_count"] == 3
    assert fusion.output_port == "relu_out" and fusion.count_expr == ""


def test_fuse_dag_swiglu_style_pattern():
    # TestFuseDAGSwiGLUStylePattern (optimizer/optimizer_test.go:51-80)
    graph = Graph(inputs=["gate", "up"], outputs={"result": "swiglu"}, nodes=[
        GraphNode("sig_gate", "activation.sigmoid", ["gate"]),
        GraphNode("swiglu", "math.mul", ["sig_gate", "up"]),
    ])
    stats = G.fuse(graph)
    assert (stats.clusters, stats.nodes_fused) == (1, 2)
    assert len(graph.nodes) == 1
    fusion = graph.nodes[0].attributes[G.FUSE_ATTRIBUTE_AST]
    assert fusion.root.type == G.NODE_MUL
    assert fusion.root.children[0].type == G.NODE_SIGMOID
    assert fusion.root.children[1].type == G.NODE_INPUT
    assert "gate" in fusion.input_ports and "up" in fusion.input_ports


def test_fuse_dag_residual_chain():
    # TestFuseDAGResidualChain (optimizer/optimizer_test.go:82-107)
    graph = Graph(inputs=["a", "b", "c"], outputs={"y": "relu_out"}, nodes=[
        GraphNode("inner_sum", "math.add", ["a", "b"]),
        GraphNode("outer_sum", "math.add", ["inner_sum", "c"]),
        GraphNode("relu_out", "activation.relu", ["outer_sum"]),
    ])
    stats = G.fuse(graph)
    assert (stats.clusters, stats.nodes_fused) == (1, 3)
    fusion = graph.nodes[0].attributes[G.FUSE_ATTRIBUTE_AST]
    assert fusion.root.type == G.NODE_RELU
    assert fusion.root.children[0].type == G.NODE_ADD
    assert fusion.root.children[0].children[0].type == G.NODE_ADD
    assert fusion.input_ports == ["a", "b", "c"]


def test_fuse_stops_at_non_elementwise():
    # TestFuseStopsAtNonElementwise (optimizer/optimizer_test.go:109-131)
    graph = Graph(inputs=["x", "weight"], outputs={"result": "relu_out"}, nodes=[
        GraphNode("scaled", "math.mul", ["x", "x"]),
        GraphNode("projected", "projection.linear", ["scaled"]),
        GraphNode("relu_out", "activation.relu", ["projected"]),
    ])
    assert G.fuse(graph).clusters == 0
    assert [n.op for n in graph.nodes] == ["math.mul", "projection.linear", "activation.relu"]


def test_fuse_skips_shared_intermediate():
    # TestFuseSkipsSharedIntermediate (optimizer/optimizer_test.go:133-153)
    graph = Graph(inputs=["x", "y"], outputs={"residual": "relu_out", "projected": "projected"}, nodes=[
        GraphNode("add_out", "math.add", ["x", "y"]),
        GraphNode("relu_out", "activation.relu", ["add_out"]),
        GraphNode("projected", "projection.linear", ["add_out"]),
    ])
    assert G.fuse(graph).clusters == 0
    assert len(graph.nodes) == 3


def test_elementwise_ops_lists_mapped_ops():
    # TestElementwiseOpsListsMappedOps (optimizer/optimizer_test.go:270-279)
    ops = G.elementwise_ops()
    for op in ("math.add", "math.mul", "activation.relu", "activation.gelu"):
        assert op in ops
    assert len(ops) == 18  # 20 table rows minus the disabled sin/cos


def test_elementwise_table_quirks():
    # optimizer/elementwise.go:27-36, 44-54
    assert G.is_elementwise_op("math.sign") == (G.NODE_NEG, True)  # placeholder mapping kept
    assert G.is_elementwise_op("math.sin") == (G.NODE_INVALID, False)
    assert G.is_elementwise_op("math.cos") == (G.NODE_INVALID, False)
    assert G.is_elementwise_op("activation.swish") == (G.NODE_SILU, True)
    assert G.is_elementwise_op("activation.swiglu") == (G.NODE_INVALID, False)  # Llama's swiglu node is not fused
    assert G.is_elementwise_op("  Math.ADD\t\n") == (G.NODE_ADD, True)  # TrimSpace + ToLower
    assert G.is_elementwise_op("math.matmul") == (G.NODE_INVALID, False)
    assert G.is_elementwise_op("") == (G.NODE_INVALID, False)


# ---- the BASELINE chains (SwiGLU and the f16 gelu chain) ---------------------------

def test_fuse_swiglu_graph_is_one_node():
    # swish(gate) -> mul(., up) => Mul(Silu(In0), In1), inputs [gate, up]
    graph = Graph(inputs=["gate", "up"], outputs={"y": "h"}, execution_dtype=M.BFLOAT16, nodes=[
        GraphNode("act", "activation.swish", ["gate"], input_types=[M.BFLOAT16], output_type=M.BFLOAT16),
        GraphNode("h", "math.mul", ["act", "up"], input_types=[M.BFLOAT16, M.BFLOAT16], output_type=M.BFLOAT16),
    ])
    assert G.fuse(graph).clusters == 1
    (node,) = graph.nodes
    fusion = node.attributes[G.FUSE_ATTRIBUTE_AST]
    assert node_types(fusion.root) == [G.NODE_MUL, G.NODE_SILU, G.NODE_INPUT, G.NODE_INPUT]
    assert [n.input_index for n in fusion.root.preorder() if n.type == G.NODE_INPUT] == [0, 1]
    assert fusion.input_ports == ["gate", "up"] and fusion.dtype == M.BFLOAT16
    # fusionInputTypes: boundary ports take the consumers' InputTypes (optimizer/fuse.go:303-350)
    assert node.input_types == [M.BFLOAT16, M.BFLOAT16] and node.output_type == M.BFLOAT16


def gelu_chain_graph():
    # add(x, bias) -> mul(., s) -> gelu -> add(., residual); s is a constant node
    return Graph(inputs=["x", "bias", "residual"], outputs={"out": "y"}, execution_dtype=M.FLOAT16, nodes=[
        GraphNode("s", "math.constant", [], attributes={"value": 1.1}),
        GraphNode("a", "math.add", ["x", "bias"], input_types=[M.FLOAT16, M.FLOAT16], output_type=M.FLOAT16),
        GraphNode("m", "math.mul", ["a", "s"], input_types=[M.FLOAT16, M.FLOAT32], output_type=M.FLOAT16),
        GraphNode("g", "activation.gelu", ["m"], input_types=[M.FLOAT16], output_type=M.FLOAT16),
        GraphNode("y", "math.add", ["g", "residual"], input_types=[M.FLOAT16, M.FLOAT16], output_type=M.FLOAT16),
    ])


def test_fuse_gelu_chain_keeps_constant_external():
    # => Add(Gelu(Mul(Add(In0, In1), In2)), In3), inputs [x, bias, s, residual];
    # the constant node is not elementwise, so it stays an input.
    graph = gelu_chain_graph()
    stats = G.run(graph)
    assert stats.constant_fold.nodes_folded == 0 and stats.fusion.clusters == 1
    nodes = graph.nodes
    assert [n.op for n in nodes] == ["math.constant", G.FUSE_OP]
    fusion = nodes[1].attributes[G.FUSE_ATTRIBUTE_AST]
    assert node_types(fusion.root) == [G.NODE_ADD, G.NODE_GELU, G.NODE_MUL, G.NODE_ADD, G.NODE_INPUT,
                                       G.NODE_INPUT, G.NODE_INPUT, G.NODE_INPUT]
    assert fusion.input_ports == ["x", "bias", "s", "residual"]
    assert nodes[1].input_types == [M.FLOAT16, M.FLOAT16, M.FLOAT32, M.FLOAT16]


# ---- Fuse: the conditions of buildOperand --------------------------------------------

def test_fuse_graph_output_is_not_absorbed():
    # Outputs count as consumers (optimizer/fuse.go:75-77): add_out stays materialised.
    graph = Graph(inputs=["x", "y"], outputs={"sum": "add_out", "r": "relu_out"}, nodes=[
        GraphNode("add_out", "math.add", ["x", "y"]),
        GraphNode("relu_out", "activation.relu", ["add_out"]),
    ])
    assert G.fuse(graph).clusters == 0
    assert [n.op for n in graph.nodes] == ["math.add", "activation.relu"]


def test_fuse_deduplicates_external_inputs():
    # mul(x, x) -> relu: x is one port read twice (optimizer/fuse.go:255-265)
    graph = Graph(inputs=["x"], outputs={"r": "r"}, nodes=[
        GraphNode("sq", "math.mul", ["x", "x"]), GraphNode("r", "activation.relu", ["sq"])])
    assert G.fuse(graph).clusters == 1
    fusion = graph.nodes[0].attributes[G.FUSE_ATTRIBUTE_AST]
    assert fusion.input_ports == ["x"]
    assert [n.input_index for n in fusion.root.preorder() if n.type == G.NODE_INPUT] == [0, 0]


def test_fuse_value_read_twice_by_one_node_stays_external():
    # consumerCount counts every read, so t feeding mul(t, t) is not inlined
    graph = Graph(inputs=["x"], outputs={"r": "r"}, nodes=[
        GraphNode("t", "activation.tanh", ["x"]), GraphNode("r", "math.mul", ["t", "t"])])
    assert G.fuse(graph).clusters == 0


def test_fuse_two_clusters_and_singletons():
    graph = Graph(inputs=["a", "b", "w"], outputs={"o": "out"}, nodes=[
        GraphNode("e1", "math.exp", ["a"]),
        GraphNode("s1", "math.sub", ["e1", "b"]),
        GraphNode("proj", "projection.linear", ["s1", "w"]),
        GraphNode("n1", "math.neg", ["proj"]),
        GraphNode("lone", "math.abs", ["b"]),
        GraphNode("out", "math.max", ["n1", "lone"]),
    ])
    stats = G.fuse(graph)
    # out absorbs n1 and lone; s1 absorbs e1; proj is opaque
    assert (stats.clusters, stats.nodes_fused, stats.nodes_removed) == (2, 5, 3)
    nodes = graph.nodes
    assert [n.id for n in nodes] == ["s1", "proj", "out"]
    top = nodes[2].attributes[G.FUSE_ATTRIBUTE_AST]
    assert node_types(top.root) == [G.NODE_MAX, G.NODE_NEG, G.NODE_INPUT, G.NODE_ABS, G.NODE_INPUT]
    assert top.input_ports == ["proj", "b"]
    assert top.contained_node_ids == ["n1", "lone", "out"]


def test_fuse_single_elementwise_node_is_not_fused():
    graph = Graph(inputs=["x"], outputs={"y": "y"}, nodes=[GraphNode("y", "activation.relu", ["x"])])
    assert G.fuse(graph).clusters == 0
    assert graph.nodes[0].op == "activation.relu"


# ---- fusion preserves what the graph computes -----------------------------------------

UNARY = [G.NODE_NEG, G.NODE_ABS, G.NODE_SQRT, G.NODE_EXP, G.NODE_LOG, G.NODE_RELU, G.NODE_SIGMOID,
         G.NODE_TANH, G.NODE_SILU, G.NODE_GELU, G.NODE_LEAKY_RELU]
BINARY = [G.NODE_ADD, G.NODE_SUB, G.NODE_MUL, G.NODE_DIV, G.NODE_MAX, G.NODE_MIN]
OP_OF = {G.NODE_ADD: "math.add", G.NODE_SUB: "math.sub", G.NODE_MUL: "math.mul", G.NODE_DIV: "math.div",
         G.NODE_MAX: "math.max", G.NODE_MIN: "math.min", G.NODE_NEG: "math.neg", G.NODE_ABS: "math.abs",
         G.NODE_SQRT: "math.sqrt", G.NODE_EXP: "math.exp", G.NODE_LOG: "math.log", G.NODE_RELU: "activation.relu",
         G.NODE_SIGMOID: "activation.sigmoid", G.NODE_TANH: "activation.tanh", G.NODE_SILU: "activation.swish",
         G.NODE_GELU: "activation.gelu", G.NODE_LEAKY_RELU: "activation.leaky_relu"}


def random_graph(rng, n_inputs, n_nodes):
    names = [f"in{k}" for k in range(n_inputs)]
    nodes = []
    for i in range(n_nodes):
        r = rng.random()
        if r < 0.1:
            op, ins = "projection.opaque", [names[rng.integers(len(names))]]
        elif r < 0.5:
            t = UNARY[rng.integers(len(UNARY))]
            op, ins = OP_OF[t], [names[rng.integers(len(names))]]
        else:
            t = BINARY[rng.integers(len(BINARY))]
            op, ins = OP_OF[t], [names[rng.integers(len(names))] for _ in range(2)]
        nodes.append(GraphNode(f"n{i}", op, ins))
        names.append(f"n{i}")
    outputs = {"last": f"n{n_nodes - 1}"}
    if rng.random() < 0.5:
        outputs["mid"] = f"n{rng.integers(n_nodes)}"
    return [f"in{k}" for k in range(n_inputs)], outputs, nodes


def evaluate(nodes, inputs, count):
    """Node-by-node f32 evaluation with the oracle; opaque ops are a fixed
    elementwise stand-in (x*0.5+1) so that they can sit inside a graph."""
    env = dict(inputs)
    for node in nodes:
        if node.op == G.FUSE_OP:
            fusion = node.attributes[G.FUSE_ATTRIBUTE_AST]
            flat = [(n.type, n.input_index, n.value) for n in fusion.root.preorder()]
            env[node.id] = O.run(flat, [env[p] for p in fusion.input_ports], count)
        elif node.op == "projection.opaque":
            env[node.id] = (env[node.inputs[0]] * np.float32(0.5) + np.float32(1.0)).astype(np.float32)
        else:
            t, _ = G.is_elementwise_op(node.op)
            args = [env[i] for i in node.inputs]
            env[node.id] = O.eval_unary(t, args[0]) if len(args) == 1 else O.eval_binary(t, *args)
    return env


def test_fuse_preserves_graph_semantics():
    rng = np.random.default_rng(0x5EED)
    count = 257
    for trial in range(60):
        ins, outs, nodes = random_graph(rng, int(rng.integers(1, 4)), int(rng.integers(2, 12)))
        data = {name: rng.normal(0, 2, count).astype(np.float32) for name in ins}
        before = evaluate(nodes, data, count)
        graph = Graph(inputs=ins, outputs=outs, nodes=nodes)
        stats = G.fuse(graph)
        fused_nodes = graph.nodes
        assert len(fused_nodes) == len(nodes) - stats.nodes_removed
        after = evaluate(fused_nodes, data, count)
        for key, value in outs.items():
            np.testing.assert_array_equal(before[value].view(np.uint32), after[value].view(np.uint32),
                                          err_msg=f"trial {trial} output {key}")
        for node in fused_nodes:  # every materialised value keeps its bits
            np.testing.assert_array_equal(before[node.id].view(np.uint32), after[node.id].view(np.uint32))


# ---- optimizer/constant_fold_test.go --------------------------------------------------

def test_constant_fold_binary_add():
    graph = Graph(outputs={"y": "sum"}, nodes=[
        GraphNode("a", "math.constant", attributes={"value": 1.5}),
        GraphNode("b", "math.constant", attributes={"value": 2.5}),
        GraphNode("sum", "math.add", ["a", "b"]),
    ])
    assert G.constant_fold(graph).nodes_folded == 1
    node = graph.nodes[2]
    assert node.op == "math.constant" and node.inputs == [] and node.attributes["value"] == 4.0


def test_constant_fold_chains_transitively():
    graph = Graph(outputs={"y": "relu_out"}, nodes=[
        GraphNode("a", "math.constant", attributes={"value": -3.0}),
        GraphNode("two", "math.constant", attributes={"value": 2.0}),
        GraphNode("scaled", "math.mul", ["a", "two"]),
        GraphNode("relu_out", "activation.relu", ["scaled"]),
    ])
    assert G.constant_fold(graph).nodes_folded == 2
    nodes = graph.nodes
    assert nodes[2].op == "math.constant" and nodes[2].attributes["value"] == -6.0
    assert nodes[3].op == "math.constant" and nodes[3].attributes["value"] == 0.0


def test_constant_fold_leaves_non_constant_inputs_alone():
    graph = Graph(inputs=["x"], outputs={"y": "sum"}, nodes=[
        GraphNode("k", "math.constant", attributes={"value": 7.0}),
        GraphNode("sum", "math.add", ["x", "k"]),
    ])
    assert G.constant_fold(graph).nodes_folded == 0
    assert graph.nodes[1].op == "math.add"


def test_constant_fold_unary_evaluations():
    graph = Graph(outputs={"y": "out"}, nodes=[
        GraphNode("a", "math.constant", attributes={"value": 0.5}),
        GraphNode("exp_out", "math.exp", ["a"]),
        GraphNode("tanh_out", "activation.tanh", ["a"]),
        GraphNode("out", "activation.sigmoid", ["a"]),
    ])
    assert G.constant_fold(graph).nodes_folded == 3
    nodes = graph.nodes
    assert nodes[1].attributes["value"] == pytest.approx(math.exp(0.5), abs=1e-9)
    assert nodes[2].attributes["value"] == pytest.approx(math.tanh(0.5), abs=1e-9)
    assert nodes[3].attributes["value"] == pytest.approx(1.0 / (1.0 + math.exp(-0.5)), abs=1e-9)


def test_run_pipeline_folds_then_fuses():
    graph = Graph(inputs=["x"], outputs={"y": "relu_out"}, nodes=[
        GraphNode("k", "math.constant", attributes={"value": 2.0}),
        GraphNode("scaled", "math.mul", ["x", "k"]),
        GraphNode("relu_out", "activation.relu", ["scaled"]),
    ])
    stats = G.run(graph)
    assert stats.constant_fold.nodes_folded == 0 and stats.fusion.clusters == 1


def test_run_options_disable_passes():
    def fresh():
        return Graph(inputs=["x"], outputs={"y": "r"}, nodes=[
            GraphNode("a", "math.constant", attributes={"value": 2.0}),
            GraphNode("b", "math.exp", ["a"]),
            GraphNode("m", "math.mul", ["x", "b"]),
            GraphNode("r", "activation.relu", ["m"])])
    g = fresh()
    st = G.run(g, disable_constant_fold=True)
    assert st.constant_fold.nodes_folded == 0 and st.fusion.clusters == 1
    g = fresh()
    st = G.run(g, disable_fusion=True)
    assert st.constant_fold.nodes_folded == 1 and st.fusion.clusters == 0
    assert [n.op for n in g.nodes] == ["math.constant", "math.constant", "math.mul", "activation.relu"]


def f64_bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


FOLD_VALUES = [0.0, -0.0, 0.5, -0.5, 1.0, -3.0, 2.25, 7.0, -7.5, 20.0, -20.0, 1e-300, 700.0, -745.0,
               math.inf, -math.inf, math.nan]


@pytest.mark.parametrize("t", UNARY)
def test_constant_fold_unary_matches_oracle(t):
    # evaluateUnary (optimizer/constant_fold.go:165-203) against the oracle's
    # restatement; exact for the arithmetic rows, within 1 f64 ulp for libm.
    nodes = [GraphNode("c%d" % i, "math.constant", attributes={"value": v}) for i, v in enumerate(FOLD_VALUES)]
    nodes += [GraphNode("u%d" % i, OP_OF[t], ["c%d" % i]) for i in range(len(FOLD_VALUES))]
    graph = Graph(nodes=nodes)
    assert G.constant_fold(graph).nodes_folded == len(FOLD_VALUES)
    got = [n.attributes["value"] for n in graph.nodes[len(FOLD_VALUES):]]
    for v, g in zip(FOLD_VALUES, got):
        want = O.fold(t, [v])
        if math.isnan(want):
            assert math.isnan(g), (t, v)
        elif t in (G.NODE_EXP, G.NODE_LOG, G.NODE_TANH, G.NODE_SIGMOID, G.NODE_SILU, G.NODE_GELU):
            assert abs(f64_bits(g) - f64_bits(want)) <= 1 or g == want, (t, v, g, want)
        else:
            assert f64_bits(g) == f64_bits(want), (t, v, g, want)


def test_constant_fold_binary_matches_oracle():
    vals = FOLD_VALUES
    for t in BINARY:
        for a in vals:
            for b in vals:
                graph = Graph(nodes=[GraphNode("a", "math.constant", attributes={"value": a}),
                                     GraphNode("b", "math.constant", attributes={"value": b}),
                                     GraphNode("r", OP_OF[t], ["a", "b"])])
                folded = G.constant_fold(graph).nodes_folded
                want = O.fold(t, [a, b])
                if want is None:  # Div by zero is not folded
                    assert folded == 0 and graph.nodes[2].op == OP_OF[t], (t, a, b)
                    continue
                got = graph.nodes[2].attributes["value"]
                assert (math.isnan(got) and math.isnan(want)) or f64_bits(got) == f64_bits(want), (t, a, b, got, want)


def test_constant_fold_quirks():
    graph = Graph(nodes=[
        GraphNode("nz", "math.constant", attributes={"value": -0.0}),
        GraphNode("nan", "math.constant", attributes={"value": math.nan}),
        GraphNode("zero", "math.constant", attributes={"value": 0.0}),
        GraphNode("r1", "activation.relu", ["nz"]),    # operand > 0 ? operand : 0  -> +0
        GraphNode("r2", "activation.relu", ["nan"]),   # NaN folds to 0, unlike evalCPU (NaN)
        GraphNode("d", "math.div", ["nz", "zero"]),    # not folded
        GraphNode("mx", "math.max", ["nz", "zero"]),   # Go math.Max(-0, +0) = +0
        GraphNode("mn", "math.min", ["zero", "nz"]),   # Go math.Min(+0, -0) = -0
        GraphNode("mxn", "math.max", ["nan", "zero"]),
        GraphNode("no_value", "math.constant"),        # no "value": not a constant
        GraphNode("x", "math.neg", ["no_value"]),
        GraphNode("odd", "math.add", ["zero"]),        # arity mismatch: not folded
    ])
    assert G.constant_fold(graph).nodes_folded == 5
    v = {n.id: n.attributes.get("value") for n in graph.nodes}
    assert f64_bits(v["r1"]) == 0 and f64_bits(v["r2"]) == 0
    assert f64_bits(v["mx"]) == 0 and f64_bits(v["mn"]) == f64_bits(-0.0)
    assert math.isnan(v["mxn"])
    ops = {n.id: n.op for n in graph.nodes}
    assert ops["d"] == "math.div" and ops["x"] == "math.neg" and ops["odd"] == "math.add"


# ---- codegen/codegen_test.go: AttachKernels with the HIP target ------------------------

def relu_fuse_graph():
    fusion = FusionAST(ASTNode(G.NODE_RELU, [ASTNode(G.NODE_INPUT, input_index=0)]), ["x"], "y")
    return Graph(inputs=["x"], outputs={"out": "y"}, nodes=[
        GraphNode("y", G.FUSE_OP, ["x"], attributes={G.FUSE_ATTRIBUTE_AST: fusion})])


def test_attach_kernels_to_graph():
    # TestAttachKernelsToGraph (codegen/codegen_test.go:163-212), HIP target
    graph = relu_fuse_graph()
    assert G.attach_kernels(graph) == 1
    kernels = graph.nodes[0].attributes[G.KERNEL_ATTRIBUTE]
    hip = kernels.For(G.TARGET_HIP)
    assert hip is not None and hip.target() == G.TARGET_HIP
    assert kernels.For(G.TARGET_CPU) is None and kernels.For(G.TARGET_METAL) is None
    assert kernels.targets() == [G.TARGET_HIP]
    assert hip.kernel_name() == "fused_y" and hip.num_inputs() == 1
    src = hip.source()
    assert "void fused_y(" in src and "(x0 < 0.0f) ? 0.0f : x0" in src


def test_attach_kernels_targets_without_emitter():
    graph = relu_fuse_graph()
    assert G.attach_kernels(graph, targets=[G.TARGET_CPU, G.TARGET_METAL, 7]) == 1
    assert G.KERNEL_ATTRIBUTE not in graph.nodes[0].attributes  # an empty KernelSet


def test_attach_kernels_missing_fusion_attribute():
    graph = Graph(inputs=["x"], outputs={"o": "b"}, nodes=[
        GraphNode("a", G.FUSE_OP, ["x"], attributes={G.FUSE_ATTRIBUTE_AST: relu_fuse_graph().nodes[0]
                                                     .attributes[G.FUSE_ATTRIBUTE_AST]}),
        GraphNode("b", G.FUSE_OP, ["a"])])
    with pytest.raises(M.MFHError) as e:
        G.attach_kernels(graph)
    assert 'codegen: fused node "b" missing "fusion_ast" attribute' in str(e.value)
    assert e.value.attached == 1


def test_attach_kernels_rejects_unreadable_dtype():
    graph = relu_fuse_graph()
    node = GraphNode("z", G.FUSE_OP, ["q"], input_types=[M.INT8],
                     attributes={G.FUSE_ATTRIBUTE_AST: FusionAST(
                         ASTNode(G.NODE_ABS, [ASTNode(G.NODE_INPUT)]), ["q"], "z")})
    graph.add_node(node)
    with pytest.raises(M.MFHError) as e:
        G.attach_kernels(graph)
    assert e.value.code == -2 and 'codegen: emit "z"' in str(e.value) and "is i8" in str(e.value)


def test_attach_kernels_rejects_arity_mismatch():
    # A math.mul node with one input (optimizer/optimizer_test.go:170-185 builds
    # one) fuses into a Mul with one child; EmitHIP refuses it.
    graph = Graph(inputs=["x"], outputs={"y": "r"}, nodes=[
        GraphNode("m", "math.mul", ["x"]), GraphNode("r", "activation.relu", ["m"])])
    assert G.fuse(graph).clusters == 1
    with pytest.raises(M.MFHError) as e:
        G.attach_kernels(graph)
    assert "has 1 children, its arity is 2" in str(e.value)


def test_attach_kernels_uses_port_types():
    graph = gelu_chain_graph()
    G.run(graph)
    assert G.attach_kernels(graph, flags=M.FUSION_PRECISE) == 1
    src = graph.nodes[1].attributes[G.KERNEL_ATTRIBUTE].For(G.TARGET_HIP).source()
    assert "mfh_ldw4_f16<1>(p0" in src and "mfh_ld4_f32<1>(p2" in src and "mfh_st4_f16(pout" in src
    assert "precise transcendentals" in src


def test_graph_call_requires_init():
    graph = relu_fuse_graph()
    G.attach_kernels(graph)
    if M.lib().mfh_init(0) == 0:
        pytest.skip("a GPU is present; graph calls are covered by the GPU tests")
    with pytest.raises(M.MFHError) as e:
        graph.call({"x": (0, M.FLOAT32, 0)}, {})
    assert e.value.code == -6


# ---- mfh_graph_output_shape: outputs sized before a call, with no device -----------

def _shape_inputs(n=16384, period=4096, dt=M.FLOAT16):
    return {"x": (None, dt, n), "bias": (None, dt, period), "residual": (None, dt, n)}


def test_output_shape_of_unfused_and_fused_graph():
    graph = gelu_chain_graph()
    assert graph.output_shape(_shape_inputs(), "out") == (M.FLOAT16, 16384)
    G.run(graph)
    G.attach_kernels(graph)
    assert graph.output_shape(_shape_inputs(), "out") == (M.FLOAT16, 16384)
    # a repeating row and a scalar broadcast to the node's length
    assert graph.output_shape(_shape_inputs(n=4096 * 3), "out") == (M.FLOAT16, 4096 * 3)


def test_output_shape_dtype_fallbacks_and_input_outputs():
    def g(exec_dt, out_t):
        return Graph(inputs=["a", "b"], outputs={"y": "s", "a_again": "a", "c": "k"}, execution_dtype=exec_dt,
                     nodes=[GraphNode("k", "math.constant", [], attributes={"value": 2.0}),
                            GraphNode("s", "math.add", ["a", "b"], output_type=out_t)])
    ins = {"a": (None, M.BFLOAT16, 10), "b": (None, M.BFLOAT16, 1)}
    # OutputType, else ExecutionDType, else Float32 (the graph call's rule)
    assert g(M.FLOAT16, M.BFLOAT16).output_shape(ins, "y") == (M.BFLOAT16, 10)
    assert g(M.FLOAT16, 0).output_shape(ins, "y") == (M.FLOAT16, 10)
    assert g(0, 0).output_shape(ins, "y") == (M.FLOAT32, 10)
    assert g(0, 0).output_shape(ins, "a_again") == (M.BFLOAT16, 10)
    assert g(0, 0).output_shape(ins, "c") == (M.FLOAT32, 1)


def test_output_shape_errors_match_the_call():
    graph = gelu_chain_graph()
    with pytest.raises(M.MFHError) as e:
        graph.output_shape(_shape_inputs(period=4095), "out")
    assert e.value.code == -3 and "operand \"bias\" has 4095 elements" in str(e.value)  # SHAPE_MISMATCH
    with pytest.raises(M.MFHError) as e:
        graph.output_shape(_shape_inputs(), "nope")
    assert "unknown output \"nope\"" in str(e.value)
    ins = _shape_inputs()
    del ins["residual"]
    with pytest.raises(M.MFHError) as e:
        graph.output_shape(ins, "out")
    assert "neither a bound input nor an earlier node" in str(e.value)
    with pytest.raises(M.MFHError) as e:
        graph.output_shape({**_shape_inputs(), "x": (None, M.F8E4M3, 16384)}, "out")
    assert e.value.code == -2  # MFH_ERR_DTYPE_UNSUPPORTED
