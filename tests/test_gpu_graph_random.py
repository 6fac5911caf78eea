"""GPU differential test of the whole graph path on random graphs: build,
ConstantFold + Fuse (optimizer.Run), AttachKernels with the HIP target,
mfh_graph_call, checked against the oracle's node-by-node evaluation of the
same optimised graph (CPUKernel.Run for fused nodes, evalCPU for the rest,
codegen/cpu.go:59-214, each node's output stored in its dtype).

The ops are the ones whose f32 result is exact or correctly rounded (add,
sub, mul, div, max, min, neg, abs, relu, sqrt), so every output must match
to the bit (NaN positions included).  A second set of graphs adds every
transcendental op the optimizer fuses (exp, log, sigmoid, tanh, swish, gelu,
leaky_relu), compiled with MFH_FUSION_PRECISE (the reference's f64 results,
rounded once), and must match to the bit as well; so must the same graphs
over f32 inputs and outputs at default flags, whose kernels all stream f32
and take the rounding-tested activations.  Inputs mix storage dtypes and operand
modes (full, a repeating row, a scalar); nodes get random output types;
outputs include intermediates read later and inputs passed through.  Each
graph is called three times (plain launches, capture, replay) and, for half
the seeds, over several streams.
"""
import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd import graph as G
from manifesto_amd import plan as P
from manifesto_amd.graph import Graph, GraphNode
import oracle as O

from gpu_util import compare_storage, empty_dev, log, stream, to_dev, to_host

pytestmark = pytest.mark.gpu

UNARY = ["math.neg", "math.abs", "activation.relu", "math.sqrt"]
BINARY = ["math.add", "math.sub", "math.mul", "math.div", "math.max", "math.min"]
DTYPES = [O.FLOAT32, O.BFLOAT16, O.FLOAT16]
SIZE = {O.FLOAT32: 4, O.BFLOAT16: 2, O.FLOAT16: 2}
NP = {O.FLOAT32: np.float32, O.BFLOAT16: np.uint16, O.FLOAT16: np.uint16}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def random_graph(rng, n, d):
    inputs = {}
    for k in range(int(rng.integers(1, 4))):
        count = [n, d, 1][int(rng.choice(3, p=[0.6, 0.25, 0.15]))]
        inputs[f"in{k}"] = (DTYPES[int(rng.integers(3))], count)
    names = list(inputs)
    nodes = []
    if rng.random() < 0.5:
        nodes.append(GraphNode("k0", "math.constant", [], attributes={"value": float(rng.normal(0, 2))}))
        names.append("k0")
    n_nodes = int(rng.integers(3, 11))
    for i in range(n_nodes):
        pick = lambda: names[int(rng.integers(len(names)))]  # noqa: E731
        if rng.random() < 0.4:
            op, ins = UNARY[int(rng.integers(len(UNARY)))], [pick()]
        else:
            op, ins = BINARY[int(rng.integers(len(BINARY)))], [pick(), pick()]
        out_t = [0, O.FLOAT32, O.BFLOAT16, O.FLOAT16][int(rng.integers(4))]
        nodes.append(GraphNode(f"n{i}", op, ins, output_type=out_t))
        names.append(f"n{i}")
    outputs = {"last": f"n{n_nodes - 1}"}
    if rng.random() < 0.6:
        outputs["mid"] = f"n{int(rng.integers(n_nodes))}"
    if rng.random() < 0.2:
        outputs["pass"] = "in0"
    return inputs, nodes, outputs


def oracle_values(graph, data):
    """Storage array and dtype of every value of the optimised graph."""
    store = dict(data)  # name -> (storage array, dtype)
    f32 = {k: O.decode(a, dt) for k, (a, dt) in data.items()}
    for node in graph.nodes:
        if node.op == "math.constant":
            f32[node.id] = np.array([node.attributes["value"]], np.float64).astype(np.float32)  # fl32(Value)
            store[node.id] = (f32[node.id], O.FLOAT32)
            continue
        out_dt = node.output_type or O.FLOAT32
        if node.op == G.FUSE_OP:
            fusion = node.attributes[G.FUSE_ATTRIBUTE_AST]
            flat = [(x.type, x.input_index, x.value) for x in fusion.root.preorder()]
            args = [f32[p] for p in fusion.input_ports]
        else:
            t, _ = G.is_elementwise_op(node.op)
            flat = O.flatten((t, *[("in", k) for k in range(len(node.inputs))]))
            args = [f32[p] for p in node.inputs]
        count = max(a.size for a in args)
        periods = [0 if a.size == count else a.size for a in args]
        v = O.run(flat, args, count, periods)
        store[node.id] = (O.encode(v, out_dt), out_dt)
        f32[node.id] = O.decode(store[node.id][0], out_dt)
    return store


@pytest.mark.parametrize("seed", range(16))
def test_random_graph_matches_the_oracle(seed):
    rng = np.random.default_rng(0x5EED + 100 + seed)
    rows, d = 101, 12
    n = rows * d  # not a multiple of 8: every vector path has a tail
    inputs, nodes, outputs = random_graph(rng, n, d)
    graph = Graph(inputs=list(inputs), outputs=outputs, execution_dtype=O.FLOAT32, nodes=nodes)
    G.run(graph)
    G.attach_kernels(graph)
    if seed % 2:
        P.set_max_streams(graph, 3)
    log(f"random graph {seed}: {[(nd.id, nd.op) for nd in graph.nodes]}")
    data = {}
    for name, (dt, count) in inputs.items():
        a = rng.normal(0, 2, count).astype(np.float32)
        a[rng.random(count) < 0.05] *= -1e30  # overflow to inf in products, NaN from sqrt and inf - inf
        data[name] = (O.encode(a, dt), dt)
    want = oracle_values(graph, data)
    keep, ins = [], {}
    for name, (a, dt) in data.items():
        t, p = to_dev(a)
        keep.append(t)
        ins[name] = (p, dt, a.size)
    shapes = {key: graph.output_shape({k: (None, dt, a.size) for k, (a, dt) in data.items()}, key) for key in outputs}
    outs, views = {}, {}
    for key, (dt, count) in shapes.items():
        t, p = empty_dev(count * SIZE[dt])
        outs[key], views[key] = t, (p, dt, count)
    for call in range(3):  # the same buffers: plain launches, capture, replay
        for t in outs.values():
            t.fill_(0xA5)
        graph.call(ins, views, stream())
        for key, value in outputs.items():
            w, wdt = want[value]
            dt, count = shapes[key]
            assert (dt, count) == (wdt, w.size), f"seed {seed} output {key}: shape"
            got = to_host(outs[key], NP[dt])
            compare_storage(got, w.view(NP[dt]), dt, 0, f"seed {seed} call {call} output {key} ({value})")
    assert graph.replayed_calls() == 1


TRANSCENDENTAL = ["math.exp", "math.log", "activation.sigmoid", "activation.tanh", "activation.swish",
                  "activation.gelu", "activation.leaky_relu"]


def random_graph_transcendental(rng, n, d, dtypes=DTYPES, out_types=(0, O.FLOAT32, O.BFLOAT16, O.FLOAT16)):
    """random_graph's shapes and operand modes over every elementwise op the
    optimizer fuses, inputs in `dtypes`, node outputs in `out_types` (0: the
    execution dtype).  A gelu reads max(x, -4.5): below -4.9 the reference's
    own gelu (1 + tanh cancelling in f64) is rounding noise that two correct
    f64 evaluations may place a quantum apart."""
    inputs = {}
    for k in range(int(rng.integers(1, 4))):
        count = [n, d, 1][int(rng.choice(3, p=[0.6, 0.25, 0.15]))]
        inputs[f"in{k}"] = (dtypes[int(rng.integers(len(dtypes)))], count)
    names = list(inputs)
    nodes = [GraphNode("floor", "math.constant", [], attributes={"value": -4.5})]
    n_nodes = int(rng.integers(3, 11))
    for i in range(n_nodes):
        pick = lambda: names[int(rng.integers(len(names)))]  # noqa: E731
        out_t = out_types[int(rng.integers(len(out_types)))]
        r = rng.random()
        if r < 0.45:
            op = TRANSCENDENTAL[int(rng.integers(len(TRANSCENDENTAL)))]
            src = pick()
            if op == "activation.gelu":
                nodes.append(GraphNode(f"g{i}", "math.max", [src, "floor"]))
                src = f"g{i}"
            nodes.append(GraphNode(f"n{i}", op, [src], output_type=out_t))
        elif r < 0.6:
            nodes.append(GraphNode(f"n{i}", UNARY[int(rng.integers(len(UNARY)))], [pick()], output_type=out_t))
        else:
            nodes.append(GraphNode(f"n{i}", BINARY[int(rng.integers(len(BINARY)))], [pick(), pick()],
                                   output_type=out_t))
        names.append(f"n{i}")
    outputs = {"last": f"n{n_nodes - 1}"}
    if rng.random() < 0.6:
        outputs["mid"] = f"n{int(rng.integers(n_nodes))}"
    return inputs, nodes, outputs


@pytest.mark.parametrize("seed", range(12))
def test_random_transcendental_graph_precise_matches_the_oracle(seed):
    # MFH_FUSION_PRECISE gives every transcendental the reference's f64 value
    # rounded once, fused or not: bit-identical to the oracle's evaluation of
    # the optimised graph, NaN where it is NaN.
    check_transcendental_graph(seed, 0x5EED + 300 + seed, M.FUSION_PRECISE, DTYPES,
                               (0, O.FLOAT32, O.BFLOAT16, O.FLOAT16))


@pytest.mark.parametrize("seed", range(12))
def test_random_f32_transcendental_graph_matches_the_oracle_at_default_flags(seed):
    # f32 inputs and node outputs: every kernel streams f32, so its Sigmoid,
    # Silu and Gelu take the rounding-tested forms at default flags, and the
    # graph is bit-identical to the oracle's evaluation as under
    # MFH_FUSION_PRECISE.
    check_transcendental_graph(seed, 0x5EED + 400 + seed, 0, [O.FLOAT32], (0, O.FLOAT32))


def check_transcendental_graph(seed, rng_seed, flags, dtypes, out_types):
    rng = np.random.default_rng(rng_seed)
    rows, d = 101, 12
    n = rows * d  # not a multiple of 8: every vector path has a tail
    inputs, nodes, outputs = random_graph_transcendental(rng, n, d, dtypes, out_types)
    graph = Graph(inputs=list(inputs), outputs=outputs, execution_dtype=O.FLOAT32, nodes=nodes)
    G.run(graph)
    G.attach_kernels(graph, flags=flags)
    log(f"transcendental graph {seed} (flags {flags}): {[(nd.id, nd.op) for nd in graph.nodes]}")
    data = {}
    for name, (dt, count) in inputs.items():
        a = rng.normal(0, 2, count).astype(np.float32)
        a[rng.random(count) < 0.03] *= -1e30
        data[name] = (O.encode(a, dt), dt)
    want = oracle_values(graph, data)
    keep, ins = [], {}
    for name, (a, dt) in data.items():
        t, p = to_dev(a)
        keep.append(t)
        ins[name] = (p, dt, a.size)
    shapes = {key: graph.output_shape({k: (None, dt, a.size) for k, (a, dt) in data.items()}, key) for key in outputs}
    outs, views = {}, {}
    for key, (dt, count) in shapes.items():
        t, p = empty_dev(count * SIZE[dt])
        outs[key], views[key] = t, (p, dt, count)
    for call in range(3):
        for t in outs.values():
            t.fill_(0xA5)
        graph.call(ins, views, stream())
        for key, value in outputs.items():
            w, wdt = want[value]
            dt, count = shapes[key]
            assert (dt, count) == (wdt, w.size), f"seed {seed} output {key}: shape"
            got = to_host(outs[key], NP[dt])
            compare_storage(got, w.view(NP[dt]), dt, 0, f"seed {seed} call {call} output {key} ({value})")
    assert graph.replayed_calls() == 1
