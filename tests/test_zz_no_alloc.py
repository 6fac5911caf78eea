"""GPU tests of mfh_graph_call_noalloc (include/mfh_graph.h), the graph call
that allocates nothing: its constants and intermediates live in the
library's static device scratch.  No counterpart in the reference; it is
checked bit for bit against mfh_graph_call (runtime.Backend.CallGraph,
runtime/executor.go:22-27) on the same values, and through it against the
oracle.
"""
import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd import graph as G
from manifesto_amd.graph import Graph, GraphNode
import oracle as O

from gpu_util import log

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # MFH_GRAPH_SCRATCH_BYTES
D = 4096  # bias period


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def torch_mod():
    import torch
    return torch


def dev(a):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).copy()).cuda()


def empty(nbytes):
    torch = torch_mod()
    return torch.full((nbytes,), 0xA5, dtype=torch.uint8, device="cuda")


def gelu_chain_graph(with_mid=True):
    # The gelu chain of BASELINE config 4 left unfused: one kernel per node,
    # a constant and the intermediates in the workspace; with `with_mid` the
    # f32 middle value is also a graph output (written to the caller's
    # buffer, then read from there by the next node).
    outputs = {"out": "y", "mid": "m"} if with_mid else {"out": "y"}
    return Graph(inputs=["x", "bias", "residual"], outputs=outputs,
                 execution_dtype=O.FLOAT16, nodes=[
                     GraphNode("s", "math.constant", [], attributes={"value": 1.1}),
                     GraphNode("a", "math.add", ["x", "bias"], input_types=[O.FLOAT16, O.FLOAT16],
                               output_type=O.FLOAT16),
                     GraphNode("m", "math.mul", ["a", "s"], input_types=[O.FLOAT16, O.FLOAT32],
                               output_type=O.FLOAT32),
                     GraphNode("g", "activation.gelu", ["m"], input_types=[O.FLOAT32], output_type=O.FLOAT16),
                     GraphNode("y", "math.add", ["g", "residual"], input_types=[O.FLOAT16, O.FLOAT16],
                               output_type=O.FLOAT16)])


def chain_values(rng, rows):
    n = rows * D
    x = O.encode(rng.normal(0, 1, n).astype(np.float32), O.FLOAT16)
    r = O.encode(rng.normal(0, 1, n).astype(np.float32), O.FLOAT16)
    bias = O.encode(rng.normal(0, 0.02, D).astype(np.float32), O.FLOAT16)
    return x, bias, r


def run_chain(graph, vals, noalloc, stream, with_mid=True):
    x, bias, r = vals
    n = x.size
    dx, db, dr = dev(x), dev(bias), dev(r)
    out, mid = empty(2 * n), empty(4 * n if with_mid else 4)
    ins = {"x": (dx.data_ptr(), O.FLOAT16, n), "bias": (db.data_ptr(), O.FLOAT16, D),
           "residual": (dr.data_ptr(), O.FLOAT16, n)}
    outs = {"out": (out.data_ptr(), O.FLOAT16, n)}
    if with_mid:
        outs["mid"] = (mid.data_ptr(), O.FLOAT32, n)
    (graph.call_noalloc if noalloc else graph.call)(ins, outs, stream)
    M.stream_sync(stream)
    return out.cpu().numpy().view(np.uint16), mid.cpu().numpy().view(np.uint32)


def oracle_chain(vals):
    x, bias, r = vals
    n = x.size
    a = O.f32_to_f16(O.decode(x, O.FLOAT16) + np.tile(O.decode(bias, O.FLOAT16), n // D))
    m = (O.decode(a, O.FLOAT16) * np.float32(1.1)).astype(np.float32)
    g = O.f32_to_f16(O.eval_unary(O.N_GELU, m))
    y = O.f32_to_f16(O.decode(g, O.FLOAT16) + O.decode(r, O.FLOAT16))
    return y, m.view(np.uint32)


@pytest.mark.parametrize("with_mid", [True, False])
def test_noalloc_matches_graph_call_twice_in_a_row(with_mid):
    torch = torch_mod()
    stream = torch.cuda.Stream()
    s = stream.cuda_stream
    rng = np.random.default_rng(0x5EED + 4)
    big, small = chain_values(rng, 300), chain_values(rng, 37)
    graph = gelu_chain_graph(with_mid)
    assert G.attach_kernels(graph, flags=M.FUSION_PRECISE) == 0  # no fused node: one kernel per node
    log(f"noalloc: graph_call big and small (loads the kernels), with_mid={with_mid}")
    want_big = run_chain(graph, big, False, s, with_mid)
    want_small = run_chain(graph, small, False, s, with_mid)
    # the regular call holds its intermediates in its own workspace
    assert graph.workspace_bytes() > 0
    log("noalloc: noalloc big then small")
    got_big = run_chain(graph, big, True, s, with_mid)
    got_small = run_chain(graph, small, True, s, with_mid)
    for got, want, what in ((got_big, want_big, "big"), (got_small, want_small, "small")):
        assert np.array_equal(got[0], want[0]), f"{what}: out"
        assert np.array_equal(got[1], want[1]), f"{what}: mid"
    # and the regular call agrees with the oracle (f64 gelu: ties only)
    y, m = oracle_chain(small)
    if with_mid:
        assert np.array_equal(want_small[1], m)
    assert np.mean(want_small[0] == y) > 0.9999


def test_noalloc_fused_graph_writes_outputs_in_place():
    torch = torch_mod()
    s = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(0x5EED + 3)
    graph = Graph(inputs=["gate", "up"], outputs={"y": "h"}, execution_dtype=O.BFLOAT16, nodes=[
        GraphNode("act", "activation.swish", ["gate"], input_types=[O.BFLOAT16], output_type=O.BFLOAT16),
        GraphNode("h", "math.mul", ["act", "up"], input_types=[O.BFLOAT16, O.BFLOAT16], output_type=O.BFLOAT16)])
    assert G.run(graph).fusion.clusters == 1
    assert G.attach_kernels(graph) == 1
    for n in ((1 << 20) + 13, 4099):
        g = O.encode(rng.normal(0, 1, n).astype(np.float32), O.BFLOAT16)
        u = O.encode(rng.normal(0, 1, n).astype(np.float32), O.BFLOAT16)
        dg, du = dev(g), dev(u)
        o1, o2 = empty(2 * n), empty(2 * n)
        ins = {"gate": (dg.data_ptr(), O.BFLOAT16, n), "up": (du.data_ptr(), O.BFLOAT16, n)}
        graph.call(ins, {"y": (o1.data_ptr(), O.BFLOAT16, n)}, s)
        graph.call_noalloc(ins, {"y": (o2.data_ptr(), O.BFLOAT16, n)}, s)
        M.stream_sync(s)
        assert torch.equal(o1, o2), n


def test_noalloc_refusals():
    torch = torch_mod()
    s = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(5)
    # a graph whose kernels were never loaded: refused before anything runs
    fresh = gelu_chain_graph()
    G.attach_kernels(fresh, flags=M.FUSION_PRECISE)
    with pytest.raises(M.MFHError, match="has no kernel"):
        run_chain(fresh, chain_values(rng, 2), True, s)
    # more scratch than the static array holds: the f16 sum and the f32
    # product of 3 * 2^22 elements are live together (72 MiB), and so are
    # the product and the f16 gelu
    graph = gelu_chain_graph(with_mid=False)
    G.attach_kernels(graph, flags=M.FUSION_PRECISE)
    vals = chain_values(rng, 3072)
    run_chain(graph, vals, False, s, with_mid=False)  # loads the kernels; its own workspace grows
    assert graph.workspace_bytes() > SCRATCH_BYTES
    with pytest.raises(M.MFHError, match=f"bytes of scratch, the static scratch holds {SCRATCH_BYTES}"):
        run_chain(graph, vals, True, s, with_mid=False)
    # a call that fits still runs after the refusal
    small = chain_values(rng, 3)
    assert np.array_equal(run_chain(graph, small, True, s, with_mid=False)[0],
                          run_chain(graph, small, False, s, with_mid=False)[0])


def test_noalloc_under_stream_capture():
    # The intended caller: a stream being captured into a HIP graph.  The
    # captured call is replayed several times with eager work and
    # synchronisations between replays; every replay matches the eager call.
    torch = torch_mod()
    rng = np.random.default_rng(0x5EED + 6)
    vals = chain_values(rng, 64)
    graph = gelu_chain_graph()
    G.attach_kernels(graph, flags=M.FUSION_PRECISE)
    x, bias, r = vals
    n = x.size
    dx, db, dr = dev(x), dev(bias), dev(r)
    out, mid = empty(2 * n), empty(4 * n)
    ins = {"x": (dx.data_ptr(), O.FLOAT16, n), "bias": (db.data_ptr(), O.FLOAT16, D),
           "residual": (dr.data_ptr(), O.FLOAT16, n)}
    outs = {"out": (out.data_ptr(), O.FLOAT16, n), "mid": (mid.data_ptr(), O.FLOAT32, n)}
    s = torch.cuda.Stream()
    graph.call(ins, outs, s.cuda_stream)  # loads the kernels
    M.stream_sync(s.cuda_stream)
    want_out, want_mid = out.clone(), mid.clone()
    other = gelu_chain_graph()  # a second graph's calls overwrite the scratch between replays
    G.attach_kernels(other, flags=M.FUSION_PRECISE)
    small = chain_values(rng, 5)
    run_chain(other, small, False, s.cuda_stream)
    cg = torch.cuda.CUDAGraph()
    log("noalloc: capture")
    with torch.cuda.graph(cg, stream=s):
        graph.call_noalloc(ins, outs, s.cuda_stream)
    for k in range(3):
        out.fill_(0)
        mid.fill_(0)
        run_chain(other, small, True, s.cuda_stream)
        torch.cuda.synchronize()
        cg.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_out), f"replay {k}: out"
        assert torch.equal(mid, want_mid), f"replay {k}: mid"
