"""GPU tests of multi-stream graph execution: mfh_graph_call with
ScheduleStreams' StreamIDs mapped to HIP streams and its SyncEvents to HIP
events (ir/stream_scheduler.go:56, ir/sync_event.go).

A wide graph of exact elementwise ops (neg, abs, relu, max, min and single
f32 roundings of add / sub / mul) runs with MaxStreams 1 and 4; every output
must equal the numpy float32 evaluation of the same ops bit for bit, on
repeated calls from alternating caller streams, so that a missing wait or a
workspace region reused while another stream still reads it shows up as a
wrong value.
"""
import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd import plan as P
from manifesto_amd.graph import Graph, GraphNode

from gpu_util import empty_dev, log, to_dev, to_host, torch_mod

pytestmark = pytest.mark.gpu

F32 = M.FLOAT32


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def wide_graph():
    nodes = [
        GraphNode("a1", "math.neg", ["x"]), GraphNode("a2", "math.abs", ["a1"]),
        GraphNode("a3", "activation.relu", ["a2"]),
        GraphNode("b1", "math.abs", ["y"]), GraphNode("b2", "math.neg", ["b1"]),
        GraphNode("b3", "math.max", ["b2", "a1"]),
        GraphNode("c1", "math.mul", ["x", "y"]), GraphNode("c2", "math.sub", ["c1", "x"]),
        GraphNode("d", "math.add", ["a3", "b3"]), GraphNode("e", "math.min", ["d", "c2"]),
        GraphNode("f", "math.mul", ["e", "c1"]),
    ]
    return Graph(inputs=["x", "y"], execution_dtype=F32, nodes=nodes,
                 outputs={"f": "f", "a3": "a3", "c2": "c2", "c2_again": "c2"})


def expected(x, y):
    a1 = -x
    a3 = np.maximum(np.abs(a1), np.float32(0))
    b3 = np.maximum(-np.abs(y), a1)
    c1 = x * y
    c2 = c1 - x
    d = a3 + b3
    e = np.minimum(d, c2)
    return {"f": e * c1, "a3": a3, "c2": c2, "c2_again": c2}


def run(graph, x, y, stream, reps):
    torch = torch_mod()
    n = x.size
    tx, px = to_dev(x)
    ty, py = to_dev(y)
    outs = {k: empty_dev(4 * n) for k in ("f", "a3", "c2", "c2_again")}
    want = expected(x, y)
    side = torch.cuda.Stream()
    for r in range(reps):
        s = stream if r % 2 == 0 else side.cuda_stream
        for t, _ in outs.values():
            t.fill_(0xA5)
        torch.cuda.synchronize()
        graph.call({"x": (px, F32, n), "y": (py, F32, n)}, {k: (p, F32, n) for k, (t, p) in outs.items()}, s)
        torch.cuda.synchronize()
        for k, (t, _) in outs.items():
            got = to_host(t, np.float32)
            bad = np.flatnonzero(got.view(np.uint32) != want[k].view(np.uint32))
            assert bad.size == 0, f"call {r} output {k}: {bad.size} mismatches, first at {bad[:4]}"


@pytest.mark.parametrize("max_streams", [1, 4])
def test_wide_graph_on_streams(max_streams):
    n = (1 << 22) + 77
    log(f"graph streams max_streams={max_streams} n={n}")
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, n).astype(np.float32)
    y = rng.normal(0, 1, n).astype(np.float32)
    graph = wide_graph()
    P.set_max_streams(graph, max_streams)
    run(graph, x, y, torch_mod().cuda.current_stream().cuda_stream, 4)
    used = P.streams_used(graph)
    assert used == (1 if max_streams == 1 else 3)
    log(f"graph streams max_streams={max_streams} used={used} ok")


def test_streams_schedule_matches_plan_graph():
    graph = wide_graph()
    t = P.plan_graph(graph, {"x": (F32, 64), "y": (F32, 64)}, max_streams=4)
    streams = [t.stream(i) for i in range(t.num_nodes)]
    # a-chain and the merges on stream 0, b-chain on 1, c-chain on 2
    assert streams == [0, 0, 0, 1, 1, 0, 2, 2, 0, 0, 0]


def test_multi_stream_workspace_grows_and_small_second_call():
    graph = wide_graph()
    P.set_max_streams(graph, 4)
    rng = np.random.default_rng(12)
    s = torch_mod().cuda.current_stream().cuda_stream
    for n in ((1 << 20) + 3, 4099, (1 << 21) + 1):
        log(f"graph streams resize n={n}")
        x = rng.normal(0, 1, n).astype(np.float32)
        y = rng.normal(0, 1, n).astype(np.float32)
        run(graph, x, y, s, 2)


def test_set_max_streams_rejects_bad_values():
    graph = wide_graph()
    with pytest.raises(M.MFHError, match="1 to 64"):
        P.set_max_streams(graph, 0)
    with pytest.raises(M.MFHError, match="1 to 64"):
        P.set_max_streams(graph, 65)
