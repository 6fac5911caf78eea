"""GPU tests of graph-call replay: the second call of a plan (the same value
names, dtypes, counts and output aliasing) is captured as a HIP graph, and
later calls launch that graph, with the arguments of the launches whose
buffers changed updated in place.

Every call's outputs are checked against numpy float32 evaluations of the same
exact ops (one IEEE f32 rounding each), with the inputs rewritten by eager
torch work and a synchronisation between calls, so a replay that reads stale
inputs, skips a node or misses a changed constant shows up as a wrong value.
"""
import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd import graph as G
from manifesto_amd import plan as P
from manifesto_amd.abi import check
from manifesto_amd.graph import Graph, GraphNode

from gpu_util import log, torch_mod

pytestmark = pytest.mark.gpu

F32 = M.FLOAT32


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def chain_graph(fuse=True):
    # k = 0.75; a = x * k; b = a + y; c = relu(b); d = -c; e = max(d, x)
    g = Graph(inputs=["x", "y"], outputs={"e": "e", "c": "c"}, execution_dtype=F32, nodes=[
        GraphNode("k", "math.constant", [], attributes={"value": 0.75}),
        GraphNode("a", "math.mul", ["x", "k"]), GraphNode("b", "math.add", ["a", "y"]),
        GraphNode("c", "activation.relu", ["b"]), GraphNode("d", "math.neg", ["c"]),
        GraphNode("e", "math.max", ["d", "x"])])
    if fuse:
        G.run(g)
        G.attach_kernels(g)
    return g


def chain_expected(x, y, k=0.75):
    # the evaluator's rules: relu v < 0 ? 0 : v, max l > r ? l : r (codegen/cpu.go)
    b = x * np.float32(k) + y
    c = np.where(b < 0, np.float32(0), b)
    d = -c
    return {"e": np.where(d > x, d, x), "c": c}


class Buffers:
    def __init__(self, n, keys):
        torch = torch_mod()
        self.n = n
        self.x = torch.empty(n, device="cuda")
        self.y = torch.empty(n, device="cuda")
        self.out = {k: torch.empty(n, device="cuda") for k in keys}

    def fill(self, rng):
        torch = torch_mod()
        x = rng.normal(0, 1, self.n).astype(np.float32)
        y = rng.normal(0, 1, self.n).astype(np.float32)
        self.x.copy_(torch.from_numpy(x))  # eager work between calls
        self.y.copy_(torch.from_numpy(y))
        for t in self.out.values():
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        return x, y

    def call(self, graph, stream=None):
        torch = torch_mod()
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        graph.call({"x": self.x, "y": self.y}, self.out, s)

    def check(self, want, what):
        torch = torch_mod()
        torch.cuda.synchronize()
        for k, t in self.out.items():
            got = t.cpu().numpy()
            bad = np.flatnonzero(got.view(np.uint32) != want[k].view(np.uint32))
            assert bad.size == 0, f"{what} output {k}: {bad.size} mismatches, first at {bad[:4]}"


def test_replays_follow_new_input_contents():
    rng = np.random.default_rng(21)
    g = chain_graph()
    b = Buffers((1 << 20) + 5, ["e", "c"])
    for call in range(6):
        log(f"graph replay call {call}")
        x, y = b.fill(rng)
        b.call(g)
        b.check(chain_expected(x, y), f"call {call}")
    # call 0 launches, call 1 is captured, calls 2-5 replay
    assert g.replayed_calls() == 4


def test_replays_dropped_when_the_graph_changes():
    rng = np.random.default_rng(22)
    g = chain_graph()
    b = Buffers(4099, ["e", "c"])
    for _ in range(3):
        x, y = b.fill(rng)
        b.call(g)
        b.check(chain_expected(x, y), "before the change")
    assert g.replayed_calls() == 1
    # change the constant (node 0): the next calls must use 1.5
    assert g.nodes[0].op == G.CONSTANT_OP
    check(G._L().mfh_graph_set_attribute(g._h, 0, b"value", 1.5))
    for call in range(4):
        x, y = b.fill(rng)
        b.call(g)
        b.check(chain_expected(x, y, 1.5), f"after the change, call {call}")
    assert g.replayed_calls() == 3


def test_replays_per_buffer_set():
    rng = np.random.default_rng(23)
    g = chain_graph()
    sets = [Buffers(3 << 16, ["e", "c"]), Buffers(3 << 16, ["e", "c"])]
    for call in range(6):
        b = sets[call % 2]
        x, y = b.fill(rng)
        b.call(g)
        b.check(chain_expected(x, y), f"set {call % 2} call {call}")
    # call 0 launches, call 1 is captured, calls 2-5 replay bound to their set
    assert g.replayed_calls() == 4


def test_replay_off():
    rng = np.random.default_rng(24)
    g = chain_graph()
    g.set_replay(False)
    b = Buffers(1000, ["e", "c"])
    for call in range(4):
        x, y = b.fill(rng)
        b.call(g)
        b.check(chain_expected(x, y), f"call {call}")
    assert g.replayed_calls() == 0


def test_multi_stream_replay():
    rng = np.random.default_rng(25)
    nodes = [GraphNode("a1", "math.neg", ["x"]), GraphNode("a2", "math.abs", ["a1"]),
             GraphNode("b1", "math.abs", ["y"]), GraphNode("b2", "math.max", ["b1", "a1"]),
             GraphNode("c1", "math.mul", ["x", "y"]), GraphNode("d", "math.add", ["a2", "b2"]),
             GraphNode("e", "math.sub", ["d", "c1"])]
    g = Graph(inputs=["x", "y"], outputs={"e": "e", "b2": "b2"}, execution_dtype=F32, nodes=nodes)
    P.set_max_streams(g, 4)
    b = Buffers((1 << 21) + 1, ["e", "b2"])
    for call in range(5):
        log(f"multi-stream replay call {call}")
        x, y = b.fill(rng)
        b.call(g)
        a1 = -x
        b1 = np.abs(y)
        b2 = np.where(b1 > a1, b1, a1)
        b.check({"b2": b2, "e": (np.abs(a1) + b2) - x * y}, f"call {call}")
    assert P.streams_used(g) == 3
    assert g.replayed_calls() == 3


# the refused call leaves the second capture empty, which torch warns about
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_call_inside_a_caller_capture():
    torch = torch_mod()
    rng = np.random.default_rng(26)
    g = chain_graph()
    b = Buffers(1 << 18, ["e", "c"])
    x, y = b.fill(rng)
    b.call(g)  # sizes the workspace and uploads the constants outside the capture
    b.check(chain_expected(x, y), "warm-up")
    tg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(tg):
        b.call(g, torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        log(f"caller capture replay {rep}")
        x, y = b.fill(rng)
        tg.replay()
        b.check(chain_expected(x, y), f"torch graph replay {rep}")
    # unfused, the graph keeps a, b and d in its workspace: a larger call
    # inside a capture would have to grow it, which is refused
    g = chain_graph(fuse=False)
    x, y = b.fill(rng)
    b.call(g)
    b.check(chain_expected(x, y), "unfused warm-up")
    assert g.workspace_bytes() > 256
    big = Buffers(1 << 20, ["e", "c"])
    big.fill(rng)
    tg2 = torch.cuda.CUDAGraph()
    with pytest.raises(M.MFHError, match="must grow"):
        with torch.cuda.graph(tg2):
            big.call(g, torch.cuda.current_stream().cuda_stream)


def test_plans_follow_new_buffers_and_output_aliasing():
    # With replay off every call runs as plain launches from the plan of its
    # signature (names, dtypes, counts, which outputs share a buffer): new
    # buffers of the same shapes reuse the plan with their pointers rebound,
    # and an output bound twice to one buffer, then to two, is planned apart.
    torch = torch_mod()
    rng = np.random.default_rng(27)
    g = Graph(inputs=["x", "y"], outputs={"e": "e", "e2": "e", "c": "c"}, execution_dtype=F32, nodes=[
        GraphNode("k", "math.constant", [], attributes={"value": 0.75}),
        GraphNode("a", "math.mul", ["x", "k"]), GraphNode("b", "math.add", ["a", "y"]),
        GraphNode("c", "activation.relu", ["b"]), GraphNode("d", "math.neg", ["c"]),
        GraphNode("e", "math.max", ["d", "x"])])
    g.set_replay(False)
    n = (1 << 18) + 3
    for call in range(6):
        x = rng.normal(0, 1, n).astype(np.float32)
        y = rng.normal(0, 1, n).astype(np.float32)
        tx, ty = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()  # new buffers every call
        e = torch.full((n,), float("nan"), device="cuda")
        c = torch.full((n,), float("nan"), device="cuda")
        shared = call % 3 == 1
        e2 = e if shared else torch.full((n,), float("nan"), device="cuda")
        g.call({"x": tx, "y": ty}, {"e": e, "e2": e2, "c": c}, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        want = chain_expected(x, y)
        for name, t in (("e", e), ("e2", e2), ("c", c)):
            got = t.cpu().numpy()
            key = "c" if name == "c" else "e"
            bad = np.flatnonzero(got.view(np.uint32) != want[key].view(np.uint32))
            assert bad.size == 0, f"call {call} ({'shared' if shared else 'separate'}) output {name}: {bad.size} bad"
        log(f"plan reuse call {call}: {'shared' if shared else 'separate'} e/e2 ok")
    assert g.replayed_calls() == 0


def test_outputs_bound_over_inputs():
    # An output may be bound to an input's buffer.  It is written in place
    # only where the launch computing it is that input's one reader, element
    # for element; otherwise it is computed in the workspace and copied out
    # after the last launch, so that every launch reads the input as it was.
    torch = torch_mod()
    rng = np.random.default_rng(28)
    n = (1 << 16) + 7
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def fresh():
        return rng.normal(0, 1, n).astype(np.float32), rng.normal(0, 1, n).astype(np.float32)

    def same(got, want, what):
        got = got.cpu().numpy()
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:4]}"

    # unfused chain with c bound over x: x is read by the first launch and
    # the last; four calls on the same buffers (launch, capture, 2 replays)
    g = chain_graph(fuse=False)
    tx, ty = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    e = torch.empty(n, device="cuda")
    for call in range(4):
        x, y = fresh()
        tx.copy_(torch.from_numpy(x))
        ty.copy_(torch.from_numpy(y))
        e.fill_(float("nan"))
        torch.cuda.synchronize()
        g.call({"x": tx, "y": ty}, {"e": e, "c": tx}, stream())
        torch.cuda.synchronize()
        want = chain_expected(x, y)
        same(e, want["e"], f"chain call {call}: e")
        same(tx, want["c"], f"chain call {call}: c over x")
        log(f"in-place chain call {call} ok")
    assert g.replayed_calls() == 2

    # one fused launch reading x and y element for element: written in place
    k = np.float32(0.75)
    g = Graph(inputs=["x", "y"], outputs={"s": "s"}, execution_dtype=F32, nodes=[
        GraphNode("k", "math.constant", [], attributes={"value": 0.75}),
        GraphNode("a", "math.mul", ["x", "k"]), GraphNode("s", "math.add", ["a", "y"])])
    G.run(g)
    G.attach_kernels(g)
    g.set_replay(False)
    for call, target in enumerate(["x", "y", None, "x"]):
        x, y = fresh()
        tx, ty = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
        out = {"x": tx, "y": ty, None: torch.full((n,), float("nan"), device="cuda")}[target]
        g.call({"x": tx, "y": ty}, {"s": out}, stream())
        torch.cuda.synchronize()
        same(out, x * k + y, f"fused call {call} (s over {target})")
        if target:
            assert g.workspace_bytes() < 4 * n, "written in place: no room for s in the workspace"
        log(f"in-place fused call {call} over {target} ok")

    # s bound one element into x's buffer: computed aside, copied out
    store = torch.empty(n + 1, device="cuda")
    x, y = fresh()
    store[:n].copy_(torch.from_numpy(x))
    ty = torch.from_numpy(y).cuda()
    g.call({"x": store[:n], "y": ty}, {"s": store[1:]}, stream())
    torch.cuda.synchronize()
    same(store[1:], x * k + y, "s overlapping x by all but one element")
    assert g.workspace_bytes() >= 4 * n

    # x passed straight through to xc while s is bound over x: xc gets x as
    # it was
    g = Graph(inputs=["x", "y"], outputs={"s": "s", "xc": "x"}, execution_dtype=F32, nodes=[
        GraphNode("s", "math.add", ["x", "y"])])
    x, y = fresh()
    tx, ty = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    xc = torch.full((n,), float("nan"), device="cuda")
    g.call({"x": tx, "y": ty}, {"s": tx, "xc": xc}, stream())
    torch.cuda.synchronize()
    same(xc, x, "x passed through")
    same(tx, x + y, "s over x")


def fresh_views(torch, n, pad):
    """A new buffer of n floats, misaligned by one element when `pad`."""
    store = torch.empty(n + 1, device="cuda")
    return store[1:] if pad else store[:n]


@pytest.mark.parametrize("fuse", [False, True])
def test_replays_on_fresh_buffers(fuse):
    # New buffers on every call, every third one misaligned by one element, so
    # that launches switch between the vector and the element path: calls 2
    # onwards replay the captured graph with the changed launches rebound.
    torch = torch_mod()
    rng = np.random.default_rng(29 + fuse)
    g = chain_graph(fuse=fuse)
    n = (1 << 16) + 3
    for call in range(9):
        pad = call % 3 == 2
        x = rng.normal(0, 1, n).astype(np.float32)
        y = rng.normal(0, 1, n).astype(np.float32)
        tx, ty = fresh_views(torch, n, pad), fresh_views(torch, n, pad)
        te, tc = fresh_views(torch, n, pad), fresh_views(torch, n, not pad)
        tx.copy_(torch.from_numpy(x))
        ty.copy_(torch.from_numpy(y))
        te.fill_(float("nan"))
        tc.fill_(float("nan"))
        torch.cuda.synchronize()
        g.call({"x": tx, "y": ty}, {"e": te, "c": tc}, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        want = chain_expected(x, y)
        for k, t in (("e", te), ("c", tc)):
            got = t.cpu().numpy()
            bad = np.flatnonzero(got.view(np.uint32) != want[k].view(np.uint32))
            assert bad.size == 0, f"call {call} (pad {pad}) output {k}: {bad.size} mismatches"
        log(f"fresh-buffer call {call} (fused {fuse}, pad {pad}) ok")
    assert g.replayed_calls() == 7


def test_replays_rotate_buffer_sets_back_to_back():
    # Three buffer sets in turn, calls queued back to back with no host
    # synchronisation between them: the two executables take turns, each
    # rebound only once its previous launch has finished.
    torch = torch_mod()
    rng = np.random.default_rng(31)
    g = chain_graph(fuse=False)
    sets = [Buffers((1 << 17) + 9, ["e", "c"]) for _ in range(3)]
    inputs = [b.fill(rng) for b in sets]
    outs = []
    for call in range(12):
        b = sets[call % 3]
        out = {k: torch.empty(b.n, device="cuda") for k in ("e", "c")}
        g.call({"x": b.x, "y": b.y}, out, torch.cuda.current_stream().cuda_stream)
        outs.append((call % 3, out))
    torch.cuda.synchronize()
    for call, (k, out) in enumerate(outs):
        want = chain_expected(*inputs[k])
        for key, t in out.items():
            got = t.cpu().numpy()
            bad = np.flatnonzero(got.view(np.uint32) != want[key].view(np.uint32))
            assert bad.size == 0, f"call {call} set {k} output {key}: {bad.size} mismatches"
    assert g.replayed_calls() == 10


def test_replays_rebind_output_copies():
    # s bound one element into x's buffer is computed aside and copied out
    # after the last launch; on fresh buffers the replayed copy follows them.
    torch = torch_mod()
    rng = np.random.default_rng(32)
    k = np.float32(0.75)
    g = Graph(inputs=["x", "y"], outputs={"s": "s"}, execution_dtype=F32, nodes=[
        GraphNode("k", "math.constant", [], attributes={"value": 0.75}),
        GraphNode("a", "math.mul", ["x", "k"]), GraphNode("s", "math.add", ["a", "y"])])
    G.run(g)
    G.attach_kernels(g)
    n = (1 << 15) + 1
    for call in range(6):
        x = rng.normal(0, 1, n).astype(np.float32)
        y = rng.normal(0, 1, n).astype(np.float32)
        store = torch.empty(n + 1, device="cuda")
        store[:n].copy_(torch.from_numpy(x))
        ty = torch.from_numpy(y).cuda()
        torch.cuda.synchronize()
        g.call({"x": store[:n], "y": ty}, {"s": store[1:]}, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = store[1:].cpu().numpy()
        want = x * k + y
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"call {call}: {bad.size} mismatches"
    assert g.replayed_calls() == 4


def test_multi_stream_replays_only_on_captured_buffers():
    # A plan on several streams is not rebound: it replays on the buffers it
    # was captured with and runs plain launches on any others, with the
    # right results either way.
    rng = np.random.default_rng(33)
    nodes = [GraphNode("a1", "math.neg", ["x"]), GraphNode("a2", "math.abs", ["a1"]),
             GraphNode("b1", "math.abs", ["y"]), GraphNode("b2", "math.max", ["b1", "a1"]),
             GraphNode("c1", "math.mul", ["x", "y"]), GraphNode("d", "math.add", ["a2", "b2"]),
             GraphNode("e", "math.sub", ["d", "c1"])]
    g = Graph(inputs=["x", "y"], outputs={"e": "e", "b2": "b2"}, execution_dtype=F32, nodes=nodes)
    P.set_max_streams(g, 4)
    n = (1 << 18) + 5
    a, b = Buffers(n, ["e", "b2"]), Buffers(n, ["e", "b2"])
    # a: plain, b: captured, a: plain, b: replay, fresh: plain, b: replay
    for call, buf in enumerate([a, b, a, b, Buffers(n, ["e", "b2"]), b]):
        x, y = buf.fill(rng)
        buf.call(g)
        a1 = -x
        b1 = np.abs(y)
        b2 = np.where(b1 > a1, b1, a1)
        buf.check({"b2": b2, "e": (np.abs(a1) + b2) - x * y}, f"call {call}")
        log(f"multi-stream call {call} ok")
    assert P.streams_used(g) == 3
    assert g.replayed_calls() == 2


def test_replays_across_a_workspace_growth():
    # Small calls are captured and replayed; a larger call grows the
    # workspace, which drops every captured graph; small calls on new buffers
    # then run plain once, are captured again and replay, all bit-exact.
    torch = torch_mod()
    rng = np.random.default_rng(34)
    g = chain_graph(fuse=False)
    sizes = [4099, 4099, 4099, 1 << 18, 4099, 4099, 4099, 4099]
    for call, n in enumerate(sizes):
        b = Buffers(n, ["e", "c"])
        x, y = b.fill(rng)
        b.call(g)
        b.check(chain_expected(x, y), f"call {call} (n {n})")
        log(f"growth call {call} n {n}: replayed so far {g.replayed_calls()}")
    # small plan: plain, capture, replay; the large call grows the workspace and
    # drops it; small again: plain, capture, replay, replay
    assert g.replayed_calls() == 3
