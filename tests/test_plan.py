"""CPU tests of the workspace planner and stream scheduler (include/mfh_plan.h).

The reference's own tests (ir/planner_test.go, ir/stream_scheduler_test.go,
compiler/plan_test.go) are restated case by case against libmfh and against
the oracle restatement (oracle/plan.py); random topologies then compare the
two exactly, and brute force pins what both must satisfy: every allocation is
the lowest aligned offset free of live intervals, every producer -> consumer
edge is ordered by stream order and waits, and the stream-aware placement
never lets two concurrently live values share memory.
"""
import random

import pytest

import manifesto_amd as M
from manifesto_amd import graph as G
from manifesto_amd import plan as P
from oracle import plan as OP

F32 = M.FLOAT32


# ---- helpers --------------------------------------------------------------------

def linear_topology(port_count, dims=(64, 64)):
    """makeLinearTopology (ir/planner_test.go:21-40): node i reads port i and
    writes port i + 1."""
    t = P.Topology()
    ports = [t.port(F32, *dims) for _ in range(port_count)]
    for i in range(port_count - 1):
        t.node("step", [ports[i]], [ports[i + 1]])
    return t, ports


def diamond(t):
    a, b, c, d = (t.port(F32, 4) for _ in range(4))
    t.node("A", [], [a])
    t.node("B", [a], [b])
    t.node("C", [a], [c])
    t.node("D", [b, c], [d])


def fan_out(t):
    a, b, c, d = (t.port(F32, 4) for _ in range(4))
    t.node("A", [], [a])
    t.node("B", [a], [b])
    t.node("C", [a], [c])
    t.node("D", [a], [d])


def random_topology(rng, n_nodes, n_inputs=2, max_in=3, sym=False):
    """A random DAG in topological order: (libmfh Topology, oracle nodes,
    oracle ports).  Each node writes one or two ports and reads up to
    `max_in` earlier ports or graph inputs."""
    t = P.Topology()
    oports, onodes = {}, []

    def new_port():
        dt = rng.choice([M.FLOAT32, M.BFLOAT16, M.FLOAT16, M.INT4, M.UINT8])
        dims = [rng.randint(1, 40) for _ in range(rng.randint(0, 2))]
        if sym and dims and rng.random() < 0.3:
            dims[0] = "B"
        h = t.port(dt, *dims)
        oports[h] = OP.Port(dt, list(dims))
        return h

    avail = [new_port() for _ in range(n_inputs)]
    for i in range(n_nodes):
        k = rng.randint(0, min(max_in, len(avail)))
        ins = rng.sample(avail, k)
        if rng.random() < 0.1:
            ins.append(None)
        outs = [new_port() for _ in range(1 if rng.random() < 0.8 else 2)]
        t.node(f"n{i}", ins, outs)
        onodes.append(OP.Node(f"n{i}", list(ins), list(outs)))
        avail += outs
    if sym:
        t.bind("B", 3)
    return t, onodes, oports


def schedule_of(t):
    return [(t.node_id(i), t.stream(i), [(e.event_id, e.stream_id, e.wait) for e in t.barriers(i)])
            for i in range(t.num_nodes)]


def oracle_schedule(nodes):
    return [(n.id, n.stream, list(n.barriers)) for n in nodes]


def happens_before(sched):
    """Transitive closure of stream order and signal -> wait edges over a
    schedule [(id, stream, barriers)] in step order: hb[j] = steps strictly
    before j."""
    n = len(sched)
    hb = [set() for _ in range(n)]
    last, signal = {}, {}
    for j, (_, stream, barriers) in enumerate(sched):
        preds = []
        if stream in last:
            preds.append(last[stream])
        for e, s, wait in barriers:
            if wait and e in signal:
                preds.append(signal[e])
        for p in preds:
            hb[j] |= hb[p] | {p}
        for e, s, wait in barriers:
            if not wait:
                signal[e] = j
        last[stream] = j
    return hb


# ---- ir/stream_scheduler_test.go ---------------------------------------------------

def test_schedule_linear_topology_single_stream():
    t = P.Topology()
    a, b, c = (t.port(F32, 4) for _ in range(3))
    t.node("A", [], [a])
    t.node("B", [a], [b])
    t.node("C", [b], [c])
    t.schedule_streams(4)
    assert [t.stream(i) for i in range(3)] == [0, 0, 0]
    assert all(t.barriers(i) == [] for i in range(3))


def test_schedule_diamond_emits_sync():
    t = P.Topology()
    diamond(t)
    t.schedule_streams(4)
    assert [t.stream(i) for i in range(4)] == [0, 0, 1, 0]
    # C opened stream 1 from A on stream 0 (event 1); D merges on stream 0 and
    # waits for C on stream 1 (event 2), which C signals
    assert t.barriers(0) == [P.SyncEvent(1, 0, False)] and t.barriers(1) == []
    assert t.barriers(2) == [P.SyncEvent(1, 0, True), P.SyncEvent(2, 1, False)]
    assert t.barriers(3) == [P.SyncEvent(2, 1, True)]


def test_schedule_fan_out_assigns_distinct_streams():
    t = P.Topology()
    fan_out(t)
    t.schedule_streams(4)
    assert [t.stream(i) for i in range(4)] == [0, 0, 1, 2]
    assert t.barriers(1) == []
    assert any(e.wait and e.stream_id == 0 for e in t.barriers(2))
    assert any(e.wait and e.stream_id == 0 for e in t.barriers(3))
    # A signals once per waiting stream
    assert sorted(t.barriers(0), key=lambda e: e.event_id) == [P.SyncEvent(1, 0, False), P.SyncEvent(2, 0, False)]


def test_schedule_max_streams_cap():
    t = P.Topology()
    fan_out(t)
    t.schedule_streams(2)
    assert len({t.stream(i) for i in range(4)}) <= 2
    assert [t.stream(i) for i in range(4)] == [0, 0, 1, 0]


def test_schedule_serial_max_streams_1():
    t = P.Topology()
    diamond(t)
    t.schedule_streams(1)
    assert [t.stream(i) for i in range(4)] == [0] * 4
    assert all(t.barriers(i) == [] for i in range(4))


def test_schedule_empty_topology():
    P.Topology().schedule_streams(4)


def test_schedule_assigns_node_ids():
    t = P.Topology()
    diamond(t)
    t.schedule_streams(0)  # MaxStreams < 1: topology width
    assert [t.node_id(i) for i in range(4)] == [1, 2, 3, 4]


# ---- ir/planner_test.go -----------------------------------------------------------

def test_assign_port_ids_unique_and_first_appearance_order():
    t, ports = linear_topology(4)
    t.assign_port_ids()
    ids = [t.port_id(p) for p in ports]
    assert 0 not in ids and len(set(ids)) == 4
    # node 0 writes port 1 (ID 1) then reads port 0 (ID 2); later outputs follow
    assert ids == [2, 1, 3, 4]


def test_assign_port_ids_idempotent_and_keeps_preset_ids():
    t, ports = linear_topology(4)
    t.assign_port_ids()
    first = [t.port_id(p) for p in ports]
    t.assign_port_ids()
    assert [t.port_id(p) for p in ports] == first
    t = P.Topology()
    a, b, c = t.port(F32, 1, id=7), t.port(F32, 1), t.port(F32, 1)
    t.node("n", [a], [b])
    t.node("m", [b], [c])
    t.assign_port_ids()
    assert [t.port_id(p) for p in (a, b, c)] == [7, 8, 9]


def test_liveness_linear_chain():
    t, ports = linear_topology(4)
    t.assign_port_ids()
    iv = {v[0]: v for v in t.liveness()}
    assert len(iv) == 4
    assert iv[t.port_id(ports[0])][1:3] == (0, 0)  # unproduced input: step 0 to its consumer
    assert iv[t.port_id(ports[1])][1:3] == (0, 1)
    assert all(v[3] == 64 * 64 * 4 for v in iv.values())


def test_liveness_multi_consumer():
    t = P.Topology()
    inp, shared, o1, o2 = (t.port(F32, 32, 32) for _ in range(4))
    t.node("produce", [inp], [shared])
    t.node("consume1", [shared], [o1])
    t.node("consume2", [shared], [o2])
    t.assign_port_ids()
    iv = {v[0]: v for v in t.liveness()}
    assert iv[t.port_id(shared)][1:3] == (0, 2)


def test_liveness_rejects_unbound_symbol():
    t = P.Topology()
    p = t.port(F32, "B", 768)
    t.node("use", [p], [])
    t.assign_port_ids()
    with pytest.raises(M.MFHError, match=r'port id=1 \(unproduced input\): dim\[0\] symbol "B" is unbound'):
        t.liveness()


def test_liveness_resolves_bound_symbols():
    t = P.Topology()
    p = t.port(F32, "B", 768)
    t.node("use", [p], [])
    t.assign_port_ids()
    t.bind("B", 4)
    (iv,) = t.liveness()
    assert iv[3] == 4 * 768 * 4


def test_port_byte_size_scalar_and_packed():
    t = P.Topology()
    s, q, b = t.port(F32), t.port(M.INT4, 3, 5), t.port(16, 9)  # Bool packs 8 per byte
    t.node("use", [s, q, b], [])
    t.assign_port_ids()
    sizes = {v[0]: v[3] for v in t.liveness()}
    assert [sizes[t.port_id(p)] for p in (s, q, b)] == [4, 8, 2]


def test_allocate_offsets_disjoint_intervals_share_offset():
    total, out = P.allocate_offsets([(1, 0, 2, 128), (2, 3, 5, 128)], 64)
    assert out[0][4] == out[1][4] and total == 128


def test_allocate_offsets_overlapping_intervals_distinct():
    total, out = P.allocate_offsets([(1, 0, 5, 128), (2, 3, 7, 128)], 64)
    assert out[0][4] != out[1][4] and total == 256


def test_allocate_offsets_touching_intervals_overlap():
    # inclusive ranges: an interval ending at step 3 conflicts with one starting there
    total, out = P.allocate_offsets([(1, 0, 3, 64), (2, 3, 5, 64)], 64)
    assert out[0][4] != out[1][4] and total == 128


def test_allocate_offsets_rounds_to_alignment():
    total, out = P.allocate_offsets([(1, 0, 5, 17), (2, 3, 7, 17)], 64)
    assert all(v[3] == 64 and v[4] % 64 == 0 for v in out)
    assert total == 128


def test_allocate_offsets_empty_and_bad_align():
    assert P.allocate_offsets([], 64) == (0, [])
    with pytest.raises(M.MFHError, match="power of two"):
        P.allocate_offsets([(1, 0, 1, 8)], 48)


def test_plan_workspace_linear_topology():
    t, ports = linear_topology(4)
    t.plan_workspace(0)  # default alignment
    size, align, allocs = t.workspace()
    assert size > 0 and align == 64 and len(allocs) == 4
    for p in ports:
        off = t.port_offset(p)
        assert off is not None and off % 64 == 0


def test_plan_workspace_rejects_non_power_of_two_align():
    t, _ = linear_topology(3)
    with pytest.raises(M.MFHError, match="planner: Align=48 must be a power of two"):
        t.plan_workspace(48)


# ---- compiler/plan_test.go over mfh graphs -------------------------------------------

def chain_graph(n, extra_inputs=()):
    nodes = [G.GraphNode(f"n{i}", "math.neg", ["x" if i == 1 else f"n{i - 1}"]) for i in range(1, n + 1)]
    return G.Graph(["x", *extra_inputs], {"out": f"n{n}"}, nodes, M.FLOAT32)


def test_plan_graph_non_overlapping_offsets():
    g = chain_graph(2)
    t = P.plan_graph(g, {"x": (M.FLOAT32, 16)})  # 64 bytes per tensor
    size, align, allocs = t.workspace()
    assert size >= 64 and size % 64 == 0 and align == 64
    assert all(v[3] >= 64 and v[4] % 64 == 0 for v in allocs)
    for i in range(t.num_nodes):
        (out,) = t.node_ports(i, True)
        assert t.port_offset(out) is not None
    # producer outputs are the consumers' inputs (one port per edge)
    assert t.node_ports(0, True) == t.node_ports(1, False)


def test_plan_graph_reuses_offsets_when_lifetimes_do_not_overlap():
    g = chain_graph(3)
    t = P.plan_graph(g, {"x": (M.FLOAT32, 64)})  # 256 bytes per tensor
    size, _, allocs = t.workspace()
    assert size <= 512
    assert len({v[4] for v in allocs}) <= 2
    assert t.io_offset("x", False) == t.port_offset(t.node_ports(0, False)[0])
    assert t.io_offset("out", True) == t.port_offset(t.node_ports(2, True)[0])


def test_plan_graph_unconsumed_input_has_no_allocation():
    g = chain_graph(1, ["unused"])
    with pytest.raises(M.MFHError, match='graph input "unused" has no workspace allocation'):
        P.plan_graph(g, {"x": (M.FLOAT32, 8), "unused": (M.FLOAT32, 8)})


def test_plan_graph_streams_for_independent_branches():
    g = G.Graph(["x", "y"], {"out": "c"}, [G.GraphNode("a", "math.neg", ["x"]), G.GraphNode("b", "math.abs", ["y"]),
                                          G.GraphNode("c", "math.add", ["a", "b"])], M.FLOAT32)
    t = P.plan_graph(g, {"x": (M.FLOAT32, 32), "y": (M.BFLOAT16, 32)}, max_streams=4)
    assert [t.stream(i) for i in range(3)] == [0, 1, 0]
    assert t.barriers(2) == [P.SyncEvent(1, 1, True)] and t.barriers(1) == [P.SyncEvent(1, 1, False)]
    sizes = {v[0]: v[3] for v in t.workspace()[2]}
    assert sizes[t.port_id(t.node_ports(1, False)[0])] == 64  # the bf16 input: 32 x 2 bytes


# ---- random topologies: libmfh == oracle, both == brute force -------------------------

@pytest.mark.parametrize("seed", range(40))
def test_random_topologies_match_oracle(seed):
    rng = random.Random(seed)
    t, nodes, ports = random_topology(rng, rng.randint(1, 24), sym=seed % 4 == 0)
    bindings = {"B": 3} if seed % 4 == 0 else {}
    t.assign_port_ids()
    OP.assign_port_ids(nodes, ports)
    assert [t.port_id(h) for h in sorted(ports)] == [ports[h].id for h in sorted(ports)]
    live = t.liveness()
    olive = OP.analyze_liveness(nodes, ports, bindings)
    assert [v[:4] for v in live] == olive
    align = rng.choice([1, 16, 64, 256])
    total, out = P.allocate_offsets([v[:4] for v in live], align)
    assert (total, out) == OP.allocate_offsets(olive, align)
    t.plan_workspace(align)
    size, _, allocs = t.workspace()
    assert (size, allocs) == (total, out)
    max_streams = seed % 5  # 0 = topology width
    t.schedule_streams(max_streams)
    OP.schedule_streams(nodes, max_streams)
    assert schedule_of(t) == oracle_schedule(nodes)


@pytest.mark.parametrize("seed", range(40))
def test_allocation_is_lowest_free_and_never_overlaps(seed):
    rng = random.Random(1000 + seed)
    align = rng.choice([8, 64, 256])
    ivs = []
    for pid in range(1, rng.randint(1, 30) + 1):
        s = rng.randint(0, 20)
        ivs.append((pid, s, s + rng.randint(0, 6), rng.randint(0, 700)))
    rng.shuffle(ivs)
    total, out = P.allocate_offsets(ivs, align)
    placed = []
    for pid, start, end, size, off in out:
        assert size == -(-size // align) * align and off % align == 0
        live = [(o, z) for (s2, e2, z, o) in placed if e2 >= start]
        # brute force: the lowest aligned offset clear of every live block
        want = 0
        while any(want < o + z and o < want + size for o, z in live):
            want += align
        assert off == want
        placed.append((start, end, size, off))
    for i, a in enumerate(placed):
        for b in placed[:i]:
            if a[0] <= b[1] and b[0] <= a[1]:  # live ranges intersect (inclusive)
                assert a[3] + a[2] <= b[3] or b[3] + b[2] <= a[3]
    assert total == max([o + z for (_, _, z, o) in placed], default=0)


@pytest.mark.parametrize("seed", range(40))
def test_schedule_orders_every_edge(seed):
    rng = random.Random(2000 + seed)
    t, nodes, ports = random_topology(rng, rng.randint(2, 30), n_inputs=rng.randint(0, 3), max_in=3)
    max_streams = rng.choice([0, 1, 2, 3, 8])
    t.schedule_streams(max_streams)
    sched = schedule_of(t)
    if max_streams >= 1:
        assert len({s for _, s, _ in sched}) <= max_streams
    if max_streams == 1:
        assert all(b == [] for _, _, b in sched)
    hb = happens_before(sched)
    producer = {}
    for j, n in enumerate(nodes):
        for h in n.outputs:
            producer.setdefault(h, j)
        for h in n.inputs:
            if h in producer and producer[h] < j:
                assert producer[h] in hb[j], (seed, n.name, h)
    # every wait has its signal on an earlier node of the stream it names
    signals = {e: (j, s) for j, (_, _, b) in enumerate(sched) for e, s, w in b if not w}
    for j, (_, stream, b) in enumerate(sched):
        for e, s, w in b:
            if w:
                assert e in signals and signals[e][0] < j and sched[signals[e][0]][1] == s != stream


@pytest.mark.parametrize("seed", range(40))
def test_stream_workspace_never_shares_memory_between_concurrent_values(seed):
    rng = random.Random(3000 + seed)
    t, nodes, ports = random_topology(rng, rng.randint(2, 30), n_inputs=rng.randint(0, 2))
    t.schedule_streams(rng.choice([2, 3, 4, 8]))
    t.plan_stream_workspace(64)
    sched = schedule_of(t)
    hb = happens_before(sched)
    t.assign_port_ids()
    # values: produced ports with their producer and readers
    vals = {}
    for j, n in enumerate(nodes):
        for h in n.outputs:
            pid = t.port_id(h)
            if pid not in vals:
                vals[pid] = {"producer": j, "users": {j}, "off": t.port_offset(h)}
    for j, n in enumerate(nodes):
        for h in n.inputs:
            if h is not None and t.port_id(h) in vals and j > vals[t.port_id(h)]["producer"]:
                vals[t.port_id(h)]["users"].add(j)
    _, _, allocs = t.workspace()
    size = {v[0]: v[3] for v in allocs}
    items = sorted(vals.items())
    for i, (pa, a) in enumerate(items):
        for pb, b in items[:i]:
            if not (a["off"] < b["off"] + size[pb] and b["off"] < a["off"] + size[pa]):
                continue
            # sharing memory: one value's every user precedes the other's producer
            first, second = (a, b) if a["producer"] < b["producer"] else (b, a)
            assert all(u in hb[second["producer"]] for u in first["users"]), (seed, pa, pb)


@pytest.mark.parametrize("seed", range(20))
def test_stream_workspace_on_one_stream_is_plan_workspace(seed):
    rng = random.Random(4000 + seed)
    t1, nodes, ports = random_topology(rng, rng.randint(1, 25), n_inputs=0)
    rng = random.Random(4000 + seed)
    t2, _, _ = random_topology(rng, rng.randint(1, 25), n_inputs=0)
    t1.schedule_streams(1)
    t1.plan_stream_workspace(64)
    t2.plan_workspace(64)
    assert t1.workspace() == t2.workspace()
