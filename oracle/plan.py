"""CPU oracle for the planning IR — TEST INFRASTRUCTURE ONLY.

A plain-Python restatement of the reference's workspace planner
(ir/planner.go: AssignPortIDs :107-170, AnalyzeLiveness :186-280,
AllocateOffsets :296-350, chooseLowestNonConflictingOffset :376-411,
PortByteSize :437-480) and stream scheduler (ir/stream_scheduler.go:
ScheduleStreams :56-141, collectPredecessorStreams :179-212, pickStream
:229-287).  Only ``tests/`` import it, as the checker of libmfh's planner.

Parity: pinned by the reference's own tests (ir/planner_test.go,
ir/stream_scheduler_test.go, compiler/plan_test.go, restated in
tests/test_plan.py) and by brute force (every allocation is the lowest
aligned offset free of live intervals; every producer -> consumer edge is
ordered by stream order and waits).  One deliberate choice: where a node
waits on several streams, the reference numbers the events in Go map order
(unspecified); here, as in libmfh, in ascending stream order.

A topology is ``(nodes, ports)``: ``nodes`` a list of ``Node``; ``ports`` a
dict handle -> ``Port``.  Node inputs / outputs hold port handles or None.
"""
from __future__ import annotations

from dataclasses import dataclass, field

# DType.BytesFor (dtype/dtype.go:57-101): element sizes; Int4 and Bool packed.
_SIZE = {1: 8, 2: 4, 3: 2, 4: 2, 5: 1, 6: 1, 7: 8, 8: 4, 9: 2, 10: 1, 12: 8, 13: 4, 14: 2, 15: 1, 17: 8, 18: 16}
INT4, BOOL = 11, 16


def bytes_for(dtype: int, elements: int) -> int:
    if elements < 0:
        raise ValueError(f"dtype: negative element count {elements}")
    if dtype == INT4:
        return (elements + 1) // 2
    if dtype == BOOL:
        return (elements + 7) // 8
    if dtype not in _SIZE:
        raise ValueError(f"dtype: unsupported dtype {dtype}")
    return elements * _SIZE[dtype]


@dataclass
class Port:
    dtype: int
    dims: list  # ints (static) or str (symbols)
    id: int = 0


@dataclass
class Node:
    name: str
    inputs: list
    outputs: list
    id: int = 0
    stream: int = 0
    barriers: list = field(default_factory=list)  # (event_id, stream_id, wait)


def assign_port_ids(nodes, ports) -> None:
    seen, nxt = set(), 1
    for n in nodes:
        for h in n.outputs + n.inputs:
            if h is None or h in seen:
                continue
            seen.add(h)
            nxt = max(nxt, ports[h].id + 1)
    seen = set()
    for n in nodes:
        for h in n.outputs + n.inputs:
            if h is None or h in seen:
                continue
            seen.add(h)
            if ports[h].id == 0:
                ports[h].id = nxt
                nxt += 1


def port_byte_size(port: Port, bindings: dict) -> int:
    if not port.dims:
        return bytes_for(port.dtype, 1)
    count = 1
    for k, d in enumerate(port.dims):
        if isinstance(d, str):
            if d not in bindings:
                raise KeyError(f"dim[{k}] symbol {d!r} is unbound")
            count *= bindings[d]
        else:
            count *= d
    return bytes_for(port.dtype, count)


def analyze_liveness(nodes, ports, bindings=None):
    """[(port_id, start, end, size)] ordered by (start, port_id)."""
    bindings = bindings or {}
    iv = {}
    for step, n in enumerate(nodes):
        for h in n.outputs:
            if h is None or ports[h].id == 0 or ports[h].id in iv:
                continue
            iv[ports[h].id] = [ports[h].id, step, step, port_byte_size(ports[h], bindings)]
        for h in n.inputs:
            if h is None or ports[h].id == 0:
                continue
            pid = ports[h].id
            if pid not in iv:
                iv[pid] = [pid, 0, step, port_byte_size(ports[h], bindings)]
            elif step > iv[pid][2]:
                iv[pid][2] = step
    return sorted((tuple(v) for v in iv.values()), key=lambda v: (v[1], v[0]))


def align_up(v: int, align: int) -> int:
    return v if align <= 1 else (v + align - 1) // align * align


def lowest_free(size: int, live, align: int) -> int:
    candidate = 0
    blocks = sorted(live)
    while True:
        for off, sz in blocks:
            if candidate >= off + sz or candidate + size <= off:
                continue
            candidate = align_up(off + sz, align)
            break
        else:
            return candidate


def allocate_offsets(intervals, align: int = 64):
    """intervals: (port_id, start, end, size); returns (total, [(port_id,
    start, end, size, offset)]) in allocation order."""
    if align <= 0:
        align = 64
    work = sorted(intervals, key=lambda v: (v[1], v[0]))
    live, out, high = [], [], 0
    for pid, start, end, size in work:
        size = align_up(size, align)
        live = [b for b in live if b[2] >= start]
        off = lowest_free(size, [(b[0], b[1]) for b in live], align)
        live.append((off, size, end))
        out.append((pid, start, end, size, off))
        high = max(high, off + size)
    return (align_up(high, align) if out else 0), out


def schedule_streams(nodes, max_streams: int) -> None:
    if not nodes:
        return
    if max_streams < 1:
        max_streams = len(nodes)
    producer = {}
    for i, n in enumerate(nodes):
        for h in n.outputs:
            if h is not None and h not in producer:
                producer[h] = i
    last, nxt_stream, nxt_event = {}, 0, 1
    for index, node in enumerate(nodes):
        if node.id == 0:
            node.id = index + 1
        preds = {}
        for h in node.inputs:
            if h is None or h not in producer:
                continue
            p = nodes[producer[h]]
            if p.stream not in preds or p.id > preds[p.stream]:
                preds[p.stream] = p.id
        if not preds:
            if nxt_stream < max_streams:
                assigned, nxt_stream = nxt_stream, nxt_stream + 1
            else:
                assigned = 0
        elif len(preds) == 1:
            (only, pred), = preds.items()
            if last.get(only, 0) == pred:
                assigned = only
            elif nxt_stream < max_streams:
                assigned, nxt_stream = nxt_stream, nxt_stream + 1
            else:
                assigned = only
        else:
            assigned = min(preds)
        node.stream = assigned
        last[assigned] = node.id
        for s in sorted(preds):
            if s == assigned:
                continue
            e, nxt_event = nxt_event, nxt_event + 1
            node.barriers.append((e, s, True))
            prod = next(n for n in nodes if n.id == preds[s])
            prod.barriers.append((e, s, False))
