"""Workspace planning and stream scheduling of the mfh ABI (include/mfh_plan.h).

Mirrors the reference's planning IR: ir.Topology / ir.Node / ir.Port,
ir.PlanWorkspace (ir/planner.go), ir.ScheduleStreams (ir/stream_scheduler.go)
and compiler.PlanGraph (compiler/plan.go).  Ports and nodes are built through
handles; planner and scheduler output is read back per port and node.  All of
it runs in libmfh.so on the host.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from .abi import check, lib


class Interval(ctypes.Structure):
    """ir.Interval: a port's live range over node steps and its placement."""
    _fields_ = [("port_id", ctypes.c_int32), ("start", ctypes.c_int32), ("end", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("size", ctypes.c_int64), ("offset", ctypes.c_int64)]

    def astuple(self):
        return (self.port_id, self.start, self.end, self.size, self.offset)


class _SyncEvent(ctypes.Structure):
    _fields_ = [("event_id", ctypes.c_int32), ("stream_id", ctypes.c_int32), ("wait", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


@dataclass(frozen=True)
class SyncEvent:
    """ir.SyncEvent (ir/sync_event.go)."""
    event_id: int
    stream_id: int
    wait: bool


_declared = False


def _L():
    global _declared
    L = lib()
    if not _declared:
        c = ctypes
        vp, i32, i64, u8, cp = c.c_void_p, c.c_int32, c.c_int64, c.c_uint8, c.c_char_p
        sig = {
            "mfh_topology_create": (c.c_int, [c.POINTER(vp)]),
            "mfh_topology_release": (c.c_int, [vp]),
            "mfh_topology_add_port": (c.c_int, [vp, u8, c.POINTER(i64), c.POINTER(cp), i32, i32, c.POINTER(i32)]),
            "mfh_topology_add_node": (c.c_int, [vp, cp, c.POINTER(i32), i32, c.POINTER(i32), i32, c.POINTER(i32)]),
            "mfh_topology_bind": (c.c_int, [vp, cp, i64]),
            "mfh_topology_num_nodes": (i32, [vp]),
            "mfh_topology_num_ports": (i32, [vp]),
            "mfh_topology_assign_port_ids": (c.c_int, [vp]),
            "mfh_topology_port_id": (i32, [vp, i32]),
            "mfh_topology_liveness": (c.c_int, [vp, c.POINTER(Interval), i32, c.POINTER(i32)]),
            "mfh_allocate_offsets": (c.c_int, [c.POINTER(Interval), i32, i64, c.POINTER(i64)]),
            "mfh_topology_plan_workspace": (c.c_int, [vp, i64]),
            "mfh_topology_plan_stream_workspace": (c.c_int, [vp, i64]),
            "mfh_topology_workspace": (c.c_int, [vp, c.POINTER(i64), c.POINTER(i64), c.POINTER(i32)]),
            "mfh_topology_allocation": (c.c_int, [vp, i32, c.POINTER(Interval)]),
            "mfh_topology_port_offset": (c.c_int, [vp, i32, c.POINTER(i64)]),
            "mfh_topology_schedule_streams": (c.c_int, [vp, i32]),
            "mfh_topology_node_name": (cp, [vp, i32]),
            "mfh_topology_node_id": (i32, [vp, i32]),
            "mfh_topology_node_stream": (i32, [vp, i32]),
            "mfh_topology_node_barriers": (i32, [vp, i32, c.POINTER(_SyncEvent), i32]),
            "mfh_topology_node_ports": (i32, [vp, i32, i32, c.POINTER(i32), i32]),
            "mfh_topology_io_offset": (c.c_int, [vp, cp, i32, c.POINTER(i64)]),
            "mfh_graph_plan": (c.c_int, [vp, vp, i32, i64, i32, c.POINTER(vp)]),
            "mfh_graph_set_max_streams": (c.c_int, [vp, i32]),
            "mfh_graph_streams_used": (i32, [vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _declared = True
    return L


@dataclass(frozen=True)
class Dim:
    """ir.Dimension: a static size, or a symbol bound at planning time."""
    static: int = 0
    symbol: str = ""


def allocate_offsets(intervals, align: int = 64):
    """ir.AllocateOffsets: `intervals` are (port_id, start, end, size)
    tuples; returns (total, [(port_id, start, end, size, offset), ...]) in
    allocation order."""
    arr = (Interval * max(1, len(intervals)))()
    for k, (pid, start, end, size) in enumerate(intervals):
        arr[k].port_id, arr[k].start, arr[k].end, arr[k].size = pid, start, end, size
    total = ctypes.c_int64()
    check(_L().mfh_allocate_offsets(arr, len(intervals), align, ctypes.byref(total)))
    return total.value, [arr[k].astuple() for k in range(len(intervals))]


class Topology:
    """ir.Topology built port by port and node by node."""

    def __init__(self, handle=None):
        if handle is None:
            handle = ctypes.c_void_p()
            check(_L().mfh_topology_create(ctypes.byref(handle)))
        self._h = handle

    def port(self, dtype: int, *dims, id: int = 0) -> int:
        """A port whose shape is `dims` (ints, or strings naming symbols, or
        Dim); returns its handle."""
        n = len(dims)
        sizes = (ctypes.c_int64 * max(1, n))()
        syms = (ctypes.c_char_p * max(1, n))()
        for k, d in enumerate(dims):
            if isinstance(d, Dim):
                d = d.symbol or d.static
            if isinstance(d, str):
                syms[k] = d.encode()
            else:
                sizes[k] = d
        h = ctypes.c_int32()
        check(_L().mfh_topology_add_port(self._h, dtype, sizes, syms, n, id, ctypes.byref(h)))
        return h.value

    def node(self, name: str, inputs=(), outputs=()) -> int:
        """A node reading `inputs` and writing `outputs` (port handles; None
        is a nil port); returns its index."""
        ins = [-1 if p is None else p for p in inputs]
        outs = [-1 if p is None else p for p in outputs]
        a = (ctypes.c_int32 * max(1, len(ins)))(*ins)
        b = (ctypes.c_int32 * max(1, len(outs)))(*outs)
        h = ctypes.c_int32()
        check(_L().mfh_topology_add_node(self._h, name.encode(), a, len(ins), b, len(outs), ctypes.byref(h)))
        return h.value

    def bind(self, symbol: str, value: int) -> None:
        check(_L().mfh_topology_bind(self._h, symbol.encode(), value))

    @property
    def num_nodes(self) -> int:
        return _L().mfh_topology_num_nodes(self._h)

    def assign_port_ids(self) -> None:
        check(_L().mfh_topology_assign_port_ids(self._h))

    def port_id(self, port: int) -> int:
        return _L().mfh_topology_port_id(self._h, port)

    def liveness(self):
        """AnalyzeLiveness: [(port_id, start, end, size, 0), ...]."""
        n = ctypes.c_int32()
        check(_L().mfh_topology_liveness(self._h, None, 0, ctypes.byref(n)))
        arr = (Interval * max(1, n.value))()
        check(_L().mfh_topology_liveness(self._h, arr, n.value, ctypes.byref(n)))
        return [arr[k].astuple() for k in range(n.value)]

    def plan_workspace(self, align: int = 64) -> None:
        check(_L().mfh_topology_plan_workspace(self._h, align))

    def plan_stream_workspace(self, align: int = 64) -> None:
        check(_L().mfh_topology_plan_stream_workspace(self._h, align))

    def workspace(self):
        """(Size, Align, [allocation tuples])."""
        size, align, n = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
        check(_L().mfh_topology_workspace(self._h, ctypes.byref(size), ctypes.byref(align), ctypes.byref(n)))
        out = []
        for k in range(n.value):
            iv = Interval()
            check(_L().mfh_topology_allocation(self._h, k, ctypes.byref(iv)))
            out.append(iv.astuple())
        return size.value, align.value, out

    def port_offset(self, port: int) -> int | None:
        off = ctypes.c_int64()
        if _L().mfh_topology_port_offset(self._h, port, ctypes.byref(off)) != 0:
            return None
        return off.value

    def schedule_streams(self, max_streams: int = 0) -> None:
        check(_L().mfh_topology_schedule_streams(self._h, max_streams))

    def node_name(self, node: int) -> str:
        return _L().mfh_topology_node_name(self._h, node).decode()

    def node_id(self, node: int) -> int:
        return _L().mfh_topology_node_id(self._h, node)

    def stream(self, node: int) -> int:
        return _L().mfh_topology_node_stream(self._h, node)

    def barriers(self, node: int):
        L = _L()
        n = L.mfh_topology_node_barriers(self._h, node, None, 0)
        arr = (_SyncEvent * max(1, n))()
        L.mfh_topology_node_barriers(self._h, node, arr, n)
        return [SyncEvent(arr[k].event_id, arr[k].stream_id, bool(arr[k].wait)) for k in range(n)]

    def node_ports(self, node: int, outputs: bool):
        L = _L()
        n = L.mfh_topology_node_ports(self._h, node, int(outputs), None, 0)
        arr = (ctypes.c_int32 * max(1, n))()
        L.mfh_topology_node_ports(self._h, node, int(outputs), arr, n)
        return list(arr[:n])

    def io_offset(self, name: str, output: bool) -> int:
        off = ctypes.c_int64()
        check(_L().mfh_topology_io_offset(self._h, name.encode(), int(output), ctypes.byref(off)))
        return off.value

    def close(self) -> None:
        if getattr(self, "_h", None):
            _L().mfh_topology_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def plan_graph(graph, inputs: dict, align: int = 64, max_streams: int = 1) -> Topology:
    """compiler.PlanGraph for a manifesto_amd.graph.Graph; `inputs` maps
    input names to (dtype, count) pairs or tensors (shapes only)."""
    vals = {}
    for name, v in inputs.items():
        if hasattr(v, "data_ptr"):
            vals[name] = v
        else:
            dt, count = v
            vals[name] = (None, dt, count)
    arr = graph._values(vals)
    h = ctypes.c_void_p()
    check(_L().mfh_graph_plan(graph._h, ctypes.cast(arr, ctypes.c_void_p), len(vals), align, max_streams,
                              ctypes.byref(h)))
    return Topology(h)


def set_max_streams(graph, max_streams: int) -> None:
    """The MaxStreams a graph's calls schedule with (1: the caller's stream)."""
    check(_L().mfh_graph_set_max_streams(graph._h, max_streams))


def streams_used(graph) -> int:
    return _L().mfh_graph_streams_used(graph._h)
