"""Graph layer of the mfh ABI (include/mfh_graph.h): ast.Graph, the optimizer's
ConstantFold / Fuse passes, codegen's AttachKernels with the HIP target and
CallGraph-style execution.

Names follow the reference's Go packages (ast/graph.go, optimizer/,
codegen/) so that tests written against this module read like the
reference's own tests.  Everything runs in libmfh.so; this module only moves
arguments across the C ABI.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

from . import abi
from .abi import AstNode, MFHError, check, lib

FUSE_OP = "optimizer.fusion"                 # optimizer/fuse.go:16
FUSE_ATTRIBUTE_AST = "fusion_ast"            # optimizer/fuse.go:22
CONSTANT_OP = "math.constant"                # optimizer/constant_fold.go:23
CONSTANT_ATTRIBUTE_VALUE = "value"           # optimizer/constant_fold.go:16
KERNEL_ATTRIBUTE = "compiled_kernel"         # codegen/codegen.go:28

TARGET_CPU, TARGET_METAL, TARGET_HIP = 0, 1, 2

# optimizer.NodeType (optimizer/fusion_ast.go:30-65)
NODE_NAMES = ["Invalid", "Input", "Constant", "Add", "Sub", "Mul", "Div", "Max", "Min", "Neg", "Abs",
              "Sqrt", "Exp", "Log", "ReLU", "Sigmoid", "Tanh", "Silu", "Gelu", "LeakyReLU"]
(NODE_INVALID, NODE_INPUT, NODE_CONSTANT, NODE_ADD, NODE_SUB, NODE_MUL, NODE_DIV, NODE_MAX, NODE_MIN,
 NODE_NEG, NODE_ABS, NODE_SQRT, NODE_EXP, NODE_LOG, NODE_RELU, NODE_SIGMOID, NODE_TANH, NODE_SILU,
 NODE_GELU, NODE_LEAKY_RELU) = range(20)

_ARITY = {NODE_INPUT: 0, NODE_CONSTANT: 0, **{t: 2 for t in range(NODE_ADD, NODE_NEG)},
          **{t: 1 for t in range(NODE_NEG, NODE_LEAKY_RELU + 1)}}

OPT_DISABLE_CONSTANT_FOLD = 1
OPT_DISABLE_FUSION = 4


def arity(node_type: int) -> int:
    """NodeType.Arity (optimizer/fusion_ast.go:168-180)."""
    return _ARITY.get(node_type, -1)


class _FusionInfo(ctypes.Structure):
    _fields_ = [("nodes", ctypes.POINTER(AstNode)), ("child_counts", ctypes.POINTER(ctypes.c_int32)),
                ("n_nodes", ctypes.c_int32), ("n_input_ports", ctypes.c_int32), ("n_contained", ctypes.c_int32),
                ("dtype", ctypes.c_uint8), ("reserved", ctypes.c_uint8 * 3),
                ("output_port", ctypes.c_char_p), ("count_expr", ctypes.c_char_p)]


class _FusionStats(ctypes.Structure):
    _fields_ = [("clusters", ctypes.c_int32), ("nodes_fused", ctypes.c_int32), ("nodes_removed", ctypes.c_int32)]


class Value(ctypes.Structure):
    """mfh_value: one device tensor crossing mfh_graph_call."""
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.c_void_p), ("dtype", ctypes.c_uint8),
                ("reserved", ctypes.c_uint8 * 7), ("count", ctypes.c_int64)]


_declared = False


def _L():
    global _declared
    L = lib()
    if not _declared:
        c = ctypes
        vp, i32, i64, u8, cp = c.c_void_p, c.c_int32, c.c_int64, c.c_uint8, c.c_char_p
        strs = c.POINTER(c.c_char_p)
        sig = {
            "mfh_graph_create": (c.c_int, [u8, c.POINTER(vp)]),
            "mfh_graph_release": (c.c_int, [vp]),
            "mfh_graph_add_input": (c.c_int, [vp, cp]),
            "mfh_graph_set_output": (c.c_int, [vp, cp, cp]),
            "mfh_graph_add_node": (c.c_int, [vp, cp, cp, strs, i32]),
            "mfh_graph_set_attribute": (c.c_int, [vp, i32, cp, c.c_double]),
            "mfh_graph_set_types": (c.c_int, [vp, i32, c.POINTER(u8), i32, u8]),
            "mfh_graph_set_fusion": (c.c_int, [vp, i32, c.POINTER(AstNode), c.POINTER(i32), i32, strs, i32, cp, u8]),
            "mfh_graph_num_nodes": (i32, [vp]),
            "mfh_graph_node_id": (cp, [vp, i32]),
            "mfh_graph_node_op": (cp, [vp, i32]),
            "mfh_graph_node_num_inputs": (i32, [vp, i32]),
            "mfh_graph_node_input": (cp, [vp, i32, i32]),
            "mfh_graph_node_attribute": (c.c_int, [vp, i32, cp, c.POINTER(c.c_double)]),
            "mfh_graph_node_attribute_key": (cp, [vp, i32, i32]),
            "mfh_graph_node_metadata": (c.c_int, [vp, i32, cp, c.POINTER(i64)]),
            "mfh_graph_node_types": (i32, [vp, i32, c.POINTER(u8), i32, c.POINTER(u8)]),
            "mfh_graph_fusion": (c.c_int, [vp, i32, c.POINTER(_FusionInfo)]),
            "mfh_graph_fusion_input_port": (cp, [vp, i32, i32]),
            "mfh_graph_fusion_contained_id": (cp, [vp, i32, i32]),
            "mfh_optimizer_is_elementwise_op": (i32, [cp]),
            "mfh_optimizer_elementwise_ops": (i32, [c.POINTER(c.c_char_p), i32]),
            "mfh_optimizer_constant_fold": (c.c_int, [vp, c.POINTER(i32)]),
            "mfh_optimizer_fuse": (c.c_int, [vp, c.POINTER(_FusionStats)]),
            "mfh_optimizer_run": (c.c_int, [vp, c.c_uint32, c.POINTER(i32), c.POINTER(_FusionStats)]),
            "mfh_codegen_attach_kernels": (c.c_int, [vp, c.POINTER(i32), i32, c.c_uint32, c.POINTER(i32)]),
            "mfh_graph_kernel": (c.c_int, [vp, i32, i32, c.POINTER(vp)]),
            "mfh_graph_call": (c.c_int, [vp, c.POINTER(Value), i32, c.POINTER(Value), i32, vp]),
            "mfh_graph_call_noalloc": (c.c_int, [vp, c.POINTER(Value), i32, c.POINTER(Value), i32, vp]),
            "mfh_graph_output_shape": (c.c_int, [vp, c.POINTER(Value), i32, cp, c.POINTER(u8), c.POINTER(i64)]),
            "mfh_graph_workspace_bytes": (i64, [vp]),
            "mfh_graph_set_replay": (c.c_int, [vp, i32]),
            "mfh_graph_replayed_calls": (i64, [vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _declared = True
    return L


def _s(b) -> str | None:
    return b.decode() if b is not None else None


def _strs(items):
    arr = (ctypes.c_char_p * max(1, len(items)))(*[x.encode() for x in items])
    return arr


# ---- FusionAST ----------------------------------------------------------------

@dataclass
class ASTNode:
    """optimizer.ASTNode (optimizer/fusion_ast.go:70-76)."""
    type: int
    children: list = field(default_factory=list)
    value: float = 0.0
    input_index: int = 0

    def preorder(self):
        yield self
        for c in self.children:
            yield from c.preorder()


@dataclass
class FusionAST:
    """optimizer.FusionAST (optimizer/fusion_ast.go:86-113)."""
    root: ASTNode
    input_ports: list
    output_port: str = ""
    count_expr: str = ""
    dtype: int = 0
    contained_node_ids: list = field(default_factory=list)


def _tree(nodes, counts, pos=0):
    n = nodes[pos]
    node = ASTNode(n.type, [], n.value, n.input_index)
    pos += 1
    for _ in range(counts[pos - 1]):
        child, pos = _tree(nodes, counts, pos)
        node.children.append(child)
    return node, pos


# ---- kernels ------------------------------------------------------------------

class HIPKernel:
    """The TargetHIP kernel of a fused node; owned by its graph."""

    def __init__(self, graph, handle):
        self._graph = graph  # keeps the graph (and the kernel) alive
        self._h = handle

    def target(self) -> int:
        return TARGET_HIP

    def source(self) -> str:
        return lib().mfh_fusion_source(self._h).decode()

    def kernel_name(self) -> str:
        return lib().mfh_fusion_kernel_name(self._h).decode()

    def num_inputs(self) -> int:
        return lib().mfh_fusion_num_inputs(self._h)

    def run(self, inputs, out: int, count: int, stream: int = 0) -> None:
        ptrs = (ctypes.c_void_p * max(1, len(inputs)))(*inputs)
        check(lib().mfh_fusion_launch(self._h, ptrs, len(inputs), out, count, stream))


class KernelSet:
    """codegen.KernelSet (codegen/attach.go:14-58) read from a node."""

    def __init__(self, graph, index):
        self._graph, self._index = graph, index

    def For(self, target: int):  # noqa: N802  (the reference's method name)
        h = ctypes.c_void_p()
        check(_L().mfh_graph_kernel(self._graph._h, self._index, target, ctypes.byref(h)))
        return HIPKernel(self._graph, h) if h.value else None

    def targets(self):
        return [t for t in (TARGET_CPU, TARGET_METAL, TARGET_HIP) if self.For(t) is not None]


# ---- ast.Graph -------------------------------------------------------------------

@dataclass
class GraphNode:
    """ast.GraphNode (ast/graph.go:31-45) as given to or read from a graph.

    ``attributes`` holds float attributes (the "value" of a math.constant
    node) and, when read back, ``FUSE_ATTRIBUTE_AST`` -> FusionAST and
    ``KERNEL_ATTRIBUTE`` -> KernelSet.  ``input_types`` / ``output_type`` are
    the dtypes of InputTypes / OutputType.
    """
    id: str
    op: str
    inputs: list = field(default_factory=list)
    attributes: dict = field(default_factory=dict)
    metadata: dict = field(default_factory=dict)
    input_types: list = field(default_factory=list)
    output_type: int = 0


class Graph:
    """ast.Graph held by libmfh (nodes, inputs, outputs, ExecutionDType)."""

    def __init__(self, inputs=(), outputs=None, nodes=(), execution_dtype: int = 0):
        h = ctypes.c_void_p()
        check(_L().mfh_graph_create(execution_dtype, ctypes.byref(h)))
        self._h = h
        for name in inputs:
            check(_L().mfh_graph_add_input(self._h, name.encode()))
        for key, value in (outputs or {}).items():
            check(_L().mfh_graph_set_output(self._h, key.encode(), value.encode()))
        for node in nodes:
            self.add_node(node)

    def add_node(self, node: GraphNode) -> int:
        L = _L()
        check(L.mfh_graph_add_node(self._h, node.id.encode(), node.op.encode(), _strs(node.inputs),
                                   len(node.inputs)))
        index = L.mfh_graph_num_nodes(self._h) - 1
        for key, value in node.attributes.items():
            if key == FUSE_ATTRIBUTE_AST:
                self._set_fusion(index, value)
            elif isinstance(value, (int, float)):
                check(L.mfh_graph_set_attribute(self._h, index, key.encode(), float(value)))
        if node.input_types or node.output_type:
            types = (ctypes.c_uint8 * max(1, len(node.input_types)))(*node.input_types)
            check(L.mfh_graph_set_types(self._h, index, types, len(node.input_types), node.output_type))
        return index

    def _set_fusion(self, index: int, fusion: FusionAST) -> None:
        flat = list(fusion.root.preorder()) if fusion.root is not None else []
        nodes = (AstNode * max(1, len(flat)))(*[AstNode(n.type, n.input_index, n.value) for n in flat])
        counts = (ctypes.c_int32 * max(1, len(flat)))(*[len(n.children) for n in flat])
        check(_L().mfh_graph_set_fusion(self._h, index, nodes, counts, len(flat), _strs(fusion.input_ports),
                                        len(fusion.input_ports), fusion.output_port.encode(), fusion.dtype))

    def _node(self, i: int) -> GraphNode:
        L, h = _L(), self._h
        node = GraphNode(_s(L.mfh_graph_node_id(h, i)), _s(L.mfh_graph_node_op(h, i)),
                         [_s(L.mfh_graph_node_input(h, i, k)) for k in range(L.mfh_graph_node_num_inputs(h, i))])
        k = 0
        while (key := L.mfh_graph_node_attribute_key(h, i, k)) is not None:
            v = ctypes.c_double()
            check(L.mfh_graph_node_attribute(h, i, key, ctypes.byref(v)))
            node.attributes[key.decode()] = v.value
            k += 1
        m = ctypes.c_int64()
        if L.mfh_graph_node_metadata(h, i, b"fused_node_count", ctypes.byref(m)) == 0:
            node.metadata["fused_node_count"] = m.value
        info = _FusionInfo()
        if L.mfh_graph_fusion(h, i, ctypes.byref(info)) == 0:
            root, _ = _tree(info.nodes, info.child_counts)
            node.attributes[FUSE_ATTRIBUTE_AST] = FusionAST(
                root, [_s(L.mfh_graph_fusion_input_port(h, i, k)) for k in range(info.n_input_ports)],
                _s(info.output_port), _s(info.count_expr), info.dtype,
                [_s(L.mfh_graph_fusion_contained_id(h, i, k)) for k in range(info.n_contained)])
        ks = KernelSet(self, i)
        if any(ks.For(t) is not None for t in (TARGET_CPU, TARGET_METAL, TARGET_HIP)):
            node.attributes[KERNEL_ATTRIBUTE] = ks
        cap = 64
        types = (ctypes.c_uint8 * cap)()
        out_t = ctypes.c_uint8()
        n = L.mfh_graph_node_types(h, i, types, cap, ctypes.byref(out_t))
        node.input_types = list(types[:min(n, cap)])
        node.output_type = out_t.value
        return node

    @property
    def nodes(self):
        return [self._node(i) for i in range(_L().mfh_graph_num_nodes(self._h))]

    def workspace_bytes(self) -> int:
        return _L().mfh_graph_workspace_bytes(self._h)

    def set_replay(self, enabled: bool) -> None:
        """Replays of calls with one plan (names, dtypes, counts, aliasing) as
        one captured HIP graph, rebound to each call's buffers (on by
        default)."""
        check(_L().mfh_graph_set_replay(self._h, int(enabled)))

    def replayed_calls(self) -> int:
        return _L().mfh_graph_replayed_calls(self._h)

    def call(self, inputs: dict, outputs: dict, stream: int = 0) -> None:
        """runtime.Backend.CallGraph on the device: `inputs` maps input names
        and `outputs` output keys to (device pointer, dtype, count) triples or
        to torch tensors."""
        ins, outs = self._values(inputs), self._values(outputs)
        check(_L().mfh_graph_call(self._h, ins, len(inputs), outs, len(outputs), stream))

    def output_shape(self, inputs: dict, key: str) -> tuple:
        """(dtype, count) that a call with `inputs` gives output `key`; only
        the inputs' dtypes and counts are read, (ptr, dtype, count) triples
        with ptr None included."""
        ins = self._values(inputs)
        dt, n = ctypes.c_uint8(), ctypes.c_int64()
        check(_L().mfh_graph_output_shape(self._h, ins, len(inputs), key.encode(), ctypes.byref(dt), ctypes.byref(n)))
        return dt.value, n.value

    def call_noalloc(self, inputs: dict, outputs: dict, stream: int = 0) -> None:
        """mfh_graph_call_noalloc: the same call with its constants and
        intermediates in the library's static device scratch, nothing
        allocated, compiled or loaded (an earlier `call` with the same value
        dtypes and operand modes loads the kernels)."""
        ins, outs = self._values(inputs), self._values(outputs)
        check(_L().mfh_graph_call_noalloc(self._h, ins, len(inputs), outs, len(outputs), stream))

    @staticmethod
    def _values(mapping):
        arr = (Value * max(1, len(mapping)))()
        keep = []
        for k, (name, v) in enumerate(mapping.items()):
            if hasattr(v, "data_ptr"):
                v = (v.data_ptr(), _torch_dtype(v), v.numel())
            ptr, dt, count = v
            b = name.encode()
            keep.append(b)
            arr[k].name, arr[k].data, arr[k].dtype, arr[k].count = b, ptr, dt, count
        arr._keep = keep
        return arr

    def close(self) -> None:
        if getattr(self, "_h", None):
            _L().mfh_graph_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _torch_dtype(t) -> int:
    import torch
    return {torch.float32: abi.FLOAT32, torch.float16: abi.FLOAT16, torch.bfloat16: abi.BFLOAT16}.get(t.dtype, 0)


# ---- optimizer -------------------------------------------------------------------

@dataclass
class FusionStats:
    clusters: int = 0
    nodes_fused: int = 0
    nodes_removed: int = 0


@dataclass
class ConstantFoldStats:
    nodes_folded: int = 0


@dataclass
class Stats:
    constant_fold: ConstantFoldStats
    fusion: FusionStats


def is_elementwise_op(op: str):
    """isElementwiseOp (optimizer/elementwise.go:44-54): (NodeType, eligible)."""
    t = _L().mfh_optimizer_is_elementwise_op(op.encode())
    return t, t != NODE_INVALID


def elementwise_ops():
    """ElementwiseOps (optimizer/elementwise.go:61-74)."""
    L = _L()
    n = L.mfh_optimizer_elementwise_ops(None, 0)
    arr = (ctypes.c_char_p * n)()
    L.mfh_optimizer_elementwise_ops(arr, n)
    return [s.decode() for s in arr]


def _stats(st: _FusionStats) -> FusionStats:
    return FusionStats(st.clusters, st.nodes_fused, st.nodes_removed)


def fuse(graph: Graph) -> FusionStats:
    """Fuse (optimizer/fuse.go:54-159)."""
    st = _FusionStats()
    check(_L().mfh_optimizer_fuse(graph._h, ctypes.byref(st)))
    return _stats(st)


def constant_fold(graph: Graph) -> ConstantFoldStats:
    """ConstantFold (optimizer/constant_fold.go:40-109)."""
    n = ctypes.c_int32()
    check(_L().mfh_optimizer_constant_fold(graph._h, ctypes.byref(n)))
    return ConstantFoldStats(n.value)


def run(graph: Graph, disable_constant_fold: bool = False, disable_fusion: bool = False) -> Stats:
    """optimizer.Run (optimizer/run.go:56-113) over ConstantFold and Fuse."""
    opts = (OPT_DISABLE_CONSTANT_FOLD if disable_constant_fold else 0) | (OPT_DISABLE_FUSION if disable_fusion else 0)
    n, st = ctypes.c_int32(), _FusionStats()
    check(_L().mfh_optimizer_run(graph._h, opts, ctypes.byref(n), ctypes.byref(st)))
    return Stats(ConstantFoldStats(n.value), _stats(st))


# ---- codegen ---------------------------------------------------------------------

def attach_kernels(graph: Graph, targets=None, flags: int = 0) -> int:
    """AttachKernels (codegen/attach.go:67-113); default targets {TargetHIP}."""
    targets = list(targets or [])
    arr = (ctypes.c_int32 * max(1, len(targets)))(*targets)
    n = ctypes.c_int32()
    rc = _L().mfh_codegen_attach_kernels(graph._h, arr, len(targets), flags, ctypes.byref(n))
    if rc != 0:
        err = MFHError(rc, abi.last_error())
        err.attached = n.value
        raise err
    return n.value
