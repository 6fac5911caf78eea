/*
 * mfh_graph.h — C ABI of the compile-and-dispatch layer around the HIP
 * codegen target: the manifest compute graph (ast.Graph), the optimizer
 * passes that produce FusionASTs from it (ConstantFold, Fuse), the codegen
 * attach step that lowers every fused node for gfx950 (AttachKernels with a
 * HIP target), and CallGraph-style execution of the result on the device.
 *
 * It mirrors the reference's Go interfaces for a host that is not Go; a Go
 * host keeps its own optimizer and binds only mfh_fusion_* (mfh.h).
 * Strings passed in are copied; strings returned live until the graph is
 * modified or released.  A graph is not thread-safe: calls on one graph,
 * mfh_graph_call included, must not overlap.
 */
#ifndef MFH_GRAPH_H
#define MFH_GRAPH_H

#include "mfh.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mfh_graph mfh_graph;

/* ---- ast.Graph (ast/graph.go:15-45) --------------------------------------- */

/* Empty graph; `execution_dtype` is Graph.ExecutionDType (0 = Invalid). */
int mfh_graph_create(uint8_t execution_dtype, mfh_graph** graph);
int mfh_graph_release(mfh_graph* graph);

/* Graph.Inputs: a name bound by the caller at mfh_graph_call. */
int mfh_graph_add_input(mfh_graph* graph, const char* name);

/* Graph.Outputs[key] = value (a node ID or an input name).  A key set twice
 * keeps the last value, as a Go map assignment does. */
int mfh_graph_set_output(mfh_graph* graph, const char* key, const char* value);

/* Appends GraphNode{ID: id, Op: op, Inputs: inputs}. */
int mfh_graph_add_node(mfh_graph* graph, const char* id, const char* op, const char* const* inputs,
                       int32_t n_inputs);

/* GraphNode.Attributes[key] = value (float64), e.g. the "value" of a
 * math.constant node (optimizer/constant_fold.go:16). */
int mfh_graph_set_attribute(mfh_graph* graph, int32_t node, const char* key, double value);

/* GraphNode.InputTypes[k].DType and OutputType.DType (ast/graph.go:38-45);
 * 0 (Invalid) where the typer left a port untyped. */
int mfh_graph_set_types(mfh_graph* graph, int32_t node, const uint8_t* input_types, int32_t n_input_types,
                        uint8_t output_type);

/* Stores a FusionAST under Attributes["fusion_ast"] (optimizer/fuse.go:27),
 * as a caller that builds a FuseOp node by hand does (codegen/codegen_test.go:
 * 163-188).  `nodes` is the pre-order tree; child_counts[i] is the number of
 * children of nodes[i] (NULL: NodeType.Arity of each node). */
int mfh_graph_set_fusion(mfh_graph* graph, int32_t node, const mfh_ast_node* nodes, const int32_t* child_counts,
                         int32_t n_nodes, const char* const* input_ports, int32_t n_input_ports,
                         const char* output_port, uint8_t dtype);

/* ---- reading a graph back ------------------------------------------------- */

int32_t mfh_graph_num_nodes(const mfh_graph* graph);
const char* mfh_graph_node_id(const mfh_graph* graph, int32_t node);
const char* mfh_graph_node_op(const mfh_graph* graph, int32_t node);
int32_t mfh_graph_node_num_inputs(const mfh_graph* graph, int32_t node);
const char* mfh_graph_node_input(const mfh_graph* graph, int32_t node, int32_t slot);

/* MFH_OK and *value when the attribute / metadata entry is present,
 * MFH_ERR_INVALID_ARGUMENT when it is not. */
int mfh_graph_node_attribute(const mfh_graph* graph, int32_t node, const char* key, double* value);
/* The k-th numeric attribute key of a node (sorted), NULL past the end. */
const char* mfh_graph_node_attribute_key(const mfh_graph* graph, int32_t node, int32_t k);
int mfh_graph_node_metadata(const mfh_graph* graph, int32_t node, const char* key, int64_t* value);

/* Number of InputTypes; copies up to `cap` of them and the OutputType. */
int32_t mfh_graph_node_types(const mfh_graph* graph, int32_t node, uint8_t* input_types, int32_t cap,
                             uint8_t* output_type);

/* The FusionAST of a fused node (optimizer/fusion_ast.go:86-113).  `nodes`
 * and `child_counts` describe the tree in pre-order. */
typedef struct {
    const mfh_ast_node* nodes;
    const int32_t* child_counts;
    int32_t n_nodes;
    int32_t n_input_ports;
    int32_t n_contained;
    uint8_t dtype;
    uint8_t reserved[3];
    const char* output_port;
    const char* count_expr;
} mfh_fusion_info;

/* MFH_ERR_INVALID_ARGUMENT when the node holds no FusionAST. */
int mfh_graph_fusion(const mfh_graph* graph, int32_t node, mfh_fusion_info* info);
const char* mfh_graph_fusion_input_port(const mfh_graph* graph, int32_t node, int32_t k);
/* ContainedNodeIDs in graph order (the reference leaves their order to Go's
 * map iteration, optimizer/fuse.go:293-301). */
const char* mfh_graph_fusion_contained_id(const mfh_graph* graph, int32_t node, int32_t k);

/* ---- optimizer: elementwise table (optimizer/elementwise.go:15-74) -------- */

/* isElementwiseOp: the NodeType an op string fuses as (trimmed, lower-case),
 * 0 when the op is not fusion-eligible. */
int32_t mfh_optimizer_is_elementwise_op(const char* op);

/* ElementwiseOps: the eligible op strings.  Returns their number and stores
 * up to `cap` static strings in `ops` (in table order). */
int32_t mfh_optimizer_elementwise_ops(const char** ops, int32_t cap);

/* ---- optimizer passes ----------------------------------------------------- */

typedef struct {
    int32_t clusters;
    int32_t nodes_fused;
    int32_t nodes_removed;
} mfh_fusion_stats; /* FusionStats, optimizer/fuse.go:32-36 */

/* ConstantFold (optimizer/constant_fold.go:40-109). */
int mfh_optimizer_constant_fold(mfh_graph* graph, int32_t* nodes_folded);

/* Fuse (optimizer/fuse.go:54-159). */
int mfh_optimizer_fuse(mfh_graph* graph, mfh_fusion_stats* stats);

/* Run (optimizer/run.go:56-113) restricted to the passes this library
 * implements: ConstantFold then Fuse.  Options bits disable a pass. */
#define MFH_OPT_DISABLE_CONSTANT_FOLD 1u
#define MFH_OPT_DISABLE_FUSION 4u
int mfh_optimizer_run(mfh_graph* graph, uint32_t options, int32_t* nodes_folded, mfh_fusion_stats* stats);

/* ---- codegen attach (codegen/codegen.go:34-99, codegen/attach.go) --------- */

/* codegen.Target values; TargetHIP follows TargetMetal. */
#define MFH_TARGET_CPU 0
#define MFH_TARGET_METAL 1
#define MFH_TARGET_HIP 2

/* AttachKernels: for every FuseOp node, EmitFusion for `targets` (NULL or
 * empty: {TargetHIP}) and store the KernelSet under
 * Attributes["compiled_kernel"].  TargetCPU and TargetMetal have no emitter
 * in this library and, like an unknown target in EmitFusion's switch, yield
 * no kernel.  `flags` are mfh_fusion_compile's (MFH_FUSION_PRECISE); the
 * graph keeps them for the one-node kernels of unfused elementwise nodes. */
int mfh_codegen_attach_kernels(mfh_graph* graph, const int32_t* targets, int32_t n_targets, uint32_t flags,
                               int32_t* attached);

/* KernelSet.For(target) of a node: its compiled HIP kernel for full-length
 * operands of the declared dtypes (usable with mfh_fusion_source /
 * kernel_name / launch), or *kernel = NULL when the node has none.  Owned by
 * the graph. */
int mfh_graph_kernel(const mfh_graph* graph, int32_t node, int32_t target, const mfh_kernel** kernel);

/* ---- execution (runtime.Backend.CallGraph, runtime/executor.go:22-27) ----- */

/* One device tensor crossing the call: a flat buffer of `count` elements of
 * `dtype` (Float32, Float16 or BFloat16). */
typedef struct {
    const char* name; /* graph input name, or graph output key */
    void* data;
    uint8_t dtype;
    uint8_t reserved[7];
    int64_t count;
} mfh_value;

/* Runs the graph's nodes in order on `stream`:
 *   - FuseOp nodes through their KernelSet's HIP kernel,
 *   - elementwise nodes left unfused as one-node kernels,
 *   - math.constant nodes as scalar operands fl32(value).
 * An operand of `count` elements in a node of n elements is read in full
 * (count == n), as a scalar (count == 1) or as a repeating row (n % count ==
 * 0); anything else is MFH_ERR_SHAPE_MISMATCH.  A node's output has the
 * node's OutputType, else the graph's ExecutionDType, else Float32.
 * Intermediates live in one device workspace per graph, laid out by value
 * lifetime and kept across calls.  Every bound output receives its value; an
 * output with no binding is computed and dropped.  An output may share its
 * buffer with an input (an update in place): it is written in place when the
 * input is the same buffer with the same element size and count and only
 * the launch that computes the output reads that input; otherwise it is
 * computed in the workspace and copied out after the last launch, so every
 * launch reads the input as it was.  Outputs of different values must not
 * share or overlap buffers.  Calls on one graph must
 * not overlap in host threads (they share its workspace, streams and replay
 * cache); different graphs may be called from different threads.  Work
 * queued on different caller streams is ordered by the graph itself. */
int mfh_graph_call(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs,
                   int32_t n_outputs, void* stream);

/* The dtype and element count that mfh_graph_call with these inputs gives
 * output `key` (a key of Graph.Outputs), so that a caller can allocate the
 * outputs before the call.  Only the inputs' names, dtypes and counts are
 * read (data may be NULL); nothing is compiled, allocated or queued, and no
 * device is needed.  The same errors as mfh_graph_call for the same
 * bindings.  No counterpart in the reference, whose CallGraph returns
 * outputs it allocates itself (runtime/executor.go:70-72); the backend-level
 * call, mfh_backend_graph_call (mfh_backend.h), uses it to do the same. */
int mfh_graph_output_shape(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, const char* key,
                           uint8_t* dtype, int64_t* count);

/* Bytes of the graph's device workspace (0 before the first call). */
int64_t mfh_graph_workspace_bytes(const mfh_graph* graph);

/* Bytes of the per-device static scratch of mfh_graph_call_noalloc. */
#define MFH_GRAPH_SCRATCH_BYTES (64u << 20)

/* mfh_graph_call without allocating anything on the device.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same bindings, results and errors as mfh_graph_call, except:
 *   - the call's constants and intermediates live in one static device
 *     scratch array of MFH_GRAPH_SCRATCH_BYTES per GPU (held from mfh_init
 *     until the process ends); a call that needs more fails with
 *     MFH_ERR_INVALID_ARGUMENT before anything is queued;
 *   - everything runs as plain kernel launches (and device-to-device copies
 *     for outputs not written in place) on `stream`: no auxiliary streams,
 *     events, replay capture, host-to-device copies or memsets;
 *   - it compiles and loads no kernel: each one the call needs must have been
 *     loaded by an earlier mfh_graph_call with the same value dtypes and the
 *     same operand modes (full, scalar, repeating row of the same length),
 *     else MFH_ERR_INVALID_ARGUMENT;
 *   - every call on one GPU, whatever its graph, uses that GPU's one scratch
 *     array and leaves its contents there.  Nothing in it needs to start at
 *     zero (each call writes its constants, and every intermediate is written
 *     before it is read), but calls that overlap on one GPU (different
 *     streams, or threads, without ordering between them) race. */
int mfh_graph_call_noalloc(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs,
                           int32_t n_outputs, void* stream);

/* Launch replay (no counterpart in the reference, whose CallGraph dispatches
 * node by node): calls with the same plan (value names, dtypes, counts,
 * which output bindings share a buffer or overlap an input, stream budget)
 * share one HIP graph.  The plan's first call runs as plain launches, its
 * second is captured, and every later call launches the captured graph with
 * one hipGraphLaunch, whatever its buffers: the launches and output copies
 * whose buffers differ from the ones the graph was last bound to get their
 * arguments updated in place first.  Two executables per plan take turns,
 * so that one still running is never updated (a call may wait for the call
 * before last).  A plan that runs on several streams is not rebound: its
 * calls replay only on buffers an executable already holds and otherwise run
 * as plain launches.  Up to 8 plans are kept per graph (least recently used
 * dropped); any change to the graph drops them.  A call made on a stream
 * that is itself being captured runs as plain launches into that capture.
 * Enabled by default; mfh_graph_set_replay(graph, 0) turns it off.
 * mfh_graph_replayed_calls counts the calls that ran as replays. */
int mfh_graph_set_replay(mfh_graph* graph, int32_t enabled);
int64_t mfh_graph_replayed_calls(const mfh_graph* graph);

#ifdef __cplusplus
}
#endif
#endif /* MFH_GRAPH_H */
