/* mfh_plan.h — static workspace planning and stream scheduling for graphs run
 * on the HIP backend.
 *
 * Restates the reference's planning IR for the elementwise path:
 *   - ir.Topology / ir.Node / ir.Port (ir/topology.go, ir/node.go, ir/port.go)
 *     as an opaque mfh_topology built port by port and node by node;
 *   - ir.AssignPortIDs, ir.AnalyzeLiveness, ir.AllocateOffsets and
 *     ir.PlanWorkspace (ir/planner.go:43-513);
 *   - ir.ScheduleStreams (ir/stream_scheduler.go:56-297) with its SyncEvents
 *     (ir/sync_event.go);
 *   - compiler.PlanGraph (compiler/plan.go:29-290) for an mfh_graph.
 * The graph executor (mfh_graph_call) runs on the same scheduler: StreamID k
 * becomes a HIP stream (0 = the caller's), a SyncEvent becomes a HIP event
 * recorded after its producer and waited on before its consumer.
 *
 * All functions here are host-only and need no device, except that
 * mfh_graph_plan compiles the HIP kernels of unfused nodes (hiprtc) as a
 * graph call would.
 */
#ifndef MFH_PLAN_H
#define MFH_PLAN_H

#include <stddef.h>
#include <stdint.h>

#include "mfh.h"
#include "mfh_graph.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mfh_topology mfh_topology;

int mfh_topology_create(mfh_topology** topology);
int mfh_topology_release(mfh_topology* topology);

/* An ir.Port whose PortType has `dtype` and `rank` dimensions: dimension k is
 * static dims[k], or symbolic when `symbols` and symbols[k] are non-NULL
 * (ir.Dimension.IsSymbolic, ir/port_type.go:88).  `id` presets Port.ID
 * (0 = unassigned until AssignPortIDs).  *port receives the port's handle
 * (its index), which nodes and read-back calls use. */
int mfh_topology_add_port(mfh_topology* topology, uint8_t dtype, const int64_t* dims, const char* const* symbols,
                          int32_t rank, int32_t id, int32_t* port);

/* An ir.Node appended to Topology.Nodes (which must be in topological
 * order).  `inputs` / `outputs` hold port handles; -1 is a nil port.  A port
 * shared by a producer's outputs and a consumer's inputs is the edge. */
int mfh_topology_add_node(mfh_topology* topology, const char* name, const int32_t* inputs, int32_t n_inputs,
                          const int32_t* outputs, int32_t n_outputs, int32_t* node);

/* SymbolMap entry used to size symbolic dimensions. */
int mfh_topology_bind(mfh_topology* topology, const char* symbol, int64_t value);

int32_t mfh_topology_num_nodes(const mfh_topology* topology);
int32_t mfh_topology_num_ports(const mfh_topology* topology);

/* ir.AssignPortIDs (ir/planner.go:107-170): sequential IDs by first
 * appearance (each node's outputs, then its inputs); preset IDs are kept
 * and numbering continues above the largest.  Idempotent. */
int mfh_topology_assign_port_ids(mfh_topology* topology);
int32_t mfh_topology_port_id(const mfh_topology* topology, int32_t port);

/* ir.Interval: a port's live range over node steps and its placement. */
typedef struct {
    int32_t port_id;
    int32_t start;
    int32_t end;
    int32_t reserved;
    int64_t size;
    int64_t offset;
} mfh_interval;

/* ir.AnalyzeLiveness (ir/planner.go:186-280): one interval per distinct
 * port ID seen (IDs 0 are skipped), ordered by (start, port_id).  Fails with
 * the reference's message when a dimension's symbol is unbound.  *n is the
 * interval count even when `cap` is smaller. */
int mfh_topology_liveness(const mfh_topology* topology, mfh_interval* intervals, int32_t cap, int32_t* n);

/* ir.AllocateOffsets (ir/planner.go:296-427): interval colouring.  Sorts
 * `intervals` in place by (start, port_id), rounds each size up to `align`
 * (<= 0: 64; must be a power of two) and gives each the lowest aligned
 * offset that overlaps no interval still live at its start (ranges are
 * inclusive: an interval ending at step s still conflicts with one starting
 * at s).  *total = the aligned high-water mark. */
int mfh_allocate_offsets(mfh_interval* intervals, int32_t n, int64_t align, int64_t* total);

/* ir.PlanWorkspace (ir/planner.go:43-96): AssignPortIDs, AnalyzeLiveness,
 * AllocateOffsets, then Port.Allocation for every planned port.  `align` <= 0
 * means 64; a non-power-of-two fails ("planner: Align=%d must be a power of
 * two"). */
int mfh_topology_plan_workspace(mfh_topology* topology, int64_t align);

/* Topology.Workspace after planning: Size, Align and the number of
 * Allocations; mfh_topology_allocation reads the k-th (allocation order). */
int mfh_topology_workspace(const mfh_topology* topology, int64_t* size, int64_t* align, int32_t* n_allocations);
int mfh_topology_allocation(const mfh_topology* topology, int32_t k, mfh_interval* interval);

/* Port.Allocation.BaseOffset; MFH_ERR_INVALID_ARGUMENT when the port has no
 * allocation (not planned, or an ID-0 port). */
int mfh_topology_port_offset(const mfh_topology* topology, int32_t port, int64_t* offset);

/* ir.SyncEvent (ir/sync_event.go): a signal (wait = 0) recorded on stream
 * `stream_id` after the node runs, or a wait (wait = 1) the node's stream
 * issues on that stream's event before the node runs. */
typedef struct {
    int32_t event_id;
    int32_t stream_id;
    int32_t wait;
    int32_t reserved;
} mfh_sync_event;

/* ir.ScheduleStreams (ir/stream_scheduler.go:56-287): assigns Node.StreamID
 * and SyncBarriers (`max_streams` < 1: as many streams as nodes).  A node
 * whose ID is 0 gets index + 1.  Where a node waits on several streams the
 * reference assigns event IDs in Go map order (unspecified); here they are
 * assigned in ascending predecessor-stream order. */
int mfh_topology_schedule_streams(mfh_topology* topology, int32_t max_streams);
const char* mfh_topology_node_name(const mfh_topology* topology, int32_t node);
int32_t mfh_topology_node_id(const mfh_topology* topology, int32_t node);
int32_t mfh_topology_node_stream(const mfh_topology* topology, int32_t node);
/* Copies up to `cap` barriers of the node in emission order; returns their
 * count (-1 for a bad handle). */
int32_t mfh_topology_node_barriers(const mfh_topology* topology, int32_t node, mfh_sync_event* events, int32_t cap);
/* A node's port handles (-1 for nil ports); returns the count. */
int32_t mfh_topology_node_ports(const mfh_topology* topology, int32_t node, int32_t outputs, int32_t* ports,
                                int32_t cap);

/* Workspace placement for a schedule that runs on several streams; the
 * reference has no counterpart (its planner assumes one stream of execution).
 * Like PlanWorkspace over the ports that nodes produce, but two values may
 * share memory only when every node touching the earlier one (its producer
 * and its readers) is ordered before the later one's producer, by stream
 * order and the nodes' wait barriers.  Call after
 * mfh_topology_schedule_streams.  Ports no node produces (graph inputs) get
 * no allocation; when every consumed port is produced and all nodes share
 * one stream, the offsets are PlanWorkspace's.  mfh_graph_call places its
 * intermediates this way. */
int mfh_topology_plan_stream_workspace(mfh_topology* topology, int64_t align);

/* compiler.PlanGraph (compiler/plan.go:242-290) for `graph`, with the value
 * shapes a call with `inputs` (dtype and count; data unused) would have:
 * one planning node per graph node in order, each with one output port of
 * its value's dtype and element count, the graph inputs as boundary ports,
 * then PlanWorkspace(align) and ScheduleStreams(max_streams).  A math.constant
 * node's port is one Float32.  Graph I/O offsets (Topology.InputPorts /
 * OutputPorts, compiler/plan.go:179-228) are read with
 * mfh_topology_io_offset.  The caller releases *topology. */
int mfh_graph_plan(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, int64_t align, int32_t max_streams,
                   mfh_topology** topology);

/* Topology.InputPorts[name] (output = 0) or OutputPorts[name] (output = 1). */
int mfh_topology_io_offset(const mfh_topology* topology, const char* name, int32_t output, int64_t* offset);

/* The MaxStreams mfh_graph_call schedules with (default 1: every node on the
 * caller's stream).  With more, independent nodes run on graph-owned HIP
 * streams (default priority) joined back into the caller's stream before the
 * call's output copies; the workspace then reuses a region only once every
 * reader of its previous value is ordered before the new writer. */
int mfh_graph_set_max_streams(mfh_graph* graph, int32_t max_streams);
/* HIP streams the last call used (1 = the caller's only). */
int32_t mfh_graph_streams_used(const mfh_graph* graph);

#ifdef __cplusplus
}
#endif
#endif /* MFH_PLAN_H */
