// plan.hpp — the planning IR shared by the topology ABI (plan.cpp) and the
// graph executor (graph.cpp): ports, nodes, liveness, interval colouring and
// the stream scheduler.
#ifndef MFH_PLAN_HPP
#define MFH_PLAN_HPP

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/mfh_plan.h"

namespace mfh {

// ir.Port with its PortType (dtype and dimensions) and Port.Allocation.
struct PlanPort {
    int32_t id = 0;
    uint8_t dtype = 0;
    std::vector<int64_t> dims;
    std::vector<std::string> symbols;  // "" for a static dimension
    bool allocated = false;
    int64_t offset = 0;
};

// ir.Node: its ports (handles into Topology::ports, -1 = nil) and the
// scheduler's output.
struct PlanNode {
    std::string name;
    int32_t id = 0;
    std::vector<int32_t> inputs, outputs;
    int32_t stream = 0;
    std::vector<mfh_sync_event> barriers;
};

struct Topology {
    std::vector<PlanPort> ports;
    std::vector<PlanNode> nodes;
    std::map<std::string, int64_t> bindings;
    bool planned = false;
    int64_t ws_size = 0, ws_align = 0;
    std::vector<mfh_interval> allocations;
    std::map<std::string, int64_t> input_ports, output_ports;  // Topology.InputPorts / OutputPorts
};

void assign_port_ids(Topology& t);
int analyze_liveness(const Topology& t, std::vector<mfh_interval>* out);
// Returns the aligned high-water mark; `align` must be a power of two.
int64_t allocate_offsets(std::vector<mfh_interval>& intervals, int64_t align);
int plan_workspace(Topology& t, int64_t align);
int schedule_streams(Topology& t, int32_t max_streams);

// Placement of values run across several streams.  A value conflicts with a
// later one unless every step that touches it (its producer and readers) is
// ordered strictly before the later value's producer; `before[j]` is the set
// of steps ordered before step j.  With one stream this is allocate_offsets'
// rule (an interval ending before the next one starts).
struct OrderedValue {
    int producer = 0;
    std::vector<int> users;  // steps that read it; kPinned keeps it to the end
    int64_t size = 0;
    int64_t offset = 0;
};
constexpr int kPinned = -1;
using StepSet = std::vector<uint64_t>;
// Steps ordered before each step by stream order and the wait barriers of a
// schedule (nodes in step order).
std::vector<StepSet> order_of(const std::vector<PlanNode>& nodes);
int64_t place_ordered(std::vector<OrderedValue>& values, const std::vector<StepSet>& before, int64_t align);

}  // namespace mfh

struct mfh_topology : mfh::Topology {};

#endif  // MFH_PLAN_HPP
