// plan.cpp — workspace planner and stream scheduler (include/mfh_plan.h).
//
// The algorithms restate the reference's planning IR step for step so that
// offsets, stream IDs and sync events agree with it on the same topology:
// ir/planner.go (AssignPortIDs, AnalyzeLiveness, AllocateOffsets,
// PlanWorkspace, PortByteSize) and ir/stream_scheduler.go (ScheduleStreams,
// pickStream).  place_ordered / order_of extend the colouring rule to
// schedules that run on several HIP streams.
#include <algorithm>
#include <cinttypes>
#include <cstring>
#include <map>
#include <unordered_map>

#include "common.hpp"
#include "plan.hpp"

namespace mfh {
namespace {

bool power_of_two(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int64_t align_to(int64_t v, int64_t align)
{
    if (align <= 1) return v;
    return (v + align - 1) & ~(align - 1);
}

// DType.Size's error for dtypes without a size (dtype/dtype.go:57-74).
bool sized(int dt)
{
    switch (dt) {
    case kInt4: case kBool: case kComplex64: case kComplex128: return true;
    default: return dtype_size(dt) > 0;
    }
}

// PortByteSize (ir/planner.go:437-480); `what` prefixes the message as
// AnalyzeLiveness wraps it.
int port_byte_size(const Topology& t, const PlanPort& p, const char* what, int64_t* out)
{
    if (p.dims.empty()) {
        if (!sized(p.dtype))
            return fail(MFH_ERR_INVALID_ARGUMENT, "port id=%d%s: dtype %s rejected scalar size: dtype: unsupported dtype %d",
                        (int)p.id, what, dtype_string(p.dtype), (int)p.dtype);
        *out = bytes_for(p.dtype, 1);
        return MFH_OK;
    }
    int64_t elements = 1;
    for (size_t k = 0; k < p.dims.size(); k++) {
        if (p.symbols[k].empty()) {
            elements *= p.dims[k];
            continue;
        }
        auto it = t.bindings.find(p.symbols[k]);
        if (it == t.bindings.end())
            return fail(MFH_ERR_INVALID_ARGUMENT,
                        "port id=%d%s: dim[%d] symbol \"%s\" is unbound (run unifier first to populate bindings)",
                        (int)p.id, what, (int)k, p.symbols[k].c_str());
        elements *= it->second;
    }
    if (elements < 0)
        return fail(MFH_ERR_INVALID_ARGUMENT, "port id=%d%s: dtype %s rejected %lld elements: dtype: negative element count %lld",
                    (int)p.id, what, dtype_string(p.dtype), (long long)elements, (long long)elements);
    if (!sized(p.dtype))
        return fail(MFH_ERR_INVALID_ARGUMENT, "port id=%d%s: dtype %s rejected %lld elements: dtype: unsupported dtype %d",
                    (int)p.id, what, dtype_string(p.dtype), (long long)elements, (int)p.dtype);
    *out = bytes_for(p.dtype, elements);
    return MFH_OK;
}

bool by_start_then_port(const mfh_interval& a, const mfh_interval& b)
{
    if (a.start != b.start) return a.start < b.start;
    return a.port_id < b.port_id;
}

struct Block {
    int64_t offset, size;
};

// chooseLowestNonConflictingOffset (ir/planner.go:376-411).
int64_t lowest_free(int64_t size, std::vector<Block> live, int64_t align)
{
    if (live.empty()) return 0;
    std::stable_sort(live.begin(), live.end(), [](const Block& a, const Block& b) { return a.offset < b.offset; });
    int64_t candidate = 0;
    for (;;) {
        bool conflict = false;
        for (const Block& b : live) {
            if (candidate >= b.offset + b.size) continue;
            if (candidate + size <= b.offset) continue;
            candidate = align_to(b.offset + b.size, align);
            conflict = true;
            break;
        }
        if (!conflict) return candidate;
    }
}

}  // namespace

// AssignPortIDs (ir/planner.go:107-170).
void assign_port_ids(Topology& t)
{
    std::vector<char> seen(t.ports.size(), 0);
    int32_t next = 1;
    auto visit = [&](int32_t h, bool assign) {
        if (h < 0 || seen[h]) return;
        seen[h] = 1;
        PlanPort& p = t.ports[h];
        if (!assign) {
            if (p.id >= next) next = p.id + 1;
        } else if (p.id == 0) {
            p.id = next++;
        }
    };
    for (bool assign : {false, true}) {
        std::fill(seen.begin(), seen.end(), 0);
        for (const PlanNode& n : t.nodes) {
            for (int32_t h : n.outputs) visit(h, assign);
            for (int32_t h : n.inputs) visit(h, assign);
        }
    }
}

// AnalyzeLiveness (ir/planner.go:186-280).
int analyze_liveness(const Topology& t, std::vector<mfh_interval>* out)
{
    out->clear();
    std::unordered_map<int32_t, size_t> at;  // port ID -> index in *out
    for (size_t step = 0; step < t.nodes.size(); step++) {
        const PlanNode& n = t.nodes[step];
        for (int32_t h : n.outputs) {
            if (h < 0 || t.ports[h].id == 0 || at.count(t.ports[h].id)) continue;
            int64_t size;
            MFH_TRY(port_byte_size(t, t.ports[h], "", &size));
            at.emplace(t.ports[h].id, out->size());
            out->push_back(mfh_interval{t.ports[h].id, (int32_t)step, (int32_t)step, 0, size, 0});
        }
        for (int32_t h : n.inputs) {
            if (h < 0 || t.ports[h].id == 0) continue;
            auto it = at.find(t.ports[h].id);
            if (it == at.end()) {
                // an unproduced input (graph input, weight) is live from step 0
                int64_t size;
                MFH_TRY(port_byte_size(t, t.ports[h], " (unproduced input)", &size));
                at.emplace(t.ports[h].id, out->size());
                out->push_back(mfh_interval{t.ports[h].id, 0, (int32_t)step, 0, size, 0});
                continue;
            }
            mfh_interval& iv = (*out)[it->second];
            if ((int32_t)step > iv.end) iv.end = (int32_t)step;
        }
    }
    std::sort(out->begin(), out->end(), by_start_then_port);
    return MFH_OK;
}

// AllocateOffsets (ir/planner.go:296-350).
int64_t allocate_offsets(std::vector<mfh_interval>& work, int64_t align)
{
    if (align <= 0) align = 64;
    if (work.empty()) return 0;
    std::stable_sort(work.begin(), work.end(), by_start_then_port);
    struct Live {
        int64_t offset, size;
        int32_t end;
    };
    std::vector<Live> live;
    int64_t high = 0;
    for (mfh_interval& iv : work) {
        iv.size = align_to(iv.size, align);
        // evict blocks that ended strictly before this start (inclusive ranges)
        live.erase(std::remove_if(live.begin(), live.end(), [&](const Live& b) { return b.end < iv.start; }),
                   live.end());
        std::vector<Block> blocks;
        for (const Live& b : live) blocks.push_back(Block{b.offset, b.size});
        iv.offset = lowest_free(iv.size, blocks, align);
        live.push_back(Live{iv.offset, iv.size, iv.end});
        high = std::max(high, iv.offset + iv.size);
    }
    return align_to(high, align);
}

// PlanWorkspace (ir/planner.go:43-96) with attachAllocationsToPorts (:482-513).
int plan_workspace(Topology& t, int64_t align)
{
    if (align <= 0) align = 64;
    if (!power_of_two(align))
        return fail(MFH_ERR_INVALID_ARGUMENT, "planner: Align=%lld must be a power of two", (long long)align);
    assign_port_ids(t);
    std::vector<mfh_interval> intervals;
    MFH_TRY(analyze_liveness(t, &intervals));
    const int64_t total = allocate_offsets(intervals, align);
    t.ws_size = total;
    t.ws_align = align;
    t.allocations = intervals;
    t.planned = true;
    std::unordered_map<int32_t, int64_t> offset_of;
    for (const mfh_interval& iv : intervals) offset_of.emplace(iv.port_id, iv.offset);
    std::vector<char> seen(t.ports.size(), 0);
    auto attach = [&](int32_t h) {
        if (h < 0 || seen[h]) return;
        seen[h] = 1;
        auto it = offset_of.find(t.ports[h].id);
        if (it == offset_of.end()) return;
        t.ports[h].allocated = true;
        t.ports[h].offset = it->second;
    };
    for (const PlanNode& n : t.nodes) {
        for (int32_t h : n.outputs) attach(h);
        for (int32_t h : n.inputs) attach(h);
    }
    return MFH_OK;
}

// ScheduleStreams (ir/stream_scheduler.go:56-141) with buildProducerIndex,
// collectPredecessorStreams and pickStream (:150-287).
int schedule_streams(Topology& t, int32_t max_streams)
{
    if (t.nodes.empty()) return MFH_OK;
    if (max_streams < 1) max_streams = (int32_t)t.nodes.size();
    std::unordered_map<int32_t, int> producer_of;  // port handle -> first producing node
    for (int i = 0; i < (int)t.nodes.size(); i++)
        for (int32_t h : t.nodes[i].outputs)
            if (h >= 0) producer_of.emplace(h, i);
    std::unordered_map<int32_t, int32_t> stream_last;  // stream -> last node ID assigned to it
    int32_t next_stream = 0, next_event = 1;
    auto last_on = [&](int32_t s) {
        auto it = stream_last.find(s);
        return it == stream_last.end() ? 0 : it->second;
    };
    for (int index = 0; index < (int)t.nodes.size(); index++) {
        PlanNode& node = t.nodes[index];
        if (node.id == 0) node.id = index + 1;
        // predecessor stream -> most recent producer ID on it
        std::map<int32_t, int32_t> preds;
        for (int32_t h : node.inputs) {
            if (h < 0) continue;
            auto it = producer_of.find(h);
            if (it == producer_of.end()) continue;
            const PlanNode& p = t.nodes[it->second];
            auto e = preds.find(p.stream);
            if (e == preds.end() || p.id > e->second) preds[p.stream] = p.id;
        }
        int32_t assigned;
        if (preds.empty()) {
            assigned = next_stream < max_streams ? next_stream++ : 0;
        } else if (preds.size() == 1) {
            const int32_t only = preds.begin()->first, pred = preds.begin()->second;
            if (last_on(only) == pred) assigned = only;  // continue the serial chain
            else if (next_stream < max_streams) assigned = next_stream++;
            else assigned = only;
        } else {
            assigned = preds.begin()->first;  // merge on the lowest predecessor stream
        }
        node.stream = assigned;
        stream_last[assigned] = node.id;
        for (const auto& kv : preds) {
            if (kv.first == assigned) continue;
            const int32_t event = next_event++;
            node.barriers.push_back(mfh_sync_event{event, kv.first, 1, 0});
            PlanNode* producer = nullptr;
            for (PlanNode& n : t.nodes)
                if (n.id == kv.second) {
                    producer = &n;
                    break;
                }
            if (!producer)
                return fail(MFH_ERR_INVALID_ARGUMENT,
                            "scheduler: node \"%s\" (id=%d) waits on stream %d producer id=%d, but no such node exists",
                            node.name.c_str(), (int)node.id, (int)kv.first, (int)kv.second);
            producer->barriers.push_back(mfh_sync_event{event, kv.first, 0, 0});
        }
    }
    return MFH_OK;
}

std::vector<StepSet> order_of(const std::vector<PlanNode>& nodes)
{
    const size_t n = nodes.size(), words = (n + 63) / 64;
    std::vector<StepSet> before(n, StepSet(words, 0));
    std::unordered_map<int32_t, int> last_on;   // stream -> last step on it
    std::unordered_map<int32_t, int> signaller;  // event ID -> step recording it
    auto absorb = [&](StepSet& into, int k) {
        for (size_t w = 0; w < words; w++) into[w] |= before[k][w];
        into[k / 64] |= 1ull << (k % 64);
    };
    for (int j = 0; j < (int)n; j++) {
        auto it = last_on.find(nodes[j].stream);
        if (it != last_on.end()) absorb(before[j], it->second);
        for (const mfh_sync_event& e : nodes[j].barriers) {
            if (!e.wait) continue;
            auto s = signaller.find(e.event_id);
            if (s != signaller.end()) absorb(before[j], s->second);
        }
        for (const mfh_sync_event& e : nodes[j].barriers)
            if (!e.wait) signaller[e.event_id] = j;
        last_on[nodes[j].stream] = j;
    }
    return before;
}

int64_t place_ordered(std::vector<OrderedValue>& values, const std::vector<StepSet>& before, int64_t align)
{
    std::vector<size_t> order(values.size());
    for (size_t i = 0; i < order.size(); i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(),
                     [&](size_t a, size_t b) { return values[a].producer < values[b].producer; });
    auto ordered_before = [&](int u, int step) {
        return u != kPinned && u != step && ((before[step][u / 64] >> (u % 64)) & 1u);
    };
    std::vector<size_t> placed;
    int64_t high = 0;
    for (size_t i : order) {
        OrderedValue& w = values[i];
        w.size = align_to(w.size, align);
        std::vector<Block> live;
        for (size_t j : placed) {
            const OrderedValue& v = values[j];
            bool dead = ordered_before(v.producer, w.producer);
            for (int u : v.users) dead = dead && ordered_before(u, w.producer);
            if (!dead) live.push_back(Block{v.offset, v.size});
        }
        w.offset = lowest_free(w.size, live, align);
        placed.push_back(i);
        high = std::max(high, w.offset + w.size);
    }
    return align_to(high, align);
}

}  // namespace mfh

using namespace mfh;

namespace {

PlanNode* topo_node(const mfh_topology* t, int32_t i)
{
    if (!t || i < 0 || i >= (int32_t)t->nodes.size()) return nullptr;
    return const_cast<PlanNode*>(&t->nodes[i]);
}

bool topo_port(const mfh_topology* t, int32_t h) { return t && h >= 0 && h < (int32_t)t->ports.size(); }

}  // namespace

extern "C" {

int mfh_topology_create(mfh_topology** topology)
{
    if (!topology) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_create: out-pointer is NULL");
    *topology = new mfh_topology();
    return MFH_OK;
}

int mfh_topology_release(mfh_topology* topology)
{
    delete topology;
    return MFH_OK;
}

int mfh_topology_add_port(mfh_topology* t, uint8_t dtype, const int64_t* dims, const char* const* symbols,
                          int32_t rank, int32_t id, int32_t* port)
{
    if (!t || rank < 0 || (rank > 0 && !dims && !symbols))
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_add_port: topology and dims are required");
    PlanPort p;
    p.id = id;
    p.dtype = dtype;
    for (int32_t k = 0; k < rank; k++) {
        const char* sym = symbols ? symbols[k] : nullptr;
        p.symbols.push_back(sym ? sym : "");
        p.dims.push_back(dims && !sym ? dims[k] : 0);
    }
    t->ports.push_back(std::move(p));
    if (port) *port = (int32_t)t->ports.size() - 1;
    return MFH_OK;
}

int mfh_topology_add_node(mfh_topology* t, const char* name, const int32_t* inputs, int32_t n_inputs,
                          const int32_t* outputs, int32_t n_outputs, int32_t* node)
{
    if (!t || n_inputs < 0 || n_outputs < 0 || (n_inputs > 0 && !inputs) || (n_outputs > 0 && !outputs))
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_add_node: bad port list");
    PlanNode n;
    n.name = name ? name : "";
    for (int32_t k = 0; k < n_inputs + n_outputs; k++) {
        const int32_t h = k < n_inputs ? inputs[k] : outputs[k - n_inputs];
        if (h != -1 && !topo_port(t, h))
            return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_add_node: node \"%s\": no port %d", n.name.c_str(), (int)h);
        (k < n_inputs ? n.inputs : n.outputs).push_back(h);
    }
    t->nodes.push_back(std::move(n));
    if (node) *node = (int32_t)t->nodes.size() - 1;
    return MFH_OK;
}

int mfh_topology_bind(mfh_topology* t, const char* symbol, int64_t value)
{
    if (!t || !symbol || !*symbol) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_bind: symbol is required");
    t->bindings[symbol] = value;
    return MFH_OK;
}

int32_t mfh_topology_num_nodes(const mfh_topology* t) { return t ? (int32_t)t->nodes.size() : -1; }
int32_t mfh_topology_num_ports(const mfh_topology* t) { return t ? (int32_t)t->ports.size() : -1; }

int mfh_topology_assign_port_ids(mfh_topology* t)
{
    if (!t) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_assign_port_ids: topology is required");
    assign_port_ids(*t);
    return MFH_OK;
}

int32_t mfh_topology_port_id(const mfh_topology* t, int32_t port) { return topo_port(t, port) ? t->ports[port].id : -1; }

int mfh_topology_liveness(const mfh_topology* t, mfh_interval* intervals, int32_t cap, int32_t* n)
{
    if (!t || cap < 0 || (cap > 0 && !intervals))
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_liveness: topology and buffer are required");
    std::vector<mfh_interval> out;
    MFH_TRY(analyze_liveness(*t, &out));
    for (int32_t k = 0; k < cap && k < (int32_t)out.size(); k++) intervals[k] = out[k];
    if (n) *n = (int32_t)out.size();
    return MFH_OK;
}

int mfh_allocate_offsets(mfh_interval* intervals, int32_t n, int64_t align, int64_t* total)
{
    if (n < 0 || (n > 0 && !intervals)) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_allocate_offsets: bad interval list");
    if (align <= 0) align = 64;
    if (!power_of_two(align))
        return fail(MFH_ERR_INVALID_ARGUMENT, "planner: Align=%lld must be a power of two", (long long)align);
    std::vector<mfh_interval> work(intervals, intervals + n);
    const int64_t size = allocate_offsets(work, align);
    std::copy(work.begin(), work.end(), intervals);
    if (total) *total = size;
    return MFH_OK;
}

int mfh_topology_plan_workspace(mfh_topology* t, int64_t align)
{
    if (!t) return fail(MFH_ERR_INVALID_ARGUMENT, "planner: topology is required");
    return plan_workspace(*t, align);
}

int mfh_topology_workspace(const mfh_topology* t, int64_t* size, int64_t* align, int32_t* n_allocations)
{
    if (!t) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_workspace: topology is required");
    if (size) *size = t->ws_size;
    if (align) *align = t->ws_align;
    if (n_allocations) *n_allocations = (int32_t)t->allocations.size();
    return MFH_OK;
}

int mfh_topology_allocation(const mfh_topology* t, int32_t k, mfh_interval* interval)
{
    if (!t || !interval || k < 0 || k >= (int32_t)t->allocations.size())
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_allocation: no allocation %d", (int)k);
    *interval = t->allocations[k];
    return MFH_OK;
}

int mfh_topology_port_offset(const mfh_topology* t, int32_t port, int64_t* offset)
{
    if (!topo_port(t, port) || !offset) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_port_offset: no port %d", (int)port);
    if (!t->ports[port].allocated)
        return fail(MFH_ERR_INVALID_ARGUMENT, "planner: port %d (id=%d) has no allocation", (int)port, (int)t->ports[port].id);
    *offset = t->ports[port].offset;
    return MFH_OK;
}

int mfh_topology_plan_stream_workspace(mfh_topology* t, int64_t align)
{
    if (!t) return fail(MFH_ERR_INVALID_ARGUMENT, "planner: topology is required");
    if (align <= 0) align = 64;
    if (!power_of_two(align))
        return fail(MFH_ERR_INVALID_ARGUMENT, "planner: Align=%lld must be a power of two", (long long)align);
    assign_port_ids(*t);
    // one value per produced port ID, in port-ID order (the colouring's
    // tie-break), with the steps that read it
    std::map<int32_t, OrderedValue> by_id;
    std::map<int32_t, int32_t> handle_of;
    for (int step = 0; step < (int)t->nodes.size(); step++)
        for (int32_t h : t->nodes[step].outputs) {
            if (h < 0 || t->ports[h].id == 0 || by_id.count(t->ports[h].id)) continue;
            OrderedValue v;
            v.producer = step;
            MFH_TRY(port_byte_size(*t, t->ports[h], "", &v.size));
            by_id.emplace(t->ports[h].id, v);
            handle_of.emplace(t->ports[h].id, h);
        }
    for (int step = 0; step < (int)t->nodes.size(); step++)
        for (int32_t h : t->nodes[step].inputs) {
            if (h < 0) continue;
            auto it = by_id.find(t->ports[h].id);
            if (it != by_id.end() && step > it->second.producer) it->second.users.push_back(step);
        }
    std::vector<OrderedValue> values;
    std::vector<int32_t> ids;
    for (auto& kv : by_id) {
        ids.push_back(kv.first);
        values.push_back(kv.second);
    }
    const int64_t total = place_ordered(values, order_of(t->nodes), align);
    t->allocations.clear();
    std::unordered_map<int32_t, int64_t> offset_of;
    for (size_t k = 0; k < values.size(); k++) {
        int32_t end = values[k].producer;
        for (int u : values[k].users) end = std::max(end, (int32_t)u);
        t->allocations.push_back(mfh_interval{ids[k], values[k].producer, end, 0, values[k].size, values[k].offset});
        offset_of.emplace(ids[k], values[k].offset);
    }
    std::stable_sort(t->allocations.begin(), t->allocations.end(), by_start_then_port);
    for (PlanPort& p : t->ports) {
        auto it = offset_of.find(p.id);
        p.allocated = p.id != 0 && it != offset_of.end();
        if (p.allocated) p.offset = it->second;
    }
    t->ws_size = total;
    t->ws_align = align;
    t->planned = true;
    return MFH_OK;
}

int mfh_topology_schedule_streams(mfh_topology* t, int32_t max_streams)
{
    if (!t) return fail(MFH_ERR_INVALID_ARGUMENT, "scheduler: topology is required");
    return schedule_streams(*t, max_streams);
}

const char* mfh_topology_node_name(const mfh_topology* t, int32_t node)
{
    const PlanNode* n = topo_node(t, node);
    return n ? n->name.c_str() : nullptr;
}

int32_t mfh_topology_node_id(const mfh_topology* t, int32_t node)
{
    const PlanNode* n = topo_node(t, node);
    return n ? n->id : -1;
}

int32_t mfh_topology_node_stream(const mfh_topology* t, int32_t node)
{
    const PlanNode* n = topo_node(t, node);
    return n ? n->stream : -1;
}

int32_t mfh_topology_node_barriers(const mfh_topology* t, int32_t node, mfh_sync_event* events, int32_t cap)
{
    const PlanNode* n = topo_node(t, node);
    if (!n) return -1;
    for (int32_t k = 0; k < cap && k < (int32_t)n->barriers.size(); k++) events[k] = n->barriers[k];
    return (int32_t)n->barriers.size();
}

int32_t mfh_topology_node_ports(const mfh_topology* t, int32_t node, int32_t outputs, int32_t* ports, int32_t cap)
{
    const PlanNode* n = topo_node(t, node);
    if (!n) return -1;
    const std::vector<int32_t>& v = outputs ? n->outputs : n->inputs;
    for (int32_t k = 0; k < cap && k < (int32_t)v.size(); k++) ports[k] = v[k];
    return (int32_t)v.size();
}

int mfh_topology_io_offset(const mfh_topology* t, const char* name, int32_t output, int64_t* offset)
{
    if (!t || !name || !offset) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_io_offset: bad arguments");
    const auto& m = output ? t->output_ports : t->input_ports;
    auto it = m.find(name);
    if (it == m.end())
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_topology_io_offset: no graph %s \"%s\"", output ? "output" : "input", name);
    *offset = it->second;
    return MFH_OK;
}

}  // extern "C"
