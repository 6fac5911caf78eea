// graph.cpp — the compile-and-dispatch layer around the HIP codegen target:
// the manifest compute graph (ast.Graph), the optimizer's ConstantFold and
// Fuse passes, codegen's AttachKernels with a HIP target, and CallGraph-style
// execution of the lowered graph on HIP streams.
//
// The passes restate the reference's Go semantics (file:line at each) so that
// a C++ host gets the FusionASTs the Go compiler would hand to EmitHIP.
// Execution launches the nodes in graph order on the streams ScheduleStreams
// assigns (plan.cpp); a value passed between nodes lives in one per-graph
// device workspace at offsets from the planner's interval colouring, so a
// steady-state call allocates nothing.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mfh_graph.h"
#include "../../include/mfh_plan.h"
#include "common.hpp"
#include "fusion.hpp"
#include "plan.hpp"
#include "scratch.hpp"

namespace mfh {
namespace {

const char* const kFuseOp = "optimizer.fusion";        // optimizer/fuse.go:16
const char* const kFuseAttributeAST = "fusion_ast";    // optimizer/fuse.go:22
const char* const kConstantOp = "math.constant";       // optimizer/constant_fold.go:23
const char* const kConstantValue = "value";            // optimizer/constant_fold.go:16
const char* const kFusedNodeCount = "fused_node_count";  // optimizer/fuse.go:131

bool hip_storage(int dt) { return dt == kFloat32 || dt == kFloat16 || dt == kBFloat16; }

// ---- elementwise table (optimizer/elementwise.go:15-36) ---------------------

struct OpEntry {
    const char* op;
    int32_t type;
};

// Op string -> NodeType.  kNodeInvalid rows exist but are disabled, as in the
// reference (sin/cos).  "math.sign" maps to Neg there as a placeholder; the
// mapping is kept so that graphs fuse identically.
const OpEntry kElementwiseTable[] = {
    {"math.add", kNodeAdd},   {"math.sub", kNodeSub},   {"math.mul", kNodeMul},
    {"math.div", kNodeDiv},   {"math.max", kNodeMax},   {"math.min", kNodeMin},
    {"math.neg", kNodeNeg},   {"math.abs", kNodeAbs},   {"math.sqrt", kNodeSqrt},
    {"math.exp", kNodeExp},   {"math.log", kNodeLog},   {"math.sign", kNodeNeg},
    {"math.sin", kNodeInvalid}, {"math.cos", kNodeInvalid},
    {"activation.relu", kNodeReLU},       {"activation.sigmoid", kNodeSigmoid},
    {"activation.tanh", kNodeTanh},       {"activation.swish", kNodeSilu},
    {"activation.gelu", kNodeGelu},       {"activation.leaky_relu", kNodeLeakyReLU},
};

bool is_space(unsigned char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r'; }

// isElementwiseOp (optimizer/elementwise.go:44-54): strings.TrimSpace +
// strings.ToLower, then the table; disabled rows are not eligible.  Only
// ASCII white space and letters are folded (every table key is ASCII).
int32_t elementwise_type(const std::string& op)
{
    size_t b = 0, e = op.size();
    while (b < e && is_space((unsigned char)op[b])) b++;
    while (e > b && is_space((unsigned char)op[e - 1])) e--;
    std::string key = op.substr(b, e - b);
    for (char& c : key)
        if (c >= 'A' && c <= 'Z') c = (char)(c - 'A' + 'a');
    for (const OpEntry& row : kElementwiseTable)
        if (key == row.op) return row.type;
    return kNodeInvalid;
}

// ---- FusionAST (optimizer/fusion_ast.go:70-113) -----------------------------

struct ASTNode {
    int32_t type = kNodeInvalid;
    int32_t input_index = 0;
    double value = 0.0;
    std::vector<std::unique_ptr<ASTNode>> children;
};

std::unique_ptr<ASTNode> input_leaf(int index)
{
    auto n = std::make_unique<ASTNode>();
    n->type = kNodeInput;
    n->input_index = index;
    return n;
}

struct FusionAST {
    std::unique_ptr<ASTNode> root;
    std::vector<std::string> input_ports;
    std::string output_port;
    std::string count_expr;  // never set by Fuse (optimizer/fuse.go:108-114)
    uint8_t dtype = kInvalid;
    std::vector<std::string> contained_node_ids;

    // pre-order view for the ABI, rebuilt on demand
    std::vector<mfh_ast_node> flat;
    std::vector<int32_t> child_counts;
    void flatten()
    {
        flat.clear();
        child_counts.clear();
        if (root) walk(*root);
    }
    void walk(const ASTNode& n)
    {
        flat.push_back(mfh_ast_node{n.type, n.input_index, n.value});
        child_counts.push_back((int32_t)n.children.size());
        for (const auto& c : n.children) walk(*c);
    }
};

// ---- HIP kernels (the TargetHIP member of a KernelSet) -----------------------

struct KernelDeleter {
    void operator()(mfh_kernel* k) const { (void)mfh_fusion_release(k); }
};
using KernelPtr = std::unique_ptr<mfh_kernel, KernelDeleter>;

std::string signature(const std::vector<mfh_operand>& ops)
{
    std::string s;
    for (const mfh_operand& op : ops)
        s += std::to_string(op.dtype) + ":" + std::to_string(op.mode) + ":" + std::to_string(op.period) + ";";
    return s;
}

// One FusionAST lowered for gfx950.  Operand dtypes and broadcast modes are
// only known at dispatch, so the kernel keeps one compiled variant per operand
// signature; the full-length variant of the declared dtypes is compiled when
// the kernel is emitted (and is what KernelSet.For hands out).
struct HIPKernel {
    std::string identifier;
    std::vector<std::string> inputs;
    std::vector<mfh_ast_node> nodes;  // pre-order, child counts == arity
    std::vector<uint8_t> declared;    // per input: declared dtype or kInvalid
    uint8_t out_dtype = kFloat32;
    uint32_t flags = 0;
    std::map<std::string, KernelPtr> variants;
    const mfh_kernel* full = nullptr;

    // The variant for `ops` if it was compiled before, else NULL.
    const mfh_kernel* find(const std::vector<mfh_operand>& ops) const
    {
        auto it = variants.find(signature(ops));
        return it == variants.end() ? nullptr : it->second.get();
    }

    int variant(const std::vector<mfh_operand>& ops, const mfh_kernel** out)
    {
        std::string key = signature(ops);
        auto it = variants.find(key);
        if (it == variants.end()) {
            mfh_kernel* k = nullptr;
            MFH_TRY(emit_hip(nodes.data(), (int)nodes.size(), ops.data(), (int)ops.size(), out_dtype,
                             identifier.c_str(), flags, &k));
            it = variants.emplace(key, KernelPtr(k)).first;
        }
        *out = it->second.get();
        return MFH_OK;
    }
};

struct KernelSet {  // codegen/attach.go:14-16
    std::map<int32_t, std::shared_ptr<HIPKernel>> kernels;
    HIPKernel* For(int32_t target) const
    {
        auto it = kernels.find(target);
        return it == kernels.end() ? nullptr : it->second.get();
    }
};

// ---- ast.Graph ---------------------------------------------------------------

struct GraphNode {
    std::string id;
    std::string op;
    std::vector<std::string> inputs;
    std::map<std::string, double> attributes;  // numeric Attributes
    std::map<std::string, int64_t> metadata;
    std::shared_ptr<FusionAST> fusion;  // Attributes["fusion_ast"]
    std::shared_ptr<KernelSet> kernels;  // Attributes["compiled_kernel"]
    std::vector<uint8_t> input_types;    // InputTypes[k].DType
    uint8_t output_type = kInvalid;      // OutputType.DType
    std::shared_ptr<HIPKernel> solo;     // one-node kernel of an unfused elementwise node
};

// A call's launches, placement and streams for one signature of bindings
// (defined with the execution code below).
struct PlannedCall;
constexpr int kMaxPlans = 8;

}  // namespace
}  // namespace mfh

struct mfh_graph {
    std::vector<std::unique_ptr<mfh::GraphNode>> nodes;
    std::vector<std::string> inputs;
    std::vector<std::pair<std::string, std::string>> outputs;  // key -> value
    uint8_t execution_dtype = mfh::kInvalid;
    // device workspace: constants first, then the intermediate values
    void* ws = nullptr;
    int64_t ws_bytes = 0;
    std::vector<float> ws_constants;  // the constants the workspace holds
    bool ws_constants_valid = false;
    uint32_t codegen_flags = 0;  // of the last AttachKernels; also used for unfused nodes
    // stream mapping: StreamID k > 0 runs on aux[k - 1], StreamID 0 on the
    // caller's stream; events[e] is SyncEvent e
    int32_t max_streams = 1;
    int32_t streams_used = 0;
    std::vector<hipStream_t> aux;
    std::vector<hipEvent_t> events;
    std::vector<hipEvent_t> joins;  // per aux stream, back into the caller's
    hipEvent_t fork = nullptr;
    // Recorded after a call's last work: call n records done_ring[n % 4], and
    // `done` is the latest of them, so a call's end can still be waited for a
    // few calls later.
    static constexpr int kDoneRing = 4;
    hipEvent_t done_ring[kDoneRing] = {};
    hipEvent_t done = nullptr;
    uint64_t call_seq = 0;  // calls recorded so far
    hipStream_t last_stream = nullptr;
    bool called = false;
    // calls replayed as HIP graphs, one per plan (below); cleared by any
    // change to the graph
    bool replay = true;
    bool replay_broken = false;
    uint64_t replay_generation = 0;  // module generation of the captured calls
    int64_t replayed = 0;
    hipStream_t capture = nullptr;
    // calls planned before, keyed by their bindings without the pointers;
    // cleared by any change to the graph
    std::vector<std::unique_ptr<mfh::PlannedCall>> plans;
    uint64_t plan_clock = 0;
};

namespace mfh {
namespace {

using Graph = mfh_graph;

// ---- Fuse (optimizer/fuse.go:54-265) -----------------------------------------

struct ClusterBuilder {
    const Graph& graph;
    const std::unordered_map<std::string, int>& producers;
    const std::unordered_map<std::string, int>& consumers;
    const std::vector<char>& absorbed;
    std::set<int> members;  // absorbedIndices
    std::vector<std::string> inputs;
    std::unordered_map<std::string, int> input_index;

    std::unique_ptr<ASTNode> external(const std::string& name)
    {
        auto it = input_index.find(name);
        if (it != input_index.end()) return input_leaf(it->second);
        int k = (int)inputs.size();
        inputs.push_back(name);
        input_index.emplace(name, k);
        return input_leaf(k);
    }

    // build (optimizer/fuse.go:203-223)
    std::unique_ptr<ASTNode> build(const GraphNode& node)
    {
        int32_t type = elementwise_type(node.op);
        if (type == kNodeInvalid) return external(node.id);
        members.insert(producers.at(node.id));
        auto n = std::make_unique<ASTNode>();
        n->type = type;
        for (const std::string& name : node.inputs) n->children.push_back(operand(name));
        return n;
    }

    // buildOperand (optimizer/fuse.go:228-256): inline the producer only when
    // it is an elementwise node with exactly one consumer that no cluster has
    // taken yet.
    std::unique_ptr<ASTNode> operand(const std::string& name)
    {
        auto p = producers.find(name);
        if (p == producers.end()) return external(name);
        const int index = p->second;
        if (absorbed[index] || members.count(index)) return external(name);
        auto c = consumers.find(name);
        if (c == consumers.end() || c->second != 1) return external(name);
        const GraphNode& producer = *graph.nodes[index];
        if (elementwise_type(producer.op) == kNodeInvalid) return external(name);
        return build(producer);
    }
};

// fusionInputTypes / boundaryInputPortType (optimizer/fuse.go:303-350): a
// port's type is its producer's OutputType, else the InputTypes slot of the
// first node that reads it.
std::vector<uint8_t> fusion_input_types(const Graph& g, const std::vector<std::string>& names)
{
    std::unordered_map<std::string, uint8_t> produced;
    for (const auto& n : g.nodes)
        if (n && n->output_type != kInvalid) produced[n->id] = n->output_type;
    std::vector<uint8_t> out(names.size(), kInvalid);
    for (size_t k = 0; k < names.size(); k++) {
        auto it = produced.find(names[k]);
        if (it != produced.end()) {
            out[k] = it->second;
            continue;
        }
        bool found = false;
        for (const auto& n : g.nodes) {
            if (!n) continue;
            for (size_t s = 0; s < n->inputs.size() && !found; s++)
                if (n->inputs[s] == names[k] && s < n->input_types.size()) {
                    out[k] = n->input_types[s];
                    found = true;
                }
            if (found) break;
        }
    }
    return out;
}

int fuse(Graph& g, mfh_fusion_stats* stats)
{
    mfh_fusion_stats st{0, 0, 0};
    const int n = (int)g.nodes.size();
    std::unordered_map<std::string, int> producers;
    for (int i = 0; i < n; i++) producers[g.nodes[i]->id] = i;
    std::unordered_map<std::string, int> consumers;
    for (const auto& node : g.nodes)
        for (const std::string& name : node->inputs) consumers[name]++;
    for (const auto& kv : g.outputs) consumers[kv.second]++;  // outputs stay materialised

    std::vector<char> visited(n, 0), absorbed(n, 0);
    // Reverse walk: a consumer absorbs its eligible producers before they can
    // become roots of their own (optimizer/fuse.go:82-140).
    for (int index = n - 1; index >= 0; index--) {
        if (visited[index] || absorbed[index]) continue;
        GraphNode& node = *g.nodes[index];
        if (elementwise_type(node.op) == kNodeInvalid) {
            visited[index] = 1;
            continue;
        }
        ClusterBuilder cb{g, producers, consumers, absorbed, {}, {}, {}};
        std::unique_ptr<ASTNode> root = cb.build(node);
        const int size = (int)cb.members.size();
        if (size <= 1) {  // a lone node is not worth a fused kernel
            visited[index] = 1;
            continue;
        }
        auto fusion = std::make_shared<FusionAST>();
        fusion->root = std::move(root);
        fusion->input_ports = cb.inputs;
        fusion->output_port = node.id;
        fusion->dtype = g.execution_dtype;
        for (int m : cb.members) fusion->contained_node_ids.push_back(g.nodes[m]->id);

        auto fused = std::make_unique<GraphNode>();
        fused->id = node.id;
        fused->op = kFuseOp;
        fused->inputs = cb.inputs;
        fused->input_types = fusion_input_types(g, cb.inputs);
        fused->output_type = node.output_type;
        fused->fusion = std::move(fusion);
        fused->metadata[kFusedNodeCount] = size;
        g.nodes[index] = std::move(fused);
        visited[index] = 1;
        for (int m : cb.members)
            if (m != index) absorbed[m] = 1;
        st.clusters++;
        st.nodes_fused += size;
        st.nodes_removed += size - 1;
    }
    std::vector<std::unique_ptr<GraphNode>> kept;
    kept.reserve(n);
    for (int i = 0; i < n; i++)
        if (!absorbed[i]) kept.push_back(std::move(g.nodes[i]));
    g.nodes = std::move(kept);
    if (stats) *stats = st;
    return MFH_OK;
}

// ---- ConstantFold (optimizer/constant_fold.go:40-225) ------------------------

// math.Max / math.Min of Go: NaN wins, +0 > -0, then the ordinary order.
double go_max(double a, double b)
{
    if (std::isinf(a) && a > 0) return a;
    if (std::isinf(b) && b > 0) return b;
    if (std::isnan(a) || std::isnan(b)) return std::nan("");
    if (a == 0 && a == b) return std::signbit(a) ? b : a;
    return a > b ? a : b;
}

double go_min(double a, double b)
{
    if (std::isinf(a) && a < 0) return a;
    if (std::isinf(b) && b < 0) return b;
    if (std::isnan(a) || std::isnan(b)) return std::nan("");
    if (a == 0 && a == b) return std::signbit(a) ? a : b;
    return a < b ? a : b;
}

double bits_f64(uint64_t b)
{
    double d;
    std::memcpy(&d, &b, sizeof d);
    return d;
}

// evaluateUnary (optimizer/constant_fold.go:165-203), f64 throughout; the
// libm functions are the C library's (within an f64 ulp of Go's math).
bool evaluate_unary(int32_t type, double x, double* r)
{
    switch (type) {
    case kNodeNeg: *r = -x; return true;
    case kNodeAbs: *r = std::fabs(x); return true;
    case kNodeSqrt: *r = std::sqrt(x); return true;
    case kNodeExp: *r = std::exp(x); return true;
    case kNodeLog: *r = std::log(x); return true;
    case kNodeReLU: *r = x > 0 ? x : 0.0; return true;  // NaN and -0 fold to +0
    case kNodeSigmoid: *r = 1.0 / (1.0 + std::exp(-x)); return true;
    case kNodeTanh: *r = std::tanh(x); return true;
    case kNodeSilu: *r = x / (1.0 + std::exp(-x)); return true;
    case kNodeGelu: {
        // 2/pi as Go's constant arithmetic rounds it (exact, then to f64)
        const double inner = std::sqrt(bits_f64(0x3FE45F306DC9C883ull)) * (x + 0.044715 * x * x * x);
        *r = 0.5 * x * (1.0 + std::tanh(inner));
        return true;
    }
    case kNodeLeakyReLU: *r = x >= 0 ? x : 0.01 * x; return true;
    default: return false;
    }
}

// evaluateBinary (optimizer/constant_fold.go:205-225); x/0 is not folded.
bool evaluate_binary(int32_t type, double a, double b, double* r)
{
    switch (type) {
    case kNodeAdd: *r = a + b; return true;
    case kNodeSub: *r = a - b; return true;
    case kNodeMul: *r = a * b; return true;
    case kNodeDiv:
        if (b == 0) return false;
        *r = a / b;
        return true;
    case kNodeMax: *r = go_max(a, b); return true;
    case kNodeMin: *r = go_min(a, b); return true;
    default: return false;
    }
}

int constant_fold(Graph& g, int32_t* folded_out)
{
    int32_t folded = 0;
    std::unordered_map<std::string, double> values;
    for (const auto& node : g.nodes) {
        if (node->op != kConstantOp) continue;
        auto it = node->attributes.find(kConstantValue);
        if (it != node->attributes.end()) values[node->id] = it->second;
    }
    // One forward sweep: a node folds when every input is a known constant,
    // which chains through nodes folded earlier in the sweep.
    for (auto& node : g.nodes) {
        if (node->op == kConstantOp) continue;
        const int32_t type = elementwise_type(node->op);
        if (type == kNodeInvalid) continue;
        std::vector<double> operands;
        bool all = true;
        for (const std::string& name : node->inputs) {
            auto it = values.find(name);
            if (it == values.end()) {
                all = false;
                break;
            }
            operands.push_back(it->second);
        }
        if (!all) continue;
        double r = 0.0;
        bool ok = false;
        const int arity = node_arity(type);
        if (arity == 1 && operands.size() == 1) ok = evaluate_unary(type, operands[0], &r);
        if (arity == 2 && operands.size() == 2) ok = evaluate_binary(type, operands[0], operands[1], &r);
        if (!ok) continue;
        node->op = kConstantOp;
        node->inputs.clear();
        node->attributes[kConstantValue] = r;
        values[node->id] = r;
        folded++;
    }
    if (folded_out) *folded_out = folded;
    return MFH_OK;
}

// ---- EmitHIP for a fused node ------------------------------------------------

int flatten_checked(const ASTNode& n, std::vector<mfh_ast_node>& out)
{
    const int arity = node_arity(n.type);
    if (arity < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: unsupported node type %d", n.type);
    if ((int)n.children.size() != arity)
        return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: a node of type %d has %d children, its arity is %d",
                    n.type, (int)n.children.size(), arity);
    out.push_back(mfh_ast_node{n.type, n.input_index, n.value});
    for (const auto& c : n.children) MFH_TRY(flatten_checked(*c, out));
    return MFH_OK;
}

// The dtype a node's output is stored in: OutputType, else the FusionAST /
// graph execution dtype, else Float32 (CPUKernel's output, codegen/cpu.go:59).
int output_dtype(uint8_t output_type, uint8_t fallback, uint8_t* out)
{
    uint8_t dt = output_type != kInvalid ? output_type : fallback != kInvalid ? fallback : (uint8_t)kFloat32;
    if (!hip_storage(dt))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "codegen hip: output dtype %s is not Float32/Float16/BFloat16",
                    dtype_name(dt));
    *out = dt;
    return MFH_OK;
}

int emit_node_kernel(const ASTNode& root, const std::vector<std::string>& ports, const std::string& identifier,
                     const std::vector<uint8_t>& input_types, uint8_t out_dtype, uint32_t flags,
                     std::shared_ptr<HIPKernel>* out)
{
    auto k = std::make_shared<HIPKernel>();
    k->identifier = identifier;
    k->inputs = ports;
    k->out_dtype = out_dtype;
    k->flags = flags;
    MFH_TRY(flatten_checked(root, k->nodes));
    std::vector<mfh_operand> ops(ports.size());
    for (size_t i = 0; i < ports.size(); i++) {
        uint8_t dt = i < input_types.size() ? input_types[i] : (uint8_t)kInvalid;
        if (dt != kInvalid && !hip_storage(dt))
            return fail(MFH_ERR_DTYPE_UNSUPPORTED, "codegen hip: input %d (\"%s\") is %s; the HIP target reads "
                        "Float32, Float16 and BFloat16", (int)i, ports[i].c_str(), dtype_name(dt));
        k->declared.push_back(dt);
        ops[i] = mfh_operand{dt != kInvalid ? dt : (uint8_t)kFloat32, MFH_OPERAND_FULL, {0}, 0};
    }
    MFH_TRY(k->variant(ops, &k->full));
    *out = std::move(k);
    return MFH_OK;
}

int attach_kernels(Graph& g, const int32_t* targets, int32_t n_targets, uint32_t flags, int32_t* attached_out)
{
    int32_t attached = 0;
    auto done = [&](int rc) {
        if (attached_out) *attached_out = attached;
        return rc;
    };
    if (g.codegen_flags != flags)
        for (auto& node : g.nodes) node->solo.reset();
    g.codegen_flags = flags;
    std::vector<int32_t> ts;
    if (targets && n_targets > 0) ts.assign(targets, targets + n_targets);
    else ts.push_back(MFH_TARGET_HIP);
    for (auto& node : g.nodes) {
        if (!node || node->op != kFuseOp) continue;
        if (!node->fusion || !node->fusion->root)
            return done(fail(MFH_ERR_INVALID_ARGUMENT, "codegen: fused node \"%s\" missing \"%s\" attribute",
                             node->id.c_str(), kFuseAttributeAST));
        auto set = std::make_shared<KernelSet>();
        for (int32_t t : ts) {
            if (t != MFH_TARGET_HIP) continue;  // no CPU / Metal emitter in this library
            uint8_t odt;
            std::shared_ptr<HIPKernel> k;
            int rc = output_dtype(node->output_type, node->fusion->dtype, &odt);
            if (rc == MFH_OK)
                rc = emit_node_kernel(*node->fusion->root, node->fusion->input_ports, node->fusion->output_port,
                                      node->input_types, odt, flags, &k);
            if (rc != MFH_OK) {
                std::string msg = mfh_last_error();
                return done(fail(rc, "codegen: emit \"%s\": %s", node->id.c_str(), msg.c_str()));
            }
            set->kernels[t] = std::move(k);
        }
        node->kernels = std::move(set);
        attached++;
    }
    return done(MFH_OK);
}

// ---- execution ---------------------------------------------------------------

constexpr int64_t kAlign = 256;
int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct Slot {
    enum Kind { kInput, kConst, kArena, kBound } kind = kArena;
    void* ptr = nullptr;  // inputs and bound outputs
    int64_t offset = 0;   // arena / constant offset in the workspace
    uint8_t dtype = kFloat32;
    int64_t count = 0;
    int producer = -1;          // step that writes it
    std::vector<int> readers;   // steps that read it
    bool pinned = false;        // read by the output copies after the last step
    int out_index = -1;         // kBound: the output binding written in place
};

struct Step {
    HIPKernel* kernel = nullptr;
    const mfh_kernel* resolved = nullptr;  // kernel's variant for `ops`, once looked up
    int node = -1;  // graph node index
    std::vector<int> operands;
    std::vector<mfh_operand> ops;
    int result = -1;
    int64_t count = 0;
};

struct Copy {
    int slot;
    const mfh_value* to;
    int to_index;  // of `to` in the call's output bindings
};

// A call's values and launches, before placement and streams.
struct Prepared {
    std::vector<Slot> slots;
    std::vector<Step> steps;
    std::vector<Copy> copies;
    std::vector<float> constants;
    std::vector<int> node_slot;   // graph node -> the slot it defines
    std::vector<int> input_slot;  // graph input -> its slot, -1 when unbound
};

int operand_mode(int64_t c, int64_t n, mfh_operand* op)
{
    if (c == n) op->mode = MFH_OPERAND_FULL;
    else if (c == 1) op->mode = MFH_OPERAND_SCALAR;
    else if (c > 1 && n % c == 0) {
        op->mode = MFH_OPERAND_PERIODIC;
        op->period = c;
    } else
        return MFH_ERR_SHAPE_MISMATCH;
    return MFH_OK;
}

// Binds inputs and outputs and lowers every node to a launch.  With
// `shapes_only` the values' data pointers are not needed (planning); without
// `may_compile` an unfused node whose one-node kernel was never generated is
// an error instead of a compile, except with `shapes_only`, where such a node
// keeps a null kernel and takes the dtype its kernel would produce (a shape
// query, which needs no device).
int prepare(Graph& g, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs, int32_t n_outputs,
            bool shapes_only, Prepared* P, bool may_compile = true)
{
    if ((n_inputs > 0 && !inputs) || (n_outputs > 0 && !outputs) || n_inputs < 0 || n_outputs < 0)
        return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: bad value list");
    std::vector<Slot>& slots = P->slots;
    std::unordered_map<std::string, int> named;  // value name -> latest slot
    std::set<std::string> graph_inputs(g.inputs.begin(), g.inputs.end());
    for (int32_t i = 0; i < n_inputs; i++) {
        const mfh_value& v = inputs[i];
        std::string name = v.name ? v.name : "";
        if (!graph_inputs.count(name)) return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: unknown input \"%s\"", name.c_str());
        if (named.count(name)) return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: input \"%s\" bound twice", name.c_str());
        if (!hip_storage(v.dtype))
            return fail(MFH_ERR_DTYPE_UNSUPPORTED, "graph call: input \"%s\" is %s; values are Float32/Float16/BFloat16",
                        name.c_str(), dtype_name(v.dtype));
        if (v.count < 0 || (!shapes_only && v.count > 0 && !v.data))
            return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: input \"%s\" has no data", name.c_str());
        Slot s;
        s.kind = Slot::kInput;
        s.ptr = v.data;
        s.dtype = v.dtype;
        s.count = v.count;
        named[name] = (int)slots.size();
        slots.push_back(s);
    }
    P->input_slot.assign(g.inputs.size(), -1);
    for (size_t k = 0; k < g.inputs.size(); k++) {
        auto it = named.find(g.inputs[k]);
        if (it != named.end()) P->input_slot[k] = it->second;
    }
    // Output bindings by value name.
    std::multimap<std::string, const mfh_value*> bound;
    for (int32_t i = 0; i < n_outputs; i++) {
        std::string key = outputs[i].name ? outputs[i].name : "";
        auto it = std::find_if(g.outputs.begin(), g.outputs.end(), [&](const auto& kv) { return kv.first == key; });
        if (it == g.outputs.end()) return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: unknown output \"%s\"", key.c_str());
        bound.emplace(it->second, &outputs[i]);
    }
    std::unordered_map<std::string, int> last_def;
    for (int i = 0; i < (int)g.nodes.size(); i++) last_def[g.nodes[i]->id] = i;

    P->node_slot.assign(g.nodes.size(), -1);
    for (int i = 0; i < (int)g.nodes.size(); i++) {
        GraphNode& node = *g.nodes[i];
        if (node.op == kConstantOp) {
            auto it = node.attributes.find(kConstantValue);
            if (it == node.attributes.end())
                return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: constant \"%s\" has no value", node.id.c_str());
            Slot s;
            s.kind = Slot::kConst;
            s.offset = (int64_t)P->constants.size() * 4;
            s.count = 1;
            P->constants.push_back((float)it->second);  // fl32(Value), codegen/cpu.go:130-131
            named[node.id] = P->node_slot[i] = (int)slots.size();
            slots.push_back(s);
            continue;
        }
        HIPKernel* kernel = nullptr;
        if (node.op == kFuseOp) {
            kernel = node.kernels ? node.kernels->For(MFH_TARGET_HIP) : nullptr;
            if (!kernel)
                return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: fused node \"%s\" has no HIP kernel attached",
                            node.id.c_str());
            if (kernel->inputs.size() != node.inputs.size())
                return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: fused node \"%s\" has %d inputs, its kernel %d",
                            node.id.c_str(), (int)node.inputs.size(), (int)kernel->inputs.size());
        } else if (int32_t type = elementwise_type(node.op); type && !node.solo && shapes_only && !may_compile) {
            if ((int)node.inputs.size() != node_arity(type))
                return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: node \"%s\" (%s) has %d inputs, want %d",
                            node.id.c_str(), node.op.c_str(), (int)node.inputs.size(), node_arity(type));
        } else if (int32_t type = elementwise_type(node.op)) {
            if (!node.solo && !may_compile)
                return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: node \"%s\" has no kernel yet (make one "
                            "mfh_graph_call with these values first)", node.id.c_str());
            if (!node.solo) {
                if ((int)node.inputs.size() != node_arity(type))
                    return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: node \"%s\" (%s) has %d inputs, want %d",
                                node.id.c_str(), node.op.c_str(), (int)node.inputs.size(), node_arity(type));
                ASTNode root;
                root.type = type;
                for (size_t k = 0; k < node.inputs.size(); k++) root.children.push_back(input_leaf((int)k));
                uint8_t odt;
                MFH_TRY(output_dtype(node.output_type, g.execution_dtype, &odt));
                MFH_TRY(emit_node_kernel(root, node.inputs, node.id, node.input_types, odt, g.codegen_flags,
                                         &node.solo));
            }
            kernel = node.solo.get();
        } else {
            return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: node \"%s\": op \"%s\" has no HIP lowering",
                        node.id.c_str(), node.op.c_str());
        }
        const int t = (int)P->steps.size();
        Step st;
        st.kernel = kernel;
        st.node = i;
        for (const std::string& name : node.inputs) {
            auto it = named.find(name);
            if (it == named.end())
                return fail(MFH_ERR_INVALID_ARGUMENT,
                            "graph call: node \"%s\" reads \"%s\", which is neither a bound input nor an earlier node",
                            node.id.c_str(), name.c_str());
            st.operands.push_back(it->second);
            st.count = std::max(st.count, slots[it->second].count);
        }
        for (size_t k = 0; k < st.operands.size(); k++) {
            Slot& s = slots[st.operands[k]];
            mfh_operand op{s.dtype, MFH_OPERAND_FULL, {0}, 0};
            if (operand_mode(s.count, st.count, &op) != MFH_OK)
                return fail(MFH_ERR_SHAPE_MISMATCH, "graph call: node \"%s\": operand \"%s\" has %lld elements, "
                            "the node %lld", node.id.c_str(), node.inputs[k].c_str(), (long long)s.count,
                            (long long)st.count);
            if (kernel && k < kernel->declared.size() && kernel->declared[k] != kInvalid &&
                kernel->declared[k] != s.dtype)
                return fail(MFH_ERR_DTYPE_UNSUPPORTED, "graph call: node \"%s\": operand \"%s\" is %s, declared %s",
                            node.id.c_str(), node.inputs[k].c_str(), dtype_name(s.dtype),
                            dtype_name(kernel->declared[k]));
            st.ops.push_back(op);
            s.readers.push_back(t);
        }
        Slot out;
        if (kernel) out.dtype = kernel->out_dtype;
        else MFH_TRY(output_dtype(node.output_type, g.execution_dtype, &out.dtype));
        out.count = st.count;
        out.kind = Slot::kArena;
        out.producer = t;
        // The node that finally defines a bound output writes straight into
        // the caller's buffer when it matches.
        auto range = bound.equal_range(node.id);
        if (last_def[node.id] == i && range.first != range.second) {
            const mfh_value* b = range.first->second;
            if (b->dtype == out.dtype && b->count == out.count && b->data) {
                out.kind = Slot::kBound;
                out.ptr = b->data;
                out.out_index = (int)(b - outputs);
            }
        }
        st.result = (int)slots.size();
        named[node.id] = P->node_slot[i] = st.result;
        slots.push_back(out);
        P->steps.push_back(std::move(st));
    }
    // An output buffer that overlaps an input's is written in place only
    // where nothing can read a changed input: the input is the same buffer
    // with the same element size and count, and its one reader is the
    // launch that writes the output, element for element.  Otherwise the
    // output goes through the workspace and is copied out after every
    // launch.
    std::set<int> passed_through;  // input slots copied straight to an output
    for (const auto& kv : bound) {
        auto it = named.find(kv.first);
        if (it != named.end() && slots[it->second].kind == Slot::kInput) passed_through.insert(it->second);
    }
    for (Slot& s : slots) {
        if (s.kind != Slot::kBound) continue;
        const uintptr_t lo = (uintptr_t)s.ptr, hi = lo + (uintptr_t)s.count * dtype_size(s.dtype);
        for (int j = 0; j < n_inputs; j++) {
            const Slot& in = slots[j];  // inputs come first
            const uintptr_t l = (uintptr_t)in.ptr, h = l + (uintptr_t)in.count * dtype_size(in.dtype);
            if (!in.ptr || in.count <= 0 || h <= lo || hi <= l) continue;
            const bool same = in.ptr == s.ptr && dtype_size(in.dtype) == dtype_size(s.dtype) && in.count == s.count &&
                              !passed_through.count(j) &&
                              std::all_of(in.readers.begin(), in.readers.end(), [&](int r) { return r == s.producer; });
            if (!same) {
                s.kind = Slot::kArena;
                s.ptr = nullptr;
                s.out_index = -1;
                break;
            }
        }
    }
    // Bound outputs not written in place are copied at the end.
    for (const auto& kv : bound) {
        auto it = named.find(kv.first);
        if (it == named.end())
            return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: output value \"%s\" is never defined", kv.first.c_str());
        Slot& s = slots[it->second];
        const mfh_value* b = kv.second;
        if (b->dtype != s.dtype || b->count != s.count)
            return fail(b->dtype != s.dtype ? MFH_ERR_DTYPE_UNSUPPORTED : MFH_ERR_SHAPE_MISMATCH,
                        "graph call: output \"%s\" holds %s[%lld]; value \"%s\" is %s[%lld]", b->name,
                        dtype_name(b->dtype), (long long)b->count, kv.first.c_str(), dtype_name(s.dtype),
                        (long long)s.count);
        if (s.count > 0 && !b->data)
            return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: output \"%s\" has no data", b->name);
        if (s.kind == Slot::kBound && s.ptr == b->data) continue;
        s.pinned = true;
        P->copies.push_back(Copy{it->second, b, (int)(b - outputs)});
    }
    // inputs passed straight through are copied before anything else is
    // written into an output buffer
    std::stable_partition(P->copies.begin(), P->copies.end(),
                          [&](const Copy& c) { return slots[c.slot].kind == Slot::kInput; });
    return MFH_OK;
}

// The launches as planning nodes: one per step, reading its operands' slots
// and writing its result's.  Constants and graph inputs have no producer, so
// they order nothing.
Topology launch_topology(const Graph& g, const Prepared& P)
{
    Topology t;
    t.ports.resize(P.slots.size());
    for (const Step& st : P.steps) {
        PlanNode n;
        n.name = g.nodes[st.node]->id;
        n.inputs.assign(st.operands.begin(), st.operands.end());
        n.outputs.push_back(st.result);
        t.nodes.push_back(std::move(n));
    }
    return t;
}

int graph_streams(Graph& g, int n_streams, int n_events)
{
    while ((int)g.aux.size() < n_streams - 1) {
        hipStream_t s;
        MFH_TRY(check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags(graph stream)"));
        g.aux.push_back(s);
        hipEvent_t e;
        MFH_TRY(check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags"));
        g.joins.push_back(e);
    }
    while ((int)g.events.size() < n_events) {
        hipEvent_t e;
        MFH_TRY(check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags"));
        g.events.push_back(e);
    }
    if (!g.fork) MFH_TRY(check_hip(hipEventCreateWithFlags(&g.fork, hipEventDisableTiming), "hipEventCreateWithFlags"));
    for (hipEvent_t& e : g.done_ring)
        if (!e) MFH_TRY(check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags"));
    return MFH_OK;
}

// The node that the last launch on a capturing stream added to the capture
// (nullptr if the stream is not capturing or has no single last node).
hipGraphNode_t captured_node(hipStream_t s)
{
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    hipGraph_t graph = nullptr;
    const hipGraphNode_t* deps = nullptr;
    size_t n = 0;
    if (hipStreamGetCaptureInfo_v2(s, &status, &id, &graph, &deps, &n) != hipSuccess ||
        status != hipStreamCaptureStatusActive || n != 1 || !deps)
        return nullptr;
    return deps[0];
}

// The launches of one call on `ls` and the graph's other streams: fork from
// `ls`, every node with its waits and signals, join back into `ls`, then the
// output copies.  With `ls` capturing, this records the call as a graph, and
// `nodes` (if given) receives each step's node and then each copy's, nullptr
// where nothing was launched or copied.
int launch_all(Graph& g, Prepared& P, const Topology& topo, int n_streams, hipStream_t ls, void* workspace,
               bool may_load = true, std::vector<hipGraphNode_t>* nodes = nullptr)
{
    std::vector<Slot>& slots = P.slots;
    if (n_streams > 1) {
        MFH_TRY(check_hip(hipEventRecord(g.fork, ls), "hipEventRecord(fork)"));
        for (int s = 1; s < n_streams; s++)
            MFH_TRY(check_hip(hipStreamWaitEvent(g.aux[s - 1], g.fork, 0), "hipStreamWaitEvent(fork)"));
    }
    char* base = static_cast<char*>(workspace);
    auto addr = [&](const Slot& s) -> void* {
        return s.kind == Slot::kInput || s.kind == Slot::kBound ? s.ptr : base + s.offset;
    };
    auto on = [&](int32_t id) { return id == 0 ? ls : g.aux[id - 1]; };
    std::vector<const void*> ptrs;
    for (size_t t = 0; t < P.steps.size(); t++) {
        Step& st = P.steps[t];
        const PlanNode& pn = topo.nodes[t];
        hipStream_t s = on(pn.stream);
        for (const mfh_sync_event& e : pn.barriers)
            if (e.wait) MFH_TRY(check_hip(hipStreamWaitEvent(s, g.events[e.event_id], 0), "hipStreamWaitEvent(barrier)"));
        const mfh_kernel* k = st.resolved;
        if (!k) {
            if (may_load) MFH_TRY(st.kernel->variant(st.ops, &k));
            else if (!(k = st.kernel->find(st.ops)))
                return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: node \"%s\" has no kernel for these operands "
                            "yet (make one mfh_graph_call with these values first)", g.nodes[st.node]->id.c_str());
            st.resolved = k;  // variants are never dropped while the graph keeps this plan
        }
        ptrs.clear();
        for (int o : st.operands) ptrs.push_back(addr(slots[o]));
        MFH_TRY(run_hip(k, ptrs.data(), (int)ptrs.size(), addr(slots[st.result]), st.count, s, may_load));
        if (nodes) nodes->push_back(st.count > 0 ? captured_node(s) : nullptr);
        for (const mfh_sync_event& e : pn.barriers)
            if (!e.wait) MFH_TRY(check_hip(hipEventRecord(g.events[e.event_id], s), "hipEventRecord(barrier)"));
    }
    for (int s = 1; s < n_streams; s++) {
        MFH_TRY(check_hip(hipEventRecord(g.joins[s - 1], g.aux[s - 1]), "hipEventRecord(join)"));
        MFH_TRY(check_hip(hipStreamWaitEvent(ls, g.joins[s - 1], 0), "hipStreamWaitEvent(join)"));
    }
    for (const Copy& c : P.copies) {
        const Slot& s = slots[c.slot];
        const size_t bytes = (size_t)s.count * dtype_size(s.dtype);
        if (bytes)
            MFH_TRY(check_hip(hipMemcpyAsync(c.to->data, addr(s), bytes, hipMemcpyDeviceToDevice, ls),
                              "hipMemcpyAsync(graph output)"));
        if (nodes) nodes->push_back(bytes ? captured_node(ls) : nullptr);
    }
    return MFH_OK;
}

// Places a call's values in its workspace and returns the bytes it needs:
// constants first, then the intermediates, placed so that a region is reused
// only after every launch touching its previous value is ordered before the
// new writer.  A step's result never shares memory with its operands, and a
// value copied out at the end is kept to the end.
int64_t lay_out(Prepared& P, const Topology& topo)
{
    std::vector<Slot>& slots = P.slots;
    const int64_t const_bytes = align_up((int64_t)P.constants.size() * 4);
    std::vector<OrderedValue> values;
    std::vector<int> value_slot;
    for (int i = 0; i < (int)slots.size(); i++) {
        const Slot& s = slots[i];
        if (s.kind != Slot::kArena) continue;
        OrderedValue v;
        v.producer = s.producer;
        v.users = s.readers;
        if (s.pinned) v.users.push_back(kPinned);
        v.size = std::max<int64_t>(1, s.count) * dtype_size(s.dtype);
        values.push_back(std::move(v));
        value_slot.push_back(i);
    }
    const int64_t arena = place_ordered(values, order_of(topo.nodes), kAlign);
    for (size_t k = 0; k < values.size(); k++) slots[value_slot[k]].offset = const_bytes + values[k].offset;
    return const_bytes + arena;
}

struct PlannedCall {
    std::string key;
    Prepared P;
    Topology topo;
    int n_streams = 1, n_events = 0;
    int64_t need = 0;
    uint64_t tick = 0;
    // Replay.  The plan's second call is captured as a HIP graph; later calls
    // launch it, with the arguments of the launches whose buffers differ from
    // those an executable was last bound to updated in place.  Two
    // executables take turns, so that one whose last launch may still be
    // running is never updated.
    int calls = 0;
    hipGraph_t graph = nullptr;
    std::vector<hipGraphNode_t> step_node;  // per step; nullptr: nothing launched
    std::vector<hipKernelNodeParams> step_params;
    std::vector<hipGraphNode_t> copy_node;  // per copy; nullptr: nothing copied
    struct Exec {
        hipGraphExec_t exec = nullptr;
        bool launched = false;
        uint64_t last_call = 0;           // the graph call that launched it last
        std::vector<const void*> bound;  // the addresses its nodes hold (call_addresses)
    };
    Exec execs[2];
    int turn = 0;
    std::vector<const void*> captured;  // the addresses the graph was captured with
    std::vector<size_t> addr_at;        // where each step's, then each copy's, addresses start
    std::vector<const void*> cur;       // this call's addresses
};

// Frees a plan's captured graph and executables; the caller has waited for
// their launches.
void release_replay(PlannedCall& p)
{
    for (PlannedCall::Exec& e : p.execs) {
        if (e.exec) (void)hipGraphExecDestroy(e.exec);
        e = PlannedCall::Exec{};
    }
    if (p.graph) (void)hipGraphDestroy(p.graph);
    p.graph = nullptr;
    p.step_node.clear();
    p.step_params.clear();
    p.copy_node.clear();
    p.captured.clear();
    p.calls = 0;
    p.turn = 0;
}

// The addresses each launch and output copy of a planned call reads and
// writes, into p.cur: per step its operands then its result, per copy its
// destination and source; p.addr_at[i] is where entry i starts.
void call_addresses(PlannedCall& p, void* workspace)
{
    const Prepared& P = p.P;
    char* base = static_cast<char*>(workspace);
    auto addr = [&](const Slot& s) -> const void* {
        return s.kind == Slot::kInput || s.kind == Slot::kBound ? s.ptr : base + s.offset;
    };
    const bool first = p.addr_at.empty();
    p.cur.clear();
    for (const Step& st : P.steps) {
        if (first) p.addr_at.push_back(p.cur.size());
        for (int o : st.operands) p.cur.push_back(addr(P.slots[o]));
        p.cur.push_back(addr(P.slots[st.result]));
    }
    for (const Copy& c : P.copies) {
        if (first) p.addr_at.push_back(p.cur.size());
        p.cur.push_back(c.to->data);
        p.cur.push_back(addr(P.slots[c.slot]));
    }
    if (first) p.addr_at.push_back(p.cur.size());
}

// What a call's plan depends on besides the graph: value names, dtypes and
// counts, which bindings have data, which output bindings share a buffer,
// which inputs each output's buffer overlaps, the stream budget.  Not the
// pointers: a call on new buffers of the same shapes reuses the plan with
// its pointers rebound.
std::string plan_key(const Graph& g, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs,
                     int32_t n_outputs)
{
    std::string key;
    char buf[64];
    for (int32_t i = 0; i < n_inputs; i++) {
        key += inputs[i].name ? inputs[i].name : "";
        snprintf(buf, sizeof buf, "|%u|%lld|%d;", (unsigned)inputs[i].dtype, (long long)inputs[i].count,
                 inputs[i].data != nullptr);
        key += buf;
    }
    key += "->";
    for (int32_t i = 0; i < n_outputs; i++) {
        int alias = i;  // the first binding with the same buffer
        for (int32_t j = 0; j < i; j++)
            if (outputs[j].data == outputs[i].data) {
                alias = j;
                break;
            }
        key += outputs[i].name ? outputs[i].name : "";
        snprintf(buf, sizeof buf, "|%u|%lld|%d|%d", (unsigned)outputs[i].dtype, (long long)outputs[i].count,
                 outputs[i].data != nullptr, alias);
        key += buf;
        // the inputs whose buffers it overlaps, and whether exactly
        const mfh_value& o = outputs[i];
        const uintptr_t lo = (uintptr_t)o.data, hi = lo + (uintptr_t)std::max<int64_t>(0, o.count) * dtype_size(o.dtype);
        for (int32_t j = 0; j < n_inputs; j++) {
            const mfh_value& v = inputs[j];
            const uintptr_t l = (uintptr_t)v.data, h = l + (uintptr_t)std::max<int64_t>(0, v.count) * dtype_size(v.dtype);
            if (!o.data || !v.data || h <= lo || hi <= l) continue;
            const bool same = v.data == o.data && v.count == o.count && dtype_size(v.dtype) == dtype_size(o.dtype);
            snprintf(buf, sizeof buf, "/%d%c", (int)j, same ? '=' : '~');
            key += buf;
        }
        key += ";";
    }
    snprintf(buf, sizeof buf, "s=%d", (int)g.max_streams);
    return key + buf;
}

// Points a cached plan at this call's buffers.
void rebind(Prepared& P, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs)
{
    for (int32_t i = 0; i < n_inputs; i++) P.slots[i].ptr = inputs[i].data;  // prepare() puts inputs first
    for (Slot& s : P.slots)
        if (s.kind == Slot::kBound) s.ptr = outputs[s.out_index].data;
    for (Copy& c : P.copies) c.to = &outputs[c.to_index];
}

// The plan of a call: prepared, scheduled and laid out on its signature's
// first call, rebound to the call's buffers after that.  Prepare, stream
// scheduling and placement took about a third of a plain call's host time.
int plan_call(Graph& g, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs, int32_t n_outputs,
              PlannedCall** out)
{
    const std::string key = plan_key(g, inputs, n_inputs, outputs, n_outputs);
    for (auto& p : g.plans)
        if (p->key == key) {
            rebind(p->P, inputs, n_inputs, outputs);
            p->tick = ++g.plan_clock;
            *out = p.get();
            return MFH_OK;
        }
    auto p = std::make_unique<PlannedCall>();
    MFH_TRY(prepare(g, inputs, n_inputs, outputs, n_outputs, false, &p->P));
    p->topo = launch_topology(g, p->P);
    MFH_TRY(schedule_streams(p->topo, g.max_streams));
    for (const PlanNode& n : p->topo.nodes) {
        p->n_streams = std::max(p->n_streams, n.stream + 1);
        for (const mfh_sync_event& e : n.barriers) p->n_events = std::max(p->n_events, e.event_id + 1);
    }
    p->need = lay_out(p->P, p->topo);
    p->key = key;
    p->tick = ++g.plan_clock;
    if ((int)g.plans.size() >= kMaxPlans) {
        // forget the least recently used plan, after the launches of its graph
        auto old = std::min_element(g.plans.begin(), g.plans.end(),
                                    [](const auto& a, const auto& b) { return a->tick < b->tick; });
        if ((*old)->graph && g.done) (void)hipEventSynchronize(g.done);
        release_replay(**old);
        g.plans.erase(old);
    }
    g.plans.push_back(std::move(p));
    *out = g.plans.back().get();
    return MFH_OK;
}

// Waits for the last call, then drops every captured call.
void drop_replays(Graph& g)
{
    bool any = false;
    for (const auto& p : g.plans) any = any || p->graph;
    if (any && g.done) (void)hipEventSynchronize(g.done);
    for (auto& p : g.plans) release_replay(*p);
}

// Points executable `e` of plan `p` at the addresses `cur`: the launches and
// copies whose addresses differ from those it holds get new arguments (the
// launch shape run_hip would choose for them: the vector path depends on
// alignment).  `e` must have no launch still running.
int bind_exec(PlannedCall& p, PlannedCall::Exec& e)
{
    const std::vector<const void*>& cur = p.cur;
    auto same = [&](size_t i) {
        return std::equal(cur.begin() + (long)p.addr_at[i], cur.begin() + (long)p.addr_at[i + 1],
                          e.bound.begin() + (long)p.addr_at[i]);
    };
    const size_t ns = p.P.steps.size();
    for (size_t t = 0; t < ns; t++) {
        if (!p.step_node[t] || same(t)) continue;
        const Step& st = p.P.steps[t];
        const void* const* a = cur.data() + p.addr_at[t];
        const int n_in = (int)(p.addr_at[t + 1] - p.addr_at[t]) - 1;
        HipLaunch l;
        MFH_TRY(prepare_hip(st.resolved, a, n_in, const_cast<void*>(a[n_in]), st.count, true, &l));
        l.bind();
        hipKernelNodeParams kp = p.step_params[t];
        kp.gridDim = dim3(l.grid);
        kp.blockDim = dim3(l.block);
        kp.kernelParams = l.args.data();
        kp.extra = nullptr;
        MFH_TRY(check_hip(hipGraphExecKernelNodeSetParams(e.exec, p.step_node[t], &kp),
                          "hipGraphExecKernelNodeSetParams(graph call)"));
    }
    for (size_t c = 0; c < p.P.copies.size(); c++) {
        const size_t i = ns + c;
        if (!p.copy_node[c] || same(i)) continue;
        const Slot& sl = p.P.slots[p.P.copies[c].slot];
        const void* const* a = cur.data() + p.addr_at[i];
        MFH_TRY(check_hip(hipGraphExecMemcpyNodeSetParams1D(e.exec, p.copy_node[c], const_cast<void*>(a[0]), a[1],
                                                            (size_t)sl.count * dtype_size(sl.dtype),
                                                            hipMemcpyDeviceToDevice),
                          "hipGraphExecMemcpyNodeSetParams1D(graph call)"));
    }
    e.bound = cur;
    return MFH_OK;
}

// Launches plan `p`'s captured graph for this call's buffers: an executable
// already bound to them, else the next one in turn, once its last launch has
// finished, bound to them.  A plan on several streams is not rebound (its
// rebinding and graph launch took more host time than its plain launches:
// 185 against 163 us for 32 nodes on four streams); such a call sets
// `launched` false and runs as plain launches.
int replay_call(Graph& g, PlannedCall& p, hipStream_t stream, bool* launched)
{
    *launched = false;
    call_addresses(p, g.ws);
    PlannedCall::Exec* e = nullptr;
    for (PlannedCall::Exec& x : p.execs)
        if (x.exec && x.bound == p.cur) e = &x;
    if (!e && p.n_streams > 1) return MFH_OK;
    if (!e) {
        e = &p.execs[p.turn];
        p.turn ^= 1;
        if (!e->exec) {
            MFH_TRY(check_hip(hipGraphInstantiate(&e->exec, p.graph, nullptr, nullptr, 0),
                              "hipGraphInstantiate(graph call)"));
            e->bound = p.captured;
        } else if (e->launched) {
            // its last call's event, or a later call's in the same ring slot
            MFH_TRY(check_hip(hipEventSynchronize(g.done_ring[e->last_call % Graph::kDoneRing]),
                              "hipEventSynchronize(graph call replay)"));
        }
        MFH_TRY(bind_exec(p, *e));
    }
    MFH_TRY(check_hip(hipGraphLaunch(e->exec, stream), "hipGraphLaunch(graph call)"));
    e->launched = true;
    e->last_call = g.call_seq;
    *launched = true;
    return MFH_OK;
}

// Captures this call's launches on the graph's capture stream as plan `p`'s
// graph and launches it on `stream`.  Returns false (nothing launched) where
// capture is not available or a launch's node cannot be told apart.
bool capture_call(Graph& g, PlannedCall& p, hipStream_t stream)
{
    if (!g.capture && hipStreamCreateWithFlags(&g.capture, hipStreamNonBlocking) != hipSuccess) return false;
    if (hipStreamBeginCapture(g.capture, hipStreamCaptureModeThreadLocal) != hipSuccess) return false;
    std::vector<hipGraphNode_t> nodes;
    const int rc = launch_all(g, p.P, p.topo, p.n_streams, g.capture, g.ws, true, &nodes);
    hipGraph_t graph = nullptr;
    const hipError_t end = hipStreamEndCapture(g.capture, &graph);
    const size_t ns = p.P.steps.size();
    bool ok = rc == MFH_OK && end == hipSuccess && graph && nodes.size() == ns + p.P.copies.size();
    std::vector<hipKernelNodeParams> params(ns);
    for (size_t i = 0; ok && i < nodes.size(); i++) {
        if (i < ns) {
            if (p.P.steps[i].count > 0)
                ok = nodes[i] && hipGraphKernelNodeGetParams(nodes[i], &params[i]) == hipSuccess;
        } else {
            const Slot& sl = p.P.slots[p.P.copies[i - ns].slot];
            if (sl.count > 0) ok = nodes[i] != nullptr;
        }
    }
    // Everything that can fail comes before the launch: a call that falls
    // back to plain launches must not have run already.
    hipGraphExec_t exec = nullptr;
    if (ok && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) ok = false;
    if (ok && hipGraphLaunch(exec, stream) != hipSuccess) ok = false;
    if (!ok) {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipGetLastError();
        return false;
    }
    p.graph = graph;
    p.step_node.assign(nodes.begin(), nodes.begin() + (long)ns);
    p.copy_node.assign(nodes.begin() + (long)ns, nodes.end());
    p.step_params = std::move(params);
    call_addresses(p, g.ws);
    p.captured = p.cur;
    p.execs[0].exec = exec;
    p.execs[0].bound = p.captured;
    p.execs[0].launched = true;
    p.execs[0].last_call = g.call_seq;
    p.turn = 1;
    return true;
}

// A change to the graph: every captured call and every plan goes.
void forget_calls(Graph& g)
{
    drop_replays(g);
    g.plans.clear();
}

int graph_call(Graph& g, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs, int32_t n_outputs,
               hipStream_t stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (g.replay_generation != module_generation()) {
        // captured calls hold function handles of unloaded modules
        drop_replays(g);
        g.replay_generation = module_generation();
    }

    // A call the caller is capturing runs as plain launches into their graph.
    hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
    MFH_TRY(check_hip(hipStreamIsCapturing(stream, &capturing), "hipStreamIsCapturing"));
    const bool captured = capturing != hipStreamCaptureStatusNone;
    const bool replayable = g.replay && !g.replay_broken && !captured;

    // Launches, streams (ScheduleStreams over the launches,
    // ir/stream_scheduler.go:56) and placement, planned once per signature
    // and rebound to this call's buffers.
    PlannedCall* plan = nullptr;
    MFH_TRY(plan_call(g, inputs, n_inputs, outputs, n_outputs, &plan));
    Prepared& P = plan->P;
    const Topology& topo = plan->topo;
    const int n_streams = plan->n_streams, n_events = plan->n_events;
    const int64_t need = plan->need;
    if (need > g.ws_bytes && captured)
        return fail(MFH_ERR_INVALID_ARGUMENT,
                    "graph call: the workspace must grow to %lld bytes while the caller's stream is being captured; "
                    "make the same call once before capturing", (long long)need);
    if (need > g.ws_bytes) {
        // captured calls address the old workspace
        drop_replays(g);
        if (g.ws) {
            // the previous workspace may still be read by queued work
            MFH_TRY(check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"));
            MFH_TRY(check_hip(hipFree(g.ws), "hipFree"));
            g.ws = nullptr;
            g.ws_bytes = 0;
        }
        MFH_TRY(check_hip(hipMalloc(&g.ws, (size_t)need), "hipMalloc(graph workspace)"));
        g.ws_bytes = need;
        g.ws_constants_valid = false;
    }
    MFH_TRY(graph_streams(g, n_streams, n_events));
    // The workspace is shared by every call: work on a new caller stream
    // waits for the previous call to finish with it.  (A capturing caller
    // orders its capture itself.)
    if (!captured && g.called && g.last_stream != stream)
        MFH_TRY(check_hip(hipStreamWaitEvent(stream, g.done, 0), "hipStreamWaitEvent(previous call)"));
    const bool new_constants = !P.constants.empty() && (!g.ws_constants_valid || g.ws_constants != P.constants);
    if (new_constants && captured)
        return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: the graph's constants must be uploaded while the caller's "
                    "stream is being captured; make the same call once before capturing");
    if (new_constants) {
        g.ws_constants = P.constants;
        MFH_TRY(check_hip(hipMemcpyAsync(g.ws, g.ws_constants.data(), P.constants.size() * 4, hipMemcpyHostToDevice,
                                         stream), "hipMemcpyAsync(graph constants)"));
        g.ws_constants_valid = true;
    }

    // A plan's first call runs as plain launches (and loads every kernel it
    // needs); its second is captured as a HIP graph, and later calls launch
    // that graph, bound to their buffers.
    bool launched = false;
    if (replayable && plan->graph) {
        MFH_TRY(replay_call(g, *plan, stream, &launched));
        if (launched) g.replayed++;
    } else if (replayable && plan->calls >= 1) {
        launched = capture_call(g, *plan, stream);
        // capture is not available here: this call and later ones run as
        // plain launches
        if (!launched) g.replay_broken = true;
    }
    if (!launched) MFH_TRY(launch_all(g, P, topo, n_streams, stream, g.ws));
    g.streams_used = n_streams;
    if (captured) return MFH_OK;
    plan->calls++;
    hipEvent_t done = g.done_ring[g.call_seq % Graph::kDoneRing];
    MFH_TRY(check_hip(hipEventRecord(done, stream), "hipEventRecord(call done)"));
    g.done = done;
    g.call_seq++;
    g.last_stream = stream;
    g.called = true;
    return MFH_OK;
}

// mfh_graph_call on the caller's stream alone, with the call's constants and
// intermediates in the static device scratch, and nothing compiled, loaded
// or allocated.
int graph_call_noalloc(Graph& g, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs,
                       int32_t n_outputs, hipStream_t stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    void* base = nullptr;
    MFH_TRY(scratch_address(dev->ordinal, &base));
    Prepared P;
    MFH_TRY(prepare(g, inputs, n_inputs, outputs, n_outputs, false, &P, false));
    Topology topo = launch_topology(g, P);
    MFH_TRY(schedule_streams(topo, 1));
    for (const PlanNode& n : topo.nodes)
        if (n.stream != 0 || !n.barriers.empty())
            return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: node \"%s\" was scheduled off the caller's stream",
                        n.name.c_str());
    const int64_t need = lay_out(P, topo);
    if (need > (int64_t)MFH_GRAPH_SCRATCH_BYTES)
        return fail(MFH_ERR_INVALID_ARGUMENT, "graph call (no allocation): the call needs %lld bytes of scratch, "
                    "the static scratch holds %lld", (long long)need, (long long)MFH_GRAPH_SCRATCH_BYTES);
    // Every kernel must be loaded already; checked before anything is queued.
    for (const Step& st : P.steps)
        if (!st.kernel->find(st.ops))
            return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: node \"%s\" has no kernel for these operands yet "
                        "(make one mfh_graph_call with these values first)", g.nodes[st.node]->id.c_str());
    if (!P.constants.empty())
        MFH_TRY(put_constants(static_cast<float*>(base), P.constants.data(), (int64_t)P.constants.size(), stream));
    return launch_all(g, P, topo, 1, stream, base, false);
}

// The dtype and element count a call with these inputs gives output `key`,
// by prepare()'s rules, from the inputs' names, dtypes and counts alone.
int output_shape(Graph& g, const mfh_value* inputs, int32_t n_inputs, const std::string& key, uint8_t* dtype,
                 int64_t* count)
{
    auto it = std::find_if(g.outputs.begin(), g.outputs.end(), [&](const auto& kv) { return kv.first == key; });
    if (it == g.outputs.end()) return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: unknown output \"%s\"", key.c_str());
    Prepared P;
    MFH_TRY(prepare(g, inputs, n_inputs, nullptr, 0, true, &P, false));
    int slot = -1;
    for (size_t i = 0; i < g.nodes.size(); i++)
        if (g.nodes[i]->id == it->second) slot = P.node_slot[i];
    for (size_t k = 0; slot < 0 && k < g.inputs.size(); k++)
        if (g.inputs[k] == it->second) slot = P.input_slot[k];
    if (slot < 0)
        return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: output value \"%s\" is never defined", it->second.c_str());
    *dtype = P.slots[slot].dtype;
    *count = P.slots[slot].count;
    return MFH_OK;
}

// compiler.PlanGraph (compiler/plan.go:242-290): buildPlanningTopology
// (:29-90), PlanWorkspace, attachGraphIOPorts (:179-228), ScheduleStreams.
// The graph is taken in its own order (graph calls need it topological).
int plan_graph(Graph& g, const mfh_value* inputs, int32_t n_inputs, int64_t align, int32_t max_streams, Topology* t)
{
    Prepared P;
    MFH_TRY(prepare(g, inputs, n_inputs, nullptr, 0, true, &P));
    auto port_for = [&](const Slot& s) {
        PlanPort p;
        p.dtype = s.kind == Slot::kConst ? kFloat32 : s.dtype;
        p.dims = {s.count};
        p.symbols = {""};
        t->ports.push_back(p);
        return (int32_t)t->ports.size() - 1;
    };
    std::map<std::string, int32_t> boundary, produced;
    for (size_t k = 0; k < g.inputs.size(); k++) {
        if (g.inputs[k].empty() || boundary.count(g.inputs[k])) continue;
        const int slot = P.input_slot[k];
        if (slot < 0) {
            // an input the call leaves unbound has no shape to plan with
            boundary[g.inputs[k]] = -1;
            continue;
        }
        boundary[g.inputs[k]] = port_for(P.slots[slot]);
    }
    for (size_t i = 0; i < g.nodes.size(); i++) {
        const GraphNode& node = *g.nodes[i];
        PlanNode n;
        n.name = node.id;
        for (const std::string& name : node.inputs) {
            auto p = produced.find(name);
            if (p != produced.end()) {
                n.inputs.push_back(p->second);
                continue;
            }
            auto b = boundary.find(name);
            n.inputs.push_back(b != boundary.end() ? b->second : -1);
        }
        const int32_t out = port_for(P.slots[P.node_slot[i]]);
        n.outputs.push_back(out);
        produced[node.id] = out;
        t->nodes.push_back(std::move(n));
    }
    MFH_TRY(plan_workspace(*t, align));
    for (const auto& kv : boundary) {
        if (kv.second < 0 || !t->ports[kv.second].allocated)
            return fail(MFH_ERR_INVALID_ARGUMENT, "compiler: graph input \"%s\" has no workspace allocation", kv.first.c_str());
        t->input_ports[kv.first] = t->ports[kv.second].offset;
    }
    for (const auto& kv : g.outputs) {
        if (kv.first.empty()) continue;
        auto p = produced.find(kv.second);
        if (p == produced.end() || !t->ports[p->second].allocated)
            return fail(MFH_ERR_INVALID_ARGUMENT, "compiler: graph output \"%s\" producer \"%s\" has no workspace allocation",
                        kv.first.c_str(), kv.second.c_str());
        t->output_ports[kv.first] = t->ports[p->second].offset;
    }
    return schedule_streams(*t, max_streams);
}

}  // namespace
}  // namespace mfh
using namespace mfh;

namespace {

GraphNode* node_at(const mfh_graph* g, int32_t i)
{
    if (!g || i < 0 || i >= (int32_t)g->nodes.size()) return nullptr;
    return g->nodes[i].get();
}

int bad_node(const char* what, int32_t i)
{
    return fail(MFH_ERR_INVALID_ARGUMENT, "%s: no node %d", what, (int)i);
}

std::string str_or_empty(const char* s) { return s ? s : ""; }

// Rebuilds a tree from its pre-order list; `pos` advances past the subtree.
int parse_tree(const mfh_ast_node* nodes, const int32_t* child_counts, int32_t n, int32_t* pos,
               std::unique_ptr<ASTNode>* out, int depth)
{
    if (*pos >= n) return fail(MFH_ERR_INVALID_ARGUMENT, "fusion: the node list ends inside the tree");
    if (depth > 4096) return fail(MFH_ERR_INVALID_ARGUMENT, "fusion: tree deeper than 4096");
    const int32_t at = (*pos)++;
    auto node = std::make_unique<ASTNode>();
    node->type = nodes[at].type;
    node->input_index = nodes[at].input_index;
    node->value = nodes[at].value;
    int32_t kids = child_counts ? child_counts[at] : node_arity(node->type);
    if (kids < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "fusion: node %d has unknown type %d", (int)at, node->type);
    for (int32_t c = 0; c < kids; c++) {
        std::unique_ptr<ASTNode> child;
        MFH_TRY(parse_tree(nodes, child_counts, n, pos, &child, depth + 1));
        node->children.push_back(std::move(child));
    }
    *out = std::move(node);
    return MFH_OK;
}

}  // namespace

extern "C" {

int mfh_graph_create(uint8_t execution_dtype, mfh_graph** graph)
{
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_create: graph out-pointer is NULL");
    *graph = new mfh_graph();
    (*graph)->execution_dtype = execution_dtype;
    return MFH_OK;
}

int mfh_graph_release(mfh_graph* graph)
{
    if (!graph) return MFH_OK;
    int rc = MFH_OK;
    const bool device_state = graph->ws || graph->fork || graph->done_ring[0] || !graph->aux.empty() || !graph->events.empty() ||
                              graph->capture || !graph->plans.empty();
    if (device_state) {
        drop_replays(*graph);
        const Device* dev;
        rc = bind_device(&dev);
        if (rc == MFH_OK && graph->ws) rc = check_hip(hipFree(graph->ws), "hipFree(graph workspace)");
        if (rc == MFH_OK) {
            // hipFree waited for the device; the streams and events are idle
            for (hipStream_t s : graph->aux) (void)hipStreamDestroy(s);
            for (hipEvent_t e : graph->events) (void)hipEventDestroy(e);
            for (hipEvent_t e : graph->joins) (void)hipEventDestroy(e);
            if (graph->capture) (void)hipStreamDestroy(graph->capture);
            if (graph->fork) (void)hipEventDestroy(graph->fork);
            for (hipEvent_t e : graph->done_ring)
                if (e) (void)hipEventDestroy(e);
        }
    }
    delete graph;
    return rc;
}

int mfh_graph_add_input(mfh_graph* graph, const char* name)
{
    if (graph) forget_calls(*graph);
    if (!graph || !name) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_add_input: graph and name are required");
    graph->inputs.push_back(name);
    return MFH_OK;
}

int mfh_graph_set_output(mfh_graph* graph, const char* key, const char* value)
{
    if (graph) forget_calls(*graph);
    if (!graph || !key || !value)
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_set_output: graph, key and value are required");
    for (auto& kv : graph->outputs)
        if (kv.first == key) {
            kv.second = value;
            return MFH_OK;
        }
    graph->outputs.emplace_back(key, value);
    return MFH_OK;
}

int mfh_graph_add_node(mfh_graph* graph, const char* id, const char* op, const char* const* inputs, int32_t n_inputs)
{
    if (graph) forget_calls(*graph);
    if (!graph || !id || !op) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_add_node: graph, id and op are required");
    if (n_inputs < 0 || (n_inputs > 0 && !inputs))
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_add_node: bad input list");
    auto node = std::make_unique<GraphNode>();
    node->id = id;
    node->op = op;
    for (int32_t k = 0; k < n_inputs; k++) {
        if (!inputs[k]) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_add_node: input %d is NULL", (int)k);
        node->inputs.push_back(inputs[k]);
    }
    graph->nodes.push_back(std::move(node));
    return MFH_OK;
}

int mfh_graph_set_attribute(mfh_graph* graph, int32_t node, const char* key, double value)
{
    if (graph) forget_calls(*graph);
    GraphNode* n = node_at(graph, node);
    if (!n) return bad_node("mfh_graph_set_attribute", node);
    if (!key) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_set_attribute: key is NULL");
    n->attributes[key] = value;
    return MFH_OK;
}

int mfh_graph_set_types(mfh_graph* graph, int32_t node, const uint8_t* input_types, int32_t n_input_types,
                        uint8_t output_type)
{
    if (graph) forget_calls(*graph);
    GraphNode* n = node_at(graph, node);
    if (!n) return bad_node("mfh_graph_set_types", node);
    if (n_input_types < 0 || (n_input_types > 0 && !input_types))
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_set_types: bad type list");
    n->input_types.assign(input_types, input_types + n_input_types);
    n->output_type = output_type;
    return MFH_OK;
}

int mfh_graph_set_fusion(mfh_graph* graph, int32_t node, const mfh_ast_node* nodes, const int32_t* child_counts,
                         int32_t n_nodes, const char* const* input_ports, int32_t n_input_ports,
                         const char* output_port, uint8_t dtype)
{
    if (graph) forget_calls(*graph);
    GraphNode* n = node_at(graph, node);
    if (!n) return bad_node("mfh_graph_set_fusion", node);
    if (!nodes || n_nodes <= 0) return fail(MFH_ERR_INVALID_ARGUMENT, "fusion: root is required");
    if (n_input_ports < 0 || (n_input_ports > 0 && !input_ports))
        return fail(MFH_ERR_INVALID_ARGUMENT, "fusion: bad input port list");
    auto f = std::make_shared<FusionAST>();
    int32_t pos = 0;
    MFH_TRY(parse_tree(nodes, child_counts, n_nodes, &pos, &f->root, 0));
    if (pos != n_nodes)
        return fail(MFH_ERR_INVALID_ARGUMENT, "fusion: %d node(s) after the end of the tree", (int)(n_nodes - pos));
    for (int32_t k = 0; k < n_input_ports; k++) f->input_ports.push_back(str_or_empty(input_ports[k]));
    f->output_port = str_or_empty(output_port);
    f->dtype = dtype;
    n->fusion = std::move(f);
    n->kernels.reset();
    return MFH_OK;
}

int32_t mfh_graph_num_nodes(const mfh_graph* graph) { return graph ? (int32_t)graph->nodes.size() : -1; }

const char* mfh_graph_node_id(const mfh_graph* graph, int32_t node)
{
    GraphNode* n = node_at(graph, node);
    return n ? n->id.c_str() : nullptr;
}

const char* mfh_graph_node_op(const mfh_graph* graph, int32_t node)
{
    GraphNode* n = node_at(graph, node);
    return n ? n->op.c_str() : nullptr;
}

int32_t mfh_graph_node_num_inputs(const mfh_graph* graph, int32_t node)
{
    GraphNode* n = node_at(graph, node);
    return n ? (int32_t)n->inputs.size() : -1;
}

const char* mfh_graph_node_input(const mfh_graph* graph, int32_t node, int32_t slot)
{
    GraphNode* n = node_at(graph, node);
    if (!n || slot < 0 || slot >= (int32_t)n->inputs.size()) return nullptr;
    return n->inputs[slot].c_str();
}

int mfh_graph_node_attribute(const mfh_graph* graph, int32_t node, const char* key, double* value)
{
    GraphNode* n = node_at(graph, node);
    if (!n) return bad_node("mfh_graph_node_attribute", node);
    auto it = key ? n->attributes.find(key) : n->attributes.end();
    if (it == n->attributes.end())
        return fail(MFH_ERR_INVALID_ARGUMENT, "node \"%s\" has no attribute \"%s\"", n->id.c_str(), key ? key : "");
    if (value) *value = it->second;
    return MFH_OK;
}

const char* mfh_graph_node_attribute_key(const mfh_graph* graph, int32_t node, int32_t k)
{
    GraphNode* n = node_at(graph, node);
    if (!n || k < 0 || k >= (int32_t)n->attributes.size()) return nullptr;
    auto it = n->attributes.begin();
    std::advance(it, k);
    return it->first.c_str();
}

int mfh_graph_node_metadata(const mfh_graph* graph, int32_t node, const char* key, int64_t* value)
{
    GraphNode* n = node_at(graph, node);
    if (!n) return bad_node("mfh_graph_node_metadata", node);
    auto it = key ? n->metadata.find(key) : n->metadata.end();
    if (it == n->metadata.end())
        return fail(MFH_ERR_INVALID_ARGUMENT, "node \"%s\" has no metadata \"%s\"", n->id.c_str(), key ? key : "");
    if (value) *value = it->second;
    return MFH_OK;
}

int32_t mfh_graph_node_types(const mfh_graph* graph, int32_t node, uint8_t* input_types, int32_t cap,
                             uint8_t* output_type)
{
    GraphNode* n = node_at(graph, node);
    if (!n) return -1;
    for (int32_t k = 0; input_types && k < cap && k < (int32_t)n->input_types.size(); k++)
        input_types[k] = n->input_types[k];
    if (output_type) *output_type = n->output_type;
    return (int32_t)n->input_types.size();
}

int mfh_graph_fusion(const mfh_graph* graph, int32_t node, mfh_fusion_info* info)
{
    GraphNode* n = node_at(graph, node);
    if (!n) return bad_node("mfh_graph_fusion", node);
    if (!n->fusion) return fail(MFH_ERR_INVALID_ARGUMENT, "node \"%s\" holds no FusionAST", n->id.c_str());
    if (!info) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_fusion: info is NULL");
    FusionAST& f = *n->fusion;
    f.flatten();
    info->nodes = f.flat.data();
    info->child_counts = f.child_counts.data();
    info->n_nodes = (int32_t)f.flat.size();
    info->n_input_ports = (int32_t)f.input_ports.size();
    info->n_contained = (int32_t)f.contained_node_ids.size();
    info->dtype = f.dtype;
    info->output_port = f.output_port.c_str();
    info->count_expr = f.count_expr.c_str();
    return MFH_OK;
}

const char* mfh_graph_fusion_input_port(const mfh_graph* graph, int32_t node, int32_t k)
{
    GraphNode* n = node_at(graph, node);
    if (!n || !n->fusion || k < 0 || k >= (int32_t)n->fusion->input_ports.size()) return nullptr;
    return n->fusion->input_ports[k].c_str();
}

const char* mfh_graph_fusion_contained_id(const mfh_graph* graph, int32_t node, int32_t k)
{
    GraphNode* n = node_at(graph, node);
    if (!n || !n->fusion || k < 0 || k >= (int32_t)n->fusion->contained_node_ids.size()) return nullptr;
    return n->fusion->contained_node_ids[k].c_str();
}

int32_t mfh_optimizer_is_elementwise_op(const char* op) { return op ? elementwise_type(op) : kNodeInvalid; }

int32_t mfh_optimizer_elementwise_ops(const char** ops, int32_t cap)
{
    int32_t count = 0;
    for (const OpEntry& row : kElementwiseTable) {
        if (row.type == kNodeInvalid) continue;
        if (ops && count < cap) ops[count] = row.op;
        count++;
    }
    return count;
}

int mfh_optimizer_constant_fold(mfh_graph* graph, int32_t* nodes_folded)
{
    if (graph) forget_calls(*graph);
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "optimizer: graph is required");
    return constant_fold(*graph, nodes_folded);
}

int mfh_optimizer_fuse(mfh_graph* graph, mfh_fusion_stats* stats)
{
    if (graph) forget_calls(*graph);
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "optimizer: graph is required");
    return fuse(*graph, stats);
}

int mfh_optimizer_run(mfh_graph* graph, uint32_t options, int32_t* nodes_folded, mfh_fusion_stats* stats)
{
    if (graph) forget_calls(*graph);
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "optimizer: graph is required");
    if (nodes_folded) *nodes_folded = 0;
    if (stats) *stats = mfh_fusion_stats{0, 0, 0};
    if (!(options & MFH_OPT_DISABLE_CONSTANT_FOLD)) MFH_TRY(constant_fold(*graph, nodes_folded));
    if (!(options & MFH_OPT_DISABLE_FUSION)) MFH_TRY(fuse(*graph, stats));
    return MFH_OK;
}

int mfh_codegen_attach_kernels(mfh_graph* graph, const int32_t* targets, int32_t n_targets, uint32_t flags,
                               int32_t* attached)
{
    if (graph) forget_calls(*graph);
    if (attached) *attached = 0;
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "codegen: graph is required");
    return attach_kernels(*graph, targets, n_targets, flags, attached);
}

int mfh_graph_kernel(const mfh_graph* graph, int32_t node, int32_t target, const mfh_kernel** kernel)
{
    if (!kernel) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_kernel: kernel out-pointer is NULL");
    *kernel = nullptr;
    GraphNode* n = node_at(graph, node);
    if (!n) return bad_node("mfh_graph_kernel", node);
    HIPKernel* k = n->kernels ? n->kernels->For(target) : nullptr;
    if (k) *kernel = k->full;
    return MFH_OK;
}

int mfh_graph_call(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs,
                   int32_t n_outputs, void* stream)
{
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: graph is required");
    return graph_call(*graph, inputs, n_inputs, outputs, n_outputs, (hipStream_t)stream);
}

int64_t mfh_graph_workspace_bytes(const mfh_graph* graph) { return graph ? graph->ws_bytes : -1; }

int mfh_graph_output_shape(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, const char* key,
                           uint8_t* dtype, int64_t* count)
{
    if (!graph || !key || !dtype || !count)
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_output_shape: graph, key, dtype and count are required");
    return output_shape(*graph, inputs, n_inputs, key, dtype, count);
}

int mfh_graph_call_noalloc(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, const mfh_value* outputs,
                           int32_t n_outputs, void* stream)
{
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "graph is NULL");
    return graph_call_noalloc(*graph, inputs, n_inputs, outputs, n_outputs, (hipStream_t)stream);
}

int mfh_graph_set_max_streams(mfh_graph* graph, int32_t max_streams)
{
    if (graph) forget_calls(*graph);
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_set_max_streams: graph is required");
    if (max_streams < 1 || max_streams > 64)
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_set_max_streams: %d streams; 1 to 64 are supported", (int)max_streams);
    graph->max_streams = max_streams;
    return MFH_OK;
}

int32_t mfh_graph_streams_used(const mfh_graph* graph) { return graph ? graph->streams_used : -1; }

int mfh_graph_set_replay(mfh_graph* graph, int32_t enabled)
{
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_graph_set_replay: graph is required");
    drop_replays(*graph);
    graph->replay = enabled != 0;
    graph->replay_broken = false;
    return MFH_OK;
}

int64_t mfh_graph_replayed_calls(const mfh_graph* graph) { return graph ? graph->replayed : -1; }

int mfh_graph_plan(mfh_graph* graph, const mfh_value* inputs, int32_t n_inputs, int64_t align, int32_t max_streams,
                   mfh_topology** topology)
{
    if (!graph || !topology) return fail(MFH_ERR_INVALID_ARGUMENT, "compiler: graph is required");
    *topology = nullptr;
    auto t = std::make_unique<mfh_topology>();
    MFH_TRY(plan_graph(*graph, inputs, n_inputs, align, max_streams, t.get()));
    *topology = t.release();
    return MFH_OK;
}

}  // extern "C"
