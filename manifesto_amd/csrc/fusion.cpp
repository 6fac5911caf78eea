// fusion.cpp — the HIP codegen target for FusionAST (EmitHIP) and its
// execution (HIPKernel.Run).
//
// EmitHIP is the gfx950 counterpart of EmitCPU / EmitMetal (codegen/cpu.go:97,
// codegen/metal.go:79): one kernel per FusionAST whose body is the fused
// expression, evaluated per element with the reference's f32 semantics
// (codegen/cpu.go:126-214).  Unlike the Metal template (f32 buffers, one
// element per thread) the generated kernel
//   * reads each operand in its storage dtype (f32 / bf16 / f16) and decodes in
//     registers, so a bf16 or f16 tensor needs no separate cast pass,
//   * encodes the result to the output dtype with the reference's rounding,
//   * moves 8 elements per thread per step with 16-byte loads and stores in a
//     grid-stride loop, and reads broadcast operands (a [period] bias, a
//     scalar) in place of pre-expanded copies.
// The source is compiled for gfx950 by hiprtc with -ffp-contract=off, so
// every Add/Sub/Mul/Div rounds on its own as in Go, and cached by its text.
#include <hip/hiprtc.h>

#include <unistd.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "fusion.hpp"

namespace mfh {

#include "mfh_prelude.inc"  // kPrelude: codec.hpp + devmath.hpp + fusion_io.hpp

namespace {

// Threads per workgroup of a generated kernel unless the launch config sets
// a size: one wave.  Measured on MI355X at the BASELINE sizes (one-shot grids,
// same kernels otherwise): the SwiGLU chain +3% and the f16 gelu chain +1%
// against 256-thread workgroups (128 threads: +1% and -4%); a no-compute
// 2:1 read:write stream +2-4% with 64 or 128.
constexpr int kFusedThreads = 64;
// Blocks per CU that make every grid one-shot (capped by the work itself).
constexpr int kOneShotBlocksPerCu = 1 << 16;

const char* io_suffix(int dtype)
{
    switch (dtype) {
    case kFloat32: return "f32";
    case kBFloat16: return "bf16";
    case kFloat16: return "f16";
    default: return nullptr;
    }
}

std::string hex32(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    char buf[32];
    snprintf(buf, sizeof buf, "mfh_fromfbits(0x%08xu)", u);
    return buf;
}

// Pre-order list -> child links; -1 if malformed.
int link(const std::vector<mfh_ast_node>& nodes, int idx, std::vector<int>& c0, std::vector<int>& c1)
{
    if (idx >= (int)nodes.size()) return -1;
    int arity = node_arity(nodes[idx].type);
    if (arity < 0) return -1;
    int next = idx + 1;
    for (int k = 0; k < arity; k++) {
        (k == 0 ? c0 : c1)[idx] = next;
        next = link(nodes, next, c0, c1);
        if (next < 0) return -1;
    }
    return next;
}

// How an Emitter evaluates Sigmoid, Silu and Gelu.
enum class Form {
    kFast,      // branch-free fast forms; each ORs the element's flag `qe`
    kFallback,  // the reference forms as real calls (recomputing flagged elements)
    kRounded,   // the rounding-tested f64 forms; each ORs `qe` (chains that stream f32, MFH_FUSION_PRECISE)
    kPrecise,   // the reference forms inline (MFH_FUSION_PRECISE | MFH_FUSION_NO_ROUNDING_TEST)
};

bool is_fast_activation(int type) { return type == kNodeSigmoid || type == kNodeSilu || type == kNodeGelu; }

bool is_transcendental(int type)
{
    return type == kNodeExp || type == kNodeLog || type == kNodeTanh || is_fast_activation(type);
}

// Cancellation guards.  A fast activation's value a' is within 2 f32 ulps of
// the reference's a, i.e. |a' - a| <= 2^-22 |a|, and every op between it and
// the output is IEEE-exact in both evaluations except for that difference.
// An Add/Sub s = a + b whose result is much smaller than a turns it into an
// error of up to 2^-22 |a| / |s| relative to s, which for a 16-bit output can
// exceed one storage ulp (config 4: gelu + residual cancelling to an f16
// denormal).  The generated code flags the element when |s| F < |a| and
// recomputes flagged elements with the reference forms.  With e the operand's
// error in f32 ulps (2 for the activation, one more for each Mul, Div, Sqrt or
// LeakyReLU between it and the Add/Sub) and m the output's mantissa bits
// (10 for f16, 7 for bf16), F = 0.7 2^(22-m) / e: unflagged, the difference
// is at most e 2^-23 F |s| = 0.7 2^(-1-m) |s|, under 0.7 of the storage ulp
// of s (which exceeds 2^(-1-m) |s|), plus one f32 rounding of s; the two
// rounded results are then at most one storage ulp apart.  f16 denormal
// results are covered by the same test (unflagged, |a| < F 2^-14 and the
// difference is under 2^-25).  The guarantee is made where the activation
// reaches the output through exactly one Add/Sub and no other transcendental
// node (the BASELINE chains); other paths keep the node-envelope contract.
// f32 outputs carry every f32 ulp of the node, so they take no guard; nor do
// chains whose activations take the reference's values (`exact`: the
// rounding-tested and reference forms).
struct Guard {
    int factor = 0;  // flag when |s| factor < M; 0 = no guard
    bool lhs = false, rhs = false;  // which operands carry an activation's error (M = the max of those)
};

std::vector<Guard> plan_guards(const std::vector<mfh_ast_node>& nodes, const std::vector<int>& c0,
                               const std::vector<int>& c1, uint8_t out_dtype, bool exact)
{
    const int n = (int)nodes.size();
    std::vector<Guard> guards(n);
    const int mantissa = out_dtype == kFloat16 ? 10 : out_dtype == kBFloat16 ? 7 : 0;
    if (exact || mantissa == 0) return guards;
    std::vector<int> parent(n, -1);
    for (int i = 0; i < n; i++) {
        if (c0[i] >= 0) parent[c0[i]] = i;
        if (c1[i] >= 0) parent[c1[i]] = i;
    }
    // Per Add/Sub: the error of each operand in f32 ulps (0: none), or off
    // when an activation below it reaches the output by another Add/Sub or
    // through another transcendental node.
    std::vector<int> ulps_lhs(n, 0), ulps_rhs(n, 0);
    std::vector<bool> off(n, false);
    for (int a = 0; a < n; a++) {
        if (!is_fast_activation(nodes[a].type)) continue;
        int rounding = 0, add = -1, adds = 0;
        bool lhs = false, other = false;
        for (int from = a, p = parent[a]; p >= 0; from = p, p = parent[p]) {
            const int t = nodes[p].type;
            if (t == kNodeAdd || t == kNodeSub) {
                if (adds++ == 0) {
                    add = p;
                    lhs = from == c0[p];
                }
            } else if (t == kNodeMul || t == kNodeDiv || t == kNodeSqrt || t == kNodeLeakyReLU) {
                if (adds == 0) rounding++;
            } else if (is_transcendental(t)) {
                other = true;
            }
        }
        if (add < 0) continue;
        if (adds > 1 || other) {
            off[add] = true;
            continue;
        }
        // relative errors add through Mul/Div: a sum over the side's
        // activations bounds the side's error
        (lhs ? ulps_lhs[add] : ulps_rhs[add]) += 2 + rounding;
    }
    for (int i = 0; i < n; i++) {
        if (off[i] || (ulps_lhs[i] == 0 && ulps_rhs[i] == 0)) continue;
        const int factor = (int)(0.7 * std::ldexp(1.0, 22 - mantissa) / (ulps_lhs[i] + ulps_rhs[i]));
        if (factor < 2) continue;
        guards[i].factor = factor;
        guards[i].lhs = ulps_lhs[i] > 0;
        guards[i].rhs = ulps_rhs[i] > 0;
    }
    return guards;
}

struct Emitter {
    const std::vector<mfh_ast_node>& nodes;
    const std::vector<int>& c0;
    const std::vector<int>& c1;
    Form form;
    const std::vector<Guard>* guards = nullptr;  // kFast only
    std::string prefix = "t";
    // Vector loop only: inputs held as packed f16 words w<k>[u][j >> 1]
    // (empty in the element loop).
    std::vector<bool> packed16 = {};
    std::string body = "";
    int tmp = 0;
    // Set once the element's flag `qe` has been written: a fast activation or
    // a guard was emitted.
    bool flagged = false;

    std::string fresh() { return prefix + std::to_string(tmp++); }

    std::string let(const std::string& expr)
    {
        std::string name = fresh();
        body += "        const float " + name + " = " + expr + ";\n";
        return name;
    }

    std::string activation(const char* name, const std::string& a)
    {
        const std::string fn = std::string("mfh_") + name;
        if (form == Form::kPrecise) return let(fn + "_ref(" + a + ")");
        if (form == Form::kFallback) return let(fn + "_rare(" + a + ")");
        flagged = true;
        return let(fn + (form == Form::kRounded ? "_cr(" : "_fast(") + a + ", qe)");
    }

    // s = a + b (or a - b): the cancellation guard of node idx, if planned.
    std::string guarded(int idx, const std::string& s, const std::string& a, const std::string& b)
    {
        if (form != Form::kFast || !guards || (*guards)[idx].factor == 0) return s;
        const Guard& g = (*guards)[idx];
        std::string m = g.lhs && g.rhs ? "mfh_maxf(mfh_absf(" + a + "), mfh_absf(" + b + "))"
                        : g.lhs        ? "mfh_absf(" + a + ")"
                                       : "mfh_absf(" + b + ")";
        body += "        qe |= !(mfh_absf(" + s + ") * " + std::to_string(g.factor) + ".0f >= " + m + ");\n";
        flagged = true;
        return s;
    }

    // Returns the name holding node idx's value for the current element.
    std::string emit(int idx)
    {
        const mfh_ast_node& n = nodes[idx];
        switch (n.type) {
        case kNodeInput: return "x" + std::to_string(n.input_index);
        case kNodeConstant: return let(hex32((float)n.value));  // float32(node.Value)
        default: break;
        }
        if (n.type == kNodeAdd) {
            // An f16 input leaf is added straight from its packed word.
            auto word = [&](int child) -> std::string {
                const mfh_ast_node& leaf = nodes[child];
                if (leaf.type != kNodeInput || leaf.input_index >= (int)packed16.size() || !packed16[leaf.input_index])
                    return "";
                return "w" + std::to_string(leaf.input_index) + "[u][j >> 1]";
            };
            std::string wa = word(c0[idx]), wb = word(c1[idx]);
            if (!wa.empty() && !wb.empty()) return let("mfh_add_hh(" + wa + ", j & 1, " + wb + ", j & 1)");
            // a leaf carries no activation error: the guard's operand is the other side
            if (!wb.empty()) {
                std::string a = emit(c0[idx]);
                return guarded(idx, let("mfh_add_fh(" + a + ", " + wb + ", j & 1)"), a, a);
            }
            if (!wa.empty()) {
                std::string b = emit(c1[idx]);
                return guarded(idx, let("mfh_add_fh(" + b + ", " + wa + ", j & 1)"), b, b);
            }
        }
        std::string a = emit(c0[idx]);
        if (node_arity(n.type) == 2) {
            std::string b = emit(c1[idx]);
            switch (n.type) {
            case kNodeAdd: return guarded(idx, let(a + " + " + b), a, b);
            case kNodeSub: return guarded(idx, let(a + " - " + b), a, b);
            case kNodeMul: return let(a + " * " + b);
            case kNodeDiv: return let(a + " / " + b);
            case kNodeMax: return let("(" + a + " > " + b + ") ? " + a + " : " + b);
            case kNodeMin: return let("(" + a + " < " + b + ") ? " + a + " : " + b);
            }
        }
        switch (n.type) {
        case kNodeNeg: return let("-" + a);
        case kNodeAbs: return let("(" + a + " < 0.0f) ? -" + a + " : " + a);
        case kNodeSqrt: return let("mfh_sqrtf(" + a + ")");
        case kNodeExp: return let("mfh_exp_ref(" + a + ")");
        case kNodeLog: return let("mfh_log_ref(" + a + ")");
        case kNodeReLU: return let("(" + a + " < 0.0f) ? 0.0f : " + a);
        case kNodeSigmoid: return activation("sigmoid", a);
        case kNodeTanh: return let("mfh_tanh_ref(" + a + ")");
        case kNodeSilu: return activation("silu", a);
        case kNodeGelu: return activation("gelu", a);
        case kNodeLeakyReLU: {
            std::string scaled = let("0.01f * " + a);
            return let("(" + a + " >= 0.0f) ? " + a + " : " + scaled);
        }
        }
        return let("0.0f");  // unreachable: validated
    }
};

std::string sanitize(const std::string& port)
{
    std::string s;
    for (char ch : port) s += ((ch >= 'a' && ch <= 'z') || (ch >= 'A' && ch <= 'Z') || (ch >= '0' && ch <= '9')) ? ch : '_';
    return s.empty() ? "anon" : s;
}

std::string operand_index(const mfh_operand& op, const char* elem)
{
    if (op.mode == MFH_OPERAND_PERIODIC) return std::string("(") + elem + " % " + std::to_string(op.period) + "LL)";
    return elem;
}

// ---- compiled-code cache -----------------------------------------------------

struct CodeObject {
    std::vector<char> code;
    std::string kernel_name;
    std::mutex mu;
    int device = -1;
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
};

std::mutex g_cache_mu;
std::unordered_map<std::string, std::shared_ptr<CodeObject>> g_cache;
// Bumped whenever a loaded module is unloaded, so that holders of function
// handles (captured graph calls) know theirs may be gone.
std::atomic<uint64_t> g_module_generation{0};

const char* const kCompileOptions[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                                       "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature",
                                       "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16"};

// ---- compiled code kept on disk between processes ----------------------------
//
// One file per kernel, named by a hash of what produced it.  A file holds the
// compiler identity (hiprtc version and options), the full kernel source and
// the code object, followed by a checksum; it is used only when identity and
// source match this compile exactly and the checksum holds, so a hash
// collision, a stale or a truncated file costs a compile and nothing else.
// Files are written under a temporary name and renamed into place, so
// processes sharing the directory never read a partial file.  The directory
// must be trusted like any code the process loads.

std::mutex g_disk_mu;
std::string g_disk_dir;
bool g_disk_dir_set = false;
std::atomic<int64_t> g_disk_hits{0}, g_compiles{0};

constexpr char kDiskMagic[8] = {'M', 'F', 'H', 'K', 'O', 'D', 'E', '1'};
constexpr uint64_t kDiskMaxBytes = uint64_t(256) << 20;

uint64_t fnv1a(const void* data, size_t n, uint64_t h = 1469598103934665603ull)
{
    const unsigned char* p = static_cast<const unsigned char*>(data);
    for (size_t i = 0; i < n; i++) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}

std::string disk_dir()
{
    std::lock_guard<std::mutex> lock(g_disk_mu);
    if (!g_disk_dir_set) {
        const char* env = std::getenv("MFH_KERNEL_CACHE_DIR");
        g_disk_dir = env ? env : "";
        g_disk_dir_set = true;
    }
    return g_disk_dir;
}

std::string compiler_identity()
{
    int major = 0, minor = 0;
    (void)hiprtcVersion(&major, &minor);
    std::string id = "hiprtc " + std::to_string(major) + "." + std::to_string(minor);
    for (const char* o : kCompileOptions) id += std::string(" ") + o;
    return id;
}

void put_blob(std::string& out, const void* p, uint64_t n)
{
    out.append(reinterpret_cast<const char*>(&n), sizeof n);
    out.append(static_cast<const char*>(p), n);
}

std::string disk_path(const std::string& dir, const std::string& identity, const std::string& source)
{
    const uint64_t h = fnv1a(source.data(), source.size(), fnv1a(identity.data(), identity.size()));
    char name[40];
    std::snprintf(name, sizeof name, "/%016llx.hsaco", (unsigned long long)h);
    return dir + name;
}

// The code object stored for (identity, source), if a whole, matching file holds one.
bool disk_load(const std::string& path, const std::string& identity, const std::string& source, std::vector<char>* code)
{
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    std::string data;
    std::vector<char> buf(1 << 16);
    size_t n;
    while ((n = std::fread(buf.data(), 1, buf.size(), f)) > 0 && data.size() <= kDiskMaxBytes) data.append(buf.data(), n);
    std::fclose(f);
    size_t at = 0;
    auto take = [&](std::string* blob) {
        uint64_t len;
        if (data.size() - at < sizeof len) return false;
        std::memcpy(&len, data.data() + at, sizeof len);
        at += sizeof len;
        if (len > data.size() - at) return false;
        blob->assign(data.data() + at, len);
        at += len;
        return true;
    };
    if (data.size() < sizeof kDiskMagic + sizeof(uint64_t) || std::memcmp(data.data(), kDiskMagic, sizeof kDiskMagic))
        return false;
    const size_t body = data.size() - sizeof(uint64_t);
    uint64_t sum;
    std::memcpy(&sum, data.data() + body, sizeof sum);
    if (sum != fnv1a(data.data(), body)) return false;
    data.resize(body);
    at = sizeof kDiskMagic;
    std::string id, src, obj;
    if (!take(&id) || !take(&src) || !take(&obj) || at != data.size()) return false;
    if (id != identity || src != source || obj.empty()) return false;
    code->assign(obj.begin(), obj.end());
    return true;
}

// Best effort: a directory that cannot be written only costs later compiles.
void disk_store(const std::string& path, const std::string& identity, const std::string& source,
                const std::vector<char>& code)
{
    std::string data(kDiskMagic, sizeof kDiskMagic);
    put_blob(data, identity.data(), identity.size());
    put_blob(data, source.data(), source.size());
    put_blob(data, code.data(), code.size());
    const uint64_t sum = fnv1a(data.data(), data.size());
    data.append(reinterpret_cast<const char*>(&sum), sizeof sum);
    static std::atomic<uint64_t> serial{0};
    const std::string tmp = path + ".tmp." + std::to_string((long long)getpid()) + "." + std::to_string(serial++);
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return;
    const bool ok = std::fwrite(data.data(), 1, data.size(), f) == data.size();
    if (std::fclose(f) != 0 || !ok || std::rename(tmp.c_str(), path.c_str()) != 0) std::remove(tmp.c_str());
}

int compile_source(const std::string& source, const std::string& kernel_name, std::shared_ptr<CodeObject>* out)
{
    {
        std::lock_guard<std::mutex> lock(g_cache_mu);
        auto it = g_cache.find(source);
        if (it != g_cache.end()) {
            *out = it->second;
            return MFH_OK;
        }
    }
    const std::string dir = disk_dir();
    std::string identity, path;
    if (!dir.empty()) {
        identity = compiler_identity();
        path = disk_path(dir, identity, source);
        auto obj = std::make_shared<CodeObject>();
        if (disk_load(path, identity, source, &obj->code)) {
            obj->kernel_name = kernel_name;
            g_disk_hits++;
            std::lock_guard<std::mutex> lock(g_cache_mu);
            *out = g_cache.emplace(source, obj).first->second;
            return MFH_OK;
        }
    }
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, source.c_str(), (kernel_name + ".hip").c_str(), 0, nullptr, nullptr) != HIPRTC_SUCCESS)
        return fail(MFH_ERR_COMPILE, "codegen hip: hiprtcCreateProgram failed");
    hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof kCompileOptions / sizeof kCompileOptions[0]),
                                           kCompileOptions);
    if (rc != HIPRTC_SUCCESS) {
        size_t log_size = 0;
        hiprtcGetProgramLogSize(prog, &log_size);
        std::string log(log_size + 1, '\0');
        hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        return fail(MFH_ERR_COMPILE, "codegen hip: compiling %s failed: %s", kernel_name.c_str(), log.c_str());
    }
    auto obj = std::make_shared<CodeObject>();
    size_t size = 0;
    hiprtcGetCodeSize(prog, &size);
    obj->code.resize(size);
    hiprtcGetCode(prog, obj->code.data());
    hiprtcDestroyProgram(&prog);
    obj->kernel_name = kernel_name;
    g_compiles++;
    if (!dir.empty()) disk_store(path, identity, source, obj->code);
    std::lock_guard<std::mutex> lock(g_cache_mu);
    auto it = g_cache.emplace(source, obj).first;
    *out = it->second;
    return MFH_OK;
}

int load_function(CodeObject& obj, int device, bool may_load, hipFunction_t* fn)
{
    std::lock_guard<std::mutex> lock(obj.mu);
    if (obj.function && obj.device == device) {
        *fn = obj.function;
        return MFH_OK;
    }
    if (!may_load)
        return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: kernel %s is not loaded on device %d",
                    obj.kernel_name.c_str(), device);
    if (obj.module) {
        g_module_generation.fetch_add(1);
        (void)hipModuleUnload(obj.module);
        obj.module = nullptr;
        obj.function = nullptr;
    }
    MFH_TRY(check_hip(hipModuleLoadData(&obj.module, obj.code.data()), "hipModuleLoadData"));
    MFH_TRY(check_hip(hipModuleGetFunction(&obj.function, obj.module, obj.kernel_name.c_str()), "hipModuleGetFunction"));
    obj.device = device;
    *fn = obj.function;
    return MFH_OK;
}

}  // namespace

int node_arity(int type)
{
    switch (type) {
    case kNodeInput: case kNodeConstant: return 0;
    case kNodeNeg: case kNodeAbs: case kNodeSqrt: case kNodeExp: case kNodeLog: case kNodeReLU:
    case kNodeSigmoid: case kNodeTanh: case kNodeSilu: case kNodeGelu: case kNodeLeakyReLU: return 1;
    case kNodeAdd: case kNodeSub: case kNodeMul: case kNodeDiv: case kNodeMax: case kNodeMin: return 2;
    default: return -1;
    }
}

}  // namespace mfh

// The opaque handle of the C ABI: one compiled FusionAST (HIPKernel).
struct mfh_kernel {
    std::string identifier;
    std::string kernel_name;
    std::string source;
    std::vector<mfh_operand> inputs;
    uint8_t out_dtype = mfh::kFloat32;
    int vec = 8;     // elements per work item
    int unroll = 1;  // work items per thread per step
    int block = mfh::kFusedThreads;  // threads per workgroup
    int auto_bpc = 4;  // workgroups per CU unless the launch config sets one
    bool periods_vectorizable = true;
    std::shared_ptr<mfh::CodeObject> code;
};

namespace mfh {

int emit_hip(const mfh_ast_node* nodes, int n_nodes, const mfh_operand* inputs, int n_inputs,
             uint8_t out_dtype, const char* output_port, uint32_t flags, mfh_kernel** out)
{
    if (!out) return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: kernel out-pointer is NULL");
    *out = nullptr;
    if (!nodes || n_nodes <= 0) return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: fusion root is required");
    if (n_inputs < 0 || (n_inputs > 0 && !inputs))
        return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: bad input list");
    if (!io_suffix(out_dtype))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "codegen hip: output dtype %s is not f32/bf16/f16", dtype_name(out_dtype));
    std::vector<mfh_ast_node> list(nodes, nodes + n_nodes);
    for (int i = 0; i < n_nodes; i++) {
        if (node_arity(list[i].type) < 0)
            return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: unsupported node type %d", list[i].type);
        if (list[i].type == kNodeInput && (list[i].input_index < 0 || list[i].input_index >= n_inputs))
            return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: input index %d out of range [0, %d)",
                        list[i].input_index, n_inputs);
    }
    std::vector<int> c0(n_nodes, -1), c1(n_nodes, -1);
    if (link(list, 0, c0, c1) != n_nodes)
        return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: the node list is not one pre-order tree");

    // Work item width: 8 elements when the output and every streamed operand
    // are 16-bit (one 16-byte access per lane), 4 when any is f32.
    int vec = out_dtype == kFloat32 ? 4 : 8;
    for (int k = 0; k < n_inputs; k++) {
        const mfh_operand& op = inputs[k];
        if (!io_suffix(op.dtype))
            return fail(MFH_ERR_DTYPE_UNSUPPORTED, "codegen hip: input %d dtype %s is not f32/bf16/f16", k, dtype_name(op.dtype));
        if (op.mode > MFH_OPERAND_SCALAR)
            return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: input %d has unknown mode %d", k, op.mode);
        if (op.mode == MFH_OPERAND_PERIODIC && op.period <= 0)
            return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: input %d period must be positive", k);
        if (op.mode != MFH_OPERAND_SCALAR && op.dtype == kFloat32) vec = 4;
    }
    bool periods_vectorizable = true;
    for (int k = 0; k < n_inputs; k++)
        if (inputs[k].mode == MFH_OPERAND_PERIODIC && inputs[k].period % vec != 0) periods_vectorizable = false;

    const bool precise = (flags & MFH_FUSION_PRECISE) != 0;
    // Launch shape: a one-shot grid (one block per `block` x unroll items, so each
    // block streams one chunk and exits and the blocks sweep memory in
    // dispatch order).  Measured on MI355X against grid-stride loops at 4-24
    // blocks per CU: +11% on the SwiGLU chain and +9% on the f16 gelu chain;
    // a no-compute 2:1 read:write stream gains 17% the same way.  One item per
    // thread, except where the element math is mostly f64 (Sigmoid, and the
    // rounding-tested forms of chains that stream f32 and of
    // MFH_FUSION_PRECISE): two items per thread give a sigmoid chain 0-3% and
    // the precise SwiGLU chain 5.6% (the precise gelu chain -1%, within the
    // noise of six alternating runs), while SwiGLU, Silu, add/mul chains and
    // (since its 2^f runs on v_exp_f32) the gelu chain lose 2-6% and the
    // reference forms inline (MFH_FUSION_NO_ROUNDING_TEST) gain nothing.
    // Workgroups of one wave (kFusedThreads).  mfh_set_launch_config("fused",
    // ...) and mfh_set_launch_threads("fused", ...) override these.
    // Chains that stream f32 (an f32 output or a full or periodic f32
    // operand) show every f32 ulp of their activations: they take the
    // rounding-tested forms, whose results are the reference's, at about
    // twice the instructions of the f32 forms, which their 4-byte elements
    // leave room for (MFH_FUSION_SHORT_QUOTIENT keeps the 16-bit chains'
    // forms).  So do MFH_FUSION_PRECISE kernels unless
    // MFH_FUSION_NO_ROUNDING_TEST asks for the reference forms inline.
    const bool streams_f32 = vec == 4 && (flags & MFH_FUSION_SHORT_QUOTIENT) == 0;
    const bool rounded = precise ? (flags & MFH_FUSION_NO_ROUNDING_TEST) == 0 : streams_f32;
    bool f64_fast = false;
    for (const mfh_ast_node& node : list)
        if (is_fast_activation(node.type) && (rounded || (!precise && node.type == kNodeSigmoid)))
            f64_fast = true;
    const int unroll = items_per_thread(Kern::kFused) > 0 ? items_per_thread(Kern::kFused) : f64_fast ? 2 : 1;
    const int auto_bpc = kOneShotBlocksPerCu;
    const int block = threads_per_block(Kern::kFused) > 0 ? threads_per_block(Kern::kFused) : kFusedThreads;
    // Non-temporal loads for the streamed (full-length) operands when the
    // kernel reads at least as many bytes per element as it writes.
    int read_bytes = 0;
    for (int k = 0; k < n_inputs; k++)
        if (inputs[k].mode == MFH_OPERAND_FULL) read_bytes += inputs[k].dtype == kFloat32 ? 4 : 2;
    const bool stream_loads = read_bytes >= (out_dtype == kFloat32 ? 4 : 2);

    // Element loop: every operand decoded to f32.  Vector loop: f16 operands
    // stay packed words so that adds can take them directly.  Without
    // MFH_FUSION_PRECISE each element runs the fast forms and the planned
    // cancellation guards, which set its flag `qe`; flagged elements are then
    // recomputed with the reference forms (real calls), so the item's main
    // body has no branch.  The rounding-tested forms set the flag instead (no
    // guards: their results are the reference's); with
    // MFH_FUSION_NO_ROUNDING_TEST every element runs the reference forms.
    const Form main_form = rounded ? Form::kRounded : precise ? Form::kPrecise : Form::kFast;
    const std::vector<Guard> guards = plan_guards(list, c0, c1, out_dtype, main_form != Form::kFast);
    std::vector<bool> packed16(n_inputs, false);
    for (int k = 0; k < n_inputs; k++)
        packed16[k] = inputs[k].mode != MFH_OPERAND_SCALAR && inputs[k].dtype == kFloat16;
    Emitter em{list, c0, c1, main_form, &guards};
    const std::string result = em.emit(0);
    Emitter emf{list, c0, c1, Form::kFallback, nullptr, "f"};
    const std::string fresult = em.flagged ? emf.emit(0) : "";
    Emitter emv{list, c0, c1, main_form, &guards, "t", packed16};
    const std::string vresult = emv.emit(0);
    Emitter emvf{list, c0, c1, Form::kFallback, nullptr, "f", packed16};
    const std::string vfresult = emv.flagged ? emvf.emit(0) : "";

    std::string identifier = output_port && *output_port ? output_port : "anon";
    std::string kernel_name = "fused_" + sanitize(output_port ? output_port : "");
    const char* osfx = io_suffix(out_dtype);
    const std::string V = std::to_string(vec), U = std::to_string(unroll), B = std::to_string(block);

    std::string src;
    src.reserve(sizeof(kPrelude) + 4096);
    src += kPrelude;
    src += "\n// EmitHIP: fusion '" + identifier + "'" + (precise ? " (precise transcendentals)" : "") +
           ", " + V + " elements per item, " + U + " item(s) per thread per step" +
           (stream_loads ? ", streamed loads" : "") + "\n";
    src += "extern \"C\" __global__ __launch_bounds__(" + B + ") void " + kernel_name + "(\n";
    for (int k = 0; k < n_inputs; k++) src += "    const void* __restrict__ p" + std::to_string(k) + ",\n";
    src += "    void* __restrict__ pout, mfh_i64 n, mfh_i64 nvec)\n{\n";
    src += "    const mfh_i64 stride = (mfh_i64)gridDim.x * " + B + ";\n";
    src += "    const mfh_i64 tid = (mfh_i64)blockIdx.x * " + B + " + threadIdx.x;\n";
    for (int k = 0; k < n_inputs; k++)
        if (inputs[k].mode == MFH_OPERAND_SCALAR)
            src += "    const float s" + std::to_string(k) + " = mfh_ld1_" + io_suffix(inputs[k].dtype) + "(p" +
                   std::to_string(k) + ", 0);\n";
    // vector loop: loads of all items first, then compute and store
    src += "    for (mfh_i64 v = tid; v < nvec; v += stride * " + U + ") {\n";
    for (int k = 0; k < n_inputs; k++) {
        if (inputs[k].mode == MFH_OPERAND_SCALAR) continue;
        if (packed16[k]) src += "        mfh_u32 w" + std::to_string(k) + "[" + U + "][" + std::to_string(vec / 2) + "];\n";
        else src += "        float a" + std::to_string(k) + "[" + U + "][" + V + "];\n";
    }
    src += "#pragma unroll\n        for (int u = 0; u < " + U + "; u++) {\n";
    src += "            const mfh_i64 it = v + u * stride;\n            if (it < nvec) {\n";
    src += "                const mfh_i64 e0 = it * " + V + ";\n";
    for (int k = 0; k < n_inputs; k++) {
        if (inputs[k].mode == MFH_OPERAND_SCALAR) continue;
        std::string ks = std::to_string(k);
        const std::string nt = stream_loads && inputs[k].mode == MFH_OPERAND_FULL ? "<1>" : "";
        if (packed16[k])
            src += "                mfh_ldw" + V + "_f16" + nt + "(p" + ks + ", " + operand_index(inputs[k], "e0") +
                   ", w" + ks + "[u]);\n";
        else
            src += "                mfh_ld" + V + "_" + io_suffix(inputs[k].dtype) + nt + "(p" + ks + ", " +
                   operand_index(inputs[k], "e0") + ", a" + ks + "[u]);\n";
    }
    src += "            }\n        }\n";
    src += "#pragma unroll\n        for (int u = 0; u < " + U + "; u++) {\n";
    src += "            const mfh_i64 it = v + u * stride;\n            if (it >= nvec) break;\n";
    std::string operands;
    for (int k = 0; k < n_inputs; k++) {
        std::string ks = std::to_string(k);
        std::string value = inputs[k].mode == MFH_OPERAND_SCALAR ? "s" + ks
                            : packed16[k] ? "mfh_h2f(w" + ks + "[u][j >> 1], j & 1)"
                                          : "a" + ks + "[u][j]";
        operands += "        const float x" + ks + " = " + value + ";\n";
    }
    src += "            float r[" + V + "];\n";
    if (emv.flagged) src += "            bool qv[" + V + "];\n";
    src += "#pragma unroll\n            for (int j = 0; j < " + V + "; j++) {\n";
    src += operands;
    if (emv.flagged) src += "        bool qe = false;\n";
    src += emv.body;
    src += "                r[j] = " + vresult + ";\n";
    if (emv.flagged) src += "                qv[j] = qe;\n";
    src += "            }\n";
    if (emv.flagged) {
        // the item's flagged elements again, with the reference forms
        src += "            bool qany = false;\n#pragma unroll\n            for (int j = 0; j < " + V +
               "; j++) qany |= qv[j];\n";
        src += "            if (qany) {\n#pragma unroll\n                for (int j = 0; j < " + V +
               "; j++) {\n                    if (!qv[j]) continue;\n";
        src += operands + emvf.body;
        src += "                    r[j] = " + vfresult + ";\n                }\n            }\n";
    }
    src += "            mfh_st" + V + "_" + osfx + "(pout, it * " + V + ", r);\n        }\n    }\n";
    // scalar tail (and the whole range when the vector path is off)
    src += "    for (mfh_i64 i = nvec * " + V + " + tid; i < n; i += stride) {\n";
    for (int k = 0; k < n_inputs; k++) {
        std::string ks = std::to_string(k);
        if (inputs[k].mode == MFH_OPERAND_SCALAR)
            src += "        const float x" + ks + " = s" + ks + ";\n";
        else
            src += "        const float x" + ks + " = mfh_ld1_" + io_suffix(inputs[k].dtype) + "(p" + ks + ", " +
                   operand_index(inputs[k], "i") + ");\n";
    }
    if (em.flagged) src += "        bool qe = false;\n";
    src += em.body;
    src += "        float res = " + result + ";\n";
    if (em.flagged) src += "        if (qe) {\n" + emf.body + "        res = " + fresult + ";\n        }\n";
    src += std::string("        mfh_st1_") + osfx + "(pout, i, res);\n    }\n}\n";

    auto kernel = std::make_unique<mfh_kernel>();
    kernel->identifier = identifier;
    kernel->kernel_name = kernel_name;
    kernel->source = std::move(src);
    kernel->inputs.assign(inputs, inputs + n_inputs);
    kernel->out_dtype = out_dtype;
    kernel->vec = vec;
    kernel->unroll = unroll;
    kernel->block = block;
    kernel->auto_bpc = auto_bpc;
    kernel->periods_vectorizable = periods_vectorizable;
    MFH_TRY(compile_source(kernel->source, kernel_name, &kernel->code));
    *out = kernel.release();
    return MFH_OK;
}

void HipLaunch::bind()
{
    args.clear();
    args.reserve(ptrs.size() + 3);
    for (const void*& p : ptrs) args.push_back(&p);
    args.push_back(&out);
    args.push_back(&count);
    args.push_back(&nvec);
}

int prepare_hip(const mfh_kernel* kernel, const void* const* inputs, int n_inputs, void* out, int64_t count,
                bool may_load, HipLaunch* launch)
{
    launch->grid = 0;
    if (!kernel) return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: kernel is empty");
    if (n_inputs != (int)kernel->inputs.size())
        return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: kernel \"%s\" expects %d inputs, got %d",
                    kernel->identifier.c_str(), (int)kernel->inputs.size(), n_inputs);
    if (count < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: negative count %lld", (long long)count);
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (count == 0) return MFH_OK;
    if (!out) return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: output buffer is NULL");
    // The vector path needs every streamed buffer aligned to one item's bytes.
    auto item_aligned = [&](const void* p, int dtype) {
        uintptr_t bytes = (uintptr_t)kernel->vec * (dtype == kFloat32 ? 4 : 2);
        return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
    };
    bool vec_ok = kernel->periods_vectorizable && item_aligned(out, kernel->out_dtype);
    for (int k = 0; k < n_inputs; k++) {
        if (!inputs[k])
            return fail(MFH_ERR_INVALID_ARGUMENT, "codegen hip: input %d is NULL", k);
        if (kernel->inputs[k].mode != MFH_OPERAND_SCALAR && !item_aligned(inputs[k], kernel->inputs[k].dtype))
            vec_ok = false;
    }
    MFH_TRY(load_function(*kernel->code, dev->ordinal, may_load, &launch->fn));
    const int64_t nvec = vec_ok ? count / kernel->vec : 0;
    int64_t items = nvec > 0 ? (nvec + kernel->unroll - 1) / kernel->unroll : count;
    int64_t need = (items + kernel->block - 1) / kernel->block;
    int bpc = blocks_per_cu(Kern::kFused) > 0 ? blocks_per_cu(Kern::kFused) : kernel->auto_bpc;
    int64_t cap = std::min<int64_t>((int64_t)dev->compute_units * bpc, (int64_t(1) << 32) / kernel->block - 1);
    launch->grid = (unsigned)std::max<int64_t>(1, std::min(need, cap));
    launch->block = (unsigned)kernel->block;
    launch->ptrs.assign(inputs, inputs + n_inputs);
    launch->out = out;
    launch->count = count;
    launch->nvec = nvec;
    return MFH_OK;
}

int run_hip(const mfh_kernel* kernel, const void* const* inputs, int n_inputs, void* out, int64_t count,
            hipStream_t stream, bool may_load)
{
    HipLaunch l;
    MFH_TRY(prepare_hip(kernel, inputs, n_inputs, out, count, may_load, &l));
    if (l.grid == 0) return MFH_OK;
    l.bind();
    return check_hip(hipModuleLaunchKernel(l.fn, l.grid, 1, 1, l.block, 1, 1, 0, stream, l.args.data(), nullptr),
                     "hipModuleLaunchKernel");
}

uint64_t module_generation() { return g_module_generation.load(); }

void release_kernel_cache()
{
    std::lock_guard<std::mutex> lock(g_cache_mu);
    g_module_generation.fetch_add(1);
    for (auto& kv : g_cache) {
        std::lock_guard<std::mutex> obj_lock(kv.second->mu);
        if (kv.second->module) (void)hipModuleUnload(kv.second->module);
        kv.second->module = nullptr;
        kv.second->function = nullptr;
    }
    g_cache.clear();
}

}  // namespace mfh

using namespace mfh;

extern "C" {

int mfh_fusion_compile(const mfh_ast_node* nodes, int32_t n_nodes, const mfh_operand* inputs, int32_t n_inputs,
                       uint8_t out_dtype, const char* output_port, uint32_t flags, mfh_kernel** kernel)
{
    return emit_hip(nodes, n_nodes, inputs, n_inputs, out_dtype, output_port, flags, kernel);
}

int mfh_fusion_cache_dir(const char* dir)
{
    std::lock_guard<std::mutex> lock(g_disk_mu);
    g_disk_dir = dir ? dir : "";
    while (g_disk_dir.size() > 1 && g_disk_dir.back() == '/') g_disk_dir.pop_back();
    g_disk_dir_set = true;
    return MFH_OK;
}

int mfh_fusion_cache_stats(int64_t* compiles, int64_t* disk_hits)
{
    if (compiles) *compiles = g_compiles.load();
    if (disk_hits) *disk_hits = g_disk_hits.load();
    return MFH_OK;
}

const char* mfh_fusion_source(const mfh_kernel* kernel) { return kernel ? kernel->source.c_str() : nullptr; }
const char* mfh_fusion_kernel_name(const mfh_kernel* kernel) { return kernel ? kernel->kernel_name.c_str() : nullptr; }
const char* mfh_fusion_identifier(const mfh_kernel* kernel) { return kernel ? kernel->identifier.c_str() : nullptr; }
int32_t mfh_fusion_num_inputs(const mfh_kernel* kernel) { return kernel ? (int32_t)kernel->inputs.size() : -1; }

int mfh_fusion_launch(const mfh_kernel* kernel, const void* const* inputs, int32_t n_inputs, void* out,
                      int64_t count, void* stream)
{
    return run_hip(kernel, inputs, n_inputs, out, count, (hipStream_t)stream);
}

int mfh_fusion_release(mfh_kernel* kernel)
{
    delete kernel;
    return MFH_OK;
}

}  // extern "C"
