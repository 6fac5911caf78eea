// runtime.cpp — device binding, memory, copies, streams and error state.
#include <atomic>
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "common.hpp"
#include "scratch.hpp"

namespace mfh {

namespace {
thread_local std::string t_last_error;
// Sticky errors of entry points without an error channel, one per stream the
// failed work was meant for: each stream's owner collects its own at its
// next synchronisation, whichever thread fails or syncs first.
struct Sticky {
    int code = MFH_OK;
    std::string msg;
};
std::mutex g_sticky_mu;
std::unordered_map<hipStream_t, Sticky> g_sticky;
std::mutex g_init_mu;
Device g_device;
std::atomic<bool> g_ready{false};

std::string vformat(const char* fmt, va_list ap)
{
    char buf[1024];
    vsnprintf(buf, sizeof buf, fmt, ap);
    return buf;
}
}  // namespace

int fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    t_last_error = vformat(fmt, ap);
    va_end(ap);
    return code;
}

void fail_sticky(hipStream_t stream, int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::string msg = vformat(fmt, ap);
    va_end(ap);
    std::lock_guard<std::mutex> lock(g_sticky_mu);
    Sticky& e = g_sticky[stream];
    if (e.code == MFH_OK) {  // the first failure on a stream is the one reported
        e.code = code;
        e.msg = msg;
    }
    t_last_error = msg;
}

int take_sticky(hipStream_t stream)
{
    std::lock_guard<std::mutex> lock(g_sticky_mu);
    auto it = g_sticky.find(stream);
    if (it == g_sticky.end()) return MFH_OK;
    const int code = it->second.code;
    t_last_error = it->second.msg;
    g_sticky.erase(it);
    return code;
}

void drop_sticky(hipStream_t stream)
{
    std::lock_guard<std::mutex> lock(g_sticky_mu);
    g_sticky.erase(stream);
}

int check_hip(hipError_t err, const char* what)
{
    if (err == hipSuccess) return MFH_OK;
    return fail(MFH_ERR_DEVICE, "%s: %s", what, hipGetErrorString(err));
}

int dtype_size(int dtype)
{
    switch (dtype) {
    case kFloat64: case kInt64: case kUint64: return 8;
    case kFloat32: case kInt32: case kUint32: return 4;
    case kFloat16: case kBFloat16: case kInt16: case kUint16: return 2;
    case kF8E4M3: case kF8E5M2: case kInt8: case kUint8: return 1;
    default: return 0;
    }
}

const char* dtype_name(int dtype)
{
    switch (dtype) {
    case kFloat64: return "f64";
    case kFloat32: return "f32";
    case kFloat16: return "f16";
    case kBFloat16: return "bf16";
    case kF8E4M3: return "fp8e4m3";
    case kF8E5M2: return "fp8e5m2";
    case kInt64: return "i64";
    case kInt32: return "i32";
    case kInt16: return "i16";
    case kInt8: return "i8";
    case kInt4: return "i4";
    case kUint64: return "u64";
    case kUint32: return "u32";
    case kUint16: return "u16";
    case kUint8: return "u8";
    case kBool: return "bool";
    default: return "invalid";
    }
}

const char* dtype_string(int dt)
{
    switch (dt) {
    case kInvalid: return "INVALID";
    case kFloat64: return "F64";
    case kFloat32: return "F32";
    case kFloat16: return "F16";
    case kBFloat16: return "BF16";
    case kF8E4M3: return "F8E4M3";
    case kF8E5M2: return "F8E5M2";
    case kInt64: return "I64";
    case kInt32: return "I32";
    case kInt16: return "I16";
    case kInt8: return "I8";
    case kInt4: return "I4";
    case kUint64: return "U64";
    case kUint32: return "U32";
    case kUint16: return "U16";
    case kUint8: return "U8";
    case kBool: return "BOOL";
    case kComplex64: return "C64";
    case kComplex128: return "C128";
    default: {
        thread_local char buf[24];
        snprintf(buf, sizeof buf, "DTYPE(%d)", dt);
        return buf;
    }
    }
}

int64_t bytes_for(int dt, int64_t elements)
{
    if (elements < 0) return -1;
    switch (dt) {
    case kInt4: return (elements + 1) / 2;
    case kBool: return (elements + 7) / 8;
    case kComplex64: return elements * 8;
    case kComplex128: return elements * 16;
    default: {
        const int size = dtype_size(dt);
        return size > 0 ? elements * size : -1;
    }
    }
}

int bind_device(const Device** out)
{
    if (!g_ready.load(std::memory_order_acquire))
        return fail(MFH_ERR_NOT_INITIALIZED, "mfh: mfh_init has not been called");
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess || current != g_device.ordinal)
        MFH_TRY(check_hip(hipSetDevice(g_device.ordinal), "hipSetDevice"));
    *out = &g_device;
    return MFH_OK;
}

void release_kernel_cache();  // fusion.cpp

// ---- launch shapes ------------------------------------------------------------

namespace {
struct LaunchCfg {
    const char* name;
    std::atomic<int> bpc;
    std::atomic<int> unroll;  // 0: the kernel family chooses (fused: per kernel)
    std::atomic<int> threads;  // threads per workgroup; 0: the family's default
    unsigned allowed;          // workgroup sizes the family runs: bit k set for 2^k threads
    int default_bpc = 0, default_unroll = 0, default_threads = 0;  // filled from the initial values
};
// Large enough that every thread runs exactly one step at any size that
// fits in HBM (the grid is also capped by the work itself): "one-shot"
// grids, whose blocks each stream one chunk and exit.
constexpr int kMaxBlocksPerCu = 1 << 16;
// Defaults measured on MI355X (256 CUs) with streaming loads and stores:
// every family runs one-shot, FP8 and Int4 with two items per thread, axpy
// and the casts with one.  Workgroup sizes (BASELINE sizes, graph-timed
// bench, against 256 threads): FP8 128 (+0.4%; 64 is slower), axpy 64
// (+2.3%; 128 is slower), Int4 512 (+0.5% in the bench's paired runs, +1.3%
// with eager launches at 1x and 4x the BASELINE size; 128 and 64 lose 2-3%,
// 1024 loses 3-10%).  0 for the fused
// family means "per kernel": each generated kernel carries its shape (see
// fusion.cpp), one-wave workgroups unless set; for the casts "per cast"
// (cast_threads in dequant.hip).
constexpr unsigned kSizes64To256 = (1u << 6) | (1u << 7) | (1u << 8);
constexpr unsigned kSizes64To512 = kSizes64To256 | (1u << 9);
constexpr unsigned kSizes64To1024 = kSizes64To512 | (1u << 10);
LaunchCfg g_cfg[(int)Kern::kCount] = {
    {"fp8", {kMaxBlocksPerCu}, {2}, {128}, kSizes64To256},
    {"int4", {kMaxBlocksPerCu}, {2}, {512}, kSizes64To512},
    {"axpy", {kMaxBlocksPerCu}, {1}, {64}, kSizes64To256},
    {"axpy16", {kMaxBlocksPerCu}, {1}, {64}, kSizes64To256},
    {"convert", {kMaxBlocksPerCu}, {0}, {0}, kSizes64To256},  // 0: per cast
    {"fused", {0}, {0}, {0}, kSizes64To1024},
};

bool threads_supported(const LaunchCfg& c, int threads)
{
    return threads > 0 && threads <= 1024 && (threads & (threads - 1)) == 0 &&
           (c.allowed & (unsigned)threads) != 0;
}

std::string allowed_sizes(const LaunchCfg& c)
{
    std::string text;
    for (int t = 64; t <= 1024; t *= 2)
        if (c.allowed & (unsigned)t) text += (text.empty() ? "" : ", ") + std::to_string(t);
    return text;
}
std::once_flag g_cfg_env_once;

void read_cfg_env()
{
    for (auto& c : g_cfg) {
        c.default_bpc = c.bpc.load();
        c.default_unroll = c.unroll.load();
        c.default_threads = c.threads.load();
    }
    const char* all = std::getenv("MFH_BLOCKS_PER_CU");
    for (auto& c : g_cfg) {
        std::string upper(c.name);
        for (auto& ch : upper) ch = (char)toupper(ch);
        const char* bpc = std::getenv(("MFH_BPC_" + upper).c_str());
        if (!bpc) bpc = all;
        const char* un = std::getenv(("MFH_UNROLL_" + upper).c_str());
        if (bpc && atoi(bpc) > 0 && atoi(bpc) <= kMaxBlocksPerCu) c.bpc = atoi(bpc);
        if (un && (atoi(un) == 1 || atoi(un) == 2 || atoi(un) == 4)) c.unroll = atoi(un);
        const char* th = std::getenv(("MFH_THREADS_" + upper).c_str());
        if (th && threads_supported(c, atoi(th))) c.threads = atoi(th);
    }
}

LaunchCfg* find_cfg(const char* name)
{
    std::call_once(g_cfg_env_once, read_cfg_env);
    if (!name) return nullptr;
    for (auto& c : g_cfg)
        if (strcmp(c.name, name) == 0) return &c;
    return nullptr;
}
}  // namespace

int blocks_per_cu(Kern k)
{
    std::call_once(g_cfg_env_once, read_cfg_env);
    return g_cfg[(int)k].bpc.load(std::memory_order_relaxed);
}

int items_per_thread(Kern k)
{
    std::call_once(g_cfg_env_once, read_cfg_env);
    return g_cfg[(int)k].unroll.load(std::memory_order_relaxed);
}

int threads_per_block(Kern k)
{
    std::call_once(g_cfg_env_once, read_cfg_env);
    return g_cfg[(int)k].threads.load(std::memory_order_relaxed);
}

}  // namespace mfh

using namespace mfh;

extern "C" {

int mfh_version(void) { return 100; }

const char* mfh_last_error(void) { return t_last_error.c_str(); }

int mfh_take_sticky_error(void* stream) { return take_sticky((hipStream_t)stream); }

int mfh_init(int device)
{
    std::lock_guard<std::mutex> lock(g_init_mu);
    if (g_ready.load() && g_device.ordinal == device) return MFH_OK;
    int count = 0;
    MFH_TRY(check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount"));
    if (device < 0 || device >= count)
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_init: device %d out of range [0, %d)", device, count);
    MFH_TRY(check_hip(hipSetDevice(device), "hipSetDevice"));
    hipDeviceProp_t prop;
    MFH_TRY(check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"));
    // the allocation-free graph call's scratch address on this device
    MFH_TRY(scratch_setup(device));
    g_device.ordinal = device;
    g_device.compute_units = prop.multiProcessorCount;
    g_device.total_bytes = (int64_t)prop.totalGlobalMem;
    g_ready.store(true, std::memory_order_release);
    return MFH_OK;
}

int mfh_shutdown(void)
{
    std::lock_guard<std::mutex> lock(g_init_mu);
    release_kernel_cache();
    g_ready.store(false);
    return MFH_OK;
}

int mfh_capabilities(int64_t* max_bytes, int32_t* native_alignment, int32_t* compute_units)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (max_bytes) *max_bytes = dev->total_bytes;
    if (native_alignment) *native_alignment = 256;
    if (compute_units) *compute_units = dev->compute_units;
    return MFH_OK;
}

int mfh_set_launch_config(const char* kernel, int32_t blocks_per_cu, int32_t items_per_thread)
{
    LaunchCfg* c = find_cfg(kernel);
    if (!c) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_set_launch_config: unknown kernel family \"%s\"", kernel ? kernel : "(null)");
    if (blocks_per_cu > kMaxBlocksPerCu || blocks_per_cu < -1)
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_set_launch_config: blocks_per_cu %d is not in -1..%d", blocks_per_cu,
                    kMaxBlocksPerCu);
    if (items_per_thread < -1 || (items_per_thread > 0 && items_per_thread != 1 && items_per_thread != 2 &&
                                  items_per_thread != 4))
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_set_launch_config: items_per_thread must be 1, 2 or 4 (or 0, -1)");
    if (blocks_per_cu > 0) c->bpc = blocks_per_cu;
    else if (blocks_per_cu == -1) c->bpc = c->default_bpc;
    if (items_per_thread > 0) c->unroll = items_per_thread;
    else if (items_per_thread == -1) c->unroll = c->default_unroll;
    return MFH_OK;
}

int mfh_get_launch_config(const char* kernel, int32_t* blocks_per_cu, int32_t* items_per_thread)
{
    LaunchCfg* c = find_cfg(kernel);
    if (!c) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_get_launch_config: unknown kernel family \"%s\"", kernel ? kernel : "(null)");
    if (blocks_per_cu) *blocks_per_cu = c->bpc;
    if (items_per_thread) *items_per_thread = c->unroll;
    return MFH_OK;
}

int mfh_set_launch_threads(const char* kernel, int32_t threads)
{
    LaunchCfg* c = find_cfg(kernel);
    if (!c) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_set_launch_threads: unknown kernel family \"%s\"", kernel ? kernel : "(null)");
    if (threads == 0) return MFH_OK;
    if (threads == -1) {
        c->threads = c->default_threads;
        return MFH_OK;
    }
    if (!threads_supported(*c, threads))
        return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_set_launch_threads: \"%s\" kernels run workgroups of %s threads, not %d",
                    c->name, allowed_sizes(*c).c_str(), threads);
    c->threads = threads;
    return MFH_OK;
}

int mfh_get_launch_threads(const char* kernel, int32_t* threads)
{
    LaunchCfg* c = find_cfg(kernel);
    if (!c) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_get_launch_threads: unknown kernel family \"%s\"", kernel ? kernel : "(null)");
    if (threads) *threads = c->threads;
    return MFH_OK;
}

int mfh_alloc(void** ptr, size_t bytes)
{
    if (!ptr) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_alloc: ptr is NULL");
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    *ptr = nullptr;
    if (bytes == 0) return MFH_OK;
    return check_hip(hipMalloc(ptr, bytes), "hipMalloc");
}

int mfh_free(void* ptr)
{
    if (!ptr) return MFH_OK;
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    return check_hip(hipFree(ptr), "hipFree");
}

int mfh_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (bytes == 0) return MFH_OK;
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream),
                     "hipMemcpyAsync(H2D)");
}

int mfh_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (bytes == 0) return MFH_OK;
    MFH_TRY(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream),
                      "hipMemcpyAsync(D2H)"));
    return check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int mfh_stream_sync(void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    MFH_TRY(check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize"));
    return take_sticky((hipStream_t)stream);
}

}  // extern "C"
