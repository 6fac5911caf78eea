// backend.cpp — the HIP tensor backend: device-resident tensors behind the
// tensor.Backend / tensor.Tensor contract (tensor/backend.go:18-68,
// tensor/tensor.go:53-130), uploads that stream through pinned staging and
// dequantise FP8 / Int4 on the device, and the resident axpy
// (runtime/axpy.go:44-93).
//
// A backend owns one HIP stream, a ring of two pinned host chunks and two
// device staging chunks.  An upload copies chunk i into a pinned slot (split
// over the host copy threads of hostcopy.cpp) while the DMA (and dequant
// kernel) of chunk i-1 runs from the other slot; a slot is reused once the
// event recorded after its last reader has fired.
// Tensors share their storage with their views; the storage and the backend
// state outlive a released backend handle until the last tensor handle goes,
// so a stale tensor reports closed instead of touching freed memory.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <vector>

#include "../../include/mfh_backend.h"
#include "backend_internal.hpp"
#include "common.hpp"
#include "hostcopy.hpp"

namespace mfh {
namespace {

constexpr size_t kChunk = 16u << 20;  // bytes of source data per staging chunk
constexpr int kRing = 2;

bool stored_as_is(int dt) { return dt == kFloat32 || dt == kFloat16 || dt == kBFloat16; }
bool dequantised(int dt) { return dt == kF8E4M3 || dt == kF8E5M2 || dt == kInt4; }

struct Storage {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool freed = false;
    bool pending = false;
    hipEvent_t done = nullptr;       // recorded after the last queued work that touches it
    hipStream_t writer = nullptr;    // stream of the last resident axpy that wrote it
    // Set once mfh_tensor_dispatch_pointer has handed the device address out:
    // the caller's own launches on it are not ordered through `done`.
    std::atomic<bool> exposed{false};
};

struct BackendState {
    std::mutex mu;
    int device = -1;
    bool closed = false;
    hipStream_t stream = nullptr;
    void* pinned[kRing] = {nullptr, nullptr};
    void* dstage[kRing] = {nullptr, nullptr};
    hipEvent_t slot_free[kRing] = {nullptr, nullptr};
    // The slot the next chunk takes.  It carries over from one upload to the
    // next, so the first chunk of an upload queued behind an asynchronous one
    // fills the slot that upload's last chunk is not using.
    int next_slot = 0;
    std::set<std::shared_ptr<Storage>> owned;
    // Device blocks of closed tensors, kept for later tensors of the same
    // byte size: a hipMalloc of a 117 MB tensor took about a tenth of its
    // PCIe upload.  A block enters only after every queued use of it has
    // finished (a close waits for that), so a new tensor gets idle memory.
    // At most kCacheCap bytes are kept; hipMalloc failure and shutdown
    // return them.
    static constexpr size_t kCacheCap = size_t(2) << 30;
    std::multimap<size_t, void*> cache;
    size_t cached = 0;

    ~BackendState() { shut(); }

    int alloc(size_t bytes, void** p)
    {
        auto it = cache.find(bytes);
        if (it != cache.end()) {
            *p = it->second;
            cached -= bytes;
            cache.erase(it);
            return MFH_OK;
        }
        if (hipMalloc(p, bytes) == hipSuccess) return MFH_OK;
        (void)hipGetLastError();
        trim(0);
        return check_hip(hipMalloc(p, bytes), "hipMalloc");
    }

    // `p` must be idle: no queued work may still touch it.
    int release(void* p, size_t bytes)
    {
        if (bytes > kCacheCap) return check_hip(hipFree(p), "hipFree");
        cache.emplace(bytes, p);
        cached += bytes;
        return trim(kCacheCap);
    }

    int trim(size_t cap)
    {
        int rc = MFH_OK;
        while (cached > cap && !cache.empty()) {
            auto it = cache.begin();  // smallest first: the big blocks are the expensive ones to remake
            const int r = check_hip(hipFree(it->second), "hipFree");
            if (rc == MFH_OK) rc = r;
            cached -= it->first;
            cache.erase(it);
        }
        return rc;
    }

    // Frees everything; storage handles left in tensors see `freed`.
    int shut()
    {
        if (closed) return MFH_OK;
        closed = true;
        int rc = MFH_OK;
        auto keep = [&](hipError_t e, const char* what) {
            if (e != hipSuccess && rc == MFH_OK) rc = check_hip(e, what);
        };
        if (stream) keep(hipStreamSynchronize(stream), "hipStreamSynchronize");
        for (const auto& s : owned) {
            // work queued on another backend's stream (a resident axpy) may
            // still touch it
            if (s->pending && s->done) keep(hipEventSynchronize(s->done), "hipEventSynchronize");
            if (s->done) keep(hipEventDestroy(s->done), "hipEventDestroy");
            s->done = nullptr;
            if (s->ptr) keep(hipFree(s->ptr), "hipFree");
            s->ptr = nullptr;
            s->freed = true;
            s->pending = false;
        }
        owned.clear();
        keep(trim(0) == MFH_OK ? hipSuccess : hipErrorUnknown, "hipFree(block cache)");
        for (int i = 0; i < kRing; i++) {
            if (pinned[i]) keep(hipHostFree(pinned[i]), "hipHostFree");
            if (dstage[i]) keep(hipFree(dstage[i]), "hipFree");
            if (slot_free[i]) keep(hipEventDestroy(slot_free[i]), "hipEventDestroy");
            pinned[i] = dstage[i] = nullptr;
            slot_free[i] = nullptr;
        }
        if (stream) {
            drop_sticky(stream);
            keep(hipStreamDestroy(stream), "hipStreamDestroy");
        }
        stream = nullptr;
        return rc;
    }
};

}  // namespace
}  // namespace mfh

struct mfh_backend {
    std::shared_ptr<mfh::BackendState> state;
};

struct mfh_tensor {
    std::shared_ptr<mfh::BackendState> backend;
    std::shared_ptr<mfh::Storage> storage;
    bool owner = true;  // views share storage without owning it
    bool closed = false;
    int64_t offset = 0;  // bytes from the storage base (slices)
    std::vector<int64_t> dims;
    int64_t elements = 0;
    uint8_t dtype = mfh::kInvalid;
};

namespace mfh {
namespace {

int backend_ok(const mfh_backend* b, const Device** dev)
{
    if (!b || !b->state) return fail(MFH_ERR_INVALID_ARGUMENT, "backend is NULL");
    if (b->state->closed) return fail(MFH_ERR_CLOSED, "tensor: backend closed");
    return bind_device(dev);
}

bool tensor_dead(const mfh_tensor* t) { return !t || t->closed || !t->storage || t->storage->freed; }

int tensor_ok(const mfh_tensor* t)
{
    if (!t) return fail(MFH_ERR_INVALID_ARGUMENT, "tensor is NULL");
    if (tensor_dead(t)) return fail(MFH_ERR_TENSOR_CLOSED, "tensor: closed");
    return MFH_OK;
}

// The device address of a live tensor, for this library's own launches,
// which order themselves through the storage's `done` event.
void* device_address(const mfh_tensor* t)
{
    if (tensor_dead(t) || !t->storage->ptr) return nullptr;
    return static_cast<uint8_t*>(t->storage->ptr) + t->offset;
}

}  // namespace

// NewShape (tensor/shape.go:32-60): negative dimensions and overflowing
// products are invalid; any zero dimension makes the element count zero.
int make_shape(const int64_t* shape, int32_t rank, std::vector<int64_t>* dims, int64_t* elements)
{
    if (rank < 0 || (rank > 0 && !shape)) return fail(MFH_ERR_SHAPE_INVALID, "tensor: invalid shape");
    dims->assign(shape, shape + rank);
    int64_t n = 1;
    bool zero = false;
    for (int32_t i = 0; i < rank; i++) {
        if (shape[i] < 0)
            return fail(MFH_ERR_SHAPE_INVALID, "tensor: invalid shape: dimension %d is negative (%lld)", (int)i,
                        (long long)shape[i]);
        if (shape[i] == 0) {
            zero = true;
            continue;
        }
        if (n > INT64_MAX / shape[i])
            return fail(MFH_ERR_SHAPE_INVALID, "tensor: invalid shape: element count overflows int");
        n *= shape[i];
    }
    *elements = zero ? 0 : n;
    return MFH_OK;
}

namespace {

int ensure_staging(BackendState& s)
{
    for (int i = 0; i < kRing; i++) {
        if (!s.pinned[i]) MFH_TRY(check_hip(hipHostMalloc(&s.pinned[i], kChunk, hipHostMallocDefault), "hipHostMalloc"));
        if (!s.dstage[i]) MFH_TRY(check_hip(hipMalloc(&s.dstage[i], kChunk), "hipMalloc(staging)"));
        if (!s.slot_free[i])
            MFH_TRY(check_hip(hipEventCreateWithFlags(&s.slot_free[i], hipEventDisableTiming), "hipEventCreate"));
    }
    return MFH_OK;
}

struct MemorySource : Source {
    const uint8_t* base;
    explicit MemorySource(const void* p) : base(static_cast<const uint8_t*>(p)) {}
    int read(void* dst, size_t offset, size_t len) override
    {
        std::memcpy(dst, base + offset, len);
        return MFH_OK;
    }
};

// Queues the upload of `n_src` source bytes holding `elements` elements into
// `dst` (already allocated for the stored dtype) on the backend stream.
// A scaled Int4 chunk holds whole scale groups of nibbles; its scales follow
// its nibbles in the same staging slot (at a 16-byte aligned offset) and
// cross PCIe in the same copy.
int stream_in(BackendState& s, const Plan& p, Source& src, size_t n_src, int64_t elements, Storage& dst)
{
    if (n_src == 0) return MFH_OK;
    MFH_TRY(ensure_staging(s));
    const bool convert = dequantised(p.src) || p.out != p.src;
    const bool scaled4 = p.src == kInt4 && p.scales;
    const size_t ssize = scaled4 ? (size_t)dtype_size(p.scale_dt) : 0;
    // Source bytes per chunk: whole Int4 bytes and whole scale groups, with
    // room for the chunk's scales.
    size_t chunk = kChunk;
    if (scaled4) {
        const int64_t unit = p.group % 2 ? 2 * p.group : p.group;  // nibbles: whole groups and whole bytes
        const double bytes_per_nibble = 0.5 + (double)ssize / (double)p.group;
        const int64_t units = (int64_t)(((double)kChunk - 16.0) / bytes_per_nibble) / unit;
        if (units < 1)
            return fail(MFH_ERR_INVALID_ARGUMENT, "upload: group %lld exceeds a staging chunk", (long long)p.group);
        chunk = (size_t)(units * unit / 2);
    }
    const int out_size = dtype_size(p.out);
    size_t done = 0;
    while (done < n_src) {
        const int slot = s.next_slot;
        s.next_slot = (slot + 1) % kRing;
        const size_t len = std::min(chunk, n_src - done);
        int64_t first = 0, count = 0;  // elements of this chunk
        if (p.src == kInt4) {
            first = (int64_t)done * 2;
            count = std::min<int64_t>((int64_t)len * 2, elements - first);
        } else if (convert) {
            const int in_size = dtype_size(p.src);
            first = (int64_t)done / in_size;
            count = (int64_t)len / in_size;
        }
        const size_t scale_at = (len + 15) & ~(size_t)15;
        const size_t scale_len = scaled4 ? (size_t)((count + p.group - 1) / p.group) * ssize : 0;
        MFH_TRY(check_hip(hipEventSynchronize(s.slot_free[slot]), "hipEventSynchronize"));
        uint8_t* slot_at = static_cast<uint8_t*>(s.pinned[slot]);
        MFH_TRY(for_each_piece(len, [&](size_t lo, size_t hi) { return src.read(slot_at + lo, done + lo, hi - lo); }));
        if (scaled4)
            MFH_TRY(p.scales->read(static_cast<uint8_t*>(s.pinned[slot]) + scale_at, (size_t)(first / p.group) * ssize,
                                   scale_len));
        if (!convert) {
            MFH_TRY(check_hip(hipMemcpyAsync(static_cast<uint8_t*>(dst.ptr) + done, s.pinned[slot], len,
                                             hipMemcpyHostToDevice, s.stream), "hipMemcpyAsync(H2D)"));
        } else {
            const size_t copy = scaled4 ? scale_at + scale_len : len;
            MFH_TRY(check_hip(hipMemcpyAsync(s.dstage[slot], s.pinned[slot], copy, hipMemcpyHostToDevice, s.stream),
                              "hipMemcpyAsync(H2D)"));
            void* out = static_cast<uint8_t*>(dst.ptr) + first * out_size;
            int rc;
            if (p.src == kF8E4M3 || p.src == kF8E5M2)
                rc = mfh_dequant_fp8(out, (uint8_t)p.out, s.dstage[slot], (uint8_t)p.src, count, p.scale, s.stream);
            else if (scaled4)
                rc = mfh_dequant_int4(out, (uint8_t)p.out, s.dstage[slot], count,
                                      static_cast<const uint8_t*>(s.dstage[slot]) + scale_at, (uint8_t)p.scale_dt,
                                      p.group, s.stream);
            else
                rc = mfh_convert(out, (uint8_t)p.out, s.dstage[slot], (uint8_t)p.src, count, s.stream);
            MFH_TRY(rc);
        }
        MFH_TRY(check_hip(hipEventRecord(s.slot_free[slot], s.stream), "hipEventRecord"));
        done += len;
    }
    return MFH_OK;
}

int wait_storage(Storage& st)
{
    if (st.pending && st.done) MFH_TRY(check_hip(hipEventSynchronize(st.done), "hipEventSynchronize"));
    st.pending = false;
    return MFH_OK;
}

// Marks work just queued on `stream` as the storage's last: every later
// reader, close or backend shutdown waits for it through `done`.
int mark_pending(Storage& st, hipStream_t stream)
{
    if (!st.done) MFH_TRY(check_hip(hipEventCreateWithFlags(&st.done, hipEventDisableTiming), "hipEventCreate"));
    MFH_TRY(check_hip(hipEventRecord(st.done, stream), "hipEventRecord"));
    st.pending = true;
    return MFH_OK;
}

// The sticky error a tensor's owner sees at Sync / Download: its backend
// stream's first, else that of the stream whose resident axpy last wrote it.
int take_tensor_sticky(hipStream_t own, const Storage& st)
{
    int rc = take_sticky(own);
    if (rc == MFH_OK && st.writer && st.writer != own) rc = take_sticky(st.writer);
    return rc;
}

// Holds the mutexes of distinct backend states, taken in address order so
// that threads combining the same backends in different roles cannot
// deadlock.
struct StateLocks {
    std::vector<std::unique_lock<std::mutex>> held;
    explicit StateLocks(std::vector<BackendState*> states)
    {
        std::sort(states.begin(), states.end());
        states.erase(std::unique(states.begin(), states.end()), states.end());
        for (BackendState* b : states) held.emplace_back(b->mu);
    }
};

}  // namespace

int upload_from(mfh_backend* b, const int64_t* shape, int32_t rank, const Plan& plan, Source& source,
                size_t n_bytes, bool wait, mfh_tensor** out)
{
    if (!out) return fail(MFH_ERR_INVALID_ARGUMENT, "upload: tensor out-pointer is NULL");
    *out = nullptr;
    const Device* dev;
    MFH_TRY(backend_ok(b, &dev));
    BackendState& s = *b->state;
    std::lock_guard<std::mutex> lock(s.mu);
    auto t = std::make_unique<mfh_tensor>();
    MFH_TRY(make_shape(shape, rank, &t->dims, &t->elements));
    const int64_t expected = bytes_for(plan.src, t->elements);
    if (expected < 0) return fail(MFH_ERR_DTYPE_UNSUPPORTED, "tensor: dtype not supported by backend");
    if ((int64_t)n_bytes != expected)
        return fail(MFH_ERR_SHAPE_MISMATCH, "tensor: shape mismatch: %zu bytes for %lld elements of %s (want %lld)",
                    n_bytes, (long long)t->elements, dtype_string(plan.src), (long long)expected);
    auto st = std::make_shared<Storage>();
    st->bytes = (size_t)t->elements * dtype_size(plan.out);
    if (st->bytes) MFH_TRY(s.alloc(st->bytes, &st->ptr));
    int rc = stream_in(s, plan, source, n_bytes, t->elements, *st);
    if (rc == MFH_OK) rc = check_hip(hipEventCreateWithFlags(&st->done, hipEventDisableTiming), "hipEventCreate");
    if (rc == MFH_OK) rc = check_hip(hipEventRecord(st->done, s.stream), "hipEventRecord");
    if (rc == MFH_OK && wait) rc = check_hip(hipEventSynchronize(st->done), "hipEventSynchronize");
    if (rc != MFH_OK) {
        (void)hipStreamSynchronize(s.stream);
        if (st->done) (void)hipEventDestroy(st->done);
        if (st->ptr) (void)hipFree(st->ptr);
        return rc;
    }
    st->pending = !wait;
    s.owned.insert(st);
    t->backend = b->state;
    t->storage = std::move(st);
    t->dtype = (uint8_t)plan.out;
    *out = t.release();
    return MFH_OK;
}

namespace {

int upload(mfh_backend* b, const int64_t* shape, int32_t rank, const Plan& plan, const void* bytes, size_t n_bytes,
           bool wait, mfh_tensor** out)
{
    if (n_bytes > 0 && !bytes) {
        if (out) *out = nullptr;
        return fail(MFH_ERR_INVALID_ARGUMENT, "upload: bytes are NULL");
    }
    MemorySource src(bytes);
    return upload_from(b, shape, rank, plan, src, n_bytes, wait, out);
}

}  // namespace
}  // namespace mfh

using namespace mfh;

extern "C" {

int mfh_backend_open(int device, mfh_backend** backend)
{
    if (!backend) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_backend_open: backend out-pointer is NULL");
    *backend = nullptr;
    MFH_TRY(mfh_init(device));
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    auto b = std::make_unique<mfh_backend>();
    b->state = std::make_shared<BackendState>();
    b->state->device = dev->ordinal;
    MFH_TRY(check_hip(hipStreamCreate(&b->state->stream), "hipStreamCreate"));
    *backend = b.release();
    return MFH_OK;
}

const char* mfh_backend_location(const mfh_backend* backend) { return backend ? "hip" : nullptr; }

int32_t mfh_backend_supported_dtypes(const mfh_backend* backend, uint8_t* dtypes, int32_t cap)
{
    static const uint8_t kTypes[] = {kFloat32, kFloat16, kBFloat16, kF8E4M3, kF8E5M2, kInt4};
    if (!backend) return -1;
    for (int32_t i = 0; dtypes && i < cap && i < (int32_t)sizeof kTypes; i++) dtypes[i] = kTypes[i];
    return (int32_t)sizeof kTypes;
}

int32_t mfh_backend_supported_layouts(const mfh_backend* backend, uint8_t* layouts, int32_t cap)
{
    if (!backend) return -1;
    if (layouts && cap > 0) layouts[0] = 0;  // LayoutDense
    return 1;
}

int mfh_backend_capabilities(const mfh_backend* backend, mfh_backend_caps* caps)
{
    const Device* dev;
    MFH_TRY(backend_ok(backend, &dev));
    if (!caps) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_backend_capabilities: caps is NULL");
    *caps = mfh_backend_caps{dev->total_bytes, 1, 0, 0, 256, 1, 0};
    return MFH_OK;
}

int mfh_backend_upload(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t source_dtype,
                       const void* bytes, size_t n_bytes, mfh_tensor** tensor)
{
    if (!stored_as_is(source_dtype) && !dequantised(source_dtype)) {
        if (tensor) *tensor = nullptr;
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "tensor: dtype not supported by backend (%s)", dtype_string(source_dtype));
    }
    Plan p;
    p.src = source_dtype;
    p.out = stored_as_is(source_dtype) ? source_dtype : kBFloat16;
    return upload(backend, shape, rank, p, bytes, n_bytes, true, tensor);
}

int mfh_backend_upload_async(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t source_dtype,
                             const void* bytes, size_t n_bytes, mfh_tensor** tensor)
{
    if (!stored_as_is(source_dtype) && !dequantised(source_dtype)) {
        if (tensor) *tensor = nullptr;
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "tensor: dtype not supported by backend (%s)", dtype_string(source_dtype));
    }
    Plan p;
    p.src = source_dtype;
    p.out = stored_as_is(source_dtype) ? source_dtype : kBFloat16;
    return upload(backend, shape, rank, p, bytes, n_bytes, false, tensor);
}

int mfh_backend_upload_sparse(mfh_backend* backend)
{
    const Device* dev;
    MFH_TRY(backend_ok(backend, &dev));
    return fail(MFH_ERR_LAYOUT_UNSUPPORTED, "tensor: layout not supported");
}

}  // extern "C"

namespace {

int upload_fp8(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t fp8_dtype, const void* codes,
               size_t n_bytes, float scale, uint8_t out_dtype, bool wait, mfh_tensor** tensor)
{
    if (tensor) *tensor = nullptr;
    if (fp8_dtype != kF8E4M3 && fp8_dtype != kF8E5M2)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "upload_fp8: %s is not an FP8 dtype", dtype_string(fp8_dtype));
    if (!stored_as_is(out_dtype))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "upload_fp8: output dtype %s is not F32/F16/BF16", dtype_string(out_dtype));
    Plan p;
    p.src = fp8_dtype;
    p.out = out_dtype;
    p.scale = scale;
    return upload(backend, shape, rank, p, codes, n_bytes, wait, tensor);
}

int upload_int4(mfh_backend* backend, const int64_t* shape, int32_t rank, const void* packed, size_t n_bytes,
                const void* group_scales, uint8_t scale_dtype, int64_t group, uint8_t out_dtype, bool wait,
                mfh_tensor** tensor)
{
    if (tensor) *tensor = nullptr;
    const Device* dev;
    MFH_TRY(backend_ok(backend, &dev));
    if (scale_dtype != kFloat32 && scale_dtype != kFloat16 && scale_dtype != kBFloat16)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "upload_int4: scale dtype %s is not F32/F16/BF16", dtype_string(scale_dtype));
    if (!stored_as_is(out_dtype))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "upload_int4: output dtype %s is not F32/F16/BF16", dtype_string(out_dtype));
    if (group <= 0) return fail(MFH_ERR_INVALID_ARGUMENT, "upload_int4: group must be positive, got %lld", (long long)group);
    std::vector<int64_t> dims;
    int64_t elements;
    MFH_TRY(make_shape(shape, rank, &dims, &elements));
    const int64_t n_scales = (elements + group - 1) / group;
    if (n_scales > 0 && !group_scales) return fail(MFH_ERR_INVALID_ARGUMENT, "upload_int4: group scales are NULL");
    MemorySource scales(group_scales);
    Plan p;
    p.src = kInt4;
    p.out = out_dtype;
    p.scales = &scales;
    p.scale_dt = scale_dtype;
    p.group = group;
    return upload(backend, shape, rank, p, packed, n_bytes, wait, tensor);
}

}  // namespace

extern "C" {

int mfh_backend_upload_fp8(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t fp8_dtype,
                           const void* codes, size_t n_bytes, float scale, uint8_t out_dtype, mfh_tensor** tensor)
{
    return upload_fp8(backend, shape, rank, fp8_dtype, codes, n_bytes, scale, out_dtype, true, tensor);
}

int mfh_backend_upload_fp8_async(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t fp8_dtype,
                                 const void* codes, size_t n_bytes, float scale, uint8_t out_dtype,
                                 mfh_tensor** tensor)
{
    return upload_fp8(backend, shape, rank, fp8_dtype, codes, n_bytes, scale, out_dtype, false, tensor);
}

int mfh_backend_upload_int4(mfh_backend* backend, const int64_t* shape, int32_t rank, const void* packed,
                            size_t n_bytes, const void* group_scales, uint8_t scale_dtype, int64_t group,
                            uint8_t out_dtype, mfh_tensor** tensor)
{
    return upload_int4(backend, shape, rank, packed, n_bytes, group_scales, scale_dtype, group, out_dtype, true,
                       tensor);
}

int mfh_backend_upload_int4_async(mfh_backend* backend, const int64_t* shape, int32_t rank, const void* packed,
                                  size_t n_bytes, const void* group_scales, uint8_t scale_dtype, int64_t group,
                                  uint8_t out_dtype, mfh_tensor** tensor)
{
    return upload_int4(backend, shape, rank, packed, n_bytes, group_scales, scale_dtype, group, out_dtype, false,
                       tensor);
}

int mfh_backend_download(mfh_backend* backend, const mfh_tensor* tensor, uint8_t* dtype, void* dst, size_t dst_bytes,
                         size_t* n_bytes)
{
    const Device* dev;
    MFH_TRY(backend_ok(backend, &dev));
    MFH_TRY(tensor_ok(tensor));
    BackendState& s = *backend->state;
    std::lock_guard<std::mutex> lock(s.mu);
    Storage& st = *tensor->storage;
    MFH_TRY(wait_storage(st));
    const size_t bytes = (size_t)tensor->elements * dtype_size(tensor->dtype);
    if (dtype) *dtype = tensor->dtype;
    if (n_bytes) *n_bytes = bytes;
    if (bytes == 0) return MFH_OK;
    if (!dst || dst_bytes < bytes)
        return fail(MFH_ERR_INVALID_ARGUMENT, "download: destination holds %zu bytes, need %zu", dst_bytes, bytes);
    MFH_TRY(ensure_staging(s));
    const uint8_t* src = static_cast<const uint8_t*>(st.ptr) + tensor->offset;
    // D2H into the pinned ring; the host copy of chunk i-1 overlaps the DMA of chunk i.
    size_t prev_len = 0, prev_at = 0;
    int prev_slot = -1;
    for (size_t at = 0, c = 0; at < bytes || prev_slot >= 0; c++) {
        int slot = (int)(c % kRing);
        size_t len = at < bytes ? std::min(kChunk, bytes - at) : 0;
        if (len) {
            MFH_TRY(check_hip(hipMemcpyAsync(s.pinned[slot], src + at, len, hipMemcpyDeviceToHost, s.stream),
                              "hipMemcpyAsync(D2H)"));
            MFH_TRY(check_hip(hipEventRecord(s.slot_free[slot], s.stream), "hipEventRecord"));
        }
        if (prev_slot >= 0) {
            MFH_TRY(check_hip(hipEventSynchronize(s.slot_free[prev_slot]), "hipEventSynchronize"));
            MFH_TRY(copy_parallel(static_cast<uint8_t*>(dst) + prev_at, s.pinned[prev_slot], prev_len));
        }
        prev_slot = len ? slot : -1;
        prev_at = at;
        prev_len = len;
        at += len;
    }
    return take_tensor_sticky(s.stream, st);
}

int mfh_backend_close(mfh_backend* backend)
{
    if (!backend || !backend->state) return MFH_OK;
    std::lock_guard<std::mutex> lock(backend->state->mu);
    if (backend->state->closed) return MFH_OK;
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    return backend->state->shut();
}

int mfh_backend_release(mfh_backend* backend)
{
    if (!backend) return MFH_OK;
    int rc = mfh_backend_close(backend);
    delete backend;
    return rc;
}

uint8_t mfh_tensor_dtype(const mfh_tensor* t) { return t ? t->dtype : (uint8_t)kInvalid; }
int64_t mfh_tensor_len(const mfh_tensor* t) { return t ? t->elements : -1; }
int64_t mfh_tensor_bytes(const mfh_tensor* t) { return t ? bytes_for(t->dtype, t->elements) : -1; }

int32_t mfh_tensor_shape(const mfh_tensor* t, int64_t* dims, int32_t cap)
{
    if (!t) return -1;
    for (int32_t i = 0; dims && i < cap && i < (int32_t)t->dims.size(); i++) dims[i] = t->dims[i];
    return (int32_t)t->dims.size();
}

const char* mfh_tensor_location(const mfh_tensor* t) { return t ? "hip" : nullptr; }

int32_t mfh_tensor_state(const mfh_tensor* t)
{
    if (tensor_dead(t)) return MFH_STATE_CLOSED;
    std::lock_guard<std::mutex> lock(t->backend->mu);  // other threads mark and clear the same storage
    Storage& st = *t->storage;
    if (st.pending && st.done) {
        const Device* dev;
        if (bind_device(&dev) == MFH_OK && hipEventQuery(st.done) == hipErrorNotReady) return MFH_STATE_PENDING;
        st.pending = false;
    }
    return MFH_STATE_READY;
}

void* mfh_tensor_dispatch_pointer(const mfh_tensor* t)
{
    void* p = device_address(t);
    if (p) t->storage->exposed.store(true, std::memory_order_relaxed);
    return p;
}

int mfh_tensor_sync(mfh_tensor* t)
{
    MFH_TRY(tensor_ok(t));
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    std::lock_guard<std::mutex> lock(t->backend->mu);
    MFH_TRY(wait_storage(*t->storage));
    if (t->backend->stream) MFH_TRY(check_hip(hipStreamSynchronize(t->backend->stream), "hipStreamSynchronize"));
    return take_tensor_sticky(t->backend->stream, *t->storage);
}

int mfh_tensor_slice(const mfh_tensor* t, int64_t start, int64_t length, mfh_tensor** view)
{
    if (!view) return fail(MFH_ERR_INVALID_ARGUMENT, "slice: view out-pointer is NULL");
    *view = nullptr;
    MFH_TRY(tensor_ok(t));
    if (t->dtype == kInt4 || t->dtype == kBool)
        return fail(MFH_ERR_INVALID_ARGUMENT, "slice: packed dtype %s", dtype_string(t->dtype));
    if (start < 0 || length < 0 || start > t->elements || length > t->elements - start)
        return fail(MFH_ERR_SHAPE_INVALID, "tensor: invalid shape: slice [%lld, +%lld) out of range [0, %lld]",
                    (long long)start, (long long)length, (long long)t->elements);
    auto v = std::make_unique<mfh_tensor>(*t);
    v->owner = false;
    v->offset = t->offset + start * dtype_size(t->dtype);
    v->dims = {length};
    v->elements = length;
    *view = v.release();
    return MFH_OK;
}

int mfh_tensor_reshape(const mfh_tensor* t, const int64_t* dims, int32_t rank, mfh_tensor** view)
{
    if (!view) return fail(MFH_ERR_INVALID_ARGUMENT, "reshape: view out-pointer is NULL");
    *view = nullptr;
    MFH_TRY(tensor_ok(t));
    std::vector<int64_t> d;
    int64_t n;
    MFH_TRY(make_shape(dims, rank, &d, &n));
    if (n != t->elements)
        return fail(MFH_ERR_SHAPE_MISMATCH, "tensor: shape mismatch: reshape product %lld != original %lld",
                    (long long)n, (long long)t->elements);
    auto v = std::make_unique<mfh_tensor>(*t);
    v->owner = false;
    v->dims = std::move(d);
    *view = v.release();
    return MFH_OK;
}

int mfh_tensor_close(mfh_tensor* t)
{
    if (!t || t->closed) return MFH_OK;
    t->closed = true;
    if (!t->owner || !t->storage || t->storage->freed) return MFH_OK;
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    std::lock_guard<std::mutex> lock(t->backend->mu);
    Storage& st = *t->storage;
    // Close blocks until the tensor's own queued work is done (tensor.Tensor
    // Close drains in-flight async ops): uploads, resident axpys and graph
    // calls on any backend's stream, the last of which `done` follows.  Other
    // work on the device is not waited for.
    int rc = wait_storage(st);
    if (st.done) (void)hipEventDestroy(st.done);
    st.done = nullptr;
    if (st.ptr) {
        // A block whose address was handed out may still be in use by the
        // caller's own launches, on any stream: only a device-wide wait (the
        // one hipFree would make) orders after those.  The idle block then
        // goes to the backend's cache.
        const int wrc = st.exposed.load(std::memory_order_relaxed)
                            ? check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize")
                            : MFH_OK;
        const int frc = wrc == MFH_OK && rc == MFH_OK ? t->backend->release(st.ptr, st.bytes)
                                                      : check_hip(hipFree(st.ptr), "hipFree");
        if (rc == MFH_OK) rc = wrc != MFH_OK ? wrc : frc;
    }
    st.ptr = nullptr;
    st.freed = true;
    t->backend->owned.erase(t->storage);
    return rc;
}

int mfh_tensor_release(mfh_tensor* t)
{
    if (!t) return MFH_OK;
    int rc = mfh_tensor_close(t);
    delete t;
    return rc;
}

int mfh_axpy_onto_resident(mfh_backend* backend, mfh_tensor* y, const mfh_tensor* x, float alpha)
{
    const Device* dev;
    MFH_TRY(backend_ok(backend, &dev));
    MFH_TRY(tensor_ok(y));
    MFH_TRY(tensor_ok(x));
    // Location is "hip" for every tensor of this library (runtime/axpy.go:68-70).
    if (y->dtype != x->dtype)
        return fail(MFH_ERR_INVALID_ARGUMENT, "math.axpy: y dtype %s does not match x dtype %s", dtype_string(y->dtype),
                    dtype_string(x->dtype));
    if (y->elements != x->elements)
        return fail(MFH_ERR_INVALID_ARGUMENT, "math.axpy: y length %lld does not match x length %lld",
                    (long long)y->elements, (long long)x->elements);
    if (!stored_as_is(y->dtype))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "math.axpy: dtype %s has no device axpy", dtype_string(y->dtype));
    BackendState& s = *backend->state;
    // y and x may belong to other backends: their owners' state changes
    // (close, download, shutdown) are held off while the launch is queued.
    StateLocks locks({&s, y->backend.get(), x->backend.get()});
    if (s.closed) return fail(MFH_ERR_CLOSED, "tensor: backend closed");
    MFH_TRY(tensor_ok(y));
    MFH_TRY(tensor_ok(x));
    Storage& ys = *y->storage;
    Storage& xs = *x->storage;
    // Order after work still queued on the tensors (uploads, earlier axpys),
    // on whichever stream it runs.
    for (Storage* st : {&ys, &xs})
        if (st->pending && st->done)
            MFH_TRY(check_hip(hipStreamWaitEvent(s.stream, st->done, 0), "hipStreamWaitEvent"));
    mfh_axpy(device_address(y), device_address(x), y->elements, alpha, y->dtype, s.stream);
    // Later readers of y, and closes of either tensor through its own
    // backend, wait for this launch.
    MFH_TRY(mark_pending(ys, s.stream));
    if (&xs != &ys) MFH_TRY(mark_pending(xs, s.stream));
    ys.writer = s.stream;
    return MFH_OK;
}

int mfh_backend_graph_call(mfh_backend* backend, mfh_graph* graph, const char* const* input_names,
                           const mfh_tensor* const* inputs, int32_t n_inputs, const char* const* output_keys,
                           int32_t n_outputs, mfh_tensor** outputs)
{
    if (n_outputs < 0 || (n_outputs > 0 && (!outputs || !output_keys)) || n_inputs < 0 ||
        (n_inputs > 0 && (!inputs || !input_names)))
        return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: bad input or output list");
    for (int32_t j = 0; j < n_outputs; j++) outputs[j] = nullptr;
    if (!graph) return fail(MFH_ERR_INVALID_ARGUMENT, "graph call: graph is required");
    const Device* dev;
    MFH_TRY(backend_ok(backend, &dev));
    std::vector<BackendState*> states{backend->state.get()};
    for (int32_t k = 0; k < n_inputs; k++) {
        MFH_TRY(tensor_ok(inputs[k]));
        states.push_back(inputs[k]->backend.get());
    }
    // Inputs may belong to other backends: their owners' state changes
    // (close, download, shutdown) are held off while the call is queued.
    StateLocks locks(states);
    BackendState& s = *backend->state;
    if (s.closed) return fail(MFH_ERR_CLOSED, "tensor: backend closed");
    std::vector<mfh_value> ins((size_t)n_inputs);
    for (int32_t k = 0; k < n_inputs; k++) {
        MFH_TRY(tensor_ok(inputs[k]));
        const mfh_tensor& t = *inputs[k];
        ins[k] = mfh_value{input_names[k], device_address(&t), t.dtype, {0}, t.elements};
    }
    // One flat tensor per output key, of the dtype and length the call gives it.
    std::vector<std::unique_ptr<mfh_tensor>> made;
    std::vector<mfh_value> outs((size_t)n_outputs);
    auto undo = [&](int rc) {
        (void)hipStreamSynchronize(s.stream);
        for (auto& t : made) {
            Storage& st = *t->storage;
            if (st.done) (void)hipEventDestroy(st.done);
            if (st.ptr) (void)hipFree(st.ptr);
            st.done = nullptr;
            st.ptr = nullptr;
        }
        return rc;
    };
    for (int32_t j = 0; j < n_outputs; j++) {
        uint8_t dt = kInvalid;
        int64_t n = 0;
        int rc = mfh_graph_output_shape(graph, ins.data(), n_inputs, output_keys[j], &dt, &n);
        if (rc != MFH_OK) return undo(rc);
        auto t = std::make_unique<mfh_tensor>();
        t->backend = backend->state;
        t->storage = std::make_shared<Storage>();
        t->dims = {n};
        t->elements = n;
        t->dtype = dt;
        t->storage->bytes = (size_t)n * dtype_size(dt);
        made.push_back(std::move(t));
        Storage& st = *made.back()->storage;
        if (st.bytes && (rc = s.alloc(st.bytes, &st.ptr)) != MFH_OK) return undo(rc);
        outs[j] = mfh_value{output_keys[j], st.ptr, dt, {0}, n};
    }
    // Order after work still queued on the inputs (uploads, axpys, earlier
    // graph calls), on whichever stream it runs.
    for (int32_t k = 0; k < n_inputs; k++) {
        Storage& st = *inputs[k]->storage;
        if (st.pending && st.done) {
            int rc = check_hip(hipStreamWaitEvent(s.stream, st.done, 0), "hipStreamWaitEvent");
            if (rc != MFH_OK) return undo(rc);
        }
    }
    int rc = mfh_graph_call(graph, ins.data(), n_inputs, outs.data(), n_outputs, s.stream);
    if (rc != MFH_OK) return undo(rc);
    // Later readers of the outputs, and closes of the inputs through their
    // own backends, wait for the call.
    for (int32_t k = 0; k < n_inputs; k++)
        if ((rc = mark_pending(*inputs[k]->storage, s.stream)) != MFH_OK) return undo(rc);
    for (auto& t : made)
        if ((rc = mark_pending(*t->storage, s.stream)) != MFH_OK) return undo(rc);
    for (int32_t j = 0; j < n_outputs; j++) {
        s.owned.insert(made[j]->storage);
        outputs[j] = made[j].release();
    }
    return MFH_OK;
}

}  // extern "C"
