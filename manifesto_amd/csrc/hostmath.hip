// hostmath.hip — the runtime's vector math on gfx950: axpy (runtime/axpy.go),
// scalar broadcast and linspace (runtime/executor_math.go).
//
// axpy moves 12 bytes per f32 element (read x, read y, write y) and does two
// flops, so it is an HBM stream: 16-byte vectors, one-shot grid by default, with
// non-temporal loads and stores (each byte is touched once).  The
// product is rounded before the add (the library is built with
// -ffp-contract=off), as the Go loop at runtime/axpy.go:115-117 computes it.
#include "launch.hpp"

namespace mfh {
namespace {

template <int DT>
MFH_DEV float dec16(mfh_u32 h)
{
    return DT == kBFloat16 ? mfh_bf16_to_f32(h) : mfh_f16_to_f32(h);
}

template <int DT>
MFH_DEV mfh_u32 enc16x2(float lo, float hi)
{
    if constexpr (DT == kBFloat16) return mfh_bf16x2_rne(lo, hi);
    else return mfh_f16x2_rne(lo, hi);
}

MFH_DEV float axpy_step(float y, float x, float alpha)
{
    float product = alpha * x;
    return y + product;
}

// A block of BS threads takes chunks of BS * U consecutive 16-byte items
// (thread t holds items t, t + BS, ...), one-shot by default, so the launch
// sweeps x and y in dispatch order: 6.5 TB/s at 64 threads x 1 item against
// 6.2 for the best grid-stride shape, once x and y outgrow the Infinity Cache.
template <int U, int BS>
__global__ __launch_bounds__(BS) void k_axpy_f32(float* __restrict__ y, const float* __restrict__ x,
                                                     mfh_i64 n, float alpha, int vec_ok)
{
    constexpr mfh_i64 kChunk = (mfh_i64)BS * U;
    const mfh_i64 nvec = vec_ok ? (n >> 2) : 0;
    const mfh_i64 nchunks = (nvec + kChunk - 1) / kChunk;
    u32x4* yv = reinterpret_cast<u32x4*>(y);
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    for (mfh_i64 c = blockIdx.x; c < nchunks; c += gridDim.x) {
        const mfh_i64 first = c * kChunk + threadIdx.x;
        u32x4 a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const mfh_i64 i = first + u * BS;
            if (i < nvec) {
                a[u] = load_nt(&xv[i]);
                b[u] = load_nt(&yv[i]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const mfh_i64 i = first + u * BS;
            if (i >= nvec) break;
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; k++) o[k] = mfh_bits(axpy_step(mfh_f32(b[u][k]), mfh_f32(a[u][k]), alpha));
            store_nt(&yv[i], o);
        }
    }
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 i = nvec * 4 + (mfh_i64)blockIdx.x * BS + threadIdx.x; i < n; i += stride)
        y[i] = axpy_step(y[i], x[i], alpha);
}

// 16-bit storage: decode, the same f32 step, re-encode (axpyOntoHost tensor
// path, runtime/axpy.go:120-161, in one pass instead of five).
template <int DT, int U, int BS>
__global__ __launch_bounds__(BS) void k_axpy16(mfh_u16* __restrict__ y, const mfh_u16* __restrict__ x,
                                                   mfh_i64 n, float alpha, int vec_ok)
{
    constexpr mfh_i64 kChunk = (mfh_i64)BS * U;
    const mfh_i64 nvec = vec_ok ? (n >> 3) : 0;
    const mfh_i64 nchunks = (nvec + kChunk - 1) / kChunk;
    u32x4* yv = reinterpret_cast<u32x4*>(y);
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    for (mfh_i64 c = blockIdx.x; c < nchunks; c += gridDim.x) {
        const mfh_i64 first = c * kChunk + threadIdx.x;
        u32x4 a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const mfh_i64 i = first + u * BS;
            if (i < nvec) {
                a[u] = load_nt(&xv[i]);
                b[u] = load_nt(&yv[i]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const mfh_i64 i = first + u * BS;
            if (i >= nvec) break;
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float lo = axpy_step(dec16<DT>(b[u][k] & 0xffffu), dec16<DT>(a[u][k] & 0xffffu), alpha);
                float hi = axpy_step(dec16<DT>(b[u][k] >> 16), dec16<DT>(a[u][k] >> 16), alpha);
                o[k] = enc16x2<DT>(lo, hi);
            }
            store_nt(&yv[i], o);
        }
    }
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 i = nvec * 8 + (mfh_i64)blockIdx.x * BS + threadIdx.x; i < n; i += stride) {
        float r = axpy_step(dec16<DT>(y[i]), dec16<DT>(x[i]), alpha);
        y[i] = (mfh_u16)(enc16x2<DT>(r, 0.0f) & 0xffffu);
    }
}

template <int DT, int BS>
void launch_axpy16(int u, unsigned grid, hipStream_t s, mfh_u16* y, const mfh_u16* x, int64_t n, float alpha,
                   int vec_ok)
{
    if (u == 4) k_axpy16<DT, 4, BS><<<grid, BS, 0, s>>>(y, x, n, alpha, vec_ok);
    else if (u == 2) k_axpy16<DT, 2, BS><<<grid, BS, 0, s>>>(y, x, n, alpha, vec_ok);
    else k_axpy16<DT, 1, BS><<<grid, BS, 0, s>>>(y, x, n, alpha, vec_ok);
}

template <int DT>
MFH_DEV float load_f(const void* p, mfh_i64 i)
{
    if constexpr (DT == kFloat32) return static_cast<const float*>(p)[i];
    else return dec16<DT>(static_cast<const mfh_u16*>(p)[i]);
}

template <int DT>
MFH_DEV void store_f(void* p, mfh_i64 i, float v)
{
    if constexpr (DT == kFloat32) static_cast<float*>(p)[i] = v;
    else static_cast<mfh_u16*>(p)[i] = (mfh_u16)(enc16x2<DT>(v, 0.0f) & 0xffffu);
}

MFH_DEV float apply_op(float v, float s, int op)
{
    switch (op) {
    case 0: return v + s;
    case 1: return v - s;
    case 2: return v * s;
    default: return v / s;
    }
}

template <int IN, int OUT>
__global__ __launch_bounds__(kBlock) void k_scalar_broadcast(void* __restrict__ out, const void* __restrict__ in,
                                                             mfh_i64 n, float s, int op)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    for (mfh_i64 i = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        store_f<OUT>(out, i, apply_op(load_f<IN>(in, i), s, op));
}

template <int OUT>
__global__ __launch_bounds__(kBlock) void k_linspace(void* __restrict__ out, mfh_i64 n, float start,
                                                     float stop, float step, int pin_first, int pin_last)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    for (mfh_i64 i = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float scaled = (float)i * step;
        float v = start + scaled;
        if (pin_first && i == 0) v = start;
        if (pin_last && i == n - 1) v = stop;
        store_f<OUT>(out, i, v);
    }
}

template <int OP>
MFH_DEV float apply(float v, float s)
{
    if constexpr (OP == 0) return v + s;
    else if constexpr (OP == 1) return v - s;
    else if constexpr (OP == 2) return v * s;
    else return v / s;
}

// E consecutive elements of a 16-byte-aligned item row as f32: E = 4 or 8.
template <int DT, int E, bool NT>
MFH_DEV void load_item(const void* p, mfh_i64 item, float (&v)[E])
{
    auto ld = [](const auto* q) { return NT ? load_nt(q) : *q; };
    if constexpr (DT == kFloat32) {
        const u32x4* q = reinterpret_cast<const u32x4*>(p) + item * (E / 4);
#pragma unroll
        for (int h = 0; h < E / 4; h++) {
            const u32x4 w = ld(q + h);
#pragma unroll
            for (int k = 0; k < 4; k++) v[4 * h + k] = mfh_f32(w[k]);
        }
    } else if constexpr (E == 4) {
        const u32x2 w = ld(reinterpret_cast<const u32x2*>(p) + item);
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = dec16<DT>((w[k >> 1] >> (16 * (k & 1))) & 0xffffu);
    } else {
        const u32x4 w = ld(reinterpret_cast<const u32x4*>(p) + item);
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = dec16<DT>((w[k >> 1] >> (16 * (k & 1))) & 0xffffu);
    }
}

// The 16-byte output item of E elements (4 f32, or 8 bf16/f16 with RNE).
template <int DT, int E>
MFH_DEV u32x4 pack_item(const float (&v)[E])
{
    if constexpr (DT == kFloat32) return u32x4{mfh_bits(v[0]), mfh_bits(v[1]), mfh_bits(v[2]), mfh_bits(v[3])};
    else return u32x4{enc16x2<DT>(v[0], v[1]), enc16x2<DT>(v[2], v[3]), enc16x2<DT>(v[4], v[5]),
                      enc16x2<DT>(v[6], v[7])};
}

// Vector forms: one 16-byte output item per thread (4 f32 or 8 16-bit
// elements), one-shot grid, streaming stores; loads non-temporal when the
// input is at least as wide as the output.  The element kernels above keep
// misaligned buffers and the tails.  The element form stored 2 or 4 bytes
// per lane: 3.6 TB/s for an f32 broadcast and 4.5 for an f32 linspace.
template <int IN, int OUT, int OP>
__global__ __launch_bounds__(kBlock) void k_scalar_broadcast_vec(void* __restrict__ out, const void* __restrict__ in,
                                                                 mfh_i64 n, float s)
{
    constexpr int E = OUT == kFloat32 ? 4 : 8;
    constexpr bool kNt = (IN == kFloat32) || (OUT != kFloat32);
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    const mfh_i64 nitems = n / E;
    for (mfh_i64 it = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; it < nitems; it += stride) {
        float v[E];
        load_item<IN, E, kNt>(in, it, v);
#pragma unroll
        for (int k = 0; k < E; k++) v[k] = apply<OP>(v[k], s);
        store_nt(reinterpret_cast<u32x4*>(out) + it, pack_item<OUT, E>(v));
    }
    for (mfh_i64 i = nitems * E + (mfh_i64)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        store_f<OUT>(out, i, apply<OP>(load_f<IN>(in, i), s));
}

template <int OUT>
__global__ __launch_bounds__(kBlock) void k_linspace_vec(void* __restrict__ out, mfh_i64 n, float start, float stop,
                                                         float step, int pin_first, int pin_last)
{
    constexpr int E = OUT == kFloat32 ? 4 : 8;
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    const mfh_i64 nitems = n / E;
    auto at = [&](mfh_i64 i) {
        float v = start + (float)i * step;
        if (pin_first && i == 0) v = start;
        if (pin_last && i == n - 1) v = stop;
        return v;
    };
    for (mfh_i64 it = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; it < nitems; it += stride) {
        float v[E];
#pragma unroll
        for (int k = 0; k < E; k++) v[k] = at(it * E + k);
        store_nt(reinterpret_cast<u32x4*>(out) + it, pack_item<OUT, E>(v));
    }
    for (mfh_i64 i = nitems * E + (mfh_i64)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        store_f<OUT>(out, i, at(i));
}

int check_float_dtype(int dt, const char* what)
{
    if (dt == kFloat32 || dt == kBFloat16 || dt == kFloat16) return MFH_OK;
    return fail(MFH_ERR_DTYPE_UNSUPPORTED, "%s: dtype %s is not f32/bf16/f16", what, dtype_name(dt));
}

template <int IN, int OUT>
void launch_broadcast_vec(unsigned grid, hipStream_t s, void* out, const void* in, int64_t n, float scalar, int op)
{
    switch (op) {
    case 0: k_scalar_broadcast_vec<IN, OUT, 0><<<grid, kBlock, 0, s>>>(out, in, n, scalar); break;
    case 1: k_scalar_broadcast_vec<IN, OUT, 1><<<grid, kBlock, 0, s>>>(out, in, n, scalar); break;
    case 2: k_scalar_broadcast_vec<IN, OUT, 2><<<grid, kBlock, 0, s>>>(out, in, n, scalar); break;
    default: k_scalar_broadcast_vec<IN, OUT, 3><<<grid, kBlock, 0, s>>>(out, in, n, scalar); break;
    }
}

template <int IN>
int launch_broadcast(int out_dt, const Device* dev, hipStream_t s, void* out, const void* in, int64_t n,
                     float scalar, int op)
{
    // vector items need the output 16-byte aligned and the input aligned to
    // the item's bytes (16 for f32 sources, 8 or 16 for 16-bit ones)
    const int e = out_dt == kFloat32 ? 4 : 8;
    const uintptr_t in_align = IN == kFloat32 ? 16 : (uintptr_t)e * 2;
    if (n >= e && (reinterpret_cast<uintptr_t>(out) & 15) == 0 && (reinterpret_cast<uintptr_t>(in) & (in_align - 1)) == 0) {
        const unsigned grid = grid_for(n / e, dev, Kern::kConvert);
        switch (out_dt) {
        case kFloat32: launch_broadcast_vec<IN, kFloat32>(grid, s, out, in, n, scalar, op); break;
        case kBFloat16: launch_broadcast_vec<IN, kBFloat16>(grid, s, out, in, n, scalar, op); break;
        default: launch_broadcast_vec<IN, kFloat16>(grid, s, out, in, n, scalar, op); break;
        }
        return launch_status("k_scalar_broadcast_vec");
    }
    const unsigned grid = grid_for(n, dev, Kern::kConvert);
    switch (out_dt) {
    case kFloat32: k_scalar_broadcast<IN, kFloat32><<<grid, kBlock, 0, s>>>(out, in, n, scalar, op); break;
    case kBFloat16: k_scalar_broadcast<IN, kBFloat16><<<grid, kBlock, 0, s>>>(out, in, n, scalar, op); break;
    default: k_scalar_broadcast<IN, kFloat16><<<grid, kBlock, 0, s>>>(out, in, n, scalar, op); break;
    }
    return launch_status("k_scalar_broadcast");
}

}  // namespace
}  // namespace mfh

using namespace mfh;

extern "C" {

void mfh_axpy(void* y, const void* x, int64_t count, float alpha, uint8_t dtype, void* stream)
{
    hipStream_t s = (hipStream_t)stream;
    const Device* dev;
    if (bind_device(&dev) != MFH_OK) {
        fail_sticky(s, MFH_ERR_NOT_INITIALIZED, "mfh_axpy: mfh_init has not been called");
        return;
    }
    if (count < 0) {
        fail_sticky(s, MFH_ERR_INVALID_ARGUMENT, "mfh_axpy: negative count %lld", (long long)count);
        return;
    }
    if (count == 0) return;
    if (!y || !x) {
        fail_sticky(s, MFH_ERR_INVALID_ARGUMENT, "mfh_axpy: NULL buffer");
        return;
    }
    int vec_ok = aligned16(y) && aligned16(x);
    switch (dtype) {
    case kFloat32: {
        int64_t items = vec_ok ? std::max<int64_t>(count >> 2, 1) : count;
        const int u = items_per_thread(Kern::kAxpy);
        auto* yy = static_cast<float*>(y);
        auto* xx = static_cast<const float*>(x);
        with_block(threads_per_block(Kern::kAxpy), [&](auto block) {
            constexpr int BS = decltype(block)::value;
            const unsigned grid = grid_for(items, dev, Kern::kAxpy, u, BS);
            if (u == 4) k_axpy_f32<4, BS><<<grid, BS, 0, s>>>(yy, xx, count, alpha, vec_ok);
            else if (u == 2) k_axpy_f32<2, BS><<<grid, BS, 0, s>>>(yy, xx, count, alpha, vec_ok);
            else k_axpy_f32<1, BS><<<grid, BS, 0, s>>>(yy, xx, count, alpha, vec_ok);
            return 0;
        });
        break;
    }
    case kBFloat16:
    case kFloat16: {
        int64_t items = vec_ok ? std::max<int64_t>(count >> 3, 1) : count;
        const int u = items_per_thread(Kern::kAxpy16);
        auto* yy = static_cast<mfh_u16*>(y);
        auto* xx = static_cast<const mfh_u16*>(x);
        with_block(threads_per_block(Kern::kAxpy16), [&](auto block) {
            constexpr int BS = decltype(block)::value;
            const unsigned grid = grid_for(items, dev, Kern::kAxpy16, u, BS);
            if (dtype == kBFloat16) launch_axpy16<kBFloat16, BS>(u, grid, s, yy, xx, count, alpha, vec_ok);
            else launch_axpy16<kFloat16, BS>(u, grid, s, yy, xx, count, alpha, vec_ok);
            return 0;
        });
        break;
    }
    default:
        fail_sticky(s, MFH_ERR_DTYPE_UNSUPPORTED, "mfh_axpy: dtype %s is not f32/bf16/f16", dtype_name(dtype));
        return;
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) fail_sticky(s, MFH_ERR_DEVICE, "mfh_axpy: launch failed: %s", hipGetErrorString(err));
}

int mfh_scalar_broadcast(void* out, uint8_t out_dtype, const void* in, uint8_t in_dtype, int64_t count,
                         float scalar, int32_t op, void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    MFH_TRY(check_float_dtype(out_dtype, "mfh_scalar_broadcast"));
    MFH_TRY(check_float_dtype(in_dtype, "mfh_scalar_broadcast"));
    if (op < 0 || op > 3) return fail(MFH_ERR_INVALID_ARGUMENT, "math.scalar_broadcast: unsupported op %d", op);
    if (op == 3 && scalar == 0.0f)
        return fail(MFH_ERR_INVALID_ARGUMENT, "math.scalar_broadcast: scalar divisor must be nonzero");
    if (count < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "math.scalar_broadcast: negative count");
    if (count == 0) return MFH_OK;
    if (!out || !in) return fail(MFH_ERR_INVALID_ARGUMENT, "math.scalar_broadcast: NULL buffer");
    hipStream_t s = (hipStream_t)stream;
    switch (in_dtype) {
    case kFloat32: return launch_broadcast<kFloat32>(out_dtype, dev, s, out, in, count, scalar, op);
    case kBFloat16: return launch_broadcast<kBFloat16>(out_dtype, dev, s, out, in, count, scalar, op);
    default: return launch_broadcast<kFloat16>(out_dtype, dev, s, out, in, count, scalar, op);
    }
}

int mfh_linspace(void* out, uint8_t out_dtype, int64_t count, float start, float stop, int32_t endpoint,
                 void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    MFH_TRY(check_float_dtype(out_dtype, "math.linspace"));
    if (count <= 0) return fail(MFH_ERR_INVALID_ARGUMENT, "math.linspace: count must be positive");
    if (!out) return fail(MFH_ERR_INVALID_ARGUMENT, "math.linspace: NULL buffer");
    int64_t intervals = count == 1 ? 1 : (endpoint ? count - 1 : count);
    float diff = stop - start;
    float step = diff / (float)intervals;
    // count == 1 returns start itself; with the endpoint both ends are pinned.
    int pin_first = (count == 1 || endpoint) ? 1 : 0;
    int pin_last = (count > 1 && endpoint) ? 1 : 0;
    hipStream_t s = (hipStream_t)stream;
    const int e = out_dtype == kFloat32 ? 4 : 8;
    if (count >= e && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
        const unsigned grid = grid_for(count / e, dev, Kern::kConvert);
        switch (out_dtype) {
        case kFloat32: k_linspace_vec<kFloat32><<<grid, kBlock, 0, s>>>(out, count, start, stop, step, pin_first, pin_last); break;
        case kBFloat16: k_linspace_vec<kBFloat16><<<grid, kBlock, 0, s>>>(out, count, start, stop, step, pin_first, pin_last); break;
        default: k_linspace_vec<kFloat16><<<grid, kBlock, 0, s>>>(out, count, start, stop, step, pin_first, pin_last); break;
        }
        return launch_status("k_linspace_vec");
    }
    unsigned grid = grid_for(count, dev, Kern::kConvert);
    switch (out_dtype) {
    case kFloat32: k_linspace<kFloat32><<<grid, kBlock, 0, s>>>(out, count, start, stop, step, pin_first, pin_last); break;
    case kBFloat16: k_linspace<kBFloat16><<<grid, kBlock, 0, s>>>(out, count, start, stop, step, pin_first, pin_last); break;
    default: k_linspace<kFloat16><<<grid, kBlock, 0, s>>>(out, count, start, stop, step, pin_first, pin_last); break;
    }
    return launch_status("k_linspace");
}

}  // extern "C"
