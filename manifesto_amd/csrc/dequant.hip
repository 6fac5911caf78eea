// dequant.hip — FP8 / Int4 dequantisation and dtype conversion for gfx950.
//
// All of these are HBM streams.  A work item is the input that produces one
// 16-byte output vector; item i of every thread sits next to item i of its
// neighbours, so each store instruction of a wave writes 1 KiB contiguously
// and each load instruction reads a contiguous span.  Threads take U items
// per step (loads first, then converts and stores): FP8 in one-shot chunks
// per workgroup, the others in grid-stride loops.  A scalar loop finishes the
// elements after the last whole item, and does all of them when a pointer is
// not aligned for the vector path.
//
// FP8: the output for a code depends only on (code, format, scale), so each
// workgroup first builds the 256-entry table in LDS with the exact rules of
// codec.hpp; every element is then one LDS read.
#include "launch.hpp"

namespace mfh {

int launch_status(const char* what) { return check_hip(hipGetLastError(), what); }

namespace {

template <int OUT>
MFH_DEV mfh_u32 encode_one(float v)
{
    if constexpr (OUT == kFloat32) return mfh_bits(v);
    else if constexpr (OUT == kBFloat16) return mfh_bf16_rne(v);
    else return mfh_f16_rne(v);
}

template <int OUT>
MFH_DEV mfh_u32 encode_pair(float lo, float hi)
{
    if constexpr (OUT == kBFloat16) return mfh_bf16x2_rne(lo, hi);
    else return mfh_f16x2_rne(lo, hi);
}

template <int OUT>
MFH_DEV void store_one(void* out, mfh_i64 i, mfh_u32 enc)
{
    if constexpr (OUT == kFloat32) static_cast<mfh_u32*>(out)[i] = enc;
    else static_cast<mfh_u16*>(out)[i] = (mfh_u16)enc;
}

// ---------------------------------------------------------------------------
// FP8 -> {f32, bf16, f16}
// ---------------------------------------------------------------------------

// Item = 8 codes (16-bit output) or 4 codes (f32 output) -> one 16-byte store.
// A block of BS threads takes chunks of BS * U consecutive items (thread t
// holds items t, t + BS, ...), so each store instruction of a wave writes
// 1 KiB contiguously; with BS < 256 the table build takes 256 / BS entries
// per thread.  The grid normally has one block per chunk ("one-shot": no
// block outlives its chunk, so the blocks sweep memory in dispatch order) and
// loops only when there are more chunks than the largest grid.  A block
// issues its first chunk's loads before building the table, so the load
// latency covers the build; stores are streaming (StreamOut: non-temporal)
// and so are the code loads (+0.6% against plain loads; Int4's nibbles lose
// 0.8% that way and stay plain).
// Measured at [4096, 14336] on MI355X with the codes coming from HBM:
// 6.1-6.2 TB/s, within 3% of a bf16 -> f32 cast moving the same bytes.
// One table entry's decode by gfx950's converter (v_cvt_f32_fp8 /
// v_cvt_f32_bf8), which decodes every finite and infinite OCP E4M3 / E5M2
// code exactly and writes one canonical NaN for every NaN code; NaN codes
// take the reference's bits instead, which keep the sign and, for E5M2, the
// two mantissa bits (dtype/fp8.go:43-45,155-161).  Branch-free, a few VALU
// instructions per entry where the integer decode (mfh_e4m3_bits /
// mfh_e5m2_bits) normalises subnormals in divergent branches.
MFH_DEV mfh_u32 fp8_bits_hw(mfh_u32 code, bool e5m2)
{
    const float f = e5m2 ? __builtin_amdgcn_cvt_f32_bf8((int)code, 0) : __builtin_amdgcn_cvt_f32_fp8((int)code, 0);
    const mfh_u32 nan = ((code & 0x80u) << 24) | 0x7fc00000u | (e5m2 ? (code & 3u) << 21 : 0u);
    return f != f ? nan : mfh_bits(f);
}

template <int OUT, int U, int BS>
__global__ __launch_bounds__(BS) void k_dequant_fp8(const mfh_u8* __restrict__ in,
                                                        void* __restrict__ out, mfh_i64 n,
                                                        float scale, int fmt, int vec_ok)
{
    __shared__ mfh_u32 lut[256];
    constexpr int kCodes = OUT == kFloat32 ? 4 : 8;
    constexpr mfh_i64 kChunk = (mfh_i64)BS * U;
    const mfh_u32 t = threadIdx.x;
    const mfh_i64 nitems = vec_ok ? n / kCodes : 0;
    const mfh_i64 nchunks = (nitems + kChunk - 1) / kChunk;
    u32x2 w[U];
    auto load = [&](mfh_i64 c) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const mfh_i64 i = c * kChunk + u * BS + t;
            if (i < nitems) {
                if constexpr (kCodes == 8) w[u] = load_nt(&reinterpret_cast<const u32x2*>(in)[i]);
                else w[u] = u32x2{reinterpret_cast<const mfh_u32*>(in)[i], 0u};
            }
        }
    };
    mfh_i64 c = blockIdx.x;
    if (c < nchunks) load(c);
    for (mfh_u32 e = t; e < 256; e += BS)
        lut[e] = encode_one<OUT>(mfh_scale_mul(mfh_f32(fp8_bits_hw(e, fmt == kF8E5M2)), scale));
    __syncthreads();
    for (; c < nchunks; c += gridDim.x) {
        if (c != (mfh_i64)blockIdx.x) load(c);
        const mfh_i64 first = c * kChunk;
        const StreamOut dst(reinterpret_cast<u32x4*>(out) + first, nitems - first);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = u * BS + (int)t;
            if (first + j >= nitems) break;
            const mfh_u32 x = w[u][0], y = w[u][1];
            if constexpr (OUT == kFloat32) {
                dst.store(j, u32x4{lut[x & 0xffu], lut[(x >> 8) & 0xffu], lut[(x >> 16) & 0xffu], lut[x >> 24]});
            } else {
                dst.store(j, u32x4{lut[x & 0xffu] | (lut[(x >> 8) & 0xffu] << 16),
                                   lut[(x >> 16) & 0xffu] | (lut[x >> 24] << 16),
                                   lut[y & 0xffu] | (lut[(y >> 8) & 0xffu] << 16),
                                   lut[(y >> 16) & 0xffu] | (lut[y >> 24] << 16)});
            }
        }
    }
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 i = nitems * kCodes + (mfh_i64)blockIdx.x * BS + t; i < n; i += stride)
        store_one<OUT>(out, i, lut[in[i]]);
}

// ---------------------------------------------------------------------------
// Int4 (+ group scale) -> {f32, bf16, f16}
// ---------------------------------------------------------------------------

// A group scale in two steps, the stored bits then their value, so that a
// kernel can issue every load before it widens the first scale.
template <int SDT>
MFH_DEV mfh_u32 scale_bits(const void* scales, mfh_i64 g)
{
    if constexpr (SDT == kFloat32) return static_cast<const mfh_u32*>(scales)[g];
    else if constexpr (SDT == kFloat16 || SDT == kBFloat16) return static_cast<const mfh_u16*>(scales)[g];
    else return 0;
}

template <int SDT>
MFH_DEV float scale_value(mfh_u32 bits)
{
    if constexpr (SDT == kFloat32) return mfh_f32(bits);
    else if constexpr (SDT == kFloat16) return mfh_f16_to_f32((mfh_u16)bits);
    else if constexpr (SDT == kBFloat16) return mfh_bf16_to_f32((mfh_u16)bits);
    else return 1.0f;  // plain conversion: no scale
}

template <int SDT>
MFH_DEV float load_scale(const void* scales, mfh_i64 g)
{
    return scale_value<SDT>(scale_bits<SDT>(scales, g));
}

MFH_DEV bool finite_f32(float f) { return (mfh_bits(f) & 0x7f800000u) != 0x7f800000u; }

// Item = 8 nibbles (4 packed bytes, 16-bit output) or 4 nibbles (2 bytes,
// f32 output) sharing one scale -> one 16-byte store.  The vector path needs
// a power-of-two group (2^group_shift >= the item); other groups run the
// element loop.  A block of BS threads takes chunks of BS * U consecutive
// items (thread t holds items t, t + BS, ...), one-shot by default, with
// streaming stores (StreamOut) addressed from the chunk's first item.  The
// chunks are contiguous, as FP8's: a grid-stride loop whose U items per
// thread sat a grid apart made the launch sweep U regions of the tensor at
// once, which on this write-heavy mix ran 5.2 against 6.2 TB/s once the
// nibbles no longer fit in the Infinity Cache.
template <int OUT, int SDT, int U, int BS>
__global__ __launch_bounds__(BS) void k_dequant_int4(const mfh_u8* __restrict__ packed,
                                                         const void* __restrict__ scales,
                                                         void* __restrict__ out, mfh_i64 n,
                                                         mfh_i64 group, int group_shift, int vec_ok)
{
    constexpr int kElems = OUT == kFloat32 ? 4 : 8;
    constexpr mfh_i64 kChunk = (mfh_i64)BS * U;
    const mfh_i64 nitems = vec_ok ? n / kElems : 0;
    const mfh_i64 nchunks = (nitems + kChunk - 1) / kChunk;
    const int t = (int)threadIdx.x;
    for (mfh_i64 c = blockIdx.x; c < nchunks; c += gridDim.x) {
        const mfh_i64 first = c * kChunk;
        // Lane addresses are 32-bit offsets from uniform bases: the chunk's
        // first packed item and its first item's group scale (element e0,
        // group g0, e0 = g0 * group + r).  Items past the end load the last
        // item instead of branching: a guarded load made the compiler wait
        // for each scale inside its branch, one round trip per item, before
        // issuing the next item's loads (5.3 against 6.2 TB/s).
        const int last = (int)min<mfh_i64>(kChunk, nitems - first) - 1;
        const mfh_i64 e0 = first * kElems;
        const mfh_i64 g0 = e0 >> group_shift;
        const mfh_u64 r = (mfh_u64)(e0 - (g0 << group_shift));
        constexpr mfh_u32 kItemBytes = kElems / 2, kScaleBytes = SDT == kFloat32 ? 4 : 2;
        const char* items = reinterpret_cast<const char*>(packed) + first * kItemBytes;
        const char* group0 = static_cast<const char*>(scales) + g0 * kScaleBytes;
        // The item's group relative to g0 is (r + j kElems) >> group_shift.
        // A chunk spans fewer than 2^20 elements, so for larger groups the
        // same formula with shift 20 and r' = 2^20 - (elements from e0 to
        // the next group boundary), or 0 when that boundary lies past the
        // chunk, gives the same 0 or 1: every item runs one 32-bit add and
        // shift.
        static_assert(kChunk * kElems < (1 << 20), "a chunk spans fewer than 2^20 elements");
        const bool small_group = group_shift <= 20;
        const mfh_u64 to_next = (1ull << min(group_shift, 62)) - r;
        const mfh_u32 gr = small_group ? (mfh_u32)r : to_next >= (1u << 20) ? 0u : (1u << 20) - (mfh_u32)to_next;
        const int gs = small_group ? group_shift : 20;
        mfh_u32 w[U], sb[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const mfh_u32 j = (mfh_u32)min(u * BS + t, last);
            if constexpr (kElems == 8) w[u] = *reinterpret_cast<const mfh_u32*>(items + j * kItemBytes);
            else w[u] = *reinterpret_cast<const mfh_u16*>(items + j * kItemBytes);
            sb[u] = scale_bits<SDT>(group0 + ((gr + j * kElems) >> gs) * kScaleBytes, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the chunk ahead of the first wait
        float s[U];
#pragma unroll
        for (int u = 0; u < U; u++) s[u] = scale_value<SDT>(sb[u]);
        // The buffer descriptor ends at the last item: stores past it are dropped.
        const StreamOut dst(reinterpret_cast<u32x4*>(out) + first, nitems - first);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = u * BS + t;
            float f[kElems];
#pragma unroll
            for (int k = 0; k < kElems; k++) f[k] = (float)mfh_int4_at(w[u], k) * s[u];
            if (!finite_f32(s[u])) {  // Inf/NaN scale: apply the explicit NaN rules (rare)
#pragma unroll
                for (int k = 0; k < kElems; k++) f[k] = mfh_scale_mul((float)mfh_int4_at(w[u], k), s[u]);
            }
            if constexpr (OUT == kFloat32)
                dst.store(j, u32x4{mfh_bits(f[0]), mfh_bits(f[1]), mfh_bits(f[2]), mfh_bits(f[3])});
            else
                dst.store(j, u32x4{encode_pair<OUT>(f[0], f[1]), encode_pair<OUT>(f[2], f[3]),
                                   encode_pair<OUT>(f[4], f[5]), encode_pair<OUT>(f[6], f[7])});
        }
    }
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 i = nitems * kElems + (mfh_i64)blockIdx.x * BS + threadIdx.x; i < n; i += stride) {
        mfh_u32 byte = packed[i >> 1];
        float q = (float)mfh_int4_at(byte, (mfh_u32)(i & 1));
        float s = load_scale<SDT>(scales, i / group);
        store_one<OUT>(out, i, encode_one<OUT>(mfh_scale_mul(q, s)));
    }
}

// ---------------------------------------------------------------------------
// Generic conversion of 1/2/4/8-byte numeric dtypes -> {f32, bf16, f16}
// ---------------------------------------------------------------------------

// f64 -> f32 with x86 cvtsd2ss NaN behaviour (quiet bit set, top payload kept).
MFH_DEV float f64_to_f32(double d)
{
    mfh_u64 b = __builtin_bit_cast(mfh_u64, d);
    if ((b & 0x7fffffffffffffffull) > 0x7ff0000000000000ull)
        return mfh_f32((mfh_u32)((b >> 32) & 0x80000000u) | 0x7fc00000u |
                       (mfh_u32)((b >> 29) & 0x3fffffu));
    return (float)d;
}

// BytesToFloat32 (dtype/convert/convert.go:85-146) for element i.
template <int IN>
MFH_DEV float decode_at(const void* in, mfh_i64 i)
{
    if constexpr (IN == kFloat64) return f64_to_f32(static_cast<const double*>(in)[i]);
    else if constexpr (IN == kFloat32) return static_cast<const float*>(in)[i];
    else if constexpr (IN == kFloat16) return mfh_f16_to_f32(static_cast<const mfh_u16*>(in)[i]);
    else if constexpr (IN == kBFloat16) return mfh_bf16_to_f32(static_cast<const mfh_u16*>(in)[i]);
    else if constexpr (IN == kInt64) return (float)(double)static_cast<const long long*>(in)[i];
    else if constexpr (IN == kInt32) return (float)(double)static_cast<const int*>(in)[i];
    else if constexpr (IN == kInt16) return (float)static_cast<const short*>(in)[i];
    else if constexpr (IN == kInt8) return (float)static_cast<const signed char*>(in)[i];
    else if constexpr (IN == kUint64) return (float)(double)static_cast<const mfh_u64*>(in)[i];
    else if constexpr (IN == kUint32) return (float)(double)static_cast<const mfh_u32*>(in)[i];
    else if constexpr (IN == kUint16) return (float)static_cast<const mfh_u16*>(in)[i];
    else return (float)static_cast<const mfh_u8*>(in)[i];
}

template <int IN, int OUT>
__global__ __launch_bounds__(kBlock) void k_convert(const void* __restrict__ in, void* __restrict__ out,
                                                    mfh_i64 n)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    for (mfh_i64 i = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        store_one<OUT>(out, i, encode_one<OUT>(decode_at<IN>(in, i)));
}

template <int IN>
MFH_DEV float dec16(mfh_u32 h)
{
    return IN == kBFloat16 ? mfh_bf16_to_f32(h) : mfh_f16_to_f32(h);
}

// 16-bit storage -> any output, one 16-byte store per item: 8 elements for a
// 16-bit output, 4 for f32.  (The cast that sits between a bf16/f16 tensor and
// an f32 fusion in the reference.)
template <int IN, int OUT, int BS, int U>
__global__ __launch_bounds__(BS) void k_convert16_vec(const void* __restrict__ in, void* __restrict__ out,
                                                          mfh_i64 nitems)
{
    const mfh_i64 chunk = (mfh_i64)BS * U;  // items of a workgroup, thread t holding t, t + BS, ...
    u32x4* dst = reinterpret_cast<u32x4*>(out);
    for (mfh_i64 base = (mfh_i64)blockIdx.x * chunk; base < nitems; base += (mfh_i64)gridDim.x * chunk) {
        if constexpr (OUT == kFloat32) {
            u32x2 w[U];
#pragma unroll
            for (int u = 0; u < U; u++)  // past-the-end items load the last one again
                w[u] = reinterpret_cast<const u32x2*>(in)[min(base + u * BS + (mfh_i64)threadIdx.x, nitems - 1)];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const mfh_i64 v = base + u * BS + (mfh_i64)threadIdx.x;
                if (v < nitems)
                    store_nt(&dst[v], u32x4{mfh_bits(dec16<IN>(w[u][0] & 0xffffu)), mfh_bits(dec16<IN>(w[u][0] >> 16)),
                                            mfh_bits(dec16<IN>(w[u][1] & 0xffffu)), mfh_bits(dec16<IN>(w[u][1] >> 16))});
            }
        } else {
            u32x4 w[U];
#pragma unroll
            for (int u = 0; u < U; u++)
                w[u] = load_nt(reinterpret_cast<const u32x4*>(in) + min(base + u * BS + (mfh_i64)threadIdx.x, nitems - 1));
#pragma unroll
            for (int u = 0; u < U; u++) {
                const mfh_i64 v = base + u * BS + (mfh_i64)threadIdx.x;
                u32x4 o;
#pragma unroll
                for (int k = 0; k < 4; k++)
                    o[k] = encode_pair<OUT>(dec16<IN>(w[u][k] & 0xffffu), dec16<IN>(w[u][k] >> 16));
                if (v < nitems) store_nt(&dst[v], o);
            }
        }
    }
}

// Byte size of an unpacked numeric dtype, at compile time.
template <int DT>
constexpr int size_of()
{
    return DT == kFloat64 || DT == kInt64 || DT == kUint64 ? 8
           : DT == kFloat32 || DT == kInt32 || DT == kUint32 ? 4
           : DT == kFloat16 || DT == kBFloat16 || DT == kInt16 || DT == kUint16 ? 2 : 1;
}

// BytesToFloat32 (decode_at) of element k of a register copy of consecutive
// elements of dtype IN, `w` holding them as little-endian dwords.
template <int IN>
MFH_DEV float decode_reg(const mfh_u32* w, int k)
{
    constexpr int S = size_of<IN>();
    if constexpr (S == 8) {
        const mfh_u64 b = (mfh_u64)w[2 * k] | ((mfh_u64)w[2 * k + 1] << 32);
        if constexpr (IN == kFloat64) return f64_to_f32(__builtin_bit_cast(double, b));
        else if constexpr (IN == kInt64) return (float)(double)(long long)b;
        else return (float)(double)b;
    } else if constexpr (S == 4) {
        if constexpr (IN == kFloat32) return mfh_f32(w[k]);
        else if constexpr (IN == kInt32) return (float)(double)(int)w[k];
        else return (float)(double)w[k];
    } else if constexpr (S == 2) {
        const mfh_u32 h = (w[k >> 1] >> ((k & 1) * 16)) & 0xffffu;
        if constexpr (IN == kFloat16) return mfh_f16_to_f32(h);
        else if constexpr (IN == kBFloat16) return mfh_bf16_to_f32(h);
        else if constexpr (IN == kInt16) return (float)(short)h;
        else return (float)h;
    } else {
        const mfh_u32 b = (w[k >> 2] >> ((k & 3) * 8)) & 0xffu;
        if constexpr (IN == kInt8) return (float)(signed char)b;
        else return (float)b;
    }
}

// Any unpacked numeric dtype -> {f32, bf16, f16}, one 16-byte store per item
// (4 elements for f32 output, 8 for 16-bit) and the item's source bytes read
// with 4-, 8- or 16-byte loads (up to four 16-byte loads for 8-byte
// sources): the element loop's 1-, 2- or 4-byte accesses moved 1.4-3.8 TB/s,
// and this layout, like every streaming kernel here, writes 1 KiB per wave
// store instruction.  Loads are non-temporal when an item reads at least as
// many bytes as it writes.  Elements past the last whole item run the
// element loop.
template <int IN, int OUT, int BS, int U>
__global__ __launch_bounds__(BS) void k_convert_vec(const void* __restrict__ in, void* __restrict__ out,
                                                        mfh_i64 n)
{
    constexpr int E = OUT == kFloat32 ? 4 : 8;      // elements per item
    constexpr int B = E * size_of<IN>();            // source bytes per item
    constexpr int W = B / 4;                        // source dwords per item
    const mfh_i64 nitems = n / E;
    const mfh_i64 chunk = (mfh_i64)BS * U;          // items of a workgroup, thread t holding t, t + BS, ...
    u32x4* dst = reinterpret_cast<u32x4*>(out);
    for (mfh_i64 base = (mfh_i64)blockIdx.x * chunk; base < nitems; base += (mfh_i64)gridDim.x * chunk) {
        mfh_u32 w[U][W];
#pragma unroll
        for (int u = 0; u < U; u++) {
            // past-the-end items load the last item again (no branch around
            // the loads); their stores are skipped
            const mfh_i64 v = min(base + u * BS + (mfh_i64)threadIdx.x, nitems - 1);
            const char* src = static_cast<const char*>(in) + v * B;
            if constexpr (B >= 16) {
#pragma unroll
                for (int q = 0; q < B / 16; q++) {
                    const u32x4 x = load_nt(reinterpret_cast<const u32x4*>(src) + q);
                    w[u][4 * q] = x[0], w[u][4 * q + 1] = x[1], w[u][4 * q + 2] = x[2], w[u][4 * q + 3] = x[3];
                }
            } else if constexpr (B == 8) {
                const u32x2 x = *reinterpret_cast<const u32x2*>(src);
                w[u][0] = x[0], w[u][1] = x[1];
            } else {
                w[u][0] = *reinterpret_cast<const mfh_u32*>(src);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            u32x4 o;
            if constexpr (OUT == kFloat32) {
#pragma unroll
                for (int k = 0; k < 4; k++) o[k] = mfh_bits(decode_reg<IN>(w[u], k));
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++)
                    o[k] = encode_pair<OUT>(decode_reg<IN>(w[u], 2 * k), decode_reg<IN>(w[u], 2 * k + 1));
            }
            const mfh_i64 v = base + u * BS + (mfh_i64)threadIdx.x;
            if (v < nitems) store_nt(&dst[v], o);
        }
    }
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 i = nitems * E + (mfh_i64)blockIdx.x * BS + threadIdx.x; i < n; i += stride)
        store_one<OUT>(out, i, encode_one<OUT>(decode_at<IN>(in, i)));
}

// f32 -> 16-bit storage, 4 elements per item (16-byte load, 8-byte store).
template <int OUT, int BS>
__global__ __launch_bounds__(BS) void k_narrow_f32_vec(const u32x4* __restrict__ in,
                                                           u32x2* __restrict__ out, mfh_i64 nitems)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 v = (mfh_i64)blockIdx.x * BS + threadIdx.x; v < nitems; v += stride) {
        u32x4 a = load_nt(in + v);
        store_nt(&out[v], u32x2{encode_pair<OUT>(mfh_f32(a[0]), mfh_f32(a[1])),
                                encode_pair<OUT>(mfh_f32(a[2]), mfh_f32(a[3]))});
    }
}

// Sources wider than the output (8-byte -> f32 / bf16 / f16, 4-byte integers
// -> bf16 / f16): one 16-byte source piece per lane per step, its 16 / S
// elements stored together (a 4- or 8-byte store), so that every load
// instruction reads 1 KiB contiguously.  The generic item layout, which
// loads two or four adjacent 16-byte pieces per 16-byte store, ran f64 ->
// f32 at 6.19 TB/s against 6.9 this way.  The last n % (16 / S) elements are
// the first workgroup's.
template <int IN, int OUT, int BS>
__global__ __launch_bounds__(BS) void k_narrow_vec(const u32x4* __restrict__ in, void* __restrict__ out, mfh_i64 n)
{
    constexpr int S = size_of<IN>();
    constexpr int E = 16 / S;  // elements per piece: 2 or 4
    static_assert(S == 4 || S == 8, "4- and 8-byte sources");
    const mfh_i64 npieces = n / E;
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 v = (mfh_i64)blockIdx.x * BS + threadIdx.x; v < npieces; v += stride) {
        const u32x4 a = load_nt(in + v);
        const mfh_u32 w[4] = {a[0], a[1], a[2], a[3]};
        if constexpr (OUT == kFloat32) {
            static_assert(E == 2, "f32 output from 8-byte sources");
            store_nt(static_cast<u32x2*>(out) + v, u32x2{mfh_bits(decode_reg<IN>(w, 0)), mfh_bits(decode_reg<IN>(w, 1))});
        } else if constexpr (E == 2) {
            store_nt(static_cast<mfh_u32*>(out) + v, encode_pair<OUT>(decode_reg<IN>(w, 0), decode_reg<IN>(w, 1)));
        } else {
            store_nt(static_cast<u32x2*>(out) + v, u32x2{encode_pair<OUT>(decode_reg<IN>(w, 0), decode_reg<IN>(w, 1)),
                                                         encode_pair<OUT>(decode_reg<IN>(w, 2), decode_reg<IN>(w, 3))});
        }
    }
    const mfh_i64 i = npieces * E + threadIdx.x;
    if (blockIdx.x == 0 && threadIdx.x < E && i < n) store_one<OUT>(out, i, encode_one<OUT>(decode_at<IN>(in, i)));
}

bool aligned(const void* p, unsigned bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0; }

// ---------------------------------------------------------------------------
// Any numeric dtype -> one byte per element: FP8 (BytesToFloat8E4M3 /
// BytesToFloat8E5M2, dtype/convert/convert.go:194-232: BytesToFloat32, then
// the saturating RNE quantiser of codec.hpp) or Int8 (BytesToInt8, :235-263:
// BytesToFloat64, saturation to [-128, 127], truncation toward zero)
// ---------------------------------------------------------------------------

// int8(v) after BytesToInt8's saturation.  A NaN passes both of the
// reference's comparisons and Go converts it to 0 on amd64 and arm64; -Inf
// and +Inf saturate.  Values in range truncate toward zero (v_cvt_i32_f32 /
// v_cvt_i32_f64 truncate).
template <typename F>
MFH_DEV mfh_u32 i8_of(F v)
{
    const F c = v < F(-128) ? F(-128) : (v > F(127) ? F(127) : v);
    return c == c ? (mfh_u32)(int)c & 0xffu : 0u;
}

template <int ENC>
MFH_DEV mfh_u32 encode_byte(float v)
{
    if constexpr (ENC == kF8E4M3) return mfh_e4m3_encode(v);
    else if constexpr (ENC == kF8E5M2) return mfh_e5m2_encode(v);
    else return i8_of(v);
}

// BytesToFloat32 of element i for every source dtype, FP8 and Int4 included.
template <int IN>
MFH_DEV float decode_any(const void* in, mfh_i64 i)
{
    if constexpr (IN == kF8E4M3) return mfh_f32(mfh_e4m3_bits(static_cast<const mfh_u8*>(in)[i]));
    else if constexpr (IN == kF8E5M2) return mfh_f32(mfh_e5m2_bits(static_cast<const mfh_u8*>(in)[i]));
    else if constexpr (IN == kInt4)
        return (float)mfh_int4_at(static_cast<const mfh_u8*>(in)[i >> 1], (mfh_u32)(i & 1));
    else return decode_at<IN>(in, i);
}

// The output byte of element i.  Int8 from f64 truncates the f64 value
// itself (its f32 rounding could cross an integer); every other source is
// exact in f32, or (64-bit integers) rounds monotonically, which saturation
// and truncation cannot tell apart from its f64 value.
template <int IN, int ENC>
MFH_DEV mfh_u32 byte_at(const void* in, mfh_i64 i)
{
    if constexpr (ENC == kInt8 && IN == kFloat64) return i8_of(static_cast<const double*>(in)[i]);
    else return encode_byte<ENC>(decode_any<IN>(in, i));
}

// The same for element k of a register copy of consecutive elements.
template <int IN, int ENC>
MFH_DEV mfh_u32 byte_reg(const mfh_u32* w, int k)
{
    if constexpr (ENC == kInt8 && IN == kFloat64)
        return i8_of(__builtin_bit_cast(double, (mfh_u64)w[2 * k] | ((mfh_u64)w[2 * k + 1] << 32)));
    else return encode_byte<ENC>(decode_reg<IN>(w, k));
}

// Output bytes 4j .. 4j + 3 of a register copy of P consecutive elements,
// element 4j + k in byte k (bytes past P are zero codes).  FP8 codes leave
// the hardware converter four at a time.
template <int IN, int ENC, int P>
MFH_DEV mfh_u32 word_reg(const mfh_u32* w, int j)
{
    if constexpr (ENC == kF8E4M3 || ENC == kF8E5M2) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = 4 * j + k < P ? decode_reg<IN>(w, 4 * j + k) : 0.0f;
        return mfh_fp8x4_encode<ENC == kF8E5M2>(v[0], v[1], v[2], v[3]);
    } else {
        mfh_u32 word = 0u;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (4 * j + k < P) word |= byte_reg<IN, ENC>(w, 4 * j + k) << (8 * k);
        return word;
    }
}

// The output bytes of elements e0 .. e0 + 3, read from memory, element e0 + k in byte k.
template <int IN, int ENC>
MFH_DEV mfh_u32 word_at(const void* in, mfh_i64 e0)
{
    if constexpr (ENC == kF8E4M3 || ENC == kF8E5M2) {
        return mfh_fp8x4_encode<ENC == kF8E5M2>(decode_any<IN>(in, e0), decode_any<IN>(in, e0 + 1),
                                                decode_any<IN>(in, e0 + 2), decode_any<IN>(in, e0 + 3));
    } else {
        mfh_u32 word = 0u;
#pragma unroll
        for (int k = 0; k < 4; k++) word |= byte_at<IN, ENC>(in, e0 + k) << (8 * k);
        return word;
    }
}

// FP8 and Int4 sources, and any source whose buffers are not aligned for
// k_encode_byte_wave: item = 16 elements decoded one by one -> one 16-byte
// store of codes when the output is 16-byte aligned, else the element loop.
template <int IN, int ENC>
__global__ __launch_bounds__(kBlock) void k_encode_byte(const void* __restrict__ in, mfh_u8* __restrict__ out,
                                                        mfh_i64 n, int vec_ok)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    const mfh_i64 nitems = vec_ok ? n / 16 : 0;
    u32x4* dst = reinterpret_cast<u32x4*>(out);
    for (mfh_i64 v = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; v < nitems; v += stride) {
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; q++) o[q] = word_at<IN, ENC>(in, v * 16 + 4 * q);
        store_nt(&dst[v], o);
    }
    for (mfh_i64 i = nitems * 16 + (mfh_i64)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        out[i] = (mfh_u8)byte_at<IN, ENC>(in, i);
}

// Unpacked numeric dtype -> one byte per element with every load instruction
// of a wave reading 1 KiB contiguously: a wave takes chunks of 4 KiB of
// source, lane l the 16-byte pieces l, l + 64, l + 128 and l + 192 of its
// chunk, and writes the 16 / size output bytes of each piece next to its
// neighbours' (16-, 8-, 4- or 2-byte stores).  Lanes taking two adjacent
// pieces each, so that 2-byte sources store 16 bytes at a time, split every
// load instruction over 2 KiB: bf16 -> e4m3 ran 4% slower that way.  One lane
// taking 16 consecutive elements (64 bytes of f32) spreads each load
// instruction over 4 KiB: f32 -> e4m3 ran at 4.4 TB/s that way.  Elements
// past the last whole chunk run the element loop.
template <int IN, int ENC, int BS>
__global__ __launch_bounds__(BS) void k_encode_byte_wave(const void* __restrict__ in, mfh_u8* __restrict__ out,
                                                             mfh_i64 n)
{
    constexpr int S = size_of<IN>();
    constexpr int P = 16 / S;          // elements (and output bytes) per 16-byte piece
    constexpr int kPieces = 4;         // pieces per lane per chunk
    constexpr mfh_i64 kChunk = 64 * kPieces * P;  // elements per wave chunk
    const int lane = (int)threadIdx.x & 63;
    const mfh_i64 waves = (mfh_i64)gridDim.x * (BS / 64);
    const mfh_i64 nchunks = n / kChunk;
    for (mfh_i64 c = (mfh_i64)blockIdx.x * (BS / 64) + (threadIdx.x >> 6); c < nchunks; c += waves) {
        u32x4 x[kPieces];
#pragma unroll
        for (int q = 0; q < kPieces; q++)
            x[q] = load_nt(reinterpret_cast<const u32x4*>(in) + c * (64 * kPieces) + q * 64 + lane);
#pragma unroll
        for (int q = 0; q < kPieces; q++) {
            const mfh_u32 w[4] = {x[q][0], x[q][1], x[q][2], x[q][3]};
            mfh_u32 code[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < (P + 3) / 4; j++) code[j] = word_reg<IN, ENC, P>(w, j);
            const mfh_i64 e0 = c * kChunk + (mfh_i64)(q * 64 + lane) * P;
            if constexpr (P == 16) store_nt(reinterpret_cast<u32x4*>(out + e0), u32x4{code[0], code[1], code[2], code[3]});
            else if constexpr (P == 8) store_nt(reinterpret_cast<u32x2*>(out + e0), u32x2{code[0], code[1]});
            else if constexpr (P == 4) store_nt(reinterpret_cast<mfh_u32*>(out + e0), code[0]);
            else store_nt(reinterpret_cast<mfh_u16*>(out + e0), (mfh_u16)code[0]);
        }
    }
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    for (mfh_i64 i = nchunks * kChunk + (mfh_i64)blockIdx.x * BS + threadIdx.x; i < n; i += stride)
        out[i] = (mfh_u8)byte_at<IN, ENC>(in, i);
}

// Workgroup size of a cast unless the launch config sets one.  Measured at
// 2^26 elements against 256 threads: one wave wins wherever the output is at
// most twice the source (f32 -> bf16 +13%, f32 copy +4%, bf16 -> f32 +3.5%,
// int32 -> f32 +3%, FP8 encode +1%) and loses where it is four times the
// source (int8 -> f32 -19%), which keeps 256.
int cast_threads(int in_dt, int out_size)
{
    const int set = threads_per_block(Kern::kConvert);
    if (set > 0) return set;
    const int src = dtype_size(in_dt);
    return src > 0 && out_size >= 4 * src ? 256 : 64;
}

template <int ENC, int BS>
int launch_encode_byte_wave(const Device* dev, mfh_u8* out, const void* in, int in_dt, int64_t n, int size,
                            hipStream_t stream)
{
    const int64_t chunk_elems = 64 * 4 * (16 / size);
    const unsigned grid = grid_for(std::max<int64_t>(n / chunk_elems, 1) * 64, dev, Kern::kConvert, 1, BS);
    switch (in_dt) {
#define MFH_ENCODE_WAVE_CASE(DT) \
    case DT: k_encode_byte_wave<DT, ENC, BS><<<grid, BS, 0, stream>>>(in, out, n); break;
        MFH_ENCODE_WAVE_CASE(kFloat64)
        MFH_ENCODE_WAVE_CASE(kFloat32)
        MFH_ENCODE_WAVE_CASE(kFloat16)
        MFH_ENCODE_WAVE_CASE(kBFloat16)
        MFH_ENCODE_WAVE_CASE(kInt64)
        MFH_ENCODE_WAVE_CASE(kInt32)
        MFH_ENCODE_WAVE_CASE(kInt16)
        MFH_ENCODE_WAVE_CASE(kInt8)
        MFH_ENCODE_WAVE_CASE(kUint64)
        MFH_ENCODE_WAVE_CASE(kUint32)
        MFH_ENCODE_WAVE_CASE(kUint16)
        MFH_ENCODE_WAVE_CASE(kUint8)
#undef MFH_ENCODE_WAVE_CASE
    default:
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: input dtype %s is not supported", dtype_name(in_dt));
    }
    return launch_status("k_encode_byte_wave");
}

template <int ENC>
int launch_encode_byte(const Device* dev, mfh_u8* out, const void* in, int in_dt, int64_t n, hipStream_t stream)
{
    // unpacked numeric sources: whole 4 KiB source chunks per wave when the
    // source is 16-byte aligned and the output aligned for the kernel's
    // stores (16 / size bytes)
    const int size = in_dt == kF8E4M3 || in_dt == kF8E5M2 || in_dt == kInt4 ? 0 : dtype_size(in_dt);
    if (size > 0 && aligned16(in) && (reinterpret_cast<uintptr_t>(out) & (uintptr_t)(16 / size - 1)) == 0)
        return with_block(cast_threads(in_dt, 1), [&](auto block) {
            return launch_encode_byte_wave<ENC, decltype(block)::value>(dev, out, in, in_dt, n, size, stream);
        });
    const int vec_ok = aligned16(out) && n >= 16;
    const int64_t items = vec_ok ? n / 16 : n;
    const unsigned grid = grid_for(items, dev, Kern::kConvert);
    switch (in_dt) {
#define MFH_ENCODE_CASE(DT) \
    case DT: k_encode_byte<DT, ENC><<<grid, kBlock, 0, stream>>>(in, out, n, vec_ok); break;
        MFH_ENCODE_CASE(kFloat64)
        MFH_ENCODE_CASE(kFloat32)
        MFH_ENCODE_CASE(kFloat16)
        MFH_ENCODE_CASE(kBFloat16)
        MFH_ENCODE_CASE(kF8E4M3)
        MFH_ENCODE_CASE(kF8E5M2)
        MFH_ENCODE_CASE(kInt64)
        MFH_ENCODE_CASE(kInt32)
        MFH_ENCODE_CASE(kInt16)
        MFH_ENCODE_CASE(kInt8)
        MFH_ENCODE_CASE(kInt4)
        MFH_ENCODE_CASE(kUint64)
        MFH_ENCODE_CASE(kUint32)
        MFH_ENCODE_CASE(kUint16)
        MFH_ENCODE_CASE(kUint8)
#undef MFH_ENCODE_CASE
    default:
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: input dtype %s is not supported", dtype_name(in_dt));
    }
    return launch_status("k_encode_byte");
}

// ---------------------------------------------------------------------------
// Any numeric dtype -> packed Int4: BytesToInt8's value (saturated to
// [-128, 127], truncated, NaN -> 0), then int4Encode (dtype/int4.go:60-70):
// clamped to [-8, 7], low nibble first.  An odd count leaves the last byte's
// high nibble 0, as a fresh Int4Vector holds it (tensor/int4vector.go:74-87).
// ---------------------------------------------------------------------------

template <int IN>
MFH_DEV mfh_u32 nibble_at(const void* in, mfh_i64 i)
{
    const int v = (int)(signed char)byte_at<IN, kInt8>(in, i);
    return (mfh_u32)(v < -8 ? -8 : (v > 7 ? 7 : v)) & 0xfu;
}

// The same for element k of a register copy of consecutive elements.
// Integer sources clamp the integer itself: every integer type converts to
// f64 monotonically, so saturating and truncating its f64 value and then
// clamping gives the same nibble, without the float round trip.
template <int IN>
MFH_DEV mfh_u32 nibble_reg(const mfh_u32* w, int k)
{
    constexpr int S = size_of<IN>();
    int v;
    if constexpr (IN == kInt8 || IN == kInt16) {
        const int x = __builtin_amdgcn_sbfe((int)w[k * S / 4], (k * 8 * S) & 31, 8 * S);
        v = x < -8 ? -8 : (x > 7 ? 7 : x);
    } else if constexpr (IN == kUint8 || IN == kUint16) {
        const mfh_u32 x = __builtin_amdgcn_ubfe(w[k * S / 4], (k * 8 * S) & 31, 8 * S);
        v = x > 7u ? 7 : (int)x;
    } else if constexpr (IN == kInt32) {
        const int x = (int)w[k];
        v = x < -8 ? -8 : (x > 7 ? 7 : x);
    } else if constexpr (IN == kUint32) {
        v = w[k] > 7u ? 7 : (int)w[k];
    } else if constexpr (IN == kInt64) {
        const long long x = (long long)((mfh_u64)w[2 * k] | ((mfh_u64)w[2 * k + 1] << 32));
        v = x < -8 ? -8 : (x > 7 ? 7 : (int)x);
    } else if constexpr (IN == kUint64) {
        const mfh_u64 x = (mfh_u64)w[2 * k] | ((mfh_u64)w[2 * k + 1] << 32);
        v = x > 7u ? 7 : (int)x;
    } else {
        const int x = (int)(signed char)byte_reg<IN, kInt8>(w, k);
        v = x < -8 ? -8 : (x > 7 ? 7 : x);
    }
    return (mfh_u32)v & 0xfu;
}

// Item = 32 elements -> one 16-byte store of nibbles (16-byte aligned
// output), then the byte loop for the rest.
template <int IN>
__global__ __launch_bounds__(kBlock) void k_encode_int4(const void* __restrict__ in, mfh_u8* __restrict__ out,
                                                        mfh_i64 n, int vec_ok)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    const mfh_i64 nitems = vec_ok ? n / 32 : 0;
    u32x4* dst = reinterpret_cast<u32x4*>(out);
    for (mfh_i64 v = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; v < nitems; v += stride) {
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            mfh_u32 word = 0u;
#pragma unroll
            for (int k = 0; k < 8; k++) word |= nibble_at<IN>(in, v * 32 + 8 * q + k) << (4 * k);
            o[q] = word;
        }
        store_nt(&dst[v], o);
    }
    const mfh_i64 nbytes = (n + 1) / 2;
    for (mfh_i64 b = nitems * 16 + (mfh_i64)blockIdx.x * kBlock + threadIdx.x; b < nbytes; b += stride) {
        const mfh_u32 lo = nibble_at<IN>(in, 2 * b);
        const mfh_u32 hi = 2 * b + 1 < n ? nibble_at<IN>(in, 2 * b + 1) : 0u;
        out[b] = (mfh_u8)(lo | (hi << 4));
    }
}

// Unpacked numeric sources, laid out as k_encode_byte_wave: a wave takes 4 KiB
// of source, lane l its 16-byte pieces l, l + 64, l + 128 and l + 192, so
// every load instruction reads 1 KiB contiguously; the 16 / size elements of
// a piece leave as 8 / size bytes of nibbles next to the neighbours' ones.
// Elements past the last whole chunk run the byte loop.
template <int IN, int BS>
__global__ __launch_bounds__(BS) void k_encode_int4_wave(const void* __restrict__ in, mfh_u8* __restrict__ out,
                                                             mfh_i64 n)
{
    constexpr int S = size_of<IN>();
    constexpr int P = 16 / S;  // elements per 16-byte piece
    constexpr int kPieces = 4;
    constexpr mfh_i64 kChunk = 64 * kPieces * P;
    const int lane = (int)threadIdx.x & 63;
    const mfh_i64 waves = (mfh_i64)gridDim.x * (BS / 64);
    const mfh_i64 nchunks = n / kChunk;
    for (mfh_i64 c = (mfh_i64)blockIdx.x * (BS / 64) + (threadIdx.x >> 6); c < nchunks; c += waves) {
        u32x4 x[kPieces];
#pragma unroll
        for (int q = 0; q < kPieces; q++) x[q] = load_nt(reinterpret_cast<const u32x4*>(in) + c * (64 * kPieces) + q * 64 + lane);
#pragma unroll
        for (int q = 0; q < kPieces; q++) {
            const mfh_u32 w[4] = {x[q][0], x[q][1], x[q][2], x[q][3]};
            mfh_u32 code[2] = {0u, 0u};
#pragma unroll
            for (int k = 0; k < P; k++) code[k >> 3] |= nibble_reg<IN>(w, k) << (4 * (k & 7));
            mfh_u8* o = out + (c * kChunk + (mfh_i64)(q * 64 + lane) * P) / 2;
            if constexpr (P == 16) store_nt(reinterpret_cast<u32x2*>(o), u32x2{code[0], code[1]});
            else if constexpr (P == 8) store_nt(reinterpret_cast<mfh_u32*>(o), code[0]);
            else if constexpr (P == 4) store_nt(reinterpret_cast<mfh_u16*>(o), (mfh_u16)code[0]);
            else *o = (mfh_u8)code[0];
        }
    }
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    const mfh_i64 nbytes = (n + 1) / 2;
    for (mfh_i64 b = nchunks * kChunk / 2 + (mfh_i64)blockIdx.x * BS + threadIdx.x; b < nbytes; b += stride) {
        const mfh_u32 lo = nibble_at<IN>(in, 2 * b);
        const mfh_u32 hi = 2 * b + 1 < n ? nibble_at<IN>(in, 2 * b + 1) : 0u;
        out[b] = (mfh_u8)(lo | (hi << 4));
    }
}

template <int BS>
int launch_encode_int4_wave(const Device* dev, mfh_u8* out, const void* in, int in_dt, int64_t n, int size,
                            hipStream_t stream)
{
    const int64_t chunk_elems = 64 * 4 * (16 / size);
    const unsigned grid = grid_for(std::max<int64_t>(n / chunk_elems, 1) * 64, dev, Kern::kConvert, 1, BS);
    switch (in_dt) {
#define MFH_ENCODE_I4_WAVE_CASE(DT) \
    case DT: k_encode_int4_wave<DT, BS><<<grid, BS, 0, stream>>>(in, out, n); break;
        MFH_ENCODE_I4_WAVE_CASE(kFloat64)
        MFH_ENCODE_I4_WAVE_CASE(kFloat32)
        MFH_ENCODE_I4_WAVE_CASE(kFloat16)
        MFH_ENCODE_I4_WAVE_CASE(kBFloat16)
        MFH_ENCODE_I4_WAVE_CASE(kInt64)
        MFH_ENCODE_I4_WAVE_CASE(kInt32)
        MFH_ENCODE_I4_WAVE_CASE(kInt16)
        MFH_ENCODE_I4_WAVE_CASE(kInt8)
        MFH_ENCODE_I4_WAVE_CASE(kUint64)
        MFH_ENCODE_I4_WAVE_CASE(kUint32)
        MFH_ENCODE_I4_WAVE_CASE(kUint16)
        MFH_ENCODE_I4_WAVE_CASE(kUint8)
#undef MFH_ENCODE_I4_WAVE_CASE
    default:
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: input dtype %s is not supported", dtype_name(in_dt));
    }
    return launch_status("k_encode_int4_wave");
}

int launch_encode_int4(const Device* dev, mfh_u8* out, const void* in, int in_dt, int64_t n, hipStream_t stream)
{
    // unpacked numeric sources aligned to 16 bytes, the output aligned to one
    // piece's bytes of nibbles (8 / size), take the wave layout
    const int size = in_dt == kF8E4M3 || in_dt == kF8E5M2 || in_dt == kInt4 ? 0 : dtype_size(in_dt);
    if (size > 0 && aligned16(in) && (reinterpret_cast<uintptr_t>(out) & (uintptr_t)(std::max(1, 8 / size) - 1)) == 0)
        return with_block(cast_threads(in_dt, 1), [&](auto block) {
            return launch_encode_int4_wave<decltype(block)::value>(dev, out, in, in_dt, n, size, stream);
        });
    const int vec_ok = aligned16(out) && n >= 32;
    const int64_t items = vec_ok ? n / 32 : (n + 1) / 2;
    const unsigned grid = grid_for(items, dev, Kern::kConvert);
    switch (in_dt) {
#define MFH_ENCODE_I4_CASE(DT) \
    case DT: k_encode_int4<DT><<<grid, kBlock, 0, stream>>>(in, out, n, vec_ok); break;
        MFH_ENCODE_I4_CASE(kFloat64)
        MFH_ENCODE_I4_CASE(kFloat32)
        MFH_ENCODE_I4_CASE(kFloat16)
        MFH_ENCODE_I4_CASE(kBFloat16)
        MFH_ENCODE_I4_CASE(kF8E4M3)
        MFH_ENCODE_I4_CASE(kF8E5M2)
        MFH_ENCODE_I4_CASE(kInt64)
        MFH_ENCODE_I4_CASE(kInt32)
        MFH_ENCODE_I4_CASE(kInt16)
        MFH_ENCODE_I4_CASE(kInt8)
        MFH_ENCODE_I4_CASE(kInt4)
        MFH_ENCODE_I4_CASE(kUint64)
        MFH_ENCODE_I4_CASE(kUint32)
        MFH_ENCODE_I4_CASE(kUint16)
        MFH_ENCODE_I4_CASE(kUint8)
#undef MFH_ENCODE_I4_CASE
    default:
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: input dtype %s is not supported", dtype_name(in_dt));
    }
    return launch_status("k_encode_int4");
}

// ---------------------------------------------------------------------------
// Any numeric dtype -> f64 (BytesToFloat64, dtype/convert/convert.go:36-79)
// ---------------------------------------------------------------------------

// float64(float32) as Go compiles it on amd64 (cvtss2sd), on the bits: exact
// for every number (denormals renormalised, so no device denormal mode is
// involved), a NaN quieted with its sign and payload kept.
MFH_DEV mfh_u64 f64_bits_of_f32(mfh_u32 b)
{
    const mfh_u64 sign = (mfh_u64)(b >> 31) << 63;
    const mfh_u32 e = (b >> 23) & 0xffu, m = b & 0x7fffffu;
    if (e == 0xffu) return sign | 0x7ff0000000000000ull | (m ? 0x0008000000000000ull : 0ull) | ((mfh_u64)m << 29);
    if (e != 0u) return sign | ((mfh_u64)(e + 896u) << 52) | ((mfh_u64)m << 29);
    if (m == 0u) return sign;
    const int p = 31 - __builtin_clz(m);  // top set bit of the denormal's fraction, 0..22
    return sign | ((mfh_u64)(p + 874) << 52) | (((mfh_u64)m << (52 - p)) & 0xfffffffffffffull);
}

// The f64 bits of element k of a register copy of consecutive elements
// (Int4: nibble k of the copy).  Integers convert with correctly rounded
// int -> f64 conversions (the 64-bit ones as two exact halves and one add).
template <int IN>
MFH_DEV mfh_u64 f64_reg(const mfh_u32* w, int k)
{
    if constexpr (IN == kFloat64) return (mfh_u64)w[2 * k] | ((mfh_u64)w[2 * k + 1] << 32);
    else if constexpr (IN == kInt64)
        return __builtin_bit_cast(mfh_u64, (double)(long long)((mfh_u64)w[2 * k] | ((mfh_u64)w[2 * k + 1] << 32)));
    else if constexpr (IN == kUint64)
        return __builtin_bit_cast(mfh_u64, (double)((mfh_u64)w[2 * k] | ((mfh_u64)w[2 * k + 1] << 32)));
    else if constexpr (IN == kInt32) return __builtin_bit_cast(mfh_u64, (double)(int)w[k]);
    else if constexpr (IN == kUint32) return __builtin_bit_cast(mfh_u64, (double)w[k]);
    else if constexpr (IN == kInt4) return __builtin_bit_cast(mfh_u64, (double)mfh_int4_at(w[k >> 3], (mfh_u32)(k & 7)));
    else if constexpr (IN == kF8E4M3 || IN == kF8E5M2) {
        const mfh_u32 code = (w[k >> 2] >> ((k & 3) * 8)) & 0xffu;
        return f64_bits_of_f32(IN == kF8E4M3 ? mfh_e4m3_bits(code) : mfh_e5m2_bits(code));
    } else if constexpr (IN == kInt16 || IN == kUint16 || IN == kInt8 || IN == kUint8)
        return __builtin_bit_cast(mfh_u64, (double)decode_reg<IN>(w, k));  // exact in f32
    else return f64_bits_of_f32(mfh_bits(decode_reg<IN>(w, k)));          // f32, f16, bf16
}

// Element i from memory (tails, misaligned buffers).
template <int IN>
MFH_DEV mfh_u64 f64_at(const void* in, mfh_i64 i)
{
    if constexpr (IN == kInt4) {
        const mfh_u32 byte = static_cast<const mfh_u8*>(in)[i >> 1];
        return __builtin_bit_cast(mfh_u64, (double)mfh_int4_at(byte, (mfh_u32)(i & 1)));
    } else {
        constexpr int S = IN == kF8E4M3 || IN == kF8E5M2 ? 1 : size_of<IN>();
        mfh_u32 w[2] = {0u, 0u};
        const mfh_u8* p = static_cast<const mfh_u8*>(in) + i * S;
#pragma unroll
        for (int b = 0; b < S; b++) w[b >> 2] |= (mfh_u32)p[b] << (8 * (b & 3));
        return f64_reg<IN>(w, 0);
    }
}

// Item = 2 elements -> one 16-byte store; the item's 2 * size source bytes
// (one byte for two Int4 nibbles) are one load.  Elements past the last whole
// item, and every element when a buffer is not aligned, run the element loop.
template <int IN, int BS>
__global__ __launch_bounds__(BS) void k_widen_f64(const void* __restrict__ in, void* __restrict__ out, mfh_i64 n,
                                                      int vec_ok)
{
    constexpr int S = IN == kF8E4M3 || IN == kF8E5M2 ? 1 : IN == kInt4 ? 0 : size_of<IN>();
    const mfh_i64 stride = (mfh_i64)gridDim.x * BS;
    const mfh_i64 nitems = vec_ok ? n / 2 : 0;
    u32x4* dst = reinterpret_cast<u32x4*>(out);
    for (mfh_i64 v = (mfh_i64)blockIdx.x * BS + threadIdx.x; v < nitems; v += stride) {
        mfh_u32 w[4] = {0u, 0u, 0u, 0u};
        if constexpr (S == 8) {
            const u32x4 x = load_nt(reinterpret_cast<const u32x4*>(in) + v);
            w[0] = x[0], w[1] = x[1], w[2] = x[2], w[3] = x[3];
        } else if constexpr (S == 4) {
            const u32x2 x = reinterpret_cast<const u32x2*>(in)[v];
            w[0] = x[0], w[1] = x[1];
        } else if constexpr (S == 2) {
            w[0] = reinterpret_cast<const mfh_u32*>(in)[v];
        } else if constexpr (S == 1) {
            w[0] = reinterpret_cast<const mfh_u16*>(in)[v];
        } else {
            w[0] = static_cast<const mfh_u8*>(in)[v];  // Int4: two nibbles
        }
        const mfh_u64 a = f64_reg<IN>(w, 0), b = f64_reg<IN>(w, 1);
        store_nt(&dst[v], u32x4{(mfh_u32)a, (mfh_u32)(a >> 32), (mfh_u32)b, (mfh_u32)(b >> 32)});
    }
    for (mfh_i64 i = nitems * 2 + (mfh_i64)blockIdx.x * BS + threadIdx.x; i < n; i += stride)
        static_cast<mfh_u64*>(out)[i] = f64_at<IN>(in, i);
}

int launch_widen_f64(const Device* dev, void* out, const void* in, int in_dt, int64_t n, hipStream_t stream)
{
    const int size = in_dt == kF8E4M3 || in_dt == kF8E5M2 ? 1 : in_dt == kInt4 ? 0 : dtype_size(in_dt);
    if (size == 0 && in_dt != kInt4)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: input dtype %s is not supported", dtype_name(in_dt));
    const int vec_ok = aligned16(out) && aligned(in, (unsigned)std::max(1, 2 * size)) && n >= 2;
    return with_block(cast_threads(in_dt, 8), [&](auto block) {
        constexpr int BS = decltype(block)::value;
        const unsigned grid = vec_ok ? grid_for(n / 2, dev, Kern::kConvert, 1, BS) : grid_for(n, dev, Kern::kConvert, 1, BS);
        switch (in_dt) {
#define MFH_WIDEN_CASE(DT) \
    case DT: k_widen_f64<DT, BS><<<grid, BS, 0, stream>>>(in, out, n, vec_ok); break;
            MFH_WIDEN_CASE(kFloat64)
            MFH_WIDEN_CASE(kFloat32)
            MFH_WIDEN_CASE(kFloat16)
            MFH_WIDEN_CASE(kBFloat16)
            MFH_WIDEN_CASE(kF8E4M3)
            MFH_WIDEN_CASE(kF8E5M2)
            MFH_WIDEN_CASE(kInt64)
            MFH_WIDEN_CASE(kInt32)
            MFH_WIDEN_CASE(kInt16)
            MFH_WIDEN_CASE(kInt8)
            MFH_WIDEN_CASE(kInt4)
            MFH_WIDEN_CASE(kUint64)
            MFH_WIDEN_CASE(kUint32)
            MFH_WIDEN_CASE(kUint16)
            MFH_WIDEN_CASE(kUint8)
#undef MFH_WIDEN_CASE
        default:
            return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: input dtype %s is not supported", dtype_name(in_dt));
        }
        return launch_status("k_widen_f64");
    });
}

bool is_out_dtype(int dt) { return dt == kFloat32 || dt == kBFloat16 || dt == kFloat16; }

template <template <int> class F, typename... A>
int by_out(int out_dt, A... args)
{
    switch (out_dt) {
    case kFloat32: return F<kFloat32>::run(args...);
    case kBFloat16: return F<kBFloat16>::run(args...);
    case kFloat16: return F<kFloat16>::run(args...);
    default: return fail(MFH_ERR_DTYPE_UNSUPPORTED, "output dtype %s is not f32/bf16/f16", dtype_name(out_dt));
    }
}

template <int OUT>
struct Fp8Launch {
    static int run(const Device* dev, void* out, const void* in, int fmt, int64_t n, float scale,
                   hipStream_t stream)
    {
        constexpr int codes = OUT == kFloat32 ? 4 : 8;
        int vec_ok = aligned(in, codes) && aligned16(out);
        int64_t items = vec_ok ? std::max<int64_t>(n / codes, 1) : n;
        const mfh_u8* src = static_cast<const mfh_u8*>(in);
        const int u = items_per_thread(Kern::kFp8);
        return with_block(threads_per_block(Kern::kFp8), [&](auto block) {
            constexpr int BS = decltype(block)::value;
            const unsigned grid = grid_for(items, dev, Kern::kFp8, u, BS);
            if (u == 4) k_dequant_fp8<OUT, 4, BS><<<grid, BS, 0, stream>>>(src, out, n, scale, fmt, vec_ok);
            else if (u == 2) k_dequant_fp8<OUT, 2, BS><<<grid, BS, 0, stream>>>(src, out, n, scale, fmt, vec_ok);
            else k_dequant_fp8<OUT, 1, BS><<<grid, BS, 0, stream>>>(src, out, n, scale, fmt, vec_ok);
            return launch_status("k_dequant_fp8");
        });
    }
};

int log2_exact(int64_t g)
{
    if (g <= 0 || (g & (g - 1)) != 0) return -1;
    int s = 0;
    while ((int64_t(1) << s) < g) s++;
    return s;
}

template <int OUT>
struct Int4Launch {
    static int run(const Device* dev, void* out, const void* packed, int64_t n, const void* scales,
                   int scale_dt, int64_t group, hipStream_t stream)
    {
        constexpr int elems = OUT == kFloat32 ? 4 : 8;
        int shift = log2_exact(group);
        int vec_ok = aligned(packed, elems / 2) && aligned16(out) && shift >= 0 && group >= elems;
        int64_t items = vec_ok ? std::max<int64_t>(n / elems, 1) : n;
        const int u = items_per_thread(Kern::kInt4);
        const mfh_u8* p = static_cast<const mfh_u8*>(packed);
        return with_block_to_512(threads_per_block(Kern::kInt4), [&](auto block) {
            constexpr int BS = decltype(block)::value;
            const unsigned grid = grid_for(items, dev, Kern::kInt4, u, BS);
            if (u == 4) launch<4, BS>(grid, p, scales, scale_dt, out, n, group, shift, vec_ok, stream);
            else if (u == 2) launch<2, BS>(grid, p, scales, scale_dt, out, n, group, shift, vec_ok, stream);
            else launch<1, BS>(grid, p, scales, scale_dt, out, n, group, shift, vec_ok, stream);
            return launch_status("k_dequant_int4");
        });
    }

    template <int U, int BS>
    static void launch(unsigned grid, const mfh_u8* p, const void* scales, int scale_dt, void* out, int64_t n,
                       int64_t group, int shift, int vec_ok, hipStream_t stream)
    {
        switch (scale_dt) {
        case kFloat32: k_dequant_int4<OUT, kFloat32, U, BS><<<grid, BS, 0, stream>>>(p, scales, out, n, group, shift, vec_ok); break;
        case kFloat16: k_dequant_int4<OUT, kFloat16, U, BS><<<grid, BS, 0, stream>>>(p, scales, out, n, group, shift, vec_ok); break;
        case kBFloat16: k_dequant_int4<OUT, kBFloat16, U, BS><<<grid, BS, 0, stream>>>(p, scales, out, n, group, shift, vec_ok); break;
        default: k_dequant_int4<OUT, kInvalid, U, BS><<<grid, BS, 0, stream>>>(p, scales, out, n, group, shift, vec_ok); break;
        }
    }
};

template <int OUT>
struct ConvertLaunch {
    static int run(const Device* dev, void* out, const void* in, int in_dt, int64_t n, hipStream_t stream)
    {
        return with_block(cast_threads(in_dt, OUT == kFloat32 ? 4 : 2), [&](auto block) {
            return run_bs<decltype(block)::value>(dev, out, in, in_dt, n, stream);
        });
    }

    template <int BS>
    static int run_bs(const Device* dev, void* out, const void* in, int in_dt, int64_t n, hipStream_t stream)
    {
        constexpr int per = OUT == kFloat32 ? 4 : 8;
        if ((in_dt == kBFloat16 || in_dt == kFloat16) && aligned(in, per * 2) && aligned16(out) && n % per == 0) {
            int64_t nitems = n / per;
            // one item per thread unless the launch config sets two: the
            // widening to f32 ran 1% slower with two
            const int u = items_per_thread(Kern::kConvert) >= 2 ? 2 : 1;
            unsigned grid = grid_for(nitems, dev, Kern::kConvert, u, BS);
            if (in_dt == kBFloat16 && u == 2) k_convert16_vec<kBFloat16, OUT, BS, 2><<<grid, BS, 0, stream>>>(in, out, nitems);
            else if (in_dt == kBFloat16) k_convert16_vec<kBFloat16, OUT, BS, 1><<<grid, BS, 0, stream>>>(in, out, nitems);
            else if (u == 2) k_convert16_vec<kFloat16, OUT, BS, 2><<<grid, BS, 0, stream>>>(in, out, nitems);
            else k_convert16_vec<kFloat16, OUT, BS, 1><<<grid, BS, 0, stream>>>(in, out, nitems);
            return launch_status("k_convert16_vec");
        }
        {
            // 8-byte sources, and 4-byte integers to 16-bit: one 16-byte
            // source piece per lane
            const int sz = dtype_size(in_dt);
            const bool narrow = in_dt == kFloat64 || in_dt == kInt64 || in_dt == kUint64 ||
                                (OUT != kFloat32 && (in_dt == kInt32 || in_dt == kUint32));
            const unsigned out_bytes = (unsigned)(16 / std::max(sz, 1) * size_of<OUT>());
            if (narrow && aligned16(in) && aligned(out, out_bytes)) {
                const unsigned grid = grid_for(std::max<int64_t>(n / (16 / sz), 1), dev, Kern::kConvert, 1, BS);
                const u32x4* src = static_cast<const u32x4*>(in);
                switch (in_dt) {
                case kFloat64: k_narrow_vec<kFloat64, OUT, BS><<<grid, BS, 0, stream>>>(src, out, n); break;
                case kInt64: k_narrow_vec<kInt64, OUT, BS><<<grid, BS, 0, stream>>>(src, out, n); break;
                case kUint64: k_narrow_vec<kUint64, OUT, BS><<<grid, BS, 0, stream>>>(src, out, n); break;
                default:
                    if constexpr (OUT != kFloat32) {
                        if (in_dt == kInt32) k_narrow_vec<kInt32, OUT, BS><<<grid, BS, 0, stream>>>(src, out, n);
                        else k_narrow_vec<kUint32, OUT, BS><<<grid, BS, 0, stream>>>(src, out, n);
                    }
                    break;
                }
                return launch_status("k_narrow_vec");
            }
        }
        if constexpr (OUT != kFloat32) {
            if (in_dt == kFloat32 && aligned16(in) && aligned(out, 8) && n % 4 == 0) {
                int64_t nitems = n / 4;
                k_narrow_f32_vec<OUT, BS><<<grid_for(nitems, dev, Kern::kConvert, 1, BS), BS, 0, stream>>>(
                    static_cast<const u32x4*>(in), static_cast<u32x2*>(out), nitems);
                return launch_status("k_narrow_f32_vec");
            }
        }
        // every other source: whole 16-byte output items when both buffers
        // are aligned for them, else the element loop (256 threads)
        const int src_size = dtype_size(in_dt);
        const bool vec = src_size > 0 && aligned(in, (unsigned)std::min(per * src_size, 16)) && aligned16(out);
        // items per thread: two where the output is four times the source
        // (int8 -> f32 +14%), one elsewhere (same-width copies lose 2-3%
        // with two, 2x widening gains nothing), unless the launch config
        // sets them
        const int set_u = items_per_thread(Kern::kConvert);
        const int u = set_u > 0 ? (set_u >= 2 ? 2 : 1) : (size_of<OUT>() >= 4 * src_size ? 2 : 1);
        const unsigned grid = vec ? grid_for(std::max<int64_t>(n / per, 1), dev, Kern::kConvert, u, BS)
                                  : grid_for(n, dev, Kern::kConvert);
        switch (in_dt) {
#define MFH_CONVERT_CASE(DT)                                                                  \
    case DT:                                                                              \
        if (vec && u == 2) k_convert_vec<DT, OUT, BS, 2><<<grid, BS, 0, stream>>>(in, out, n); \
        else if (vec) k_convert_vec<DT, OUT, BS, 1><<<grid, BS, 0, stream>>>(in, out, n); \
        else k_convert<DT, OUT><<<grid, kBlock, 0, stream>>>(in, out, n);                 \
        break;
        MFH_CONVERT_CASE(kFloat64)
        MFH_CONVERT_CASE(kFloat32)
        MFH_CONVERT_CASE(kFloat16)
        MFH_CONVERT_CASE(kBFloat16)
        MFH_CONVERT_CASE(kInt64)
        MFH_CONVERT_CASE(kInt32)
        MFH_CONVERT_CASE(kInt16)
        MFH_CONVERT_CASE(kInt8)
        MFH_CONVERT_CASE(kUint64)
        MFH_CONVERT_CASE(kUint32)
        MFH_CONVERT_CASE(kUint16)
        MFH_CONVERT_CASE(kUint8)
#undef MFH_CONVERT_CASE
        default:
            return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: input dtype %s is not supported",
                        dtype_name(in_dt));
        }
        return launch_status("k_convert");
    }
};

}  // namespace
}  // namespace mfh

using namespace mfh;

extern "C" {

int mfh_dequant_fp8(void* out, uint8_t out_dtype, const void* in, uint8_t fp8_dtype, int64_t count,
                    float scale, void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (fp8_dtype != kF8E4M3 && fp8_dtype != kF8E5M2)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_dequant_fp8: %s is not an FP8 dtype", dtype_name(fp8_dtype));
    if (count < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_dequant_fp8: negative count %lld", (long long)count);
    if (!is_out_dtype(out_dtype))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "output dtype %s is not f32/bf16/f16", dtype_name(out_dtype));
    if (count == 0) return MFH_OK;
    if (!out || !in) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_dequant_fp8: NULL buffer");
    return by_out<Fp8Launch>(out_dtype, dev, out, in, (int)fp8_dtype, count, scale, (hipStream_t)stream);
}

int mfh_dequant_int4(void* out, uint8_t out_dtype, const void* packed, int64_t count, const void* scales,
                     uint8_t scale_dtype, int64_t group, void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (scale_dtype != kFloat32 && scale_dtype != kFloat16 && scale_dtype != kBFloat16)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_dequant_int4: scale dtype %s is not f32/f16/bf16",
                    dtype_name(scale_dtype));
    if (group <= 0) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_dequant_int4: group must be positive, got %lld", (long long)group);
    if (count < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_dequant_int4: negative count %lld", (long long)count);
    if (!is_out_dtype(out_dtype))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "output dtype %s is not f32/bf16/f16", dtype_name(out_dtype));
    if (count == 0) return MFH_OK;
    if (!out || !packed || !scales) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_dequant_int4: NULL buffer");
    return by_out<Int4Launch>(out_dtype, dev, out, packed, count, scales, (int)scale_dtype, group,
                              (hipStream_t)stream);
}

int mfh_convert(void* out, uint8_t out_dtype, const void* in, uint8_t in_dtype, int64_t count, void* stream)
{
    const Device* dev;
    MFH_TRY(bind_device(&dev));
    if (count < 0) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_convert: negative count %lld", (long long)count);
    const bool to_byte = out_dtype == kF8E4M3 || out_dtype == kF8E5M2 || out_dtype == kInt8;
    if (!is_out_dtype(out_dtype) && !to_byte && out_dtype != kFloat64 && out_dtype != kInt4)
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: output dtype %s is not f64/f32/bf16/f16/fp8/i8/i4",
                    dtype_name(out_dtype));
    if (count == 0) return MFH_OK;
    if (!out || !in) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_convert: NULL buffer");
    hipStream_t s = (hipStream_t)stream;
    mfh_u8* bytes = static_cast<mfh_u8*>(out);
    if (out_dtype == kF8E4M3) return launch_encode_byte<kF8E4M3>(dev, bytes, in, in_dtype, count, s);
    if (out_dtype == kF8E5M2) return launch_encode_byte<kF8E5M2>(dev, bytes, in, in_dtype, count, s);
    if (out_dtype == kInt8) return launch_encode_byte<kInt8>(dev, bytes, in, in_dtype, count, s);
    if (out_dtype == kInt4) return launch_encode_int4(dev, bytes, in, in_dtype, count, s);
    if (out_dtype == kFloat64) return launch_widen_f64(dev, out, in, in_dtype, count, s);
    if (in_dtype == kF8E4M3 || in_dtype == kF8E5M2)
        return by_out<Fp8Launch>(out_dtype, dev, out, in, (int)in_dtype, count, 1.0f, s);
    if (in_dtype == kInt4)
        return by_out<Int4Launch>(out_dtype, dev, out, in, count, (const void*)in, (int)kInvalid,
                                  (int64_t)1 << 62, s);
    return by_out<ConvertLaunch>(out_dtype, dev, out, in, (int)in_dtype, count, s);
}

}  // extern "C"
