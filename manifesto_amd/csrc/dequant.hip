// dequant.hip — FP8 / Int4 dequantisation and dtype conversion for gfx950.
//
// All three are HBM-bound streams.  Each thread moves 16-byte vectors
// (global_load/store_dwordx4) in a grid-stride loop; a scalar tail loop
// finishes counts that are not a multiple of the vector width, and the same
// loop does everything when a pointer is not 16-byte aligned.
//
// FP8: the output for a code depends only on (code, format, scale), so each
// workgroup first builds the 256-entry table in LDS with the exact rules of
// codec.hpp and then every element is one LDS lookup.
#include <cstdlib>

#include "launch.hpp"

namespace mfh {

int blocks_per_cu()
{
    static const int value = [] {
        const char* env = std::getenv("MFH_BLOCKS_PER_CU");
        int v = env ? std::atoi(env) : 0;
        return (v > 0 && v <= 64) ? v : 8;
    }();
    return value;
}

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
MFH_DEV void store_one(void* out, mfh_i64 i, mfh_u32 enc)
{
    if constexpr (OUT == kFloat32) static_cast<mfh_u32*>(out)[i] = enc;
    else static_cast<mfh_u16*>(out)[i] = (mfh_u16)enc;
}

// ---------------------------------------------------------------------------
// FP8 -> {f32, bf16, f16}
// ---------------------------------------------------------------------------

template <int OUT>
__global__ __launch_bounds__(kBlock) void k_dequant_fp8(const mfh_u8* __restrict__ in,
                                                        void* __restrict__ out, mfh_i64 n,
                                                        float scale, int fmt, int vec_ok)
{
    __shared__ mfh_u32 lut[256];
    const mfh_u32 t = threadIdx.x;
    {
        mfh_u32 bits = fmt == kF8E4M3 ? mfh_e4m3_bits(t) : mfh_e5m2_bits(t);
        lut[t] = encode_one<OUT>(mfh_scale_mul(mfh_f32(bits), scale));
    }
    __syncthreads();

    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    const mfh_i64 nvec = vec_ok ? (n >> 4) : 0;
    const u32x4* src = reinterpret_cast<const u32x4*>(in);
    for (mfh_i64 v = (mfh_i64)blockIdx.x * kBlock + t; v < nvec; v += stride) {
        u32x4 w = src[v];
        if constexpr (OUT == kFloat32) {
            u32x4* dst = reinterpret_cast<u32x4*>(out) + 4 * v;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                mfh_u32 x = w[q];
                u32x4 o = {lut[x & 0xffu], lut[(x >> 8) & 0xffu], lut[(x >> 16) & 0xffu], lut[x >> 24]};
                dst[q] = o;
            }
        } else {
            u32x4* dst = reinterpret_cast<u32x4*>(out) + 2 * v;
            mfh_u32 p[8];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                mfh_u32 x = w[q];
                p[2 * q] = lut[x & 0xffu] | (lut[(x >> 8) & 0xffu] << 16);
                p[2 * q + 1] = lut[(x >> 16) & 0xffu] | (lut[x >> 24] << 16);
            }
            u32x4 o0 = {p[0], p[1], p[2], p[3]};
            u32x4 o1 = {p[4], p[5], p[6], p[7]};
            dst[0] = o0;
            dst[1] = o1;
        }
    }
    for (mfh_i64 i = nvec * 16 + (mfh_i64)blockIdx.x * kBlock + t; i < n; i += stride)
        store_one<OUT>(out, i, lut[in[i]]);
}

// ---------------------------------------------------------------------------
// Int4 (+ group scale) -> {f32, bf16, f16}
// ---------------------------------------------------------------------------

template <int SDT>
MFH_DEV float load_scale(const void* scales, mfh_i64 g)
{
    if constexpr (SDT == kFloat32) return static_cast<const float*>(scales)[g];
    else if constexpr (SDT == kFloat16) return mfh_f16_to_f32(static_cast<const mfh_u16*>(scales)[g]);
    else if constexpr (SDT == kBFloat16) return mfh_bf16_to_f32(static_cast<const mfh_u16*>(scales)[g]);
    else return 1.0f;  // plain conversion: no scale
}

MFH_DEV bool finite_f32(float f) { return (mfh_bits(f) & 0x7f800000u) != 0x7f800000u; }

// One 16-byte vector = 32 nibbles = 32 outputs sharing one scale.
template <int OUT>
MFH_DEV void int4_vector(u32x4 w, float s, void* out, mfh_i64 v)
{
    const bool fast = finite_f32(s);  // then no product is NaN
    if constexpr (OUT == kFloat32) {
        u32x4* dst = reinterpret_cast<u32x4*>(out) + 8 * v;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float f[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                float qv = (float)mfh_int4_at(w[q], k);
                f[k] = fast ? qv * s : mfh_scale_mul(qv, s);
            }
            u32x4 a = {mfh_bits(f[0]), mfh_bits(f[1]), mfh_bits(f[2]), mfh_bits(f[3])};
            u32x4 b = {mfh_bits(f[4]), mfh_bits(f[5]), mfh_bits(f[6]), mfh_bits(f[7])};
            dst[2 * q] = a;
            dst[2 * q + 1] = b;
        }
    } else {
        u32x4* dst = reinterpret_cast<u32x4*>(out) + 4 * v;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            mfh_u32 p[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float lo = (float)mfh_int4_at(w[q], 2 * k);
                float hi = (float)mfh_int4_at(w[q], 2 * k + 1);
                if (fast) {
                    lo = lo * s;
                    hi = hi * s;
                } else {
                    lo = mfh_scale_mul(lo, s);
                    hi = mfh_scale_mul(hi, s);
                }
                if constexpr (OUT == kBFloat16) p[k] = mfh_bf16x2_rne(lo, hi);
                else p[k] = mfh_f16_rne(lo) | (mfh_f16_rne(hi) << 16);
            }
            u32x4 o = {p[0], p[1], p[2], p[3]};
            dst[q] = o;
        }
    }
}

template <int OUT, int SDT>
__global__ __launch_bounds__(kBlock) void k_dequant_int4(const mfh_u8* __restrict__ packed,
                                                         const void* __restrict__ scales,
                                                         void* __restrict__ out, mfh_i64 n,
                                                         mfh_i64 group, int vec_ok)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    const mfh_i64 nvec = vec_ok ? (n >> 5) : 0;
    const u32x4* src = reinterpret_cast<const u32x4*>(packed);
    for (mfh_i64 v = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; v < nvec; v += stride) {
        u32x4 w = src[v];
        float s = load_scale<SDT>(scales, (v * 32) / group);
        int4_vector<OUT>(w, s, out, v);
    }
    for (mfh_i64 i = nvec * 32 + (mfh_i64)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
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

// 16-bit storage -> 16-bit storage, eight elements per thread (the cast that
// sits between a bf16/f16 tensor and an f32 fusion in the reference).
template <int IN, int OUT>
__global__ __launch_bounds__(kBlock) void k_convert16_vec(const u32x4* __restrict__ in,
                                                          void* __restrict__ out, mfh_i64 nvec)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    for (mfh_i64 v = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; v < nvec; v += stride) {
        u32x4 w = in[v];
        float f[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            mfh_u32 h = (w[k / 2] >> (16 * (k & 1))) & 0xffffu;
            f[k] = IN == kBFloat16 ? mfh_bf16_to_f32(h) : mfh_f16_to_f32(h);
        }
        if constexpr (OUT == kFloat32) {
            u32x4* dst = reinterpret_cast<u32x4*>(out) + 2 * v;
            u32x4 a = {mfh_bits(f[0]), mfh_bits(f[1]), mfh_bits(f[2]), mfh_bits(f[3])};
            u32x4 b = {mfh_bits(f[4]), mfh_bits(f[5]), mfh_bits(f[6]), mfh_bits(f[7])};
            dst[0] = a;
            dst[1] = b;
        } else {
            mfh_u32 p[4];
#pragma unroll
            for (int k = 0; k < 4; k++)
                p[k] = OUT == kBFloat16 ? mfh_bf16x2_rne(f[2 * k], f[2 * k + 1])
                                        : (mfh_f16_rne(f[2 * k]) | (mfh_f16_rne(f[2 * k + 1]) << 16));
            u32x4 o = {p[0], p[1], p[2], p[3]};
            reinterpret_cast<u32x4*>(out)[v] = o;
        }
    }
}

// f32 -> 16-bit storage, eight elements per thread.
template <int OUT>
__global__ __launch_bounds__(kBlock) void k_narrow_f32_vec(const u32x4* __restrict__ in,
                                                           u32x4* __restrict__ out, mfh_i64 nvec)
{
    const mfh_i64 stride = (mfh_i64)gridDim.x * kBlock;
    for (mfh_i64 v = (mfh_i64)blockIdx.x * kBlock + threadIdx.x; v < nvec; v += stride) {
        u32x4 a = in[2 * v], b = in[2 * v + 1];
        float f[8] = {mfh_f32(a[0]), mfh_f32(a[1]), mfh_f32(a[2]), mfh_f32(a[3]),
                      mfh_f32(b[0]), mfh_f32(b[1]), mfh_f32(b[2]), mfh_f32(b[3])};
        mfh_u32 p[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            p[k] = OUT == kBFloat16 ? mfh_bf16x2_rne(f[2 * k], f[2 * k + 1])
                                    : (mfh_f16_rne(f[2 * k]) | (mfh_f16_rne(f[2 * k + 1]) << 16));
        u32x4 o = {p[0], p[1], p[2], p[3]};
        out[v] = o;
    }
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
        int vec_ok = aligned16(in) && aligned16(out);
        int64_t items = vec_ok ? std::max<int64_t>(n >> 4, 1) : n;
        k_dequant_fp8<OUT><<<grid_for(items, dev), kBlock, 0, stream>>>(
            static_cast<const mfh_u8*>(in), out, n, scale, fmt, vec_ok);
        return launch_status("k_dequant_fp8");
    }
};

template <int OUT>
struct Int4Launch {
    static int run(const Device* dev, void* out, const void* packed, int64_t n, const void* scales,
                   int scale_dt, int64_t group, hipStream_t stream)
    {
        int vec_ok = aligned16(packed) && aligned16(out) && group % 32 == 0;
        int64_t items = vec_ok ? std::max<int64_t>(n >> 5, 1) : n;
        unsigned grid = grid_for(items, dev);
        const mfh_u8* p = static_cast<const mfh_u8*>(packed);
        switch (scale_dt) {
        case kFloat32: k_dequant_int4<OUT, kFloat32><<<grid, kBlock, 0, stream>>>(p, scales, out, n, group, vec_ok); break;
        case kFloat16: k_dequant_int4<OUT, kFloat16><<<grid, kBlock, 0, stream>>>(p, scales, out, n, group, vec_ok); break;
        case kBFloat16: k_dequant_int4<OUT, kBFloat16><<<grid, kBlock, 0, stream>>>(p, scales, out, n, group, vec_ok); break;
        default: k_dequant_int4<OUT, kInvalid><<<grid, kBlock, 0, stream>>>(p, scales, out, n, group, vec_ok); break;
        }
        return launch_status("k_dequant_int4");
    }
};

template <int OUT>
struct ConvertLaunch {
    static int run(const Device* dev, void* out, const void* in, int in_dt, int64_t n, hipStream_t stream)
    {
        if ((in_dt == kBFloat16 || in_dt == kFloat16) && aligned16(in) && aligned16(out) && n % 8 == 0) {
            int64_t nvec = n / 8;
            const u32x4* src = static_cast<const u32x4*>(in);
            unsigned grid = grid_for(nvec, dev);
            if (in_dt == kBFloat16) k_convert16_vec<kBFloat16, OUT><<<grid, kBlock, 0, stream>>>(src, out, nvec);
            else k_convert16_vec<kFloat16, OUT><<<grid, kBlock, 0, stream>>>(src, out, nvec);
            return launch_status("k_convert16_vec");
        }
        if constexpr (OUT != kFloat32) {
            if (in_dt == kFloat32 && aligned16(in) && aligned16(out) && n % 8 == 0) {
                int64_t nvec = n / 8;
                k_narrow_f32_vec<OUT><<<grid_for(nvec, dev), kBlock, 0, stream>>>(
                    static_cast<const u32x4*>(in), static_cast<u32x4*>(out), nvec);
                return launch_status("k_narrow_f32_vec");
            }
        }
        unsigned grid = grid_for(n, dev);
        switch (in_dt) {
#define MFH_CONVERT_CASE(DT) \
    case DT: k_convert<DT, OUT><<<grid, kBlock, 0, stream>>>(in, out, n); break;
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
    if (!is_out_dtype(out_dtype))
        return fail(MFH_ERR_DTYPE_UNSUPPORTED, "mfh_convert: output dtype %s is not f32/bf16/f16", dtype_name(out_dtype));
    if (count == 0) return MFH_OK;
    if (!out || !in) return fail(MFH_ERR_INVALID_ARGUMENT, "mfh_convert: NULL buffer");
    hipStream_t s = (hipStream_t)stream;
    if (in_dtype == kF8E4M3 || in_dtype == kF8E5M2)
        return by_out<Fp8Launch>(out_dtype, dev, out, in, (int)in_dtype, count, 1.0f, s);
    if (in_dtype == kInt4)
        return by_out<Int4Launch>(out_dtype, dev, out, in, count, (const void*)in, (int)kInvalid,
                                  (int64_t)1 << 62, s);
    return by_out<ConvertLaunch>(out_dtype, dev, out, in, (int)in_dtype, count, s);
}

}  // extern "C"
