// codec.hpp — bit-exact dtype codecs for gfx950 device code.
//
// Shared by the ahead-of-time kernels and, as text, by the prelude of every
// JIT-compiled fused kernel, so it uses no includes and no std types.
//
// Each function reproduces the bit rules of manifesto's Go codecs:
//   F8E4M3.Float32   dtype/fp8.go:39-70
//   F8E5M2.Float32   dtype/fp8.go:149-183
//   NewF8E4M3FromFloat32 / NewF8E5M2FromFloat32  dtype/fp8.go:77-136,190-249
//   NewBfloat16FromFloat32  dtype/bfloat16.go:41-55
//   f16bitsToF32bits / f32bitsToF16bits  dtype/float16.go:222-315
//   int4 nibbles     dtype/convert/decoders.go:262-289
// The 16-bit conversions are single gfx950 instructions: v_cvt_pk_bf16_f32,
// v_cvt_pk_f16_f32 / v_cvt_f16_f32 and v_cvt_f32_f16.  Their results equal
// the Go rules bit for bit on every input, NaN payloads and denormals
// included (checked over all 2^32 f32 and all 2^16 f16 inputs on MI355X;
// tests/test_gpu_dequant.py keeps that check), so no fix-up code is needed.
// FP8 encode runs through v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 between an
// input map and a NaN fix-up that make its codes the reference's.
#ifndef MFH_CODEC_HPP
#define MFH_CODEC_HPP

typedef unsigned char mfh_u8;
typedef unsigned short mfh_u16;
typedef unsigned int mfh_u32;
typedef int mfh_i32;
typedef long long mfh_i64;
typedef unsigned long long mfh_u64;
typedef float mfh_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 mfh_bf16x2 __attribute__((ext_vector_type(2)));

#define MFH_DEV __device__ inline __attribute__((always_inline))

MFH_DEV float mfh_f32(mfh_u32 u) { return __builtin_bit_cast(float, u); }
MFH_DEV mfh_u32 mfh_bits(float f) { return __builtin_bit_cast(mfh_u32, f); }
MFH_DEV bool mfh_isnan(float f) { return (mfh_bits(f) & 0x7fffffffu) > 0x7f800000u; }

// ---- FP8 -> f32 bits ------------------------------------------------------

// E4M3: S.1111.111 is NaN (sign kept, canonical quiet payload), no Inf;
// subnormal m*2^-9 is renormalised (the Go loop shifts until bit 3 is set).
MFH_DEV mfh_u32 mfh_e4m3_bits(mfh_u32 code)
{
    mfh_u32 sign = (code & 0x80u) << 24;
    mfh_u32 mag = code & 0x7fu;
    mfh_u32 e = mag >> 3, m = mag & 7u;
    if (e == 0u) {
        mfh_u32 shift = (mfh_u32)__builtin_clz(m | 1u) - 28u;  // 1->3, 2..3->2, 4..7->1
        m = (m << shift) & 7u;
        e = 1u - shift;                                         // wraps like the Go uint32
    }
    mfh_u32 normal = sign | ((e + 120u) << 23) | (m << 20);
    mfh_u32 out = mag == 0u ? sign : normal;
    return mag == 0x7fu ? (sign | 0x7fc00000u) : out;
}

// E5M2: exponent 31 is Inf (m == 0) or a quiet NaN carrying m at bit 21.
MFH_DEV mfh_u32 mfh_e5m2_bits(mfh_u32 code)
{
    mfh_u32 sign = (code & 0x80u) << 24;
    mfh_u32 e = (code >> 2) & 0x1fu, m = code & 3u;
    if (e == 0x1fu) return sign | (m == 0u ? 0x7f800000u : (0x7fc00000u | (m << 21)));
    if (e == 0u) {
        if (m == 0u) return sign;
        mfh_u32 shift = (mfh_u32)__builtin_clz(m) - 29u;  // 1->2, 2..3->1
        m = (m << shift) & 3u;
        e = 1u - shift;
    }
    return sign | ((e + 112u) << 23) | (m << 21);
}

// ---- f32 -> FP8 ---------------------------------------------------------------

// NewF8E4M3FromFloat32 / NewF8E5M2FromFloat32 (dtype/fp8.go:77-136,190-249):
// saturating round-to-nearest-even with the reference's exact case split,
// whose results are kept as they are:
//   * NaN -> 0x7f whatever its sign;
//   * above the largest finite value (448 / 57344) and Inf -> 0x7e/0xfe
//     (E4M3) or +-Inf 0x7c/0xfc (E5M2);
//   * a value whose biased exponent reaches the top field value (E4M3
//     [256, 448], E5M2 none below 57344) saturates the same way;
//   * below the smallest normal the mantissa with its hidden bit is shifted
//     right by (mantissa bits + 20 - e) resp. (21 - e) for biased e <= 0 and
//     rounded; a result that reaches the hidden-bit position becomes the
//     smallest normal (so E4M3 [2^-7, 2^-6) all give 0x08); biased e below
//     -3 (E4M3) / -1 (E5M2) gives signed zero.
//
// gfx950's v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 encode two f32 values into
// OCP E4M3 / E5M2 with round-to-nearest-even.  Outside NaN they give the
// reference's code for every input once the input is first moved to a value
// whose hardware code is the reference's (mfh_fp8_prep; checked over all
// 2^32 f32 inputs on MI355X, and tests/test_gpu_encode.py keeps the check):
//   * |x| below 2^-10 (E4M3) / 2^-16 (E5M2) -> 0: there the reference's
//     shifted mantissa rounds to zero, where the hardware would round the top
//     of the range up to the smallest subnormal;
//   * |x| below the smallest normal 2^-6 / 2^-14 -> min(2|x|, smallest
//     normal): the reference's subnormal shift is one bit short, so its code
//     for |x| is the IEEE code of 2|x|, and whatever reaches the normal range
//     stops at the smallest normal's code 0x08 / 0x04;
//   * |x| >= 248 (E4M3: what rounds into the top binade) or > 57344 (E5M2),
//     Inf included -> 448 / Inf, whose codes are the saturation codes
//     0x7e / 0x7c;
//   * the sign is put back; NaN passes through.
// The hardware writes every NaN as 0xff (E4M3) / 0xfe (E5M2), bytes that no
// other input gives, and mfh_fp8_nan_fix turns them into 0x7f.
template <bool E5>
MFH_DEV float mfh_fp8_prep(float v)
{
    constexpr mfh_u32 kZero = E5 ? 0x37800000u : 0x3a800000u;  // 2^-16 / 2^-10
    constexpr mfh_u32 kMinN = E5 ? 0x38800000u : 0x3c800000u;  // 2^-14 / 2^-6
    constexpr float kSatAt = E5 ? 57344.0f : 248.0f;
    constexpr mfh_u32 kSatTo = E5 ? 0x7f800000u : 0x43e00000u;  // Inf / 448
    const mfh_u32 u = mfh_bits(v);
    const mfh_u32 a = u & 0x7fffffffu;
    // 2|x| is a + 1 << 23 for the normal |x| that get here; the median of
    // a, 2a and the smallest normal is min(2a, smallest normal) below it and
    // a from it on (a NaN's a stays the median)
    const mfh_u32 d = a + 0x00800000u;
    const mfh_u32 lo = d < kMinN ? d : kMinN;
    mfh_u32 m = a > lo ? a : lo;
    m = a < kZero ? 0u : m;
    const float af = mfh_f32(a);
    m = (E5 ? af > kSatAt : af >= kSatAt) ? kSatTo : m;  // false for NaN
    return mfh_f32(m | (u & 0x80000000u));
}

// The hardware's NaN bytes of a word of codes -> 0x7f.  E4M3: a byte whose
// low 7 bits are all set is 0xff from a NaN (0x7f is never produced);
// E5M2: a byte whose low 7 bits are 0x7d..0x7f is 0xfe from a NaN.
template <bool E5>
MFH_DEV mfh_u32 mfh_fp8_nan_fix(mfh_u32 w)
{
    const mfh_u32 hit = ((w & 0x7f7f7f7fu) + (E5 ? 0x03030303u : 0x01010101u)) & 0x80808080u;
    if constexpr (E5) return (w | (hit >> 7)) & ~hit;  // 0xfe -> 0x7f
    else return w & ~hit;                              // 0xff -> 0x7f
}

// Four values -> four codes, value k in byte k.
template <bool E5>
MFH_DEV mfh_u32 mfh_fp8x4_encode(float v0, float v1, float v2, float v3)
{
    mfh_u32 w;
    if constexpr (E5) {
        w = (mfh_u32)__builtin_amdgcn_cvt_pk_bf8_f32(mfh_fp8_prep<true>(v0), mfh_fp8_prep<true>(v1), 0, false);
        w = (mfh_u32)__builtin_amdgcn_cvt_pk_bf8_f32(mfh_fp8_prep<true>(v2), mfh_fp8_prep<true>(v3), (int)w, true);
    } else {
        w = (mfh_u32)__builtin_amdgcn_cvt_pk_fp8_f32(mfh_fp8_prep<false>(v0), mfh_fp8_prep<false>(v1), 0, false);
        w = (mfh_u32)__builtin_amdgcn_cvt_pk_fp8_f32(mfh_fp8_prep<false>(v2), mfh_fp8_prep<false>(v3), (int)w, true);
    }
    return mfh_fp8_nan_fix<E5>(w);
}

// One value -> its code.
template <bool E5>
MFH_DEV mfh_u32 mfh_fp8_encode(float v)
{
    mfh_u32 w;
    if constexpr (E5) w = (mfh_u32)__builtin_amdgcn_cvt_pk_bf8_f32(mfh_fp8_prep<true>(v), 0.0f, 0, false);
    else w = (mfh_u32)__builtin_amdgcn_cvt_pk_fp8_f32(mfh_fp8_prep<false>(v), 0.0f, 0, false);
    return mfh_fp8_nan_fix<E5>(w) & 0xffu;
}

MFH_DEV mfh_u32 mfh_e4m3_encode(float v) { return mfh_fp8_encode<false>(v); }
MFH_DEV mfh_u32 mfh_e5m2_encode(float v) { return mfh_fp8_encode<true>(v); }

// ---- BF16 -------------------------------------------------------------------

MFH_DEV float mfh_bf16_to_f32(mfh_u32 h) { return mfh_f32(h << 16); }

// The Go rule in integer form (dtype/bfloat16.go:41-55): NaN -> top half |
// 0x0040, else RNE via + 0x7fff + the kept LSB.  Host-side statement of what
// v_cvt_pk_bf16_f32 computes.
MFH_DEV mfh_u32 mfh_bf16_rne_sw(float v)
{
    mfh_u32 b = mfh_bits(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x0040u;
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

typedef _Float16 mfh_f16x2 __attribute__((ext_vector_type(2)));

// Two values -> packed bf16x2 (lo in bits 0..15), v_cvt_pk_bf16_f32.
MFH_DEV mfh_u32 mfh_bf16x2_rne(float lo, float hi)
{
    mfh_f32x2 v = {lo, hi};
    return __builtin_bit_cast(mfh_u32, __builtin_convertvector(v, mfh_bf16x2));
}

MFH_DEV mfh_u32 mfh_bf16_rne(float v) { return mfh_bf16x2_rne(v, 0.0f) & 0xffffu; }

// ---- F16 --------------------------------------------------------------------

// f16bitsToF32bits: exact widening, a NaN becomes sign | 0x7fc00000 |
// payload << 13 (v_cvt_f32_f16).
MFH_DEV float mfh_f16_to_f32(mfh_u32 h) { return (float)__builtin_bit_cast(_Float16, (mfh_u16)h); }

// f32bitsToF16bits: RNE with overflow to Inf, NaN -> sign | 0x7e00 |
// payload >> 13 (v_cvt_f16_f32).
MFH_DEV mfh_u32 mfh_f16_rne(float v) { return (mfh_u32)__builtin_bit_cast(mfh_u16, (_Float16)v); }

// Two values -> packed f16x2 (lo in bits 0..15), v_cvt_pk_f16_f32.
MFH_DEV mfh_u32 mfh_f16x2_rne(float lo, float hi)
{
    mfh_f32x2 v = {lo, hi};
    return __builtin_bit_cast(mfh_u32, __builtin_convertvector(v, mfh_f16x2));
}

// ---- Int4 -------------------------------------------------------------------

// Nibble k (0..7) of a 32-bit word, sign-extended: element 2j is the low
// nibble of byte j.
MFH_DEV mfh_i32 mfh_int4_at(mfh_u32 word, mfh_u32 k)
{
    return __builtin_amdgcn_sbfe((mfh_i32)word, k * 4u, 4u);
}

// ---- scale multiply -----------------------------------------------------------

// One IEEE multiply with the NaN rules of an x86 mulss(decoded, scale) made
// explicit, so the result never depends on which NaN the hardware forwards:
// a NaN operand comes back quieted (the decoded value first) and Inf * 0 is
// the x86 default NaN 0xffc00000.  Branch-free.
MFH_DEV float mfh_scale_mul(float decoded, float scale)
{
    mfh_u32 d = mfh_bits(decoded), s = mfh_bits(scale);
    mfh_u32 da = d & 0x7fffffffu, sa = s & 0x7fffffffu;
    mfh_u32 r = mfh_bits(decoded * scale);
    r = ((da == 0x7f800000u && sa == 0u) || (da == 0u && sa == 0x7f800000u)) ? 0xffc00000u : r;
    r = sa > 0x7f800000u ? (s | 0x00400000u) : r;
    r = da > 0x7f800000u ? (d | 0x00400000u) : r;
    return mfh_f32(r);
}

#endif  // MFH_CODEC_HPP
