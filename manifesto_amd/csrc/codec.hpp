// codec.hpp — bit-exact dtype codecs for gfx950 device code.
//
// Shared by the ahead-of-time kernels and, as text, by the prelude of every
// JIT-compiled fused kernel, so it uses no includes and no std types.
//
// Each function reproduces the bit rules of manifesto's Go codecs:
//   F8E4M3.Float32   dtype/fp8.go:39-70
//   F8E5M2.Float32   dtype/fp8.go:149-183
//   NewBfloat16FromFloat32  dtype/bfloat16.go:41-55
//   f16bitsToF32bits / f32bitsToF16bits  dtype/float16.go:222-315
//   int4 nibbles     dtype/convert/decoders.go:262-289
// The 16-bit conversions are single gfx950 instructions: v_cvt_pk_bf16_f32,
// v_cvt_pk_f16_f32 / v_cvt_f16_f32 and v_cvt_f32_f16.  Their results equal
// the Go rules bit for bit on every input, NaN payloads and denormals
// included (checked over all 2^32 f32 and all 2^16 f16 inputs on MI355X;
// tests/test_gpu_dequant.py keeps that check), so no fix-up code is needed.
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
// MB = mantissa bits, BIAS = exponent bias, EMAX = top exponent field value,
// SAT = saturation code, MAXF = bits of the largest finite value.
template <int MB, int BIAS, int EMAX, int MINSUB, mfh_u32 SAT, mfh_u32 MAXF>
MFH_DEV mfh_u32 mfh_fp8_encode(float value)
{
    // The same cases, computed for every element without a branch (the
    // per-case branches of a direct transcription diverge within a wave):
    constexpr mfh_u32 drop = 23 - MB;                  // 20 (E4M3) or 21 (E5M2)
    constexpr mfh_u32 kNormal = (128u - BIAS) << 23;   // |x| from here on has biased e >= 1
    const mfh_u32 u = mfh_bits(value);
    const mfh_u32 a = u & 0x7fffffffu;
    // e >= 1: the exponent and top MB mantissa bits rounded to nearest even
    // by one integer add; a carry out of the mantissa bumps the exponent,
    // which is the reference's "m >= 1 << MB: m = 0, e++" step
    const mfh_u32 r = a + ((1u << (drop - 1u)) - 1u) + ((a >> drop) & 1u);
    const mfh_u32 normal = (r >> drop) - ((127u - BIAS) << MB);
    // e <= 0: the hidden-bit mantissa shifted right by drop - e and rounded
    // to nearest even is |x| * 2^(BIAS + MB) rounded to an integer (exact
    // scaling, then the 2^23 round-to-integer add); below biased e = MINSUB
    // zero; a result reaching 1 << MB stays there
    constexpr float kScale = (float)(1u << (BIAS + MB));
    constexpr float kZeroBelow = MINSUB + MB >= 0 ? (float)(1u << (MINSUB + MB >= 0 ? MINSUB + MB : 0))
                                                  : 1.0f / (float)(1u << (MINSUB + MB < 0 ? -(MINSUB + MB) : 0));
    const float y = mfh_f32(a) * kScale;
    const mfh_u32 t = mfh_bits((y < kZeroBelow ? 0.0f : y) + 8388608.0f) - 0x4b000000u;
    const mfh_u32 sub = t < (1u << MB) ? t : (1u << MB);
    mfh_u32 code = a < kNormal ? sub : normal;
    // above the largest finite value, Inf, and a rounded biased exponent at
    // the top field value saturate
    code = (a > MAXF || r >= ((mfh_u32)(EMAX + 127 - BIAS) << 23)) ? SAT : code;
    code |= (u >> 24) & 0x80u;
    return a > 0x7f800000u ? 0x7fu : code;             // NaN, whatever its sign
}

MFH_DEV mfh_u32 mfh_e4m3_encode(float v) { return mfh_fp8_encode<3, 7, 15, -3, 0x7eu, 0x43e00000u>(v); }
MFH_DEV mfh_u32 mfh_e5m2_encode(float v) { return mfh_fp8_encode<2, 15, 31, -1, 0x7cu, 0x47600000u>(v); }

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
