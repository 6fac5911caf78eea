// devmath.hpp — the activation math of fused chains, for gfx950.
//
// Like codec.hpp this file is also the text prelude of every JIT-compiled
// fused kernel, so it uses no includes.  It compiles for the host as well
// (MFH_HOST_MATH), which lets the CPU tests measure its accuracy.
//
// Reference semantics (codegen/cpu.go:186-200): Sigmoid, Silu and Gelu are
// evaluated in f64 and rounded once to f32.  The fast forms below compute in
// f32 with error-free corrections and stay within 2 f32 ulps of that; the
// reference forms (mfh_*_ref) restate the f64 formulas, and the
// rounding-tested forms (mfh_*_cr) give their results at lower cost.
//
//   e^a:          a log2(e) = k + f, |f| <= 1/2, with k from the
//                 round-to-integer constant 1.5 * 2^23 and f formed with
//                 log2(e) split into two f32 parts; 2^f by the hardware
//                 v_exp_f32 and 2^k added into the result's exponent field
//                 (silu: within budget over every f32 input, checked on the
//                 GPU).
//   2^f:          for |f| <= 1/2 the hardware v_exp_f32 where the argument
//                 is formed and reduced in f64 (gelu: within budget over
//                 every f32 input, checked on the GPU), or a degree-8 f64
//                 polynomial (sigmoid, gen_exp_poly.py).
//   n * sigmoid(z) = n / (1 + E), E = e^-z, with z clamped (v_med3) to a
//                 range where E is a normal f32 and 1 + E is formed
//                 without a rounding tie, and the quotient corrected by one
//                 residual step.  Arguments outside that range (where the
//                 result underflows, the reference cancels, or the result
//                 is v itself) and NaN take the f64 reference form, a
//                 branch no wave enters for normal data.
//
// Cost on gfx950 (measured issue rates, in units of one f32 FMA): f32
// add/mul/fma 1; conversions, ldexp, rndne, med3, min/max, compares and
// selects ~1.5; f64 add/mul ~1.7; f64 fma 2; v_rcp_f32 3.3; v_rcp_f64 6.
// Plain f32 arithmetic is what is cheap, so the kernels reduce in f32 where
// the argument allows and use f64 only to form an argument that f32 cannot
// hold precisely enough (gelu's cubic).
#ifndef MFH_DEVMATH_HPP
#define MFH_DEVMATH_HPP

#ifdef MFH_HOST_MATH
#include <cmath>
#define MFH_MATH inline
#define MFH_RARE inline
#define mfh_fmaf(a, b, c) std::fma((float)(a), (float)(b), (float)(c))
#define mfh_fma(a, b, c) std::fma((double)(a), (double)(b), (double)(c))
#define mfh_rintf(x) std::nearbyint((float)(x))
#define mfh_rint(x) std::nearbyint((double)(x))
#define mfh_ldexpf(x, k) std::ldexp((float)(x), (int)(k))
#define mfh_ldexp(x, k) std::ldexp((double)(x), (int)(k))
#define mfh_rcpf(x) (1.0f / (float)(x))
#define mfh_rcp(x) (1.0 / (double)(x))
// Host stand-in for the hardware 2^x (v_exp_f32): libm's exp2f, which is more
// accurate, so the host sweep does not model gelu's device error; the GPU
// tests check the device gelu over every f32 input instead.
#define mfh_exp2f_hw(x) std::exp2((float)(x))
#define mfh_tanh_f64(x) std::tanh((double)(x))
#define mfh_exp_f64(x) std::exp((double)(x))
#define mfh_log_f64(x) std::log((double)(x))
#define mfh_sqrtf(x) std::sqrt((float)(x))
#define MFH_KEEP(x) ((void)0)
#define mfh_med3f(x, lo, hi) std::fmin(std::fmax((float)(x), (float)(lo)), (float)(hi))
#define mfh_absf(x) std::fabs((float)(x))
#define mfh_maxf(a, b) std::fmax((float)(a), (float)(b))
#define mfh_minf(a, b) std::fmin((float)(a), (float)(b))
#define mfh_is_nan_or_inf_class(v) (std::isnan(v) || std::isinf(v))
inline unsigned mfh_fbits(float f) { unsigned u; __builtin_memcpy(&u, &f, 4); return u; }
inline float mfh_fromfbits(unsigned u) { float f; __builtin_memcpy(&f, &u, 4); return f; }
inline int mfh_low_int(double d) { unsigned long long u; __builtin_memcpy(&u, &d, 8); return (int)(unsigned)u; }
#else
extern "C" __device__ double __ocml_tanh_f64(double);
extern "C" __device__ double __ocml_exp_f64(double);
extern "C" __device__ double __ocml_log_f64(double);
#define MFH_MATH __device__ inline __attribute__((always_inline))
// The reference forms behind the fast ones' rare branches are real calls: the
// constants of the f64 tanh / exp they inline were otherwise hoisted into
// every thread's prologue (about 3 VALU instructions per element of a
// one-item-per-thread launch) although no wave takes the branch.
#define MFH_RARE __device__ __attribute__((noinline))
#define mfh_fmaf(a, b, c) __builtin_fmaf((a), (b), (c))
#define mfh_fma(a, b, c) __builtin_fma((a), (b), (c))
#define mfh_rintf(x) __builtin_rintf(x)
#define mfh_rint(x) __builtin_rint(x)
#define mfh_ldexpf(x, k) __builtin_amdgcn_ldexpf((x), (k))
#define mfh_ldexp(x, k) __builtin_amdgcn_ldexp((x), (k))
#define mfh_rcpf(x) __builtin_amdgcn_rcpf(x)
#define mfh_rcp(x) __builtin_amdgcn_rcp(x)
#define mfh_exp2f_hw(x) __builtin_amdgcn_exp2f(x)
#define mfh_tanh_f64(x) __ocml_tanh_f64(x)
#define mfh_exp_f64(x) __ocml_exp_f64(x)
#define mfh_log_f64(x) __ocml_log_f64(x)
#define mfh_sqrtf(x) __builtin_sqrtf(x)
// Pins a value in a VGPR at this point: keeps LLVM from sinking the whole
// computation of x into a divergent branch around a cheap special-case
// select (which serialises the unrolled elements).  Emits no instruction.
#define MFH_KEEP(x) __asm__ volatile("" : "+v"(x))
#define mfh_med3f(x, lo, hi) __builtin_amdgcn_fmed3f((x), (lo), (hi))
// |x| is a source modifier on gfx950 (no instruction of its own).
#define mfh_absf(x) __builtin_fabsf(x)
#define mfh_maxf(a, b) __builtin_fmaxf((a), (b))
#define mfh_minf(a, b) __builtin_fminf((a), (b))
__device__ inline unsigned mfh_fbits(float f) { return __builtin_bit_cast(unsigned, f); }
__device__ inline float mfh_fromfbits(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ inline int mfh_low_int(double d) { return (int)(unsigned)__builtin_bit_cast(unsigned long long, d); }
#endif

#define MFH_LOG2E_F 1.44269502162933349609375f         // 0x3fb8aa3b
#define MFH_LOG2E_LO_F 1.925963033500011e-08f           // 0x32a57060 = fl32(log2(e) - MFH_LOG2E_F)
#define MFH_ROUND_INT_F 12582912.0f                     // 1.5 * 2^23
#define MFH_LOG2E_D 1.4426950408889634                  // 0x3ff71547652b82fe
#define MFH_LN2_D 0.6931471805599453                    // 0x3fe62e42fefa39ef
#define MFH_SQRT_2_OVER_PI_D 0.7978845608028654         // 0x3fe9884533d43651 = sqrt(fl64(2/pi))
#define MFH_GELU_A_D 0.044715                           // 0x3fa6e4e26d4801f7

// 2^f for |f| <= 1/2 in f64: degree 8, relative error below 2^-39.9 with
// Horner rounding (the f64 fit of gen_exp_poly.py).
MFH_MATH double mfh_exp2_poly_d(double f)
{
    double q = 0x1.6208e89aaa738p-20;
    q = mfh_fma(q, f, 0x1.00daa1a549b84p-16);
    q = mfh_fma(q, f, 0x1.430a636ccd334p-13);
    q = mfh_fma(q, f, 0x1.5d87488d46abap-10);
    q = mfh_fma(q, f, 0x1.3b2ab618fb075p-7);
    q = mfh_fma(q, f, 0x1.c6b08dd4189f3p-5);
    q = mfh_fma(q, f, 0x1.ebfbdff8ccfeap-3);
    q = mfh_fma(q, f, 0x1.62e42fef863fep-1);
    return mfh_fma(q, f, 1.0);
}

// e^-m for m in [-87, 87]: -m log2(e) = k + f, |f| <= 1/2.  fma(m, -L, C)
// with C = 1.5 * 2^23 rounds -m L to the integer k and holds it in its low
// mantissa bits; f = -m L - k is formed by one fma (exact product, one
// rounding) and corrected by the tail of log2(e), so its error is a few
// 2^-26; 2^f is v_exp_f32; 2^k goes straight into the exponent field, which
// (bits(C + k) << 23) does modulo 2^32 because C's low nine bits are zero.
// The result stays a normal f32 (exponent field 1..253) over the range.
MFH_MATH float mfh_exp_neg(float m)
{
    const float kb = mfh_fmaf(m, -MFH_LOG2E_F, MFH_ROUND_INT_F);
    float f = mfh_fmaf(m, -MFH_LOG2E_F, -(kb - MFH_ROUND_INT_F));
    f = mfh_fmaf(m, -MFH_LOG2E_LO_F, f);
    return mfh_fromfbits(mfh_fbits(mfh_exp2f_hw(f)) + (mfh_fbits(kb) << 23));
}

// n / (1 + e): d = fl(1 + e), then one residual step corrects the quotient
// for the reciprocal's error.  The rounding of d is left in (at most half an
// ulp of the quotient), which the 2-ulp Silu and Gelu budgets allow as long
// as 1 + e is not a rounding tie: every e in [2^24, 2^25) makes it one, so
// callers keep e below 2^24.
MFH_MATH float mfh_div_one_plus(float n, float e)
{
    float d = 1.0f + e;
    float r = mfh_rcpf(d);
    float q = n * r;
    float res = mfh_fmaf(-q, d, n);
    return mfh_fmaf(res, r, q);
}

MFH_MATH bool mfh_is_inf(float v) { return (mfh_fbits(v) & 0x7fffffffu) == 0x7f800000u; }
MFH_MATH bool mfh_is_nan(float v) { return (mfh_fbits(v) & 0x7fffffffu) > 0x7f800000u; }

// Reference forms (codegen/cpu.go:186-200), f64 then one rounding.
MFH_MATH float mfh_sigmoid_ref(float v) { return (float)(1.0 / (1.0 + mfh_exp_f64(-(double)v))); }
MFH_MATH float mfh_silu_ref(float v) { return (float)((double)v / (1.0 + mfh_exp_f64(-(double)v))); }

// gelu in the reference's f64 form 0.5 v (1 + tanh(inner)), with
// s = e^(-2 inner) and y = 2 / (s + 1).  For inner <= -0.625 tanh is
// -(1 - y), the form in which Go's math.Tanh (and glibc's) evaluates it there
// (s = e^(2|inner|)), and 1 + tanh is formed as 1 - (1 - y) with the same f64
// roundings, because in that range 1 + tanh cancels and its result carries
// the f64 quantum of exactly that expression.  Above it 1 + tanh(inner) = y
// exactly, and y is faithful (one f64 exp, one division), so the f32 result is
// that of any faithful f64 tanh but for f64 rounding ties.  One exp and one
// division serve both ranges: a third of the instructions of an f64 tanh,
// whose double-word steps the fast forms' flagged elements would otherwise
// pay for.
MFH_MATH float mfh_gelu_ref(float v)
{
    const double d = (double)v;
    const double inner = MFH_SQRT_2_OVER_PI_D * (d + MFH_GELU_A_D * d * d * d);
    const double y = 2.0 / (mfh_exp_f64(-2.0 * inner) + 1.0);
    const double one_plus_th = inner > -0.625 ? y : 1.0 - (1.0 - y);
    return (float)(0.5 * d * one_plus_th);
}

// Each fast activation comes in two parts: mfh_<name>_fast(v, rare) is
// branch-free and sets `rare` for the inputs it does not cover, and
// mfh_<name>(v) returns the reference form for those and the fast value for
// all others.  Generated kernels call the fast forms for every element of an
// item and then recompute the flagged elements through mfh_<name>, so the
// results are the same and the item's main body has no branch.
//
// Ranges are reduced by the round-to-integer constant C = 1.5 * 2^52:
// fma(a, b, C) = C + rint(a b) for |a b| < 2^51, whose low word is that
// integer as an int32, and fma(a, b, -(that - C)) is the remainder rounded
// once; three f64 operations where rint, a subtraction and an integer
// conversion took four (f64 runs at half the f32 rate on gfx950).
#define MFH_ROUND_INT_D 6755399441055744.0  // 1.5 * 2^52

// 1 + 2^t in f64 for |t| < 2^31, by the round-to-integer reduction and the
// degree-8 polynomial (2^-39.9).
MFH_MATH double mfh_one_plus_2exp(double t)
{
    const double tk = t + MFH_ROUND_INT_D;
    const double kd = tk - MFH_ROUND_INT_D;
    return 1.0 + mfh_ldexp(mfh_exp2_poly_d(t - kd), mfh_low_int(tk));
}

// 1 / den: the hardware reciprocal and one Newton step.
MFH_MATH double mfh_recip_newton(double den)
{
    const double r = mfh_rcp(den);
    return mfh_fma(r, mfh_fma(-den, r, 1.0), r);
}

// sigmoid(v) = 1 / (1 + 2^t), t = -v log2(e), all in f64: for v < 0 the
// result is ~e^v and inherits the full relative error of E, which an f32
// exponential (0.9 ulp) plus the final rounding would push past the 1-ulp
// Sigmoid budget on a few inputs.  In f64 (2^f to 2^-39.9, reciprocal plus one
// Newton step) the single rounding to f32 is the only error that matters.
// Below -708 (and -Inf, NaN) the reference's form; +Inf gives 1 by itself.
// mfh_sigmoid_z is that f64 value (and sets den = 1 + E).
MFH_MATH double mfh_sigmoid_z(float v, double& den)
{
    const double x = (double)mfh_med3f(v, -708.0f, 800.0f);
    const double tk = mfh_fma(x, -MFH_LOG2E_D, MFH_ROUND_INT_D);
    const double kd = tk - MFH_ROUND_INT_D;
    den = 1.0 + mfh_ldexp(mfh_exp2_poly_d(mfh_fma(x, -MFH_LOG2E_D, -kd)), mfh_low_int(tk));
    return mfh_recip_newton(den);
}

MFH_MATH float mfh_sigmoid_fast(float v, bool& rare)
{
    double den;
    const double z = mfh_sigmoid_z(v, den);
    rare |= !(v >= -708.0f);
    return (float)z;
}

// silu(v) = v / (1 + e^-v).  One clamp to [-16.5, 87] serves the
// computation and the rare test: every v it changes takes the f64 form, i.e.
// v < -16.5 (and -Inf), where e^-v reaches 2^24 and 1 + e^-v would be a
// rounding tie (those inputs reached 3 ulps), NaN, and v > 87 (+Inf
// included), where the result is v itself (the quotient's residual step
// would turn +Inf into NaN).  Within 2 f32 ulps of the reference over every
// f32 input (measured on the device).  The SwiGLU kernel's main body
// (decode, silu, multiply, pack) takes 16 VALU instructions per element this
// way, against 28 with a polynomial e^-v and an exact tail of 1 + e^-v, which
// kept it within 70% of the HBM roofline only once the clock had settled.
MFH_MATH float mfh_silu_fast(float v, bool& rare)
{
    const float m = mfh_med3f(v, -16.5f, 87.0f);
    rare |= m != v;
    return mfh_div_one_plus(v, mfh_exp_neg(m));
}

// silu in f64 for the rounding-tested form below (chains that stream f32,
// whose results show every f32 ulp of the node, and MFH_FUSION_PRECISE), as
// the fast sigmoid makes it: e^-v = 2^t by the round-to-integer reduction and
// the degree-8 polynomial (2^-39.9), the reciprocal of 1 + e^-v plus one
// Newton step, times v.  mfh_silu_z is that f64 value for m = v inside the
// clamp [-708, 800], and sets den = 1 + e^-v.
MFH_MATH double mfh_silu_z(float m, double& den)
{
    const double x = (double)m;
    den = mfh_one_plus_2exp(x * -MFH_LOG2E_D);
    return x * mfh_recip_newton(den);
}

// Fast gelu = v / (1 + E), E = e^(-2 inner) = 2^t with
// t = -2 inner log2(e) = d w, w = KA + KB d^2, formed and reduced in f64 (the
// cubic needs more than f32's 24 bits where E is large) and 2^f, |f| <= 1/2,
// evaluated by the hardware v_exp_f32 (one instruction for the polynomial's
// six; measured on MI355X: the gelu chain +2-3%).  Within 2 f32 ulps of the
// reference over every f32 input (measured on the device: 96.4% identical,
// the same as with the polynomial).  One clamp
// to [-4.9, 1024] serves the computation and the rare test: every v it
// changes takes the reference form, i.e. v < -4.9 (inner < -9.3), where the
// reference's 1 + tanh cancels in f64, NaN, and v > 1024 (+Inf included).
// Inside the clamp |t| < 1.2e8, so k fits the int32 of the round-to-integer
// trick, and above v = 14 E underflows to 0 and the result is v, as the
// reference's tanh is exactly 1 there.
#define MFH_GELU_KA (-2.0 * MFH_SQRT_2_OVER_PI_D * MFH_LOG2E_D)
#define MFH_GELU_KB (-2.0 * MFH_SQRT_2_OVER_PI_D * MFH_GELU_A_D * MFH_LOG2E_D)
MFH_MATH float mfh_gelu_e(float c)
{
    const double d = (double)c;
    const double w = mfh_fma(d * d, MFH_GELU_KB, MFH_GELU_KA);
    const double tk = mfh_fma(w, d, MFH_ROUND_INT_D);
    const double kd = tk - MFH_ROUND_INT_D;
    const float p = mfh_exp2f_hw((float)mfh_fma(w, d, -kd));
    return mfh_ldexpf(p, mfh_low_int(tk));
}

MFH_MATH float mfh_gelu_fast(float v, bool& rare)
{
    const float c = mfh_med3f(v, -4.9f, 1024.0f);
    rare |= c != v;
    return mfh_div_one_plus(v, mfh_gelu_e(c));
}

// gelu in f64 for the rounding-tested form below: the same argument t = d w
// in f64, then 2^t, the quotient and the product with v in f64 as
// mfh_silu_z makes them.  mfh_gelu_z is that f64 value for c inside the fast
// form's clamp, and sets den = 1 + E.
MFH_MATH double mfh_gelu_z(float c, double& den)
{
    const double d = (double)c;
    den = mfh_one_plus_2exp(mfh_fma(d * d, MFH_GELU_KB, MFH_GELU_KA) * d);
    return d * mfh_recip_newton(den);
}

// Rounding-tested forms (chains that stream f32, MFH_FUSION_PRECISE kernels,
// and the recomputation of flagged elements below): mfh_<name>_cr(v, rare)
// returns the f32 rounding of the reference's f64 value wherever it leaves
// `rare` unset, at about two thirds of the instructions of the reference
// form.  It computes the f64 value z as the forms above do (2^f by the
// degree-8 polynomial, 2^-39.9; the reciprocal and one Newton step; the
// argument's own rounding below 2^-45), within 2^-39.7 of the exact
// function, relative.  The reference's f64 value (correctly rounded
// division, exp within 1 ulp) lies within 2^-50 of it, and so does the
// reference form mfh_<name>_ref; gelu adds the quantum of the reference's
// 1 - (1 - y) (below).  Two values that close to each other round to the
// same f32 unless an f32 rounding midpoint lies between them: z is flagged
// where its 29 bits below the f32 mantissa lie within `margin` f64 ulps of
// the midpoint 2^28, with a margin of 2^15 f64 ulps, at least 2^-38 |z|
// (three times the distance allowed), so about one element in 2^13 is
// flagged.  So are results that are not normal f32 numbers (the test
// assumes f32 keeps 23 bits above those 29) and arguments outside a form's
// range.  Generated kernels recompute flagged elements through
// mfh_<name>_rare, so the results are the reference forms' everywhere.

// True where a value within `margin` f64 ulps of z may round to another f32
// than z does.  z must round to a normal f32 of magnitude above 2^-126.
MFH_MATH bool mfh_near_f32_midpoint(double z, unsigned margin)
{
    const unsigned low = (unsigned)mfh_low_int(z) & 0x1fffffffu;
    return low - (0x10000000u - margin) < 2u * margin;
}

// False for NaN, infinities, zeros, subnormals and 2^-126 itself, which an
// f64 value below the normal range can round up to.  The tests here combine
// with & and | rather than && and ||, which became one branch per element.
MFH_MATH bool mfh_f32_normal_above_min(float r)
{
    const float a = mfh_absf(r);
    return (a > 0x1p-126f) & (a <= 0x1.fffffep127f);
}

MFH_MATH float mfh_sigmoid_cr(float v, bool& rare)
{
    double den;
    const double z = mfh_sigmoid_z(v, den);
    const float r = (float)z;
    rare |= !(v >= -708.0f) | !mfh_f32_normal_above_min(r) | mfh_near_f32_midpoint(z, 1u << 15);
    return r;
}

MFH_MATH float mfh_silu_cr(float v, bool& rare)
{
    const float m = mfh_med3f(v, -708.0f, 800.0f);
    double den;
    const double z = mfh_silu_z(m, den);
    const float r = (float)z;
    rare |= (m != v) | !mfh_f32_normal_above_min(r) | mfh_near_f32_midpoint(z, 1u << 15);
    return r;
}

// Where inner <= -0.625 the reference forms 1 + tanh as 1 - (1 - y),
// y = 2 / (1 + E): y rounded to a multiple of 2^-53, at most 2^-54 from it,
// which is (1 + E)/4 f64 ulps of z; and its tanh may stand up to 2^-53 off
// there, another (1 + E)/2.  A margin of 2^15 + (1 + E) f64 ulps (at most
// 2^15 + 2^23.4 inside the clamp) covers both, so z takes y as it is.  The
// clamp is the fast form's, [-4.9, 1024]: every v it changes is flagged.
MFH_MATH float mfh_gelu_cr(float v, bool& rare)
{
    const float c = mfh_med3f(v, -4.9f, 1024.0f);
    double den;
    const double z = mfh_gelu_z(c, den);
    const float r = (float)z;
    rare |= (c != v) | !mfh_f32_normal_above_min(r) | mfh_near_f32_midpoint(z, (1u << 15) + (unsigned)den);
    return r;
}

// mfh_<name>_rare: the reference's result as a real call (MFH_RARE), which
// the generated kernels use to recompute flagged elements: the
// rounding-tested form above, and the reference form where that one flags the
// input too (a guard's recomputation in the f16 gelu chain: 49 VALU
// instructions where the test decides, 18 of them moves of the polynomial's
// constants, against 67 for the reference form).  mfh_<name>(v): the fast
// form, or that result where the fast one sets its flag (the host accuracy
// sweep measures these).
#define MFH_FAST_OR_REF(name, fast, ref)                                \
    MFH_MATH float name(float v)                                        \
    {                                                                   \
        bool rare = false;                                              \
        float s = fast(v, rare);                                        \
        MFH_KEEP(s);                                                    \
        if (rare) s = ref(v);                                           \
        return s;                                                       \
    }
#define MFH_RARE_FORM(name)                                             \
    MFH_RARE float mfh_##name##_rare(float v)                           \
    {                                                                   \
        bool rare = false;                                              \
        float s = mfh_##name##_cr(v, rare);                             \
        MFH_KEEP(s);                                                    \
        if (rare) s = mfh_##name##_ref(v);                              \
        return s;                                                       \
    }
MFH_RARE_FORM(sigmoid)
MFH_RARE_FORM(silu)
MFH_RARE_FORM(gelu)
#undef MFH_RARE_FORM
MFH_FAST_OR_REF(mfh_sigmoid, mfh_sigmoid_fast, mfh_sigmoid_rare)
MFH_FAST_OR_REF(mfh_silu, mfh_silu_fast, mfh_silu_rare)
MFH_FAST_OR_REF(mfh_gelu, mfh_gelu_fast, mfh_gelu_rare)

// mfh_<name>_p(v): the rounding-tested form, or the reference form where it
// sets its flag (the host accuracy sweep measures these).
MFH_FAST_OR_REF(mfh_sigmoid_p, mfh_sigmoid_cr, mfh_sigmoid_ref)
MFH_FAST_OR_REF(mfh_silu_p, mfh_silu_cr, mfh_silu_ref)
MFH_FAST_OR_REF(mfh_gelu_p, mfh_gelu_cr, mfh_gelu_ref)
#undef MFH_FAST_OR_REF

MFH_MATH float mfh_exp_ref(float v) { return (float)mfh_exp_f64((double)v); }
MFH_MATH float mfh_log_ref(float v) { return (float)mfh_log_f64((double)v); }
MFH_MATH float mfh_tanh_ref(float v) { return (float)mfh_tanh_f64((double)v); }

#endif  // MFH_DEVMATH_HPP
