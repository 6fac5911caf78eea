// devmath.hpp — the activation math of fused chains, for gfx950.
//
// Like codec.hpp this file is also the text prelude of every JIT-compiled
// fused kernel, so it uses no includes.  It compiles for the host as well
// (MFH_HOST_MATH), which lets the CPU tests measure its accuracy.
//
// Reference semantics (codegen/cpu.go:186-200): Sigmoid, Silu and Gelu are
// evaluated in f64 and rounded once to f32.  The fast forms below compute in
// f32 with error-free corrections and stay within 2 f32 ulps of that; the
// MFH_FUSION_PRECISE forms (mfh_*_ref) restate the f64 formulas.
//
//   e^a, a <= 0:  Cody & Waite reduction a = k ln2 + r (ln2 split into a
//                 16-bit head and an f32 tail), e^r by a degree-6 polynomial
//                 (constants from gen_exp_poly.py), result kept as p * 2^k so
//                 that nothing underflows before the final scaling.
//   v * sigmoid(z) = v / (1 + e^-z)            for z >= 0
//                  = (v p / (1 + p 2^k)) 2^k   for z < 0, e^z = p 2^k
//                 with the quotient corrected by one residual step that also
//                 absorbs the rounding of 1 + e^-|z| and of v p.
#ifndef MFH_DEVMATH_HPP
#define MFH_DEVMATH_HPP

#ifdef MFH_HOST_MATH
#include <cmath>
#define MFH_MATH inline
#define mfh_fmaf(a, b, c) std::fma((float)(a), (float)(b), (float)(c))
#define mfh_fma(a, b, c) std::fma((double)(a), (double)(b), (double)(c))
#define mfh_rintf(x) std::nearbyint((float)(x))
#define mfh_rint(x) std::nearbyint((double)(x))
#define mfh_ldexpf(x, k) std::ldexp((float)(x), (int)(k))
#define mfh_rcpf(x) (1.0f / (float)(x))
#define mfh_fmax(a, b) std::fmax((double)(a), (double)(b))
#define mfh_fmaxf(a, b) std::fmax((float)(a), (float)(b))
#define mfh_tanh_f64(x) std::tanh((double)(x))
#define mfh_exp_f64(x) std::exp((double)(x))
#define mfh_log_f64(x) std::log((double)(x))
#define mfh_sqrtf(x) std::sqrt((float)(x))
inline unsigned mfh_fbits(float f) { unsigned u; __builtin_memcpy(&u, &f, 4); return u; }
inline float mfh_fromfbits(unsigned u) { float f; __builtin_memcpy(&f, &u, 4); return f; }
#else
extern "C" __device__ double __ocml_tanh_f64(double);
extern "C" __device__ double __ocml_exp_f64(double);
extern "C" __device__ double __ocml_log_f64(double);
#define MFH_MATH __device__ inline __attribute__((always_inline))
#define mfh_fmaf(a, b, c) __builtin_fmaf((a), (b), (c))
#define mfh_fma(a, b, c) __builtin_fma((a), (b), (c))
#define mfh_rintf(x) __builtin_rintf(x)
#define mfh_rint(x) __builtin_rint(x)
#define mfh_ldexpf(x, k) __builtin_amdgcn_ldexpf((x), (k))
#define mfh_rcpf(x) __builtin_amdgcn_rcpf(x)
#define mfh_fmax(a, b) __builtin_fmax((a), (b))
#define mfh_fmaxf(a, b) __builtin_fmaxf((a), (b))
#define mfh_tanh_f64(x) __ocml_tanh_f64(x)
#define mfh_exp_f64(x) __ocml_exp_f64(x)
#define mfh_log_f64(x) __ocml_log_f64(x)
#define mfh_sqrtf(x) __builtin_sqrtf(x)
__device__ inline unsigned mfh_fbits(float f) { return __builtin_bit_cast(unsigned, f); }
__device__ inline float mfh_fromfbits(unsigned u) { return __builtin_bit_cast(float, u); }
#endif

#define MFH_LOG2E_F 1.44269502162933349609375f         // 0x3fb8aa3b
#define MFH_LN2_HI_F 0.693145751953125f                 // 0x3f317200, 16 bits
#define MFH_LN2_LO_F 1.428606765330187e-06f             // 0x35bfbe8e
#define MFH_LOG2E_D 1.4426950408889634                  // 0x3ff71547652b82fe
#define MFH_LN2_D 0.6931471805599453                    // 0x3fe62e42fefa39ef
#define MFH_SQRT_2_OVER_PI_D 0.7978845608028654         // 0x3fe9884533d43651 = sqrt(fl64(2/pi))
#define MFH_GELU_A_D 0.044715                           // 0x3fa6e4e26d4801f7

// e^r for |r| <= ln2/2 (+ margin): 1 + r(c1 + r(c2 + ... + r c6)).
MFH_MATH float mfh_exp_poly(float r)
{
    float q = 0.0013859282480552793f;            // 0x3ab5a809
    q = mfh_fmaf(q, r, 0.0083747748285532f);     // 0x3c09365a
    q = mfh_fmaf(q, r, 0.04166772589087486f);    // 0x3d2aabc7
    q = mfh_fmaf(q, r, 0.1666642129421234f);     // 0x3e2aaa06
    q = mfh_fmaf(q, r, 0.4999999403953552f);     // 0x3efffffe
    q = mfh_fmaf(q, r, 1.0f);
    return mfh_fmaf(q, r, 1.0f);
}

// e^a = p * 2^k for a <= 0 (a clamped at -200, far below the f32 range).
MFH_MATH float mfh_exp_neg(float a, int* k)
{
    a = mfh_fmaxf(a, -200.0f);
    float kf = mfh_rintf(a * MFH_LOG2E_F);
    float r = mfh_fmaf(kf, -MFH_LN2_HI_F, a);
    r = mfh_fmaf(kf, -MFH_LN2_LO_F, r);
    *k = (int)kf;
    return mfh_exp_poly(r);
}

// Same with an f64 argument: the reduction runs in f64, so the argument's
// own f64 accuracy carries through to r.
MFH_MATH float mfh_exp_neg_d(double a, int* k)
{
    a = mfh_fmax(a, -200.0);
    double kd = mfh_rint(a * MFH_LOG2E_D);
    double r = mfh_fma(kd, -MFH_LN2_D, a);
    *k = (int)kd;
    return mfh_exp_poly((float)r);
}

// n * sigmoid(z) given e^-|z| = p * 2^k, z_neg = (z < 0).
MFH_MATH float mfh_mul_sigmoid(float n, bool z_neg, float p, int k)
{
    float t = mfh_ldexpf(p, k);
    float d = 1.0f + t;
    float dl = t - (d - 1.0f);              // 1 + t == d + dl exactly
    float nh = z_neg ? n * p : n;
    float nl = z_neg ? mfh_fmaf(n, p, -nh) : 0.0f;
    float r = mfh_rcpf(d);
    float q = nh * r;
    float e = mfh_fmaf(-q, d, nh);
    e = e + nl;
    e = mfh_fmaf(-q, dl, e);
    q = mfh_fmaf(e, r, q);
    return z_neg ? mfh_ldexpf(q, k) : q;
}

// The reference's results at +-Inf: silu/gelu(+Inf) = +Inf, (-Inf) = NaN
// (Inf/Inf and Inf*0 in f64); sigmoid(+-Inf) = 1, 0.
MFH_MATH bool mfh_is_inf(float v) { return (mfh_fbits(v) & 0x7fffffffu) == 0x7f800000u; }

MFH_MATH float mfh_sigmoid(float v)
{
    int k;
    float p = mfh_exp_neg(-__builtin_fabsf(v), &k);
    float s = mfh_mul_sigmoid(1.0f, v < 0.0f, p, k);
    return mfh_is_inf(v) ? (v > 0.0f ? 1.0f : 0.0f) : s;
}

MFH_MATH float mfh_silu(float v)
{
    int k;
    float p = mfh_exp_neg(-__builtin_fabsf(v), &k);
    float s = mfh_mul_sigmoid(v, v < 0.0f, p, k);
    s = v < -200.0f ? -0.0f : s;  // v e^v is below the f32 range (and v p could overflow)
    return mfh_is_inf(v) ? (v > 0.0f ? v : mfh_fromfbits(0xffc00000u)) : s;
}

// Reference forms (codegen/cpu.go:186-200), f64 then one rounding.
MFH_MATH float mfh_sigmoid_ref(float v) { return (float)(1.0 / (1.0 + mfh_exp_f64(-(double)v))); }
MFH_MATH float mfh_silu_ref(float v) { return (float)((double)v / (1.0 + mfh_exp_f64(-(double)v))); }

// Kept out of line on the device: it runs only for rare inputs.
#ifdef MFH_HOST_MATH
inline float mfh_gelu_ref(float v)
#else
__device__ __attribute__((noinline)) float mfh_gelu_ref(float v)
#endif
{
    double d = (double)v;
    double inner = MFH_SQRT_2_OVER_PI_D * (d + MFH_GELU_A_D * d * d * d);
    return (float)(0.5 * d * (1.0 + mfh_tanh_f64(inner)));
}

// Below v = -4.9 the reference's 1 + tanh(inner) cancels in f64, so its
// result carries the f64 quantum of tanh; that rare range runs the reference
// form itself.  Elsewhere inner is formed in f64 with the reference's
// operation order and gelu = v * sigmoid(2 inner).
MFH_MATH float mfh_gelu(float v)
{
    if (v < -4.9f) return mfh_gelu_ref(v);
    double d = (double)v;
    double z = 2.0 * (MFH_SQRT_2_OVER_PI_D * (d + MFH_GELU_A_D * d * d * d));
    int k;
    float p = mfh_exp_neg_d(-__builtin_fabs(z), &k);
    float s = mfh_mul_sigmoid(v, z < 0.0, p, k);
    return mfh_is_inf(v) ? v : s;  // -Inf took the reference path
}

MFH_MATH float mfh_exp_ref(float v) { return (float)mfh_exp_f64((double)v); }
MFH_MATH float mfh_log_ref(float v) { return (float)mfh_log_f64((double)v); }
MFH_MATH float mfh_tanh_ref(float v) { return (float)mfh_tanh_f64((double)v); }

#endif  // MFH_DEVMATH_HPP
