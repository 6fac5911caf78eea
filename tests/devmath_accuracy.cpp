// Host build of the fused-kernel activation math (devmath.hpp, MFH_HOST_MATH)
// measured against the oracle's restatement of codegen/cpu.go:186-200 over a
// strided sweep of every f32 bit pattern.  One line per function:
//   <name> max_ulp=<m> over_tol=<n> nan_mismatch=<k> exact=<fraction> samples=<s>
// The rounding-tested forms (<name>_p: mfh_<name>_cr, or the reference form
// where it flags the input) add
//   ref_mismatch=<bit patterns that differ from mfh_<name>_ref> flagged=<fraction>
//   max_rel_err_log2=<log2 of the largest |z - f(v)| / |f(v)|>
// where z is the f64 value the form rounds (mfh_<name>_z) and f(v) the same
// formula in long double, over the inputs inside the form's range whose
// result is a normal f32.
// Usage: devmath_accuracy <stride> <threads> [name,name,...]
#define MFH_HOST_MATH
#include "../manifesto_amd/csrc/devmath.hpp"
#include "../oracle/oracle.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

static int64_t ulp_key(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? (int64_t)0x80000000u - (int64_t)u : (int64_t)u;
}

struct Fn {
    const char* name;
    int node;  // optimizer.NodeType of the oracle's evaluator
    float (*fn)(float);
    int tol;
    float (*cr)(float, bool&) = nullptr;  // rounding-tested form: its flag,
    float (*ref)(float) = nullptr;        // the reference form it must reproduce,
    double (*z)(float) = nullptr;         // the f64 value it rounds (NaN outside its range)
    long double (*exact)(long double) = nullptr;
};

// The rounding-tested forms' f64 values, inside each form's argument range.
static double sigmoid_z(float v)
{
    double den;
    return v >= -708.0f ? mfh_sigmoid_z(v, den) : NAN;
}
static double silu_z(float v)
{
    double den;
    return v >= -708.0f && v <= 800.0f ? mfh_silu_z(v, den) : NAN;
}
static double gelu_z(float v)
{
    double den;
    return v >= -4.9f && v <= 1024.0f ? mfh_gelu_z(v, den) : NAN;
}
static long double sigmoid_exact(long double v) { return 1.0L / (1.0L + std::exp(-v)); }
static long double silu_exact(long double v) { return v / (1.0L + std::exp(-v)); }
// v / (1 + e^(-2 inner)) = (v/2)(1 + tanh(inner)) without the cancellation
// of 1 + tanh, with the reference's f64 constants.
static long double gelu_exact(long double v)
{
    const long double inner = (long double)MFH_SQRT_2_OVER_PI_D * (v + (long double)MFH_GELU_A_D * v * v * v);
    return v / (1.0L + std::exp(-2.0L * inner));
}

static uint32_t bits_of(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

int main(int argc, char** argv)
{
    const uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 4099;
    const int threads = argc > 2 ? std::atoi(argv[2]) : 4;
    const Fn fns[] = {
        {"sigmoid", 15, mfh_sigmoid, 1}, {"silu", 17, mfh_silu, 2}, {"gelu", 18, mfh_gelu, 2},
        {"exp_ref", 12, mfh_exp_ref, 1}, {"log_ref", 13, mfh_log_ref, 1}, {"tanh_ref", 16, mfh_tanh_ref, 1},
        {"sigmoid_ref", 15, mfh_sigmoid_ref, 1}, {"silu_ref", 17, mfh_silu_ref, 1}, {"gelu_ref", 18, mfh_gelu_ref, 1},
        {"sigmoid_p", 15, mfh_sigmoid_p, 1, mfh_sigmoid_cr, mfh_sigmoid_ref, sigmoid_z, sigmoid_exact},
        {"silu_p", 17, mfh_silu_p, 1, mfh_silu_cr, mfh_silu_ref, silu_z, silu_exact},
        {"gelu_p", 18, mfh_gelu_p, 1, mfh_gelu_cr, mfh_gelu_ref, gelu_z, gelu_exact},
    };
    const char* only = argc > 3 ? argv[3] : nullptr;
    for (const Fn& f : fns) {
        if (only) {
            const char* hit = std::strstr(only, f.name);
            size_t len = std::strlen(f.name);
            if (!hit || (hit != only && hit[-1] != ',') || (hit[len] != ',' && hit[len] != '\0')) continue;
        }
        std::vector<int64_t> max_ulp(threads, 0), over(threads, 0), nan_bad(threads, 0), exact(threads, 0),
            count(threads, 0), ref_bad(threads, 0), flagged(threads, 0);
        std::vector<double> max_rel(threads, 0.0);
        std::vector<std::thread> pool;
        for (int w = 0; w < threads; w++)
            pool.emplace_back([&, w] {
                for (uint64_t u = (uint64_t)w * stride; u < (1ull << 32); u += stride * (uint64_t)threads) {
                    uint32_t bits = (uint32_t)u;
                    float v;
                    std::memcpy(&v, &bits, 4);
                    float want = orc_eval_unary(f.node, v);
                    float got = f.fn(v);
                    count[w]++;
                    if (f.cr) {
                        bool rare = false;
                        (void)f.cr(v, rare);
                        flagged[w] += rare;
                        const float r = f.ref(v);
                        if (bits_of(got) != bits_of(r) && !(std::isnan(got) && std::isnan(r))) ref_bad[w]++;
                        const double z = f.z(v);
                        const long double e = f.exact((long double)v);
                        if (!std::isnan(z) && std::isnormal((float)e)) {
                            const double rel = (double)(std::fabs((long double)z - e) / std::fabs(e));
                            if (rel > max_rel[w]) max_rel[w] = rel;
                        }
                    }
                    if (std::isnan(want) || std::isnan(got)) {
                        if (std::isnan(want) != std::isnan(got)) nan_bad[w]++;
                        else exact[w]++;
                        continue;
                    }
                    int64_t d = std::llabs(ulp_key(want) - ulp_key(got));
                    if (d == 0) exact[w]++;
                    if (d > f.tol) over[w]++;
                    if (d > max_ulp[w]) max_ulp[w] = d;
                }
            });
        for (auto& t : pool) t.join();
        int64_t m = 0, o = 0, nb = 0, ex = 0, n = 0, rb = 0, fl = 0;
        double mr = 0.0;
        for (int w = 0; w < threads; w++) {
            m = max_ulp[w] > m ? max_ulp[w] : m;
            o += over[w];
            nb += nan_bad[w];
            ex += exact[w];
            n += count[w];
            rb += ref_bad[w];
            fl += flagged[w];
            mr = max_rel[w] > mr ? max_rel[w] : mr;
        }
        std::printf("%s max_ulp=%lld over_tol=%lld nan_mismatch=%lld exact=%.6f samples=%lld", f.name,
                    (long long)m, (long long)o, (long long)nb, (double)ex / (double)n, (long long)n);
        if (f.cr)
            std::printf(" ref_mismatch=%lld flagged=%.6f max_rel_err_log2=%.2f", (long long)rb, (double)fl / (double)n,
                        mr > 0.0 ? std::log2(mr) : -1100.0);
        std::printf("\n");
    }
    return 0;
}
