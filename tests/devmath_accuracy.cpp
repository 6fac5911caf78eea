// Host build of the fused-kernel activation math (devmath.hpp, MFH_HOST_MATH)
// measured against the oracle's restatement of codegen/cpu.go:186-200 over a
// strided sweep of every f32 bit pattern.  One line per function:
//   <name> max_ulp=<m> over_tol=<n> nan_mismatch=<k> exact=<fraction> samples=<s>
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
};

int main(int argc, char** argv)
{
    const uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 4099;
    const int threads = argc > 2 ? std::atoi(argv[2]) : 4;
    const Fn fns[] = {
        {"sigmoid", 15, mfh_sigmoid, 1}, {"silu", 17, mfh_silu, 2}, {"gelu", 18, mfh_gelu, 2},
        {"silu_x", 17, mfh_silu_x, 2}, {"gelu_x", 18, mfh_gelu_x, 2},
        {"exp_ref", 12, mfh_exp_ref, 1}, {"log_ref", 13, mfh_log_ref, 1}, {"tanh_ref", 16, mfh_tanh_ref, 1},
        {"sigmoid_ref", 15, mfh_sigmoid_ref, 1}, {"silu_ref", 17, mfh_silu_ref, 1}, {"gelu_ref", 18, mfh_gelu_ref, 1},
    };
    const char* only = argc > 3 ? argv[3] : nullptr;
    for (const Fn& f : fns) {
        if (only) {
            const char* hit = std::strstr(only, f.name);
            size_t len = std::strlen(f.name);
            if (!hit || (hit != only && hit[-1] != ',') || (hit[len] != ',' && hit[len] != '\0')) continue;
        }
        std::vector<int64_t> max_ulp(threads, 0), over(threads, 0), nan_bad(threads, 0), exact(threads, 0),
            count(threads, 0);
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
        int64_t m = 0, o = 0, nb = 0, ex = 0, n = 0;
        for (int w = 0; w < threads; w++) {
            m = max_ulp[w] > m ? max_ulp[w] : m;
            o += over[w];
            nb += nan_bad[w];
            ex += exact[w];
            n += count[w];
        }
        std::printf("%s max_ulp=%lld over_tol=%lld nan_mismatch=%lld exact=%.6f samples=%lld\n", f.name,
                    (long long)m, (long long)o, (long long)nb, (double)ex / (double)n, (long long)n);
    }
    return 0;
}
