// Host-only checks of manifesto_amd/csrc/hostcopy.cpp (the staging copy
// pool), built by tests/test_hostcopy.py with g++ (also under ThreadSanitizer)
// and run once per MFH_COPY_THREADS setting.  Prints one line per check and
// exits non-zero on the first failure.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "common.hpp"
#include "hostcopy.hpp"

namespace mfh {
thread_local std::string t_error;
int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_error = buf;
    return code;
}
}  // namespace mfh
extern "C" const char* mfh_last_error(void) { return mfh::t_error.c_str(); }

#define CHECK(cond, ...)                                     \
    do {                                                     \
        if (!(cond)) {                                       \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                        \
            std::printf("\n");                               \
            return 1;                                        \
        }                                                    \
    } while (0)

int main()
{
    std::printf("threads %d\n", mfh::host_copy_threads());
    // every byte of [0, len) is visited by exactly one piece
    for (size_t len : {size_t(0), size_t(1), size_t(4095), (size_t(2) << 20) - 1, size_t(2) << 20,
                       (size_t(2) << 20) + 1, (size_t(37) << 20) + 13}) {
        std::vector<unsigned char> hits(len + 1, 0);
        std::atomic<int> pieces{0};
        int rc = mfh::for_each_piece(len, [&](size_t lo, size_t hi) {
            for (size_t i = lo; i < hi; i++) hits[i]++;
            pieces++;
            return MFH_OK;
        });
        CHECK(rc == MFH_OK, "len %zu: rc %d", len, rc);
        for (size_t i = 0; i < len; i++) CHECK(hits[i] == 1, "len %zu: byte %zu visited %d times", len, i, hits[i]);
        CHECK(hits[len] == 0, "len %zu: wrote past the end", len);
        CHECK(len == 0 ? pieces == 0 : pieces >= 1, "len %zu: %d pieces", len, pieces.load());
    }
    std::printf("coverage ok\n");
    // copies equal memcpy
    std::vector<unsigned char> a((size_t(33) << 20) + 7), b(a.size() + 1, 0xA5);
    for (size_t i = 0; i < a.size(); i++) a[i] = (unsigned char)(i * 131 + (i >> 11));
    CHECK(mfh::copy_parallel(b.data(), a.data(), a.size()) == MFH_OK, "copy rc");
    CHECK(std::memcmp(a.data(), b.data(), a.size()) == 0 && b[a.size()] == 0xA5, "copy differs");
    std::printf("copy ok\n");
    // a failing piece's code and message reach the calling thread
    const size_t bad_at = (size_t(21) << 20) + 5;
    int rc = mfh::for_each_piece(size_t(40) << 20, [&](size_t lo, size_t hi) {
        if (lo <= bad_at && bad_at < hi) return mfh::fail(-4, "piece [%zu, %zu) failed", lo, hi);
        return MFH_OK;
    });
    CHECK(rc == -4, "error rc %d", rc);
    CHECK(std::strstr(mfh_last_error(), "failed") != nullptr, "message '%s'", mfh_last_error());
    std::printf("error ok: %s\n", mfh_last_error());
    // callers on several threads at once
    std::vector<std::thread> ts;
    std::atomic<int> bad{0};
    for (int k = 0; k < 6; k++)
        ts.emplace_back([&, k] {
            std::vector<unsigned char> src((size_t(5) << 20) + k), dst(src.size());
            for (int rep = 0; rep < 20; rep++) {
                for (size_t i = 0; i < src.size(); i += 4099) src[i] = (unsigned char)(k + rep + i);
                if (mfh::copy_parallel(dst.data(), src.data(), src.size()) != MFH_OK || dst != src) bad++;
            }
        });
    for (auto& t : ts) t.join();
    CHECK(bad == 0, "%d concurrent copies differ", bad.load());
    std::printf("concurrent ok\n");
    return 0;
}
