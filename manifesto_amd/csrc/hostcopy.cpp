// hostcopy.cpp — a persistent pool of host threads for the staging copies
// of uploads, downloads and SafeTensors reads.  One thread copying a 16 MiB
// chunk at a time into pinned memory capped host-buffer uploads at 23-28
// GB/s of source bytes, below what the link carries, while the device work
// behind each chunk (DMA, dequant) sat idle part of the time.
#include "hostcopy.hpp"

#include <algorithm>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "common.hpp"

namespace mfh {
namespace {

constexpr size_t kMinPiece = 2u << 20;

class Pool {
public:
    ~Pool()
    {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : threads_) t.join();
    }

    // Runs fn(0), ..., fn(n - 1) on the pool's threads and the caller's;
    // one job at a time.
    void run(int n, const std::function<void(int)>& fn)
    {
        std::lock_guard<std::mutex> one(run_mu_);
        std::unique_lock<std::mutex> lk(mu_);
        while ((int)threads_.size() < std::min(n, host_copy_threads()) - 1)
            threads_.emplace_back([this] { worker(); });
        job_ = &fn;
        total_ = n;
        next_ = 0;
        finished_ = 0;
        cv_.notify_all();
        take(lk);
        done_.wait(lk, [&] { return finished_ == total_; });
        job_ = nullptr;
    }

private:
    void take(std::unique_lock<std::mutex>& lk)
    {
        while (job_ && next_ < total_) {
            const int k = next_++;
            const std::function<void(int)>* fn = job_;
            lk.unlock();
            (*fn)(k);
            lk.lock();
            if (++finished_ == total_) done_.notify_all();
        }
    }

    void worker()
    {
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return stop_ || (job_ && next_ < total_); });
            if (stop_) return;
            take(lk);
        }
    }

    std::mutex run_mu_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    std::vector<std::thread> threads_;
    const std::function<void(int)>* job_ = nullptr;
    int total_ = 0, next_ = 0, finished_ = 0;
    bool stop_ = false;
};

Pool& pool()
{
    static Pool p;
    return p;
}

}  // namespace

int host_copy_threads()
{
    static const int n = [] {
        const char* env = std::getenv("MFH_COPY_THREADS");
        if (env && std::atoi(env) >= 1 && std::atoi(env) <= 32) return std::atoi(env);
        const unsigned hw = std::thread::hardware_concurrency();
        return (int)std::max(1u, std::min(8u, hw / 2));
    }();
    return n;
}

int for_each_piece(size_t len, const std::function<int(size_t lo, size_t hi)>& part)
{
    const int pieces = (int)std::min<size_t>((size_t)host_copy_threads(), std::max<size_t>(1, len / kMinPiece));
    if (pieces <= 1) return len ? part(0, len) : MFH_OK;
    // 4 KiB-aligned cuts keep every piece's copy on whole pages
    const size_t step = ((len + pieces - 1) / pieces + 4095) & ~(size_t)4095;
    std::vector<int> rc(pieces, MFH_OK);
    std::vector<std::string> msg(pieces);
    pool().run(pieces, [&](int k) {
        const size_t lo = std::min(len, (size_t)k * step), hi = std::min(len, lo + step);
        if (lo < hi && (rc[k] = part(lo, hi)) != MFH_OK) msg[k] = mfh_last_error();
    });
    for (int k = 0; k < pieces; k++)
        if (rc[k] != MFH_OK) return fail(rc[k], "%s", msg[k].c_str());
    return MFH_OK;
}

int copy_parallel(void* dst, const void* src, size_t len)
{
    return for_each_piece(len, [&](size_t lo, size_t hi) {
        std::memcpy(static_cast<uint8_t*>(dst) + lo, static_cast<const uint8_t*>(src) + lo, hi - lo);
        return MFH_OK;
    });
}

}  // namespace mfh
