// hostcopy.hpp — host-side copies into and out of the pinned staging ring,
// split over a small pool of threads.
#ifndef MFH_HOSTCOPY_HPP
#define MFH_HOSTCOPY_HPP

#include <cstddef>
#include <functional>

namespace mfh {

// Runs part(lo, hi) over [0, len) cut into pieces of at least 2 MiB, on up to
// host_copy_threads() threads (the caller's included), and returns when all
// have finished: MFH_OK, or the first failing piece's code with its message
// re-raised on the calling thread.  part must be safe to run concurrently on
// disjoint ranges.
int for_each_piece(size_t len, const std::function<int(size_t lo, size_t hi)>& part);

// memcpy through for_each_piece.
int copy_parallel(void* dst, const void* src, size_t len);

// Threads a copy may use: MFH_COPY_THREADS when set (1 to 32), else half the
// hardware threads, at most 8.
int host_copy_threads();

}  // namespace mfh

#endif  // MFH_HOSTCOPY_HPP
