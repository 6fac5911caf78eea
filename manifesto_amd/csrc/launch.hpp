// launch.hpp — grid sizing and vector types shared by the ahead-of-time
// streaming kernels.
//
// Every streaming kernel here is written so that each store instruction of a
// wave writes one contiguous 1 KiB span (64 lanes x 16 bytes): on MI355X a
// wave that interleaves two 16-byte stores per lane (lane j writing bytes
// 32j..32j+15 and then 32j+16..32j+31) reaches ~4.5-5.0 TB/s on a 1:2
// read:write stream, the contiguous form ~5.6-5.8 TB/s.
#ifndef MFH_LAUNCH_HPP
#define MFH_LAUNCH_HPP

#include <algorithm>
#include <cstdint>

#include "common.hpp"
#include "codec.hpp"

namespace mfh {

typedef mfh_u32 u32x4 __attribute__((ext_vector_type(4)));
typedef mfh_u32 u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBlock = 256;  // 4 wave64 per workgroup

// Grid for `items` work items of `per_thread` items each, capped at
// compute_units * blocks_per_cu(k); threads loop over the rest.
inline unsigned grid_for(int64_t items, const Device* dev, Kern k, int per_thread = 1)
{
    int64_t threads = (items + per_thread - 1) / per_thread;
    int64_t need = (threads + kBlock - 1) / kBlock;
    int64_t cap = (int64_t)dev->compute_units * blocks_per_cu(k);
    return (unsigned)std::max<int64_t>(1, std::min(need, cap));
}

int launch_status(const char* what);

}  // namespace mfh

#endif  // MFH_LAUNCH_HPP
