// launch.hpp — grid sizing and vector types shared by the ahead-of-time
// streaming kernels.
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

// Workgroups per CU for grid-stride streaming kernels (tuned on MI355X;
// overridable with MFH_BLOCKS_PER_CU for sweeps).
int blocks_per_cu();

// Grid for `items` work items of one thread each, capped at
// compute_units * blocks_per_cu() so each thread loops over several items.
inline unsigned grid_for(int64_t items, const Device* dev)
{
    int64_t need = (items + kBlock - 1) / kBlock;
    int64_t cap = (int64_t)dev->compute_units * blocks_per_cu();
    return (unsigned)std::max<int64_t>(1, std::min(need, cap));
}

int launch_status(const char* what);

}  // namespace mfh

#endif  // MFH_LAUNCH_HPP
