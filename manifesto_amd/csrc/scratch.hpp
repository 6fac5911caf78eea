// scratch.hpp — the per-device static scratch behind mfh_graph_call_noalloc.
#ifndef MFH_SCRATCH_HPP
#define MFH_SCRATCH_HPP

#include <cstdint>

#include "common.hpp"
#include "../../include/mfh_graph.h"

namespace mfh {

// Looks up the scratch array's address on `device`, which must be current;
// once per device (mfh_init calls it).
int scratch_setup(int device);
// The address scratch_setup found on `device` (MFH_GRAPH_SCRATCH_BYTES long).
int scratch_address(int device, void** at);
// Writes n f32 values to device memory `dst` with kernel launches on
// `stream` (no copy from host memory, no memset: safe under stream capture).
int put_constants(float* dst, const float* values, int64_t n, hipStream_t stream);

}  // namespace mfh

#endif  // MFH_SCRATCH_HPP
