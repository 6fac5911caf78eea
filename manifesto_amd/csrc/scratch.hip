// scratch.hip — the fixed device scratch of the allocation-free graph call
// (mfh_graph_call_noalloc): a file-scope device array that each GPU holds
// for the life of the process, and the small kernel that writes a graph's
// constants into it.
//
// The array's name is a host-side stand-in, not a device address: host code
// uses only the per-device address that hipGetSymbolAddress returns at
// mfh_init, never the name itself.
#include <mutex>

#include "launch.hpp"
#include "scratch.hpp"

static __device__ __align__(256) unsigned char scratch[MFH_GRAPH_SCRATCH_BYTES];

namespace mfh {

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_at[kMaxDevices] = {};

// Up to kConstantsPerLaunch f32 values, passed by value in the kernel
// arguments, written by one wave.
constexpr int kConstantsPerLaunch = 32;
struct ConstantBlock {
    float v[kConstantsPerLaunch];
};

__global__ __launch_bounds__(64) void k_put_constants(float* __restrict__ dst, ConstantBlock block, int n)
{
    const int i = (int)threadIdx.x;
    if (i < n) dst[i] = block.v[i];
}

}  // namespace

int scratch_setup(int device)
{
    if (device < 0 || device >= kMaxDevices)
        return fail(MFH_ERR_INVALID_ARGUMENT, "scratch: device %d is past the %d this library tracks", device,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_at[device]) return MFH_OK;
    void* at = nullptr;
    MFH_TRY(check_hip(hipGetSymbolAddress(&at, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    if (!at) return fail(MFH_ERR_DEVICE, "hipGetSymbolAddress(scratch): no address");
    g_scratch_at[device] = at;
    return MFH_OK;
}

int scratch_address(int device, void** at)
{
    *at = nullptr;
    if (device >= 0 && device < kMaxDevices) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        *at = g_scratch_at[device];
    }
    if (!*at) return fail(MFH_ERR_NOT_INITIALIZED, "scratch: device %d has no scratch address (mfh_init)", device);
    return MFH_OK;
}

int put_constants(float* dst, const float* values, int64_t n, hipStream_t stream)
{
    for (int64_t first = 0; first < n; first += kConstantsPerLaunch) {
        ConstantBlock block;
        const int count = (int)std::min<int64_t>(kConstantsPerLaunch, n - first);
        for (int k = 0; k < kConstantsPerLaunch; k++) block.v[k] = k < count ? values[first + k] : 0.0f;
        k_put_constants<<<1, 64, 0, stream>>>(dst + first, block, count);
        MFH_TRY(launch_status("k_put_constants"));
    }
    return MFH_OK;
}

}  // namespace mfh
