// launch.hpp — grid sizing and vector types shared by the ahead-of-time
// streaming kernels.
//
// Every streaming kernel here is written so that each store instruction of a
// wave writes one contiguous 1 KiB span (64 lanes x 16 bytes): on MI355X a
// wave that interleaves two 16-byte stores per lane (lane j writing bytes
// 32j..32j+15 and then 32j+16..32j+31) ran 15-20% slower on a 1:2
// read:write stream than the contiguous form.
#ifndef MFH_LAUNCH_HPP
#define MFH_LAUNCH_HPP

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "common.hpp"
#include "codec.hpp"

namespace mfh {

typedef mfh_u32 u32x4 __attribute__((ext_vector_type(4)));
typedef mfh_u32 u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBlock = 256;  // 4 wave64 per workgroup: families without a size setting

// Grid for `items` work items of `per_thread` items each in workgroups of
// `block` threads, capped at compute_units * blocks_per_cu(k); threads loop
// over the rest.  A dispatch counts its work-items in 32 bits, so grids stay
// below 2^32 / block.
inline unsigned grid_for(int64_t items, const Device* dev, Kern k, int per_thread = 1, int block = kBlock)
{
    int64_t threads = (items + per_thread - 1) / per_thread;
    int64_t need = (threads + block - 1) / block;
    int64_t cap = std::min<int64_t>((int64_t)dev->compute_units * blocks_per_cu(k), (int64_t(1) << 32) / block - 1);
    return (unsigned)std::max<int64_t>(1, std::min(need, cap));
}

// Runs f(std::integral_constant<int, BS>{}) with BS the workgroup size
// `threads` (64, 128 or 256; anything else runs 256), so that a launcher
// picks the kernel instantiation and its grid from one reading of the
// family's setting.
template <typename F>
int with_block(int threads, F&& f)
{
    switch (threads) {
    case 64: return f(std::integral_constant<int, 64>{});
    case 128: return f(std::integral_constant<int, 128>{});
    default: return f(std::integral_constant<int, 256>{});
    }
}

// with_block, plus 512-thread workgroups for the one family that runs them
// (the Int4 dequant).
template <typename F>
int with_block_to_512(int threads, F&& f)
{
    if (threads == 512) return f(std::integral_constant<int, 512>{});
    return with_block(threads, std::forward<F>(f));
}

int launch_status(const char* what);

// Streaming 16-byte stores of a chunk: buffer stores with the non-temporal
// (nt) and sc1 cache-policy bits, addressed from the chunk's first item (the
// base is uniform across the block, so the descriptor lives in SGPRs).  On
// MI355X, with the inputs coming from HBM, nt|sc1 stores run the FP8 dequant
// (1:2 read:write) at 6.1-6.2 TB/s and the Int4 dequant (1:4) at 6.0-6.1,
// against 5.8 and 5.5 with plain stores; nt alone is 1-2% slower, sc1 alone
// 4-6%.  The descriptor's record count is the chunk's remaining bytes, so the
// hardware drops anything past the end of the output.
struct StreamOut {
    __amdgpu_buffer_rsrc_t rsrc;
    __device__ StreamOut(u32x4* base, int64_t items_left)
        : rsrc(__builtin_amdgcn_make_buffer_rsrc(
              base, 0, (int)std::min<int64_t>(items_left * 16, 0x7fffffff), kBufferConfig))
    {
    }
    __device__ void store(int item, u32x4 v) const
    {
        __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, item * 16, 0, kCachePolicy);
    }
    // Word 3 of a raw (untyped) gfx9 buffer descriptor.
    static constexpr int kBufferConfig = 0x00020000;
    // gfx950 buffer cache policy: bit 1 nt, bit 4 sc1.
    static constexpr int kCachePolicy = 2 | 16;
};

// Streaming store through a plain address (global_store ... nt).
template <typename T>
__device__ inline void store_nt(T* p, T v)
{
    __builtin_nontemporal_store(v, p);
}

// Streaming load (global_load ... nt).  Used where a kernel reads at least as
// many bytes as it writes (non-temporal loads measured +4% on a 1:1 stream
// and +8% on 2:1), and by the FP8 dequant (+0.6% with its codes coming from
// HBM); the Int4 dequant (-0.8%) and the widening casts keep plain loads.
template <typename T>
__device__ inline T load_nt(const T* p)
{
    return __builtin_nontemporal_load(p);
}

}  // namespace mfh

#endif  // MFH_LAUNCH_HPP
