// common.hpp — host-side plumbing shared by the mfh library sources:
// dtype codes, error reporting, device state.
#ifndef MFH_COMMON_HPP
#define MFH_COMMON_HPP

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <string>

#include "../../include/mfh.h"

namespace mfh {

// Wire codes of manifesto's DType (dtype/dtype.go:29-49).
enum DType : uint8_t {
    kInvalid = 0, kFloat64 = 1, kFloat32 = 2, kFloat16 = 3, kBFloat16 = 4,
    kF8E4M3 = 5, kF8E5M2 = 6, kInt64 = 7, kInt32 = 8, kInt16 = 9, kInt8 = 10,
    kInt4 = 11, kUint64 = 12, kUint32 = 13, kUint16 = 14, kUint8 = 15,
    kBool = 16, kComplex64 = 17, kComplex128 = 18,
};

// DType.Size for unpacked numeric dtypes (dtype/dtype.go:57-75); 0 otherwise.
int dtype_size(int dtype);
// DType.Name (dtype/dtype.go:140-) for messages.
const char* dtype_name(int dtype);
// DType.String (dtype/dtype.go:190-231): the wire names ("F32", "BF16", ...)
// the reference prints in its error messages.
const char* dtype_string(int dtype);
// DType.BytesFor (dtype/dtype.go:81-101): packed Int4 / Bool counts
// included; -1 for a negative count or a dtype without a size.
int64_t bytes_for(int dtype, int64_t elements);

// Sets the calling thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Records a sticky error of an entry point without an error channel against
// the stream its work was meant for; take_sticky(stream) returns and clears
// that stream's first error (MFH_OK when none) and makes its message the
// calling thread's last error; drop_sticky forgets a stream being destroyed.
void fail_sticky(hipStream_t stream, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int take_sticky(hipStream_t stream);
void drop_sticky(hipStream_t stream);
int check_hip(hipError_t err, const char* what);

struct Device {
    int ordinal = -1;
    int compute_units = 0;
    int64_t total_bytes = 0;
};
// The bound device; makes it current on the calling thread.  Returns
// MFH_ERR_NOT_INITIALIZED when mfh_init has not run.
int bind_device(const Device** out);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Streaming kernels with their own grid-size setting.
enum class Kern { kFp8, kInt4, kAxpy, kAxpy16, kConvert, kFused, kCount };

// Launch shape of a grid-stride kernel family: workgroups per CU and work
// items per thread per step.  Per-kernel defaults measured on MI355X;
// mfh_set_launch_config or MFH_BPC_<NAME> / MFH_UNROLL_<NAME> (NAME = FP8,
// INT4, AXPY, AXPY16, CONVERT, FUSED) change them.
int blocks_per_cu(Kern k);
int items_per_thread(Kern k);
// Threads per workgroup (MFH_THREADS_<NAME>, mfh_set_launch_threads); 0 for
// the fused family means each generated kernel's default.
int threads_per_block(Kern k);

}  // namespace mfh

#define MFH_TRY(expr)                  \
    do {                               \
        int mfh_rc_ = (expr);          \
        if (mfh_rc_ != MFH_OK) return mfh_rc_; \
    } while (0)

#endif  // MFH_COMMON_HPP
