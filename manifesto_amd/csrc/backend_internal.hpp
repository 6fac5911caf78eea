// backend_internal.hpp — the upload pipeline of backend.cpp as used by the
// other sources of the library (the SafeTensors loader).
#ifndef MFH_BACKEND_INTERNAL_HPP
#define MFH_BACKEND_INTERNAL_HPP

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/mfh_backend.h"
#include "common.hpp"

namespace mfh {

// Where upload bytes come from: read(dst, offset, len) fills `len` bytes of
// the pinned staging chunk `dst` with source bytes [offset, offset + len).
struct Source {
    virtual ~Source() = default;
    virtual int read(void* dst, size_t offset, size_t len) = 0;
};

// How an upload turns source bytes into stored elements.
struct Plan {
    int src = kInvalid;              // source dtype
    int out = kInvalid;              // stored dtype
    float scale = 1.0f;              // FP8
    Source* scales = nullptr;        // Int4: the group scales, read chunk by chunk beside the nibbles
    int scale_dt = kInvalid;
    int64_t group = 0;
};

// NewShape (tensor/shape.go:32-60): the dimensions and element count of
// `shape`, or MFH_ERR_SHAPE_INVALID for a negative dimension or an element
// count past INT64_MAX.
int make_shape(const int64_t* shape, int32_t rank, std::vector<int64_t>* dims, int64_t* elements);

// Checks the shape against `n_bytes` of plan.src, allocates the stored
// tensor and streams the source through the backend's staging ring (waiting
// for completion when `wait`).  Int4 group scales travel in the same staging
// slots as the nibbles they scale, so nothing else is allocated or waited for.
int upload_from(mfh_backend* backend, const int64_t* shape, int32_t rank, const Plan& plan, Source& source,
                size_t n_bytes, bool wait, mfh_tensor** out);

}  // namespace mfh

#endif  // MFH_BACKEND_INTERNAL_HPP
