/*
 * mfh_backend.h — C ABI of the HIP tensor backend: device-resident tensors
 * behind manifesto's tensor.Backend / tensor.Tensor contract
 * (tensor/backend.go:18-68, tensor/tensor.go:53-130), the dequantising upload
 * that stores FP8 / Int4 weights as BFloat16 on the device, and the resident
 * axpy of runtime/axpy.go:44-93.  A Go host binds these 1:1 (cgo); the
 * Location of every tensor here is "hip".
 *
 * Uploads stream through pinned host staging in chunks, the copy of one chunk
 * overlapping the DMA (and, for FP8 / Int4 sources, the on-device dequant) of
 * the previous one.  Every device operation of a backend runs on that
 * backend's own stream.
 */
#ifndef MFH_BACKEND_H
#define MFH_BACKEND_H

#include "mfh.h"
#include "mfh_graph.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MFH_ERR_SHAPE_INVALID (-8)  /* tensor.ErrShapeInvalid, tensor/errors.go:50 */
#define MFH_ERR_TENSOR_CLOSED (-9)  /* tensor.ErrTensorClosed, tensor/errors.go:42 */
#define MFH_ERR_LAYOUT_UNSUPPORTED (-10) /* tensor.ErrLayoutUnsupported, tensor/errors.go:23 */

typedef struct mfh_backend mfh_backend;
typedef struct mfh_tensor mfh_tensor;

/* tensor.Capabilities (tensor/backend.go:80-110). */
typedef struct {
    int64_t max_bytes;
    int32_t supports_async;
    int32_t supports_sparse;
    int32_t supports_autograd;
    int32_t native_alignment;
    int32_t numa_nodes;
    int32_t reserved;
} mfh_backend_caps;

/* tensor.State (tensor/state.go:27-30). */
#define MFH_STATE_READY 0
#define MFH_STATE_PENDING 1
#define MFH_STATE_MUTATING 2
#define MFH_STATE_CLOSED 3

/* A backend on HIP device `device` (calls mfh_init(device)). */
int mfh_backend_open(int device, mfh_backend** backend);

/* Backend.Location: "hip". */
const char* mfh_backend_location(const mfh_backend* backend);

/* Backend.SupportedDTypes: the source dtypes Upload takes without a host
 * conversion (Float32, Float16, BFloat16, Float8E4M3, Float8E5M2, Int4).
 * Returns their number and copies up to `cap`. */
int32_t mfh_backend_supported_dtypes(const mfh_backend* backend, uint8_t* dtypes, int32_t cap);

/* Backend.SupportedLayouts: {LayoutDense} (layout code 0). */
int32_t mfh_backend_supported_layouts(const mfh_backend* backend, uint8_t* layouts, int32_t cap);

/* Backend.Capabilities: device memory, async uploads, 256-byte alignment. */
int mfh_backend_capabilities(const mfh_backend* backend, mfh_backend_caps* caps);

/* Backend.Upload (tensor/backend.go:37-40): `bytes` must hold exactly
 * shape x source dtype (DType.BytesFor, dtype/dtype.go:81-101), else
 * MFH_ERR_SHAPE_MISMATCH; a negative dimension is MFH_ERR_SHAPE_INVALID.
 * Float32 / Float16 / BFloat16 are stored as given.  Float8E4M3, Float8E5M2
 * and Int4 are dequantised on the device (BytesToBFloat16,
 * dtype/convert/convert.go:155) and stored as BFloat16, which the returned
 * tensor's dtype reports, as the contract allows (tensor/backend.go:11-14).
 * Returns when the data is resident. */
int mfh_backend_upload(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t source_dtype,
                       const void* bytes, size_t n_bytes, mfh_tensor** tensor);

/* Backend.UploadAsync: the same, returning once every chunk is queued; the
 * tensor is MFH_STATE_PENDING until its DMA (and dequant) finish.  `bytes`
 * may be reused as soon as the call returns. */
int mfh_backend_upload_async(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t source_dtype,
                             const void* bytes, size_t n_bytes, mfh_tensor** tensor);

/* Backend.UploadSparse: MFH_ERR_LAYOUT_UNSUPPORTED (dense only). */
int mfh_backend_upload_sparse(mfh_backend* backend);

/* Scaled dequantising upload, the optional capability a caller type-asserts
 * like axpyDevice (no counterpart in tensor.Backend): FP8 codes times one f32
 * scale (mfh_dequant_fp8), or Int4 nibbles times per-group scales
 * (mfh_dequant_int4; `group_scales` is host memory of
 * ceil(elements / group) values of `scale_dtype`, staged chunk by chunk with
 * the nibbles they scale through the backend's pinned ring, so the upload
 * allocates nothing besides the tensor).  Stored as `out_dtype` (Float32,
 * Float16 or BFloat16). */
int mfh_backend_upload_fp8(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t fp8_dtype,
                           const void* codes, size_t n_bytes, float scale, uint8_t out_dtype, mfh_tensor** tensor);
int mfh_backend_upload_int4(mfh_backend* backend, const int64_t* shape, int32_t rank, const void* packed,
                            size_t n_bytes, const void* group_scales, uint8_t scale_dtype, int64_t group,
                            uint8_t out_dtype, mfh_tensor** tensor);

/* The same uploads with UploadAsync's return: once the source bytes (and the
 * group scales) have been copied into the staging ring and every chunk is
 * queued, so the host buffers may be reused; the tensor is
 * MFH_STATE_PENDING until its last chunk has been dequantised.  Uploads
 * queued back to back share one staging pipeline: the copy of a tensor's
 * first chunk overlaps the DMA and dequant of the previous tensor's last. */
int mfh_backend_upload_fp8_async(mfh_backend* backend, const int64_t* shape, int32_t rank, uint8_t fp8_dtype,
                                 const void* codes, size_t n_bytes, float scale, uint8_t out_dtype,
                                 mfh_tensor** tensor);
int mfh_backend_upload_int4_async(mfh_backend* backend, const int64_t* shape, int32_t rank, const void* packed,
                                  size_t n_bytes, const void* group_scales, uint8_t scale_dtype, int64_t group,
                                  uint8_t out_dtype, mfh_tensor** tensor);

/* Backend.Download (tensor/backend.go:59): waits for the tensor, copies its
 * storage to `dst` (capacity `dst_bytes`) and reports the storage dtype and
 * byte count.  Tensor.RawBytes goes through it. */
int mfh_backend_download(mfh_backend* backend, const mfh_tensor* tensor, uint8_t* dtype, void* dst,
                         size_t dst_bytes, size_t* n_bytes);

/* Backend.Close: waits for queued work and frees the storage of every
 * tensor of the backend; those tensors then fail with MFH_ERR_TENSOR_CLOSED
 * and the backend with MFH_ERR_CLOSED.  Idempotent.  mfh_backend_release
 * frees the handle itself (closing first). */
int mfh_backend_close(mfh_backend* backend);
int mfh_backend_release(mfh_backend* backend);

/* ---- tensor.Tensor ---------------------------------------------------------- */

uint8_t mfh_tensor_dtype(const mfh_tensor* tensor);
int64_t mfh_tensor_len(const mfh_tensor* tensor);
int64_t mfh_tensor_bytes(const mfh_tensor* tensor);
/* Rank; copies up to `cap` dimensions. */
int32_t mfh_tensor_shape(const mfh_tensor* tensor, int64_t* dims, int32_t cap);
const char* mfh_tensor_location(const mfh_tensor* tensor);
int32_t mfh_tensor_state(const mfh_tensor* tensor);

/* DispatchPointer (runtime/axpy.go:17-20): the device address of element 0;
 * NULL once closed. */
void* mfh_tensor_dispatch_pointer(const mfh_tensor* tensor);

/* Tensor.Sync: waits for pending work on the tensor, on whichever backend's
 * stream it was queued; reports the sticky error (mfh_axpy has no error
 * channel) of the tensor's backend stream, else of the stream whose resident
 * axpy last wrote it. */
int mfh_tensor_sync(mfh_tensor* tensor);

/* Tensor.Slice (1-D zero-copy view of `length` elements from `start`) and
 * Tensor.Reshape (metadata view, same element count, else
 * MFH_ERR_SHAPE_MISMATCH).  Views share the parent's storage; closing the
 * parent invalidates them.  Release views like tensors. */
int mfh_tensor_slice(const mfh_tensor* tensor, int64_t start, int64_t length, mfh_tensor** view);
int mfh_tensor_reshape(const mfh_tensor* tensor, const int64_t* dims, int32_t rank, mfh_tensor** view);

/* Tensor.Close: waits for the device to finish every queued use, then
 * returns the storage this tensor owns to its backend.  The backend keeps up
 * to 2 GiB of such blocks for later tensors of the same byte size (an
 * upload then skips hipMalloc) and frees them when an allocation fails and
 * at mfh_backend_close.  Idempotent.  mfh_tensor_release also frees the
 * handle. */
int mfh_tensor_close(mfh_tensor* tensor);
int mfh_tensor_release(mfh_tensor* tensor);

/* ---- runtime ------------------------------------------------------------------- */

/* axpyOntoResident (runtime/axpy.go:44-93): y <- y + alpha*x for two tensors
 * of this backend, after the reference's checks and with its messages
 * ("math.axpy: tensor location does not match backend", "... y dtype %s does
 * not match x dtype %s", "... y length %d does not match x length %d"), then
 * axpyDevice.Axpy on the backend stream.  y and x may be held by other
 * backends: the launch waits for work still queued on either, and their
 * owners' Download, Sync, Close and shutdown wait for it.  Asynchronous;
 * Sync or Download observes the result. */
int mfh_axpy_onto_resident(mfh_backend* backend, mfh_tensor* y, const mfh_tensor* x, float alpha);

/* runtime.Backend.CallGraph (runtime/executor.go:22-27, GraphCallRequest and
 * GraphCallResult at :52-72) over resident tensors: binds inputs[k] to graph
 * input input_names[k], allocates for each output_keys[j] a flat tensor of
 * this backend with the dtype and length the call gives that key
 * (mfh_graph_output_shape), and queues mfh_graph_call on the backend stream.
 * Inputs may be held by other backends and may still be pending: the call
 * waits for work queued on them, and their owners' Download, Sync, Close and
 * shutdown wait for the call.  Returns once the call is queued, with every
 * output MFH_STATE_PENDING until it has run; Sync or Download observes the
 * results.  On error no output is returned (outputs[j] == NULL) and nothing
 * stays allocated.  The graph must not be called from two threads at once
 * (mfh_graph_call). */
int mfh_backend_graph_call(mfh_backend* backend, mfh_graph* graph, const char* const* input_names,
                           const mfh_tensor* const* inputs, int32_t n_inputs, const char* const* output_keys,
                           int32_t n_outputs, mfh_tensor** outputs);

#ifdef __cplusplus
}
#endif
#endif /* MFH_BACKEND_H */
