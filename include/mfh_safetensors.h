/*
 * mfh_safetensors.h — C ABI of the SafeTensors weight reader and its
 * streaming loader onto the HIP backend.
 *
 * The index follows weights/reader.go:14-109 (IndexFile / IndexReader /
 * ReadTensor): an 8-byte little-endian header length, a JSON object mapping
 * tensor names to {dtype, shape, data_offsets} (plus an ignored
 * "__metadata__"), then the data; offsets are relative to the end of the
 * header.  dtype strings are read with dtype.Parse (dtype/dtype.go:242-287:
 * "F8_E4M3", "BF16", "I4", ...).
 *
 * mfh_safetensors_load streams one tensor from the file into device memory
 * through the backend's pinned staging ring (pread into a pinned chunk while
 * the previous chunk's DMA and dequant run) without reading the whole file
 * into host memory; FP8 / Int4 tensors arrive dequantised.
 * mfh_safetensors_load_async queues the same load and returns once the file
 * has been read.
 */
#ifndef MFH_SAFETENSORS_H
#define MFH_SAFETENSORS_H

#include "mfh_backend.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mfh_safetensors mfh_safetensors;

/* IndexFile: opens `path` and reads its header.  Malformed headers, offsets
 * outside the file and unknown dtypes fail with MFH_ERR_INVALID_ARGUMENT and
 * a "safetensors index: ..." message. */
int mfh_safetensors_open(const char* path, mfh_safetensors** file);
int mfh_safetensors_close(mfh_safetensors* file);

/* Byte offset where tensor data starts (header length + 8, the second
 * result of IndexReader) and the number of tensors. */
int64_t mfh_safetensors_data_base(const mfh_safetensors* file);
int32_t mfh_safetensors_count(const mfh_safetensors* file);

/* TensorMeta of entry `index` (in header order): name, dtype as written and
 * parsed, rank (dims copied up to `cap`), data_offsets. */
typedef struct {
    const char* name;
    const char* dtype_name;
    uint8_t dtype;
    uint8_t reserved[3];
    int32_t rank;
    int64_t begin;
    int64_t end;
} mfh_safetensors_meta;

int mfh_safetensors_entry(const mfh_safetensors* file, int32_t index, mfh_safetensors_meta* meta, int64_t* dims,
                          int32_t cap);

/* Index of tensor `name`, or -1. */
int32_t mfh_safetensors_find(const mfh_safetensors* file, const char* name);

/* ReadTensor: copies the raw bytes of `name` to host memory `dst`
 * ("safetensors: missing tensor %q" when absent). */
int mfh_safetensors_read(const mfh_safetensors* file, const char* name, void* dst, size_t dst_bytes,
                         size_t* n_bytes);

/* Streams tensor `name` onto `backend` as Backend.Upload would store it
 * (F32 / F16 / BF16 as written, F8_E4M3 / F8_E5M2 / I4 dequantised to BF16).
 * A non-NULL `scale_name` names a companion tensor (one element of F32, F16
 * or BF16) whose value scales an FP8 tensor; for an I4 tensor it names the
 * per-group scales, `group` elements each, which are read from the file
 * chunk by chunk beside the nibbles they scale.  A scale for an F32, F16 or
 * BF16 tensor is MFH_ERR_INVALID_ARGUMENT (those are stored as written);
 * other dtypes fail with MFH_ERR_DTYPE_UNSUPPORTED. */
int mfh_safetensors_load(const mfh_safetensors* file, const char* name, mfh_backend* backend,
                         const char* scale_name, int64_t group, mfh_tensor** tensor);

/* The same load as Backend.UploadAsync (tensor/backend.go:37-40) would make
 * it: returns once the file has been read and every chunk is queued, with
 * the tensor MFH_STATE_PENDING until its last DMA and dequant have run
 * (mfh_tensor_sync, mfh_backend_download and mfh_tensor_close wait for it).
 * Loads queued back to back keep the staging ring running across tensor
 * boundaries: the file read of one tensor's first chunk overlaps the DMA and
 * dequant of the previous tensor's last chunk, which a synchronous load
 * waits out. */
int mfh_safetensors_load_async(const mfh_safetensors* file, const char* name, mfh_backend* backend,
                               const char* scale_name, int64_t group, mfh_tensor** tensor);

#ifdef __cplusplus
}
#endif
#endif /* MFH_SAFETENSORS_H */
