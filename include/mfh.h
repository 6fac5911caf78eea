/*
 * mfh.h — C ABI of the MI355X (gfx950) backend for manifesto's data-parallel
 * hot path: fused elementwise chains, runtime host math (axpy, scalar
 * broadcast, linspace) and FP8 / Int4 / BF16 / F16 dequantisation.
 *
 * Plain pointers and sizes only.  Device pointers come from mfh_alloc (or any
 * hipMalloc'd memory); `stream` is a hipStream_t, NULL for the null stream.
 * Every launch is asynchronous on `stream`; mfh_stream_sync waits.
 *
 * dtype arguments are manifesto's wire codes (dtype/dtype.go:29-49):
 *   1 Float64, 2 Float32, 3 Float16, 4 BFloat16, 5 Float8E4M3, 6 Float8E5M2,
 *   7 Int64, 8 Int32, 9 Int16, 10 Int8, 11 Int4 (two per byte, low nibble
 *   first), 12 Uint64, 13 Uint32, 14 Uint16, 15 Uint8.
 *
 * Return codes: MFH_OK (0) or a negative MFH_ERR_*; mfh_last_error() gives the
 * calling thread's message.  Entry points that the reference declares without
 * an error channel (mfh_axpy mirrors axpyDevice.Axpy) record failures as a
 * sticky error of the stream the work was meant for, which that stream's
 * mfh_stream_sync (or mfh_take_sticky_error) reports, as the reference's
 * zero-host-sync rule requires (scripts/check_banned.sh:34-55).  Each stream
 * keeps its own: a thread syncing its stream never receives the failure of
 * work meant for another thread's stream.
 */
#ifndef MFH_H
#define MFH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MFH_OK 0
#define MFH_ERR_INVALID_ARGUMENT (-1)
#define MFH_ERR_DTYPE_UNSUPPORTED (-2) /* tensor.ErrDTypeUnsupported, tensor/errors.go:18 */
#define MFH_ERR_SHAPE_MISMATCH (-3)    /* tensor.ErrShapeMismatch, tensor/errors.go:28 */
#define MFH_ERR_DEVICE (-4)            /* a HIP runtime call failed */
#define MFH_ERR_COMPILE (-5)           /* hiprtc rejected a generated kernel */
#define MFH_ERR_NOT_INITIALIZED (-6)   /* mfh_init was not called */
#define MFH_ERR_CLOSED (-7)            /* tensor.ErrBackendClosed, tensor/errors.go:46 */

/* ---- runtime: device, memory, streams ---------------------------------- */

/* Library version, major*10000 + minor*100 + patch. */
int mfh_version(void);

/* Binds the library to HIP device `device` and reads its properties.
 * Replaces the device-side construction behind tensor.Backend
 * (tensor/backend.go:18-68).  Idempotent for the same device. */
int mfh_init(int device);

/* Releases the JIT kernel cache; outstanding mfh_kernel handles become
 * invalid.  tensor.Backend.Close (tensor/backend.go:64-66). */
int mfh_shutdown(void);

/* Thread-local message of the last failing call on this thread. */
const char* mfh_last_error(void);

/* Returns and clears the first sticky error left on `stream` by entry points
 * without an error channel (mfh_axpy), making its message the calling
 * thread's last error; MFH_OK when there is none.  Needs no device. */
int mfh_take_sticky_error(void* stream);

/* Capabilities (tensor/backend.go:82-110): total device bytes, native
 * alignment in bytes, number of compute units. */
int mfh_capabilities(int64_t* max_bytes, int32_t* native_alignment, int32_t* compute_units);

/* Device storage for one tensor (tensor.Backend.Upload allocates, Tensor.Close
 * releases: tensor/backend.go:40, tensor/tensor.go:75). */
int mfh_alloc(void** ptr, size_t bytes);
int mfh_free(void* ptr);

/* Host<->device copies behind Upload / Download / Tensor.RawBytes
 * (tensor/backend.go:40,59; tensor/tensor.go:109). */
int mfh_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int mfh_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);

/* Waits for `stream`; reports the stream's pending sticky error.
 * Tensor.Sync (tensor/tensor.go:114). */
int mfh_stream_sync(void* stream);

/* Launch shape of one family of streaming kernels: workgroups per compute
 * unit (the grid is also capped by the work itself, so a large value gives a
 * one-shot grid, one workgroup per chunk) and work items per thread per step
 * (1, 2 or 4).  `kernel` is "fp8", "int4", "axpy", "axpy16", "convert" or
 * "fused"; 0 keeps the current setting and -1 restores the default.  Defaults
 * are measured on MI355X and can also be set with MFH_BPC_<KERNEL> /
 * MFH_UNROLL_<KERNEL>.  "convert" reports 0 items per thread by default:
 * each cast picks its own (2 where the output is four times the source, else
 * 1; 4 runs as 2).  For "fused" the items per thread apply to kernels
 * compiled afterwards.  A deployment knob with no counterpart in the
 * reference; results do not depend on it. */
int mfh_set_launch_config(const char* kernel, int32_t blocks_per_cu, int32_t items_per_thread);
int mfh_get_launch_config(const char* kernel, int32_t* blocks_per_cu, int32_t* items_per_thread);

/* Threads per workgroup of a kernel family, the third part of its launch
 * shape.  "fp8", "axpy", "axpy16" and "convert" run 64, 128 or 256, "int4"
 * also 512 (defaults 128, 64, 64 and 512; "convert" picks per cast: 64 unless the
 * output is four times the source, then 256; its element-by-element
 * fallbacks for misaligned buffers keep 256); "fused" takes any
 * power of two from 64 to 1024 and applies it to kernels compiled afterwards
 * (default 64, one wave).  The defaults are the fastest sizes measured on
 * MI355X.  0 keeps the current setting and -1 restores the default; also
 * settable with MFH_THREADS_<KERNEL>.  mfh_get_launch_threads reports 0 for
 * "fused" and "convert" while they choose per kernel or per cast.  No
 * counterpart in the reference; results do not depend on it. */
int mfh_set_launch_threads(const char* kernel, int32_t threads);
int mfh_get_launch_threads(const char* kernel, int32_t* threads);

/* ---- runtime host math -------------------------------------------------- */

/* y <- y + alpha*x in place over `count` elements of storage dtype `dtype`
 * (Float32, Float16 or BFloat16), the product rounded to f32 before the add
 * and the sum re-encoded with round-to-nearest-even.  Same signature and
 * contract as axpyDevice.Axpy (runtime/axpy.go:13-15), called where
 * axpyOntoResident dispatches (runtime/axpy.go:84-90); the host loop it
 * replaces is runtime/axpy.go:115-117 and :145-147.  No return value: errors
 * are sticky on `stream`. */
void mfh_axpy(void* y, const void* x, int64_t count, float alpha, uint8_t dtype, void* stream);

/* out[i] = in[i] op scalar, op 0 add, 1 sub, 2 mul, 3 div, computed in f32
 * after decoding `in_dtype`, stored as `out_dtype` (Float32/Float16/BFloat16).
 * Division by zero and unknown ops are rejected like applyScalarBroadcast
 * (runtime/executor_math.go:195-234). */
int mfh_scalar_broadcast(void* out, uint8_t out_dtype, const void* in, uint8_t in_dtype,
                         int64_t count, float scalar, int32_t op, void* stream);

/* out[i] = start + i*step, step = (stop-start)/intervals in f32, endpoints
 * pinned when endpoint != 0.  runLinspace (runtime/executor_math.go:57-108). */
int mfh_linspace(void* out, uint8_t out_dtype, int64_t count, float start, float stop,
                 int32_t endpoint, void* stream);

/* ---- dtype conversion and dequantisation -------------------------------- */

/* Element-wise conversion of `count` logical elements from `in_dtype` to
 * `out_dtype` (Float64, Float32, Float16, BFloat16, Float8E4M3, Float8E5M2,
 * Int8 or Int4) with the reference's exact bit rules: BytesToFloat32
 * (dtype/convert/convert.go:85-146) followed, for 16-bit outputs, by
 * BytesToBFloat16 / BytesToFloat16 narrowing (:155-188) and, for FP8 outputs,
 * by BytesToFloat8E4M3 / BytesToFloat8E5M2 (:194-232: NewF8E4M3FromFloat32 /
 * NewF8E5M2FromFloat32, dtype/fp8.go:77-136, 190-249, saturating
 * round-to-nearest-even as the reference writes it); BytesToFloat64
 * (:36-79: float64 of each dtype's decode, a NaN quieted with its payload as
 * amd64's cvtss2sd does); BytesToInt8 (:235-263: the f64 value saturated to
 * [-128, 127], then truncated toward zero; NaN, which Go leaves to the
 * platform, gives 0 as on amd64 and arm64); Int4: that int8 value through
 * int4Encode (dtype/int4.go:60-70, clamped to [-8, 7]) packed low nibble
 * first into (count + 1) / 2 bytes, an odd count's last high nibble 0.
 * in_dtype may be any numeric code including Int4 (count nibbles). */
int mfh_convert(void* out, uint8_t out_dtype, const void* in, uint8_t in_dtype,
                int64_t count, void* stream);

/* FP8 (Float8E4M3 or Float8E5M2) -> out_dtype with a per-tensor f32 scale:
 * out = encode(fl32(decode(q) * scale)).  decode is F8E4M3.Float32 /
 * F8E5M2.Float32 (dtype/fp8.go:39-70,149-183); the scale has no counterpart
 * in the reference (BytesToBFloat16, dtype/convert/convert.go:155, is the
 * scale == 1 case).  A NaN code stays the reference's NaN; a NaN scale
 * propagates quieted; Inf*0 gives 0xffc00000 before narrowing. */
int mfh_dequant_fp8(void* out, uint8_t out_dtype, const void* in, uint8_t fp8_dtype,
                    int64_t count, float scale, void* stream);

/* Packed signed Int4 (decodeInt4ToFloat64, dtype/convert/decoders.go:262-289)
 * -> out_dtype with one scale per `group` consecutive elements:
 * out[i] = encode(fl32(q[i]) * scales[i / group]); scale_dtype is Float32,
 * Float16 or BFloat16.  The group scale has no counterpart in the reference
 * (OperationDequant4, ir/operation.go:158, names the device op). */
int mfh_dequant_int4(void* out, uint8_t out_dtype, const void* packed, int64_t count,
                     const void* scales, uint8_t scale_dtype, int64_t group, void* stream);

/* ---- fused elementwise chains ------------------------------------------- */

/* One FusionAST node (optimizer/fusion_ast.go:70-76).  A FusionAST crosses the
 * ABI as the pre-order list of its nodes; each node's children follow it, their
 * number fixed by NodeType.Arity (optimizer/fusion_ast.go:168-180).  `type` is
 * the optimizer.NodeType value: 1 Input, 2 Constant, 3 Add, 4 Sub, 5 Mul,
 * 6 Div, 7 Max, 8 Min, 9 Neg, 10 Abs, 11 Sqrt, 12 Exp, 13 Log, 14 ReLU,
 * 15 Sigmoid, 16 Tanh, 17 Silu, 18 Gelu, 19 LeakyReLU. */
typedef struct {
    int32_t type;
    int32_t input_index; /* Input: index into the input list */
    double value;        /* Constant: the literal, rounded to f32 when used */
} mfh_ast_node;

/* How a kernel input is read.  MFH_OPERAND_FULL: one value per element, as
 * CPUKernel.Run requires (codegen/cpu.go:78-85).  MFH_OPERAND_PERIODIC:
 * `period` values, element i reads index i % period (a row-broadcast bias).
 * MFH_OPERAND_SCALAR: one value read by every element.  The last two are new;
 * they give the same results as a pre-expanded FULL input. */
#define MFH_OPERAND_FULL 0
#define MFH_OPERAND_PERIODIC 1
#define MFH_OPERAND_SCALAR 2

typedef struct {
    uint8_t dtype; /* Float32, Float16 or BFloat16 storage */
    uint8_t mode;  /* MFH_OPERAND_* */
    uint8_t reserved[6];
    int64_t period; /* MFH_OPERAND_PERIODIC only */
} mfh_operand;

/* Transcendental nodes evaluated in f64 exactly as codegen/cpu.go:172-200
 * writes them (bit-identical to the reference but for f64 rounding ties).
 * Sigmoid, Silu and Gelu take f64 forms with about two thirds of the
 * reference's instructions, whose result is used where a test shows that it
 * rounds to the same f32 as the reference's value; the elements the test
 * cannot decide (about one in 2^13) are recomputed with the reference's
 * formulas.  Without it, chains that stream f32 take the same forms, and
 * chains of 16-bit operands f32 Silu and Gelu within 2 ulp and an f64
 * Sigmoid within 1. */
#define MFH_FUSION_PRECISE 1u

/* Sigmoid, Silu and Gelu in the fast forms of chains of 16-bit operands in
 * every chain (Silu and Gelu in f32 with the rounding of 1 + E left in the
 * quotient, within the 2-ulp node budget; Sigmoid in f64 within 1 ulp).
 * Without it a chain that streams f32 (an f32 output or a full or periodic
 * f32 operand), whose results show every f32 ulp of the node, evaluates them
 * as MFH_FUSION_PRECISE does, the reference's values at about twice the
 * instructions.  For measuring the 16-bit chains' forms over f32 results; no
 * counterpart in the reference. */
#define MFH_FUSION_SHORT_QUOTIENT 2u

/* With MFH_FUSION_PRECISE: every element through the reference's formulas,
 * without the rounding test.  The results are the same, at about twice the
 * instructions; for checking the test.  No counterpart in the reference. */
#define MFH_FUSION_NO_ROUNDING_TEST 4u

typedef struct mfh_kernel mfh_kernel;

/* EmitHIP: validates the tree, generates one HIP kernel for it (single pass
 * over HBM, inputs decoded and output encoded in registers) and compiles it
 * for gfx950 with hiprtc, cached by source.  The codegen target beside
 * EmitCPU / EmitMetal (codegen/cpu.go:97, codegen/metal.go:79) selected
 * through EmitFusion (codegen/codegen.go:68-99).  `output_port` names the
 * kernel like metalKernelName (codegen/metal.go:281-290); may be NULL. */
int mfh_fusion_compile(const mfh_ast_node* nodes, int32_t n_nodes, const mfh_operand* inputs,
                       int32_t n_inputs, uint8_t out_dtype, const char* output_port,
                       uint32_t flags, mfh_kernel** kernel);

/* HIPKernel.Source / KernelName / Identifier, like MetalKernel
 * (codegen/metal.go:35-56): the identifier is the output port ("anon" when
 * none was given).  The strings live until mfh_fusion_release. */
const char* mfh_fusion_source(const mfh_kernel* kernel);
const char* mfh_fusion_kernel_name(const mfh_kernel* kernel);
const char* mfh_fusion_identifier(const mfh_kernel* kernel);
int32_t mfh_fusion_num_inputs(const mfh_kernel* kernel);

/* Runs the kernel over `count` elements: CPUKernel.Run (codegen/cpu.go:59-90)
 * with device buffers.  `inputs` holds one device pointer per declared input;
 * a wrong count fails like the reference ("expects N inputs, got M"). */
int mfh_fusion_launch(const mfh_kernel* kernel, const void* const* inputs, int32_t n_inputs,
                      void* out, int64_t count, void* stream);

int mfh_fusion_release(mfh_kernel* kernel);

/* A directory where compiled kernels are kept between processes (no
 * counterpart in the reference, whose CPU and Metal kernels need no compile
 * step; for processes that would otherwise pay hiprtc's 0.3-2 s per distinct
 * kernel at every start).  A compile first looks for a file written by an
 * identical earlier compile (same hiprtc version, options and source text,
 * checked byte for byte) and otherwise writes one.  NULL or "" turns it off.
 * Default: the MFH_KERNEL_CACHE_DIR environment variable, else off.  The
 * directory must exist and be trusted like any code the process loads. */
int mfh_fusion_cache_dir(const char* dir);

/* Kernels compiled by hiprtc and kernels read from the cache directory since
 * the process started. */
int mfh_fusion_cache_stats(int64_t* compiles, int64_t* disk_hits);

#ifdef __cplusplus
}
#endif
#endif /* MFH_H */
