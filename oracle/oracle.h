/*
 * oracle.h — CPU restatement of manifesto's Go hot path (dtype codecs,
 * byte-buffer converters, the fused-chain evaluator, axpy, scalar broadcast,
 * linspace).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library (libmfh) never links,
 * loads or calls it.
 *
 * Every function cites the reference Go file:line it restates.  Build flags
 * are -O2 -ffp-contract=off: Go on amd64 with the default GOAMD64=v1 never
 * contracts a*b+c into an FMA, so neither does this restatement.
 *
 * dtype codes are manifesto's wire codes (dtype/dtype.go:29-49).
 */
#ifndef MANIFESTO_ORACLE_H
#define MANIFESTO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_FLOAT64 = 1, ORC_FLOAT32 = 2, ORC_FLOAT16 = 3, ORC_BFLOAT16 = 4,
    ORC_F8E4M3 = 5, ORC_F8E5M2 = 6, ORC_INT64 = 7, ORC_INT32 = 8,
    ORC_INT16 = 9, ORC_INT8 = 10, ORC_INT4 = 11, ORC_UINT64 = 12,
    ORC_UINT32 = 13, ORC_UINT16 = 14, ORC_UINT8 = 15
};

/* Scalar codecs. */
float    orc_e4m3_to_f32(uint8_t code);
float    orc_e5m2_to_f32(uint8_t code);
uint8_t  orc_f32_to_e4m3(float value);
uint8_t  orc_f32_to_e5m2(float value);
/* BytesToFloat8E4M3 / BytesToFloat8E5M2 after BytesToFloat32
 * (dtype/convert/convert.go:194-232): fmt 5 E4M3, 6 E5M2. */
void     orc_f32_to_fp8_buf(const float* in, int64_t n, int fmt, uint8_t* out);
uint16_t orc_f32_to_bf16(float value);
float    orc_bf16_to_f32(uint16_t bits);
float    orc_f16_to_f32(uint16_t bits);
uint16_t orc_f32_to_f16(float value);
int8_t   orc_int4_lo(uint8_t packed);
int8_t   orc_int4_hi(uint8_t packed);

/* Byte-buffer converters.  Return 0 on success, -1 on an unsupported dtype or
 * a byte count that is not a whole number of elements.  *count receives the
 * number of logical elements. */
int orc_logical_elements(int dtype, int64_t nbytes, int64_t* count);
int orc_bytes_to_f64(int dtype, const uint8_t* buf, int64_t nbytes, double* out);
int orc_bytes_to_f32(int dtype, const uint8_t* buf, int64_t nbytes, float* out);
int orc_bytes_to_bf16(int dtype, const uint8_t* buf, int64_t nbytes, uint16_t* out);
int orc_bytes_to_f16(int dtype, const uint8_t* buf, int64_t nbytes, uint16_t* out);
/* BytesToInt8 (dtype/convert/convert.go:235-263); NaN gives 0. */
int orc_bytes_to_i8(int dtype, const uint8_t* buf, int64_t nbytes, int8_t* out);
double orc_f32_to_f64(float value);
int8_t orc_f64_to_i8(double value);
void orc_f32_to_bf16_buf(const float* in, int64_t n, uint16_t* out);
void orc_f32_to_f16_buf(const float* in, int64_t n, uint16_t* out);

/* Scaled dequantisation.  The reference has no scale; the build defines
 * out = encode(fl32(decode(q)) * fl32(scale)) with one IEEE multiply. */
int orc_dequant_fp8(const uint8_t* in, int64_t n, int fp8_dtype, float scale,
                    int out_dtype, void* out);
int orc_dequant_int4(const uint8_t* packed, int64_t n, const void* scales,
                     int scale_dtype, int64_t group, int out_dtype, void* out);

/* Fused-chain evaluator.  Nodes are a pre-order flattening of the FusionAST:
 * children follow their parent, their number fixed by the node type's arity. */
typedef struct {
    int32_t type;         /* optimizer.NodeType value */
    int32_t input_index;  /* NodeInput only */
    double  value;        /* NodeConstant only */
} orc_node;

int orc_node_arity(int32_t type);
/* period[i] == 0: input i holds count values; period[i] == p > 0: input i
 * holds p values and element e reads input[i][e % p] (the same value the
 * reference reads from a pre-expanded copy). */
int orc_run(const orc_node* nodes, int n_nodes, const float* const* inputs,
            const int64_t* period, int n_inputs, float* out, int64_t count);
/* Single-node helpers for tests of the per-node formulas. */
float orc_eval_unary(int32_t type, float v);
float orc_eval_binary(int32_t type, float l, float r);

/* axpy. */
void orc_axpy_f32(float* y, const float* x, int64_t n, float alpha);
int  orc_axpy_storage(void* y, const void* x, int64_t n, float alpha, int dtype);

/* Host math. op: 0 add, 1 sub, 2 mul, 3 div. */
int orc_scalar_broadcast(const float* src, int64_t n, float scalar, int op, float* out);
int orc_linspace(float start, float stop, int64_t count, int endpoint, float* out);

/* Constant folding of one node type over f64 operands; returns 1 if folded. */
int orc_fold(int32_t type, const double* operands, int n_operands, double* out);

#ifdef __cplusplus
}
#endif
#endif
