/*
 * oracle.c — CPU restatement of manifesto's Go hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it; the product library never does.
 *
 * Parity pins (what fixes each function beyond this restatement) are
 * exercised by tests/test_oracle_*.py: golden vectors from the reference's
 * tests, closed forms over every FP8 / Int4 / F16 code, library narrowings
 * (numpy, torch) for BF16 / F16 encode, scaled FP8 dequant and 16-bit axpy,
 * numpy's f64 conversion for wide integers, and hand-derived tables for the
 * FP8 encoders' subnormal quirks.  One function is
 * "parity unpinned" in its last bit: the f64 transcendentals inside the
 * evaluator (glibc exp/log/tanh here, Go's math.Exp/Log/Tanh in the
 * reference); both are sub-ulp accurate in f64, so the f32 results agree
 * except where an f64->f32 rounding tie falls between the two libraries.
 *
 * Compile with -O2 -ffp-contract=off (no FMA contraction, as Go/amd64 v1).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t f64_bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double bits_f64(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* ------------------------------------------------------------------------ */
/* FP8.  dtype/fp8.go                                                        */
/* ------------------------------------------------------------------------ */

/* F8E4M3.Float32, dtype/fp8.go:39-70.  OCP E4M3: S.1111.111 is NaN (quiet,
 * sign kept), no infinities, subnormals normalised by shifting. */
float orc_e4m3_to_f32(uint8_t code)
{
    uint32_t sign = (uint32_t)(code >> 7) << 31;
    if ((code & 0x7f) == 0x7f) return bits_f32(sign | 0x7fc00000u);
    if ((code & 0x7f) == 0) return bits_f32(sign);
    int32_t exponent = (code >> 3) & 0x0f;
    uint32_t mantissa = code & 0x07;
    if (exponent == 0) {
        int32_t shift = 0;
        while ((mantissa & 0x08) == 0) { mantissa <<= 1; shift++; }
        mantissa &= 0x07;
        exponent = 1 - shift;
    }
    int32_t biased = exponent - 7 + 127;
    return bits_f32(sign | ((uint32_t)biased << 23) | (mantissa << 20));
}

/* F8E5M2.Float32, dtype/fp8.go:149-183.  IEEE-like: exponent 0x1f with a zero
 * mantissa is Inf, otherwise a quiet NaN carrying the mantissa at bit 21. */
float orc_e5m2_to_f32(uint8_t code)
{
    uint32_t sign = (uint32_t)(code >> 7) << 31;
    int32_t exponent = (code >> 2) & 0x1f;
    uint32_t mantissa = code & 0x03;
    if (exponent == 0x1f) {
        if (mantissa == 0) return bits_f32(sign | 0x7f800000u);
        return bits_f32(sign | 0x7fc00000u | (mantissa << 21));
    }
    if (exponent == 0) {
        if (mantissa == 0) return bits_f32(sign);
        int32_t shift = 0;
        while ((mantissa & 0x04) == 0) { mantissa <<= 1; shift++; }
        mantissa &= 0x03;
        exponent = 1 - shift;
    }
    int32_t biased = exponent - 15 + 127;
    return bits_f32(sign | ((uint32_t)biased << 23) | (mantissa << 21));
}

/* roundToNearestEven, dtype/fp8.go:263-284. */
static uint32_t rne_truncated(uint32_t truncated, uint32_t full, uint32_t shift)
{
    if (shift == 0) return truncated;
    uint32_t dropped = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (dropped < half) return truncated;
    if (dropped > half) return truncated + 1;
    if (truncated & 1u) return truncated + 1;
    return truncated;
}

/* NewF8E4M3FromFloat32, dtype/fp8.go:77-136, restated bug-for-bug: the
 * reference saturates every value whose unbiased exponent is 8 (256..448) to
 * 0x7e, and its subnormal branch shifts by 20-exponent. */
uint8_t orc_f32_to_e4m3(float value)
{
    if (isnan(value)) return 0x7f;
    uint8_t sign = 0;
    if (signbit(value)) { sign = 0x80; value = -value; }
    if (isinf(value) || value > 448.0f) return sign | 0x7e;
    if (value == 0) return sign;
    uint32_t bits = f32_bits(value);
    int32_t exponent = (int32_t)((bits >> 23) & 0xff) - 127 + 7;
    uint32_t mantissa = bits & 0x7fffff;
    if (exponent <= 0) {
        if (exponent < -3) return sign;
        uint32_t shift = (uint32_t)(20 - exponent);
        uint32_t full = (mantissa | 0x800000u) >> shift;
        uint32_t rounded = rne_truncated(full, mantissa | 0x800000u, shift);
        if (rounded >= 0x08) return sign | 0x08;
        return sign | (uint8_t)rounded;
    }
    if (exponent >= 15) return sign | 0x7e;
    uint32_t mantissa8 = mantissa >> 20;
    uint32_t rounded = rne_truncated(mantissa8, mantissa, 20);
    if (rounded >= 0x08) {
        mantissa8 = 0;
        exponent++;
        if (exponent >= 15) return sign | 0x7e;
    } else {
        mantissa8 = rounded;
    }
    return (uint8_t)(sign | (uint8_t)((uint8_t)exponent << 3) | (uint8_t)mantissa8);
}

/* NewF8E5M2FromFloat32, dtype/fp8.go:190-249 (same structure, bias 15,
 * overflow to +-Inf 0x7c/0xfc). */
uint8_t orc_f32_to_e5m2(float value)
{
    if (isnan(value)) return 0x7f;
    uint8_t sign = 0;
    if (signbit(value)) { sign = 0x80; value = -value; }
    if (isinf(value) || value > 57344.0f) return sign | 0x7c;
    if (value == 0) return sign;
    uint32_t bits = f32_bits(value);
    int32_t exponent = (int32_t)((bits >> 23) & 0xff) - 127 + 15;
    uint32_t mantissa = bits & 0x7fffff;
    if (exponent <= 0) {
        if (exponent < -1) return sign;
        uint32_t shift = (uint32_t)(21 - exponent);
        uint32_t full = (mantissa | 0x800000u) >> shift;
        uint32_t rounded = rne_truncated(full, mantissa | 0x800000u, shift);
        if (rounded >= 0x04) return sign | 0x04;
        return sign | (uint8_t)rounded;
    }
    if (exponent >= 0x1f) return sign | 0x7c;
    uint32_t mantissa8 = mantissa >> 21;
    uint32_t rounded = rne_truncated(mantissa8, mantissa, 21);
    if (rounded >= 0x04) {
        mantissa8 = 0;
        exponent++;
        if (exponent >= 0x1f) return sign | 0x7c;
    } else {
        mantissa8 = rounded;
    }
    return (uint8_t)(sign | (uint8_t)((uint8_t)exponent << 2) | (uint8_t)mantissa8);
}

void orc_f32_to_fp8_buf(const float* in, int64_t n, int fmt, uint8_t* out)
{
    for (int64_t i = 0; i < n; i++) out[i] = fmt == 5 ? orc_f32_to_e4m3(in[i]) : orc_f32_to_e5m2(in[i]);
}

/* ------------------------------------------------------------------------ */
/* BF16.  dtype/bfloat16.go                                                  */
/* ------------------------------------------------------------------------ */

/* NewBfloat16FromFloat32, dtype/bfloat16.go:41-55: NaN keeps its top half and
 * gains the quiet bit 0x0040; everything else rounds to nearest even by adding
 * 0x7fff plus the kept LSB. */
uint16_t orc_f32_to_bf16(float value)
{
    uint32_t bits = f32_bits(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t rounded = bits + 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(rounded >> 16);
}

/* BF16.Float32, dtype/bfloat16.go:82-84. */
float orc_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

/* ------------------------------------------------------------------------ */
/* F16.  dtype/float16.go                                                    */
/* ------------------------------------------------------------------------ */

/* f16bitsToF32bits, dtype/float16.go:222-255. */
float orc_f16_to_f32(uint16_t in)
{
    uint32_t sign = (uint32_t)(in & 0x8000u) << 16;
    uint32_t exp = (uint32_t)(in & 0x7c00u) >> 10;
    uint32_t coef = (uint32_t)(in & 0x03ffu) << 13;
    if (exp == 0x1f) {
        if (coef == 0) return bits_f32(sign | 0x7f800000u | coef);
        return bits_f32(sign | 0x7fc00000u | coef);
    }
    if (exp == 0) {
        if (coef == 0) return bits_f32(sign);
        exp++;
        while ((coef & 0x7f800000u) == 0) { coef <<= 1; exp--; }
        coef &= 0x007fffffu;
    }
    return bits_f32(sign | ((exp + (0x7fu - 0xfu)) << 23) | coef);
}

/* f32bitsToF16bits, dtype/float16.go:261-315: RNE, overflow to Inf, NaN keeps
 * the top payload bits and sets 0x0200. */
uint16_t orc_f32_to_f16(float value)
{
    uint32_t u32 = f32_bits(value);
    uint32_t sign = u32 & 0x80000000u;
    uint32_t exp = u32 & 0x7f800000u;
    uint32_t coef = u32 & 0x007fffffu;
    if (exp == 0x7f800000u) {
        uint32_t nan_bit = coef != 0 ? 0x0200u : 0u;
        return (uint16_t)((sign >> 16) | 0x7c00u | nan_bit | (coef >> 13));
    }
    uint32_t half_sign = sign >> 16;
    int32_t unbiased = (int32_t)(exp >> 23) - 127;
    int32_t half_exp = unbiased + 15;
    if (half_exp >= 0x1f) return (uint16_t)(half_sign | 0x7c00u);
    if (half_exp <= 0) {
        if (14 - half_exp > 24) return (uint16_t)half_sign;
        uint32_t c = coef | 0x00800000u;
        uint32_t half_coef = c >> (uint32_t)(14 - half_exp);
        uint32_t round_bit = 1u << (uint32_t)(13 - half_exp);
        if ((c & round_bit) != 0 && (c & (3u * round_bit - 1u)) != 0) half_coef++;
        return (uint16_t)(half_sign | half_coef);
    }
    uint32_t u_half_exp = (uint32_t)half_exp << 10;
    uint32_t half_coef = coef >> 13;
    uint32_t round_bit = 0x00001000u;
    if ((coef & round_bit) != 0 && (coef & (3u * round_bit - 1u)) != 0)
        return (uint16_t)((half_sign | u_half_exp | half_coef) + 1u);
    return (uint16_t)(half_sign | u_half_exp | half_coef);
}

/* ------------------------------------------------------------------------ */
/* Int4.  dtype/int4.go:72-78, dtype/convert/decoders.go:262-289             */
/* ------------------------------------------------------------------------ */

/* Element 2k is the low nibble, 2k+1 the high nibble, both sign-extended by
 * an arithmetic shift of an int8 (decoders.go:282,285). */
int8_t orc_int4_lo(uint8_t packed) { return (int8_t)((int8_t)(uint8_t)(packed << 4) >> 4); }
int8_t orc_int4_hi(uint8_t packed) { return (int8_t)((int8_t)packed >> 4); }

/* ------------------------------------------------------------------------ */
/* Byte-buffer converters.  dtype/convert/convert.go, dtype/dtype.go         */
/* ------------------------------------------------------------------------ */

static int dtype_size(int dtype)
{
    /* DType.Size, dtype/dtype.go:57-75 (numeric dtypes only). */
    switch (dtype) {
    case ORC_FLOAT64: case ORC_INT64: case ORC_UINT64: return 8;
    case ORC_FLOAT32: case ORC_INT32: case ORC_UINT32: return 4;
    case ORC_FLOAT16: case ORC_BFLOAT16: case ORC_INT16: case ORC_UINT16: return 2;
    case ORC_F8E4M3: case ORC_F8E5M2: case ORC_INT8: case ORC_UINT8: return 1;
    default: return 0;
    }
}

/* DType.LogicalElements, dtype/dtype.go:105-134 (Int4 packs two per byte). */
int orc_logical_elements(int dtype, int64_t nbytes, int64_t* count)
{
    if (nbytes < 0) return -1;
    if (dtype == ORC_INT4) { *count = nbytes * 2; return 0; }
    int size = dtype_size(dtype);
    if (size == 0 || nbytes % size != 0) return -1;
    *count = nbytes / size;
    return 0;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t* p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static uint64_t rd64(const uint8_t* p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

/* float64(float32), as Go compiles it on amd64 (cvtss2sd): exact for every
 * number, a NaN keeps its sign and payload (shifted into the top of the f64
 * fraction) and is quieted.  Stated on the bits so the result does not depend
 * on the host's conversion of signalling NaNs. */
double orc_f32_to_f64(float value)
{
    uint32_t b = f32_bits(value);
    if ((b & 0x7fffffffu) > 0x7f800000u)
        return bits_f64(((uint64_t)(b >> 31) << 63) | 0x7ff8000000000000ull | ((uint64_t)(b & 0x7fffffu) << 29));
    return (double)value;
}

/* BytesToFloat64, dtype/convert/convert.go:36-79 and the per-dtype decoders in
 * dtype/convert/decoders.go: float64 of the Float32() decode for the 32-, 16-
 * and 8-bit float dtypes (decoders.go:44-124), float64(int) of the integers
 * (:126-260), the nibbles of Int4 (:262-289). */
int orc_bytes_to_f64(int dtype, const uint8_t* buf, int64_t nbytes, double* out)
{
    int64_t n;
    if (orc_logical_elements(dtype, nbytes, &n) != 0) return -1;
    for (int64_t i = 0; i < n; i++) {
        switch (dtype) {
        case ORC_FLOAT64: out[i] = bits_f64(rd64(buf + 8 * i)); break;
        case ORC_FLOAT32: out[i] = orc_f32_to_f64(bits_f32(rd32(buf + 4 * i))); break;
        case ORC_FLOAT16: out[i] = orc_f32_to_f64(orc_f16_to_f32(rd16(buf + 2 * i))); break;
        case ORC_BFLOAT16: out[i] = orc_f32_to_f64(orc_bf16_to_f32(rd16(buf + 2 * i))); break;
        case ORC_F8E4M3: out[i] = orc_f32_to_f64(orc_e4m3_to_f32(buf[i])); break;
        case ORC_F8E5M2: out[i] = orc_f32_to_f64(orc_e5m2_to_f32(buf[i])); break;
        case ORC_INT64: out[i] = (double)(int64_t)rd64(buf + 8 * i); break;
        case ORC_INT32: out[i] = (double)(int32_t)rd32(buf + 4 * i); break;
        case ORC_INT16: out[i] = (double)(int16_t)rd16(buf + 2 * i); break;
        case ORC_INT8: out[i] = (double)(int8_t)buf[i]; break;
        case ORC_UINT64: out[i] = (double)rd64(buf + 8 * i); break;
        case ORC_UINT32: out[i] = (double)rd32(buf + 4 * i); break;
        case ORC_UINT16: out[i] = (double)rd16(buf + 2 * i); break;
        case ORC_UINT8: out[i] = (double)buf[i]; break;
        case ORC_INT4: {
            uint8_t packed = buf[i / 2];
            out[i] = (double)((i & 1) ? orc_int4_hi(packed) : orc_int4_lo(packed));
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

/* BytesToFloat32, dtype/convert/convert.go:85-146: direct f32 decode for the
 * float dtypes, everything else through BytesToFloat64 and float32(). */
int orc_bytes_to_f32(int dtype, const uint8_t* buf, int64_t nbytes, float* out)
{
    int64_t n;
    if (orc_logical_elements(dtype, nbytes, &n) != 0) return -1;
    switch (dtype) {
    case ORC_FLOAT64:
        for (int64_t i = 0; i < n; i++) out[i] = (float)bits_f64(rd64(buf + 8 * i));
        return 0;
    case ORC_FLOAT32:
        for (int64_t i = 0; i < n; i++) out[i] = bits_f32(rd32(buf + 4 * i));
        return 0;
    case ORC_FLOAT16:
        for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(rd16(buf + 2 * i));
        return 0;
    case ORC_BFLOAT16:
        for (int64_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(rd16(buf + 2 * i));
        return 0;
    case ORC_F8E4M3:
        for (int64_t i = 0; i < n; i++) out[i] = orc_e4m3_to_f32(buf[i]);
        return 0;
    case ORC_F8E5M2:
        for (int64_t i = 0; i < n; i++) out[i] = orc_e5m2_to_f32(buf[i]);
        return 0;
    default: {
        double* wide = (double*)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
        if (!wide) return -1;
        int rc = orc_bytes_to_f64(dtype, buf, nbytes, wide);
        if (rc == 0)
            for (int64_t i = 0; i < n; i++) out[i] = (float)wide[i];
        free(wide);
        return rc;
    }
    }
}

/* int8(value) after BytesToInt8's saturation (dtype/convert/convert.go:
 * 235-263): below -128 gives -128, above 127 gives 127 (so -Inf and +Inf
 * saturate), everything else truncates toward zero.  A NaN passes both
 * comparisons; Go leaves int8(NaN) to the platform, and on amd64 (cvttsd2sl,
 * whose low byte of 0x80000000 is 0) and arm64 (fcvtzs) it is 0, which this
 * build states as the rule. */
int8_t orc_f64_to_i8(double value)
{
    if (isnan(value)) return 0;
    if (value < -128.0) return -128;
    if (value > 127.0) return 127;
    return (int8_t)value;
}

/* BytesToInt8, dtype/convert/convert.go:235-263: BytesToFloat64, then
 * orc_f64_to_i8 per element. */
int orc_bytes_to_i8(int dtype, const uint8_t* buf, int64_t nbytes, int8_t* out)
{
    int64_t n;
    if (orc_logical_elements(dtype, nbytes, &n) != 0) return -1;
    double* wide = (double*)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
    if (!wide) return -1;
    int rc = orc_bytes_to_f64(dtype, buf, nbytes, wide);
    if (rc == 0)
        for (int64_t i = 0; i < n; i++) out[i] = orc_f64_to_i8(wide[i]);
    free(wide);
    return rc;
}

/* BytesToBFloat16, dtype/convert/convert.go:155-169 (f32 then RNE). */
int orc_bytes_to_bf16(int dtype, const uint8_t* buf, int64_t nbytes, uint16_t* out)
{
    int64_t n;
    if (orc_logical_elements(dtype, nbytes, &n) != 0) return -1;
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!tmp) return -1;
    int rc = orc_bytes_to_f32(dtype, buf, nbytes, tmp);
    if (rc == 0) orc_f32_to_bf16_buf(tmp, n, out);
    free(tmp);
    return rc;
}

/* BytesToFloat16, dtype/convert/convert.go:174-188 (f32 then Fromfloat32). */
int orc_bytes_to_f16(int dtype, const uint8_t* buf, int64_t nbytes, uint16_t* out)
{
    int64_t n;
    if (orc_logical_elements(dtype, nbytes, &n) != 0) return -1;
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!tmp) return -1;
    int rc = orc_bytes_to_f32(dtype, buf, nbytes, tmp);
    if (rc == 0) orc_f32_to_f16_buf(tmp, n, out);
    free(tmp);
    return rc;
}

/* EncodeFloat32ToBF16 (dtype/bfloat16.go:166-181) / Float32AsDTypeBytes
 * (runtime/session.go:431-451). */
void orc_f32_to_bf16_buf(const float* in, int64_t n, uint16_t* out)
{
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_f32_to_f16_buf(const float* in, int64_t n, uint16_t* out)
{
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Scaled dequantisation (build-defined; the reference has no scale).        */
/* ------------------------------------------------------------------------ */

/* One IEEE f32 multiply with x86 SSE NaN rules made explicit, so the result
 * does not depend on how a compiler orders the operands: a NaN operand is
 * returned quieted (the decoded value first), and Inf*0 gives the x86 default
 * NaN 0xffc00000. */
static float scale_mul(float decoded, float scale)
{
    if (isnan(decoded)) return bits_f32(f32_bits(decoded) | 0x00400000u);
    if (isnan(scale)) return bits_f32(f32_bits(scale) | 0x00400000u);
    if ((isinf(decoded) && scale == 0.0f) || (decoded == 0.0f && isinf(scale)))
        return bits_f32(0xffc00000u);
    return decoded * scale;
}

static int store_encoded(void* out, int out_dtype, int64_t i, float v)
{
    switch (out_dtype) {
    case ORC_FLOAT32: ((float*)out)[i] = v; return 0;
    case ORC_BFLOAT16: ((uint16_t*)out)[i] = orc_f32_to_bf16(v); return 0;
    case ORC_FLOAT16: ((uint16_t*)out)[i] = orc_f32_to_f16(v); return 0;
    default: return -1;
    }
}

/* Reference CPU path for FP8: BytesToBFloat16(Float8E4M3, buf) is two serial
 * passes, decode to a fresh f32 slice (convert.go:121-131) then narrow each
 * value (convert.go:162-166).  The scale multiply sits in the second pass. */
int orc_dequant_fp8(const uint8_t* in, int64_t n, int fp8_dtype, float scale,
                    int out_dtype, void* out)
{
    if (fp8_dtype != ORC_F8E4M3 && fp8_dtype != ORC_F8E5M2) return -1;
    if (out_dtype != ORC_FLOAT32 && out_dtype != ORC_BFLOAT16 && out_dtype != ORC_FLOAT16) return -1;
    float* decoded = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!decoded) return -1;
    if (fp8_dtype == ORC_F8E4M3)
        for (int64_t i = 0; i < n; i++) decoded[i] = orc_e4m3_to_f32(in[i]);
    else
        for (int64_t i = 0; i < n; i++) decoded[i] = orc_e5m2_to_f32(in[i]);
    for (int64_t i = 0; i < n; i++) store_encoded(out, out_dtype, i, scale_mul(decoded[i], scale));
    free(decoded);
    return 0;
}

static float load_scale(const void* scales, int scale_dtype, int64_t g)
{
    switch (scale_dtype) {
    case ORC_FLOAT32: return ((const float*)scales)[g];
    case ORC_FLOAT16: return orc_f16_to_f32(((const uint16_t*)scales)[g]);
    case ORC_BFLOAT16: return orc_bf16_to_f32(((const uint16_t*)scales)[g]);
    default: return NAN;
    }
}

/* Reference CPU path for Int4: BytesToFloat32(Int4, buf) goes through a f64
 * slice (convert.go:135-145, decoders.go:262-289), then float32(), then the
 * group scale and the narrowing.  Element i uses scales[i / group]. */
int orc_dequant_int4(const uint8_t* packed, int64_t n, const void* scales,
                     int scale_dtype, int64_t group, int out_dtype, void* out)
{
    if (group <= 0) return -1;
    if (scale_dtype != ORC_FLOAT32 && scale_dtype != ORC_FLOAT16 && scale_dtype != ORC_BFLOAT16) return -1;
    if (out_dtype != ORC_FLOAT32 && out_dtype != ORC_BFLOAT16 && out_dtype != ORC_FLOAT16) return -1;
    double* wide = (double*)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
    if (!wide) return -1;
    for (int64_t b = 0; 2 * b < n; b++) {
        wide[2 * b] = (double)orc_int4_lo(packed[b]);
        if (2 * b + 1 < n) wide[2 * b + 1] = (double)orc_int4_hi(packed[b]);
    }
    for (int64_t i = 0; i < n; i++) {
        float q = (float)wide[i];
        store_encoded(out, out_dtype, i, scale_mul(q, load_scale(scales, scale_dtype, i / group)));
    }
    free(wide);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Fused-chain evaluator.  codegen/cpu.go:59-214, optimizer/fusion_ast.go   */
/* ------------------------------------------------------------------------ */

enum {
    N_INVALID = 0, N_INPUT, N_CONSTANT, N_ADD, N_SUB, N_MUL, N_DIV, N_MAX, N_MIN,
    N_NEG, N_ABS, N_SQRT, N_EXP, N_LOG, N_RELU, N_SIGMOID, N_TANH, N_SILU, N_GELU,
    N_LEAKY_RELU
};

/* NodeType.Arity, optimizer/fusion_ast.go:168-180. */
int orc_node_arity(int32_t type)
{
    switch (type) {
    case N_INPUT: case N_CONSTANT: return 0;
    case N_NEG: case N_ABS: case N_SQRT: case N_EXP: case N_LOG: case N_RELU:
    case N_SIGMOID: case N_TANH: case N_SILU: case N_GELU: case N_LEAKY_RELU: return 1;
    case N_ADD: case N_SUB: case N_MUL: case N_DIV: case N_MAX: case N_MIN: return 2;
    default: return -1;
    }
}

/* One-operand cases of evalCPU, codegen/cpu.go:164-208. */
float orc_eval_unary(int32_t type, float value)
{
    switch (type) {
    case N_NEG: return -value;
    case N_ABS: return value < 0 ? -value : value;
    case N_SQRT: return (float)sqrt((double)value);
    case N_EXP: return (float)exp((double)value);
    case N_LOG: return (float)log((double)value);
    case N_RELU: return value < 0 ? 0.0f : value;
    case N_SIGMOID: return (float)(1.0 / (1.0 + exp(-(double)value)));
    case N_TANH: return (float)tanh((double)value);
    case N_SILU: return (float)((double)value / (1.0 + exp(-(double)value)));
    case N_GELU: {
        /* math.Sqrt(2.0/math.Pi): Go evaluates the constant 2/pi exactly and
         * rounds it once to f64; 0x3FE45F306DC9C883 is that rounding. */
        const double two_over_pi = bits_f64(0x3FE45F306DC9C883ull);
        double v = (double)value;
        double inner = sqrt(two_over_pi) * (v + 0.044715 * v * v * v);
        return (float)(0.5 * v * (1.0 + tanh(inner)));
    }
    case N_LEAKY_RELU: return value >= 0 ? value : 0.01f * value;
    default: return 0.0f;
    }
}

/* Two-operand cases of evalCPU, codegen/cpu.go:132-163: f32 IEEE arithmetic,
 * select-based Max/Min (a NaN comparison picks the right operand). */
float orc_eval_binary(int32_t type, float l, float r)
{
    switch (type) {
    case N_ADD: return l + r;
    case N_SUB: return l - r;
    case N_MUL: return l * r;
    case N_DIV: return l / r;
    case N_MAX: return l > r ? l : r;
    case N_MIN: return l < r ? l : r;
    default: return 0.0f;
    }
}

typedef struct {
    const orc_node* nodes;
    int32_t* child0;
    int32_t* child1;
    const float* const* inputs;
    const int64_t* period;
} orc_tree;

/* evalCPU, codegen/cpu.go:126-214. */
static float eval_node(const orc_tree* t, int32_t idx, int64_t e)
{
    const orc_node* node = &t->nodes[idx];
    switch (node->type) {
    case N_INPUT: {
        int64_t p = t->period ? t->period[node->input_index] : 0;
        return t->inputs[node->input_index][p > 0 ? e % p : e];
    }
    case N_CONSTANT: return (float)node->value;
    default: break;
    }
    int arity = orc_node_arity(node->type);
    if (arity == 1) return orc_eval_unary(node->type, eval_node(t, t->child0[idx], e));
    if (arity == 2) {
        float l = eval_node(t, t->child0[idx], e);
        float r = eval_node(t, t->child1[idx], e);
        return orc_eval_binary(node->type, l, r);
    }
    return 0.0f; /* unknown node type: codegen/cpu.go:209-210 */
}

/* Parse the pre-order list into child links; returns the index just past the
 * subtree rooted at idx, or -1 if the list is malformed. */
static int32_t link_tree(const orc_node* nodes, int n, int32_t idx, int32_t* c0, int32_t* c1)
{
    if (idx >= n) return -1;
    int arity = orc_node_arity(nodes[idx].type);
    if (arity < 0) arity = 0;
    int32_t next = idx + 1;
    for (int k = 0; k < arity; k++) {
        if (k == 0) c0[idx] = next; else c1[idx] = next;
        next = link_tree(nodes, n, next, c0, c1);
        if (next < 0) return -1;
    }
    return next;
}

/* CPUKernel.Run, codegen/cpu.go:59-90.  Returns -1 for a malformed tree or an
 * input index outside [0, n_inputs). */
int orc_run(const orc_node* nodes, int n_nodes, const float* const* inputs,
            const int64_t* period, int n_inputs, float* out, int64_t count)
{
    if (n_nodes <= 0) return -1;
    int32_t* c0 = (int32_t*)calloc((size_t)n_nodes, sizeof(int32_t));
    int32_t* c1 = (int32_t*)calloc((size_t)n_nodes, sizeof(int32_t));
    if (!c0 || !c1) { free(c0); free(c1); return -1; }
    int rc = 0;
    if (link_tree(nodes, n_nodes, 0, c0, c1) != n_nodes) rc = -1;
    for (int i = 0; rc == 0 && i < n_nodes; i++)
        if (nodes[i].type == N_INPUT && (nodes[i].input_index < 0 || nodes[i].input_index >= n_inputs))
            rc = -1;
    if (rc == 0) {
        orc_tree t = {nodes, c0, c1, inputs, period};
        for (int64_t e = 0; e < count; e++) out[e] = eval_node(&t, 0, e);
    }
    free(c0);
    free(c1);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* axpy.  runtime/axpy.go                                                    */
/* ------------------------------------------------------------------------ */

/* axpyOntoHost []float32 case, runtime/axpy.go:115-117: y += alpha*x, the
 * product rounded before the add. */
void orc_axpy_f32(float* y, const float* x, int64_t n, float alpha)
{
    for (int64_t i = 0; i < n; i++) y[i] += alpha * x[i];
}

/* axpyOntoHost tensor case, runtime/axpy.go:120-161 with float32VectorBytes
 * (:171-194): decode both to f32, the same loop, re-encode to the storage
 * dtype. */
int orc_axpy_storage(void* y, const void* x, int64_t n, float alpha, int dtype)
{
    if (dtype == ORC_FLOAT32) { orc_axpy_f32((float*)y, (const float*)x, n, alpha); return 0; }
    if (dtype != ORC_BFLOAT16 && dtype != ORC_FLOAT16) return -1;
    uint16_t* yy = (uint16_t*)y;
    const uint16_t* xx = (const uint16_t*)x;
    for (int64_t i = 0; i < n; i++) {
        float yv = dtype == ORC_BFLOAT16 ? orc_bf16_to_f32(yy[i]) : orc_f16_to_f32(yy[i]);
        float xv = dtype == ORC_BFLOAT16 ? orc_bf16_to_f32(xx[i]) : orc_f16_to_f32(xx[i]);
        yv += alpha * xv;
        yy[i] = dtype == ORC_BFLOAT16 ? orc_f32_to_bf16(yv) : orc_f32_to_f16(yv);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Host math.  runtime/executor_math.go                                      */
/* ------------------------------------------------------------------------ */

/* applyScalarBroadcast, runtime/executor_math.go:195-234 (division by zero is
 * rejected, an unknown op is rejected). */
int orc_scalar_broadcast(const float* src, int64_t n, float scalar, int op, float* out)
{
    switch (op) {
    case 0: for (int64_t i = 0; i < n; i++) out[i] = src[i] + scalar; return 0;
    case 1: for (int64_t i = 0; i < n; i++) out[i] = src[i] - scalar; return 0;
    case 2: for (int64_t i = 0; i < n; i++) out[i] = src[i] * scalar; return 0;
    case 3:
        if (scalar == 0) return -1;
        for (int64_t i = 0; i < n; i++) out[i] = src[i] / scalar;
        return 0;
    default: return -1;
    }
}

/* runLinspace, runtime/executor_math.go:57-108: start + i*step in f32 with
 * both endpoints pinned when the stop is included. */
int orc_linspace(float start, float stop, int64_t count, int endpoint, float* out)
{
    if (count <= 0) return -1;
    if (count == 1) { out[0] = start; return 0; }
    int64_t intervals = endpoint ? count - 1 : count;
    float step = (stop - start) / (float)intervals;
    for (int64_t i = 0; i < count; i++) out[i] = start + (float)i * step;
    if (intervals == count - 1) { out[0] = start; out[count - 1] = stop; }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Constant folding.  optimizer/constant_fold.go:149-225                     */
/* ------------------------------------------------------------------------ */

/* Go's math.Max / math.Min: +Inf (resp. -Inf) wins over NaN, then NaN, then
 * signed-zero ordering. */
static double go_max(double x, double y)
{
    if ((isinf(x) && x > 0) || (isinf(y) && y > 0)) return INFINITY;
    if (isnan(x) || isnan(y)) return bits_f64(0x7FF8000000000001ull);
    if (x == 0 && x == y) return signbit(x) ? y : x;
    return x > y ? x : y;
}

static double go_min(double x, double y)
{
    if ((isinf(x) && x < 0) || (isinf(y) && y < 0)) return -INFINITY;
    if (isnan(x) || isnan(y)) return bits_f64(0x7FF8000000000001ull);
    if (x == 0 && x == y) return signbit(x) ? x : y;
    return x < y ? x : y;
}

int orc_fold(int32_t type, const double* ops, int n_ops, double* out)
{
    int arity = orc_node_arity(type);
    if (arity <= 0 || arity != n_ops) return 0;
    if (arity == 1) {
        double v = ops[0];
        switch (type) {
        case N_NEG: *out = -v; return 1;
        case N_ABS: *out = fabs(v); return 1;
        case N_SQRT: *out = sqrt(v); return 1;
        case N_EXP: *out = exp(v); return 1;
        case N_LOG: *out = log(v); return 1;
        case N_RELU: *out = v > 0 ? v : 0.0; return 1;
        case N_SIGMOID: *out = 1.0 / (1.0 + exp(-v)); return 1;
        case N_TANH: *out = tanh(v); return 1;
        case N_SILU: *out = v / (1.0 + exp(-v)); return 1;
        case N_GELU: {
            const double two_over_pi = bits_f64(0x3FE45F306DC9C883ull);
            double inner = sqrt(two_over_pi) * (v + 0.044715 * v * v * v);
            *out = 0.5 * v * (1.0 + tanh(inner));
            return 1;
        }
        case N_LEAKY_RELU: *out = v >= 0 ? v : 0.01 * v; return 1;
        default: return 0;
        }
    }
    double l = ops[0], r = ops[1];
    switch (type) {
    case N_ADD: *out = l + r; return 1;
    case N_SUB: *out = l - r; return 1;
    case N_MUL: *out = l * r; return 1;
    case N_DIV: if (r == 0) return 0; *out = l / r; return 1;
    case N_MAX: *out = go_max(l, r); return 1;
    case N_MIN: *out = go_min(l, r); return 1;
    default: return 0;
    }
}
