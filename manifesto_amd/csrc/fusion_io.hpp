// fusion_io.hpp — operand loads and result stores for JIT-compiled fused
// kernels (the third part of their text prelude, after codec.hpp and
// devmath.hpp).  A vector is 8 consecutive elements: one 16-byte load or
// store for 16-bit storage, two for f32.  Decoding follows BytesToFloat32
// (dtype/convert/convert.go:85-146); encoding follows Float32AsDTypeBytes
// (runtime/session.go:431-451).
#ifndef MFH_FUSION_IO_HPP
#define MFH_FUSION_IO_HPP

typedef mfh_u32 mfh_u32x4 __attribute__((ext_vector_type(4)));

MFH_DEV void mfh_ld8_f32(const void* p, mfh_i64 e, float* a)
{
    const mfh_u32x4* q = reinterpret_cast<const mfh_u32x4*>(static_cast<const float*>(p) + e);
    mfh_u32x4 x = q[0], y = q[1];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[k] = mfh_f32(x[k]);
        a[k + 4] = mfh_f32(y[k]);
    }
}

MFH_DEV void mfh_ld8_bf16(const void* p, mfh_i64 e, float* a)
{
    mfh_u32x4 x = *reinterpret_cast<const mfh_u32x4*>(static_cast<const mfh_u16*>(p) + e);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[2 * k] = mfh_f32(x[k] << 16);
        a[2 * k + 1] = mfh_f32(x[k] & 0xffff0000u);
    }
}

MFH_DEV void mfh_ld8_f16(const void* p, mfh_i64 e, float* a)
{
    mfh_u32x4 x = *reinterpret_cast<const mfh_u32x4*>(static_cast<const mfh_u16*>(p) + e);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[2 * k] = mfh_f16_to_f32(x[k] & 0xffffu);
        a[2 * k + 1] = mfh_f16_to_f32(x[k] >> 16);
    }
}

MFH_DEV float mfh_ld1_f32(const void* p, mfh_i64 i) { return static_cast<const float*>(p)[i]; }
MFH_DEV float mfh_ld1_bf16(const void* p, mfh_i64 i) { return mfh_bf16_to_f32(static_cast<const mfh_u16*>(p)[i]); }
MFH_DEV float mfh_ld1_f16(const void* p, mfh_i64 i) { return mfh_f16_to_f32(static_cast<const mfh_u16*>(p)[i]); }

MFH_DEV void mfh_st8_f32(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x4* q = reinterpret_cast<mfh_u32x4*>(static_cast<float*>(p) + e);
    mfh_u32x4 x = {mfh_bits(r[0]), mfh_bits(r[1]), mfh_bits(r[2]), mfh_bits(r[3])};
    mfh_u32x4 y = {mfh_bits(r[4]), mfh_bits(r[5]), mfh_bits(r[6]), mfh_bits(r[7])};
    q[0] = x;
    q[1] = y;
}

MFH_DEV void mfh_st8_bf16(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x4 x = {mfh_bf16x2_rne(r[0], r[1]), mfh_bf16x2_rne(r[2], r[3]),
                   mfh_bf16x2_rne(r[4], r[5]), mfh_bf16x2_rne(r[6], r[7])};
    *reinterpret_cast<mfh_u32x4*>(static_cast<mfh_u16*>(p) + e) = x;
}

MFH_DEV void mfh_st8_f16(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x4 x;
#pragma unroll
    for (int k = 0; k < 4; k++) x[k] = mfh_f16_rne(r[2 * k]) | (mfh_f16_rne(r[2 * k + 1]) << 16);
    *reinterpret_cast<mfh_u32x4*>(static_cast<mfh_u16*>(p) + e) = x;
}

MFH_DEV void mfh_st1_f32(void* p, mfh_i64 i, float v) { static_cast<float*>(p)[i] = v; }
MFH_DEV void mfh_st1_bf16(void* p, mfh_i64 i, float v) { static_cast<mfh_u16*>(p)[i] = (mfh_u16)mfh_bf16_rne(v); }
MFH_DEV void mfh_st1_f16(void* p, mfh_i64 i, float v) { static_cast<mfh_u16*>(p)[i] = (mfh_u16)mfh_f16_rne(v); }

#endif  // MFH_FUSION_IO_HPP
