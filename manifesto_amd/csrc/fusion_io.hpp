// fusion_io.hpp — operand loads and result stores for JIT-compiled fused
// kernels (the third part of their text prelude, after codec.hpp and
// devmath.hpp).  A work item is VEC consecutive elements, VEC = 8 when every
// operand and the output are 16-bit and VEC = 4 when any is f32, so each
// lane moves one contiguous 8- or 16-byte piece per operand and the pieces of
// neighbouring lanes are adjacent.  Decoding follows BytesToFloat32
// (dtype/convert/convert.go:85-146); encoding follows Float32AsDTypeBytes
// (runtime/session.go:431-451).  Vector stores are non-temporal
// (global_store ... nt): the results are streamed out, not re-read, and
// streaming stores measured 1-2% faster on read-heavy chains and up to 25%
// on write-heavy streams.
#ifndef MFH_FUSION_IO_HPP
#define MFH_FUSION_IO_HPP

typedef mfh_u32 mfh_u32x4 __attribute__((ext_vector_type(4)));
typedef mfh_u32 mfh_u32x2 __attribute__((ext_vector_type(2)));

// Vector loads take NT = 1 for a streamed operand of a kernel that reads at
// least as many bytes as it writes (non-temporal loads measured +4% on a 1:1
// stream and +8% on 2:1, but -10% on 1:2); operands re-read across the grid
// (periodic rows such as a bias) keep NT = 0.
template <int NT, typename T>
MFH_DEV T mfh_vld(const void* p)
{
    if constexpr (NT) return __builtin_nontemporal_load(static_cast<const T*>(p));
    else return *static_cast<const T*>(p);
}

// ---- 8-element items (16-bit operands) ----

template <int NT = 0>
MFH_DEV void mfh_ld8_bf16(const void* p, mfh_i64 e, float* a)
{
    mfh_u32x4 x = mfh_vld<NT, mfh_u32x4>(static_cast<const mfh_u16*>(p) + e);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[2 * k] = mfh_f32(x[k] << 16);
        a[2 * k + 1] = mfh_f32(x[k] & 0xffff0000u);
    }
}

template <int NT = 0>
MFH_DEV void mfh_ld8_f16(const void* p, mfh_i64 e, float* a)
{
    mfh_u32x4 x = mfh_vld<NT, mfh_u32x4>(static_cast<const mfh_u16*>(p) + e);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[2 * k] = mfh_f16_to_f32(x[k] & 0xffffu);
        a[2 * k + 1] = mfh_f16_to_f32(x[k] >> 16);
    }
}

MFH_DEV void mfh_st8_bf16(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x4 x = {mfh_bf16x2_rne(r[0], r[1]), mfh_bf16x2_rne(r[2], r[3]),
                   mfh_bf16x2_rne(r[4], r[5]), mfh_bf16x2_rne(r[6], r[7])};
    __builtin_nontemporal_store(x, reinterpret_cast<mfh_u32x4*>(static_cast<mfh_u16*>(p) + e));
}

MFH_DEV void mfh_st8_f16(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x4 x = {mfh_f16x2_rne(r[0], r[1]), mfh_f16x2_rne(r[2], r[3]),
                   mfh_f16x2_rne(r[4], r[5]), mfh_f16x2_rne(r[6], r[7])};
    __builtin_nontemporal_store(x, reinterpret_cast<mfh_u32x4*>(static_cast<mfh_u16*>(p) + e));
}

// ---- 4-element items (some operand is f32) ----

template <int NT = 0>
MFH_DEV void mfh_ld4_f32(const void* p, mfh_i64 e, float* a)
{
    mfh_u32x4 x = mfh_vld<NT, mfh_u32x4>(static_cast<const float*>(p) + e);
#pragma unroll
    for (int k = 0; k < 4; k++) a[k] = mfh_f32(x[k]);
}

template <int NT = 0>
MFH_DEV void mfh_ld4_bf16(const void* p, mfh_i64 e, float* a)
{
    mfh_u32x2 x = mfh_vld<NT, mfh_u32x2>(static_cast<const mfh_u16*>(p) + e);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        a[2 * k] = mfh_f32(x[k] << 16);
        a[2 * k + 1] = mfh_f32(x[k] & 0xffff0000u);
    }
}

template <int NT = 0>
MFH_DEV void mfh_ld4_f16(const void* p, mfh_i64 e, float* a)
{
    mfh_u32x2 x = mfh_vld<NT, mfh_u32x2>(static_cast<const mfh_u16*>(p) + e);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        a[2 * k] = mfh_f16_to_f32(x[k] & 0xffffu);
        a[2 * k + 1] = mfh_f16_to_f32(x[k] >> 16);
    }
}

MFH_DEV void mfh_st4_f32(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x4 x = {mfh_bits(r[0]), mfh_bits(r[1]), mfh_bits(r[2]), mfh_bits(r[3])};
    __builtin_nontemporal_store(x, reinterpret_cast<mfh_u32x4*>(static_cast<float*>(p) + e));
}

MFH_DEV void mfh_st4_bf16(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x2 x = {mfh_bf16x2_rne(r[0], r[1]), mfh_bf16x2_rne(r[2], r[3])};
    __builtin_nontemporal_store(x, reinterpret_cast<mfh_u32x2*>(static_cast<mfh_u16*>(p) + e));
}

MFH_DEV void mfh_st4_f16(void* p, mfh_i64 e, const float* r)
{
    mfh_u32x2 x = {mfh_f16x2_rne(r[0], r[1]), mfh_f16x2_rne(r[2], r[3])};
    __builtin_nontemporal_store(x, reinterpret_cast<mfh_u32x2*>(static_cast<mfh_u16*>(p) + e));
}

// ---- f16 operands kept as packed words ----
//
// An f16 operand of the vector path is loaded as its packed 32-bit words; an
// element is word k/2, low half for even k.  Where the value feeds an Add the
// kernel adds the half directly with v_fma_mix_f32 (f16 source converted
// exactly inside the FMA, times 1.0, plus the other term, one rounding): the
// same f32 sum as converting first and adding, in one instruction instead of
// two or three.

template <int NT = 0>
MFH_DEV void mfh_ldw8_f16(const void* p, mfh_i64 e, mfh_u32* w)
{
    mfh_u32x4 x = mfh_vld<NT, mfh_u32x4>(static_cast<const mfh_u16*>(p) + e);
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = x[k];
}

template <int NT = 0>
MFH_DEV void mfh_ldw4_f16(const void* p, mfh_i64 e, mfh_u32* w)
{
    mfh_u32x2 x = mfh_vld<NT, mfh_u32x2>(static_cast<const mfh_u16*>(p) + e);
    w[0] = x[0];
    w[1] = x[1];
}

MFH_DEV float mfh_h2f(mfh_u32 w, int hi) { return mfh_f16_to_f32(hi ? w >> 16 : w & 0xffffu); }

// x + half `hi` of w.  `hi` must fold to a constant (an unrolled index).
MFH_DEV float mfh_add_fh(float x, mfh_u32 w, int hi)
{
    float r;
    if (hi) __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(x));
    else __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(x));
    return r;
}

// half `ha` of a + half `hb` of b.
MFH_DEV float mfh_add_hh(mfh_u32 a, int ha, mfh_u32 b, int hb)
{
    float r;
    if (ha && hb) __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
    else if (ha) __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
    else if (hb) __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
    else __asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// ---- single elements (tails, unaligned buffers, scalar operands) ----

MFH_DEV float mfh_ld1_f32(const void* p, mfh_i64 i) { return static_cast<const float*>(p)[i]; }
MFH_DEV float mfh_ld1_bf16(const void* p, mfh_i64 i) { return mfh_bf16_to_f32(static_cast<const mfh_u16*>(p)[i]); }
MFH_DEV float mfh_ld1_f16(const void* p, mfh_i64 i) { return mfh_f16_to_f32(static_cast<const mfh_u16*>(p)[i]); }

MFH_DEV void mfh_st1_f32(void* p, mfh_i64 i, float v) { static_cast<float*>(p)[i] = v; }
MFH_DEV void mfh_st1_bf16(void* p, mfh_i64 i, float v) { static_cast<mfh_u16*>(p)[i] = (mfh_u16)mfh_bf16_rne(v); }
MFH_DEV void mfh_st1_f16(void* p, mfh_i64 i, float v) { static_cast<mfh_u16*>(p)[i] = (mfh_u16)mfh_f16_rne(v); }

#endif  // MFH_FUSION_IO_HPP
