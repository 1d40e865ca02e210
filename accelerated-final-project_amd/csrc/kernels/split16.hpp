// fp32 operands on 16-bit MFMA (gfx950): the hi + lo fp16 split shared by
// the single-launch, flash and split-D kernels.
//
// An fp32 value x with |x| < 65504 is held as two fp16 parts, hi = x
// rounded toward zero (v_cvt_pkrtz_f16_f32) and lo = the residual rounded to
// nearest even (v_cvt_pk_f16_f32).  fp16 subnormals are produced by the
// conversion and kept by v_mfma_f32_16x16x32_f16 (checked on the MI355X), so
// |x - hi - lo| <= 2^-22 |x| for |x| >= 2^-3 and <= 2^-25 below.  A product
// is then a_hi b_hi + a_hi b_lo + a_lo b_hi: three exact fp16 products with
// fp32 accumulation (the dropped a_lo b_lo is below 2^-20 of the product),
// at about five times the rate of fp32 MFMA.  Values outside fp16's range
// are brought inside by power-of-two scales (exact), chosen per tile from
// the largest finite magnitude and undone on the fp32 results.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace atn {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short v4i16 __attribute__((ext_vector_type(4)));

// Largest magnitude an fp32 operand may have for the fp16 split.
constexpr float kF16Range = 65504.0f;

// hi + lo fp16 parts of two values, packed (see the file comment).
__device__ __forceinline__ void split2_f16(float a, float b, uint32_t& h, uint32_t& l) {
    const f16x2 hh = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a, b));
    const f16x2 lv = {(_Float16)(a - (float)hh[0]), (_Float16)(b - (float)hh[1])};
    h = __builtin_bit_cast(uint32_t, hh);
    l = __builtin_bit_cast(uint32_t, lv);
}

// The same split of a s and b s for s = 1 or a power of two (so the
// products are exact) in three instructions per pair: hi by
// v_cvt_pkrtz_f16_f32, each lo as an fp32 fma of a s minus the fp16 hi
// (exact in fp32) rounded to fp16, which the compiler emits as one
// v_fma_mix.  Written in C, not as inline asm, so that the compiler's
// hazard checks see the writes (the parts feed MFMA operands).  For s = 1
// use split2_f16_one: an fma by a known 1 is folded to an add, which does
// not take the mixed form.
__device__ __forceinline__ void split2_f16_mix(float a, float b, float s, uint32_t& h,
                                               uint32_t& l) {
    const f16x2 hh = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a * s, b * s));
    const f16x2 lv = {(_Float16)__builtin_fmaf(a, s, -(float)hh[0]),
                      (_Float16)__builtin_fmaf(b, s, -(float)hh[1])};
    h = __builtin_bit_cast(uint32_t, hh);
    l = __builtin_bit_cast(uint32_t, lv);
}
// 1.0 in a register the compiler treats as unknown (an empty asm marks it
// modified; no instruction is emitted)
__device__ __forceinline__ float unit_opaque() {
    float one = 1.f;
    asm volatile("" : "+v"(one));
    return one;
}
// split2_f16_mix for s = 1 (`one` from unit_opaque()): no multiplications
__device__ __forceinline__ void split2_f16_one(float a, float b, float one, uint32_t& h,
                                               uint32_t& l) {
    const f16x2 hh = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a, b));
    const f16x2 lv = {(_Float16)__builtin_fmaf(a, one, -(float)hh[0]),
                      (_Float16)__builtin_fmaf(b, one, -(float)hh[1])};
    h = __builtin_bit_cast(uint32_t, hh);
    l = __builtin_bit_cast(uint32_t, lv);
}

__device__ __forceinline__ v4f mfma_f16(const f16x8& a, const f16x8& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// a_hi b_hi + a_hi b_lo + a_lo b_hi accumulated into c
__device__ __forceinline__ v4f mfma_split(const f16x8& ah, const f16x8& al, const f16x8& bh,
                                          const f16x8& bl, v4f c) {
    c = mfma_f16(ah, bh, c);
    c = mfma_f16(ah, bl, c);
    return mfma_f16(al, bh, c);
}

// 8 consecutive 16-bit elements from LDS
__device__ __forceinline__ f16x8 lds8_f16(const uint16_t* p) {
    return __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(p));
}

// gfx950's transposing LDS read of 16-bit elements (ds_read_b64_tr_b16):
// the 16 lanes of a group each supply the address of 4 consecutive elements
// of one row; lane L receives column L % 16 of the group's 4 rows.
__device__ __forceinline__ uint2 lds_tr16(const uint16_t* p) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                         (__attribute__((address_space(3))) v4i16*)(p)));
}

// Power-of-two scale s for values of largest finite magnitude m (m >= 0):
// m s in [2^14, 2^15) (s = 2^(14 - e) for m in [2^e, 2^(e+1)), kept within
// [2^-114, 2^126]); 1 for m == 0.  pow2_unit(m) = 1 / s, exactly.
__device__ __forceinline__ float pow2_scale(float m) {
    int eb = (__float_as_int(m) >> 23) & 0xff;
    if (eb == 0) return 1.f;
    eb = eb < 15 ? 15 : eb;
    return __int_as_float((268 - eb) << 23);
}
__device__ __forceinline__ float pow2_unit(float m) {
    int eb = (__float_as_int(m) >> 23) & 0xff;
    if (eb == 0) return 1.f;
    eb = eb < 15 ? 15 : eb;
    return __int_as_float((eb - 14) << 23);
}
// ... only for tiles that exceed the split's range (1 otherwise)
__device__ __forceinline__ float range_scale(float m) { return m < kF16Range ? 1.f : pow2_scale(m); }
__device__ __forceinline__ float range_unit(float m) { return m < kF16Range ? 1.f : pow2_unit(m); }

// The largest finite magnitude of m and the 4 values (infinities and NaNs
// count as 0: they stay non-finite through a scaling, and must not set the
// scale of the finite values beside them).
__device__ __forceinline__ float max_finite4(float m, float4 f) {
    auto fa = [](float x) {
        const float a = fabsf(x);
        return a < INFINITY ? a : 0.f;
    };
    return fmaxf(fmaxf(m, fmaxf(fa(f.x), fa(f.y))), fmaxf(fa(f.z), fa(f.w)));
}

// 16 bytes at byte offset `off` of a raw buffer (zeros past its end).
__device__ __forceinline__ float4 ld_buf_f4(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                       __uint_as_float(v[3]));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Byte offset past every buffer (a load from it reads zeros).
constexpr int kBufOob = 0x7ffffff0;

}  // namespace atn
