// Device-side building blocks shared by the attention kernels (gfx950 only).
//
// Storage types: float (fp32) and uint16_t holding raw bfloat16 bits.  All
// arithmetic is fp32.  Reductions are wave64: DPP quad/row permutes, one
// ds_swizzle for the 16-lane hop and two v_readlane for the 32-lane hop, so
// no LDS crossbar (ds_bpermute) is used inside a wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace atn {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 <-> fp32
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Round-to-nearest-even fp32 -> bf16, NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Element access for the two storage types.
template <typename T>
struct Elem;

template <>
struct Elem<float> {
    static __device__ __forceinline__ float ld(const float* p, size_t i) { return p[i]; }
    static __device__ __forceinline__ void st(float* p, size_t i, float v) { p[i] = v; }
    // 4 consecutive elements; p + i must be 16-byte aligned.
    static __device__ __forceinline__ float4 ld4(const float* p, size_t i) {
        return *reinterpret_cast<const float4*>(p + i);
    }
    static __device__ __forceinline__ void st4(float* p, size_t i, float4 v) {
        *reinterpret_cast<float4*>(p + i) = v;
    }
    static constexpr int kVecAlign = 16;
};

template <>
struct Elem<uint16_t> {
    static __device__ __forceinline__ float ld(const uint16_t* p, size_t i) {
        return bf16_bits_to_f32(p[i]);
    }
    static __device__ __forceinline__ void st(uint16_t* p, size_t i, float v) {
        p[i] = f32_to_bf16_bits(v);
    }
    // 4 consecutive bf16 (8 bytes); p + i must be 8-byte aligned.
    static __device__ __forceinline__ float4 ld4(const uint16_t* p, size_t i) {
        uint2 w = *reinterpret_cast<const uint2*>(p + i);
        return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                           __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
    }
    static __device__ __forceinline__ void st4(uint16_t* p, size_t i, float4 v) {
        uint2 w;
        w.x = (uint32_t)f32_to_bf16_bits(v.x) | ((uint32_t)f32_to_bf16_bits(v.y) << 16);
        w.y = (uint32_t)f32_to_bf16_bits(v.z) | ((uint32_t)f32_to_bf16_bits(v.w) << 16);
        *reinterpret_cast<uint2*>(p + i) = w;
    }
    static constexpr int kVecAlign = 8;
};

// ---------------------------------------------------------------- wave64 reductions
// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
// ds_swizzle bitmask mode: and 0x1f, or 0, xor 0x10 -> lane ^ 16 within 32.
constexpr int kSwizzleXor16 = 0x401F;

template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float swz_xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kSwizzleXor16));
}

__device__ __forceinline__ float lane_read(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// max of two floats as one v_max_f32: fmaxf's IEEE semantics make the
// compiler canonicalize both operands first (two more instructions); the
// values here are never signalling NaNs
__device__ __forceinline__ float vmaxf(float a, float b) {
    float d;
    asm("v_max_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}

// max(m, |a|, |b|) as one v_max3_f32 with absolute-value modifiers (running
// magnitude maxima: the fp16 range checks of the fused K encoding and of the
// single-launch kernel's fp32 operands)
__device__ __forceinline__ float vmax3abs(float m, float a, float b) {
    float d;
    asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(d) : "v"(m), "v"(a), "v"(b));
    return d;
}

// Full-wave max; result is wave-uniform.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kDppQuadXor1>(v));
    v = fmaxf(v, dpp<kDppQuadXor2>(v));
    v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp<kDppRowMirror>(v));
    v = fmaxf(v, swz_xor16(v));
    return fmaxf(lane_read(v, 0), lane_read(v, 32));
}

// Full-wave sum; result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<kDppQuadXor1>(v);
    v += dpp<kDppQuadXor2>(v);
    v += dpp<kDppRowHalfMirror>(v);
    v += dpp<kDppRowMirror>(v);
    v += swz_xor16(v);
    return lane_read(v, 0) + lane_read(v, 32);
}

// ---------------------------------------------------------------- positional encodings
enum PeKind : int { kPeNone = 0, kPeRopeInterleaved = 1, kPeRopeHalf = 2, kPeSinusoidal = 3 };

// Angle tables for one side (Q or K).  Two layouts:
//   compact (dup = 0): a[pos*ld + f], b[pos*ld + f] indexed by frequency f
//     (the library's own tables: RoPE a = cos, b = sin, f = pair index;
//      sinusoidal a = sin, b = cos, f = d / 2);
//   caller (dup = 1): the reference's host formats -- RoPE caches
//     [pos][rotary_dim] with each value duplicated at 2i and 2i+1
//     (final/rope.cu:20-40), sinusoidal tables [pos][D] indexed by d
//     (final/sinusoidal.cu:838-855).
struct PeSide {
    const float* a;
    const float* b;
    int ld;
    int dup;
    int rotary;  // RoPE: rotated width (even); sinusoidal: unused
    int on;      // 0: this side is not encoded
};

// fp32 rotation written as separate multiply and subtract/add so the result
// equals the reference CPU path's x_e*c - x_o*s bit for bit.
__device__ __forceinline__ float rot_first(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
    return x0 * c - x1 * s;
}
__device__ __forceinline__ float rot_second(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
    return x0 * s + x1 * c;
}

// cos/sin for RoPE frequency f at position pos.
__device__ __forceinline__ void rope_cs(const PeSide& t, int pos, int f, float& c, float& s) {
    const size_t idx = (size_t)pos * t.ld + (t.dup ? 2 * f : f);
    c = t.a[idx];
    s = t.b[idx];
}

// Sinusoidal PE value for dim d at position pos (even d: sin, odd d: cos).
__device__ __forceinline__ float sin_pe(const PeSide& t, int pos, int d) {
    const size_t idx = (size_t)pos * t.ld + (t.dup ? d : (d >> 1));
    return (d & 1) ? t.b[idx] : t.a[idx];
}

// The positional encoding of this side applied to x[d..d+3] of one row
// (row pointer xr, position pos), already loaded as x (elements at or past
// dend 0: they stay 0).  d is a multiple of 4.  vec: the row may be read 4
// elements at a time (aligned for Elem<T>::ld4).  With the library's compact
// tables (dup = 0, whose rows are 16-byte aligned where a group needs it) a
// whole group of 4 reads its angles and its rotate-half partners as vectors;
// the rotation arithmetic is the same either way.
template <typename T, int PEK>
__device__ __forceinline__ float4 apply_pe4(float4 x, const T* __restrict__ xr, int pos, int d,
                                           int dend, const PeSide& pe, bool vec) {
    float v[4] = {x.x, x.y, x.z, x.w};
    if constexpr (PEK == kPeRopeInterleaved) {
        if (pe.on) {
            if (!pe.dup && (pe.ld & 1) == 0 && d + 3 < pe.rotary) {
                // frequencies d / 2 and d / 2 + 1: 8 bytes of each table
                const size_t idx = (size_t)pos * pe.ld + (d >> 1);
                const float2 c = *reinterpret_cast<const float2*>(pe.a + idx);
                const float2 sn = *reinterpret_cast<const float2*>(pe.b + idx);
                const float x0 = v[0], x1 = v[1], x2 = v[2], x3 = v[3];
                v[0] = rot_first(x0, x1, c.x, sn.x);
                v[1] = rot_second(x0, x1, c.x, sn.x);
                v[2] = rot_first(x2, x3, c.y, sn.y);
                v[3] = rot_second(x2, x3, c.y, sn.y);
            } else {
#pragma unroll
                for (int c = 0; c < 4; c += 2) {
                    const int e = d + c;  // even
                    if (e < pe.rotary) {
                        float cs, sn;
                        rope_cs(pe, pos, e >> 1, cs, sn);
                        const float x0 = v[c], x1 = v[c + 1];
                        v[c] = rot_first(x0, x1, cs, sn);
                        v[c + 1] = rot_second(x0, x1, cs, sn);
                    }
                }
            }
        }
    } else if constexpr (PEK == kPeRopeHalf) {
        if (pe.on) {
            const int h = pe.rotary >> 1;
            if (vec && !pe.dup && (h & 3) == 0 && (pe.ld & 3) == 0 && d + 3 < pe.rotary &&
                d + 3 < dend) {
                // the 4 dims lie on one side of h: their partners are the 4
                // dims h away, their frequencies 4 consecutive ones
                const bool lo = d < h;
                const float4 xp = Elem<T>::ld4(xr, lo ? d + h : d - h);
                const size_t idx = (size_t)pos * pe.ld + (lo ? d : d - h);
                const float4 c = *reinterpret_cast<const float4*>(pe.a + idx);
                const float4 sn = *reinterpret_cast<const float4*>(pe.b + idx);
                const float p[4] = {xp.x, xp.y, xp.z, xp.w};
                const float cc[4] = {c.x, c.y, c.z, c.w}, ss[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    v[k] = lo ? rot_first(v[k], p[k], cc[k], ss[k])
                              : rot_second(p[k], v[k], cc[k], ss[k]);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int e = d + c;
                    // (past dend the element stays 0: its partner is loaded
                    // from the row itself, which would make it nonzero)
                    if (e < pe.rotary && e < dend) {
                        const bool lo = e < h;
                        const int f = lo ? e : e - h;
                        const float xp = Elem<T>::ld(xr, lo ? e + h : e - h);
                        float cs, sn;
                        rope_cs(pe, pos, f, cs, sn);
                        v[c] = lo ? rot_first(v[c], xp, cs, sn) : rot_second(xp, v[c], cs, sn);
                    }
                }
            }
        }
    } else if constexpr (PEK == kPeSinusoidal) {
        if (pe.on) {
            if (!pe.dup && (pe.ld & 1) == 0 && d + 3 < dend) {
                // dims d, d + 2 take sin of frequencies d / 2, d / 2 + 1, dims
                // d + 1, d + 3 their cos: 8 bytes of each table
                const size_t idx = (size_t)pos * pe.ld + (d >> 1);
                const float2 sn = *reinterpret_cast<const float2*>(pe.a + idx);
                const float2 c = *reinterpret_cast<const float2*>(pe.b + idx);
                v[0] = v[0] + sn.x;
                v[1] = v[1] + c.x;
                v[2] = v[2] + sn.y;
                v[3] = v[3] + c.y;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (d + c < dend) v[c] = v[c] + sin_pe(pe, pos, d + c);
            }
        }
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}

// Whether pe4_batch serves this side: the library's compact tables
// (dup = 0) with rows a whole number of the vectors it reads (interleaved
// RoPE: rotary a multiple of 4; rotate-half: rotary / 2 a multiple of 4;
// sinusoidal: head_d a multiple of 4, which every caller has).
__device__ __forceinline__ bool pe4_batch_ok(int pek, const PeSide& pe) {
    if (pe.dup) return false;
    if (pek == kPeRopeInterleaved) return (pe.rotary & 3) == 0;
    if (pek == kPeRopeHalf) return (pe.rotary & 7) == 0;
    return (pe.ld & 1) == 0;
}

// The positional encoding of one group of 4 elements in two phases:
// pe4_fetch loads its operands (the angles, the rotate-half partners) and
// pe4_apply does the arithmetic, so that a caller can issue the loads of
// many groups before any arithmetic and the groups' latencies overlap
// instead of each group waiting in turn.  The group holds dims d..d + 3 (d a
// multiple of 4) of the row at xr, position pos (a row of the tables), at or
// past dend zeros.  Only where pe4_batch_ok holds, and with rows 8-byte
// aligned for T = uint16_t, 16-byte for float.  Addresses of groups that
// take no encoding (past the rotary width or dend) are clamped into the row
// and the table, so every load is valid and its result unused.  The
// arithmetic is apply_pe4's.
template <int PEK>
struct Pe4Ops {};
template <>
struct Pe4Ops<kPeRopeInterleaved> {
    float2 c, s;  // frequencies d / 2 and d / 2 + 1
};
template <>
struct Pe4Ops<kPeRopeHalf> {
    float4 c, s, p;  // 4 consecutive frequencies; the partners h away
};
template <>
struct Pe4Ops<kPeSinusoidal> {
    float2 s, c;  // sin and cos of frequencies d / 2 and d / 2 + 1
};
template <typename T, int PEK>
__device__ __forceinline__ Pe4Ops<PEK> pe4_fetch(int d, const T* __restrict__ xr, int pos,
                                                 int dend, const PeSide& pe) {
    Pe4Ops<PEK> o;
    if constexpr (PEK == kPeRopeInterleaved) {
        const size_t idx = (size_t)pos * pe.ld + (min(d, pe.rotary - 4) >> 1);
        o.c = *reinterpret_cast<const float2*>(pe.a + idx);
        o.s = *reinterpret_cast<const float2*>(pe.b + idx);
    } else if constexpr (PEK == kPeRopeHalf) {
        const int h = pe.rotary >> 1;
        const bool lo = d < h;
        const size_t idx = (size_t)pos * pe.ld + min(lo ? d : d - h, h - 4);
        o.c = *reinterpret_cast<const float4*>(pe.a + idx);
        o.s = *reinterpret_cast<const float4*>(pe.b + idx);
        // the partner h away (clamped below the rotary width, inside the
        // row, for groups that take no encoding; dend may end a slice of the
        // row, the partner lies outside it)
        o.p = Elem<T>::ld4(xr, min(lo ? d + h : d - h, pe.rotary - 4));
    } else if constexpr (PEK == kPeSinusoidal) {
        const size_t idx = (size_t)pos * pe.ld + (min(d, dend - 4) >> 1);
        o.s = *reinterpret_cast<const float2*>(pe.a + idx);
        o.c = *reinterpret_cast<const float2*>(pe.b + idx);
    }
    return o;
}
template <int PEK>
__device__ __forceinline__ float4 pe4_apply(float4 x, const Pe4Ops<PEK>& o, int d, int dend,
                                            const PeSide& pe) {
    if constexpr (PEK == kPeRopeInterleaved) {
        if (d + 3 < pe.rotary)
            x = make_float4(rot_first(x.x, x.y, o.c.x, o.s.x), rot_second(x.x, x.y, o.c.x, o.s.x),
                            rot_first(x.z, x.w, o.c.y, o.s.y), rot_second(x.z, x.w, o.c.y, o.s.y));
    } else if constexpr (PEK == kPeRopeHalf) {
        if (d + 3 < pe.rotary && d + 3 < dend) {
            const bool lo = d < (pe.rotary >> 1);
            const float v[4] = {x.x, x.y, x.z, x.w};
            const float q[4] = {o.p.x, o.p.y, o.p.z, o.p.w};
            const float cc[4] = {o.c.x, o.c.y, o.c.z, o.c.w};
            const float ss[4] = {o.s.x, o.s.y, o.s.z, o.s.w};
            float r[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                r[k] = lo ? rot_first(v[k], q[k], cc[k], ss[k]) : rot_second(q[k], v[k], cc[k], ss[k]);
            x = make_float4(r[0], r[1], r[2], r[3]);
        }
    } else if constexpr (PEK == kPeSinusoidal) {
        if (d + 3 < dend) x = make_float4(x.x + o.s.x, x.y + o.c.x, x.z + o.s.y, x.w + o.c.y);
    }
    return x;
}

// pe4_fetch and pe4_apply on N groups at once (group i: x[i], dims d[i].., row
// xr[i], position pos[i]), every load issued before any arithmetic.
template <typename T, int PEK, int N>
__device__ __forceinline__ void pe4_batch(float4 (&x)[N], const int (&d)[N],
                                          const T* const (&xr)[N], const int (&pos)[N], int dend,
                                          const PeSide& pe) {
    Pe4Ops<PEK> o[N];
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = pe4_fetch<T, PEK>(d[i], xr[i], pos[i], dend, pe);
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = pe4_apply<PEK>(x[i], o[i], d[i], dend, pe);
}

// Rotate-half over whole rows (rotary = the row's length) where a row's
// 4-dim groups lie in 2 XM consecutive lanes, group g in lane g of them: the
// partner of a group (the dims half a row away) is then in the lane XM away
// (lane ^ XM), taken by ds_swizzle instead of loaded again; only the angles
// are loaded, all before the arithmetic.  Otherwise as pe4_batch (compact
// tables, rotary / 2 a multiple of 4).
template <int XM>
__device__ __forceinline__ float swz_xor_lanes(float v) {
    static_assert(XM == 4 || XM == 8 || XM == 16, "xor within 32 lanes");
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (XM << 10)));
}
template <int N, int XM>
__device__ __forceinline__ void pe4_batch_half_lanes(float4 (&x)[N], const int (&d)[N],
                                                     const int (&pos)[N], const PeSide& pe) {
    const int h = pe.rotary >> 1;
    float4 c[N], sn[N], p[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const size_t idx = (size_t)pos[i] * pe.ld + (d[i] < h ? d[i] : d[i] - h);
        c[i] = *reinterpret_cast<const float4*>(pe.a + idx);
        sn[i] = *reinterpret_cast<const float4*>(pe.b + idx);
        p[i] = make_float4(swz_xor_lanes<XM>(x[i].x), swz_xor_lanes<XM>(x[i].y),
                           swz_xor_lanes<XM>(x[i].z), swz_xor_lanes<XM>(x[i].w));
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const bool lo = d[i] < h;
        const float v[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
        const float q[4] = {p[i].x, p[i].y, p[i].z, p[i].w};
        const float cc[4] = {c[i].x, c[i].y, c[i].z, c[i].w};
        const float ss[4] = {sn[i].x, sn[i].y, sn[i].z, sn[i].w};
        float r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            r[k] = lo ? rot_first(v[k], q[k], cc[k], ss[k]) : rot_second(q[k], v[k], cc[k], ss[k]);
        x[i] = make_float4(r[0], r[1], r[2], r[3]);
    }
}

// Loads x[d..d+3] of one row (row pointer xr, position pos), applies the
// positional encoding of this side, and returns fp32.  Elements at or past
// dend read as 0.  d is a multiple of 4.
template <typename T, int PEK>
__device__ __forceinline__ float4 load_row4_pe(const T* __restrict__ xr, int pos, int d, int dend,
                                              const PeSide& pe, bool vec_ok) {
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (vec_ok && d + 3 < dend) {
        float4 t = Elem<T>::ld4(xr, d);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (d + c < dend) v[c] = Elem<T>::ld(xr, d + c);
    }
    return apply_pe4<T, PEK>(make_float4(v[0], v[1], v[2], v[3]), xr, pos, d, dend, pe, vec_ok);
}

}  // namespace atn
