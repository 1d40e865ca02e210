// Single-launch split-D attention for short sequences and large head_dim
// (gfx950): len_q <= 64, len_k <= 128, any D.
//
// The reference's headline shapes (e.g. B=1, H=4, L=64, D=2048) move a few
// MiB and hold a 64x64 score matrix per head, so one query row per
// workgroup (final/attention.cu:209-215) leaves the chip idle.  Here the
// query rows of head bh are cut into `QB` row groups of `MB` rows, D into
// `nchunk` slices of `dc` dims, and workgroup (group g = (bh, qb), c):
//
//   1. loads its Q rows' slice and the head's K/V slices once (16-byte
//      loads, all in flight before the first LDS store; the positional
//      encoding is applied to Q and K at load) into LDS;
//   2. computes the partial scores S_c = Q[rows, c] K[:, c]^T on 16-bit
//      MFMA, up to eight independent 16x16 tiles per wave.  fp32 inputs are
//      split into hi + lo fp16 parts (split2_f16: 22 significant bits, and
//      subnormal parts, which the MFMA keeps, hold small values to 2^-25)
//      and multiplied as a_hi b_hi + a_hi b_lo + a_lo b_hi on
//      v_mfma_f32_16x16x32_f16 (exact products, fp32 accumulation; the
//      dropped a_lo b_lo is below 2^-20 of the product), at about five
//      times the throughput of fp32 MFMA
//      (v_mfma_f32_16x16x4_f32), whose dependent chains bounded this phase.
//      The split needs |x| < 65504: each workgroup tracks the largest
//      magnitude it stores, and one whose Q/K (or V) slice exceeds that
//      range stages the slice again scaled by a power of two (exact) and
//      multiplies the results back.  bf16 inputs are exact bf16 MFMA
//      operands (v_mfma_f32_16x16x32_bf16); after a positional encoding
//      they are split into hi + lo bf16 parts;
//   3. all-reduces S over the group's slices through global memory, either
//      in one gather (every workgroup reads every slice's partial of its
//      group: one memory round trip) or, when that volume is too large, as
//      a reduce-scatter then an all-gather (two round trips).  Partials are
//      always summed in slice order, so results are bit-reproducible;
//   4. exact softmax of scale * S per row (max, exp, sum, divide;
//      final/attention.cu:262-270), 16, 8 or 4 threads per row;
//   5. O[rows, slice] = P V[:, slice] on MFMA, P split into hi + lo parts
//      (fp32: fp16 parts of 2^15 P, exact power-of-two scaling, and fp32 V
//      split as Q and K are; bf16: bf16 parts), one store per output
//      element.
//
// Q and O are touched once; K and V once per row group, and the QB
// workgroups that share a K/V slice get workgroup ids QB apart by a
// multiple of the (head, slice) count, which the dispatcher's round-robin
// over the 8 XCDs puts on one XCD whenever that count is a multiple of 8,
// so the repeats hit that XCD's L2.
//
// Exchange.  Partial and reduced scores are stored and loaded with
// device-scope (agent) atomic operations, which gfx950 performs at the
// device's coherence point, so no L2 write-back or invalidate is needed.  A
// writer waits for its exchange stores to complete (s_waitcnt), then
// publishes one done word per workgroup and step; wave 0 of each reader
// polls the n done words of its group (one small word per writer keeps the
// polling traffic low; where the plan allows, each word has a 128-byte line
// of its own, since one line that every slice of a group stores to and
// polls is a hot spot at the coherence point) and the exchange words are
// then read once.  Done
// words carry a tag made of the row group g (< 2048) and the group's epoch
// word in the workspace's sync region, read at start (exchange_tag below):
// a call that has seen every slice's done word of its group knows that
// every workgroup of the group has read the epoch, so slice 0 of the group
// then stores epoch + 1.  A done word left by an earlier call, another
// group or another layout never carries the expected tag; nothing is reset
// between calls and kernel arguments never change from call to call (a
// captured HIP graph replays correctly).  Waits are bounded: on a timeout
// the workgroup sets the status word, writes NaN to its output slice and
// exits, so every wave ends; while the status word is set, later calls
// fail closed the same way until the host clears the status word (and
// moves every epoch past the failed call's).  The host launches at most as
// many workgroups as the device holds at once.
//
// XCD-local exchange (XL plans).  The dispatcher deals consecutive
// workgroup ids to the 8 XCDs round robin, each XCD with its own L2, but
// the XCD that receives id 0 varies from dispatch to dispatch (measured:
// usually XCD 0, sometimes not).  So an XL workgroup takes its XCD x from
// the XCC_ID hardware register and its place on that XCD from id / 8: with
// a grid that is a multiple of 8, every XCD receives each place 0 ..
// grid/8 - 1 exactly once whatever the starting XCD.  Place gi * n + c runs
// slice c of the XCD's gi-th row group, and each XCD takes a contiguous
// block of row groups (heads stay together, so their K/V slices are fetched
// by as few XCDs as possible).  The exchange then stays inside that XCD's
// L2: plain stores, `sc0 nt` loads (which always read L2, never a CU's
// vector L1), and one arrival counter per row group and exchange step,
// added to atomically at the L2.  Every call adds exactly kXcdUnits to each
// counter (slice c < n - 1 adds c + 1, the last slice the rest), on every
// path including failures, so a counter is a multiple of kXcdUnits between
// calls and its value at a call's start is the arrival's old value rounded
// down; no epoch, tag or reset is needed.  A wait ends when the count is
// exactly complete: since the shares differ, a slice that arrived twice or
// never makes the wait time out (reported) rather than pass early.
// Counter words are indexed by the physical XCD, so only that XCD's L2
// ever holds their lines; with at most 4 row groups per XCD each counter
// has a line of its own.
#pragma once

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "split16.hpp"

namespace atn {

// Kernel arguments (a plain aggregate shared by the translation units that
// instantiate the kernel variants).
struct FusedArgs {
    const void* Q;
    const void* K;
    const void* V;
    void* O;
    float* part;       // [G][E / 256][nchunk][256] partial scores
    float* red;        // [G][E] reduced scores (two-phase exchange)
    unsigned* epochs;  // [G] per-group epoch words (sync region)
    unsigned* done;    // [2][2048] per-workgroup done words, one set per exchange step
    int* status;       // nonzero after an exchange timeout
    int Lq, Lk, D, dc, nchunk;
    int MB, QB;        // query rows per row group, row groups per head
    int gather1;       // 1: one-gather exchange, 0: reduce-scatter + all-gather
    int G;             // row groups (heads x QB)
    unsigned* xctr;    // XL plans: arrival counters, kXcdCtrWords per XCD
    float scale;
    PeSide pq, pk;
    // Division by the plan's divisors without a division sequence: for the
    // small non-negative dividends of this kernel x / d = umulhi(x, m_d),
    // m_d = 2^32 / d rounded up (exact while x * d < 2^32; d = 1 has m = 0
    // and is taken apart).  Set by the host (fused_div_magic).
    int rstep;      // Q/K/V rows loaded per pass: 256 / (dc / 4)
    unsigned m_n, m_qb, m_bh, m_vpr, m_rstep, m_nk;
};

__host__ __device__ inline unsigned fused_div_magic(int d) {
    return d <= 1 ? 0u : (unsigned)(0xFFFFFFFFull / (unsigned)d + 1ull);
}

// One translation unit per (element type, exchange scope) instantiates the
// kernel's encoding and load-form variants (fused_small_<type>[_xl].hip), so
// that they compile in parallel; these are its entry points.
hipError_t fused_small_launch_f32(const FusedArgs& a, int pek, int form, int lds, hipStream_t st);
hipError_t fused_small_launch_f32_xl(const FusedArgs& a, int pek, int form, int lds,
                                     hipStream_t st);
hipError_t fused_small_launch_bf16(const FusedArgs& a, int pek, int form, int lds,
                                   hipStream_t st);
hipError_t fused_small_launch_bf16_xl(const FusedArgs& a, int pek, int form, int lds,
                                      hipStream_t st);
// resident workgroups per CU for this LDS size, smallest over the unit's
// variants
int fused_small_per_cu_f32(int lds);
int fused_small_per_cu_f32_xl(int lds);
int fused_small_per_cu_bf16(int lds);
int fused_small_per_cu_bf16_xl(int lds);

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kSpinLimit = 1 << 18;  // polls (each >= one memory round trip): ~0.3 s bound
// Units every call adds to an XCD-local arrival counter: a power of two (so
// 32-bit wraparound keeps counters multiples of it) above the shares 1 ..
// n - 1 of the first n - 1 slices (n <= 2048).
constexpr unsigned kXcdUnits = 1u << 23;
static_assert(2048u * 2047u / 2u < kXcdUnits, "XCD-local shares");
// Buffer cache policy of XCD-local exchange loads: sc0 | nt, served by the
// XCD's L2 on every access.
constexpr int kAuxL2 = 3;

// Positional encoding of the 4 consecutive elements v = x[d..d+3] of one
// row (row pointer xr, position pos); d is a multiple of 4 and d + 3 < D.
template <typename T, int PEK>
__device__ __forceinline__ float4 encode4(float4 v4, const T* __restrict__ xr, int pos, int d,
                                          const PeSide& pe) {
    float v[4] = {v4.x, v4.y, v4.z, v4.w};
    if constexpr (PEK == kPeRopeInterleaved) {
        if (pe.on) {
#pragma unroll
            for (int c = 0; c < 4; c += 2) {
                const int e = d + c;
                if (e < pe.rotary) {
                    float cs, sn;
                    rope_cs(pe, pos, e >> 1, cs, sn);
                    const float x0 = v[c], x1 = v[c + 1];
                    v[c] = rot_first(x0, x1, cs, sn);
                    v[c + 1] = rot_second(x0, x1, cs, sn);
                }
            }
        }
    } else if constexpr (PEK == kPeRopeHalf) {
        if (pe.on) {
            const int h = pe.rotary >> 1;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = d + c;
                if (e < pe.rotary) {
                    const bool lo = e < h;
                    const int f = lo ? e : e - h;
                    const float xp = Elem<T>::ld(xr, lo ? e + h : e - h);
                    float cs, sn;
                    rope_cs(pe, pos, f, cs, sn);
                    v[c] = lo ? rot_first(v[c], xp, cs, sn) : rot_second(xp, v[c], cs, sn);
                }
            }
        }
    } else if constexpr (PEK == kPeSinusoidal) {
        if (pe.on) {
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = v[c] + sin_pe(pe, pos, d + c);
        }
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}

// LDS geometry of one workgroup (MFMA operands as 16-bit parts).  Q, K and P rows
// are padded by 8 elements (16-byte aligned 8-element reads); V is kept
// [key][dim] with a row stride of dc + 16 elements, i.e. 32 or 96 bytes
// (mod 128), so the 4 rows x 32 bytes that each 16-lane group of a
// transposing read (ds_read_b64_tr_b16) touches fall in distinct banks; the
// softmax reads 8 rows x 4 columns of fp32 S -> stride = 4 (mod 32).  With
// an exchange (s_over_qk), S lies over the Q and K regions: it is written
// only by the exchange, after the barrier that follows the last read of Q
// and K; a single slice writes S straight from the accumulators, so S then
// has a region of its own.
struct Geo {
    int MQ, NK, dc;
    int qstr, kstr, vstr, sstr, pstr;
    int q_off, k_off, ql_off, kl_off, v_off, vl_off, s_off, p_off, red_off;  // byte offsets
    int bytes;
};

// f32: fp32 inputs (Q, K and V kept as hi + lo fp16 parts); encoded: a
// positional encoding makes Q/K non-bf16 (hi + lo bf16 parts for bf16
// inputs).
__host__ __device__ inline Geo make_geo(bool f32, bool encoded, bool s_over_qk, int Lq, int Lk,
                                        int dc) {
    Geo g{};
    g.MQ = (Lq + 15) / 16 * 16;
    g.NK = (Lk + 31) / 32 * 32;
    g.dc = dc;
    const bool split = f32 || encoded;
    g.qstr = g.kstr = dc + 8;
    g.vstr = dc + 16;   // V stored [key][dim], read transposed
    g.pstr = g.NK + 8;  // P hi and lo, [row][key]
    g.sstr = g.NK + 4;
    int off = 0;
    auto take = [&](int b) { int o = off; off += (b + 15) / 16 * 16; return o; };
    g.q_off = take(g.MQ * g.qstr * 2);
    g.k_off = take(g.NK * g.kstr * 2);
    g.ql_off = split ? take(g.MQ * g.qstr * 2) : g.q_off;
    g.kl_off = split ? take(g.NK * g.kstr * 2) : g.k_off;
    if (s_over_qk) {
        g.s_off = 0;
        off = off > g.MQ * g.sstr * 4 ? off : g.MQ * g.sstr * 4;
    } else {
        g.s_off = take(g.MQ * g.sstr * 4);
    }
    g.v_off = take(g.NK * g.vstr * 2);
    g.vl_off = f32 ? take(g.NK * g.vstr * 2) : g.v_off;
    g.p_off = take(2 * g.MQ * g.pstr * 2);
    g.red_off = take(kThreads * 16);
    g.bytes = off;
    return g;
}


// Most words one thread reads in one exchange step (the host keeps every
// plan within it).
constexpr int kMaxWords = 64;

__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exchange stores and loads of either plan: device scope (the coherence
// point past every L2), or XCD-local (plain stores; sc0 nt loads from L2).
template <bool XL>
__device__ __forceinline__ void st_x(float* p, float v) {
    if constexpr (XL) *p = v;
    else st_dev(p, v);
}
template <bool XL>
__device__ __forceinline__ float ld_x(const float* p) {
    if constexpr (XL) return __builtin_nontemporal_load(p);
    else return ld_dev(p);
}

// The XCD this wave runs on (hardware register XCC_ID, gfx94x / gfx950).
__device__ __forceinline__ unsigned xcc_id() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xfu;
}

// Tag of the done words of row group rg (< 2048) at `epoch`: the top bit is
// always set, so zero-filled memory never carries a valid tag; the epoch
// field repeats after 2^20 calls of one group.
__device__ __forceinline__ unsigned exchange_tag(unsigned epoch, int rg) {
    return 0x80000000u | ((epoch << 11) & 0x7ffff800u) | (unsigned)rg;
}

// Buffer resource over `bytes` bytes at `base` (uniform), raw (unformatted)
// 32-bit elements; loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// 16 bytes at byte offset `off`, with the device-scope cache policy (sc1)
// that agent-scope atomic loads use, so it reads the coherence point; each
// 4-byte element is single-copy atomic, which is all the exchange needs.
__device__ __forceinline__ float4 ld_dev4(__amdgpu_buffer_rsrc_t r, int off) {
    constexpr int kSc1 = 16;
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                       __uint_as_float(v[3]));
}

// 16 bytes at byte offset `off` from this XCD's L2 (sc0 nt).
__device__ __forceinline__ float4 ld_l2_4(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxL2);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                       __uint_as_float(v[3]));
}
template <bool XL>
__device__ __forceinline__ float4 ld_x4(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (XL) return ld_l2_4(r, off);
    else return ld_dev4(r, off);
}

// Exchange stores at byte offset `off` of a buffer resource: XL plans store
// plainly (the line stays in this XCD's L2), device-scope plans with the
// cache policy of agent-scope atomic stores (sc1), so the words reach the
// coherence point; a 16-byte store is four single-copy-atomic elements.
template <bool XL>
__device__ __forceinline__ void st_xb(float v, __amdgpu_buffer_rsrc_t r, int off) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, XL ? 0 : 16);
}
template <bool XL>
__device__ __forceinline__ void st_xb4(float4 v, __amdgpu_buffer_rsrc_t r, int off) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 w = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                     __float_as_uint(v.w)};
    __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, XL ? 0 : 16);
}

// Reads the words base[u * stride], u < cnt, all in flight at once.
template <bool XL, int NW>
__device__ __forceinline__ void ld_words(const float* base, int stride, int cnt, float (&w)[NW]) {
#pragma unroll
    for (int u = 0; u < NW; ++u) w[u] = u < cnt ? ld_x<XL>(base + u * stride) : 0.f;
}

// XL plans.  Wave 0: lane 0 adds `share` to the row group's arrival counter
// at word k of rc (an atomic add performed at this XCD's L2, returning the prior value,
// whose multiple of kXcdUnits is the call's base); with `wait`, the wave
// then polls the counter through L2 until exactly every slice's units of
// this call have arrived.  The other waves wait at the barrier.  A workgroup arrives
// only after every wave's exchange stores have completed (s_waitcnt before
// the barrier), so they are in L2 once the count is complete.  Returns false
// for the whole workgroup on timeout.
__device__ __forceinline__ unsigned xcd_arrive_only(__amdgpu_buffer_rsrc_t rc, int k,
                                                    unsigned share) {
    unsigned old = 0;
    if (threadIdx.x == 0)
        old = (unsigned)__builtin_amdgcn_raw_ptr_buffer_atomic_add_i32((int)share, rc, 4 * k, 0,
                                                                       0);
    return __builtin_amdgcn_readlane(old, 0) & ~(kXcdUnits - 1u);  // wave 0's is the base
}

// The wait of xcd_arrive on its own, given wave 0's base.
__device__ bool xcd_wait(__amdgpu_buffer_rsrc_t rc, int k, unsigned base, int* flag_lds) {
    if (threadIdx.x < 64) {
        bool ok = true;
        for (int it = 0;; ++it) {
            const unsigned v = __builtin_amdgcn_readfirstlane(
                __builtin_amdgcn_raw_buffer_load_b32(rc, 4 * k, 0, kAuxL2));
            if (v - base == kXcdUnits) break;
            if (it > kSpinLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (threadIdx.x == 0 && !ok) *flag_lds = 0;
    }
    __syncthreads();
    return *flag_lds != 0;
}

__device__ bool xcd_arrive(__amdgpu_buffer_rsrc_t rc, int k, unsigned share, bool wait,
                           int* flag_lds) {
    const unsigned base = xcd_arrive_only(rc, k, share);
    if (wait) return xcd_wait(rc, k, base, flag_lds);
    __syncthreads();
    return *flag_lds != 0;
}

// Wave 0 polls the done words done[0..n) until each carries `tag`, while
// the other waves wait at the barrier.  A writer stores its done word only
// after its exchange words have completed (s_waitcnt), so they can be read
// once every done word is seen.  Returns false for the whole workgroup on
// timeout.
__device__ bool wait_done(const unsigned* done, int n, int stride, unsigned tag, int* flag_lds) {
    if (threadIdx.x < 64) {
        bool ok = true;
        for (int it = 0;; ++it) {
            bool mine = true;
            for (int i = threadIdx.x; i < n; i += 64)
                mine &= __hip_atomic_load(const_cast<unsigned*>(done + i * stride),
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag;
            if (__all(mine)) break;
            if (it > kSpinLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (threadIdx.x == 0 && !ok) *flag_lds = 0;
    }
    __syncthreads();
    return *flag_lds != 0;
}

__device__ __forceinline__ void st_done(unsigned* p, unsigned tag) {
    __hip_atomic_store(p, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// NaN into rows [0, lq) of the row group starting at output row `row0`,
// dims [d0, d0 + dc).
template <typename T>
__device__ void poison_slice(T* O, size_t row0, int lq, int D, int d0, int dc) {
    const float nan = __int_as_float(0x7fc00000);
    for (int f = threadIdx.x; f < lq * dc; f += kThreads) {
        const int r = f / dc, d = d0 + f % dc;
        if (d < D) Elem<T>::st(O, (row0 + r) * D + d, nan);
    }
}

// 4 consecutive elements as loaded (fp32: 16 bytes; bf16: 8 bytes of raw
// bits), widened to fp32 on demand.
template <typename T>
struct Raw4;
template <>
struct Raw4<float> {
    typedef float4 type;
    static __device__ __forceinline__ float4 zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
    static __device__ __forceinline__ float4 ld(const float* p) {
        return *reinterpret_cast<const float4*>(p);
    }
    static __device__ __forceinline__ float4 f4(float4 v) { return v; }
    template <int Aux = 0>
    static __device__ __forceinline__ float4 ld_buf(__amdgpu_buffer_rsrc_t r, int off) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, Aux);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                           __uint_as_float(v[3]));
    }
};
template <>
struct Raw4<uint16_t> {
    typedef uint2 type;
    static __device__ __forceinline__ uint2 zero() { return make_uint2(0u, 0u); }
    static __device__ __forceinline__ uint2 ld(const uint16_t* p) {
        return *reinterpret_cast<const uint2*>(p);
    }
    static __device__ __forceinline__ float4 f4(uint2 w) {
        return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                           __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
    }
    template <int Aux = 0>
    static __device__ __forceinline__ uint2 ld_buf(__amdgpu_buffer_rsrc_t r, int off) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, Aux);
        return make_uint2(v[0], v[1]);
    }
};

// 8 consecutive 16-bit MFMA operand elements (bf16x8 or f16x8) from LDS
template <typename VT>
__device__ __forceinline__ VT lds8(const uint16_t* p) {
    return __builtin_bit_cast(VT, *reinterpret_cast<const uint4*>(p));
}

// 16x16x32 MFMA with fp32 accumulation on bf16 or fp16 operands
__device__ __forceinline__ v4f mfma16(const bf16x8& a, const bf16x8& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma16(const f16x8& a, const f16x8& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// two floats to packed bf16 by the hardware conversion (round to nearest
// even, as f32_to_bf16_bits)
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const bf16x2_hw v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// hi + lo bf16 parts of two values, packed (hi rounded to nearest even, lo
// the residual rounded; 16 significant bits): the split of bf16 inputs
// after a positional encoding (fp32 inputs use split2_f16, split16.hpp)
__device__ __forceinline__ void split2_bf16(float a, float b, uint32_t& h, uint32_t& l) {
    h = pack_bf16x2(a, b);
    l = pack_bf16x2(a - __uint_as_float(h << 16), b - __uint_as_float(h & 0xffff0000u));
}
// NT independent 16x16 MFMA accumulations sharing one A operand (k step
// 32, 8 elements per lane, contiguous along k; VT = bf16x8 or f16x8):
// acc[u] += A B_u^T over k in [0, kdim), where lane (lr, lk) reads A at a
// and tile u's B at b + u * bstep (a, b already offset to the lane's row and
// k = 8 lk); the operands of the next k step are read from LDS before this
// step's MFMAs issue.  With ALO the A operand is a_hi + a_lo (two MFMAs);
// with BLO as well the three-term product a_hi b + a_hi b_lo + a_lo b.
template <typename VT, int NT, bool ALO, bool BLO>
__device__ __forceinline__ void mma16(const uint16_t* a, const uint16_t* a_lo, const uint16_t* b,
                                      const uint16_t* b_lo, int bstep, int kdim, v4f (&acc)[NT]) {
    VT ah = lds8<VT>(a), al{};
    if constexpr (ALO) al = lds8<VT>(a_lo);
    VT bv[NT], bl[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        bv[u] = lds8<VT>(b + u * bstep);
        if constexpr (BLO) bl[u] = lds8<VT>(b_lo + u * bstep);
    }
    for (int kk = 0; kk < kdim; kk += 32) {
        const int kn = min(kk + 32, kdim - 32);
        const VT ahn = lds8<VT>(a + kn);
        VT aln{};
        if constexpr (ALO) aln = lds8<VT>(a_lo + kn);
        VT bvn[NT], bln[NT];
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            bvn[u] = lds8<VT>(b + u * bstep + kn);
            if constexpr (BLO) bln[u] = lds8<VT>(b_lo + u * bstep + kn);
        }
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            acc[u] = mfma16(ah, bv[u], acc[u]);
            if constexpr (BLO) acc[u] = mfma16(ah, bl[u], acc[u]);
            if constexpr (ALO) acc[u] = mfma16(al, bv[u], acc[u]);
        }
        ah = ahn;
        if constexpr (ALO) al = aln;
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            bv[u] = bvn[u];
            if constexpr (BLO) bl[u] = bln[u];
        }
    }
}

__device__ __forceinline__ v4i16 ds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p));
}

// PV form of mma16 (A = P as hi + lo parts): the B operand comes from V
// kept [key][dim] in LDS (row stride vstr; vb points at tile 0's first
// column, tile u's columns start nstep later; with VLO, V's lo part lies
// vlo_d elements further).  Lane (lr, lk) needs keys kk + 8 lk + 0..7 of
// column lr: in each 16-lane group lane L supplies the address of key kk +
// 8 lk + 4 h + (L % 16) / 4, columns 4 (L % 4) .. + 3, and the transposing
// read (ds_read_b64_tr_b16, a 16-bit move of either type) hands lane L keys
// 4 h + 0..3 of column L % 16 -- half h of its operand.
template <typename VT, int NT, bool VLO>
__device__ __forceinline__ void mma16_vt(const uint16_t* a, const uint16_t* a_lo,
                                         const uint16_t* vb, int vlo_d, int vstr, int nstep,
                                         int kdim, v4f (&acc)[NT]) {
    const int lane = threadIdx.x & 63;
    const uint16_t* vl = vb + (8 * (lane >> 4) + ((lane & 15) >> 2)) * vstr + 4 * (lane & 3);
    auto vread = [&](const uint16_t* p) {
        const uint2 lo = __builtin_bit_cast(uint2, ds_read_tr16(p));
        const uint2 hi = __builtin_bit_cast(uint2, ds_read_tr16(p + 4 * vstr));
        return __builtin_bit_cast(VT, make_uint4(lo.x, lo.y, hi.x, hi.y));
    };
    for (int kk = 0; kk < kdim; kk += 32) {
        const VT ah = lds8<VT>(a + kk), al = lds8<VT>(a_lo + kk);
        VT bv[NT], bl[NT];
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            const uint16_t* p = vl + kk * vstr + u * nstep;
            bv[u] = vread(p);
            if constexpr (VLO) bl[u] = vread(p + vlo_d);
        }
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            acc[u] = mfma16(ah, bv[u], acc[u]);
            if constexpr (VLO) acc[u] = mfma16(ah, bl[u], acc[u]);
            acc[u] = mfma16(al, bv[u], acc[u]);
        }
    }
}

// x / d for the kernel's small non-negative dividends, m = fused_div_magic(d).
__device__ __forceinline__ int fdiv(int x, int d, unsigned m) {
    return d == 1 ? x : (int)__umulhi((unsigned)x, m);
}

// Wave -> (16-row block, set of 16-column tiles) for an output of nrb row
// blocks and `tiles` column tiles: waves w and w + nrb share a row block and
// take every (4 / nrb)-th column tile.  Returns the number of tiles (0 for
// an idle wave).  wave < 4 and nrb <= 4, so the quotients are selects and
// the waves per row block (4, 2, 1 or 1) a power of two.
__device__ __forceinline__ int wave_tiles(int wave, int nrb, int tiles, int* rb, int* c0,
                                          int* cstep) {
    const int q = nrb == 1 ? wave : (nrb == 2 ? wave >> 1 : (nrb == 3 ? (wave == 3) : 0));
    const int lg = nrb == 1 ? 2 : (nrb == 2 ? 1 : 0);  // log2 of the waves per row block
    const int wpr = 1 << lg;
    *rb = wave - q * nrb;
    *c0 = q;
    *cstep = wpr;
    if (wave >= nrb * wpr || q >= tiles) return 0;
    return (tiles - q + wpr - 1) >> lg;
}

// Load form of a plan: how many row loads of Q (kQ) and of K and of V (kKV)
// each thread issues per round.  Forms 1-3 hold every row of the slice in
// one round of (2, 8), (4, 16) or (8, 16) loads -- the smallest that fits,
// so that no load instruction is issued for rows that do not exist -- and
// then V is loaded and written to LDS around the exchange (see the kernel);
// form 0 loops over rounds of (8, 16).  The host picks the kernel variant
// with this function.
template <int FORM>
struct LoadForm {
    static constexpr int kQ = FORM == 1 ? 2 : (FORM == 2 ? 4 : 8);
    static constexpr int kKV = FORM == 1 ? 8 : 16;
};
__host__ __device__ inline int fused_load_form(int MQ, int NK, int dc) {
    const int rstep = kThreads / (dc >> 2);
    const int nq = (MQ + rstep - 1) / rstep, nkv = (NK + rstep - 1) / rstep;
    if (nq <= LoadForm<1>::kQ && nkv <= LoadForm<1>::kKV) return 1;
    if (nq <= LoadForm<2>::kQ && nkv <= LoadForm<2>::kKV) return 2;
    if (nq <= LoadForm<3>::kQ && nkv <= LoadForm<3>::kKV) return 3;
    return 0;
}

template <typename T, int PEK, bool XL, int FORM>
__global__ __launch_bounds__(kThreads) void k_fused_small(FusedArgs a) {
    constexpr bool kBf16 = sizeof(T) == 2;
    // Q and K carry lo parts (fp32 inputs, or encoded bf16 inputs); V does
    // for fp32 inputs.  MFMA operands: fp16 parts for fp32 inputs, bf16 for
    // bf16 inputs.
    constexpr bool kSplit = !kBf16 || PEK != kPeNone;
    constexpr bool kVlo = !kBf16;
    typedef std::conditional_t<kBf16, bf16x8, f16x8> VT;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int flag;
    // fp32: per wave, whether a Q/K value (0-3) or a V value (4-7) it stored
    // is outside the fp16 split's range; the slices' largest magnitudes when
    // a slice is staged again (sh_big)
    __shared__ __align__(16) int sh_over[8];
    __shared__ float sh_big[8];

    // Every kernel argument in one batch of scalar loads, waited for once,
    // here; left alone the compiler issues each load at its first use.
    asm volatile("" ::"s"(a.Q), "s"(a.K), "s"(a.V), "s"(a.O), "s"(a.part), "s"(a.red),
                 "s"(a.epochs), "s"(a.done), "s"(a.status), "s"(a.xctr), "s"(a.Lq), "s"(a.Lk),
                 "s"(a.D), "s"(a.dc), "s"(a.nchunk), "s"(a.MB), "s"(a.QB), "s"(a.gather1),
                 "s"(a.G), "s"(a.scale), "s"(gridDim.x));
    if constexpr (PEK != kPeNone)
        asm volatile("" ::"s"(a.pq.a), "s"(a.pq.b), "s"(a.pq.ld), "s"(a.pq.dup), "s"(a.pq.rotary),
                     "s"(a.pq.on), "s"(a.pk.a), "s"(a.pk.b), "s"(a.pk.ld), "s"(a.pk.dup),
                     "s"(a.pk.rotary), "s"(a.pk.on));

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    const int lr = lane & 15, lk = lane >> 4;
    const int n = a.nchunk;
    int rg, c, xcd_slot = 0, xk1 = 1;
    if constexpr (XL) {
        // place id / 8 = gi * n + c on XCD x: slice c of the XCD's gi-th row
        // group; XCD x holds row groups [x * base + min(x, rem), + cnt)
        const int x = (int)xcc_id(), local = (int)blockIdx.x >> 3;
        const int gi = fdiv(local, n, a.m_n);
        c = local - gi * n;
        const int base = a.G >> 3, rem = a.G & 7;
        if (gi >= base + (x < rem ? 1 : 0)) return;  // no row group here (whole workgroup)
        rg = x * base + min(x, rem) + gi;
        // the row group's two counters: 32 words apart, and groups 64 apart
        // (each counter in a 128-byte line of its own) when an XCD holds at
        // most 4 row groups, else packed
        const bool spread = a.G <= 32;
        xcd_slot = x * kXcdCtrWords + (spread ? 64 * gi : 2 * gi);
        xk1 = spread ? 32 : 1;
    } else {
        // id = (qb * BH + bh) * n + c
        const int BH = a.G / a.QB;
        const int t = fdiv((int)blockIdx.x, n, a.m_n);
        c = (int)blockIdx.x - t * n;
        const int qb_ = fdiv(t, BH, a.m_bh), bh_ = t - qb_ * BH;
        rg = bh_ * a.QB + qb_;  // row group (epoch word, exchange region, tag)
    }
    const int bh = fdiv(rg, a.QB, a.m_qb), qb = rg - bh * a.QB;
    const int q0 = qb * a.MB;       // first query row of the group
    const int Lq = min(a.MB, a.Lq - q0), Lk = a.Lk, D = a.D, dc = a.dc;
    const int d0 = c * dc;
    const size_t orow0 = (size_t)bh * a.Lq + q0;  // output row of the group's row 0
    const T* __restrict__ Q = static_cast<const T*>(a.Q) + orow0 * D;
    const T* __restrict__ K = static_cast<const T*>(a.K) + (size_t)bh * Lk * D;
    const T* __restrict__ V = static_cast<const T*>(a.V) + (size_t)bh * Lk * D;
    T* __restrict__ O = static_cast<T*>(a.O);

    // The group's epoch and the status word, read once by thread 0 with
    // device-scope loads (a memory round trip).  They are issued right after
    // the slice loads, so that none of wave 0's slice loads waits behind
    // them, and consumed only once the partial scores are out (handed to
    // every thread through LDS at the barrier before the exchange).
    // (Only thread 0 reads ep_r and failed_r, and only when it loaded them:
    // left without an initial value, they need no register copy at the end
    // of its branch, which would wait for the loads -- and, in order, for
    // every slice load issued before them.  XL plans use no epoch.)
    __shared__ unsigned sh_epoch;
    __shared__ int sh_failed;
    unsigned ep_r;
    int failed_r;
    if constexpr (XL) ep_r = 0;

    // ---- 1. Q, K, V slices -> LDS.  Thread t owns 4-element column group
    // t % vpr of rows t / vpr + k * rstep of each tensor.  Loads are raw
    // buffer loads over each tensor's rows of this group or head, so rows
    // past the sequence read as zeros without a branch (a column past D
    // gets an offset past the buffer); branch-free loads let the compiler
    // count them, so a round issues kQ row loads of Q and kKV of K and of V
    // before the first is encoded and stored.  With one round (FORM != 0, a
    // template parameter, so that the one-round code is straight-line code
    // of its own) the Q and K loads are issued first thing, before the LDS
    // geometry and the rest of the set-up, and V's loads and LDS stores
    // hide behind the exchange (the placements below).  (The host sends this
    // kernel only shapes with D % 4 == 0 and aligned bases.)
    typedef typename Raw4<T>::type Raw;
    constexpr int kQ = LoadForm<FORM>::kQ, kKV = LoadForm<FORM>::kKV;
    constexpr bool defer_v = FORM != 0;
    constexpr int es = (int)sizeof(T);
    constexpr int kOob = 0x7ffffff0;  // past every buffer
    const int vpr = dc >> 2;
    const int rstep = a.rstep;  // kThreads / vpr
    const int r0 = fdiv(tid, vpr, a.m_vpr), cg = tid - r0 * vpr;
    const int col = cg * 4, d = d0 + col;
    const bool lane_ok = r0 < rstep && d < D;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(Q, Lq * D * es);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(K, Lk * D * es);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(V, Lk * D * es);
    const int off0 = (r0 * D + d) * es, ostep = rstep * D * es;
    // loads of round j: V rows j*kKV.. (all in flight)
    auto issue_v = [&](int j, Raw (&v)[kKV]) {
#pragma unroll
        for (int u = 0; u < kKV; ++u)
            v[u] = Raw4<T>::ld_buf(rv, lane_ok ? off0 + (j * kKV + u) * ostep : kOob);
    };
    // loads of round j: Q rows j*kQ.., K rows j*kKV.. and, with `with_v`, V
    // rows j*kKV.. (all in flight)
    auto issue = [&](int j, Raw (&q)[kQ], Raw (&k)[kKV], Raw (&v)[kKV], bool with_v) {
#pragma unroll
        for (int u = 0; u < kQ; ++u)
            q[u] = Raw4<T>::ld_buf(rq, lane_ok ? off0 + (j * kQ + u) * ostep : kOob);
        // all K loads, then all V loads: the K stores wait only for the loads
        // issued before the last K load
#pragma unroll
        for (int u = 0; u < kKV; ++u)
            k[u] = Raw4<T>::ld_buf(rk, lane_ok ? off0 + (j * kKV + u) * ostep : kOob);
        if (with_v) issue_v(j, v);
        // Every load stays here, in issue order: a store after them keeps the
        // compiler from sinking one into the (conditional) block that first
        // uses it, and the scheduling barrier from moving one down to shorten
        // its live range.  Either way the first Q load was issued last, and
        // waiting for it waited for every K and V load before the first LDS
        // store.  (Volatile loads, the other way to pin them, become
        // system-scope loads that bypass the L2.)  The store writes the value
        // `flag` is given before its first use anyway.
        flag = 1;
        __builtin_amdgcn_sched_barrier(0);
        if (j == 0 && tid == 0 && n > 1) {
            if constexpr (!XL)
                ep_r = __hip_atomic_load(a.epochs + rg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            failed_r = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    // One round with an exchange: V is loaded only once the partial scores
    // are out (its loads land while the workgroup waits for the group's other
    // slices, and the Q and K loads, which every workgroup issues at once,
    // do not share the memory system with them): at device scope right after
    // the partial stores, in an XL plan after the arrival (wave 0 only once
    // its wait is over).  A single slice has no wait to hide them behind, so
    // it loads V with Q and K.
    Raw bq[kQ], bk[kKV], bv[kKV];
    if constexpr (defer_v) issue(0, bq, bk, bv, n == 1);
    // The encoding operands of the first batch of Q rows and of K rows
    // (below), in the one-round forms fetched here, with the rows' loads, so
    // that their latency too hides behind the set-up.  Not where holding
    // them would bring the kernel to its 256 registers (fp32 rotate-half
    // beyond the smallest form, fp32 in the largest one-round form).
    constexpr int kEncBatch = PEK == kPeRopeHalf ? 4 : 8;
    constexpr bool kPrefetch = defer_v && PEK != kPeNone &&
                               (kBf16 || FORM == 1 || (FORM == 2 && PEK != kPeRopeHalf));
    constexpr int kPreQ = kQ < kEncBatch ? kQ : kEncBatch;
    constexpr int kPreK = kKV < kEncBatch ? kKV : kEncBatch;
    Pe4Ops<PEK> preq[kPreQ], prek[kPreK];
    auto enc_fetch = [&](bool isq, int row0, auto& o) {
        constexpr int NB = sizeof(o) / sizeof(o[0]);
        const int len = isq ? Lq : Lk, p0 = isq ? q0 : 0;
        const T* __restrict__ X = isq ? Q : K;
        const PeSide& pe = isq ? a.pq : a.pk;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int rc = min(row0 + u * rstep, len - 1);
            o[u] = pe4_fetch<T, PEK>(d, X + (size_t)rc * D, p0 + rc, D, pe);
        }
    };
    if constexpr (kPrefetch) {
        if (a.pq.on && pe4_batch_ok(PEK, a.pq)) enc_fetch(true, r0, preq);
        if (a.pk.on && pe4_batch_ok(PEK, a.pk)) enc_fetch(false, r0, prek);
    }

    const Geo g = make_geo(!kBf16, PEK != kPeNone, a.nchunk > 1, a.MB, Lk, dc);
    const int MQ = g.MQ, NK = g.NK, E = MQ * NK, nrb = MQ / 16;
    const int cq = r0 < rstep ? fdiv(MQ - r0 + rstep - 1, rstep, a.m_rstep) : 0;
    const int ckv = r0 < rstep ? fdiv(NK - r0 + rstep - 1, rstep, a.m_rstep) : 0;
    // hi and lo parts of 4 values: fp16 parts for fp32 inputs, bf16 parts
    // for bf16 inputs after a positional encoding
    auto split4 = [](const float (&e4)[4], uint2& w, uint2& wl) {
        if constexpr (kBf16) {
            split2_bf16(e4[0], e4[1], w.x, wl.x);
            split2_bf16(e4[2], e4[3], w.y, wl.y);
        } else {
            split2_f16(e4[0], e4[1], w.x, wl.x);
            split2_f16(e4[2], e4[3], w.y, wl.y);
        }
    };
    // fp32: the largest magnitudes of the Q/K values and of the V values
    // this thread stores (the fp16 split's range check)
    float big_qk = 0.f, big_v = 0.f;
    // one V row vector into LDS; s scales it by a power of two (a slice
    // staged again)
    auto store_v = [&](int row, Raw raw, float s = 1.f) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(smem + g.v_off) + row * g.vstr + col;
        if constexpr (kBf16) {
            // the raw bf16 bits, [key][dim]
            *reinterpret_cast<uint2*>(dst) = raw;
        } else {
            const float e4[4] = {raw.x * s, raw.y * s, raw.z * s, raw.w * s};
            big_v = vmax3abs(vmax3abs(big_v, e4[0], e4[1]), e4[2], e4[3]);
            uint2 w, wl;
            split4(e4, w, wl);
            *reinterpret_cast<uint2*>(dst) = w;
            *reinterpret_cast<uint2*>(dst + (g.vl_off - g.v_off) / 2) = wl;
        }
    };
    // one encoded row vector of Q (isq) or K into its LDS rows, scaled by s
    auto store_qk = [&](bool isq, int row, float4 f, float s = 1.f) {
        const float e4[4] = {f.x * s, f.y * s, f.z * s, f.w * s};
        if constexpr (!kBf16) big_qk = vmax3abs(vmax3abs(big_qk, e4[0], e4[1]), e4[2], e4[3]);
        const int off = row * (isq ? g.qstr : g.kstr) + col;
        uint16_t* hi = reinterpret_cast<uint16_t*>(smem + (isq ? g.q_off : g.k_off));
        uint2 w, wl;
        split4(e4, w, wl);
        *reinterpret_cast<uint2*>(hi + off) = w;
        if constexpr (kSplit) {
            uint16_t* lo = reinterpret_cast<uint16_t*>(smem + (isq ? g.ql_off : g.kl_off));
            *reinterpret_cast<uint2*>(lo + off) = wl;
        }
    };
    {
        // Rows kk = j * NR + u of Q (isq) or K in round j (loaded as r[NR]),
        // encoded, into LDS.  With the library's compact tables the rows go
        // kEncBatch at a time, every load of a batch (angles, rotate-half
        // partners) issued before its arithmetic, rows clamped into the
        // sequence so that every load is valid; otherwise (the caller's
        // duplicated tables) one row at a time.  A side without an encoding
        // (pe.on == 0) is stored as loaded.
        auto encode_store = [&](bool isq, int j, auto& r, auto& pre) {
            constexpr int NR = sizeof(r) / sizeof(r[0]);
            const int cnt = isq ? cq : ckv, len = isq ? Lq : Lk, p0 = isq ? q0 : 0;
            const T* __restrict__ X = isq ? Q : K;
            const PeSide& pe = isq ? a.pq : a.pk;
            if (!pe.on) {
#pragma unroll
                for (int u = 0; u < NR; ++u) {
                    const int kk = j * NR + u;
                    if (kk < cnt) store_qk(isq, r0 + kk * rstep, Raw4<T>::f4(r[u]));
                }
            } else if (pe4_batch_ok(PEK, pe)) {
#pragma unroll
                for (int b = 0; b < NR; b += kEncBatch) {
                    Pe4Ops<PEK> o[kEncBatch];
                    if (kPrefetch && b == 0) {
#pragma unroll
                        for (int u = 0; u < kEncBatch && u < NR; ++u) o[u] = pre[u];
                    } else {
#pragma unroll
                        for (int u = 0; u < kEncBatch && b + u < NR; ++u) {
                            const int rc = min(r0 + (j * NR + b + u) * rstep, len - 1);
                            o[u] = pe4_fetch<T, PEK>(d, X + (size_t)rc * D, p0 + rc, D, pe);
                        }
                    }
#pragma unroll
                    for (int u = 0; u < kEncBatch && b + u < NR; ++u) {
                        const int kk = j * NR + b + u, row = r0 + kk * rstep;
                        if (kk < cnt) {
                            float4 f = Raw4<T>::f4(r[b + u]);
                            if (lane_ok && row < len) f = pe4_apply<PEK>(f, o[u], d, D, pe);
                            store_qk(isq, row, f);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < NR; ++u) {
                    const int kk = j * NR + u, row = r0 + kk * rstep;
                    if (kk < cnt) {
                        float4 f = Raw4<T>::f4(r[u]);
                        if (lane_ok && row < len)
                            f = encode4<T, PEK>(f, X + (size_t)row * D, p0 + row, d, pe);
                        store_qk(isq, row, f);
                    }
                }
            }
        };
        // round j into LDS: Q and K (and, unless deferred, V)
        auto store_round = [&](int j, Raw (&q)[kQ], Raw (&k)[kKV], Raw (&v)[kKV],
                               bool store_v_now) {
            if constexpr (PEK != kPeNone) {
                encode_store(true, j, q, preq);
                encode_store(false, j, k, prek);
                if (store_v_now) {
#pragma unroll
                    for (int u = 0; u < kKV; ++u)
                        if (j * kKV + u < ckv) store_v(r0 + (j * kKV + u) * rstep, v[u]);
                }
                return;
            }
#pragma unroll
            for (int u = 0; u < kQ; ++u) {
                const int kk = j * kQ + u, row = r0 + kk * rstep;
                if (kk < cq) store_qk(true, row, Raw4<T>::f4(q[u]));
            }
#pragma unroll
            for (int u = 0; u < kKV; ++u) {
                const int kk = j * kKV + u, row = r0 + kk * rstep;
                if (kk < ckv) {
                    store_qk(false, row, Raw4<T>::f4(k[u]));
                    if (store_v_now) store_v(row, v[u]);
                }
            }
        };
        if constexpr (defer_v) {
            store_round(0, bq, bk, bv, false);
        } else {
            for (int j = 0; j * kQ < cq || j * kKV < ckv; ++j) {
                Raw q[kQ], k[kKV], v[kKV];
                issue(j, q, k, v, true);
                store_round(j, q, k, v, true);
            }
        }
    }
    if constexpr (!kBf16) {
        const bool over = __ballot(!(big_qk < kF16Range)) != 0;  // NaN counts as over
        if (lane == 0) sh_over[wave] = over;
    }
    if (tid == 0) flag = 1;
    __syncthreads();

    // fp32 slices with a value outside the fp16 split's range (rare): the
    // slice is loaded again and staged scaled by a power of two from its
    // largest finite magnitude, so that every scaled finite value converts;
    // the unit returned undoes the scaling exactly.  Rows past the sequence and
    // columns past D read as zeros, as in the staging above.
    auto load_row = [&](const __amdgpu_buffer_rsrc_t& r, int row) -> float4 {
        return Raw4<T>::f4(Raw4<T>::ld_buf(r, lane_ok ? (row * D + d) * es : kOob));
    };
    auto slice_max = [&](float m0, float m1, int slot) {
        // workgroup maxima of two per-thread values (slots slot, slot + 4)
        m0 = wave_max(m0);
        m1 = wave_max(m1);
        if (lane == 0) {
            sh_big[slot + wave] = m0;
            sh_big[slot + 4 + wave] = m1;
        }
        __syncthreads();
    };
    auto max4 = [&](int slot) {
        return fmaxf(fmaxf(sh_big[slot], sh_big[slot + 1]),
                     fmaxf(sh_big[slot + 2], sh_big[slot + 3]));
    };
    auto restage_qk = [&]() -> float {
        auto enc_row = [&](bool isq, int row) {
            float4 f = load_row(isq ? rq : rk, row);
            if constexpr (PEK != kPeNone)
                if (lane_ok && row < (isq ? Lq : Lk))
                    f = isq ? encode4<T, PEK>(f, Q + (size_t)row * D, q0 + row, d, a.pq)
                            : encode4<T, PEK>(f, K + (size_t)row * D, row, d, a.pk);
            return f;
        };
        // (loops kept rolled: this path must not raise the kernel's
        // register count, which sets its occupancy)
        float mq = 0.f, mk = 0.f;
        if (r0 < rstep) {
#pragma unroll 1
            for (int row = r0; row < MQ; row += rstep) {
                mq = max_finite4(mq, enc_row(true, row));
            }
#pragma unroll 1
            for (int row = r0; row < NK; row += rstep) {
                mk = max_finite4(mk, enc_row(false, row));
            }
        }
        slice_max(mq, mk, 0);
        mq = max4(0);
        mk = max4(4);
        const float sq = pow2_scale(mq), sk = pow2_scale(mk);
        if (r0 < rstep) {
#pragma unroll 1
            for (int row = r0; row < MQ; row += rstep) store_qk(true, row, enc_row(true, row), sq);
#pragma unroll 1
            for (int row = r0; row < NK; row += rstep) store_qk(false, row, enc_row(false, row), sk);
        }
        __syncthreads();
        return pow2_unit(mq) * pow2_unit(mk);
    };
    // unit of the partial scores: 1, or 1 / (sq sk) after a rescaled staging
    float unit_qk = 1.f;
    if constexpr (!kBf16) {
        const int4 ov = *reinterpret_cast<const int4*>(sh_over);
        if (ov.x | ov.y | ov.z | ov.w) unit_qk = restage_qk();
    }

    // ---- 2. partial scores S_c on MFMA.  Each wave owns one 16-row block
    // and up to 8 column tiles; the row block's A operand is read once per
    // k-step and shared by the tiles' independent accumulators.  With more
    // than one slice the partials go out as tagged words.
    // Partials of the group live in [E / 256][slice][256] order (E is a
    // multiple of 512), so that every read pattern of step 3 is one base
    // address plus a uniform stride per word.
    float* S = reinterpret_cast<float*>(smem + g.s_off);
    // the group's partials: byte offset 4 ((e / 256) n 256 + c 256 + e % 256)
    // of entry e of slice c
    const __amdgpu_buffer_rsrc_t rpart =
        make_rsrc(a.part + (size_t)rg * n * E, n > 1 ? n * E * 4 : 0);
    {
        int rb, c0, cs;
        const int cnt = wave_tiles(wave, nrb, NK / 16, &rb, &c0, &cs);
        auto store = [&](int u, const v4f& acc) {
            const int j = (c0 + u * cs) * 16 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = rb * 16 + lk * 4 + r;
                const int e = i * NK + j;
                const float v = kBf16 ? acc[r] : acc[r] * unit_qk;
                if (n > 1)
                    st_xb<XL>(v, rpart, ((e >> 8) * (n * 256) + c * 256 + (e & 255)) * 4);
                else S[i * g.sstr + j] = v;
            }
        };
        auto run = [&](auto nt_tag) {
            constexpr int NT = decltype(nt_tag)::value;
            v4f acc[NT];
#pragma unroll
            for (int u = 0; u < NT; ++u) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
            // tiles past cnt repeat the last valid tile (computed, not stored)
            const int bstep_rows = (cnt > 1 ? cs : 0) * 16;
            const uint16_t* qh = reinterpret_cast<const uint16_t*>(smem + g.q_off) +
                                 (rb * 16 + lr) * g.qstr + lk * 8;
            const uint16_t* kh = reinterpret_cast<const uint16_t*>(smem + g.k_off) +
                                 (c0 * 16 + lr) * g.kstr + lk * 8;
            const int ql_d = (g.ql_off - g.q_off) / 2, kl_d = (g.kl_off - g.k_off) / 2;
            mma16<VT, NT, kSplit, kSplit>(qh, qh + ql_d, kh, kh + kl_d, bstep_rows * g.kstr, dc,
                                          acc);
#pragma unroll
            for (int u = 0; u < NT; ++u)
                if (u < cnt) store(u, acc[u]);
        };
        if (cnt == 1) run(std::integral_constant<int, 1>{});
        else if (cnt == 2) run(std::integral_constant<int, 2>{});
        else if (cnt > 2 && cnt <= 4) run(std::integral_constant<int, 4>{});
        else if (cnt > 4) run(std::integral_constant<int, 8>{});
    }
    if constexpr (defer_v && !XL) {
        if (n > 1) {
            // after the partial stores, in issue order (kept there as the
            // slice loads are)
            __builtin_amdgcn_sched_barrier(0);
            issue_v(0, bv);
            flag = 1;
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- 3. all-reduce of S over the group's slices (tagged words, or
    // XCD-local arrival counters)
    if (n > 1) {
        // done word of slice c: rg + 32 c when the group's slices fit (each
        // in its own 128-byte line, instead of n words in one or two lines
        // that every slice of the group stores to and polls), else rg n + c
        const bool spread = n <= 64 && a.G <= 32;
        const int dstride = spread ? 32 : 1;
        unsigned* done1 = a.done + (spread ? rg : rg * n);
        unsigned* done2 = done1 + 2048;
        // XL: this slice's share of the call's units, the group's counters
        const unsigned share =
            c < n - 1 ? (unsigned)c + 1u : kXcdUnits - (unsigned)(n - 1) * (unsigned)n / 2u;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.xctr + xcd_slot, 4 * xk1 + 4);
        // reduce-scatter: this workgroup owns entries [e0, e1) of the group
        const int per_rs = fdiv(E + n - 1, n, a.m_n);
        const int e0_rs = min(E, c * per_rs), e1_rs = min(E, e0_rs + per_rs);
        // XL, on a path that leaves early: NaN into this workgroup's reduced
        // entries (late slices of the group read them), then the second
        // arrival, so the counter still gains its units
        auto xl_leave_before_step2 = [&]() {
            if (!a.gather1) {
                const float nan = __int_as_float(0x7fc00000);
                for (int e = e0_rs + tid; e < e1_rs; e += kThreads) a.red[(size_t)rg * E + e] = nan;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                xcd_arrive(rc, xk1, share, false, &flag);
            }
        };
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // stores stay above the wait
        // this wave's partials have completed: every vector memory operation
        // but the kKV V loads issued after them (vmcnt counts in issue order;
        // XL plans issue V later)
        if constexpr (defer_v && !XL) {
            static_assert(kKV == 8 || kKV == 16, "vmcnt encoding below");
            __builtin_amdgcn_s_waitcnt(kKV == 8 ? 0x0F78 : 0x4F70);  // vmcnt(kKV)
        } else {
            __builtin_amdgcn_s_waitcnt(0);
        }
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wuninitialized"
#pragma clang diagnostic ignored "-Wsometimes-uninitialized"
        if (tid == 0) {  // thread 0 loaded both (n > 1)
            sh_epoch = ep_r;
            sh_failed = failed_r;
        }
#pragma clang diagnostic pop
        __syncthreads();
        const unsigned epoch = sh_epoch;
        const unsigned tag = exchange_tag(epoch, rg);
        unsigned base1 = 0;
        if constexpr (XL) base1 = xcd_arrive_only(rc, 0, share);
        else if (tid == 0) st_done(done1 + c * dstride, tag);
        if (sh_failed) {  // an earlier call timed out: fail closed
            if constexpr (XL) {
                __syncthreads();
                xl_leave_before_step2();
            }
            poison_slice<T>(O, orow0, Lq, D, d0, dc);
            return;
        }
        // V into LDS while the other slices of the group arrive.  XL plans:
        // waves 1-3 load V only now, once the arrival is out; wave 0, which
        // polls, only once its wait is over (its atomic's return and its
        // polls would otherwise wait for V: vmcnt retires in issue order);
        // every wave then writes V to LDS while its exchange loads are in
        // flight.
        auto store_v_all = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < kKV; ++u)
                if (u < ckv) store_v(r0 + u * rstep, bv[u]);
        };
        if constexpr (defer_v) {
            if constexpr (XL) {
                if (wave != 0) {
                    __builtin_amdgcn_sched_barrier(0);
                    issue_v(0, bv);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
#pragma unroll
                for (int u = 0; u < kKV; ++u)
                    if (u < ckv) store_v(r0 + u * rstep, bv[u]);
            }
        }
        const float* pg = a.part + (size_t)rg * n * E;
        float* rd = a.red + (size_t)rg * E;
        // returns false (for the whole workgroup) on a timeout; step = the
        // exchange step that timed out
        int step = 1;
        auto exchange = [&]() -> bool {
            float w[kMaxWords];
            if constexpr (XL) {
                if (!xcd_wait(rc, 0, base1, &flag)) return false;
                if constexpr (defer_v)
                    if (wave == 0) {
                        __builtin_amdgcn_sched_barrier(0);
                        issue_v(0, bv);
                        __builtin_amdgcn_sched_barrier(0);
                    }
            } else {
                if (!wait_done(done1, n, dstride, tag, &flag)) return false;
            }
            if (a.gather1) {
                // one gather, 16-byte words: thread t sums entries 4 (t % 64)
                // .. + 3 of 256-entry blocks t / 64 + 4 i, every slice's
                // partial of each in slice order; vector u = i * n + slice.
                // Every vector slot is loaded (slots past this wave's
                // blocks from an offset past the buffer, which reads
                // zeros), so the loads carry no branches; the block and
                // slice counters are wave-uniform (scalar).
                const int nblk = E >> 8, b0 = tid >> 6;  // 256-entry blocks
                const int nb =
                    __builtin_amdgcn_readfirstlane(b0 < nblk ? (nblk - b0 + 3) / 4 : 0);
                const int cnt = nb * n;
                const __amdgpu_buffer_rsrc_t rs = make_rsrc(pg, n * E * 4);
                const int voff = (b0 * n * 256 + (tid & 63) * 4) * 4;
                constexpr int kOobX = 0x7ffffff0;  // past every buffer
                float4 w4[kMaxWords / 4];
                {
                    int i = 0, p = 0;
#pragma unroll
                    for (int u = 0; u < kMaxWords / 4; ++u) {
                        w4[u] = ld_x4<XL>(rs, u < cnt ? voff + (4 * i * n + p) * 1024 : kOobX);
                        if (++p == n) {
                            p = 0;
                            ++i;
                        }
                    }
                }
                if constexpr (XL && defer_v) store_v_all();
                // sums in slice order (the zeros past the last block are
                // never stored); 4 consecutive entries share one row of S
                const int e0 = b0 * 256 + (tid & 63) * 4;
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
                int p = 0, i = 0;
#pragma unroll
                for (int u = 0; u < kMaxWords / 4; ++u) {
                    acc.x += w4[u].x;
                    acc.y += w4[u].y;
                    acc.z += w4[u].z;
                    acc.w += w4[u].w;
                    if (++p == n) {
                        if (i < nb) {
                            const int e = e0 + i * 1024;
                            const int r = fdiv(e, NK, a.m_nk);
                            *reinterpret_cast<float4*>(&S[r * g.sstr + (e - r * NK)]) = acc;
                        }
                        acc = make_float4(0.f, 0.f, 0.f, 0.f);
                        p = 0;
                        ++i;
                    }
                }
                return true;
            }
            // reduce-scatter: this workgroup owns entries [e0, e1)
            const int e0 = e0_rs, e1 = e1_rs;
            const int cnt_e = max(0, e1 - e0);
            float* redl = reinterpret_cast<float*>(smem + g.red_off);
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(pg, n * E * 4);
            if (E % (16 * n) == 0 && cnt_e <= 4 * kThreads &&
                (n + kThreads / (cnt_e >> 2) - 1) / (kThreads / (cnt_e >> 2)) <= kMaxWords / 4) {
                // 16-byte words: G groups of cnt_e / 4 threads, each thread 4
                // consecutive entries (a 4-aligned run never crosses a
                // 256-entry block); group q sums slices q, q + G, ...
                const int c4 = cnt_e >> 2;
                const int G = kThreads / c4;  // scalar divisions, then multipliers
                const unsigned mc4 = fused_div_magic(c4), mg = fused_div_magic(G);
                const int grp = fdiv(tid, c4, mc4), el4 = tid - grp * c4;
                const int cnt = grp < G ? fdiv(n - grp + G - 1, G, mg) : 0;
                const int e = e0 + 4 * el4;
                const int voff = (((e >> 8) * n + grp) * 256 + (e & 255)) * 4;
                // slots up to the wave's largest count are loaded (a
                // wave-uniform branch; a lane's absent slots read zeros from
                // past the buffer) and every slot is summed
                constexpr int kOobX = 0x7ffffff0;
                const int cmax = __builtin_amdgcn_readfirstlane(cnt);  // lane 0: smallest group
                float4 w4[kMaxWords / 4];
#pragma unroll
                for (int u = 0; u < kMaxWords / 4; ++u)
                    w4[u] = u < cmax ? ld_x4<XL>(rs, u < cnt ? voff + u * G * 1024 : kOobX)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int u = 0; u < kMaxWords / 4; ++u) {
                    acc.x += w4[u].x;
                    acc.y += w4[u].y;
                    acc.z += w4[u].z;
                    acc.w += w4[u].w;
                }
                reinterpret_cast<float4*>(redl)[tid] = acc;
                __syncthreads();
                if (tid < c4) {
                    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
                    for (int q = 0; q < G; ++q) {
                        const float4 v = reinterpret_cast<const float4*>(redl)[q * c4 + tid];
                        sum.x += v.x;
                        sum.y += v.y;
                        sum.z += v.z;
                        sum.w += v.w;
                    }
                    st_xb4<XL>(sum, make_rsrc(rd, E * 4), (e0 + 4 * tid) * 4);
                }
            } else if (cnt_e <= kThreads) {
                // G groups of cnt_e threads; group q sums slices q, q + G, ...
                const int G = cnt_e > 0 ? kThreads / cnt_e : 1;
                const int el = cnt_e > 0 ? tid % cnt_e : 0;
                const int grp = cnt_e > 0 ? tid / cnt_e : G;
                const int cnt = grp < G ? (n - grp + G - 1) / G : 0;
                const int e = e0 + el;
                ld_words<XL, kMaxWords>(pg + ((e >> 8) * n + grp) * 256 + (e & 255), G * 256, cnt,
                                        w);
                float acc = 0.f;
#pragma unroll
                for (int u = 0; u < kMaxWords; ++u)
                    if (u < cnt) acc += w[u];
                redl[tid] = acc;
                __syncthreads();
                if (tid < cnt_e) {
                    float sum = 0.f;
                    for (int q = 0; q < G; ++q) sum += redl[q * cnt_e + tid];
                    st_x<XL>(rd + e0 + tid, sum);
                }
            } else {
                // entries e0 + tid + 256 k, every slice of each; word
                // u = k * n + slice
                const int ne = tid < cnt_e ? (cnt_e - tid + kThreads - 1) / kThreads : 0;
                const int cnt = ne * n;
                const int e = e0 + tid;
                ld_words<XL, kMaxWords>(pg + (e >> 8) * n * 256 + (e & 255), 256, cnt, w);
                float acc = 0.f;
                int p = 0, k = 0;
#pragma unroll
                for (int u = 0; u < kMaxWords; ++u) {
                    if (u < cnt) {
                        acc += w[u];
                        if (++p == n) {
                            st_x<XL>(rd + e + k * kThreads, acc);
                            acc = 0.f;
                            p = 0;
                            ++k;
                        }
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_waitcnt(0);  // this wave's reduced words have completed
            __syncthreads();
            // all-gather: the reduced S into LDS, 16-byte words (E is a
            // multiple of 512): vectors tid + 256 u
            step = 2;
            if constexpr (XL) {
                const unsigned base2 = xcd_arrive_only(rc, xk1, share);
                if constexpr (defer_v) store_v_all();
                if (!xcd_wait(rc, xk1, base2, &flag)) return false;
            } else {
                if (tid == 0) st_done(done2 + c * dstride, tag);
                if (!wait_done(done2, n, dstride, tag, &flag)) return false;
            }
            // vectors tid + 256 u, u < nv (a wave-uniform bound; a lane's
            // vectors past E read zeros from past the buffer); 4
            // consecutive entries share one row of S.  E <= 64 x 128, so
            // nv <= 8.
            constexpr int kAgMax = 8;
            const __amdgpu_buffer_rsrc_t rr = make_rsrc(rd, E * 4);
            const int nv = __builtin_amdgcn_readfirstlane(((E >> 2) + kThreads - 1) / kThreads);
            float4 w4[kAgMax];
#pragma unroll
            for (int u = 0; u < kAgMax; ++u)
                w4[u] = u < nv ? ld_x4<XL>(rr, (tid + u * kThreads) * 16)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < kAgMax; ++u) {
                const int e = 4 * (tid + u * kThreads);
                if (u < nv && e < E) {
                    const int r = fdiv(e, NK, a.m_nk);
                    *reinterpret_cast<float4*>(&S[r * g.sstr + (e - r * NK)]) = w4[u];
                }
            }
            return true;
        };
        if (!exchange()) {
            if (tid == 0)
                __hip_atomic_fetch_or(a.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if constexpr (XL)
                if (step == 1) xl_leave_before_step2();
            poison_slice<T>(O, orow0, Lq, D, d0, dc);
            return;
        }
        // this workgroup has seen words of every slice of the group, so every
        // workgroup of the group has read `epoch`: advance it
        if constexpr (!XL)
            if (c == 0 && tid == 0)
                __hip_atomic_store(a.epochs + rg, epoch + 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    if (defer_v && n == 1) {
#pragma unroll
        for (int u = 0; u < kKV; ++u)
            if (u < ckv) store_v(r0 + u * rstep, bv[u]);
    }
    if constexpr (!kBf16) {
        const bool over = __ballot(!(big_v < kF16Range)) != 0;  // NaN counts as over
        if (lane == 0) sh_over[4 + wave] = over;
    }
    __syncthreads();

    // ---- 4. softmax of scale * S: T = 16, 8 or 4 consecutive threads per
    // row (as many as 256 threads allow for MQ rows), each a run of NK / T
    // columns; DPP reductions within the T lanes; P to its own LDS region
    {
        auto run = [&](auto t_tag, auto w_tag) {
            constexpr int TT = decltype(t_tag)::value, W = decltype(w_tag)::value;
            const int i = tid / TT, j0 = (tid % TT) * W;
            if (i >= MQ) return;  // whole waves (MQ * TT is a multiple of 64)
            const bool row_ok = i < Lq;
            float v[W];
            float m = -INFINITY;
#pragma unroll
            for (int u = 0; u < W; u += 2) {
                const float2 x = *reinterpret_cast<const float2*>(&S[i * g.sstr + j0 + u]);
                v[u] = (row_ok && j0 + u < Lk) ? x.x * a.scale : -INFINITY;
                v[u + 1] = (row_ok && j0 + u + 1 < Lk) ? x.y * a.scale : -INFINITY;
                m = fmaxf(m, fmaxf(v[u], v[u + 1]));
            }
            m = fmaxf(m, dpp<kDppQuadXor1>(m));
            m = fmaxf(m, dpp<kDppQuadXor2>(m));
            if constexpr (TT >= 8) m = fmaxf(m, dpp<kDppRowHalfMirror>(m));
            if constexpr (TT >= 16) m = fmaxf(m, dpp<kDppRowMirror>(m));
            float l = 0.f;
#pragma unroll
            for (int u = 0; u < W; ++u) {
                v[u] = row_ok ? __expf(v[u] - m) : 0.f;
                l += v[u];
            }
            l += dpp<kDppQuadXor1>(l);
            l += dpp<kDppQuadXor2>(l);
            if constexpr (TT >= 8) l += dpp<kDppRowHalfMirror>(l);
            if constexpr (TT >= 16) l += dpp<kDppRowMirror>(l);
            // fp32: P scaled by 2^15 (exact; every p <= 1 converts, and small
            // p keep their bits), undone with the output
            const float inv = row_ok ? (kBf16 ? 1.0f : 32768.0f) / l : 0.f;
#pragma unroll
            for (int u = 0; u < W; u += 2) {
                const float p0 = v[u] * inv, p1 = v[u + 1] * inv;
                uint16_t* ph = reinterpret_cast<uint16_t*>(smem + g.p_off);
                uint32_t h, lo;
                if constexpr (kBf16) split2_bf16(p0, p1, h, lo);
                else split2_f16(p0, p1, h, lo);
                *reinterpret_cast<uint32_t*>(&ph[i * g.pstr + j0 + u]) = h;
                *reinterpret_cast<uint32_t*>(&ph[(MQ + i) * g.pstr + j0 + u]) = lo;
            }
        };
        using std::integral_constant;
        if (MQ <= 16) {
            switch (NK) {
                case 32: run(integral_constant<int, 16>{}, integral_constant<int, 2>{}); break;
                case 64: run(integral_constant<int, 16>{}, integral_constant<int, 4>{}); break;
                case 96: run(integral_constant<int, 16>{}, integral_constant<int, 6>{}); break;
                default: run(integral_constant<int, 16>{}, integral_constant<int, 8>{}); break;
            }
        } else if (MQ <= 32) {
            switch (NK) {
                case 32: run(integral_constant<int, 8>{}, integral_constant<int, 4>{}); break;
                case 64: run(integral_constant<int, 8>{}, integral_constant<int, 8>{}); break;
                case 96: run(integral_constant<int, 8>{}, integral_constant<int, 12>{}); break;
                default: run(integral_constant<int, 8>{}, integral_constant<int, 16>{}); break;
            }
        } else {
            switch (NK) {
                case 32: run(integral_constant<int, 4>{}, integral_constant<int, 8>{}); break;
                case 64: run(integral_constant<int, 4>{}, integral_constant<int, 16>{}); break;
                case 96: run(integral_constant<int, 4>{}, integral_constant<int, 24>{}); break;
                default: run(integral_constant<int, 4>{}, integral_constant<int, 32>{}); break;
            }
        }
    }
    __syncthreads();

    // fp32: V staged again, scaled, when a V value is outside the fp16
    // split's range (rare; see restage_qk); unit_o undoes P's 2^15 and V's
    // scale in the output
    float unit_o = 1.f;
    if constexpr (!kBf16) {
        unit_o = 1.0f / 32768.0f;
        const int4 ov = *reinterpret_cast<const int4*>(sh_over + 4);
        if (ov.x | ov.y | ov.z | ov.w) {
            float mv = 0.f;
            if (r0 < rstep)
#pragma unroll 1
                for (int row = r0; row < NK; row += rstep) mv = max_finite4(mv, load_row(rv, row));
            slice_max(mv, 0.f, 0);
            mv = max4(0);
            const float sv = pow2_scale(mv);
            if (r0 < rstep)
#pragma unroll 1
                for (int row = r0; row < NK; row += rstep)
                    store_v(row, Raw4<T>::ld_buf(rv, lane_ok ? (row * D + d) * es : kOob), sv);
            __syncthreads();
            unit_o *= pow2_unit(mv);
        }
    }

    // ---- 5. O[:, slice] = P V[:, slice] on MFMA: each wave owns one 16-row
    // block and every (4 / nrb)-th 16-dim tile, 8 tiles at a time
    {
        int rb, c0, cs;
        const int cnt = wave_tiles(wave, nrb, dc / 16, &rb, &c0, &cs);
        // output stores through a buffer resource over the group's rows:
        // 32-bit offsets, and rows past the sequence fall past its range
        constexpr int es = (int)sizeof(T);
        const __amdgpu_buffer_rsrc_t ro = make_rsrc(O + orow0 * D, Lq * D * es);
        const int obase = (rb * 16 + lk * 4) * D + d0 + lr;  // element of row 0 of the lane
        for (int t0 = 0; t0 < cnt; t0 += 8) {
            const int left = cnt - t0;
            const int tc = c0 + t0 * cs;  // first tile of this group
            auto run = [&](auto nt_tag) {
                constexpr int NT = decltype(nt_tag)::value;
                v4f acc[NT];
#pragma unroll
                for (int u = 0; u < NT; ++u) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
                const int step = (left > 1 ? cs : 0) * 16;  // repeats past `left`, unstored
                const uint16_t* ph = reinterpret_cast<const uint16_t*>(smem + g.p_off) +
                                     (rb * 16 + lr) * g.pstr + lk * 8;
                const uint16_t* vb = reinterpret_cast<const uint16_t*>(smem + g.v_off) + tc * 16;
                mma16_vt<VT, NT, kVlo>(ph, ph + MQ * g.pstr, vb, (g.vl_off - g.v_off) / 2, g.vstr,
                                       step, NK, acc);
#pragma unroll
                for (int u = 0; u < NT; ++u) {
                    if (u >= left) break;
                    const int col = (tc + u * cs) * 16;
                    if (d0 + col + lr >= D) continue;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int off = (obase + r * D + col) * es;
                        if constexpr (kBf16)
                            __builtin_amdgcn_raw_buffer_store_b16(
                                __builtin_bit_cast(uint16_t, (__bf16)acc[u][r]), ro, off, 0, 0);
                        else
                            __builtin_amdgcn_raw_buffer_store_b32(
                                __float_as_uint(acc[u][r] * unit_o), ro, off, 0, 0);
                    }
                }
            };
            if (left == 1) run(std::integral_constant<int, 1>{});
            else if (left == 2) run(std::integral_constant<int, 2>{});
            else if (left <= 4) run(std::integral_constant<int, 4>{});
            else run(std::integral_constant<int, 8>{});
        }
    }
}

// Raises the kernel's dynamic-LDS limit once to the largest size used
// (160 KiB per workgroup on gfx950).
template <typename T, int PEK, bool XL, int FORM>
hipError_t ensure_lds_limit(int lds) {
    static std::atomic<int> set{0};
    if (lds <= set.load(std::memory_order_acquire)) return hipSuccess;
    const int want = 160 * 1024 - 256;
    hipError_t e = hipFuncSetAttribute((const void*)k_fused_small<T, PEK, XL, FORM>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, want);
    if (e == hipSuccess) set.store(want, std::memory_order_release);
    return e;
}

template <typename T, int PEK, bool XL, int FORM>
hipError_t launch_t(const FusedArgs& a, int lds, hipStream_t st) {
    hipError_t e = ensure_lds_limit<T, PEK, XL, FORM>(lds);
    if (e != hipSuccess) return e;
    // XL: 8 XCDs x (row groups per XCD, rounded up) x slices
    const unsigned grid = XL ? (unsigned)(8 * ((a.G + 7) / 8) * a.nchunk)
                             : (unsigned)(a.G * a.nchunk);
    hipLaunchKernelGGL((k_fused_small<T, PEK, XL, FORM>), dim3(grid), dim3(kThreads), lds, st, a);
    return hipGetLastError();
}

template <typename T, int PEK, bool XL, int FORM>
int per_cu_t(int lds) {
    int per = 0;
    if (ensure_lds_limit<T, PEK, XL, FORM>(lds) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_fused_small<T, PEK, XL, FORM>,
                                                     kThreads, lds) != hipSuccess)
        return 0;
    return per;
}


// Launch of variant (T, XL) for encoding pek and load form `form`.
template <typename T, bool XL>
hipError_t fused_dispatch(const FusedArgs& a, int pek, int form, int lds, hipStream_t st) {
#define ATN_FUSED_PE(DV)                                                                  \
    switch (pek) {                                                                        \
        case kPeNone: return launch_t<T, kPeNone, XL, DV>(a, lds, st);                   \
        case kPeRopeInterleaved: return launch_t<T, kPeRopeInterleaved, XL, DV>(a, lds, st); \
        case kPeRopeHalf: return launch_t<T, kPeRopeHalf, XL, DV>(a, lds, st);           \
        case kPeSinusoidal: return launch_t<T, kPeSinusoidal, XL, DV>(a, lds, st);       \
        default: return hipErrorInvalidValue;                                             \
    }
    switch (form) {
        case 1: ATN_FUSED_PE(1)
        case 2: ATN_FUSED_PE(2)
        case 3: ATN_FUSED_PE(3)
        default: ATN_FUSED_PE(0)
    }
#undef ATN_FUSED_PE
}

// Occupancy of variant (T, XL): the smallest figure over every encoding and
// load form, so that the plan's residency holds for whichever variant a
// call launches.
template <typename T, bool XL, int PEK>
int fused_per_cu_pek(int lds) {
    int m = per_cu_t<T, PEK, XL, 0>(lds);
    m = std::min(m, per_cu_t<T, PEK, XL, 1>(lds));
    m = std::min(m, per_cu_t<T, PEK, XL, 2>(lds));
    return std::min(m, per_cu_t<T, PEK, XL, 3>(lds));
}
template <typename T, bool XL>
int fused_per_cu_forms(int lds) {
    return std::min(std::min(fused_per_cu_pek<T, XL, kPeNone>(lds),
                             fused_per_cu_pek<T, XL, kPeRopeInterleaved>(lds)),
                    std::min(fused_per_cu_pek<T, XL, kPeRopeHalf>(lds),
                             fused_per_cu_pek<T, XL, kPeSinusoidal>(lds)));
}

}  // namespace

}  // namespace atn
