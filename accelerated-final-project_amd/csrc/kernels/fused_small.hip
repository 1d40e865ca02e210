// Single-launch split-D attention for short sequences and large head_dim
// (gfx950): len_q <= 64, len_k <= 128, any D.
//
// The reference's headline shapes (e.g. B=1, H=4, L=64, D=2048) move a few
// MiB and hold a 64x64 score matrix per head, so one query row per
// workgroup (final/attention.cu:209-215) leaves the chip idle.  Here head bh
// is cut along D into `nchunk` slices of `dc` dims and workgroup (bh, c):
//
//   1. loads its Q/K/V slices once (16-byte loads, 8 in flight per thread;
//      the positional encoding is applied to Q and K at load) into LDS;
//   2. computes the partial scores S_c = Q[:, c] K[:, c]^T on MFMA
//      (fp32: v_mfma_f32_16x16x4_f32; bf16: v_mfma_f32_16x16x32_bf16, with
//      encoded Q/K split into hi + lo bf16 parts so nothing is lost to
//      re-rounding), four independent 16x16 tiles per wave;
//   3. all-reduces S over the head's slices through global memory: every
//      workgroup publishes S_c, meets the others at barrier A, reduces
//      1/nchunk of the entries over all slices (reduce-scatter), meets them
//      at barrier B and reads the whole reduced S (all-gather) -- a fixed
//      summation order, so results are bit-reproducible;
//   4. exact softmax of scale * S per row (max, exp, sum, divide;
//      final/attention.cu:262-270), four threads per row;
//   5. O[:, slice] = P V[:, slice] on MFMA (bf16: P split into hi + lo bf16
//      parts), one store per output element.
//
// Every Q, K, V element is read from HBM once and O is written once.
//
// Cross-workgroup exchange.  The partial and reduced scores and the barrier
// words are accessed only with device-scope (agent) atomic loads and stores,
// which gfx950 performs at the device's coherence point, so no L2 write-back
// or invalidate is needed; a workgroup waits for its own exchange stores to
// complete (s_waitcnt) before it publishes its flag.
//
// Barriers without counters.  Each head has an epoch word and each
// workgroup one 64-bit flag word, both at fixed places in the workspace's
// sync region.  A call reads its head's epoch e at start, publishes
// (e, head, 1) at barrier A and (e, head, 2) at barrier B; a waiter accepts
// phase 1 or 2 resp. exactly phase 2 of (e, head).  After barrier B every
// workgroup of the head has read e, so workgroup 0 of the head then stores
// e + 1.  Nothing needs resetting between calls, no two workgroups write the
// same word, kernel arguments do not change from call to call (a captured
// HIP graph replays correctly), and a word left by another head, another
// layout or an earlier epoch never matches.  Waits are bounded: on a
// timeout the workgroup sets the status word, writes NaN to its output
// slice and exits, so every wave ends; while the status word is set, later
// calls fail closed the same way until the host clears the sync region.
// The host launches at most as many workgroups as the device holds at once.
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace atn {

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kSpinLimit = 1 << 18;  // polls (each >= one memory round trip): ~0.3 s bound

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

// LDS geometry of one workgroup.  Element strides are chosen so that the
// MFMA operand reads are free of bank conflicts: fp32 A operands (Q, P)
// read 16 rows x 2 columns per half-wave -> row stride = 2 (mod 32); fp32 V
// (B operand of PV) reads 2 rows x 16 columns -> stride = 16 (mod 32); the
// softmax reads 8 rows x 4 columns of S -> stride = 4 (mod 32).  bf16 rows
// are padded by 8 elements (16-byte aligned 8-element reads).
struct Geo {
    int MQ, NK, dc;
    int qstr, kstr, vstr, sstr, pstr;
    int q_off, k_off, ql_off, kl_off, v_off, s_off, p_off, red_off;  // byte offsets
    int bytes;
};

// split: bf16 Q/K are kept as hi + lo parts (encoded inputs).
__host__ __device__ inline Geo make_geo(bool bf16, bool split, int Lq, int Lk, int dc) {
    Geo g{};
    g.MQ = (Lq + 15) / 16 * 16;
    g.NK = (Lk + 31) / 32 * 32;
    g.dc = dc;
    const int es = bf16 ? 2 : 4;
    if (bf16) {
        g.qstr = g.kstr = dc + 8;
        g.vstr = g.NK + 8;  // V stored transposed: [dim][key]
        g.pstr = g.NK + 8;  // P hi and lo, [row][key]
    } else {
        g.qstr = g.kstr = dc + 2;
        g.vstr = dc + 16;   // V stored [key][dim]
        g.pstr = g.NK + 2;
    }
    g.sstr = g.NK + 4;
    int off = 0;
    auto take = [&](int b) { int o = off; off += (b + 15) / 16 * 16; return o; };
    g.q_off = take(g.MQ * g.qstr * es);
    g.k_off = take(g.NK * g.kstr * es);
    g.ql_off = (bf16 && split) ? take(g.MQ * g.qstr * es) : g.q_off;
    g.kl_off = (bf16 && split) ? take(g.NK * g.kstr * es) : g.k_off;
    g.v_off = take((bf16 ? dc * g.vstr : g.NK * g.vstr) * es);
    g.s_off = take(g.MQ * g.sstr * 4);
    g.p_off = take(bf16 ? 2 * g.MQ * g.pstr * 2 : g.MQ * g.pstr * 4);
    g.red_off = take(kThreads * 4);
    g.bytes = off;
    return g;
}

struct FusedArgs {
    const void* Q;
    const void* K;
    const void* V;
    void* O;
    float* part;                // [BH][nchunk][E] partial scores
    float* red;                 // [BH][E] reduced scores
    unsigned* epochs;           // [BH] per-head epoch words (sync region)
    unsigned long long* flags;  // [BH][nchunk] barrier flags (sync region)
    int* status;                // nonzero after a barrier timeout
    int Lq, Lk, D, dc, nchunk;
    float scale;
    PeSide pq, pk;
};

__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long flag_word(unsigned epoch, int bh, int phase) {
    return ((unsigned long long)epoch << 32) | ((unsigned long long)(unsigned)bh << 2) |
           (unsigned long long)phase;
}

// Publishes `val` in this workgroup's flag, then waits until every flag of
// the head equals `want` or `want_alt`.  Returns false (for the whole
// workgroup) on timeout.
__device__ bool head_sync(unsigned long long* flags, int c, int n, unsigned long long val,
                          unsigned long long want, unsigned long long want_alt, int* status,
                          int* flag_lds) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's exchange stores have completed
    __syncthreads();
    if (threadIdx.x < 64) {
        if (threadIdx.x == 0)
            __hip_atomic_store(flags + c, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool ok = true;
        for (int it = 0;; ++it) {
            int mine = 1;
            for (int i = threadIdx.x; i < n; i += 64) {
                const unsigned long long f =
                    __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                mine &= (f == want) | (f == want_alt);
            }
            if (__all(mine)) break;
            if (it > kSpinLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (threadIdx.x == 0) {
            if (!ok) __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag_lds = ok ? 1 : 0;
        }
    }
    __syncthreads();
    return *flag_lds != 0;
}

template <typename T>
__device__ void poison_slice(T* O, int bh, int Lq, int D, int d0, int dc) {
    const float nan = __int_as_float(0x7fc00000);
    for (int f = threadIdx.x; f < Lq * dc; f += kThreads) {
        const int r = f / dc, d = d0 + f % dc;
        if (d < D) Elem<T>::st(O, ((size_t)bh * Lq + r) * D + d, nan);
    }
}

__device__ __forceinline__ bf16x8 lds8(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}

// NT independent 16x16 fp32 MFMA accumulations sharing one A operand:
// acc[u] += sum_k A[k] B_u[k] over k in [0, kdim) step 4, where lane
// (lr, lk) reads A at a[kk * ak] and tile u's B at b[u * bstep + kk * bk]
// (a, b already offset to the lane's row and k = lk).  kdim is a multiple
// of 32: the operands of 8 k-steps are read from LDS first, then the 8 x NT
// MFMAs issue back to back (no control flow inside, so the accumulators
// stay in place).
template <int NT>
__device__ __forceinline__ void mma_f32(const float* a, int ak, const float* b, int bstep,
                                        int bk, int kdim, v4f (&acc)[NT]) {
    for (int kb = 0; kb < kdim; kb += 32) {
        float av[8], bv[8][NT];
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const int kk = kb + 4 * st;
            av[st] = a[kk * ak];
#pragma unroll
            for (int u = 0; u < NT; ++u) bv[st][u] = b[u * bstep + kk * bk];
        }
#pragma unroll
        for (int st = 0; st < 8; ++st)
#pragma unroll
            for (int u = 0; u < NT; ++u)
                acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[st], bv[st][u], acc[u], 0, 0, 0);
    }
}

// bf16 form (k step 32, 8 elements per lane, contiguous along k), same
// prefetch scheme.  With ALO the A operand is a_hi + a_lo (two MFMAs); with
// BLO as well the three-term product a_hi b + a_hi b_lo + a_lo b.
template <int NT, bool ALO, bool BLO>
__device__ __forceinline__ void mma_bf16(const uint16_t* a, const uint16_t* a_lo,
                                         const uint16_t* b, const uint16_t* b_lo, int bstep,
                                         int kdim, v4f (&acc)[NT]) {
    bf16x8 ah = lds8(a), al{};
    if constexpr (ALO) al = lds8(a_lo);
    bf16x8 bv[NT], bl[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        bv[u] = lds8(b + u * bstep);
        if constexpr (BLO) bl[u] = lds8(b_lo + u * bstep);
    }
    for (int kk = 0; kk < kdim; kk += 32) {
        const int kn = min(kk + 32, kdim - 32);
        const bf16x8 ahn = lds8(a + kn);
        bf16x8 aln{};
        if constexpr (ALO) aln = lds8(a_lo + kn);
        bf16x8 bvn[NT], bln[NT];
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            bvn[u] = lds8(b + u * bstep + kn);
            if constexpr (BLO) bln[u] = lds8(b_lo + u * bstep + kn);
        }
#pragma unroll
        for (int u = 0; u < NT; ++u) {
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bv[u], acc[u], 0, 0, 0);
            if constexpr (BLO)
                acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl[u], acc[u], 0, 0, 0);
            if constexpr (ALO)
                acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bv[u], acc[u], 0, 0, 0);
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

// Wave -> (16-row block, set of 16-column tiles) for an output of nrb row
// blocks and `tiles` column tiles: waves w and w + nrb share a row block and
// take every (4 / nrb)-th column tile.  Returns the number of tiles (0 for
// an idle wave).
__device__ __forceinline__ int wave_tiles(int wave, int nrb, int tiles, int* rb, int* c0,
                                          int* cstep) {
    const int wpr = 4 / nrb;  // waves per row block (nrb <= 4)
    *rb = wave % nrb;
    *c0 = wave / nrb;
    *cstep = wpr;
    if (wave >= nrb * wpr || *c0 >= tiles) return 0;
    return (tiles - *c0 + wpr - 1) / wpr;
}

template <typename T, int PEK>
__global__ __launch_bounds__(kThreads) void k_fused_small(FusedArgs a) {
    constexpr bool kBf16 = sizeof(T) == 2;
    constexpr bool kSplit = kBf16 && PEK != kPeNone;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int flag;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
    const int lr = lane & 15, lk = lane >> 4;
    const int bh = blockIdx.x / a.nchunk, c = blockIdx.x % a.nchunk;
    const int Lq = a.Lq, Lk = a.Lk, D = a.D, dc = a.dc, n = a.nchunk;
    const int d0 = c * dc;
    const Geo g = make_geo(kBf16, kSplit, Lq, Lk, dc);
    const int MQ = g.MQ, NK = g.NK, E = MQ * NK, nrb = MQ / 16;

    const T* __restrict__ Q = static_cast<const T*>(a.Q) + (size_t)bh * Lq * D;
    const T* __restrict__ K = static_cast<const T*>(a.K) + (size_t)bh * Lk * D;
    const T* __restrict__ V = static_cast<const T*>(a.V) + (size_t)bh * Lk * D;
    T* __restrict__ O = static_cast<T*>(a.O);

    // the head's epoch and the status word, read while the slices load
    unsigned epoch = 0;
    int failed = 0;
    if (n > 1) {
        epoch = __hip_atomic_load(a.epochs + bh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        failed = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- 1. Q, K, V slices -> LDS.  Thread t owns 4-element column group
    // t % vpr of rows t / vpr, t / vpr + rstep, ... of the stacked row space
    // [Q: MQ rows | K: NK rows | V: NK rows]; 8 predicated vector loads are
    // issued before their LDS stores.  (The host sends this kernel only
    // shapes with D % 4 == 0 and aligned bases, so a vector is in or out.)
    {
        const int vpr = dc >> 2;
        const int rstep = kThreads / vpr;
        const int cg = tid % vpr, r0 = tid / vpr;
        const int d = d0 + cg * 4;
        const bool lane_ok = r0 < rstep && d < D;
        const int R = MQ + 2 * NK;
        for (int rb0 = r0; rb0 < R; rb0 += 8 * rstep) {
            float4 buf[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int row = rb0 + u * rstep;
                const bool isq = row < MQ, isk = !isq && row < MQ + NK;
                const int lrow = isq ? row : (isk ? row - MQ : row - MQ - NK);
                const T* xr = (isq ? Q : (isk ? K : V)) + (size_t)lrow * D;
                buf[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (lane_ok && row < R && lrow < (isq ? Lq : Lk)) {
                    buf[u] = Elem<T>::ld4(xr, d);
                    if constexpr (PEK != kPeNone) {
                        if (isq) buf[u] = encode4<T, PEK>(buf[u], xr, lrow, d, a.pq);
                        else if (isk) buf[u] = encode4<T, PEK>(buf[u], xr, lrow, d, a.pk);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int row = rb0 + u * rstep;
                if (!(r0 < rstep) || row >= R) continue;
                const bool isq = row < MQ, isk = !isq && row < MQ + NK;
                const int lrow = isq ? row : (isk ? row - MQ : row - MQ - NK);
                const int col = cg * 4;
                const float e4[4] = {buf[u].x, buf[u].y, buf[u].z, buf[u].w};
                if constexpr (kBf16) {
                    if (isq || isk) {
                        const int off = lrow * (isq ? g.qstr : g.kstr) + col;
                        uint16_t* hi =
                            reinterpret_cast<uint16_t*>(smem + (isq ? g.q_off : g.k_off));
                        uint2 w;
                        w.x = pack_bf16x2(e4[0], e4[1]);
                        w.y = pack_bf16x2(e4[2], e4[3]);
                        *reinterpret_cast<uint2*>(hi + off) = w;
                        if constexpr (kSplit) {
                            uint16_t* lo =
                                reinterpret_cast<uint16_t*>(smem + (isq ? g.ql_off : g.kl_off));
                            float r4[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                r4[e] = e4[e] - bf16_bits_to_f32(f32_to_bf16_bits(e4[e]));
                            uint2 wl;
                            wl.x = pack_bf16x2(r4[0], r4[1]);
                            wl.y = pack_bf16x2(r4[2], r4[3]);
                            *reinterpret_cast<uint2*>(lo + off) = wl;
                        }
                    } else {
                        uint16_t* vt = reinterpret_cast<uint16_t*>(smem + g.v_off);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            vt[(col + e) * g.vstr + lrow] = f32_to_bf16_bits(e4[e]);
                    }
                } else {
                    const int base = isq ? g.q_off : (isk ? g.k_off : g.v_off);
                    const int str = isq ? g.qstr : (isk ? g.kstr : g.vstr);
                    float* dst = reinterpret_cast<float*>(smem + base) + lrow * str + col;
                    *reinterpret_cast<float2*>(dst) = make_float2(e4[0], e4[1]);
                    *reinterpret_cast<float2*>(dst + 2) = make_float2(e4[2], e4[3]);
                }
            }
        }
    }
    __syncthreads();

    // ---- 2. partial scores S_c on MFMA.  Each wave owns one 16-row block
    // and up to 8 column tiles; the row block's A operand is read once per
    // k-step and shared by the tiles' independent accumulators.
    float* S = reinterpret_cast<float*>(smem + g.s_off);
    float* part = a.part + ((size_t)bh * n + c) * E;
    {
        int rb, c0, cs;
        const int cnt = wave_tiles(wave, nrb, NK / 16, &rb, &c0, &cs);
        auto store = [&](int u, const v4f& acc) {
            const int j = (c0 + u * cs) * 16 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = rb * 16 + lk * 4 + r;
                if (n > 1) st_dev(part + i * NK + j, acc[r]);
                else S[i * g.sstr + j] = acc[r];
            }
        };
        auto run = [&](auto nt_tag) {
            constexpr int NT = decltype(nt_tag)::value;
            v4f acc[NT];
#pragma unroll
            for (int u = 0; u < NT; ++u) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
            // tiles past cnt repeat the last valid tile (computed, not stored)
            const int bstep_rows = (cnt > 1 ? cs : 0) * 16;
            if constexpr (kBf16) {
                const uint16_t* qh = reinterpret_cast<const uint16_t*>(smem + g.q_off) +
                                     (rb * 16 + lr) * g.qstr + lk * 8;
                const uint16_t* kh = reinterpret_cast<const uint16_t*>(smem + g.k_off) +
                                     (c0 * 16 + lr) * g.kstr + lk * 8;
                const int ql_d = (g.ql_off - g.q_off) / 2, kl_d = (g.kl_off - g.k_off) / 2;
                mma_bf16<NT, kSplit, kSplit>(qh, qh + ql_d, kh, kh + kl_d, bstep_rows * g.kstr,
                                             dc, acc);
            } else {
                const float* qp = reinterpret_cast<const float*>(smem + g.q_off) +
                                  (rb * 16 + lr) * g.qstr + lk;
                const float* kp = reinterpret_cast<const float*>(smem + g.k_off) +
                                  (c0 * 16 + lr) * g.kstr + lk;
                mma_f32<NT>(qp, 1, kp, bstep_rows * g.kstr, 1, dc, acc);
            }
#pragma unroll
            for (int u = 0; u < NT; ++u)
                if (u < cnt) store(u, acc[u]);
        };
        if (cnt == 1) run(std::integral_constant<int, 1>{});
        else if (cnt == 2) run(std::integral_constant<int, 2>{});
        else if (cnt > 2 && cnt <= 4) run(std::integral_constant<int, 4>{});
        else if (cnt > 4) run(std::integral_constant<int, 8>{});
    }

    // ---- 3. all-reduce of S over the head's slices
    if (n > 1) {
        unsigned long long* fl = a.flags + (size_t)bh * n;
        const unsigned long long fa = flag_word(epoch, bh, 1), fb = flag_word(epoch, bh, 2);
        if (failed) {  // an earlier call timed out: fail closed
            poison_slice<T>(O, bh, Lq, D, d0, dc);
            return;
        }
        if (!head_sync(fl, c, n, fa, fa, fb, a.status, &flag)) {
            poison_slice<T>(O, bh, Lq, D, d0, dc);
            return;
        }
        // reduce-scatter: this workgroup owns entries [e0, e1)
        const int per = (E + n - 1) / n;
        const int e0 = c * per, e1 = min(E, e0 + per);
        const int cnt_e = max(0, e1 - e0);
        float* redl = reinterpret_cast<float*>(smem + g.red_off);
        const float* pb = a.part + (size_t)bh * n * E;
        if (cnt_e > 0 && cnt_e <= kThreads) {
            const int G = kThreads / cnt_e;  // partial groups summed in parallel
            const int el = tid % cnt_e, grp = tid / cnt_e;
            float acc = 0.f;
            if (grp < G) {
                const float* src = pb + e0 + el;
                int p = grp;
                for (; p + 7 * G < n; p += 8 * G) {
                    float x[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) x[u] = ld_dev(src + (size_t)(p + u * G) * E);
#pragma unroll
                    for (int u = 0; u < 8; ++u) acc += x[u];
                }
                for (; p < n; p += G) acc += ld_dev(src + (size_t)p * E);
            }
            redl[tid] = acc;
            __syncthreads();
            if (tid < cnt_e) {
                float s = 0.f;
                for (int q = 0; q < G; ++q) s += redl[q * cnt_e + tid];
                st_dev(a.red + (size_t)bh * E + e0 + tid, s);
            }
        } else {
            for (int e = e0 + tid; e < e1; e += kThreads) {
                const float* src = pb + e;
                float acc = 0.f;
                int p = 0;
                for (; p + 7 < n; p += 8) {
                    float x[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) x[u] = ld_dev(src + (size_t)(p + u) * E);
#pragma unroll
                    for (int u = 0; u < 8; ++u) acc += x[u];
                }
                for (; p < n; ++p) acc += ld_dev(src + (size_t)p * E);
                st_dev(a.red + (size_t)bh * E + e, acc);
            }
        }
        if (!head_sync(fl, c, n, fb, fb, fb, a.status, &flag)) {
            poison_slice<T>(O, bh, Lq, D, d0, dc);
            return;
        }
        // every workgroup of the head has read `epoch`: advance it
        if (c == 0 && tid == 0)
            __hip_atomic_store(a.epochs + bh, epoch + 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        // all-gather: the reduced S into LDS (16 loads in flight per thread)
        const float* rs = a.red + (size_t)bh * E;
        for (int base = 0; base < E; base += kThreads * 16) {
            float x[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int e = base + u * kThreads + tid;
                x[u] = e < E ? ld_dev(rs + e) : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int e = base + u * kThreads + tid;
                if (e < E) {
                    const int i = e / NK, j = e - i * NK;
                    S[i * g.sstr + j] = x[u];
                }
            }
        }
    }
    __syncthreads();

    // ---- 4. softmax of scale * S: one quad of threads per row, each thread
    // every fourth column; quad DPP reductions; P to its own LDS region
    {
        const int i = tid >> 2, q4 = tid & 3;
        const bool row_ok = i < Lq;
        auto run = [&](auto cnt_tag) {
            constexpr int C4 = decltype(cnt_tag)::value;  // NK / 4
            float v[C4];
            float m = -INFINITY;
#pragma unroll
            for (int u = 0; u < C4; ++u) {
                const int j = q4 + 4 * u;
                v[u] = (row_ok && j < Lk) ? S[i * g.sstr + j] * a.scale : -INFINITY;
                m = fmaxf(m, v[u]);
            }
            m = fmaxf(m, dpp<kDppQuadXor1>(m));
            m = fmaxf(m, dpp<kDppQuadXor2>(m));
            float l = 0.f;
#pragma unroll
            for (int u = 0; u < C4; ++u) {
                v[u] = row_ok ? __expf(v[u] - m) : 0.f;
                l += v[u];
            }
            l += dpp<kDppQuadXor1>(l);
            l += dpp<kDppQuadXor2>(l);
            const float inv = row_ok ? 1.0f / l : 0.f;
            if (i < MQ) {
#pragma unroll
                for (int u = 0; u < C4; ++u) {
                    const int j = q4 + 4 * u;
                    const float p = v[u] * inv;
                    if constexpr (kBf16) {
                        uint16_t* ph = reinterpret_cast<uint16_t*>(smem + g.p_off);
                        const uint16_t hi = f32_to_bf16_bits(p);
                        ph[i * g.pstr + j] = hi;
                        ph[(MQ + i) * g.pstr + j] = f32_to_bf16_bits(p - bf16_bits_to_f32(hi));
                    } else {
                        reinterpret_cast<float*>(smem + g.p_off)[i * g.pstr + j] = p;
                    }
                }
            }
        };
        switch (NK) {
            case 32: run(std::integral_constant<int, 8>{}); break;
            case 64: run(std::integral_constant<int, 16>{}); break;
            case 96: run(std::integral_constant<int, 24>{}); break;
            default: run(std::integral_constant<int, 32>{}); break;
        }
    }
    __syncthreads();

    // ---- 5. O[:, slice] = P V[:, slice] on MFMA: each wave owns one 16-row
    // block and every (4 / nrb)-th 16-dim tile, 8 tiles at a time
    {
        int rb, c0, cs;
        const int cnt = wave_tiles(wave, nrb, dc / 16, &rb, &c0, &cs);
        for (int t0 = 0; t0 < cnt; t0 += 8) {
            const int left = cnt - t0;
            const int tc = c0 + t0 * cs;  // first tile of this group
            auto run = [&](auto nt_tag) {
                constexpr int NT = decltype(nt_tag)::value;
                v4f acc[NT];
#pragma unroll
                for (int u = 0; u < NT; ++u) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
                const int step = (left > 1 ? cs : 0) * 16;  // repeats past `left`, unstored
                if constexpr (kBf16) {
                    const uint16_t* ph = reinterpret_cast<const uint16_t*>(smem + g.p_off) +
                                         (rb * 16 + lr) * g.pstr + lk * 8;
                    const uint16_t* vt = reinterpret_cast<const uint16_t*>(smem + g.v_off) +
                                         (tc * 16 + lr) * g.vstr + lk * 8;
                    mma_bf16<NT, true, false>(ph, ph + MQ * g.pstr, vt, vt, step * g.vstr, NK,
                                              acc);
                } else {
                    const float* pp = reinterpret_cast<const float*>(smem + g.p_off) +
                                      (rb * 16 + lr) * g.pstr + lk;
                    const float* vp = reinterpret_cast<const float*>(smem + g.v_off) +
                                      lk * g.vstr + tc * 16 + lr;
                    mma_f32<NT>(pp, 1, vp, step, g.vstr, NK, acc);
                }
#pragma unroll
                for (int u = 0; u < NT; ++u) {
                    if (u >= left) break;
                    const int dd = d0 + (tc + u * cs) * 16 + lr;
                    if (dd >= D) continue;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = rb * 16 + lk * 4 + r;
                        if (i < Lq) Elem<T>::st(O, ((size_t)bh * Lq + i) * D + dd, acc[u][r]);
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
template <typename T, int PEK>
hipError_t ensure_lds_limit(int lds) {
    static std::atomic<int> set{0};
    if (lds <= set.load(std::memory_order_acquire)) return hipSuccess;
    const int want = 160 * 1024 - 256;
    hipError_t e = hipFuncSetAttribute((const void*)k_fused_small<T, PEK>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, want);
    if (e == hipSuccess) set.store(want, std::memory_order_release);
    return e;
}

template <typename T, int PEK>
hipError_t launch_t(const FusedArgs& a, int BH, int lds, hipStream_t st) {
    hipError_t e = ensure_lds_limit<T, PEK>(lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_fused_small<T, PEK>), dim3((unsigned)(BH * a.nchunk)), dim3(kThreads),
                       lds, st, a);
    return hipGetLastError();
}

template <typename T, int PEK>
int capacity_t(int lds) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (ensure_lds_limit<T, PEK>(lds) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_fused_small<T, PEK>, kThreads, lds) !=
        hipSuccess)
        return 0;
    return cus * per;
}

}  // namespace

int fused_small_lds_bytes(int dtype, int pek, int Lq, int Lk, int dc) {
    const bool bf16 = dtype == kDtypeBF16;
    return make_geo(bf16, bf16 && pek != kPeNone, Lq, Lk, dc).bytes;
}

int fused_small_capacity(int dtype, int pek, int lds) {
    // occupancy depends on LDS and registers; the encoded variants use the
    // most registers, so their figure is the safe one for every variant
    (void)pek;
    return dtype == kDtypeF32 ? capacity_t<float, kPeRopeHalf>(lds)
                              : capacity_t<uint16_t, kPeRopeHalf>(lds);
}

hipError_t launch_fused_small(int dtype, int pek, const void* Q, const void* K, const void* V,
                              void* O, float* part, float* red, unsigned* epochs,
                              unsigned long long* flags, int* status, int BH, int Lq, int Lk,
                              int D, int dc, int nchunk, float scale, const PeSide& pq,
                              const PeSide& pk, int vec_ok, hipStream_t st) {
    (void)vec_ok;  // the host sends only vector-aligned shapes here
    FusedArgs a{Q, K, V, O, part, red, epochs, flags, status, Lq, Lk, D, dc, nchunk, scale,
                pq, pk};
    const int lds = fused_small_lds_bytes(dtype, pek, Lq, Lk, dc);
#define ATN_FUSED_CASE(T)                                                                \
    switch (pek) {                                                                       \
        case kPeNone: return launch_t<T, kPeNone>(a, BH, lds, st);                       \
        case kPeRopeInterleaved: return launch_t<T, kPeRopeInterleaved>(a, BH, lds, st); \
        case kPeRopeHalf: return launch_t<T, kPeRopeHalf>(a, BH, lds, st);               \
        case kPeSinusoidal: return launch_t<T, kPeSinusoidal>(a, BH, lds, st);           \
        default: return hipErrorInvalidValue;                                            \
    }
    if (dtype == kDtypeF32) {
        ATN_FUSED_CASE(float)
    }
    ATN_FUSED_CASE(uint16_t)
#undef ATN_FUSED_CASE
}

}  // namespace atn
