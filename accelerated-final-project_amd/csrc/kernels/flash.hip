// Flash-style fp32 attention for head_dim <= 256 at any sequence length
// (gfx950).
//
// The reference's kernel (final/attention.cu:84-191) walks the keys of one
// query row in 64-key tiles with an online softmax and keeps the running
// output in global memory.  Here a workgroup owns the query rows of its
// waves, 16 or 32 per wave (v_mfma_f32_16x16x32_f16 or 32x32x16 tiles), of
// one head and walks the head's keys in tiles of KT keys, with the running
// output of its rows in registers.  Forms: 8 waves of 16 rows (64-key tiles
// at D <= 128) and 8 waves of 32 rows (D <= 128; 64-key tiles at D <= 64, 32
// at D = 128: each wave reads a K/V tile from LDS once per 32 rows instead of
// 16, and each tile is converted once per 256 rows), the library's two; 4
// waves of 16 rows for up to 64 query rows, and of 32 rows as a tuning
// override.
//
//   Per tile: K and V rows are loaded (16-byte loads) two tiles ahead, K
//   encoded (RoPE, sinusoidal) once they land, and reduced to per-wave
//   magnitude maxima; a tile ahead, the workgroup maxima set the tile's
//   scales (K scaled by a power of two when its largest finite magnitude
//   lies outside [2^-3, 65504), V only beyond fp16's range: its scale
//   carries over into the running output) and it is stored to one of two
//   LDS buffers as hi + lo fp16 parts (the fp32 split of the single-launch
//   kernel: 22 significant bits per operand, exact products on the fp16
//   MFMAs, fp32 accumulation).  One barrier per tile orders all of it.
//   Each wave computes S^T = K Q^T for its query rows (Q in registers,
//   split once, scaled by a power of two per wave) -- transposed, so that a
//   lane holds 16 scores of ONE query: the online-softmax statistics
//   (running max m, running sum l) of a query live in the lanes that hold
//   its scores and its output row (4 lanes with 16-row tiles, 2 with
//   32-row ones), and reductions over a tile's keys are 16 values in
//   registers plus one or two row swaps (v_permlane16/32_swap).
//   P = 2^(x - m + 8) (base 2, its 2^8 via the exponent; the running max m
//   moves only when a tile's max exceeds it by more than 7) stays in
//   registers, where the accumulator layout of S^T is already the B operand
//   of O^T += V^T P^T (the keys of each 32- or 16-key block in the order
//   4g + 0..3, then 16 + 4g + 0..3 or 8 + 4g + 0..3, for lane group g; V's
//   transposing LDS read, ds_read_b64_tr_b16, takes the same order), and O^T
//   (dims x queries per MFMA tile) accumulates in registers, rescaled by
//   2^(m_old - m_new) when m moves and by the ratio of consecutive V tiles'
//   scales when they differ.
//
// The score matrix never reaches memory: per call the kernel reads Q once
// and K and V once per query block, and writes O once.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "split16.hpp"

namespace atn {

namespace {

// Tiling for head dims padded to DP (32, 64, 128 or 256), NW waves per
// workgroup (4 or 8) and RW query rows per wave (16: v_mfma_f32_16x16x32_f16
// tiles; 32: v_mfma_f32_32x32x16_f16 tiles, D <= 128), every wave sharing
// each K/V tile.  The key tile is 64 keys for bf16 inputs (HL false) and,
// with or without a positional encoding, for 8 waves of 16 rows at DP <= 128,
// of 32 rows at DP <= 64 (at DP = 128 the 32-row form's extra scores spill)
// and 4 waves of 16 rows at DP <= 64 (two workgroups per CU still fit in
// LDS), else 32 (two LDS buffers of it then leave room for two 4-wave
// workgroups per CU), and at least one load round of the workgroup.
template <int DP, bool PE, int NW, int RW, bool HL = true>
struct FlashGeo {
    static_assert(RW == 16 || (RW == 32 && DP <= 128), "forms");
    static constexpr int THREADS = 64 * NW, ROWS = RW * NW;
    static constexpr int KT0 =
        !HL || (NW == 8 && (RW == 16 ? DP <= 128 : DP <= 64)) || (NW == 4 && RW == 16 && DP <= 64)
            ? 64
            : 32;
    static constexpr int KT = KT0 > THREADS / (DP / 4) ? KT0 : THREADS / (DP / 4);
    static constexpr int MT = RW;                   // MFMA tile edge
    static constexpr int KD = RW == 16 ? 32 : 16;   // MFMA depth: dims of Q K^T, keys of P V
    static constexpr int KS = DP / KD;              // KD-deep steps of Q K^T
    static constexpr int NJ = KT / MT;              // MT-key tiles of S^T
    static constexpr int NB = KT / KD;              // KD-key blocks of P V
    static constexpr int NDT = DP / MT;             // MT-dim tiles of O^T
    static constexpr int SPT = MT * MT / 64;        // accumulator floats per lane and tile
    static constexpr int VPR = DP / 4;              // 16-byte vectors per row
    static constexpr int RSTEP = THREADS / VPR;     // rows per load round
    static constexpr int NLD = KT / RSTEP;          // load rounds per tile
    // LDS rows in 16-bit elements: K padded by 8 (16-byte fragment reads),
    // V by 16 (the transposing read's 4 rows x 32 bytes in distinct banks);
    // two buffers of TILE elements, holding hi and lo parts (HL) or hi parts
    // only (bf16 inputs, exact in fp16)
    static constexpr int KSTR = DP + 8, VSTR = DP + 16;
    static constexpr int NP = HL ? 2 : 1;  // parts per operand
    static constexpr int K_HI = 0, K_LO = KT * KSTR, V_HI = NP * KT * KSTR,
                         V_LO = V_HI + KT * VSTR;
    static constexpr int TILE = NP * (KT * KSTR + KT * VSTR);
    static constexpr int BYTES = 2 * 2 * TILE;
    static_assert(KT % RSTEP == 0 && KT % MT == 0 && KT % KD == 0, "whole tiles");
    static_assert(BYTES <= 160 * 1024, "LDS");
};

typedef float v16f __attribute__((ext_vector_type(16)));

// max without the operand canonicalization fmaxf brings (the values are
// never signalling NaNs).  Inline asm: the compiler's hazard checks do not
// cover it, so it never reads an MFMA result (the MFMA pipeline may not
// have written it yet), and a value it writes passes a compiler-visible
// instruction before a cross-lane operation or an MFMA reads it.
__device__ __forceinline__ float fmax_raw(float a, float b) { return vmaxf(a, b); }

// the lanes that hold one query's scores (RW = 16: L, L ^ 16, L ^ 32,
// L ^ 48; RW = 32: L, L ^ 32), by gfx950's row-swapping permutes:
// v_permlane16_swap and v_permlane32_swap each leave a lane its own value
// and its partner's, in registers, in the same order for both lanes of a
// pair (so sums agree bit for bit)
template <int RW>
__device__ __forceinline__ float xgroup_max(float v) {
    v = __builtin_canonicalizef(v);
    if constexpr (RW == 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                        false, false);
        v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    }
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
template <int RW>
__device__ __forceinline__ float xgroup_sum(float v) {
    if constexpr (RW == 16) {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                        false, false);
        v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    }
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// full-wave max in every lane: DPP within each row of 16 lanes, then the
// row swaps
__device__ __forceinline__ float wave_max_rows(float v) {
    v = __builtin_canonicalizef(v);
    v = fmaxf(v, dpp<kDppQuadXor1>(v));
    v = fmaxf(v, dpp<kDppQuadXor2>(v));
    v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp<kDppRowMirror>(v));
    return xgroup_max<16>(v);
}

// 4 consecutive elements at byte offset `off` of a raw buffer as fp32
// (zeros past its end): fp32 16 bytes, bf16 8 bytes
template <typename T>
__device__ __forceinline__ float4 ld4_t(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (sizeof(T) == 4) {
        return ld_buf_f4(r, off);
    } else {
        const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        return make_float4(__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                           __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u));
    }
}

// two values as fp16, rounded to nearest even, packed
__device__ __forceinline__ uint32_t pk_f16_rne(float a, float b) {
    const f16x2 h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// the form's MFMA: 16 x 16 x 32 or 32 x 32 x 16, fp16 or bf16 operands,
// fp32 sums
__device__ __forceinline__ v4f mfma_rw(const f16x8& a, const f16x8& b, const v4f& c) {
    return mfma_f16(a, b, c);
}
__device__ __forceinline__ v16f mfma_rw(const f16x8& a, const f16x8& b, const v16f& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_rw(const bf16x8_t& a, const bf16x8_t& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma_rw(const bf16x8_t& a, const bf16x8_t& b, const v16f& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// two values as bf16, rounded to nearest even (v_cvt_pk_bf16_f32), packed
__device__ __forceinline__ uint32_t pk_bf16_rne(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// T = float: fp32 inputs as hi + lo fp16 parts, three products each; T =
// uint16_t: bf16 inputs (bf16 bits), one product each, the output rounded to
// bf16 -- without an encoding ("raw") the loaded bits go to LDS as they are
// and the products run on the bf16 MFMA (exact products, fp32's exponent
// range: no scales, no tile maxima), P as bf16; with an encoding the
// encoded values are fp32, staged as one fp16 part each (a power-of-two
// scale per tile brings K and V into fp16's normal range), P as fp16.
// waves per SIMD the register allocation leaves room for: 4 (two 8-wave
// workgroups per CU) for the raw bf16 form of 8 waves of 16 rows at head_d
// <= 128, which needs few registers; else what the form itself brings
template <typename T, int DP, int PEK, int NW, int RW>
constexpr int flash_waves_per_simd() {
    return sizeof(T) == 2 && PEK == kPeNone && NW == 8 && RW == 16 && DP <= 128 ? 4 : 8 / NW;
}

template <typename T, int DP, int PEK, int NW, int RW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(
    flash_waves_per_simd<T, DP, PEK, NW, RW>()))) void k_flash(const T* __restrict__ Qg,
                                                             const T* __restrict__ Kg,
                                                             const T* __restrict__ Vg,
                                                             T* __restrict__ Og, int Lq, int LkAll,
                                                             int D, int qblocks, float scale,
                                                             PeSide pq, PeSide pk, int nsplit,
                                                             int kchunk, float* __restrict__ part,
                                                             float4* __restrict__ stats) {
    constexpr bool kBf = sizeof(T) == 2;
    constexpr bool kRaw = kBf && PEK == kPeNone;
    constexpr int es = (int)sizeof(T);
    // MFMA operands: Q K^T (op_t) and P V (pv_t).  bf16 V is never encoded,
    // so it always goes in as loaded, with P as bf16.
    typedef std::conditional_t<kRaw, bf16x8_t, f16x8> op_t;
    typedef std::conditional_t<kBf, bf16x8_t, f16x8> pv_t;
    using G = FlashGeo<DP, PEK != kPeNone, NW, RW, !kBf>;
    typedef std::conditional_t<RW == 16, v4f, v16f> acc_t;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    uint16_t* smem = reinterpret_cast<uint16_t*>(smem_raw);
    // per-wave K and V magnitude maxima of a loaded tile, by tile parity
    __shared__ float slot[2][2 * NW];

    const float one = unit_opaque();  // (see split2_f16_one)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // lane (row lr of its MFMA tiles, lane group lg)
    const int lr = lane & (RW - 1), lg = lane / RW;
    // workgroup -> (head, query block, key split); with a grid that is a
    // multiple of 8 the workgroups of a head are consecutive on one XCD (the
    // dispatcher deals ids to the 8 XCDs round robin), so its K and V stay in
    // that L2.  Split sp takes keys [sp kchunk, sp kchunk + Lk) of the head
    // (without a split: all of them, kchunk >= LkAll).
    const int nwg = (int)gridDim.x;
    int id = (int)blockIdx.x;
    if ((nwg & 7) == 0) id = (id & 7) * (nwg >> 3) + (id >> 3);
    const int per_head = qblocks * nsplit;
    const int bh = id / per_head, rem = id - bh * per_head;
    const int qb = rem / nsplit, sp = rem - qb * nsplit;
    const int kbeg = sp * kchunk;
    const int Lk = min(kchunk, LkAll - kbeg);
    const int q0 = qb * G::ROWS;
    const T* Qh = Qg + (size_t)bh * Lq * D;
    const T* Kh = Kg + ((size_t)bh * LkAll + kbeg) * D;
    const T* Vh = Vg + ((size_t)bh * LkAll + kbeg) * D;
    constexpr int kOob = kBufOob;

    // ---- Q: this wave's RW rows as the B operand of S^T = K Q^T: lane
    // (query lr, group lg) holds dims KD ks + 8 lg + 0..7, scaled by a
    // power of two from the wave's largest finite magnitude
    const int qrow = q0 + RW * wave + lr;
    op_t qh[G::KS];
    f16x8 ql[G::KS];
    float uq = 1.f;
    if constexpr (kRaw) {
        // the bf16 bits as they are (8 bytes per 4 dims; dims past D and rows
        // past Lq read as zeros)
        const __amdgpu_buffer_rsrc_t rq = buf_rsrc(Qh, Lq * D * es);
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            const int d = G::KD * ks + 8 * lg;
            const auto a = __builtin_amdgcn_raw_buffer_load_b64(rq, d < D ? (qrow * D + d) * 2 : kOob,
                                                                0, 0);
            const auto b = __builtin_amdgcn_raw_buffer_load_b64(
                rq, d + 4 < D ? (qrow * D + d + 4) * 2 : kOob, 0, 0);
            qh[ks] = __builtin_bit_cast(op_t, make_uint4(a[0], a[1], b[0], b[1]));
        }
    } else {
        float4 qv[G::KS][2];
        float mq = 0.f;
        const __amdgpu_buffer_rsrc_t rq = buf_rsrc(Qh, Lq * D * es);
        if constexpr (PEK == kPeNone) {
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int d = G::KD * ks + 8 * lg + 4 * h;
                    qv[ks][h] = ld4_t<T>(rq, d < D ? (qrow * D + d) * es : kOob);
                    mq = max_finite4(mq, qv[ks][h]);
                }
        } else {
            // The encoding needs the angles of each element, and in the MFMA
            // layout each lane holds a query row of its own: their table
            // reads would take a cache line per lane.  So the wave encodes its
            // rows with consecutive lanes on consecutive dims (coalesced, all
            // loads first), 16 rows a round, and passes them through LDS (free
            // until the first tile is staged) into the MFMA layout.
            constexpr int VPR = DP / 4, GPR = VPR / 4;  // vectors per row, per lane and round
            constexpr int NR = RW / 16, NG = NR * GPR, QSTR = DP + 4;
            static_assert(NW * 16 * QSTR * 4 <= G::BYTES, "Q staging fits the tile buffers");
            float4 x[NG];
            int dd[NG], pp[NG], rw[NG];
            const T* rr[NG];
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const int v = lane + 64 * (g % GPR);
                rw[g] = q0 + RW * wave + 16 * (g / GPR) + v / VPR;
                pp[g] = min(rw[g], Lq - 1);
                dd[g] = (v % VPR) * 4;
                rr[g] = Qh + (size_t)pp[g] * D;
                x[g] = ld4_t<T>(rq, rw[g] < Lq && dd[g] < D ? (rw[g] * D + dd[g]) * es : kOob);
            }
            if (pq.on) {
                if (PEK == kPeRopeHalf && VPR <= 32 && D == DP && pq.rotary == D &&
                    pe4_batch_ok(PEK, pq)) {
                    // a row's groups in VPR consecutive lanes: partners by lane
                    if constexpr (PEK == kPeRopeHalf && VPR <= 32 && VPR >= 8)
                        pe4_batch_half_lanes<NG, VPR / 2>(x, dd, pp, pq);
                } else if (pe4_batch_ok(PEK, pq)) {
                    pe4_batch<T, PEK, NG>(x, dd, rr, pp, D, pq);
                } else {
#pragma unroll
                    for (int g = 0; g < NG; ++g)
                        if (dd[g] < D) x[g] = apply_pe4<T, PEK>(x[g], rr[g], pp[g], dd[g], D, pq, true);
                }
            }
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                if (rw[g] >= Lq) x[g] = make_float4(0.f, 0.f, 0.f, 0.f);  // rows past Lq: zero
                mq = max_finite4(mq, x[g]);
            }
            float* qs = reinterpret_cast<float*>(smem_raw) + wave * 16 * QSTR;
#pragma unroll
            for (int rnd = 0; rnd < NR; ++rnd) {
#pragma unroll
                for (int j = 0; j < GPR; ++j) {
                    const int v = lane + 64 * j;
                    *reinterpret_cast<float4*>(qs + (v / VPR) * QSTR + (v % VPR) * 4) =
                        x[rnd * GPR + j];
                }
                if ((lr >> 4) == rnd) {  // the lanes whose query is among these rows
#pragma unroll
                    for (int ks = 0; ks < G::KS; ++ks)
#pragma unroll
                        for (int h = 0; h < 2; ++h)
                            qv[ks][h] = *reinterpret_cast<const float4*>(
                                qs + (lr & 15) * QSTR + G::KD * ks + 8 * lg + 4 * h);
                }
            }
        }
        mq = wave_max(mq);
        const float sq = pow2_scale(mq);
        uq = pow2_unit(mq);
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            uint32_t h[4], l[4];
            if constexpr (kBf) {
                h[0] = pk_f16_rne(qv[ks][0].x * sq, qv[ks][0].y * sq);
                h[1] = pk_f16_rne(qv[ks][0].z * sq, qv[ks][0].w * sq);
                h[2] = pk_f16_rne(qv[ks][1].x * sq, qv[ks][1].y * sq);
                h[3] = pk_f16_rne(qv[ks][1].z * sq, qv[ks][1].w * sq);
                qh[ks] = __builtin_bit_cast(op_t, make_uint4(h[0], h[1], h[2], h[3]));
                continue;
            }
            split2_f16(qv[ks][0].x * sq, qv[ks][0].y * sq, h[0], l[0]);
            split2_f16(qv[ks][0].z * sq, qv[ks][0].w * sq, h[1], l[1]);
            split2_f16(qv[ks][1].x * sq, qv[ks][1].y * sq, h[2], l[2]);
            split2_f16(qv[ks][1].z * sq, qv[ks][1].w * sq, h[3], l[3]);
            qh[ks] = __builtin_bit_cast(op_t, make_uint4(h[0], h[1], h[2], h[3]));
            ql[ks] = __builtin_bit_cast(f16x8, make_uint4(l[0], l[1], l[2], l[3]));
        }
    }

    // ---- K/V tiles.  Thread t loads 16-byte vector t % VPR of rows t / VPR
    // + RSTEP i (rows past Lk and columns past D read as zeros).  Tile u is
    // handled over three iterations of the loop below, with one barrier per
    // iteration: in iteration u - 2 its loads are issued before the tile
    // then computed, and after that tile its K rows are encoded (PE) and
    // its per-wave magnitude maxima go to slot[u & 1]; in iteration u - 1
    // the workgroup maxima set its scales and its hi + lo parts go to LDS
    // buffer u & 1; iteration u computes it.  Staging, loads and maxima thus
    // run beside another tile's products, and LDS holds two tiles.
    const int lrow = tid / G::VPR, lcol = (tid % G::VPR) * 4;
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(Kh, Lk * D * es);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(Vh, Lk * D * es);
    float4 kr[G::NLD], vr[G::NLD];
    uint2 kw[G::NLD], vw[G::NLD];  // raw bf16: the loaded bits
    auto issue = [&](int k0) {
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            const int key = k0 + lrow + G::RSTEP * i;
            const int off = key < Lk && lcol < D ? (key * D + lcol) * es : kOob;
            if constexpr (kRaw) {
                const auto a = __builtin_amdgcn_raw_buffer_load_b64(rk, off, 0, 0);
                kw[i] = make_uint2(a[0], a[1]);
            } else {
                kr[i] = ld4_t<T>(rk, off);
            }
            if constexpr (kBf) {
                const auto b = __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0);
                vw[i] = make_uint2(b[0], b[1]);
            } else {
                vr[i] = ld4_t<T>(rv, off);
            }
        }
    };
    // K's encoding, then the per-wave maxima of the tile's K and V
    // magnitudes (one v_max3 per value pair).  A wave whose values include
    // an infinity or NaN takes its finite values only: non-finite values
    // stay so through a scaling and must not set the scale of the finite
    // values beside them.
    auto maxima = [&](int k0, int par) {
        if constexpr (kRaw) return;  // no scales
        if constexpr (PEK != kPeNone) {
            if (pk.on && pe4_batch_ok(PEK, pk)) {
                // every group's loads at once (rows past Lk clamped, their
                // values kept zero); rotate-half over whole rows takes each
                // partner from the lane VPR / 2 away (a row's groups lie in VPR
                // consecutive lanes)
                int dd[G::NLD], pp[G::NLD];
                const T* rr[G::NLD];
#pragma unroll
                for (int i = 0; i < G::NLD; ++i) {
                    const int kc = min(k0 + lrow + G::RSTEP * i, Lk - 1);
                    dd[i] = lcol;
                    pp[i] = kbeg + kc;
                    rr[i] = Kh + (size_t)kc * D;
                }
                constexpr bool kLanes = PEK == kPeRopeHalf && G::VPR >= 8 && G::VPR <= 32;
                if (kLanes && D == DP && pk.rotary == D) {
                    if constexpr (kLanes) pe4_batch_half_lanes<G::NLD, G::VPR / 2>(kr, dd, pp, pk);
                } else {
                    pe4_batch<T, PEK, G::NLD>(kr, dd, rr, pp, D, pk);
                }
#pragma unroll
                for (int i = 0; i < G::NLD; ++i)
                    if (k0 + lrow + G::RSTEP * i >= Lk) kr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
#pragma unroll
                for (int i = 0; i < G::NLD; ++i) {
                    const int key = k0 + lrow + G::RSTEP * i;
                    if (key < Lk && lcol < D)
                        kr[i] = apply_pe4<T, PEK>(kr[i], Kh + (size_t)key * D, kbeg + key, lcol, D,
                                                  pk, true);
                }
            }
        }
        float mk = 0.f, mv = 0.f;  // (bf16 V goes in as loaded: no maximum)
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            mk = vmax3abs(mk, kr[i].x, kr[i].y);
            mk = vmax3abs(mk, kr[i].z, kr[i].w);
            if constexpr (!kBf) {
                mv = vmax3abs(mv, vr[i].x, vr[i].y);
                mv = vmax3abs(mv, vr[i].z, vr[i].w);
            }
        }
        // Usually ballots settle it with no reduction: a wave whose K values
        // all lie below kF16Range and some at 2^-3 or above (fp32 V: below
        // kF16Range) reports the sentinel 1, a value of that
        // range, so the workgroup maximum over the slots is in range exactly
        // when the true one is, and when a wave lies beyond the range its own
        // (reduced) maximum still decides the scale.  Other waves reduce.
        const bool k_ok = !__builtin_amdgcn_ballot_w64(!(mk < kF16Range)) &&
                          __builtin_amdgcn_ballot_w64(mk >= 0.125f) != 0;
        const bool v_ok = kBf || !__builtin_amdgcn_ballot_w64(!(mv < kF16Range));
        if (k_ok && v_ok) {
            mk = 1.f;
            mv = 1.f;
        } else {
            mk = wave_max_rows(mk);
            mv = kBf ? 1.f : wave_max_rows(mv);
            if (!(mk < INFINITY) || !(mv < INFINITY)) {  // the same in every lane
                mk = 0.f;
                mv = kBf ? 1.f : 0.f;
#pragma unroll
                for (int i = 0; i < G::NLD; ++i) {
                    mk = max_finite4(mk, kr[i]);
                    if constexpr (!kBf) mv = max_finite4(mv, vr[i]);
                }
                mk = wave_max_rows(mk);
                if constexpr (!kBf) mv = wave_max_rows(mv);
            }
        }
        if (lane == 0) {
            slot[par][wave] = mk;
            slot[par][NW + wave] = mv;
        }
    };
    // scales of the tile whose maxima are in slot[par] (K as it is where its
    // largest magnitude lies in [2^-3, 65504): the split then keeps 2^-22 of
    // that magnitude, one fp16 part 2^-11; else a power of two brings it to
    // [2^14, 2^15); fp32 V scaled only beyond fp16's range), and its hi + lo
    // (fp32) or hi (encoded bf16 K) fp16 parts into LDS buffer par; bf16 V
    // goes in as loaded
    auto stage = [&](int par, float& uk, float& sv, float& uv) {
        if constexpr (kRaw) {
            uk = sv = uv = 1.f;
            uint16_t* buf = smem + par * G::TILE;
#pragma unroll
            for (int i = 0; i < G::NLD; ++i) {
                const int row = lrow + G::RSTEP * i;
                *reinterpret_cast<uint2*>(buf + G::K_HI + row * G::KSTR + lcol) = kw[i];
                *reinterpret_cast<uint2*>(buf + G::V_HI + row * G::VSTR + lcol) = vw[i];
            }
            return;
        }
        float mk = slot[par][0], mv = slot[par][NW];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            mk = fmax_raw(mk, slot[par][w]);
            mv = fmax_raw(mv, slot[par][NW + w]);
        }
        const bool k_plain = mk >= 0.125f && mk < kF16Range;
        const float sk = k_plain ? 1.f : pow2_scale(mk);
        uk = k_plain ? 1.f : pow2_unit(mk);
        const bool v_plain = kBf || mv < kF16Range;
        sv = v_plain ? 1.f : pow2_scale(mv);
        uv = v_plain ? 1.f : pow2_unit(mv);
        uint16_t* buf = smem + par * G::TILE;
        auto put = [&](auto plain) {
#pragma unroll
            for (int i = 0; i < G::NLD; ++i) {
                const int row = lrow + G::RSTEP * i;
                uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
                if constexpr (kBf) {
                    const float fk = decltype(plain)::value ? 1.f : sk;
                    *reinterpret_cast<uint2*>(buf + G::K_HI + row * G::KSTR + lcol) =
                        make_uint2(pk_f16_rne(kr[i].x * fk, kr[i].y * fk),
                                   pk_f16_rne(kr[i].z * fk, kr[i].w * fk));
                    *reinterpret_cast<uint2*>(buf + G::V_HI + row * G::VSTR + lcol) = vw[i];
                    continue;
                }
                if constexpr (decltype(plain)::value) {
                    split2_f16_one(kr[i].x, kr[i].y, one, h0, l0);
                    split2_f16_one(kr[i].z, kr[i].w, one, h1, l1);
                    split2_f16_one(vr[i].x, vr[i].y, one, h2, l2);
                    split2_f16_one(vr[i].z, vr[i].w, one, h3, l3);
                } else {
                    split2_f16_mix(kr[i].x, kr[i].y, sk, h0, l0);
                    split2_f16_mix(kr[i].z, kr[i].w, sk, h1, l1);
                    split2_f16_mix(vr[i].x, vr[i].y, sv, h2, l2);
                    split2_f16_mix(vr[i].z, vr[i].w, sv, h3, l3);
                }
                *reinterpret_cast<uint2*>(buf + G::K_HI + row * G::KSTR + lcol) =
                    make_uint2(h0, h1);
                *reinterpret_cast<uint2*>(buf + G::K_LO + row * G::KSTR + lcol) =
                    make_uint2(l0, l1);
                *reinterpret_cast<uint2*>(buf + G::V_HI + row * G::VSTR + lcol) =
                    make_uint2(h2, h3);
                *reinterpret_cast<uint2*>(buf + G::V_LO + row * G::VSTR + lcol) =
                    make_uint2(l2, l3);
            }
        };
        if (k_plain && v_plain)
            put(std::true_type{});
        else
            put(std::false_type{});
    };

    // running statistics of this lane's query and its output rows (O^T
    // tiles: register r of tile t holds dim MT t + 8 (r / 4) + 4 lg + r % 4
    // of query lr): the running max m_run of the scores in units of uq (the
    // accumulators times their tile's K unit uk: powers of two, so maxima of
    // different tiles compare exactly), the sum in units of 2^(c0 m_run -
    // 8), the output in units of uv 2^(c0 m_run - 8) for the current V
    // tile's unit uv = 1 / sv; c0 turns them into base-2 exponents, and a
    // tile's accumulators take c2 = c0 uk
    const float c0 = scale * 1.44269504088896341f * uq;
    const float thr = 7.f / c0;
    float m_run = -INFINITY, l_run = 0.f, uv_prev = 1.f;
    acc_t o[G::NDT];
#pragma unroll
    for (int t = 0; t < G::NDT; ++t) o[t] = acc_t{};

    const int ntiles = (Lk + G::KT - 1) / G::KT;
    float uk, sv, uv;  // scales of the tile staged last
    issue(0);
    maxima(0, 0);
    __syncthreads();
    stage(0, uk, sv, uv);
    if (ntiles > 1) {
        issue(G::KT);
        maxima(G::KT, 1);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int k0 = t * G::KT, par = t & 1;
        const float uk_t = uk, sv_t = sv, uv_t = uv;
        if (t + 1 < ntiles) {
            stage(par ^ 1, uk, sv, uv);
            if (t + 2 < ntiles) issue(k0 + 2 * G::KT);
        }
        const uint16_t* buf = smem + par * G::TILE;

        // ---- S^T tiles: register r of s[j] = key MT j + 8 (r / 4) + 4 lg +
        // r % 4, query lr
        acc_t s[G::NJ];
#pragma unroll
        for (int j = 0; j < G::NJ; ++j) s[j] = acc_t{};
        // per KD-deep step its NP NJ fragment reads and (2 NP - 1) NJ
        // products; the reads of step ks + 1 are issued before the products
        // of step ks (two register sets), so that a step's reads are in
        // flight while the previous step multiplies instead of being waited
        // for right after their issue -- not in the form held to 128
        // registers (4 waves per SIMD), where the second set would spill: it
        // reads each step's fragments before the step's products
        constexpr bool kPre = flash_waves_per_simd<T, DP, PEK, NW, RW>() < 4;
        op_t ah[2][G::NJ];
        f16x8 al[2][G::NJ];
        auto frags = [&](int ks, int r) {
#pragma unroll
            for (int j = 0; j < G::NJ; ++j) {
                const int a = (G::MT * j + lr) * G::KSTR + G::KD * ks + 8 * lg;
                ah[r][j] = __builtin_bit_cast(op_t, lds8_f16(buf + G::K_HI + a));
                if constexpr (!kBf) al[r][j] = lds8_f16(buf + G::K_LO + a);
            }
        };
        if constexpr (kPre) {
            frags(0, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, G::NP * G::NJ, 0);  // DS reads
        }
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            const int r = kPre ? ks & 1 : 0;
            if constexpr (kPre) {
                if (ks + 1 < G::KS) frags(ks + 1, r ^ 1);
            } else {
                frags(ks, 0);
            }
#pragma unroll
            for (int j = 0; j < G::NJ; ++j) s[j] = mfma_rw(ah[r][j], qh[ks], s[j]);
            if constexpr (!kBf) {
#pragma unroll
                for (int j = 0; j < G::NJ; ++j) s[j] = mfma_rw(ah[r][j], ql[ks], s[j]);
#pragma unroll
                for (int j = 0; j < G::NJ; ++j) s[j] = mfma_rw(al[r][j], qh[ks], s[j]);
            }
            if (!kPre || ks + 1 < G::KS)
                __builtin_amdgcn_sched_group_barrier(0x100, G::NP * G::NJ, 0);  // DS reads
            __builtin_amdgcn_sched_group_barrier(0x008, (2 * G::NP - 1) * G::NJ, 0);  // MFMA
        }

        // ---- online softmax over the tile in base 2: x = S c2 with c2 =
        // scale log2(e) / (sq sk) (keys past Lk score -inf, on the last tile
        // only)
        const float c2 = c0 * uk_t;
        float mt = -INFINITY;
        if (k0 + G::KT <= Lk) {
#pragma unroll
            for (int j = 0; j < G::NJ; ++j)
#pragma unroll
                for (int r = 0; r < G::SPT; ++r) mt = fmaxf(mt, s[j][r]);
        } else {
#pragma unroll
            for (int j = 0; j < G::NJ; ++j)
#pragma unroll
                for (int r = 0; r < G::SPT; ++r) {
                    if (k0 + G::MT * j + 8 * (r >> 2) + 4 * lg + (r & 3) >= Lk)
                        s[j][r] = -INFINITY;
                    mt = fmaxf(mt, s[j][r]);
                }
        }
        // The running max moves only on the first tile and when a tile's max
        // exceeds it by more than 7 in base 2 (a factor 2^7): P = 2^(x - m +
        // 8) then stays at most 2^15 (its fp16 hi part in range), and most
        // tiles leave the output's scale alone.  (A NaN max moves it, so that
        // NaN propagates.)
        const float mtu = xgroup_max<RW>(mt) * uk_t;
        const bool move = !(m_run >= mtu - thr);
        const float m_new = move ? mtu : m_run;
        const float alpha = move ? __builtin_amdgcn_exp2f((m_run - m_new) * c0) : 1.f;  // 0 on the first tile
        m_run = m_new;
        // P = 2^(x - c0 m_run + 8), the 2^8 that keeps P's lo parts from
        // fp16's subnormal range folded into the exponent: one FMA and one
        // v_exp_f32 per score, with c0 m_run rounded once per tile.  Where
        // |c0 m_run| reaches 2^8 that rounding would reach 2^-16 of the
        // exponent (and far more for huge logits, where it would turn the
        // weights of the largest scores into garbage): such waves first
        // rewrite each score as its difference from the max (one FMA, exact
        // near the max), as a plain softmax subtracts the max.
        const float mc = m_new * c0;
        float cx = c2, nm = 8.f - mc;
        if (__builtin_amdgcn_ballot_w64(!(__builtin_fabsf(mc) < 256.f))) {
#pragma unroll
            for (int j = 0; j < G::NJ; ++j)
#pragma unroll
                for (int r = 0; r < G::SPT; ++r) s[j][r] = fmaf(s[j][r], uk_t, -m_new);
            cx = c0;
            nm = 8.f;
        }
        float ps = 0.f;
        // P as the B operand of block b: the lane's scores 8 b .. 8 b + 7 in
        // the order of s (RW = 16: elements 0..3 from tile 2b, 4..7 from
        // tile 2b + 1, i.e. keys 4 lg + 0..3, 16 + 4 lg + 0..3 of the 32-key
        // block; RW = 32: registers 8 (b % 2) + 0..7 of tile b / 2, i.e.
        // keys 4 lg + 0..3, 8 + 4 lg + 0..3 of the 16-key block)
        pv_t ph[G::NB];
        f16x8 pl[G::NB];
#pragma unroll
        for (int b = 0; b < G::NB; ++b) {
            uint32_t h[4], l[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const int i0 = 8 * b + e, i1 = i0 + 1;
                const float p0 = __builtin_amdgcn_exp2f(fmaf(s[i0 / G::SPT][i0 % G::SPT], cx, nm));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(s[i1 / G::SPT][i1 % G::SPT], cx, nm));
                if constexpr (kBf) {
                    // P as bf16 (the operand type of the products with V's
                    // bits), the sum from the same rounded values, two per
                    // v_dot2_f32_bf16
                    h[e / 2] = l[e / 2] = pk_bf16_rne(p0, p1);
                    const bf16x2_t one2 = {(__bf16)1.f, (__bf16)1.f};
                    ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, h[e / 2]),
                                                         one2, ps, false);
                } else {
                    ps += p0;
                    ps += p1;
                    split2_f16_one(p0, p1, one, h[e / 2], l[e / 2]);
                }
            }
            ph[b] = __builtin_bit_cast(pv_t, make_uint4(h[0], h[1], h[2], h[3]));
            pl[b] = __builtin_bit_cast(f16x8, make_uint4(l[0], l[1], l[2], l[3]));
        }
        l_run = l_run * alpha + ps;  // this lane's keys; summed over lane groups at the end
        const float f = alpha * (uv_prev * sv_t);  // the old output in the new tile's units
        uv_prev = uv_t;
        if (__builtin_amdgcn_ballot_w64(f != 1.f)) {  // skipped while no row's max moves
                                                      // (and V's scale stays)
#pragma unroll
            for (int dt = 0; dt < G::NDT; ++dt) o[dt] *= f;
        }

        // ---- O^T += V^T P^T: A = V^T from the transposing read (each group
        // of 16 lanes reads 4 key rows x 16 dims; a lane receives its dim's 4
        // keys), keys of block b in P's order: rows 4 lg + 0..3, then
        // KD / 2 + 4 lg + 0..3 of the block; RW = 16: dims 16 dt + lane % 16;
        // RW = 32: dims 32 dt + lane % 32
        const int vrow = 4 * lg + ((lane & 15) >> 2);
        const int vcol = (RW == 32 ? 16 * ((lane >> 4) & 1) : 0) + 4 * (lane & 3);
        // (dt, b) = (i / NB, i % NB) in turn, the fragments of step i + 1
        // read before the products of step i (two register sets; as above,
        // not in the form held to 128 registers)
        constexpr bool kVPre = kPre;
        pv_t vh[2];
        f16x8 vl[2];
        auto vfrags = [&](int i, int r) {
            const int a = (G::KD * (i % G::NB) + vrow) * G::VSTR + G::MT * (i / G::NB) + vcol;
            constexpr int half = G::KD / 2 * G::VSTR;
            const uint2 h0 = lds_tr16(buf + G::V_HI + a);
            const uint2 h1 = lds_tr16(buf + G::V_HI + a + half);
            vh[r] = __builtin_bit_cast(pv_t, make_uint4(h0.x, h0.y, h1.x, h1.y));
            if constexpr (!kBf) {
                const uint2 l0 = lds_tr16(buf + G::V_LO + a);
                const uint2 l1 = lds_tr16(buf + G::V_LO + a + half);
                vl[r] = __builtin_bit_cast(f16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
            }
        };
        if constexpr (kVPre) vfrags(0, 0);
#pragma unroll
        for (int i = 0; i < G::NDT * G::NB; ++i) {
            const int dt = i / G::NB, b = i % G::NB, r = kVPre ? i & 1 : 0;
            if constexpr (kVPre) {
                if (i + 1 < G::NDT * G::NB) vfrags(i + 1, r ^ 1);
            } else {
                vfrags(i, 0);
            }
            o[dt] = mfma_rw(vh[r], ph[b], o[dt]);
            if constexpr (!kBf) {
                o[dt] = mfma_rw(vh[r], pl[b], o[dt]);
                o[dt] = mfma_rw(vl[r], ph[b], o[dt]);
            }
        }

        if (t + 2 < ntiles) maxima(k0 + 2 * G::KT, par);
        __syncthreads();
    }

    // ---- O = O^T uv / l (the sums' common unit cancels): stores of 4
    // consecutive dims (16 bytes fp32, 8 bytes bf16 rounded to nearest even).
    // With a key split: this split's normalized output in fp32 and its
    // statistics (running max, c0, log2 of the sum in units of 2^(c0 m)),
    // which k_flash_combine weighs.
    const float l = xgroup_sum<RW>(l_run);
    const float inv = uv_prev / l;
    if (qrow < Lq) {
        if (nsplit == 1) {
            T* orow = Og + ((size_t)bh * Lq + qrow) * D;
#pragma unroll
            for (int dt = 0; dt < G::NDT; ++dt)
#pragma unroll
                for (int r = 0; r < G::SPT; r += 4) {
                    const int d = G::MT * dt + 8 * (r >> 2) + 4 * lg;
                    if (d < D)
                        Elem<T>::st4(orow, d,
                                     make_float4(o[dt][r] * inv, o[dt][r + 1] * inv,
                                                 o[dt][r + 2] * inv, o[dt][r + 3] * inv));
                }
        } else {
            const size_t prow = (size_t)(bh * nsplit + sp) * Lq + qrow;
            float* orow = part + prow * D;
#pragma unroll
            for (int dt = 0; dt < G::NDT; ++dt)
#pragma unroll
                for (int r = 0; r < G::SPT; r += 4) {
                    const int d = G::MT * dt + 8 * (r >> 2) + 4 * lg;
                    if (d < D)
                        *reinterpret_cast<float4*>(orow + d) =
                            make_float4(o[dt][r] * inv, o[dt][r + 1] * inv, o[dt][r + 2] * inv,
                                        o[dt][r + 3] * inv);
                }
            if (lg == 0) stats[prow] = make_float4(m_run, c0, __log2f(l) - 8.f, 0.f);
        }
    }
}

// Merges the key splits of k_flash: for each (head, query) row, split s
// holds its normalized output O_s and statistics (m_s, c0, g_s) with
// log2 of its weight sum = c0 m_s + g_s (c0 is the same for every split of
// a row: the query's scale does not depend on the keys).  O = sum w_s O_s /
// sum w_s with w_s = 2^((m_s - M) c0 + g_s), M = max m_s (differences of the
// maxima first, so that huge logits stay exact).  One thread per 4 dims,
// 4 rows per workgroup.
template <typename T>
__global__ __launch_bounds__(256) void k_flash_combine(const float* __restrict__ part,
                                                       const float4* __restrict__ stats,
                                                       T* __restrict__ Og, int Lq, int D,
                                                       int nsplit, int rows) {
    const int t = threadIdx.x;
    const int row = blockIdx.x * 4 + (t >> 6), d = 4 * (t & 63);
    if (row >= rows || d >= D) return;
    const int bh = row / Lq, q = row - bh * Lq;
    const size_t base = (size_t)bh * nsplit * Lq + q;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, stats[base + (size_t)s * Lq].x);
    float wsum = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < nsplit; ++s) {
        const size_t pr = base + (size_t)s * Lq;
        const float4 st = stats[pr];
        const float w = __builtin_amdgcn_exp2f(fmaf(st.x - M, st.y, st.z));
        const float4 v = *reinterpret_cast<const float4*>(part + pr * D + d);
        wsum += w;
        acc.x = fmaf(w, v.x, acc.x);
        acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z);
        acc.w = fmaf(w, v.w, acc.w);
    }
    const float inv = 1.f / wsum;
    Elem<T>::st4(Og + (size_t)row * D, d,
                 make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv));
}

// the arguments of one flash call (pointers typed by the launch)
struct FlashArgs {
    const void *Q, *K, *V;
    void* O;
    int BH, Lq, Lk, D;
    float scale;
    PeSide pq, pk;
    int nsplit, kchunk;
    float* part;
    float4* stats;
};

template <typename T, int DP, int PEK, int NW, int RW>
hipError_t launch_t(const FlashArgs& a, hipStream_t st) {
    using G = FlashGeo<DP, PEK != kPeNone, NW, RW, sizeof(T) == 4>;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)k_flash<T, DP, PEK, NW, RW>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, G::BYTES);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const int qblocks = (a.Lq + G::ROWS - 1) / G::ROWS;
    const int kchunk = a.nsplit > 1 ? a.kchunk : a.Lk;
    hipLaunchKernelGGL((k_flash<T, DP, PEK, NW, RW>), dim3((unsigned)(a.BH * qblocks * a.nsplit)),
                       dim3(G::THREADS), G::BYTES, st, static_cast<const T*>(a.Q),
                       static_cast<const T*>(a.K), static_cast<const T*>(a.V), static_cast<T*>(a.O),
                       a.Lq, a.Lk, a.D, qblocks, a.scale, a.pq, a.pk, a.nsplit, kchunk, a.part,
                       a.stats);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    const int rows = a.BH * a.Lq;
    hipLaunchKernelGGL((k_flash_combine<T>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                       a.part, a.stats, static_cast<T*>(a.O), a.Lq, a.D, a.nsplit, rows);
    return hipGetLastError();
}

// head dims padded to 32, 64, 128 (and 256 for 8 waves of 16 rows without
// an encoding)
template <typename T, int PEK, int NW, int RW>
hipError_t launch_pe(const FlashArgs& a, hipStream_t st) {
    if (a.D <= 32) return launch_t<T, 32, PEK, NW, RW>(a, st);
    if (a.D <= 64) return launch_t<T, 64, PEK, NW, RW>(a, st);
    if (a.D <= 128) return launch_t<T, 128, PEK, NW, RW>(a, st);
    if constexpr (PEK == kPeNone && NW == 8 && RW == 16) return launch_t<T, 256, PEK, NW, RW>(a, st);
    return hipErrorInvalidValue;
}

template <typename T, int PEK>
hipError_t launch_form(int form, const FlashArgs& a, hipStream_t st) {
    // head dims past 128 run 8 waves of 16 rows: two buffers of a 256-wide
    // tile leave room for one workgroup per CU, and 32-row waves would not
    // hold the query's and the output's registers
    if (a.D > 128) form = kFlashForm8x16;
    switch (form) {
        case kFlashForm4x16: return launch_pe<T, PEK, 4, 16>(a, st);
        case kFlashForm8x16: return launch_pe<T, PEK, 8, 16>(a, st);
        case kFlashForm4x32: return launch_pe<T, PEK, 4, 32>(a, st);
        case kFlashForm8x32: return launch_pe<T, PEK, 8, 32>(a, st);
        default: return hipErrorInvalidValue;
    }
}

template <typename T>
hipError_t launch_typed(int pek, int form, const FlashArgs& a, hipStream_t st) {
    switch (pek) {
        case kPeNone: return launch_form<T, kPeNone>(form, a, st);
        case kPeRopeInterleaved: return launch_form<T, kPeRopeInterleaved>(form, a, st);
        case kPeRopeHalf: return launch_form<T, kPeRopeHalf>(form, a, st);
        case kPeSinusoidal: return launch_form<T, kPeSinusoidal>(form, a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool flash_supported(int dtype, int pek, int D) {
    return (dtype == kDtypeF32 || dtype == kDtypeBF16) && D >= 1 && D % 4 == 0 &&
           D <= (pek == kPeNone ? kFlashMaxD : kFlashMaxDEncoded);
}

hipError_t launch_flash(int dtype, int pek, int form, const void* Q, const void* K, const void* V,
                        void* O, int BH, int Lq, int Lk, int D, float scale, const PeSide& pq,
                        const PeSide& pk, int nsplit, int kchunk, float* part, hipStream_t st) {
    if (nsplit < 1 || (nsplit > 1 && (part == nullptr || kchunk < 1 ||
                                      (long long)kchunk * (nsplit - 1) >= Lk)))
        return hipErrorInvalidValue;
    FlashArgs a{Q, K, V, O, BH, Lq, Lk, D, scale, pq, pk, nsplit, kchunk, part,
                reinterpret_cast<float4*>(part + (size_t)nsplit * BH * Lq * D)};
    if (dtype == kDtypeF32) return launch_typed<float>(pek, form, a, st);
    if (dtype == kDtypeBF16) return launch_typed<uint16_t>(pek, form, a, st);
    return hipErrorInvalidValue;
}

}  // namespace atn
