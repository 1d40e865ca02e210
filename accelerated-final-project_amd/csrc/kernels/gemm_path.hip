// Long-sequence bf16 attention as two dense MFMA contractions (gfx950).
//
// For len_q, len_k >= 128 the score matrix is a dense Lq x Lk product and
// the work is MFMA-bound (Lq = Lk = 1024, D = 4096,
// 512 FLOP per byte).  A flash-style workgroup would have to keep its
// output rows on chip, and at D = 4096 even 64 rows of fp32 O are 1 MiB --
// more than a CU holds (512 KiB of registers, 160 KiB of LDS).  So the
// softmax is not fused into one pass; per head:
//
//   k_encode_f16  (with a positional encoding) Q~, K~ = encoded Q, K as
//                 fp16 rows with a power-of-two scale per row; with at most
//                 four 256-row query tiles K is not encoded here but inside
//                 the GEMM (k_gemm_qk_enc: fp16 tables, no K~ round trip)
//   k_gemm  (NT)  S = scale * Q K^T, kept on chip; per row of its 256-key
//                 tile t the epilogue writes E = exp(S - m_t) (fp16, in
//                 (0, 1]) and the tile's max m_t and sum l_t of E
//   k_gemm  (NN)  O = P V with P = E g_t, the factors of each row
//                 m = max_t m_t, l = sum_t l_t exp(m_t - m),
//                 g_t = exp(m_t - m) / l computed by each workgroup for its
//                 rows (k_rowscale does it beforehand for rows of more than
//                 8 key tiles) and applied to each A chunk on its way to LDS
//                 (bf16 P, bf16 O)
//
// so the row softmax is exact (max, exp, sum, divide as in the reference,
// final/attention.cu:262-270) without an S round trip through HBM; every
// stored value is in (0, 1], for any input range.
//
// Plain bf16 inputs are exact MFMA operands.  Encoded rows are not bf16
// values any more; rounding them back to bf16 (8-bit mantissa) costs up to
// ~2e-2 of rms on single outputs, so they are kept as fp16 (11-bit
// mantissa) instead, each row scaled by a power of two that puts its
// largest magnitude in [2^14, 2^15) -- safe for any input range -- and the
// GEMM epilogue multiplies the row and column scales back (exactly).
//
// Both GEMMs use 256 x 256 output tiles per workgroup of 512 threads (8
// waves, each 64 x 128 (NT) or 128 x 64 (NN) = 8 tiles of
// v_mfma_f32_32x32x16_{f16,bf16}), a K step of 64 in double-buffered LDS
// (144 KiB) fed from a register stage two steps ahead (the QK^T GEMM with
// an even number of steps loads both tiles straight into LDS instead:
// k_gemm_qk_dma, k_gemm_qk_enc), a software-pipelined
// step (fragment reads, LDS writes and global loads interleaved with the
// MFMAs, one barrier per step), and an
// XCD-aware tile order: consecutive tile indices run on the same XCD
// (workgroups are dealt round-robin to the 8 XCDs), so concurrent
// workgroups of one head share their Q/K/V panels in that XCD's L2.  The
// PV GEMM with V loaded straight into LDS (k_gemm_pv_dma) runs one
// persistent workgroup per CU when every tile is interior, each tile's
// first loads issued before the previous tile's output stores.
//
// V enters the second GEMM as the B operand, which MFMA wants contiguous
// along K (= keys); V rows are contiguous along D, so the V tile is stored
// in LDS as it lies in memory and the MFMA operand is gathered across keys
// by gfx950's transposing LDS read (ds_read_b64_tr_b16).
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "launch.hpp"

namespace atn {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kGemmThreads = 512;            // 8 waves
// wave grid (8 / waves_n) x waves_n: NT 4 x 2 (waves of 64 x 128), NN 2 x 4
// (128 x 64: four P fragments and two transposed V fragments per sub-step)
template <bool B_NN>
constexpr int waves_n() { return B_NN ? 4 : 2; }
constexpr int kLdsRow = kBK + 8;  // 16-bit elements per LDS row (16-byte aligned, padded)
constexpr int kTileElems = kBM * kLdsRow;
constexpr int kChunkPerRow = kBK / 8;

// 8 x 8-element MFMA step on raw 16-bit operands (bf16 or fp16 bits).
template <bool F16>
__device__ __forceinline__ v16f mfma_32x32x16(const uint4& a, const uint4& b, const v16f& c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Raw buffer descriptor over one head's matrix of n 16-bit elements (the host
// keeps it below 2^31 elements, so the byte count fits the 32-bit range).
// The base and size are workgroup-uniform; readfirstlane states it, so the
// descriptor lives in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const uint16_t* base, long n) {
    const uint64_t b = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const int bytes = __builtin_amdgcn_readfirstlane((int)(uint32_t)(2 * n));
    return __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, __builtin_amdgcn_readfirstlane(soff), 0));
}

// Tile index of this workgroup with consecutive indices kept on one XCD:
// hardware deals workgroup w to XCD w % 8, so XCD x gets tiles
// [x * per, (x + 1) * per).
__device__ __forceinline__ long xcd_tile(long w, long total) {
    const long per = (total + 7) / 8;
    const long t = (w % 8) * per + w / 8;
    return t;  // may be >= total for the last XCD: caller checks
}

// NN B tile in LDS: [kBK keys][kBN columns], rows unpadded, with the 16-column
// (32-byte) chunks of key row k permuted by XOR with kNNSwz[k % 4].  The
// transposing read takes, per 16 lanes, one 32-byte chunk from each of 4
// consecutive keys (and the next chunk for the next 16 lanes); {0, 2, 5, 7}
// puts those chunks in distinct banks for 32 or 64 four-byte banks, and the
// 16-byte row writes stay whole 128 / 256-byte runs.
__device__ __forceinline__ int nn_lds_off(int k, int n) {
    const int swz = (0x7520 >> (4 * (k & 3))) & 0xf;  // {0, 2, 5, 7}[k % 4]
    return k * kBN + ((((n >> 4) ^ swz)) << 4) + (n & 15);
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4i16 ds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(p));
}

// Scheduling pattern for one sub-step: MFMA, then fragment reads, six times;
// the R reads are spread as evenly as possible (mask 0x008 = MFMA,
// 0x100 = LDS read).
template <int R>
__device__ __forceinline__ void sched_mfma_reads() {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, R / 6 + (0 < R % 6 ? 1 : 0), 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, R / 6 + (1 < R % 6 ? 1 : 0), 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, R / 6 + (2 < R % 6 ? 1 : 0), 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, R / 6 + (3 < R % 6 ? 1 : 0), 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, R / 6 + (4 < R % 6 ? 1 : 0), 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, R / 6 + (5 < R % 6 ? 1 : 0), 0);
}

// Epilogue selectors
constexpr int kOutExpF16 = 0;     // C = fp16 exp(S - tile row max), S = scale * acc; stats
constexpr int kOutBf16 = 1;       // C = bf16(acc), row stride ldc

// fp16 bits of the 8 elements of w, times f, as 8 bf16.  Each product is
// one v_fma_mix_f32 (an fp16 half of a register widened and multiplied in
// fp32, with a zero addend: the rounding of the product itself), and each
// pair is rounded to bf16 (nearest even) by gfx950's v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float f16lo_mul(uint32_t x, float f) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(f));
    return r;
}
__device__ __forceinline__ float f16hi_mul(uint32_t x, float f) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(f));
    return r;
}
__device__ __forceinline__ uint4 scale_f16x8_to_bf16(const uint4& w, float f) {
    const uint32_t x[4] = {w.x, w.y, w.z, w.w};
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bf16x2_t b = {(__bf16)f16lo_mul(x[i], f), (__bf16)f16hi_mul(x[i], f)};
        y[i] = __builtin_bit_cast(uint32_t, b);
    }
    return make_uint4(y[0], y[1], y[2], y[3]);
}

// Lane permutations by DPP with bound_ctrl set: the controls used here read
// in-range lanes only, so no old value is needed (and the compiler keeps no
// zeroed destination for it).
template <int Ctrl>
__device__ __forceinline__ float dppb(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, true));
}
// Max / sum over each half-wave (lanes with the same lane / 32): DPP within
// quads, 8 and 16 lanes, then the 16-lane hop by ds_swizzle.
// Inline asm that reads MFMA results must run after the MFMA pipeline has
// written them: the compiler places the wait states before its own
// instructions, not before inline asm.  This is the accumulator tile's
// next reader and waits 24 cycles first (an MFMA of 16 passes needs 18),
// so every MFMA issued before it has written its results.
__device__ __forceinline__ void mfma_settle(v16f& a) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a));
}

__device__ __forceinline__ float half_max(float v) {
    v = vmaxf(v, dppb<kDppQuadXor1>(v));
    v = vmaxf(v, dppb<kDppQuadXor2>(v));
    v = vmaxf(v, dppb<kDppRowHalfMirror>(v));
    v = vmaxf(v, dppb<kDppRowMirror>(v));
    return vmaxf(v, swz_xor16(v));
}
__device__ __forceinline__ float half_sum(float v) {
    v += dppb<kDppQuadXor1>(v);
    v += dppb<kDppQuadXor2>(v);
    v += dppb<kDppRowHalfMirror>(v);
    v += dppb<kDppRowMirror>(v);
    return v + swz_xor16(v);
}

// C[M x N] = A[M x K] * B^T where B is [N x K] (NT, both K-contiguous) when
// B_NN == false, or A[M x K] * B with B [K x N] N-contiguous when B_NN.
// Batched over heads: A/B/C advance by their head strides per bh.
struct GemmArgs {
    const uint16_t* A;
    const uint16_t* B;
    void* C;
    const float* rs;              // optional per-row scales [heads][M] (or NULL)
    const float* cs;              // optional per-column scales [heads][N] (or NULL)
    float* st_m;                  // NT exp epilogue: tile row maxima [heads][M][tiles_n]
    float* st_l;                  // NT exp epilogue: tile row sums of E [heads][M][tiles_n]
    const float* ga;              // NN: factors of A's rows per 256-column tile [heads][M][gt]
    int gt;                       // NN: 256-column tiles per row of A
    int M, N, K;
    long lda, ldb, ldc;           // row strides (elements)
    long sa, sb, sc;              // head strides (elements)
    int tiles_m, tiles_n, heads;  // grid decomposition
    float scale;
    const uint16_t* tab;          // fused K encoding: fp16 table (k_gemm_qk_enc)
    int tab_rows;                 // positions in tab
};

// NT exp epilogue: scores S = scale * acc * (row scale) * (column scale) of
// this 256-key tile; per row its maximum m_t over the tile's valid columns
// and the sum l_t of E = exp(S - m_t).  A row's 256 columns are 32 lanes x
// TJ tiles in each of the two column waves (wave % 2), combined through LDS
// (red: 6 x 256 floats, free once every wave is done with the K loop: the
// row maxima and sums of both column waves, then the tile's row and column
// scales).  Lane layout of acc[i][j]: column (lane % 32) and rows
// 8 (r / 4) + 4 (lane / 32) + r % 4 of each 32 x 32 tile.
// cs_lds (optional) replaces g.cs: the tile's 256 column scales in LDS.
//
// The row factor f = scale * (row scale) is positive, so with
// u = acc * (column scale) the row maximum of S is (max u) * f, and
// E = exp(u f - (max u) f) = exp2(u f log2(e) - (max u) f log2(e)): one fma
// and one exp2 per element.
template <int TI, int TJ>
__device__ __forceinline__ void nt_exp_epilogue(const GemmArgs& g, v16f (&acc)[TI][TJ],
                                                float* red, int bh, int m0, int n0, int tn,
                                                int wm, int wn, int wave, int lane,
                                                const float* cs_lds = nullptr) {
    static_assert(kGemmThreads == kBM + kBN, "one scale per thread");
    constexpr float kLog2e = 1.4426950408889634f;
    // Each thread fetches one of the tile's 256 row or 256 column scales
    // before the barrier (its latency overlaps the wait) and puts it in LDS:
    // per element, each a load from memory behind a branch, they were
    // waited for one at a time.
    const int tid = wave * 64 + lane;
    const bool col_scales = cs_lds != nullptr || g.cs != nullptr;
    float sv = 1.f;
    if (tid < kBM) {
        const int row = m0 + tid;
        if (g.rs && row < g.M) sv = g.rs[(long)bh * g.M + row];
    } else {
        const int col = n0 + tid - kBM;
        if (col_scales && col < g.N) sv = cs_lds ? cs_lds[col - n0] : g.cs[(long)bh * g.N + col];
    }
    __syncthreads();  // every wave is done with the LDS stages
    red[4 * kBM + tid] = sv;
    __syncthreads();
    const float* rsl = red + 4 * kBM;
    const float* csl = red + 5 * kBM;
    const int half = lane >> 5, lc = lane & 31, cw = wave & 1;
    const bool interior = m0 + kBM <= g.M && n0 + kBN <= g.N;
    // u = acc * (column scale); columns past N are -inf
    if (col_scales || !interior) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int cl = wn + j * 32 + lc;
            const bool ok = n0 + cl < g.N;
            const float c = csl[cl];
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = ok ? acc[i][j][r] * c : -INFINITY;
        }
    }
    // (the row maxima below read the accumulators by inline asm)
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) mfma_settle(acc[i][j]);
    float rm[TI][16], rl[TI][16];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float m = acc[i][0][r];
#pragma unroll
            for (int j = 1; j < TJ; ++j) m = vmaxf(m, acc[i][j][r]);
            rm[i][r] = half_max(m);
        }
    auto rloc = [&](int i, int r) { return wm + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3); };
    if (lc == 0)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[cw * kBM + rloc(i, r)] = rm[i][r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float mu = vmaxf(rm[i][r], red[(cw ^ 1) * kBM + rloc(i, r)]);
            const float gl = g.scale * rsl[rloc(i, r)] * kLog2e;
            // a row with no valid column keeps max u = -inf: its E are 0
            const float nb = mu == -INFINITY ? 0.f : -(mu * gl);
            float l = 0.f;
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const float e = __builtin_amdgcn_exp2f(fmaf(acc[i][j][r], gl, nb));
                acc[i][j][r] = e;
                l += e;
            }
            rl[i][r] = half_sum(l);
        }
    uint16_t* C = static_cast<uint16_t*>(g.C) + bh * g.sc;
    if (interior) {
        // E of an interior tile, stored before the row sums' exchange and
        // the statistics (the stores drain meanwhile): buffer stores, the
        // lane's (i, j) offset in a register, the row offset of r in a
        // scalar register
        const __amdgpu_buffer_rsrc_t rc = gemm_rsrc(C, (long)g.M * g.ldc);
        const uint32_t ldc = (uint32_t)g.ldc;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const uint32_t vo =
                    2u * ((uint32_t)(m0 + wm + i * 32 + 4 * half) * ldc + (uint32_t)(n0 + wn + j * 32 + lc));
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t so = 2u * (uint32_t)(8 * (r >> 2) + (r & 3)) * ldc;
                    __builtin_amdgcn_raw_buffer_store_b16(
                        __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][r]), rc, (int)vo,
                        (int)__builtin_amdgcn_readfirstlane(so), 0);
                }
            }
    }
    if (lc == 0)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[(2 + cw) * kBM + rloc(i, r)] = rl[i][r];
    __syncthreads();
    // statistics, one row per thread: m_t = (max u) f, l_t
    if (tid < kBM && m0 + tid < g.M) {
        const float mu = fmaxf(red[tid], red[kBM + tid]);
        const long si = ((long)bh * g.M + m0 + tid) * g.tiles_n + tn;
        g.st_m[si] = mu * (g.scale * rsl[tid]);
        g.st_l[si] = red[2 * kBM + tid] + red[3 * kBM + tid];
    }
    if (interior) return;
    // edge tile: columns past N (E = exp(-inf) = 0) are written too up to
    // the row stride ldc, so the padding of an E row (ldc = N rounded up to
    // 8 keys) holds zeros for the PV GEMM's 8-key chunks
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = n0 + wn + j * 32 + lc;
            if (col >= g.ldc) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + rloc(i, r);
                if (row < g.M)
                    C[(long)row * g.ldc + col] =
                        __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][r]);
            }
        }
}
// NN softmax factors of A's rows: kept in LDS ([256 rows][gt], read when a
// chunk is stored) when a row has at most kFacTiles 256-key tiles, else
// loaded with each chunk into the register stage.
constexpr int kFacTiles = 8;

template <bool F16, bool B_NN, int OUT, bool FAC_LDS = false>
__global__ __launch_bounds__(kGemmThreads) void k_gemm(GemmArgs g) {
    // one LDS block: A stages 0/1, then B^T stages 0/1 ([n][k] rows); the
    // bf16 epilogue reuses it whole as an output staging tile
    __shared__ __align__(16) uint16_t lds[4 * kTileElems];
    __shared__ float fac[FAC_LDS ? kBM * kFacTiles : 1];
    uint16_t(*As)[kTileElems] = reinterpret_cast<uint16_t(*)[kTileElems]>(lds);
    uint16_t(*Bs)[kTileElems] = reinterpret_cast<uint16_t(*)[kTileElems]>(lds + 2 * kTileElems);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long per_head = (long)g.tiles_m * g.tiles_n;
    const long total = per_head * g.heads;
    const long t = xcd_tile(blockIdx.x, total);
    if (t >= total) return;
    const int bh = __builtin_amdgcn_readfirstlane((int)(t / per_head));
    const int rem = (int)(t - (long)bh * per_head);
    // within a head: NT runs row panels outer (neighbours share the Q
    // panel); NN runs row panels fastest, so the few workgroups of one V
    // panel run together and share it in L2
    int tm, tn;
    if constexpr (B_NN) {
        tn = rem / g.tiles_m;
        tm = rem - tn * g.tiles_m;
    } else {
        tm = rem / g.tiles_n;
        tn = rem - tm * g.tiles_n;
    }
    // the tile's coordinates are workgroup-uniform: keep them (and what is
    // derived from them) in scalar registers
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kBM);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kBN);

    const uint16_t* A = g.A + bh * g.sa;
    const uint16_t* B = g.B + bh * g.sb;

    // ---- global -> register staging: each thread moves 16-byte chunks of A
    // (rows m0.., kChunkPerRow chunks of 8 per row) and of B: for NT, chunks
    // of B^T rows, the same way; for NN, chunks of the B rows (keys k0..,
    // 32 chunks of 8 columns per row), which stay N-contiguous in LDS and are
    // transposed by the LDS read (ds_read_b64_tr_b16).
    constexpr int kChunks = kBM * kBK / 8 / kGemmThreads;  // 16-byte chunks per thread per operand
    constexpr int kNNChunkPerRow = kBN / 8;
    static_assert(kChunks >= 1 && kBK * kBN / 8 / kGemmThreads == kChunks,
                  "tile too small for the thread count");
    static_assert(kBK * kBN <= kTileElems, "NN B tile does not fit its LDS stage");
    struct Stage {
        uint4 a[kChunks], b[kChunks];
        float ga[(B_NN && !FAC_LDS) ? kChunks : 1];  // NN: factor of each A chunk
    };
    // A tile that lies inside the matrices (EDGE false) loads without bounds
    // checks: straight-line code that the scheduler can spread among the
    // MFMAs.  Edge tiles zero-fill what lies outside.
    // Offsets within one head's matrix are 32-bit (the host keeps every
    // per-head matrix below 2^31 elements): a uniform base plus a per-lane
    // 32-bit offset is the global_load form with the base in SGPRs.
    auto load_chunk = [&](const uint16_t* base, long ld, int r, int c, int rmax, int cmax,
                          auto edge) -> uint4 {
        if constexpr (decltype(edge)::value) {
            if (r >= rmax || c >= cmax) return make_uint4(0, 0, 0, 0);
        }
        const uint32_t off = (uint32_t)r * (uint32_t)ld + (uint32_t)c;
        return *reinterpret_cast<const uint4*>(base + off);
    };
    const float* ga = B_NN ? g.ga + (long)bh * g.M * g.gt : nullptr;
    // Interior tiles load through buffer descriptors: one per-lane byte
    // offset per operand, constant over the K loop, and the chunk's row and
    // the step's k0 in the scalar offset, so the loads need no per-step
    // address arithmetic and no 64-bit address registers.
    const __amdgpu_buffer_rsrc_t ra = gemm_rsrc(A, (long)g.M * g.lda);
    const __amdgpu_buffer_rsrc_t rb =
        gemm_rsrc(B, B_NN ? (long)g.K * g.ldb : (long)g.N * g.ldb);
    const uint32_t va = 2u * ((uint32_t)(tid / kChunkPerRow) * (uint32_t)g.lda +
                              (uint32_t)((tid % kChunkPerRow) * 8));
    const uint32_t vb =
        B_NN ? 2u * ((uint32_t)(tid / kNNChunkPerRow) * (uint32_t)g.ldb +
                     (uint32_t)((tid % kNNChunkPerRow) * 8))
             : 2u * ((uint32_t)(tid / kChunkPerRow) * (uint32_t)g.ldb +
                     (uint32_t)((tid % kChunkPerRow) * 8));
    constexpr int kRowsPerPass = kGemmThreads / kChunkPerRow;     // A / NT B rows per u
    constexpr int kKeysPerPass = kGemmThreads / kNNChunkPerRow;   // NN B keys per u
    auto load_stage_buf = [&](Stage& r, int k0) {
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const uint32_t so = 2u * ((uint32_t)(m0 + u * kRowsPerPass) * (uint32_t)g.lda +
                                      (uint32_t)k0);
            r.a[u] = buf_ld16(ra, va, so);
            if constexpr (B_NN && !FAC_LDS) {
                const int row = tid / kChunkPerRow + u * kRowsPerPass,
                          k8 = (tid % kChunkPerRow) * 8;
                r.ga[u] = ga[(uint32_t)(m0 + row) * (uint32_t)g.gt + (uint32_t)((k0 + k8) >> 8)];
            }
        }
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const uint32_t so =
                B_NN ? 2u * ((uint32_t)(k0 + u * kKeysPerPass) * (uint32_t)g.ldb + (uint32_t)n0)
                     : 2u * ((uint32_t)(n0 + u * kRowsPerPass) * (uint32_t)g.ldb + (uint32_t)k0);
            r.b[u] = buf_ld16(rb, vb, so);
        }
    };
    auto load_stage = [&](Stage& r, int k0, auto edge) {
        if constexpr (!decltype(edge)::value) {
            load_stage_buf(r, k0);
            return;
        }
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int cidx = tid + u * kGemmThreads;
            const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
            r.a[u] = load_chunk(A, g.lda, m0 + row, k0 + k8, g.M, g.K, edge);
            if constexpr (B_NN && !FAC_LDS) {
                // a chunk's 8 keys lie in one 256-key tile of the scores
                const int gr = m0 + row;
                r.ga[u] = 0.f;
                if (!decltype(edge)::value || gr < g.M)
                    r.ga[u] = ga[(uint32_t)gr * (uint32_t)g.gt + (uint32_t)((k0 + k8) >> 8)];
            }
        }
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int cidx = tid + u * kGemmThreads;
            if constexpr (!B_NN) {
                const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
                r.b[u] = load_chunk(B, g.ldb, n0 + row, k0 + k8, g.N, g.K, edge);
            } else {
                // B is [K x N]: chunk c covers key c / 32, columns (c % 32) * 8 ..
                const int kr = cidx / kNNChunkPerRow, n8 = (cidx % kNNChunkPerRow) * 8;
                r.b[u] = load_chunk(B, g.ldb, k0 + kr, n0 + n8, g.K, g.N, edge);
            }
        }
    };
    auto store_stage = [&](const Stage& r, int s, int k0) {
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int cidx = tid + u * kGemmThreads;
            const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
            if constexpr (B_NN) {  // P = E * g: fp16 E scaled, rounded to bf16
                float f;
                if constexpr (FAC_LDS)
                    f = fac[row * kFacTiles + ((k0 + k8) >> 8)];
                else
                    f = r.ga[u];
                *reinterpret_cast<uint4*>(&As[s][row * kLdsRow + k8]) =
                    scale_f16x8_to_bf16(r.a[u], f);
            } else {
                (void)k0;
                *reinterpret_cast<uint4*>(&As[s][row * kLdsRow + k8]) = r.a[u];
            }
        }
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int cidx = tid + u * kGemmThreads;
            if constexpr (!B_NN) {
                const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
                *reinterpret_cast<uint4*>(&Bs[s][row * kLdsRow + k8]) = r.b[u];
            } else {
                const int kr = cidx / kNNChunkPerRow, n8 = (cidx % kNNChunkPerRow) * 8;
                *reinterpret_cast<uint4*>(&Bs[s][nn_lds_off(kr, n8)]) = r.b[u];
            }
        }
    };

    // ---- wave tile: TI x TJ MFMA tiles of 32 x 32
    constexpr int WN = waves_n<B_NN>();
    constexpr int TI = kBM / (kGemmThreads / 64 / WN) / 32, TJ = kBN / WN / 32;
    const int wm = (wave / WN) * (TI * 32), wn = (wave % WN) * (TJ * 32);
    v16f acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // MFMA operands of one 16-wide sub-step
    struct Frag {
        uint4 a[TI], b[TJ];
    };
    const int lrow = lane & 31, lkh = (lane >> 5) * 8;
    auto read_frag = [&](Frag& f, int s, int ks) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
            f.a[i] = *reinterpret_cast<const uint4*>(&As[s][(wm + i * 32 + lrow) * kLdsRow + ks + lkh]);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            if constexpr (!B_NN) {
                f.b[j] = *reinterpret_cast<const uint4*>(
                    &Bs[s][(wn + j * 32 + lrow) * kLdsRow + ks + lkh]);
            } else {
                // lane L supplies the address of keys ks + 8 (L / 32) + 4 h +
                // (L % 16) / 4, columns wn + 32 j + 16 ((L / 16) % 2) + 4 (L % 4);
                // the transposing read hands lane l keys ks + 8 (l / 32) + 4 h
                // + 0..3 of column wn + 32 j + l % 32: half h of its operand
                const int kr = ks + 8 * (lane >> 5) + ((lane & 15) >> 2);
                const int nc = wn + j * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
                const v4i16 lo = ds_read_tr16(&Bs[s][nn_lds_off(kr, nc)]);
                const v4i16 hi = ds_read_tr16(&Bs[s][nn_lds_off(kr + 4, nc)]);
                const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
                f.b[j] = make_uint4(l2.x, l2.y, h2.x, h2.y);
            }
        }
    };
    // NN runs the product transposed, acc[i][j] = (B^T A^T) tile: its
    // accumulator rows are output columns, so each lane ends up with four
    // consecutive output columns of one output row (see the epilogue)
    auto mma = [&](const Frag& f) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                if constexpr (B_NN)
                    acc[i][j] = mfma_32x32x16<F16>(f.b[j], f.a[i], acc[i][j]);
                else
                    acc[i][j] = mfma_32x32x16<F16>(f.a[i], f.b[j], acc[i][j]);
            }
    };

    // ---- K loop, software-pipelined over the four 16-wide sub-steps of a
    // step: sub-step q + 1's fragments are read while sub-step q's MFMAs run;
    // step kt + 1's tile (in registers since step kt - 1) goes to the other
    // LDS buffer during sub-step 0, and step kt + 2's global loads are issued
    // during sub-step 1, a whole step ahead of their use; the one barrier per
    // step sits before sub-step 3's MFMAs, so the first fragments of step
    // kt + 1 are read while those run.  Buffer kt % 2 is rewritten only in
    // step kt + 1, after every wave passed the barrier that ends its reads.
    // The last two steps are peeled (no store / no load), so the steady-state
    // step is one basic block, and sched_group_barrier interleaves its LDS
    // and global memory instructions one or two at a time between the MFMAs.
    const int nk = (g.K + kBK - 1) / kBK;
    constexpr int kReads = TI + (B_NN ? 2 : 1) * TJ;  // LDS reads per fragment set
    constexpr int kMfma = TI * TJ;                    // MFMAs per sub-step
    static_assert(kMfma >= 8 && kReads <= 12, "interleave pattern assumes 8 MFMAs per sub-step");
    auto sched_reads = [&]() { sched_mfma_reads<kReads>(); };
    Stage st;
    Frag f0, f1;
    auto step = [&](int kt, auto next, auto next2, auto edge) {
        constexpr bool N1 = decltype(next)::value, N2 = decltype(next2)::value;
        const int s = kt & 1;
        // sub-step 0: MFMAs on f0, read f1, write step kt + 1's tile
        read_frag(f1, s, 16);
        mma(f0);
        if constexpr (N1) store_stage(st, s ^ 1, (kt + 1) * kBK);
        sched_reads();
        if constexpr (N1) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, kChunks, 0);  // DS write
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, kChunks, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        // sub-step 1: MFMAs on f1, read f0, global loads of step kt + 2
        if constexpr (N2) load_stage(st, (kt + 2) * kBK, edge);
        read_frag(f0, s, 32);
        mma(f1);
        sched_reads();
        if constexpr (N2) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, kChunks, 0);  // VMEM read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, kChunks, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        // sub-step 2: MFMAs on f0, read f1
        read_frag(f1, s, 48);
        mma(f0);
        sched_reads();
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        // sub-step 3: MFMAs on f1, read step kt + 1's first fragments
        if constexpr (N1) read_frag(f0, s ^ 1, 0);
        mma(f1);
        if constexpr (N1) sched_reads();
        __builtin_amdgcn_sched_barrier(0);
    };
    auto kloop = [&](auto edge) {
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        if constexpr (FAC_LDS) {
            // the workgroup's rows' softmax factors ([row][tile], kFacTiles >=
            // gt), from the QK^T epilogue's per-(row, 256-key tile) max m_t
            // and sum l_t, with k_rowscale's arithmetic: m = max_t m_t,
            // l = sum_t l_t exp(m_t - m), g_t = exp(m_t - m) / l (0 for a row
            // with no valid key)
            if (tid < kBM) {
                const int row = m0 + tid;
                const long base = ((long)bh * g.M + row) * g.gt;
                float mt[kFacTiles], lt[kFacTiles];
                float m = -INFINITY;
#pragma unroll
                for (int t = 0; t < kFacTiles; ++t) {
                    const bool on = row < g.M && t < g.gt;
                    mt[t] = on ? g.st_m[base + t] : -INFINITY;
                    lt[t] = on ? g.st_l[base + t] : 0.f;
                    m = fmaxf(m, mt[t]);
                }
                float l = 0.f;
#pragma unroll
                for (int t = 0; t < kFacTiles; ++t)
                    if (t < g.gt) l += lt[t] * __expf(mt[t] - m);
                const float inv = 1.0f / l;
#pragma unroll
                for (int t = 0; t < kFacTiles; ++t)
                    fac[tid * kFacTiles + t] =
                        (m == -INFINITY || t >= g.gt) ? 0.f : __expf(mt[t] - m) * inv;
            }
        }
        load_stage(st, 0, edge);
        if constexpr (FAC_LDS) __syncthreads();
        store_stage(st, 0, 0);
        if (nk > 1) load_stage(st, kBK, edge);
        __syncthreads();
        read_frag(f0, 0, 0);
        int kt = 0;
        for (; kt + 2 < nk; ++kt) step(kt, T{}, T{}, edge);
        if (kt + 1 < nk) {
            step(kt, T{}, F{}, edge);
            ++kt;
        }
        step(kt, F{}, F{}, edge);
    };
    if (m0 + kBM <= g.M && n0 + kBN <= g.N && g.K % kBK == 0)
        kloop(std::integral_constant<bool, false>{});
    else
        kloop(std::integral_constant<bool, true>{});

    // ---- epilogue.  NT: lane holds column (lane % 32) and rows
    // 8 * (r / 4) + 4 * (lane / 32) + r % 4 of each 32 x 32 tile.
    // NN (transposed product): lane holds output row m0 + wm + 32 i + lane % 32
    // and columns n0 + wn + 32 j + 8 * (r / 4) + 4 * (lane / 32) + r % 4, i.e.
    // four consecutive bf16 per group of four r, stored as one 8-byte word
    // (N is a multiple of 4, so a group is wholly inside or outside).
    if constexpr (OUT == kOutBf16) {
        static_assert(B_NN, "bf16 output comes from the NN product");
        uint16_t* C = static_cast<uint16_t*>(g.C) + bh * g.sc;
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int row = m0 + wm + i * 32 + (lane & 31);
            if (row >= g.M) continue;
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int rg = 0; rg < 4; ++rg) {
                    const int col = n0 + wn + j * 32 + 8 * rg + 4 * (lane >> 5);
                    if (col >= g.N) continue;
                    uint2 w;
                    w.x = (uint32_t)f32_to_bf16_bits(acc[i][j][4 * rg]) |
                          ((uint32_t)f32_to_bf16_bits(acc[i][j][4 * rg + 1]) << 16);
                    w.y = (uint32_t)f32_to_bf16_bits(acc[i][j][4 * rg + 2]) |
                          ((uint32_t)f32_to_bf16_bits(acc[i][j][4 * rg + 3]) << 16);
                    *reinterpret_cast<uint2*>(C + (long)row * g.ldc + col) = w;
                }
        }
        return;
    }
    // ---- NT epilogue (exp of the scores, tile row statistics)
    if constexpr (OUT == kOutExpF16) {
        static_assert(!B_NN && WN == 2, "the exp epilogue is the NT product's");
        nt_exp_epilogue<TI, TJ>(g, acc, reinterpret_cast<float*>(lds), bh, m0, n0, tn, wm, wn,
                                wave, lane);
    }
}

// ---------------------------------------------------------------------------
// QK^T GEMM with K's encoding applied on its way to LDS (no K~ pass).
//
// B = raw bf16 K rows, read through the register stage together with 16
// bytes of fp16 table per 16-byte chunk, and written to LDS as unscaled fp16
// K~ (exact for raw values in fp16's range):
//   kBEncRaw       K~ = K (the query side alone is encoded)
//   kBEncSin       K~ = K + PE, table [pos][D]: sin on even dims, cos on odd
//   kBEncRope      interleaved rotation of pairs (2i, 2i + 1), table [pos][D/2]
//                  of (cos, sin) words, (1, 0) past the rotary width
//   kBEncRopeHalf  rotate-half, pairs (i, i + D/2): each K step takes 32 dims
//                  of the first half and their 32 partners (A's columns in the
//                  same order), so both halves of a rotation are in one thread
// Each value is rounded once to fp16.  A workgroup whose K tile holds a row
// with |K~| > 65504 computes its tile a second time with per-row power-of-two
// scales (the largest |K~| of each key row, tracked during the first pass,
// placed in [2^14, 2^15) as k_encode_f16 does), so any input range works.
//
// A = Q~ (k_encode_f16's fp16 rows, scales in rs) goes straight from memory
// to LDS (buffer loads with the LDS destination, no register stage): each
// wave instruction writes one 1 KiB run of 8 unpadded rows, chunk c of row r
// stored at position c ^ key(r), key(r) = (r & 7) ^ ((r >> 3) & 1), so the
// fragment reads (16 rows of one chunk per 16 lanes) hit distinct banks for
// 32 or 64 banks.  Out-of-range rows and columns load from an offset past the
// descriptor's range, which writes zeros.
//
// The stages are separate LDS arrays and the K loop runs two steps per
// iteration, so every LDS access names its stage at compile time: the
// compiler can tell the DMA's target from the tiles being read, and the one
// barrier per step waits only for the DMA (the next step's K loads stay in
// flight).
constexpr int kBEncRaw = kGemmEncRaw, kBEncSin = kGemmEncSin, kBEncRope = kGemmEncRope,
              kBEncRopeHalf = kGemmEncRopeHalf;

// v_fma_mix_f32 forms: fp32 a times one fp16 half of t, plus fp32 c, rounded
// once to fp32.
__device__ __forceinline__ float fmix_lo(float a, uint32_t t, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(t), "v"(c));
    return r;
}
__device__ __forceinline__ float fmix_hi(float a, uint32_t t, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
        : "=v"(r) : "v"(a), "v"(t), "v"(c));
    return r;
}
__device__ __forceinline__ float fmix_lo_sub(float a, uint32_t t, float c) {  // a lo(t) - c
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, -%3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(t), "v"(c));
    return r;
}
__device__ __forceinline__ float fmul_lo(float a, uint32_t t) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(t));
    return r;
}
__device__ __forceinline__ float fmul_hi(float a, uint32_t t) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(t));
    return r;
}
__device__ __forceinline__ float fadd_lo(float a, uint32_t t) {  // a + lo(t)
    float r;
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[0,0,1]" : "=v"(r) : "v"(a), "v"(t));
    return r;
}
__device__ __forceinline__ float fadd_hi(float a, uint32_t t) {  // a + hi(t)
    float r;
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "=v"(r) : "v"(a), "v"(t));
    return r;
}
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_f16(float a, float b) {  // v_cvt_pk_f16_f32 (nearest even)
    const f16x2_t v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// 8 bf16 -> 8 fp16: as they are, or plus the chunk's table values (sinusoidal),
// or rotated pairwise (interleaved RoPE).  Unscaled (SC false), mx keeps the
// largest |K~|; scaled, every value is multiplied by the row scale sc (a
// power of two) before its one rounding to fp16.
template <int BENC, bool SC = false>
__device__ __forceinline__ uint4 enc_chunk(const uint4& w, const uint4& t, float& mx,
                                           float sc = 1.f) {
    const uint32_t x[4] = {w.x, w.y, w.z, w.w};
    const uint32_t tt[4] = {t.x, t.y, t.z, t.w};
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float a = bf16_lo(x[i]), b = bf16_hi(x[i]);
        if constexpr (BENC == kBEncSin) {
            a = fadd_lo(a, tt[i]);
            b = fadd_hi(b, tt[i]);
        } else if constexpr (BENC == kBEncRope) {
            // (a, b) = dims (2i', 2i' + 1); tt[i] = (cos, sin) of pair i'
            const float a0 = a;
            a = fmix_lo_sub(a0, tt[i], fmul_hi(b, tt[i]));  // a cos - b sin
            b = fmix_hi(a0, tt[i], fmul_lo(b, tt[i]));      // a sin + b cos
        }
        if constexpr (SC) {
            a *= sc;
            b *= sc;
        } else {
            mx = vmax3abs(mx, a, b);
        }
        y[i] = pk_f16(a, b);
    }
    return make_uint4(y[0], y[1], y[2], y[3]);
}

// Rotate-half: w0 = 8 dims of the first half, w1 = their partners, t0/t1 =
// (cos, sin) words of the 8 pairs; both chunks rewritten as fp16.
template <bool SC = false>
__device__ __forceinline__ void enc_half(uint4& w0, uint4& w1, const uint4& t0, const uint4& t1,
                                         float& mx, float sc = 1.f) {
    const uint32_t x0[4] = {w0.x, w0.y, w0.z, w0.w}, x1[4] = {w1.x, w1.y, w1.z, w1.w};
    const uint32_t tt[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
    uint32_t y0[4], y1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float r0[2], r1[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float a = h ? bf16_hi(x0[i]) : bf16_lo(x0[i]);
            const float b = h ? bf16_hi(x1[i]) : bf16_lo(x1[i]);
            const uint32_t w = tt[2 * i + h];
            r0[h] = fmix_lo_sub(a, w, fmul_hi(b, w));  // a cos - b sin
            r1[h] = fmix_hi(a, w, fmul_lo(b, w));      // a sin + b cos
            if constexpr (SC) {
                r0[h] *= sc;
                r1[h] *= sc;
            } else {
                mx = vmax3abs(mx, r0[h], r1[h]);
            }
        }
        y0[i] = pk_f16(r0[0], r0[1]);
        y1[i] = pk_f16(r1[0], r1[1]);
    }
    w0 = make_uint4(y0[0], y0[1], y0[2], y0[3]);
    w1 = make_uint4(y1[0], y1[1], y1[2], y1[3]);
}

// LDS of k_gemm_qk_enc: A stages (unpadded, swizzled), B stages (padded
// rows), and the inverse key-row scales of the scaled pass.  The kernel owns
// the arrays; the tile code takes them as pointers, so that once inlined
// into the kernel every access still names its array (and the compiler can
// tell a DMA target from the tiles being read).
constexpr int kQkAElems = kBM * kBK;
struct QkEncLds {
    uint16_t *a0, *a1, *b0, *b1;
    float* kcs;
};

// One tile of k_gemm_qk_enc.  Unscaled (SC false) it returns true when a key
// row of the tile exceeds fp16's range, having put the inverse row scales in
// L.kcs; scaled, it reads its row scales there.
template <int BENC, bool SC>
__device__ __forceinline__ bool qk_enc_tile(const GemmArgs& g, const QkEncLds& L) {
    constexpr bool kHalf = BENC == kBEncRopeHalf;
    constexpr bool kTab = BENC != kBEncRaw;
    uint16_t* const a0s = L.a0;
    uint16_t* const a1s = L.a1;
    uint16_t* const b0s = L.b0;
    uint16_t* const b1s = L.b1;
    float* const kcs = L.kcs;
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto As = [&](auto S) -> uint16_t* {
        if constexpr (decltype(S)::value == 0) return a0s; else return a1s;
    };
    auto Bs = [&](auto S) -> uint16_t* {
        if constexpr (decltype(S)::value == 0) return b0s; else return b1s;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long per_head = (long)g.tiles_m * g.tiles_n;
    const long total = per_head * g.heads;
    const long t = xcd_tile(blockIdx.x, total);
    if (t >= total) return false;
    const int bh = __builtin_amdgcn_readfirstlane((int)(t / per_head));
    const int rem = (int)(t - (long)bh * per_head);
    const int tm = rem / g.tiles_n, tn = rem - tm * g.tiles_n;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kBM);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kBN);

    const __amdgpu_buffer_rsrc_t ra = gemm_rsrc(g.A + bh * g.sa, (long)g.M * g.lda);
    const __amdgpu_buffer_rsrc_t rb = gemm_rsrc(g.B + bh * g.sb, (long)g.N * g.ldb);
    const __amdgpu_buffer_rsrc_t rt = gemm_rsrc(g.tab, kTab ? (long)g.tab_rows * g.K : 0);
    constexpr uint32_t kOut = 0xfffffff0u;  // an offset past every descriptor's range

    // column of logical chunk c in a K step, and the step's first column
    const int dh = kHalf ? g.K / 2 : 0;
    auto colof = [&](int c) { return kHalf ? (c < 4 ? 8 * c : dh + 8 * (c - 4)) : 8 * c; };
    auto kbase = [&](int kt) { return kHalf ? 32 * kt : 64 * kt; };

    // ---- A: lane l of wave w, instruction u writes row 64 u + 8 w + l / 8 of
    // the tile at physical chunk l % 8, i.e. logical chunk (l % 8) ^ key(row)
    const int ar = 8 * wave + (lane >> 3);
    const int ac = (lane & 7) ^ (lane >> 3) ^ (wave & 1);
    const uint32_t a_vo = 2u * ((uint32_t)ar * (uint32_t)g.lda + (uint32_t)colof(ac));
    auto dma_a = [&](auto S, int kt, auto edge) __attribute__((always_inline)) {
        uint16_t* dst = As(S);
        const int kb = kbase(kt);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t vo = a_vo;
            uint32_t so = 2u * ((uint32_t)(m0 + 64 * u) * (uint32_t)g.lda + (uint32_t)kb);
            if constexpr (decltype(edge)::value) {
                const int row = m0 + 64 * u + ar, col = kb + colof(ac);
                vo = ((row < g.M) & (col < g.K))
                         ? 2u * ((uint32_t)row * (uint32_t)g.lda + (uint32_t)col)
                         : kOut;
                so = 0;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(dst + (64 * u + 8 * wave) * kBK), 16,
                vo, __builtin_amdgcn_readfirstlane(so), 0, 0);
        }
    };

    // ---- B: this thread's chunks u = 0..3 are key row br + 128 (u / 2),
    // logical chunk bc + 4 (u % 2) (a rotate-half pair for u = 2p, 2p + 1)
    const int br = tid >> 2, bc = tid & 3;
    const uint32_t b_vo[2] = {2u * ((uint32_t)br * (uint32_t)g.ldb + (uint32_t)colof(bc)),
                              2u * ((uint32_t)br * (uint32_t)g.ldb + (uint32_t)colof(bc + 4))};
    // table rows are positions with D 16-bit units each; sinusoidal and
    // interleaved chunks sit where K's do, rotate-half takes 32 bytes of
    // (cos, sin) words for the 8 pairs of a chunk pair
    const uint32_t t_vo[2] = {2u * ((uint32_t)br * (uint32_t)g.K + (uint32_t)colof(bc)),
                              2u * ((uint32_t)br * (uint32_t)g.K + (uint32_t)colof(bc + 4))};
    const uint32_t th_vo = 2u * (uint32_t)br * (uint32_t)g.K + 32u * (uint32_t)bc;
    struct Stage {
        uint4 b[4], t[4];
    };
    auto load_b = [&](Stage& r, int kt, auto edge) __attribute__((always_inline)) {
        constexpr bool E = decltype(edge)::value;
        const int kb = kbase(kt);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int rr = 128 * (u >> 1);
            uint32_t vo = b_vo[u & 1];
            uint32_t so = 2u * ((uint32_t)(n0 + rr) * (uint32_t)g.ldb + (uint32_t)kb);
            if constexpr (E) {
                const int row = n0 + rr + br, col = kb + colof(bc + 4 * (u & 1));
                vo = ((row < g.N) & (col < g.K))
                         ? 2u * ((uint32_t)row * (uint32_t)g.ldb + (uint32_t)col)
                         : kOut;
                so = 0;
            }
            r.b[u] = buf_ld16(rb, vo, so);
        }
        if constexpr (kTab) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int rr = 128 * (u >> 1);
                uint32_t vo, so;
                if constexpr (kHalf) {
                    // words of pairs kb + 8 bc + 4 (u % 2) .. + 3
                    vo = th_vo + 16u * (uint32_t)(u & 1);
                    so = 2u * (uint32_t)(n0 + rr) * (uint32_t)g.K + 4u * (uint32_t)kb;
                    if constexpr (E) {
                        vo = (n0 + rr + br < g.N) ? vo + so : kOut;
                        so = 0;
                    }
                } else {
                    vo = t_vo[u & 1];
                    so = 2u * ((uint32_t)(n0 + rr) * (uint32_t)g.K + (uint32_t)kb);
                    if constexpr (E) {
                        const int row = n0 + rr + br, col = kb + colof(bc + 4 * (u & 1));
                        vo = ((row < g.N) & (col < g.K)) ? vo + so : kOut;
                        so = 0;
                    }
                }
                r.t[u] = buf_ld16(rt, vo, so);
            }
        }
    };
    float mx[2] = {0.f, 0.f};  // largest |K~| of key rows br, br + 128 (unscaled pass)
    float ksc[2] = {1.f, 1.f};  // their row scales (scaled pass)
    if constexpr (SC) {
        ksc[0] = 1.0f / kcs[br];
        ksc[1] = 1.0f / kcs[br + 128];
    }
    // each chunk (pair) is stored as soon as it is encoded, which ends its
    // registers' live range before the next one's temporaries
    auto store_b = [&](auto S, Stage& r, auto scaled) __attribute__((always_inline)) {
        constexpr bool kSc = decltype(scaled)::value;
        uint16_t* dst = Bs(S);
        auto put = [&](int u) {
            *reinterpret_cast<uint4*>(&dst[(br + 128 * (u >> 1)) * kLdsRow + 8 * (bc + 4 * (u & 1))]) =
                r.b[u];
        };
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            if constexpr (kHalf) {
                enc_half<kSc>(r.b[2 * p], r.b[2 * p + 1], r.t[2 * p], r.t[2 * p + 1], mx[p], ksc[p]);
            } else {
                r.b[2 * p] = enc_chunk<BENC, kSc>(r.b[2 * p], r.t[2 * p], mx[p], ksc[p]);
                r.b[2 * p + 1] = enc_chunk<BENC, kSc>(r.b[2 * p + 1], r.t[2 * p + 1], mx[p], ksc[p]);
            }
            put(2 * p);
            put(2 * p + 1);
        }
    };

    // ---- wave tile 64 x 128 (waves 4 x 2): 2 x 4 MFMA tiles of 32 x 32
    constexpr int TI = 2, TJ = 4;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
    v16f acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    struct Frag {
        uint4 a[TI], b[TJ];
    };
    const int lrow = lane & 31, lkh = (lane >> 5) * 8;
    // sub-step q's A chunk of this lane: logical 2q + lane / 32, stored at
    // (2q + lane / 32) ^ key(row) = 2q ^ akey (key(row) = key(lrow) here)
    const int akey = ((lrow & 7) ^ ((lrow >> 3) & 1)) ^ (lane >> 5);
    const int a_row = (wm + lrow) * kBK;
    auto read_frag = [&](Frag& f, auto S, int q) __attribute__((always_inline)) {
        const uint16_t* a = As(S);
        const uint16_t* b = Bs(S);
        const int ao = a_row + (((2 * q) ^ akey) << 3);
#pragma unroll
        for (int i = 0; i < TI; ++i) f.a[i] = *reinterpret_cast<const uint4*>(&a[ao + i * 32 * kBK]);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
            f.b[j] = *reinterpret_cast<const uint4*>(&b[(wn + j * 32 + lrow) * kLdsRow + 16 * q + lkh]);
    };
    auto mma = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_32x32x16<true>(f.a[i], f.b[j], acc[i][j]);
    };

    // ---- K loop: fragment reads one sub-step ahead; the next step's Q tile
    // DMA issued in sub-step 0; the next step's K tile encoded and written to
    // LDS in sub-step 2, and the K loads of step kt + 2 issued right after it
    // into the freed register stage (a whole step before they are needed);
    // one barrier before sub-step 3
    const int nk = (g.K + kBK - 1) / kBK;
    constexpr int kReads = TI + TJ;
    Stage st;
    Frag f0, f1;
    auto step = [&](int kt, auto S, auto next, auto next2, auto edge, auto scaled)
                    __attribute__((always_inline)) {
        constexpr int s = decltype(S)::value;
        using S1 = std::integral_constant<int, s ^ 1>;
        constexpr bool N1 = decltype(next)::value, N2 = decltype(next2)::value;
        read_frag(f1, S, 1);
        mma(f0);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (N1) dma_a(S1{}, kt + 1, edge);
        __builtin_amdgcn_sched_barrier(0);
        read_frag(f0, S, 2);
        mma(f1);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        read_frag(f1, S, 3);
        mma(f0);
        if constexpr (N1) store_b(S1{}, st, scaled);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (N2) load_b(st, kt + 2, edge);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        if constexpr (N1) read_frag(f0, S1{}, 0);
        mma(f1);
        if constexpr (N1) sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
    };
    auto kloop = [&](auto edge, auto scaled) __attribute__((always_inline)) {
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        dma_a(I0{}, 0, edge);
        load_b(st, 0, edge);
        store_b(I0{}, st, scaled);
        load_b(st, 1, edge);
        __syncthreads();
        read_frag(f0, I0{}, 0);
        // nk is even (the host's condition for this kernel)
        int kt = 0;
        for (; kt + 2 < nk; kt += 2) {
            step(kt, I0{}, T{}, T{}, edge, scaled);
            step(kt + 1, I1{}, T{}, T{}, edge, scaled);
        }
        step(kt, I0{}, T{}, F{}, edge, scaled);
        step(kt + 1, I1{}, F{}, F{}, edge, scaled);
    };
    if (m0 + kBM <= g.M && n0 + kBN <= g.N && g.K % kBK == 0)
        kloop(std::integral_constant<bool, false>{}, std::integral_constant<bool, SC>{});
    else
        kloop(std::integral_constant<bool, true>{}, std::integral_constant<bool, SC>{});

    // A key row beyond fp16's range (|K~| > 65504) in the unscaled pass: the
    // tile is computed again (the scaled pass) with the row scales
    // k_encode_f16 would use (largest |K~| of the row in [2^14, 2^15)), and
    // that pass's epilogue multiplies the inverse scales back and overwrites
    // this one's output.  The four threads of a key row are one lane quad.
    bool redo = false;
    if constexpr (!SC) {
        float rmax[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const float m = fmaxf(mx[p], dpp<kDppQuadXor1>(mx[p]));
            rmax[p] = fmaxf(m, dpp<kDppQuadXor2>(m));
        }
        redo = __syncthreads_or((rmax[0] > 65504.f) | (rmax[1] > 65504.f));
        if (redo) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                int e = 0;
                if (rmax[p] > 0.f && rmax[p] <= 3.0e38f) e = 14 - ilogbf(rmax[p]);
                e = max(-100, min(100, e));
                if ((tid & 3) == 0) kcs[br + 128 * p] = ldexpf(1.0f, -e);
            }
        }
    }
    nt_exp_epilogue<TI, TJ>(g, acc, reinterpret_cast<float*>(a0s), bh, m0, n0, tn, wm, wn, wave,
                            lane, SC ? kcs : nullptr);
    return redo;
}

// The scaled pass: it only runs when a key row overflows, after the first
// pass's epilogue, so nothing of the first pass is live across it.  (Out of
// line, as a call, it made the kernel 2.6x slower: the callee's saved
// registers gave every lane a 532-byte stack.)
template <int BENC>
__device__ __forceinline__ void qk_enc_scaled_tile(const GemmArgs& g, const QkEncLds& L) {
    __syncthreads();  // every wave is done with the first pass's epilogue (LDS)
    (void)qk_enc_tile<BENC, true>(g, L);
}

template <int BENC>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_qk_enc(GemmArgs g) {
    __shared__ __align__(16) uint16_t a0s[kQkAElems];
    __shared__ __align__(16) uint16_t a1s[kQkAElems];
    __shared__ __align__(16) uint16_t b0s[kTileElems];
    __shared__ __align__(16) uint16_t b1s[kTileElems];
    __shared__ float kcs[kBN];
    const QkEncLds L{a0s, a1s, b0s, b1s, kcs};
    if (qk_enc_tile<BENC, false>(g, L)) qk_enc_scaled_tile<BENC>(g, L);
}

// ---------------------------------------------------------------------------
// QK^T GEMM with both operands loaded straight into LDS (8 waves).
//
// The tiling, fragment order and exp epilogue of k_gemm's NT form, with the
// Q and K tiles both in the swizzled, unpadded layout of k_gemm_qk_enc's Q
// tile (chunk c of row r at c ^ key(r)), filled by buffer -> LDS loads: no
// register stage and no LDS write instructions.  The loads of step kt + 2
// go into stage kt % 2 right after step kt's barrier (every wave is then
// past its last read of it) and are waited for at step kt + 1's barrier.
template <bool F16>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_qk_dma(GemmArgs g) {
    constexpr int kAElems = kBM * kBK;
    __shared__ __align__(16) uint16_t a0s[kAElems];
    __shared__ __align__(16) uint16_t a1s[kAElems];
    __shared__ __align__(16) uint16_t b0s[kAElems];
    __shared__ __align__(16) uint16_t b1s[kAElems];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto As = [&](auto S) -> uint16_t* {
        if constexpr (decltype(S)::value == 0) return a0s; else return a1s;
    };
    auto Bs = [&](auto S) -> uint16_t* {
        if constexpr (decltype(S)::value == 0) return b0s; else return b1s;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long per_head = (long)g.tiles_m * g.tiles_n;
    const long total = per_head * g.heads;
    const long t = xcd_tile(blockIdx.x, total);
    if (t >= total) return;
    const int bh = __builtin_amdgcn_readfirstlane((int)(t / per_head));
    const int rem = (int)(t - (long)bh * per_head);
    const int tm = rem / g.tiles_n, tn = rem - tm * g.tiles_n;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kBM);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kBN);

    const __amdgpu_buffer_rsrc_t ra = gemm_rsrc(g.A + bh * g.sa, (long)g.M * g.lda);
    const __amdgpu_buffer_rsrc_t rb = gemm_rsrc(g.B + bh * g.sb, (long)g.N * g.ldb);
    constexpr uint32_t kOut = 0xfffffff0u;  // an offset past every descriptor's range

    // lane l of wave w, instruction u writes row 64 u + 8 w + l / 8 of a tile
    // at physical chunk l % 8 = logical chunk (l % 8) ^ key(row)
    const int dr = 8 * wave + (lane >> 3);
    const int dc = (lane & 7) ^ (lane >> 3) ^ (wave & 1);
    const uint32_t a_vo = 2u * ((uint32_t)dr * (uint32_t)g.lda + 8u * (uint32_t)dc);
    const uint32_t b_vo = 2u * ((uint32_t)dr * (uint32_t)g.ldb + 8u * (uint32_t)dc);
    auto dma = [&](auto S, int kt, auto edge) __attribute__((always_inline)) {
        uint16_t* da = As(S);
        uint16_t* db = Bs(S);
        const int k0 = kt * kBK;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t va = a_vo, vb = b_vo;
            uint32_t sa = 2u * ((uint32_t)(m0 + 64 * u) * (uint32_t)g.lda + (uint32_t)k0);
            uint32_t sb = 2u * ((uint32_t)(n0 + 64 * u) * (uint32_t)g.ldb + (uint32_t)k0);
            if constexpr (decltype(edge)::value) {
                const int col = k0 + 8 * dc;
                va = ((m0 + 64 * u + dr < g.M) & (col < g.K)) ? va + sa : kOut;
                vb = ((n0 + 64 * u + dr < g.N) & (col < g.K)) ? vb + sb : kOut;
                sa = sb = 0;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(da + (64 * u + 8 * wave) * kBK), 16,
                va, __builtin_amdgcn_readfirstlane(sa), 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void*)(db + (64 * u + 8 * wave) * kBK), 16,
                vb, __builtin_amdgcn_readfirstlane(sb), 0, 0);
        }
    };

    constexpr int TI = 2, TJ = 4;  // waves 4 x 2 of 64 x 128
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
    v16f acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    struct Frag {
        uint4 a[TI], b[TJ];
    };
    const int lrow = lane & 31;
    const int akey = ((lrow & 7) ^ ((lrow >> 3) & 1)) ^ (lane >> 5);
    const int a_row = (wm + lrow) * kBK, b_row = (wn + lrow) * kBK;
    auto read_frag = [&](Frag& f, auto S, int q) __attribute__((always_inline)) {
        const uint16_t* a = As(S);
        const uint16_t* b = Bs(S);
        const int co = ((2 * q) ^ akey) << 3;
#pragma unroll
        for (int i = 0; i < TI; ++i)
            f.a[i] = *reinterpret_cast<const uint4*>(&a[a_row + co + i * 32 * kBK]);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
            f.b[j] = *reinterpret_cast<const uint4*>(&b[b_row + co + j * 32 * kBK]);
    };
    auto mma = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_32x32x16<F16>(f.a[i], f.b[j], acc[i][j]);
    };

    const int nk = (g.K + kBK - 1) / kBK;
    constexpr int kReads = TI + TJ;
    Frag f0, f1;
    auto step = [&](int kt, auto S, auto next, auto next2, auto edge) __attribute__((always_inline)) {
        constexpr int s = decltype(S)::value;
        using S1 = std::integral_constant<int, s ^ 1>;
        constexpr bool N1 = decltype(next)::value, N2 = decltype(next2)::value;
        read_frag(f1, S, 1);
        mma(f0);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        read_frag(f0, S, 2);
        mma(f1);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        read_frag(f1, S, 3);
        mma(f0);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        // this wave's loads of step kt + 1 (issued one step earlier, in the
        // previous loop iteration for every other step, where the compiler
        // does not carry them to the barrier's wait) are complete; then the
        // barrier makes every wave's complete
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if constexpr (N2) dma(S, kt + 2, edge);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (N1) read_frag(f0, S1{}, 0);
        mma(f1);
        if constexpr (N1) sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
    };
    auto kloop = [&](auto edge) __attribute__((always_inline)) {
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        dma(I0{}, 0, edge);
        dma(I1{}, 1, edge);
        __syncthreads();
        read_frag(f0, I0{}, 0);
        // nk is even (the host's condition for this kernel)
        int kt = 0;
        for (; kt + 2 < nk; kt += 2) {
            step(kt, I0{}, T{}, T{}, edge);
            step(kt + 1, I1{}, T{}, T{}, edge);
        }
        step(kt, I0{}, T{}, F{}, edge);
        step(kt + 1, I1{}, F{}, F{}, edge);
    };
    if (m0 + kBM <= g.M && n0 + kBN <= g.N && g.K % kBK == 0)
        kloop(std::integral_constant<bool, false>{});
    else
        kloop(std::integral_constant<bool, true>{});
    nt_exp_epilogue<TI, TJ>(g, acc, reinterpret_cast<float*>(a0s), bh, m0, n0, tn, wm, wn, wave,
                            lane);
}

// ---------------------------------------------------------------------------
// PV GEMM with V loaded straight into LDS (8 waves, rows of at most
// kFacTiles key tiles, an even number of 64-key steps).
//
// O = P V as in k_gemm's NN form: the E chunks (fp16) go through the register
// stage and are scaled by their row's softmax factor into bf16 P on their
// way to LDS (factors computed by the workgroup into an LDS table), while the
// V tile ([64 keys][256 columns], the transposing-read layout of nn_lds_off)
// is filled by buffer -> LDS loads.  Wave instruction u of wave w writes key
// rows 2 (w + 8u) and + 1 (1 KiB); lane l takes row + l / 32, physical
// 16-byte slot l % 32 of that row, i.e. logical columns 16 ((l % 32) / 2 ^
// swz(row)) + 8 (l % 2).  V's loads of step kt + 2 go into stage kt % 2
// right after step kt's barrier and are waited for at step kt + 1's barrier.
template <bool ALL_INTERIOR>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_pv_dma(GemmArgs g) {
    constexpr int kBElems = kBK * kBN;
    __shared__ __align__(16) uint16_t a0s[kTileElems];
    __shared__ __align__(16) uint16_t a1s[kTileElems];
    __shared__ __align__(16) uint16_t b0s[kBElems];
    __shared__ __align__(16) uint16_t b1s[kBElems];
    __shared__ float fac[kBM * kFacTiles];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto As = [&](auto S) -> uint16_t* {
        if constexpr (decltype(S)::value == 0) return a0s; else return a1s;
    };
    auto Bs = [&](auto S) -> uint16_t* {
        if constexpr (decltype(S)::value == 0) return b0s; else return b1s;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long per_head = (long)g.tiles_m * g.tiles_n;
    const long total = per_head * g.heads;
    // Persistent: workgroup w takes the virtual ids w, w + G, ... (G =
    // gridDim.x, a multiple of 8, so every id of w maps to w's XCD); each
    // tile's first loads are issued before the previous tile's output is
    // stored.
    const long vend = (total + 7) / 8 * 8;
    int bh = 0, m0 = 0, n0 = 0;
    bool interior = true;
    __amdgpu_buffer_rsrc_t ra, rb;
    auto set_tile = [&](long t) __attribute__((always_inline)) {
        bh = __builtin_amdgcn_readfirstlane((int)(t / per_head));
        const int rem = (int)(t - (long)bh * per_head);
        // row panels fastest: the few tiles of one V panel run together
        const int tn = rem / g.tiles_m, tm = rem - tn * g.tiles_m;
        m0 = __builtin_amdgcn_readfirstlane(tm * kBM);
        n0 = __builtin_amdgcn_readfirstlane(tn * kBN);
        interior = ALL_INTERIOR || (m0 + kBM <= g.M && n0 + kBN <= g.N);
        ra = gemm_rsrc(g.A + bh * g.sa, (long)g.M * g.lda);
        rb = gemm_rsrc(g.B + bh * g.sb, (long)g.K * g.ldb);
    };
    long vt = blockIdx.x;
    {
        const long t = xcd_tile(vt, total);
        if (t >= total) return;
        set_tile(t);
    }
    constexpr uint32_t kOut = 0xfffffff0u;  // an offset past every descriptor's range

    // ---- E chunks: thread's chunk u is row tid / 8 + 64 u, keys 8 (tid % 8) ..
    constexpr int kChunks = 4;
    const int er = tid / kChunkPerRow, ek = (tid % kChunkPerRow) * 8;
    const uint32_t a_vo = 2u * ((uint32_t)er * (uint32_t)g.lda + (uint32_t)ek);
    struct Stage {
        uint4 a[kChunks];
    };
    auto load_a = [&](Stage& r, int kt, auto edge) __attribute__((always_inline)) {
        const int k0 = kt * kBK;
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            uint32_t vo = a_vo;
            uint32_t so = 2u * ((uint32_t)(m0 + 64 * u) * (uint32_t)g.lda + (uint32_t)k0);
            if constexpr (decltype(edge)::value) {
                vo = (m0 + 64 * u + er < g.M) ? vo + so : kOut;
                so = 0;
            }
            r.a[u] = buf_ld16(ra, vo, so);
        }
    };
    auto store_a = [&](auto S, const Stage& r, int kt) __attribute__((always_inline)) {
        uint16_t* dst = As(S);
        const int ft = (kt * kBK + ek) >> 8;  // the chunk's 256-key tile
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int row = er + 64 * u;
            *reinterpret_cast<uint4*>(&dst[row * kLdsRow + ek]) =
                scale_f16x8_to_bf16(r.a[u], fac[row * kFacTiles + ft]);
        }
    };

    // ---- V: DMA into [64 keys][256 columns]
    const int vrow = lane >> 5;  // + 2 (w + 8u)
    const int vswz = (0x7520 >> (4 * ((2 * (wave & 1) + vrow) & 3))) & 0xf;  // {0,2,5,7}[row % 4]
    const int vcol = ((((lane & 31) >> 1) ^ vswz) << 4) + 8 * (lane & 1);
    const uint32_t b_vo = 2u * ((uint32_t)vrow * (uint32_t)g.ldb + (uint32_t)vcol);
    auto dma_b = [&](auto S, int kt, auto edge) __attribute__((always_inline)) {
        uint16_t* dst = Bs(S);
        const int k0 = kt * kBK;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r0 = 2 * (wave + 8 * u);
            uint32_t vo = b_vo;
            uint32_t so = 2u * ((uint32_t)(k0 + r0) * (uint32_t)g.ldb + (uint32_t)n0);
            if constexpr (decltype(edge)::value) {
                vo = (n0 + vcol < g.N) ? vo + so : kOut;
                so = 0;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void*)(dst + r0 * kBN), 16, vo,
                __builtin_amdgcn_readfirstlane(so), 0, 0);
        }
    };

    // ---- wave tile 128 x 64 (waves 2 x 4): 4 x 2 MFMA tiles, transposed
    // product (acc rows are output columns)
    constexpr int TI = 4, TJ = 2;
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    v16f acc[TI][TJ];
    struct Frag {
        uint4 a[TI], b[TJ];
    };
    const int lrow = lane & 31, lkh = (lane >> 5) * 8;
    auto read_frag = [&](Frag& f, auto S, int q) __attribute__((always_inline)) {
        const uint16_t* a = As(S);
        const uint16_t* b = Bs(S);
        const int ks = 16 * q;
#pragma unroll
        for (int i = 0; i < TI; ++i)
            f.a[i] = *reinterpret_cast<const uint4*>(&a[(wm + i * 32 + lrow) * kLdsRow + ks + lkh]);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int kr = ks + 8 * (lane >> 5) + ((lane & 15) >> 2);
            const int nc = wn + j * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
            const v4i16 lo = ds_read_tr16(&b[nn_lds_off(kr, nc)]);
            const v4i16 hi = ds_read_tr16(&b[nn_lds_off(kr + 4, nc)]);
            const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
            f.b[j] = make_uint4(l2.x, l2.y, h2.x, h2.y);
        }
    };
    auto mma = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_32x32x16<false>(f.b[j], f.a[i], acc[i][j]);
    };

    const int nk = (g.K + kBK - 1) / kBK;
    constexpr int kReads = TI + 2 * TJ;
    Stage st;
    Frag f0, f1;
    float mt[kFacTiles], lt[kFacTiles];  // the tile statistics of row m0 + tid
    auto load_stats = [&]() __attribute__((always_inline)) {
        if (tid < kBM) {
            const int row = m0 + tid;
            const long base = ((long)bh * g.M + row) * g.gt;
#pragma unroll
            for (int t2 = 0; t2 < kFacTiles; ++t2) {
                const bool on = row < g.M && t2 < g.gt;
                mt[t2] = on ? g.st_m[base + t2] : -INFINITY;
                lt[t2] = on ? g.st_l[base + t2] : 0.f;
            }
        }
    };
    auto step = [&](int kt, auto S, auto next, auto next2, auto edge) __attribute__((always_inline)) {
        constexpr int s = decltype(S)::value;
        using S1 = std::integral_constant<int, s ^ 1>;
        constexpr bool N1 = decltype(next)::value, N2 = decltype(next2)::value;
        read_frag(f1, S, 1);
        mma(f0);
        if constexpr (N1) store_a(S1{}, st, kt + 1);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (N2) load_a(st, kt + 2, edge);
        read_frag(f0, S, 2);
        mma(f1);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        read_frag(f1, S, 3);
        mma(f0);
        sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        // V of step kt + 1 (issued after the previous step's barrier, before
        // this step's E loads) is in; then the barrier makes every wave's so
        if constexpr (N2)
            __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4): this step's E loads may fly
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if constexpr (N2) dma_b(S, kt + 2, edge);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (N1) read_frag(f0, S1{}, 0);
        mma(f1);
        if constexpr (N1) sched_mfma_reads<kReads>();
        __builtin_amdgcn_sched_barrier(0);
    };
    // a tile's first loads: V of steps 0 and 1, E of step 0 and (persistent
    // form) the rows' tile statistics: one memory round trip for all of them
    auto issue = [&](auto edge) __attribute__((always_inline)) {
        dma_b(I0{}, 0, edge);
        dma_b(I1{}, 1, edge);
        load_a(st, 0, edge);
        if constexpr (ALL_INTERIOR) load_stats();
    };
    // the rows' softmax factors (as in k_gemm's NN form) into the LDS table,
    // then E of step 0 to LDS.  vmcnt(pending) waits only for this tile's
    // loads (the previous tile's kOutStores output stores were issued after
    // them);
    // the compiler's own waits for the statistics registers at the loop head
    // (in the first four waves) still cover every outstanding operation.
    auto finish = [&](auto edge, auto pending) __attribute__((always_inline)) {
        if constexpr (!ALL_INTERIOR) load_stats();
        if (tid < kBM) {
            float m = -INFINITY;
#pragma unroll
            for (int t2 = 0; t2 < kFacTiles; ++t2) m = fmaxf(m, mt[t2]);
            float l = 0.f;
#pragma unroll
            for (int t2 = 0; t2 < kFacTiles; ++t2)
                if (t2 < g.gt) l += lt[t2] * __expf(mt[t2] - m);
            const float inv = 1.0f / l;
#pragma unroll
            for (int t2 = 0; t2 < kFacTiles; ++t2)
                fac[tid * kFacTiles + t2] =
                    (m == -INFINITY || t2 >= g.gt) ? 0.f : __expf(mt[t2] - m) * inv;
        }
        if constexpr (decltype(pending)::value == 16)
            __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16)
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();  // the factor table, V of steps 0 and 1
        store_a(I0{}, st, 0);
        load_a(st, 1, edge);
        __syncthreads();
        read_frag(f0, I0{}, 0);
    };
    auto kloop = [&](auto edge) __attribute__((always_inline)) {
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        // nk is even (the host's condition for this kernel)
        int kt = 0;
        for (; kt + 2 < nk; kt += 2) {
            step(kt, I0{}, T{}, T{}, edge);
            step(kt + 1, I1{}, T{}, T{}, edge);
        }
        step(kt, I0{}, T{}, F{}, edge);
        step(kt + 1, I1{}, F{}, F{}, edge);
    };
    using EdgeF = std::integral_constant<bool, false>;
    using EdgeT = std::integral_constant<bool, true>;
    using P0 = std::integral_constant<int, 0>;
    constexpr int kOutStores = 16;  // output stores per thread and tile (store_out_lds)
    using P16 = std::integral_constant<int, kOutStores>;

    // lane: output row m0 + wm + 32 i + lane % 32, columns n0 + wn + 32 j +
    // 8 (r / 4) + 4 (lane / 32) + r % 4: four consecutive bf16 per group of r
    // (converted two at a time by the hardware, round to nearest even).
    // Interior tiles issue exactly TI * TJ * 4 = 32 stores.
    auto pack4 = [&](const v16f& a, int rg) __attribute__((always_inline)) {
        const bf16x2_t lo = {(__bf16)a[4 * rg], (__bf16)a[4 * rg + 1]};
        const bf16x2_t hi = {(__bf16)a[4 * rg + 2], (__bf16)a[4 * rg + 3]};
        return u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
    };
    static_assert(TI * TJ * 4 == 32, "interior output stores per lane");
    auto store_out = [&](int obh, int om0, int on0, bool oint) __attribute__((always_inline)) {
        uint16_t* C = static_cast<uint16_t*>(g.C) + obh * g.sc;
        if (oint) {
            // buffer stores: the lane's row offset in a register, the column
            // group's offset in a scalar register
            const __amdgpu_buffer_rsrc_t rc = gemm_rsrc(C, (long)g.M * g.ldc);
            const uint32_t ldc = (uint32_t)g.ldc;
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const uint32_t vo = 2u * ((uint32_t)(om0 + wm + i * 32 + (lane & 31)) * ldc +
                                          (uint32_t)(on0 + wn + 4 * (lane >> 5)));
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int rg = 0; rg < 4; ++rg)
                        __builtin_amdgcn_raw_buffer_store_b64(
                            pack4(acc[i][j], rg), rc, (int)vo,
                            (int)__builtin_amdgcn_readfirstlane(2u * (uint32_t)(j * 32 + 8 * rg)),
                            0);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int row = om0 + wm + i * 32 + (lane & 31);
            if (row >= g.M) continue;
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int rg = 0; rg < 4; ++rg) {
                    const int col = on0 + wn + j * 32 + 8 * rg + 4 * (lane >> 5);
                    if (col >= g.N) continue;
                    *reinterpret_cast<u32x2*>(C + (long)row * g.ldc + col) = pack4(acc[i][j], rg);
                }
        }
    };

    // Persistent form: the interior output through LDS.  Between the K loop
    // and the next tile's first E chunk the A stages are free (the next
    // tile's first V loads go to the B stages): two halves of 128 rows, each
    // written by its four waves as bf16 rows of 256 elements padded to
    // kOutRow (rows 0-63 of the half in a0s, 64-127 in a1s; every address is
    // a per-lane base plus an immediate offset), then read back and stored
    // 16 contiguous bytes per thread: a wave store
    // writes two whole 512-byte output rows, instead of 32 row pieces of 16
    // bytes 8 KiB or more apart, which the store path handles far more
    // slowly.  Each thread issues kOutStores stores.
    constexpr int kOutRow = kBN + 8;  // elements: 528-byte rows, 4 banks apart
    static_assert(64 * kOutRow <= kTileElems, "a half-tile's 64 rows fit one A stage");
    auto store_out_lds = [&](int obh, int om0, int on0) __attribute__((always_inline)) {
        uint16_t* C = static_cast<uint16_t*>(g.C) + obh * g.sc;
        const __amdgpu_buffer_rsrc_t rc = gemm_rsrc(C, (long)g.M * g.ldc);
        const uint32_t ldc = (uint32_t)g.ldc;
        const int rr = tid >> 5, ch = tid & 31;  // read: rows rr + 16 k, chunk ch
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if ((wave >> 2) == h) {
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    uint16_t* dst = i < 2 ? a0s : a1s;
                    const int r = (i & 1) * 32 + (lane & 31);  // row in the stage
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
#pragma unroll
                        for (int rg = 0; rg < 4; ++rg)
                            *reinterpret_cast<u32x2*>(
                                &dst[r * kOutRow + wn + j * 32 + 8 * rg + 4 * (lane >> 5)]) =
                                pack4(acc[i][j], rg);
                }
            }
            __syncthreads();
            // four reads in flight at a time (the other half's accumulators,
            // and the next tile's first loads, are live here)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int r = rr + 16 * (k & 3);  // row in the stage
                const uint16_t* src = (k < 4 ? a0s : a1s) + r * kOutRow + 8 * ch;
                const u32x4 v = *reinterpret_cast<const u32x4*>(src);
                const uint32_t vo =
                    2u * ((uint32_t)(om0 + 128 * h + 64 * (k >> 2) + r) * ldc +
                          (uint32_t)(on0 + 8 * ch));
                __builtin_amdgcn_raw_buffer_store_b128(v, rc, (int)vo, 0, 0);
                if ((k & 3) == 3) __builtin_amdgcn_sched_barrier(0);
            }
            // the second half overwrites the stages; after it, the next
            // tile's first E chunk does, behind finish()'s barrier
            if (h == 0) __syncthreads();
        }
    };

    auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    };
    if constexpr (!ALL_INTERIOR) {
        // ragged shapes: one tile per workgroup (the grid covers them all)
        auto body = [&](auto edge) __attribute__((always_inline)) {
            issue(edge);
            finish(edge, P0{});
            zero_acc();
            kloop(edge);
        };
        if (interior)
            body(EdgeF{});
        else
            body(EdgeT{});
        store_out(bh, m0, n0, interior);
    } else {
        issue(EdgeF{});
        // vmcnt(kOutStores) covers this tile's loads once the previous tile's
        // output stores were issued after them
        bool first = true;
        for (;;) {
            if (first)
                finish(EdgeF{}, P0{});
            else
                finish(EdgeF{}, P16{});
            zero_acc();
            kloop(EdgeF{});
            const int obh = bh, om0 = m0, on0 = n0;
            vt += gridDim.x;
            const long tn = vt < vend ? xcd_tile(vt, total) : total;
            const bool more = tn < total;
            __syncthreads();  // every wave is done with the stages and the factor table
            if (more) {
                set_tile(tn);
                issue(EdgeF{});
            }
            store_out_lds(obh, om0, on0);
            if (!more) break;
            first = false;
        }
    }
}

// Encoded rows as fp16 with a power-of-two row scale: pass 1 finds the
// largest magnitude m of the encoded row, pass 2 (re-reading the row, an L2
// hit) writes fp16(x * 2^k) with m * 2^k in [2^14, 2^15) and stores
// inv[row] = 2^-k.  One workgroup per row; positions are row % seq_len.
template <int PEK>
__global__ __launch_bounds__(256) void k_encode_f16(const uint16_t* __restrict__ in,
                                                    uint16_t* __restrict__ out,
                                                    float* __restrict__ inv, long n_rows,
                                                    int seq_len, int D, PeSide pe) {
    __shared__ float red[4];
    const int tid = threadIdx.x;
    for (long row = blockIdx.x; row < n_rows; row += gridDim.x) {
        const int pos = (int)(row % seq_len);
        const uint16_t* xr = in + row * D;
        float m = 0.f;
        for (int d = tid * 4; d < D; d += 1024) {
            const float4 v = load_row4_pe<uint16_t, PEK>(xr, pos, d, D, pe, true);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        m = wave_max(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();  // red is reused by the next row
        int k = 0;
        if (m > 0.f && m <= 3.0e38f) k = 14 - ilogbf(m);
        k = max(-100, min(100, k));
        const float up = ldexpf(1.0f, k);
        if (tid == 0) inv[row] = ldexpf(1.0f, -k);
        uint16_t* yr = out + row * D;
        for (int d = tid * 4; d < D; d += 1024) {
            const float4 v = load_row4_pe<uint16_t, PEK>(xr, pos, d, D, pe, true);
            const _Float16 h[4] = {(_Float16)(v.x * up), (_Float16)(v.y * up),
                                   (_Float16)(v.z * up), (_Float16)(v.w * up)};
            uint2 w;
            w.x = (uint32_t)__builtin_bit_cast(uint16_t, h[0]) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16);
            w.y = (uint32_t)__builtin_bit_cast(uint16_t, h[2]) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16);
            *reinterpret_cast<uint2*>(yr + d) = w;
        }
    }
}

// Per row of the scores: m = max_t m_t over its 256-key tiles, l = sum_t
// l_t exp(m_t - m) (the tiles' E sums brought to the common maximum), and
// the factor g_t = exp(m_t - m) / l that turns tile t's E into the softmax
// probabilities.  A row with no valid key (m = -inf) gets g = 0.
__global__ __launch_bounds__(256) void k_rowscale(const float* __restrict__ st_m,
                                                  const float* __restrict__ st_l,
                                                  float* __restrict__ ga, long rows, int T) {
    const long row = (long)blockIdx.x * 256 + threadIdx.x;
    if (row >= rows) return;
    const float* mr = st_m + row * T;
    const float* lr = st_l + row * T;
    float* gr = ga + row * T;
    float m = -INFINITY;
    for (int t = 0; t < T; ++t) m = fmaxf(m, mr[t]);
    if (m == -INFINITY) {
        for (int t = 0; t < T; ++t) gr[t] = 0.f;
        return;
    }
    float l = 0.f;
    for (int t = 0; t < T; ++t) l += lr[t] * __expf(mr[t] - m);
    const float inv = 1.0f / l;
    for (int t = 0; t < T; ++t) gr[t] = __expf(mr[t] - m) * inv;
}

// Register-resident encoder.  The row is split into 8-element units (for
// rotate-half, unit u < r/16 is paired with its partner unit u + r/16 so both
// halves of every rotation are in one thread) and each thread keeps its units
// in registers, so a row is read once: 16-byte loads of x, one block-wide
// max, then scaled fp16 16-byte stores.
//
// Rows at the same position (row % seq_len) share their compact table row, so
// a workgroup takes one position and up to kEncGroup rows at that position
// (stride seq_len, i.e. the same token of consecutive heads): each thread
// loads the cos/sin (or sin/cos) values of its units once and applies them to
// every row of the group, which divides the table traffic (as large as the
// data itself at fp32) by the group size.  kEncRows rows are in flight at a
// time.  Workgroup b takes position b % seq_len of group b / seq_len, so
// concurrently running workgroups stream neighbouring rows of one head.
constexpr int kEncThreads = 256;
constexpr int kEncMaxUnits = 4;  // units per thread: D <= 4 * 256 * 8 = 8192
constexpr int kEncGroup = 8;     // rows (heads) per workgroup sharing one position
constexpr int kEncRows = 2;      // rows in flight per thread

__device__ __forceinline__ void unpack_bf16x8(const uint4& w, float* v) {
    const uint32_t x[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(x[i] << 16);
        v[2 * i + 1] = __uint_as_float(x[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ uint4 pack_f16x8(const float* v, float up) {
    uint32_t x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        x[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v[2 * i] * up)) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v[2 * i + 1] * up)) << 16);
    return make_uint4(x[0], x[1], x[2], x[3]);
}

__device__ __forceinline__ void ld8f(const float* p, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void ld4f(const float* p, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
}

// S = 2 (rows of at most 128 units, U = 1): the two halves of the workgroup
// take two rows of the group at once, so no thread idles.
template <int PEK, int U, int S = 1>
__global__ __launch_bounds__(kEncThreads) void k_encode_f16_regs(const uint16_t* __restrict__ in,
                                                                 uint16_t* __restrict__ out,
                                                                 float* __restrict__ inv,
                                                                 long n_rows, int seq_len, int D,
                                                                 PeSide pe) {
    static_assert(S == 1 || (S == 2 && U == 1), "split rows: one unit per thread");
    __shared__ float red[2][kEncRows][kEncThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = S == 2 ? (int)threadIdx.x >> 7 : 0;  // this half's row of a pair
    const int tid = S == 2 ? (int)threadIdx.x & 127 : (int)threadIdx.x;  // job index
    const int pos = (int)(blockIdx.x % (unsigned)seq_len);
    const long h0 = (long)(blockIdx.x / (unsigned)seq_len) * kEncGroup;  // first row group member
    const long nh = n_rows / seq_len;
    const int nrow = (int)(nh - h0 < kEncGroup ? nh - h0 : kEncGroup);
    const bool half_pairs = PEK == kPeRopeHalf && pe.on;
    const int hu = half_pairs ? pe.rotary / 16 : 0;  // paired units (rotate-half)
    const int nunits = D / 8 - hu;                    // units handled as the "first" of a job

    // this thread's units and their table values (loaded once per workgroup)
    int d0[U], d1[U];
    bool enc[U];
    float ta[U][8], tb[U][8];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const int job = tid + k * kEncThreads;
        d0[k] = d1[k] = -1;
        enc[k] = false;
        if (job >= nunits) continue;
        // job -> first unit; rotate-half pairs jobs < hu with unit job + hu
        const int u0 = (half_pairs && job >= hu) ? job + hu : job;
        d0[k] = u0 * 8;
        if constexpr (PEK == kPeRopeHalf) {
            if (half_pairs && job < hu) {
                d1[k] = d0[k] + pe.rotary / 2;
                enc[k] = true;
                ld8f(pe.a + (size_t)pos * pe.ld + d0[k], ta[k]);
                ld8f(pe.b + (size_t)pos * pe.ld + d0[k], tb[k]);
            }
        } else if constexpr (PEK == kPeRopeInterleaved) {
            if (pe.on && d0[k] < pe.rotary) {
                enc[k] = true;
                ld4f(pe.a + (size_t)pos * pe.ld + d0[k] / 2, ta[k]);
                ld4f(pe.b + (size_t)pos * pe.ld + d0[k] / 2, tb[k]);
            }
        } else if constexpr (PEK == kPeSinusoidal) {
            if (pe.on) {
                enc[k] = true;
                ld4f(pe.a + (size_t)pos * pe.ld + d0[k] / 2, ta[k]);
                ld4f(pe.b + (size_t)pos * pe.ld + d0[k] / 2, tb[k]);
            }
        }
    }

    // row of slot rr in the batch starting at i
    auto rix = [&](int i, int rr) { return i + S * rr + sub; };
    for (int i = 0; i < nrow; i += kEncRows * S) {
        const int par = (i / (kEncRows * S)) & 1;  // red[] parity: one barrier per batch
        float v[kEncRows][U][2][8];
        // all loads of the batch first
#pragma unroll
        for (int rr = 0; rr < kEncRows; ++rr) {
            if (rix(i, rr) >= nrow) continue;
            const uint16_t* xr = in + ((h0 + rix(i, rr)) * seq_len + pos) * D;
#pragma unroll
            for (int k = 0; k < U; ++k) {
                if (d0[k] >= 0) unpack_bf16x8(*reinterpret_cast<const uint4*>(xr + d0[k]), v[rr][k][0]);
                if (d1[k] >= 0) unpack_bf16x8(*reinterpret_cast<const uint4*>(xr + d1[k]), v[rr][k][1]);
            }
        }
        float m[kEncRows];
#pragma unroll
        for (int rr = 0; rr < kEncRows; ++rr) {
            m[rr] = 0.f;
            if (rix(i, rr) >= nrow) continue;
#pragma unroll
            for (int k = 0; k < U; ++k) {
                if (d0[k] < 0) continue;
                float(&x)[2][8] = v[rr][k];
                if (enc[k]) {
                    if constexpr (PEK == kPeRopeHalf) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const float x0 = x[0][e], x1 = x[1][e];
                            x[0][e] = rot_first(x0, x1, ta[k][e], tb[k][e]);
                            x[1][e] = rot_second(x0, x1, ta[k][e], tb[k][e]);
                        }
                    } else if constexpr (PEK == kPeRopeInterleaved) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x0 = x[0][2 * e], x1 = x[0][2 * e + 1];
                            x[0][2 * e] = rot_first(x0, x1, ta[k][e], tb[k][e]);
                            x[0][2 * e + 1] = rot_second(x0, x1, ta[k][e], tb[k][e]);
                        }
                    } else if constexpr (PEK == kPeSinusoidal) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            x[0][2 * e] = x[0][2 * e] + ta[k][e];
                            x[0][2 * e + 1] = x[0][2 * e + 1] + tb[k][e];
                        }
                    }
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) m[rr] = fmaxf(m[rr], fabsf(x[0][e]));
                if (d1[k] >= 0)
#pragma unroll
                    for (int e = 0; e < 8; ++e) m[rr] = fmaxf(m[rr], fabsf(x[1][e]));
            }
        }
#pragma unroll
        for (int rr = 0; rr < kEncRows; ++rr) {
            m[rr] = wave_max(m[rr]);
            if (lane == 0) red[par][rr][wave] = m[rr];
        }
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < kEncRows; ++rr) {
            if (rix(i, rr) >= nrow) continue;
            // the row's waves: all four, or this half's two
            const float mr =
                S == 2 ? fmaxf(red[par][rr][2 * sub], red[par][rr][2 * sub + 1])
                       : fmaxf(fmaxf(red[par][rr][0], red[par][rr][1]),
                               fmaxf(red[par][rr][2], red[par][rr][3]));
            int kexp = 0;
            if (mr > 0.f && mr <= 3.0e38f) kexp = 14 - ilogbf(mr);
            kexp = max(-100, min(100, kexp));
            const float up = ldexpf(1.0f, kexp);
            const long row = (h0 + rix(i, rr)) * seq_len + pos;
            if (tid == 0) inv[row] = ldexpf(1.0f, -kexp);
            uint16_t* yr = out + row * D;
#pragma unroll
            for (int k = 0; k < U; ++k) {
                if (d0[k] >= 0) *reinterpret_cast<uint4*>(yr + d0[k]) = pack_f16x8(v[rr][k][0], up);
                if (d1[k] >= 0) *reinterpret_cast<uint4*>(yr + d1[k]) = pack_f16x8(v[rr][k][1], up);
            }
        }
    }
}

// Compute units of the current device (cached per device): the persistent
// PV GEMM runs one workgroup per CU.
int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace

hipError_t launch_gemm_qk(int f16, const uint16_t* Q, const uint16_t* K, const float* qinv,
                          const float* kinv, uint16_t* E, int ldE, float* st_m, float* st_l,
                          int BH, int Lq, int Lk, int D, float scale, hipStream_t st) {
    GemmArgs g{};
    g.A = Q;
    g.B = K;
    g.C = E;
    g.st_m = st_m;
    g.st_l = st_l;
    g.rs = qinv;
    g.cs = kinv;
    g.M = Lq;
    g.N = Lk;
    g.K = D;
    g.lda = D;
    g.ldb = D;
    g.ldc = ldE;
    g.sa = (long)Lq * D;
    g.sb = (long)Lk * D;
    g.sc = (long)Lq * ldE;
    g.tiles_m = (Lq + kBM - 1) / kBM;
    g.tiles_n = (Lk + kBN - 1) / kBN;
    g.heads = BH;
    g.scale = scale;
    const long total = (long)g.tiles_m * g.tiles_n * BH;
    const long grid = (total + 7) / 8 * 8;
    // an even number of 64-deep K steps: both operands straight into LDS
    // (config 4's QK^T: 611 us against 635 us with the register stage)
    if (D % 128 == 0) {
        if (f16)
            hipLaunchKernelGGL((k_gemm_qk_dma<true>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                               st, g);
        else
            hipLaunchKernelGGL((k_gemm_qk_dma<false>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                               st, g);
        return hipGetLastError();
    }
    if (f16)
        hipLaunchKernelGGL((k_gemm<true, false, kOutExpF16>), dim3((unsigned)grid),
                           dim3(kGemmThreads), 0, st, g);
    else
        hipLaunchKernelGGL((k_gemm<false, false, kOutExpF16>), dim3((unsigned)grid),
                           dim3(kGemmThreads), 0, st, g);
    return hipGetLastError();
}

hipError_t launch_gemm_qk_enc(int benc, const uint16_t* Qe, const uint16_t* K, const float* qinv,
                              const uint16_t* tab, int tab_rows, uint16_t* E, int ldE,
                              float* st_m, float* st_l, int BH, int Lq, int Lk, int D,
                              float scale, hipStream_t st) {
    // an even number of 64-deep K steps (the kernel runs them in pairs)
    if ((benc != kBEncRaw && (tab == nullptr || tab_rows < Lk)) || D % 128 != 0)
        return hipErrorInvalidValue;
    GemmArgs g{};
    g.A = Qe;
    g.B = K;
    g.C = E;
    g.st_m = st_m;
    g.st_l = st_l;
    g.rs = qinv;
    g.cs = nullptr;
    g.M = Lq;
    g.N = Lk;
    g.K = D;
    g.lda = D;
    g.ldb = D;
    g.ldc = ldE;
    g.sa = (long)Lq * D;
    g.sb = (long)Lk * D;
    g.sc = (long)Lq * ldE;
    g.tiles_m = (Lq + kBM - 1) / kBM;
    g.tiles_n = (Lk + kBN - 1) / kBN;
    g.heads = BH;
    g.scale = scale;
    g.tab = tab;
    g.tab_rows = tab_rows;
    const long total = (long)g.tiles_m * g.tiles_n * BH;
    const dim3 grid((unsigned)((total + 7) / 8 * 8)), block(kGemmThreads);
    switch (benc) {
        case kBEncRaw:
            hipLaunchKernelGGL((k_gemm_qk_enc<kBEncRaw>), grid, block, 0, st, g);
            break;
        case kBEncSin:
            hipLaunchKernelGGL((k_gemm_qk_enc<kBEncSin>), grid, block, 0, st, g);
            break;
        case kBEncRope:
            hipLaunchKernelGGL((k_gemm_qk_enc<kBEncRope>), grid, block, 0, st, g);
            break;
        case kBEncRopeHalf:
            hipLaunchKernelGGL((k_gemm_qk_enc<kBEncRopeHalf>), grid, block, 0, st, g);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int PEK>
static void launch_encode_regs(int jobs, const uint16_t* in, uint16_t* out, float* inv,
                               long n_rows, int seq_len, int D, const PeSide& pe, hipStream_t st) {
    const int units = (jobs + kEncThreads - 1) / kEncThreads;
    const long groups = (n_rows / seq_len + kEncGroup - 1) / kEncGroup;
    const dim3 grid((unsigned)(groups * seq_len)), block(kEncThreads);
    if (jobs <= kEncThreads / 2)
        hipLaunchKernelGGL((k_encode_f16_regs<PEK, 1, 2>), grid, block, 0, st, in, out, inv,
                           n_rows, seq_len, D, pe);
    else if (units <= 1)
        hipLaunchKernelGGL((k_encode_f16_regs<PEK, 1>), grid, block, 0, st, in, out, inv, n_rows,
                           seq_len, D, pe);
    else if (units == 2)
        hipLaunchKernelGGL((k_encode_f16_regs<PEK, 2>), grid, block, 0, st, in, out, inv, n_rows,
                           seq_len, D, pe);
    else
        hipLaunchKernelGGL((k_encode_f16_regs<PEK, 4>), grid, block, 0, st, in, out, inv, n_rows,
                           seq_len, D, pe);
}

hipError_t launch_encode_f16(int pek, const uint16_t* in, uint16_t* out, float* inv, long n_rows,
                             int seq_len, int D, const PeSide& pe, hipStream_t st) {
    const long grid = n_rows < 65536 ? n_rows : 65536;
    // register-resident form: D % 8 == 0, D <= 8192, the library's compact
    // tables, a rotary width that keeps 8-element units whole, and rows that
    // are whole sequences (n_rows a multiple of seq_len)
    const bool rope = pek == kPeRopeInterleaved || pek == kPeRopeHalf;
    const bool fast = D % 8 == 0 && D <= kEncMaxUnits * kEncThreads * 8 && seq_len > 0 &&
                      n_rows % seq_len == 0 &&
                      (pek == kPeNone || !pe.on || (pe.dup == 0 && pe.ld % 4 == 0)) &&
                      (!rope || !pe.on || pe.rotary % (pek == kPeRopeHalf ? 16 : 8) == 0);
    if (fast) {
        const int hu = (pek == kPeRopeHalf && pe.on) ? pe.rotary / 16 : 0;
        const int jobs = D / 8 - hu;
        switch (pek) {
            case kPeNone:
                launch_encode_regs<kPeNone>(jobs, in, out, inv, n_rows, seq_len, D, pe, st);
                break;
            case kPeRopeInterleaved:
                launch_encode_regs<kPeRopeInterleaved>(jobs, in, out, inv, n_rows, seq_len, D, pe,
                                                       st);
                break;
            case kPeRopeHalf:
                launch_encode_regs<kPeRopeHalf>(jobs, in, out, inv, n_rows, seq_len, D, pe, st);
                break;
            case kPeSinusoidal:
                launch_encode_regs<kPeSinusoidal>(jobs, in, out, inv, n_rows, seq_len, D, pe, st);
                break;
            default:
                return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (pek) {
        case kPeNone:
            hipLaunchKernelGGL((k_encode_f16<kPeNone>), dim3((unsigned)grid), dim3(256), 0, st, in,
                               out, inv, n_rows, seq_len, D, pe);
            break;
        case kPeRopeInterleaved:
            hipLaunchKernelGGL((k_encode_f16<kPeRopeInterleaved>), dim3((unsigned)grid), dim3(256),
                               0, st, in, out, inv, n_rows, seq_len, D, pe);
            break;
        case kPeRopeHalf:
            hipLaunchKernelGGL((k_encode_f16<kPeRopeHalf>), dim3((unsigned)grid), dim3(256), 0, st,
                               in, out, inv, n_rows, seq_len, D, pe);
            break;
        case kPeSinusoidal:
            hipLaunchKernelGGL((k_encode_f16<kPeSinusoidal>), dim3((unsigned)grid), dim3(256), 0,
                               st, in, out, inv, n_rows, seq_len, D, pe);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemm_pv(const uint16_t* E, int ldE, float* st_m, float* st_l, float* ga,
                          const uint16_t* V, uint16_t* O, int BH, int Lq, int Lk, int D,
                          hipStream_t st) {
    GemmArgs g{};
    g.A = E;
    g.B = V;
    g.C = O;
    g.st_m = st_m;
    g.st_l = st_l;
    g.ga = ga;
    g.gt = (Lk + kBN - 1) / kBN;
    // rows with at most kFacTiles key tiles: the PV workgroups turn the tile
    // statistics into softmax factors themselves; longer rows take them,
    // per chunk, from k_rowscale's output
    if (g.gt > kFacTiles) {
        hipLaunchKernelGGL(k_rowscale, dim3((unsigned)(((long)BH * Lq + 255) / 256)), dim3(256), 0,
                           st, st_m, st_l, ga, (long)BH * Lq, g.gt);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    g.M = Lq;
    g.N = D;
    g.K = Lk;
    g.lda = ldE;
    g.ldb = D;
    g.ldc = D;
    g.sa = (long)Lq * ldE;
    g.sb = (long)Lk * D;
    g.sc = (long)Lq * D;
    g.tiles_m = (Lq + kBM - 1) / kBM;
    g.tiles_n = (D + kBN - 1) / kBN;
    g.heads = BH;
    g.scale = 1.f;
    const long total = (long)g.tiles_m * g.tiles_n * BH;
    const long grid = (total + 7) / 8 * 8;
    // an even number of 64-key steps: V straight into LDS; with every tile
    // interior, one persistent workgroup per CU (a multiple of 8 of them,
    // for the XCD-aware order), else one workgroup per tile
    if (g.gt <= kFacTiles && Lk % 128 == 0) {
        const long cus = std::max(8, device_cus() / 8 * 8);
        if (Lq % kBM == 0 && D % kBN == 0)
            hipLaunchKernelGGL(k_gemm_pv_dma<true>, dim3((unsigned)std::min(grid, cus)),
                               dim3(kGemmThreads), 0, st, g);
        else
            hipLaunchKernelGGL(k_gemm_pv_dma<false>, dim3((unsigned)grid), dim3(kGemmThreads), 0,
                               st, g);
    }
    else if (g.gt <= kFacTiles)
        hipLaunchKernelGGL((k_gemm<false, true, kOutBf16, true>), dim3((unsigned)grid),
                           dim3(kGemmThreads), 0, st, g);
    else
        hipLaunchKernelGGL((k_gemm<false, true, kOutBf16, false>), dim3((unsigned)grid),
                           dim3(kGemmThreads), 0, st, g);
    return hipGetLastError();
}

}  // namespace atn
