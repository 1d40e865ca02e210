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
//                 fp16 rows with a power-of-two scale per row
//   k_gemm  (NT)  S = scale * Q K^T            (fp32 S to the workspace)
//   k_softmax_bf  P = softmax(S) per row       (exact: max, exp, sum, divide;
//                                               bf16 P)
//   k_gemm  (NN)  O = P V                      (bf16 O)
//
// Plain bf16 inputs are exact MFMA operands.  Encoded rows are not bf16
// values any more; rounding them back to bf16 (8-bit mantissa) costs up to
// ~2e-2 of rms on single outputs, so they are kept as fp16 (11-bit
// mantissa) instead, each row scaled by a power of two that puts its
// largest magnitude in [2^14, 2^15) -- safe for any input range -- and the
// GEMM epilogue multiplies the row and column scales back (exactly).
//
// Both GEMMs use 256 x 256 output tiles per workgroup of 512 threads (8
// waves, each 64 x 128 = 2 x 4 tiles of
// v_mfma_f32_32x32x16_{f16,bf16}), a K step of 64 with the global loads of
// step k + 1 in flight while step k runs its MFMAs (double-buffered LDS,
// 144 KiB), and an
// XCD-aware tile order: consecutive tile indices run on the same XCD
// (workgroups are dealt round-robin to the 8 XCDs), so concurrent
// workgroups of one head share their Q/K/V panels in that XCD's L2.
//
// V enters the second GEMM as the B operand, which MFMA wants contiguous
// along K (= keys); V rows are contiguous along D, so the V tile is
// transposed on its way into LDS.
#include "common.hpp"
#include "launch.hpp"

namespace atn {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kGemmThreads = 512;            // 8 waves
constexpr int kWavesN = 2;                   // wave grid: (8 / kWavesN) x kWavesN
constexpr int kTI = kBM / (kGemmThreads / 64 / kWavesN) / 32;  // 32x32 tiles per wave (rows)
constexpr int kTJ = kBN / kWavesN / 32;                        // (columns)
constexpr int kDepth = 1;                    // register stages of global prefetch (1 or 2)
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

// Tile index of this workgroup with consecutive indices kept on one XCD:
// hardware deals workgroup w to XCD w % 8, so XCD x gets tiles
// [x * per, (x + 1) * per).
__device__ __forceinline__ long xcd_tile(long w, long total) {
    const long per = (total + 7) / 8;
    const long t = (w % 8) * per + w / 8;
    return t;  // may be >= total for the last XCD: caller checks
}

// Epilogue selectors
constexpr int kOutScoresF32 = 0;  // C = scale * acc, fp32, row stride ldc
constexpr int kOutBf16 = 1;       // C = bf16(acc), row stride ldc

// C[M x N] = A[M x K] * B^T where B is [N x K] (NT, both K-contiguous) when
// B_NN == false, or A[M x K] * B with B [K x N] N-contiguous when B_NN.
// Batched over heads: A/B/C advance by their head strides per bh.
struct GemmArgs {
    const uint16_t* A;
    const uint16_t* B;
    void* C;
    const float* rs;              // optional per-row scales [heads][M] (or NULL)
    const float* cs;              // optional per-column scales [heads][N] (or NULL)
    int M, N, K;
    long lda, ldb, ldc;           // row strides (elements)
    long sa, sb, sc;              // head strides (elements)
    int tiles_m, tiles_n, heads;  // grid decomposition
    float scale;
};

template <bool F16, bool B_NN, int OUT>
__global__ __launch_bounds__(kGemmThreads) void k_gemm(GemmArgs g) {
    // one LDS block: A stages 0/1, then B^T stages 0/1 ([n][k] rows); the
    // bf16 epilogue reuses it whole as an output staging tile
    __shared__ __align__(16) uint16_t lds[4 * kTileElems];
    uint16_t(*As)[kTileElems] = reinterpret_cast<uint16_t(*)[kTileElems]>(lds);
    uint16_t(*Bs)[kTileElems] = reinterpret_cast<uint16_t(*)[kTileElems]>(lds + 2 * kTileElems);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long per_head = (long)g.tiles_m * g.tiles_n;
    const long total = per_head * g.heads;
    const long t = xcd_tile(blockIdx.x, total);
    if (t >= total) return;
    const int bh = (int)(t / per_head);
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
    const int m0 = tm * kBM, n0 = tn * kBN;

    const uint16_t* A = g.A + bh * g.sa;
    const uint16_t* B = g.B + bh * g.sb;

    // ---- global -> register staging: each thread moves two 16-byte chunks
    // of A (rows m0.., 4 chunks of 8 per row) and, for B^T rows (NT), two
    // chunks of B; for NN, an 8-key x 2-column block of B (8 dwords), which
    // it transposes with v_perm_b32 into two 16-byte LDS rows.  Two register
    // stages rotate with the two LDS buffers, so a step's global loads are
    // issued two MFMA phases before their data is needed.
    // A chunk c (0..1023): row = c / 4, k8 = (c % 4) * 8.
    constexpr int kChunks = kBM * kBK / 8 / kGemmThreads;  // 16-byte chunks per thread per operand
    constexpr int kVBlocks = kBK / 8 * (kBN / 2) / kGemmThreads;  // NN: 8x2 blocks per thread
    static_assert(kChunks >= 1 && kVBlocks >= 1, "tile too small for the thread count");
    struct Stage {
        uint4 a[kChunks], b[kChunks];
        uint32_t v[kVBlocks][8];
    };
    Stage st0, st1;
    // NN block b = tid + u * threads: keys 8 * (b / 128).., columns 2 * (b % 128), +1
    auto load_stage = [&](Stage& r, int k0) {
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int cidx = tid + u * kGemmThreads;
            const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
            const int gm = m0 + row, gk = k0 + k8;
            r.a[u] = make_uint4(0, 0, 0, 0);
            if (gm < g.M && gk < g.K)
                r.a[u] = *reinterpret_cast<const uint4*>(A + (long)gm * g.lda + gk);
        }
        if constexpr (!B_NN) {
#pragma unroll
            for (int u = 0; u < kChunks; ++u) {
                const int cidx = tid + u * kGemmThreads;
                const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
                const int gn = n0 + row, gk = k0 + k8;
                r.b[u] = make_uint4(0, 0, 0, 0);
                if (gn < g.N && gk < g.K)
                    r.b[u] = *reinterpret_cast<const uint4*>(B + (long)gn * g.ldb + gk);
            }
        } else {
            // B is [K x N]: blocks of 8 consecutive keys x 2 consecutive columns
#pragma unroll
            for (int u = 0; u < kVBlocks; ++u) {
                const int blk = tid + u * kGemmThreads;
                const int vkg = blk / (kBN / 2), vdp = blk % (kBN / 2);
                const int gn = n0 + 2 * vdp;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int gk = k0 + vkg * 8 + e;
                    r.v[u][e] = 0u;
                    if (gk < g.K && gn < g.N)
                        r.v[u][e] = *reinterpret_cast<const uint32_t*>(B + (long)gk * g.ldb + gn);
                }
            }
        }
    };
    auto store_stage = [&](const Stage& r, int s) {
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int cidx = tid + u * kGemmThreads;
            const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
            *reinterpret_cast<uint4*>(&As[s][row * kLdsRow + k8]) = r.a[u];
        }
        if constexpr (!B_NN) {
#pragma unroll
            for (int u = 0; u < kChunks; ++u) {
                const int cidx = tid + u * kGemmThreads;
                const int row = cidx / kChunkPerRow, k8 = (cidx % kChunkPerRow) * 8;
                *reinterpret_cast<uint4*>(&Bs[s][row * kLdsRow + k8]) = r.b[u];
            }
        } else {
            // v[e] = (B[k_e][n] | B[k_e][n + 1] << 16): gather the low halves
            // into row n and the high halves into row n + 1 of Bs[n][k]
#pragma unroll
            for (int u = 0; u < kVBlocks; ++u) {
                const int blk = tid + u * kGemmThreads;
                const int vkg = blk / (kBN / 2), vdp = blk % (kBN / 2);
                const uint32_t* v = r.v[u];
                uint4 lo, hi;
                lo.x = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
                lo.y = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);
                lo.z = __builtin_amdgcn_perm(v[5], v[4], 0x05040100u);
                lo.w = __builtin_amdgcn_perm(v[7], v[6], 0x05040100u);
                hi.x = __builtin_amdgcn_perm(v[1], v[0], 0x07060302u);
                hi.y = __builtin_amdgcn_perm(v[3], v[2], 0x07060302u);
                hi.z = __builtin_amdgcn_perm(v[5], v[4], 0x07060302u);
                hi.w = __builtin_amdgcn_perm(v[7], v[6], 0x07060302u);
                *reinterpret_cast<uint4*>(&Bs[s][(2 * vdp) * kLdsRow + vkg * 8]) = lo;
                *reinterpret_cast<uint4*>(&Bs[s][(2 * vdp + 1) * kLdsRow + vkg * 8]) = hi;
            }
        }
    };

    // ---- wave tile: 128 x 128 = 4 x 4 MFMA tiles of 32 x 32
    constexpr int TI = kTI, TJ = kTJ;
    const int wm = (wave / kWavesN) * (TI * 32), wn = (wave % kWavesN) * (TJ * 32);
    v16f acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int lrow = lane & 31, lkh = (lane >> 5) * 8;
    const int nk = (g.K + kBK - 1) / kBK;
    auto compute = [&](int s) {
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 16) {
            uint4 af[TI], bfr[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i)
                af[i] = *reinterpret_cast<const uint4*>(
                    &As[s][(wm + i * 32 + lrow) * kLdsRow + ks + lkh]);
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                bfr[j] = *reinterpret_cast<const uint4*>(
                    &Bs[s][(wn + j * 32 + lrow) * kLdsRow + ks + lkh]);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) acc[i][j] = mfma_32x32x16<F16>(af[i], bfr[j], acc[i][j]);
        }
    };

    if constexpr (kDepth == 1) {
        // one register stage: step kt + 1's loads fly during step kt's MFMAs
        load_stage(st0, 0);
        store_stage(st0, 0);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int sb = kt & 1;
            if (kt + 1 < nk) load_stage(st0, (kt + 1) * kBK);
            compute(sb);
            if (kt + 1 < nk) store_stage(st0, sb ^ 1);
            __syncthreads();
        }
    } else {
        // two register stages: step kt reads LDS buffer kt % 2 while register
        // stage (kt % 2) carries step kt + 2
        load_stage(st0, 0);
        if (nk > 1) load_stage(st1, kBK);
        store_stage(st0, 0);
        __syncthreads();
        for (int kt = 0; kt < nk; kt += 2) {
            if (kt + 2 < nk) load_stage(st0, (kt + 2) * kBK);
            compute(0);
            if (kt + 1 < nk) store_stage(st1, 1);
            __syncthreads();
            if (kt + 1 >= nk) break;
            if (kt + 3 < nk) load_stage(st1, (kt + 3) * kBK);
            compute(1);
            if (kt + 2 < nk) store_stage(st0, 0);
            __syncthreads();
        }
    }

    // ---- epilogue: lane holds column (lane % 32) and rows
    // 8 * (r / 4) + 4 * (lane / 32) + r % 4 of each 32 x 32 tile.
    // bf16 output goes through LDS (the operand buffers are free now) and
    // leaves as 16-byte row chunks.
    if constexpr (OUT == kOutBf16) {
        uint16_t* Ct = lds;  // 256 x (256 + 8) bf16 staging tile
        constexpr int kCRow = kBN + 8;
        static_assert(kBM * kCRow <= 4 * kTileElems, "output staging does not fit");
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int col = wn + j * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    Ct[row * kCRow + col] = f32_to_bf16_bits(acc[i][j][r]);
                }
            }
        __syncthreads();
        uint16_t* C = static_cast<uint16_t*>(g.C) + bh * g.sc;
        for (int cidx = tid; cidx < kBM * kBN / 8; cidx += kGemmThreads) {
            const int row = cidx / (kBN / 8), c8 = (cidx % (kBN / 8)) * 8;
            const int grow = m0 + row, gcol = n0 + c8;
            if (grow < g.M && gcol < g.N)
                *reinterpret_cast<uint4*>(C + (long)grow * g.ldc + gcol) =
                    *reinterpret_cast<const uint4*>(&Ct[row * kCRow + c8]);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = n0 + wn + j * 32 + (lane & 31);
            if (col >= g.N) continue;
            const float csc = g.cs ? g.cs[(long)bh * g.N + col] * g.scale : g.scale;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= g.M) continue;
                const long off = bh * g.sc + (long)row * g.ldc + col;
                if constexpr (OUT == kOutScoresF32) {
                    float v = acc[i][j][r] * csc;
                    if (g.rs) v *= g.rs[(long)bh * g.M + row];
                    static_cast<float*>(g.C)[off] = v;
                } else {
                    static_cast<uint16_t*>(g.C)[off] = f32_to_bf16_bits(acc[i][j][r]);
                }
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

// P[row] = bf16(softmax(S[row])) for rows of length Lk; one wave per row.
__global__ __launch_bounds__(256) void k_softmax_bf(const float* __restrict__ S,
                                                    uint16_t* __restrict__ P, long rows, int Lk) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* s = S + row * Lk;
    uint16_t* p = P + row * Lk;
    float m = -INFINITY;
    for (int j = lane; j < Lk; j += 64) m = fmaxf(m, s[j]);
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < Lk; j += 64) l += __expf(s[j] - m);
    l = wave_sum(l);
    const float inv = 1.0f / l;
    for (int j = lane; j < Lk; j += 64) p[j] = f32_to_bf16_bits(__expf(s[j] - m) * inv);
}

// Register-resident encoder: the row is split into 8-element units (for
// rotate-half, unit u < r/16 is paired with its partner unit u + r/16 so both
// halves of every rotation are in one thread); each thread keeps its units
// in registers, so the row is read once: 16-byte loads of x, 32-byte loads
// of the compact cos/sin (or sin/cos) table rows, one block-wide max, then
// scaled fp16 16-byte stores.
constexpr int kEncThreads = 256;
constexpr int kEncMaxUnits = 4;  // units per thread: D <= 4 * 256 * 8 = 8192

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

template <int PEK>
__global__ __launch_bounds__(kEncThreads) void k_encode_f16_regs(const uint16_t* __restrict__ in,
                                                                 uint16_t* __restrict__ out,
                                                                 float* __restrict__ inv,
                                                                 long n_rows, int seq_len, int D,
                                                                 PeSide pe) {
    __shared__ float red[kEncThreads / 64];
    const int tid = threadIdx.x;
    const bool half_pairs = PEK == kPeRopeHalf && pe.on;
    const int hu = half_pairs ? pe.rotary / 16 : 0;        // paired units (rotate-half)
    const int nunits = D / 8 - hu;                        // units handled as the "first" of a job
    for (long row = blockIdx.x; row < n_rows; row += gridDim.x) {
        const int pos = (int)(row % seq_len);
        const uint16_t* xr = in + row * D;
        float v[kEncMaxUnits][2][8];
        int du[kEncMaxUnits][2];
        float m = 0.f;
#pragma unroll
        for (int k = 0; k < kEncMaxUnits; ++k) {
            const int job = tid + k * kEncThreads;
            du[k][0] = du[k][1] = -1;
            if (job >= nunits) continue;
            // job -> first unit; rotate-half pairs jobs < hu with unit job + hu
            const int u0 = (half_pairs && job >= hu) ? job + hu : job;
            const int d0 = u0 * 8;
            du[k][0] = d0;
            unpack_bf16x8(*reinterpret_cast<const uint4*>(xr + d0), v[k][0]);
            if constexpr (PEK == kPeRopeHalf) {
                if (half_pairs && job < hu) {
                    const int d1 = d0 + pe.rotary / 2;
                    du[k][1] = d1;
                    unpack_bf16x8(*reinterpret_cast<const uint4*>(xr + d1), v[k][1]);
                    float c[8], sn[8];
                    ld8f(pe.a + (size_t)pos * pe.ld + d0, c);
                    ld8f(pe.b + (size_t)pos * pe.ld + d0, sn);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float x0 = v[k][0][e], x1 = v[k][1][e];
                        v[k][0][e] = rot_first(x0, x1, c[e], sn[e]);
                        v[k][1][e] = rot_second(x0, x1, c[e], sn[e]);
                    }
                }
            } else if constexpr (PEK == kPeRopeInterleaved) {
                if (pe.on && d0 < pe.rotary) {
                    float c[4], sn[4];
                    ld4f(pe.a + (size_t)pos * pe.ld + d0 / 2, c);
                    ld4f(pe.b + (size_t)pos * pe.ld + d0 / 2, sn);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x0 = v[k][0][2 * e], x1 = v[k][0][2 * e + 1];
                        v[k][0][2 * e] = rot_first(x0, x1, c[e], sn[e]);
                        v[k][0][2 * e + 1] = rot_second(x0, x1, c[e], sn[e]);
                    }
                }
            } else if constexpr (PEK == kPeSinusoidal) {
                if (pe.on) {
                    float sv[4], cv[4];
                    ld4f(pe.a + (size_t)pos * pe.ld + d0 / 2, sv);
                    ld4f(pe.b + (size_t)pos * pe.ld + d0 / 2, cv);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[k][0][2 * e] = v[k][0][2 * e] + sv[e];
                        v[k][0][2 * e + 1] = v[k][0][2 * e + 1] + cv[e];
                    }
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h)
                if (du[k][h] >= 0)
#pragma unroll
                    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[k][h][e]));
        }
        m = wave_max(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();  // red is reused by the next row
        int kexp = 0;
        if (m > 0.f && m <= 3.0e38f) kexp = 14 - ilogbf(m);
        kexp = max(-100, min(100, kexp));
        const float up = ldexpf(1.0f, kexp);
        if (tid == 0) inv[row] = ldexpf(1.0f, -kexp);
        uint16_t* yr = out + row * D;
#pragma unroll
        for (int k = 0; k < kEncMaxUnits; ++k)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                if (du[k][h] >= 0)
                    *reinterpret_cast<uint4*>(yr + du[k][h]) = pack_f16x8(v[k][h], up);
    }
}

}  // namespace

hipError_t launch_gemm_qk(int f16, const uint16_t* Q, const uint16_t* K, const float* qinv,
                          const float* kinv, float* S, int BH, int Lq, int Lk, int D, float scale,
                          hipStream_t st) {
    GemmArgs g{};
    g.A = Q;
    g.B = K;
    g.C = S;
    g.rs = qinv;
    g.cs = kinv;
    g.M = Lq;
    g.N = Lk;
    g.K = D;
    g.lda = D;
    g.ldb = D;
    g.ldc = Lk;
    g.sa = (long)Lq * D;
    g.sb = (long)Lk * D;
    g.sc = (long)Lq * Lk;
    g.tiles_m = (Lq + kBM - 1) / kBM;
    g.tiles_n = (Lk + kBN - 1) / kBN;
    g.heads = BH;
    g.scale = scale;
    const long total = (long)g.tiles_m * g.tiles_n * BH;
    const long grid = (total + 7) / 8 * 8;
    if (f16)
        hipLaunchKernelGGL((k_gemm<true, false, kOutScoresF32>), dim3((unsigned)grid),
                           dim3(kGemmThreads), 0, st, g);
    else
        hipLaunchKernelGGL((k_gemm<false, false, kOutScoresF32>), dim3((unsigned)grid),
                           dim3(kGemmThreads), 0, st, g);
    return hipGetLastError();
}

hipError_t launch_encode_f16(int pek, const uint16_t* in, uint16_t* out, float* inv, long n_rows,
                             int seq_len, int D, const PeSide& pe, hipStream_t st) {
    const long grid = n_rows < 65536 ? n_rows : 65536;
    // register-resident form: D % 8 == 0, D <= 8192, the library's compact
    // tables, and a rotary width that keeps 8-element units whole
    const bool rope = pek == kPeRopeInterleaved || pek == kPeRopeHalf;
    const bool fast = D % 8 == 0 && D <= kEncMaxUnits * kEncThreads * 8 &&
                      (pek == kPeNone || !pe.on || (pe.dup == 0 && pe.ld % 4 == 0)) &&
                      (!rope || !pe.on || pe.rotary % (pek == kPeRopeHalf ? 16 : 8) == 0);
    if (fast) {
        switch (pek) {
            case kPeNone:
                hipLaunchKernelGGL((k_encode_f16_regs<kPeNone>), dim3((unsigned)grid),
                                   dim3(kEncThreads), 0, st, in, out, inv, n_rows, seq_len, D, pe);
                break;
            case kPeRopeInterleaved:
                hipLaunchKernelGGL((k_encode_f16_regs<kPeRopeInterleaved>), dim3((unsigned)grid),
                                   dim3(kEncThreads), 0, st, in, out, inv, n_rows, seq_len, D, pe);
                break;
            case kPeRopeHalf:
                hipLaunchKernelGGL((k_encode_f16_regs<kPeRopeHalf>), dim3((unsigned)grid),
                                   dim3(kEncThreads), 0, st, in, out, inv, n_rows, seq_len, D, pe);
                break;
            case kPeSinusoidal:
                hipLaunchKernelGGL((k_encode_f16_regs<kPeSinusoidal>), dim3((unsigned)grid),
                                   dim3(kEncThreads), 0, st, in, out, inv, n_rows, seq_len, D, pe);
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

hipError_t launch_softmax_bf16(const float* S, uint16_t* P, long rows, int Lk, hipStream_t st) {
    const long grid = (rows + 3) / 4;
    hipLaunchKernelGGL(k_softmax_bf, dim3((unsigned)grid), dim3(256), 0, st, S, P, rows, Lk);
    return hipGetLastError();
}

hipError_t launch_gemm_pv(const uint16_t* P, const uint16_t* V, uint16_t* O, int BH, int Lq, int Lk,
                          int D, hipStream_t st) {
    GemmArgs g{};
    g.A = P;
    g.B = V;
    g.C = O;
    g.M = Lq;
    g.N = D;
    g.K = Lk;
    g.lda = Lk;
    g.ldb = D;
    g.ldc = D;
    g.sa = (long)Lq * Lk;
    g.sb = (long)Lk * D;
    g.sc = (long)Lq * D;
    g.tiles_m = (Lq + kBM - 1) / kBM;
    g.tiles_n = (D + kBN - 1) / kBN;
    g.heads = BH;
    g.scale = 1.f;
    const long total = (long)g.tiles_m * g.tiles_n * BH;
    const long grid = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((k_gemm<false, true, kOutBf16>), dim3((unsigned)grid), dim3(kGemmThreads), 0,
                       st, g);
    return hipGetLastError();
}

}  // namespace atn
