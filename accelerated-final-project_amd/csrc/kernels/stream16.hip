// The split-D pipeline's two contractions for fp32 inputs on 16-bit MFMA
// (gfx950): k_qk_s16 (partial scores over a D-chunk) and k_pv_s16 (O = P V).
//
// Same decomposition and memory layout as stream.hip's k_qk_partial / k_pv
// (S and P in the workspace, split along D for the scores), with the
// operands held as hi + lo fp16 parts (split16.hpp: 22 significant bits,
// three exact products per product on v_mfma_f32_16x16x32_f16) instead of
// fp32 MFMA operands.  These kernels take fp32 calls with head_d % 4 == 0
// and 16-byte aligned bases; the others stay on stream.hip's.
//
// Two tile sizes (TL): 64 x 64 output tiles in 64-deep stages (each of the 4
// waves 16 rows x 64 columns) for short sides, and 128 x 128 in 32-deep
// stages (each wave 64 x 64) where both sides of the tile reach 128: twice
// the MFMA work per byte loaded from L2 (a 64 x 64 tile's loads outrun its
// MFMAs at a CU's 64 bytes per cycle), and a wave reads each fragment of a
// stage from LDS once per 64 rows instead of once per 16.
//
// Per stage each thread holds its next stage's 16-byte loads in registers
// while the current stage computes.  Operands are split as they
// are (no scaling) while each wave tracks its largest magnitude; when any
// value of the stage exceeds fp16's range the workgroup (told through LDS
// at the barrier the stage needs anyway) loads the stage again and stages
// each tensor scaled by a power of two from its largest finite magnitude.
// Each stage accumulates into fresh registers that are added to the fp32
// result times the stage's unit.  P arrives from the softmax already
// scaled by 2^15 (exact), so that small probabilities keep their bits.
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "launch.hpp"
#include "split16.hpp"

namespace atn {

namespace {

// Geometry of a TL x TL output tile (TL = 64 or 128) over 4 waves.
template <int TL>
struct S16 {
    static constexpr int STAGE = TL == 64 ? 64 : 32;  // contraction depth per stage
    static constexpr int STR = STAGE + 8;   // LDS row stride of [row][k] parts (16-bit elements)
    static constexpr int VSTR = TL + 16;    // LDS row stride of V [key][dim] (transposing reads)
    static constexpr int WR = TL == 64 ? 16 : 64;  // rows per wave
    static constexpr int WC = 64;                  // columns per wave
    static constexpr int WN = TL / WC;             // waves along the columns (1 or 2)
    static constexpr int NI = WR / 16, NJ = WC / 16;  // 16 x 16 MFMA tiles per wave
    static constexpr int VPR = STAGE / 4;          // loader: 16-byte vectors per row
    static constexpr int LROW = 256 / VPR;         // loader: rows per round
    static constexpr int NLD = TL / LROW;          // loader: rounds per tile side
    static_assert((TL / WR) * WN == 4 && NLD * LROW == TL, "4 waves, whole rounds");
};

// Workgroup maximum of two per-thread values (slots slot .. slot + 7 of
// `sh`); every thread must call it, and the caller's next barrier may not be
// skipped before the slots are reused.
__device__ __forceinline__ void wg_max2(float& a, float& b, float* sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    a = wave_max(a);
    b = wave_max(b);
    if (lane == 0) {
        sh[wave] = a;
        sh[4 + wave] = b;
    }
    __syncthreads();
    a = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    b = fmaxf(fmaxf(sh[4], sh[5]), fmaxf(sh[6], sh[7]));
}

// 4 values scaled by s, as hi and lo fp16 parts into two LDS rows
__device__ __forceinline__ void store_split4(uint16_t* hi, uint16_t* lo, float4 v, float s) {
    uint32_t h0, l0, h1, l1;
    split2_f16(v.x * s, v.y * s, h0, l0);
    split2_f16(v.z * s, v.w * s, h1, l1);
    *reinterpret_cast<uint2*>(hi) = make_uint2(h0, h1);
    *reinterpret_cast<uint2*>(lo) = make_uint2(l0, l1);
}

// Partial scores S_split[bh][i][j] = sum over the chunk's dims of q~_id k~_jd
// for one TL x TL tile; wave w computes S^T for its WR queries and WC keys
// (keys 16 j + 4 lg + r of query 16 i + lr in each lane: four consecutive
// keys, one 16-byte store per key tile).
template <int PEK, int TL>
__global__ __launch_bounds__(256) void k_qk_s16(const float* __restrict__ Q,
                                                 const float* __restrict__ K, float* __restrict__ S,
                                                 int BH, int Lq, int Lk, int D, int dchunk,
                                                 int nsplit, int tiles_q, int tiles_k, PeSide pq,
                                                 PeSide pk) {
    using G = S16<TL>;
    __shared__ __align__(16) uint16_t sq[2][TL * G::STR];  // Q hi, lo [row][dim]
    __shared__ __align__(16) uint16_t sk[2][TL * G::STR];  // K hi, lo [key][dim]
    __shared__ float slot[8];
    __shared__ __align__(16) int flag[4];  // per wave: a value of the stage outside fp16's range

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int wr = (wave / G::WN) * G::WR, wc = (wave % G::WN) * G::WC;  // wave's rows, columns
    long wg = blockIdx.x;
    const int split = (int)(wg % nsplit);
    wg /= nsplit;
    const int tk = (int)(wg % tiles_k);
    wg /= tiles_k;
    const int tq = (int)(wg % tiles_q);
    const int bh = (int)(wg / tiles_q);
    const int q0 = tq * TL, k0 = tk * TL;
    const int dbeg = split * dchunk, dend = min(D, dbeg + dchunk);

    const float* Qh = Q + (size_t)bh * Lq * D;
    const float* Kh = K + (size_t)bh * Lk * D;
    const __amdgpu_buffer_rsrc_t rq = buf_rsrc(Qh, Lq * D * 4);
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(Kh, Lk * D * 4);
    // loader: rows lrow + LROW i, dims lcol .. + 3 of the stage
    const int lrow = tid / G::VPR, lcol = (tid % G::VPR) * 4;
    float4 qv[G::NLD], kv[G::NLD];
    auto issue = [&](int d0) {
        const int d = d0 + lcol;
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            const int qi = q0 + lrow + G::LROW * i, kj = k0 + lrow + G::LROW * i;
            if constexpr (PEK == kPeNone) {
                qv[i] = ld_buf_f4(rq, qi < Lq && d < dend ? (qi * D + d) * 4 : kBufOob);
                kv[i] = ld_buf_f4(rk, kj < Lk && d < dend ? (kj * D + d) * 4 : kBufOob);
            } else {
                qv[i] = kv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (qi < Lq && d < dend)
                    qv[i] = load_row4_pe<float, PEK>(Qh + (size_t)qi * D, qi, d, dend, pq, true);
                if (kj < Lk && d < dend)
                    kv[i] = load_row4_pe<float, PEK>(Kh + (size_t)kj * D, kj, d, dend, pk, true);
            }
        }
    };

    // the rare rescaled staging of the stage at d0 (see the file comment);
    // returns the stage's unit
    auto restage = [&](int d0) -> float {
        float4 q2[G::NLD], k2[G::NLD];
        const int d = d0 + lcol;
        float mq = 0.f, mk = 0.f;
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            const int qi = q0 + lrow + G::LROW * i, kj = k0 + lrow + G::LROW * i;
            q2[i] = k2[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (qi < Lq && d < dend)
                q2[i] = load_row4_pe<float, PEK>(Qh + (size_t)qi * D, qi, d, dend, pq, true);
            if (kj < Lk && d < dend)
                k2[i] = load_row4_pe<float, PEK>(Kh + (size_t)kj * D, kj, d, dend, pk, true);
            mq = max_finite4(mq, q2[i]);
            mk = max_finite4(mk, k2[i]);
        }
        wg_max2(mq, mk, slot);
        const float sqs = pow2_scale(mq), sks = pow2_scale(mk);
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            const int o = (lrow + G::LROW * i) * G::STR + lcol;
            store_split4(&sq[0][o], &sq[1][o], q2[i], sqs);
            store_split4(&sk[0][o], &sk[1][o], k2[i], sks);
        }
        __syncthreads();
        return pow2_unit(mq) * pow2_unit(mk);
    };

    v4f sum[G::NI][G::NJ];
#pragma unroll
    for (int i = 0; i < G::NI; ++i)
#pragma unroll
        for (int j = 0; j < G::NJ; ++j) sum[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    issue(dbeg);
    for (int d0 = dbeg; d0 < dend; d0 += G::STAGE) {
        if (d0 > dbeg) __syncthreads();  // the previous stage's LDS reads are done
        float big = 0.f;
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            const int o = (lrow + G::LROW * i) * G::STR + lcol;
            store_split4(&sq[0][o], &sq[1][o], qv[i], 1.f);
            store_split4(&sk[0][o], &sk[1][o], kv[i], 1.f);
            big = vmax3abs(vmax3abs(big, qv[i].x, qv[i].y), qv[i].z, qv[i].w);
            big = vmax3abs(vmax3abs(big, kv[i].x, kv[i].y), kv[i].z, kv[i].w);
        }
        const bool over = __ballot(!(big < kF16Range)) != 0;
        if (lane == 0) flag[wave] = over;
        if (d0 + G::STAGE < dend) issue(d0 + G::STAGE);
        __syncthreads();
        float u = 1.f;
        const int4 f = *reinterpret_cast<const int4*>(flag);
        if (f.x | f.y | f.z | f.w) u = restage(d0);
        v4f acc[G::NI][G::NJ];
#pragma unroll
        for (int i = 0; i < G::NI; ++i)
#pragma unroll
            for (int j = 0; j < G::NJ; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < G::STAGE / 32; ++ks) {
            f16x8 bh_[G::NI], bl_[G::NI];
#pragma unroll
            for (int i = 0; i < G::NI; ++i) {
                const int bq = (wr + 16 * i + lr) * G::STR + 32 * ks + 8 * lg;
                bh_[i] = lds8_f16(&sq[0][bq]);
                bl_[i] = lds8_f16(&sq[1][bq]);
            }
#pragma unroll
            for (int j = 0; j < G::NJ; ++j) {
                const int ak = (wc + 16 * j + lr) * G::STR + 32 * ks + 8 * lg;
                const f16x8 ah = lds8_f16(&sk[0][ak]), al = lds8_f16(&sk[1][ak]);
#pragma unroll
                for (int i = 0; i < G::NI; ++i)
                    acc[i][j] = mfma_split(ah, al, bh_[i], bl_[i], acc[i][j]);
            }
        }
#pragma unroll
        for (int i = 0; i < G::NI; ++i)
#pragma unroll
            for (int j = 0; j < G::NJ; ++j) sum[i][j] += acc[i][j] * u;
    }

    // S^T lane values: keys k0 + wc + 16 j + 4 lg + r of query q0 + wr + 16 i + lr
#pragma unroll
    for (int i = 0; i < G::NI; ++i) {
        const int qi = q0 + wr + 16 * i + lr;
        if (qi >= Lq) continue;
        float* srow = S + (((size_t)split * BH + bh) * Lq + qi) * Lk;
#pragma unroll
        for (int j = 0; j < G::NJ; ++j) {
            const int kj = k0 + wc + 16 * j + 4 * lg;
            if ((Lk & 3) == 0) {
                if (kj < Lk)
                    *reinterpret_cast<float4*>(srow + kj) =
                        make_float4(sum[i][j][0], sum[i][j][1], sum[i][j][2], sum[i][j][3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (kj + r < Lk) srow[kj + r] = sum[i][j][r];
            }
        }
    }
}

// O[bh][i][d] = sum_j P_ij V_jd for one TL x TL tile; wave w computes O^T
// for its WR rows and WC dims (dims 16 t + 4 lg + r of row 16 i + lr in each
// lane: one 16-byte store per dim tile).  P arrives scaled by 2^15 (in
// [0, 2^15]).
template <int TL>
__global__ __launch_bounds__(256) void k_pv_s16(const float* __restrict__ P,
                                                 const float* __restrict__ V, float* __restrict__ O,
                                                 int Lq, int Lk, int D, int tiles_q, int tiles_d) {
    using G = S16<TL>;
    __shared__ __align__(16) uint16_t sp[2][TL * G::STR];        // P hi, lo [row][key]
    __shared__ __align__(16) uint16_t sv[2][G::STAGE * G::VSTR];  // V hi, lo [key][dim]
    __shared__ float slot[8];
    __shared__ __align__(16) int flag[4];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int wr = (wave / G::WN) * G::WR, wc = (wave % G::WN) * G::WC;  // wave's rows, dims
    long wg = blockIdx.x;
    const int td = (int)(wg % tiles_d);
    wg /= tiles_d;
    const int tq = (int)(wg % tiles_q);
    const int bh = (int)(wg / tiles_q);
    const int q0 = tq * TL, d0 = td * TL;

    const float* Ph = P + (size_t)bh * Lq * Lk;
    const float* Vh = V + (size_t)bh * Lk * D;
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(Ph, Lq * Lk * 4);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(Vh, Lk * D * 4);
    const bool p_vec = (Lk & 3) == 0;
    // loaders: P rows lrow + LROW i, keys lcol .. + 3 (a stage is STAGE
    // keys); V keys vrow0 + VROWS i, dims d0 + vcol0 .. + 3 (TL dims)
    const int lrow = tid / G::VPR, lcol = (tid % G::VPR) * 4;
    constexpr int VVPR = TL / 4, VROWS = 256 / VVPR, VNLD = G::STAGE / VROWS;
    const int vrow0 = tid / VVPR, vcol0 = (tid % VVPR) * 4;
    float4 pv[G::NLD], vv[VNLD];
    auto issue = [&](int kk0) {
        const int kk = kk0 + lcol, d = d0 + vcol0;
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            const int row = q0 + lrow + G::LROW * i;
            if (p_vec) {
                pv[i] = ld_buf_f4(rp, row < Lq && kk < Lk ? (row * Lk + kk) * 4 : kBufOob);
            } else {
                float t[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const auto w = __builtin_amdgcn_raw_buffer_load_b32(
                        rp, row < Lq && kk + c < Lk ? (row * Lk + kk + c) * 4 : kBufOob, 0, 0);
                    t[c] = __uint_as_float(w);
                }
                pv[i] = make_float4(t[0], t[1], t[2], t[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < VNLD; ++i) {
            const int key = kk0 + vrow0 + VROWS * i;
            vv[i] = ld_buf_f4(rv, key < Lk && d < D ? (key * D + d) * 4 : kBufOob);
        }
    };

    // the rare rescaled staging of V for the stage at kk0; returns V's unit
    auto restage = [&](int kk0) -> float {
        float4 v2[VNLD];
        const int d = d0 + vcol0;
        float mv = 0.f, unused = 0.f;
#pragma unroll
        for (int i = 0; i < VNLD; ++i) {
            const int key = kk0 + vrow0 + VROWS * i;
            v2[i] = ld_buf_f4(rv, key < Lk && d < D ? (key * D + d) * 4 : kBufOob);
            mv = max_finite4(mv, v2[i]);
        }
        wg_max2(mv, unused, slot);
        const float svs = pow2_scale(mv);
#pragma unroll
        for (int i = 0; i < VNLD; ++i) {
            const int ov = (vrow0 + VROWS * i) * G::VSTR + vcol0;
            store_split4(&sv[0][ov], &sv[1][ov], v2[i], svs);
        }
        __syncthreads();
        return pow2_unit(mv);
    };

    v4f sum[G::NI][G::NJ];
#pragma unroll
    for (int i = 0; i < G::NI; ++i)
#pragma unroll
        for (int t = 0; t < G::NJ; ++t) sum[i][t] = v4f{0.f, 0.f, 0.f, 0.f};
    issue(0);
    for (int kk0 = 0; kk0 < Lk; kk0 += G::STAGE) {
        if (kk0 > 0) __syncthreads();  // the previous stage's LDS reads are done
        float big = 0.f;
#pragma unroll
        for (int i = 0; i < G::NLD; ++i) {
            const int op = (lrow + G::LROW * i) * G::STR + lcol;
            store_split4(&sp[0][op], &sp[1][op], pv[i], 1.f);
        }
#pragma unroll
        for (int i = 0; i < VNLD; ++i) {
            const int ov = (vrow0 + VROWS * i) * G::VSTR + vcol0;
            store_split4(&sv[0][ov], &sv[1][ov], vv[i], 1.f);
            big = vmax3abs(vmax3abs(big, vv[i].x, vv[i].y), vv[i].z, vv[i].w);
        }
        const bool over = __ballot(!(big < kF16Range)) != 0;
        if (lane == 0) flag[wave] = over;
        if (kk0 + G::STAGE < Lk) issue(kk0 + G::STAGE);
        __syncthreads();
        float u = 1.f;
        const int4 f = *reinterpret_cast<const int4*>(flag);
        if (f.x | f.y | f.z | f.w) u = restage(kk0);
        v4f acc[G::NI][G::NJ];
#pragma unroll
        for (int i = 0; i < G::NI; ++i)
#pragma unroll
            for (int t = 0; t < G::NJ; ++t) acc[i][t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < G::STAGE / 32; ++b) {
            f16x8 ph[G::NI], pl[G::NI];
#pragma unroll
            for (int i = 0; i < G::NI; ++i) {
                const int bp = (wr + 16 * i + lr) * G::STR + 32 * b + 8 * lg;
                ph[i] = lds8_f16(&sp[0][bp]);
                pl[i] = lds8_f16(&sp[1][bp]);
            }
            // V^T fragments: keys 32 b + 8 lg + 0..7 of dim wc + 16 t + lr
            const int vrow = 32 * b + 8 * lg + (lr >> 2), vcol = 4 * (lr & 3);
#pragma unroll
            for (int t = 0; t < G::NJ; ++t) {
                const int a = vrow * G::VSTR + wc + 16 * t + vcol;
                const uint2 h0 = lds_tr16(&sv[0][a]), h1 = lds_tr16(&sv[0][a + 4 * G::VSTR]);
                const uint2 l0 = lds_tr16(&sv[1][a]), l1 = lds_tr16(&sv[1][a + 4 * G::VSTR]);
                const f16x8 vh = __builtin_bit_cast(f16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
                const f16x8 vl = __builtin_bit_cast(f16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
#pragma unroll
                for (int i = 0; i < G::NI; ++i)
                    acc[i][t] = mfma_split(vh, vl, ph[i], pl[i], acc[i][t]);
            }
        }
#pragma unroll
        for (int i = 0; i < G::NI; ++i)
#pragma unroll
            for (int t = 0; t < G::NJ; ++t) sum[i][t] += acc[i][t] * u;
    }

    // P's 2^15
#pragma unroll
    for (int i = 0; i < G::NI; ++i) {
        const int row = q0 + wr + 16 * i + lr;
        if (row >= Lq) continue;
        float* orow = O + ((size_t)bh * Lq + row) * D;
#pragma unroll
        for (int t = 0; t < G::NJ; ++t) {
            const int d = d0 + wc + 16 * t + 4 * lg;
            if (d < D)
                *reinterpret_cast<float4*>(orow + d) =
                    make_float4(sum[i][t][0] * (1.0f / 32768.0f), sum[i][t][1] * (1.0f / 32768.0f),
                                sum[i][t][2] * (1.0f / 32768.0f), sum[i][t][3] * (1.0f / 32768.0f));
        }
    }
}

template <int TL>
hipError_t launch_qk_tl(int pek, const float* Q, const float* K, float* S, int BH, int Lq, int Lk,
                        int D, int dchunk, int nsplit, const PeSide& pq, const PeSide& pk,
                        hipStream_t st) {
    const int tiles_q = (Lq + TL - 1) / TL, tiles_k = (Lk + TL - 1) / TL;
    const dim3 grid((unsigned)((long)BH * tiles_q * tiles_k * nsplit)), block(256);
    switch (pek) {
        case kPeNone:
            hipLaunchKernelGGL((k_qk_s16<kPeNone, TL>), grid, block, 0, st, Q, K, S, BH, Lq, Lk,
                               D, dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        case kPeRopeInterleaved:
            hipLaunchKernelGGL((k_qk_s16<kPeRopeInterleaved, TL>), grid, block, 0, st, Q, K, S,
                               BH, Lq, Lk, D, dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        case kPeRopeHalf:
            hipLaunchKernelGGL((k_qk_s16<kPeRopeHalf, TL>), grid, block, 0, st, Q, K, S, BH, Lq,
                               Lk, D, dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        case kPeSinusoidal:
            hipLaunchKernelGGL((k_qk_s16<kPeSinusoidal, TL>), grid, block, 0, st, Q, K, S, BH,
                               Lq, Lk, D, dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

std::atomic<int> g_tile_force{0};  // 64 or 128: that tile wherever it fits; 0: by grid

// CU count of the current device (queried once per device)
int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = cache[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            c <= 0)
            c = 256;
        cache[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

// 128 x 128 tiles when their grid gives every CU two workgroups (both of a
// tile's sides reaching 128), else 64 x 64: a 128 x 128 tile loads half the
// bytes per MFMA, but with one workgroup per CU its waves have nothing to
// run beside them (measured: (4,32,512,512,128) 1.14x and (2,4,1024,1024,
// 512) 1.08x faster, (1,8,128,128,1024) 0.75x, (1,4,512,512,2048) even)
bool big_tiles(long grid128) {
    return g_tile_force.load(std::memory_order_relaxed) != 64 && grid128 >= 2L * device_cus();
}

}  // namespace

void s16_set_tile(int tile) { g_tile_force.store(tile == 64 || tile == 128 ? tile : 0); }

// (atn_tuning.splitd_tile forces either size)
hipError_t launch_qk_s16(int pek, const float* Q, const float* K, float* S, int BH, int Lq, int Lk,
                         int D, int dchunk, int nsplit, const PeSide& pq, const PeSide& pk,
                         hipStream_t st) {
    const int force = g_tile_force.load(std::memory_order_relaxed);
    if (force == 128 ? Lq >= 128 && Lk >= 128
                     : s16_fits_128(Lq, Lk) &&
                           big_tiles((long)BH * ((Lq + 127) / 128) * ((Lk + 127) / 128) * nsplit))
        return launch_qk_tl<128>(pek, Q, K, S, BH, Lq, Lk, D, dchunk, nsplit, pq, pk, st);
    return launch_qk_tl<64>(pek, Q, K, S, BH, Lq, Lk, D, dchunk, nsplit, pq, pk, st);
}

hipError_t launch_pv_s16(const float* P, const float* V, float* O, int BH, int Lq, int Lk, int D,
                         hipStream_t st) {
    const int force = g_tile_force.load(std::memory_order_relaxed);
    if (force == 128 ? Lq >= 128 && D >= 128
                     : s16_fits_128(Lq, D) &&
                           big_tiles((long)BH * ((Lq + 127) / 128) * ((D + 127) / 128))) {
        const int tiles_q = (Lq + 127) / 128, tiles_d = (D + 127) / 128;
        hipLaunchKernelGGL(k_pv_s16<128>, dim3((unsigned)((long)BH * tiles_q * tiles_d)),
                           dim3(256), 0, st, P, V, O, Lq, Lk, D, tiles_q, tiles_d);
        return hipGetLastError();
    }
    const int tiles_q = (Lq + 63) / 64, tiles_d = (D + 63) / 64;
    hipLaunchKernelGGL(k_pv_s16<64>, dim3((unsigned)((long)BH * tiles_q * tiles_d)), dim3(256), 0,
                       st, P, V, O, Lq, Lk, D, tiles_q, tiles_d);
    return hipGetLastError();
}

}  // namespace atn
