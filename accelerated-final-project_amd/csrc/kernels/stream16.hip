// The split-D pipeline's two contractions for fp32 inputs on 16-bit MFMA
// (gfx950): k_qk_s16 (partial scores over a D-chunk) and k_pv_s16 (O = P V).
//
// Same decomposition and memory layout as stream.hip's k_qk_partial / k_pv
// (64 x 64 output tiles, S and P in the workspace, split along D for the
// scores), with the operands held as hi + lo fp16 parts (split16.hpp: 22
// significant bits, three exact products per product on
// v_mfma_f32_16x16x32_f16) instead of fp32 MFMA operands: a 64-deep stage
// of a 64 x 64 tile takes 24 MFMAs of 16 cycles per wave instead of 32 of
// v_mfma_f32_32x32x2f32's 64.  These kernels take fp32 calls with head_d %
// 4 == 0 and 16-byte aligned bases; the others stay on stream.hip's.
//
// Per 64-deep stage each thread holds its next stage's 16-byte loads in
// registers while the current stage computes.  Operands are split as they
// are (no scaling) while each wave tracks its largest magnitude; when any
// value of the stage exceeds fp16's range the workgroup (told through LDS
// at the barrier the stage needs anyway) loads the stage again and stages
// each tensor scaled by a power of two from its largest finite magnitude.
// Each stage accumulates into fresh registers that are added to the fp32
// result times the stage's unit.  P arrives from the softmax already
// scaled by 2^15 (exact), so that small probabilities keep their bits.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"
#include "split16.hpp"

namespace atn {

namespace {

constexpr int kT = 64;        // output tile rows and columns
constexpr int kStage = 64;    // contraction depth staged per step
constexpr int kStr = kStage + 8;  // LDS row stride of row-major [row][k] parts (16-bit elements)
constexpr int kVStr = kT + 16;    // LDS row stride of V [key][dim] (transposing reads)

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
// for one 64 x 64 tile; wave w computes S^T for queries 16 w .. + 15 (keys
// 16 j + 4 lg + r of query lr in each lane: four consecutive keys, one
// 16-byte store per key tile).
template <int PEK>
__global__ __launch_bounds__(256) void k_qk_s16(const float* __restrict__ Q,
                                                 const float* __restrict__ K, float* __restrict__ S,
                                                 int BH, int Lq, int Lk, int D, int dchunk,
                                                 int nsplit, int tiles_q, int tiles_k, PeSide pq,
                                                 PeSide pk) {
    __shared__ __align__(16) uint16_t sq[2][kT * kStr];  // Q hi, lo [row][dim]
    __shared__ __align__(16) uint16_t sk[2][kT * kStr];  // K hi, lo [key][dim]
    __shared__ float slot[8];
    __shared__ __align__(16) int flag[4];  // per wave: a value of the stage outside fp16's range

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    long wg = blockIdx.x;
    const int split = (int)(wg % nsplit);
    wg /= nsplit;
    const int tk = (int)(wg % tiles_k);
    wg /= tiles_k;
    const int tq = (int)(wg % tiles_q);
    const int bh = (int)(wg / tiles_q);
    const int q0 = tq * kT, k0 = tk * kT;
    const int dbeg = split * dchunk, dend = min(D, dbeg + dchunk);

    const float* Qh = Q + (size_t)bh * Lq * D;
    const float* Kh = K + (size_t)bh * Lk * D;
    const __amdgpu_buffer_rsrc_t rq = buf_rsrc(Qh, Lq * D * 4);
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(Kh, Lk * D * 4);
    // loader: rows lrow + 16 i, dims lcol .. + 3 of the stage
    const int lrow = tid >> 4, lcol = (tid & 15) * 4;
    float4 qv[4], kv[4];
    auto issue = [&](int d0) {
        const int d = d0 + lcol;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qi = q0 + lrow + 16 * i, kj = k0 + lrow + 16 * i;
            if constexpr (PEK == kPeNone) {
                qv[i] = ld_buf_f4(rq, d < dend ? (qi * D + d) * 4 : kBufOob);
                kv[i] = ld_buf_f4(rk, d < dend ? (kj * D + d) * 4 : kBufOob);
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
        float4 q2[4], k2[4];
        const int d = d0 + lcol;
        float mq = 0.f, mk = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qi = q0 + lrow + 16 * i, kj = k0 + lrow + 16 * i;
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
        for (int i = 0; i < 4; ++i) {
            const int o = (lrow + 16 * i) * kStr + lcol;
            store_split4(&sq[0][o], &sq[1][o], q2[i], sqs);
            store_split4(&sk[0][o], &sk[1][o], k2[i], sks);
        }
        __syncthreads();
        return pow2_unit(mq) * pow2_unit(mk);
    };

    v4f sum[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sum[j] = v4f{0.f, 0.f, 0.f, 0.f};
    issue(dbeg);
    for (int d0 = dbeg; d0 < dend; d0 += kStage) {
        if (d0 > dbeg) __syncthreads();  // the previous stage's LDS reads are done
        float big = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int o = (lrow + 16 * i) * kStr + lcol;
            store_split4(&sq[0][o], &sq[1][o], qv[i], 1.f);
            store_split4(&sk[0][o], &sk[1][o], kv[i], 1.f);
            big = vmax3abs(vmax3abs(big, qv[i].x, qv[i].y), qv[i].z, qv[i].w);
            big = vmax3abs(vmax3abs(big, kv[i].x, kv[i].y), kv[i].z, kv[i].w);
        }
        const bool over = __ballot(!(big < kF16Range)) != 0;
        if (lane == 0) flag[wave] = over;
        if (d0 + kStage < dend) issue(d0 + kStage);
        __syncthreads();
        float u = 1.f;
        const int4 f = *reinterpret_cast<const int4*>(flag);
        if (f.x | f.y | f.z | f.w) u = restage(d0);
        v4f acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < kStage / 32; ++ks) {
            const int bq = (16 * wave + lr) * kStr + 32 * ks + 8 * lg;
            const f16x8 bh_ = lds8_f16(&sq[0][bq]), bl_ = lds8_f16(&sq[1][bq]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ak = (16 * j + lr) * kStr + 32 * ks + 8 * lg;
                acc[j] = mfma_split(lds8_f16(&sk[0][ak]), lds8_f16(&sk[1][ak]), bh_, bl_, acc[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) sum[j] += acc[j] * u;
    }

    // S^T lane values: keys k0 + 16 j + 4 lg + r of query q0 + 16 w + lr
    const int qi = q0 + 16 * wave + lr;
    if (qi < Lq) {
        float* srow = S + (((size_t)split * BH + bh) * Lq + qi) * Lk;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kj = k0 + 16 * j + 4 * lg;
            if ((Lk & 3) == 0) {
                if (kj < Lk) *reinterpret_cast<float4*>(srow + kj) = make_float4(sum[j][0], sum[j][1], sum[j][2], sum[j][3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (kj + r < Lk) srow[kj + r] = sum[j][r];
            }
        }
    }
}

// O[bh][i][d] = sum_j P_ij V_jd for one 64 x 64 tile; wave w computes O^T
// for rows 16 w .. + 15 (dims 16 t + 4 lg + r of row lr in each lane: one
// 16-byte store per dim tile).  P arrives scaled by 2^15 (in [0, 2^15]).
__global__ __launch_bounds__(256) void k_pv_s16(const float* __restrict__ P,
                                                 const float* __restrict__ V, float* __restrict__ O,
                                                 int Lq, int Lk, int D, int tiles_q, int tiles_d) {
    __shared__ __align__(16) uint16_t sp[2][kT * kStr];   // P hi, lo [row][key]
    __shared__ __align__(16) uint16_t sv[2][kT * kVStr];  // V hi, lo [key][dim]
    __shared__ float slot[8];
    __shared__ __align__(16) int flag[4];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    long wg = blockIdx.x;
    const int td = (int)(wg % tiles_d);
    wg /= tiles_d;
    const int tq = (int)(wg % tiles_q);
    const int bh = (int)(wg / tiles_q);
    const int q0 = tq * kT, d0 = td * kT;

    const float* Ph = P + (size_t)bh * Lq * Lk;
    const float* Vh = V + (size_t)bh * Lk * D;
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(Ph, Lq * Lk * 4);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(Vh, Lk * D * 4);
    const bool p_vec = (Lk & 3) == 0;
    // loaders: P rows lrow + 16 i, keys lcol .. + 3; V keys lrow + 16 i,
    // dims d0 + lcol .. + 3
    const int lrow = tid >> 4, lcol = (tid & 15) * 4;
    float4 pv[4], vv[4];
    auto issue = [&](int kk0) {
        const int kk = kk0 + lcol, d = d0 + lcol;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = q0 + lrow + 16 * i, key = kk0 + lrow + 16 * i;
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
            vv[i] = ld_buf_f4(rv, d < D ? (key * D + d) * 4 : kBufOob);
        }
    };

    // the rare rescaled staging of V for the stage at kk0; returns V's unit
    auto restage = [&](int kk0) -> float {
        float4 v2[4];
        const int d = d0 + lcol;
        float mv = 0.f, unused = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v2[i] = ld_buf_f4(rv, d < D ? ((kk0 + lrow + 16 * i) * D + d) * 4 : kBufOob);
            mv = max_finite4(mv, v2[i]);
        }
        wg_max2(mv, unused, slot);
        const float svs = pow2_scale(mv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ov = (lrow + 16 * i) * kVStr + lcol;
            store_split4(&sv[0][ov], &sv[1][ov], v2[i], svs);
        }
        __syncthreads();
        return pow2_unit(mv);
    };

    v4f sum[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) sum[t] = v4f{0.f, 0.f, 0.f, 0.f};
    issue(0);
    for (int kk0 = 0; kk0 < Lk; kk0 += kStage) {
        if (kk0 > 0) __syncthreads();  // the previous stage's LDS reads are done
        float big = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int op = (lrow + 16 * i) * kStr + lcol;
            store_split4(&sp[0][op], &sp[1][op], pv[i], 1.f);
            const int ov = (lrow + 16 * i) * kVStr + lcol;
            store_split4(&sv[0][ov], &sv[1][ov], vv[i], 1.f);
            big = vmax3abs(vmax3abs(big, vv[i].x, vv[i].y), vv[i].z, vv[i].w);
        }
        const bool over = __ballot(!(big < kF16Range)) != 0;
        if (lane == 0) flag[wave] = over;
        if (kk0 + kStage < Lk) issue(kk0 + kStage);
        __syncthreads();
        float u = 1.f;
        const int4 f = *reinterpret_cast<const int4*>(flag);
        if (f.x | f.y | f.z | f.w) u = restage(kk0);
        v4f acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < kStage / 32; ++b) {
            const int bp = (16 * wave + lr) * kStr + 32 * b + 8 * lg;
            const f16x8 ph = lds8_f16(&sp[0][bp]), pl = lds8_f16(&sp[1][bp]);
            // V^T fragments: keys 32 b + 8 lg + 0..7 of dim 16 t + lr
            const int vrow = 32 * b + 8 * lg + (lr >> 2), vcol = 4 * (lr & 3);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int a = vrow * kVStr + 16 * t + vcol;
                const uint2 h0 = lds_tr16(&sv[0][a]), h1 = lds_tr16(&sv[0][a + 4 * kVStr]);
                const uint2 l0 = lds_tr16(&sv[1][a]), l1 = lds_tr16(&sv[1][a + 4 * kVStr]);
                const f16x8 vh = __builtin_bit_cast(f16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
                const f16x8 vl = __builtin_bit_cast(f16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
                acc[t] = mfma_split(vh, vl, ph, pl, acc[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) sum[t] += acc[t] * u;
    }
    // P's 2^15
#pragma unroll
    for (int t = 0; t < 4; ++t) sum[t] *= 1.0f / 32768.0f;

    const int row = q0 + 16 * wave + lr;
    if (row < Lq) {
        float* orow = O + ((size_t)bh * Lq + row) * D;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int d = d0 + 16 * t + 4 * lg;
            if (d < D)
                *reinterpret_cast<float4*>(orow + d) =
                    make_float4(sum[t][0], sum[t][1], sum[t][2], sum[t][3]);
        }
    }
}

}  // namespace

hipError_t launch_qk_s16(int pek, const float* Q, const float* K, float* S, int BH, int Lq, int Lk,
                         int D, int dchunk, int nsplit, const PeSide& pq, const PeSide& pk,
                         hipStream_t st) {
    const int tiles_q = (Lq + kT - 1) / kT, tiles_k = (Lk + kT - 1) / kT;
    const dim3 grid((unsigned)((long)BH * tiles_q * tiles_k * nsplit)), block(256);
    switch (pek) {
        case kPeNone:
            hipLaunchKernelGGL(k_qk_s16<kPeNone>, grid, block, 0, st, Q, K, S, BH, Lq, Lk, D,
                               dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        case kPeRopeInterleaved:
            hipLaunchKernelGGL(k_qk_s16<kPeRopeInterleaved>, grid, block, 0, st, Q, K, S, BH, Lq,
                               Lk, D, dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        case kPeRopeHalf:
            hipLaunchKernelGGL(k_qk_s16<kPeRopeHalf>, grid, block, 0, st, Q, K, S, BH, Lq, Lk, D,
                               dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        case kPeSinusoidal:
            hipLaunchKernelGGL(k_qk_s16<kPeSinusoidal>, grid, block, 0, st, Q, K, S, BH, Lq, Lk,
                               D, dchunk, nsplit, tiles_q, tiles_k, pq, pk);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_pv_s16(const float* P, const float* V, float* O, int BH, int Lq, int Lk, int D,
                         hipStream_t st) {
    const int tiles_q = (Lq + kT - 1) / kT, tiles_d = (D + kT - 1) / kT;
    hipLaunchKernelGGL(k_pv_s16, dim3((unsigned)((long)BH * tiles_q * tiles_d)), dim3(256), 0, st,
                       P, V, O, Lq, Lk, D, tiles_q, tiles_d);
    return hipGetLastError();
}

}  // namespace atn
