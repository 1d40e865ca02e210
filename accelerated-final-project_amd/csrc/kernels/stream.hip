// Split-D streaming attention for any shape (gfx950).
//
// Attention with head_dim D much larger than the sequence lengths is a
// bandwidth problem: per (b,h) the score matrix is only Lq x Lk while Q, K
// and V are Lq x D / Lk x D.  One workgroup per query row (the reference's
// launch, final/attention.cu:209-215) re-streams all of K and V per query and
// keeps <= 64 of 256 threads busy; here the work is cut along D instead:
//
//   stage 1  k_qk_partial  S_part[split][bh][i][j] = sum_{d in chunk} q~_id k~_jd
//            (q~, k~ = Q/K with the positional encoding applied at load), one
//            workgroup per (bh, 64x64 score tile, D-chunk) -- every Q/K element
//            is read once when the tile covers Lq x Lk;
//   stage 2  k_softmax     P = softmax(scale * sum_split S_part) per row, exact
//            (max, exp, sum, divide -- final/attention.cu:262-270 order),
//            written scaled by 2^15 (p / (l 2^-15) = 2^15 (p / l) exactly), so
//            that the 16-bit PV operands keep small probabilities' bits;
//   stage 3  k_pv          O[bh][i][d] = sum_j P_ij V_jd, one workgroup per
//            (bh, 64 rows, 64 dims) -- every V element is read once per
//            64-row query block.
//
// All math is fp32; bf16 storage is widened at load and rounded (RNE) once
// at the final store.  Workgroups are 256 threads (4 waves) computing 64x64
// tiles, a 32x32 quadrant per wave on fp32 MFMA, from LDS-staged 32-deep
// slices.  fp32 calls with head_d % 4 == 0 and 16-byte aligned bases run
// stages 1 and 3 on 16-bit MFMA instead (stream16.hip); these kernels serve
// bf16 (head_d % 8 != 0 or misaligned), odd head dims and misaligned fp32.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace atn {

namespace {

constexpr int kTile = 64;   // rows x cols of an output tile
constexpr int kDepth = 32;  // contraction slice staged in LDS per step (loaded in two halves)
constexpr int kPad = 4;     // LDS row padding (floats), keeps float4 alignment
constexpr float kPInv = 1.0f / 32768.0f;  // P is stored times 2^15

typedef float v16f __attribute__((ext_vector_type(16)));

// One kDepth-deep slice of a 64 x 64 tile on fp32 MFMA: wave w owns the 32 x 32
// quadrant (wm, wn) = (32 (w / 2), 32 (w % 2)); As[k][row] and Bs[k][col]
// hold the slice k-major.  v_mfma_f32_32x32x2f32 takes A[row][k] from lane
// row + 32 k and B[k][col] from lane col + 32 k, one float each (fp32
// products, fp32 accumulation, twice the VALU fp32 rate).
__device__ __forceinline__ void mfma_slice(const float (*As)[kTile + kPad],
                                           const float (*Bs)[kTile + kPad], int wm, int wn,
                                           int lane, v16f& acc) {
    const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
    for (int k2 = 0; k2 < kDepth / 2; ++k2) {
        const float a = As[2 * k2 + lh][wm + lr];
        const float b = Bs[2 * k2 + lh][wn + lr];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    }
}

// Row of the tile held in accumulator register r of the lane (its column is
// wn + lane % 32).
__device__ __forceinline__ int mfma_row(int wm, int lane, int r) {
    return wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

template <typename T, int PEK>
__global__ __launch_bounds__(256) void k_qk_partial(const T* __restrict__ Q,
                                                     const T* __restrict__ K,
                                                     float* __restrict__ S, int BH, int Lq, int Lk,
                                                     int D, int dchunk, int nsplit, int tiles_q,
                                                     int tiles_k, PeSide pq, PeSide pk,
                                                     int vec_ok) {
    __shared__ float Qs[kDepth][kTile + kPad];
    __shared__ float Ks[kDepth][kTile + kPad];

    const int tid = threadIdx.x;
    long wg = blockIdx.x;
    const int split = (int)(wg % nsplit);
    wg /= nsplit;
    const int tk = (int)(wg % tiles_k);
    wg /= tiles_k;
    const int tq = (int)(wg % tiles_q);
    const int bh = (int)(wg / tiles_q);

    const int q0 = tq * kTile, k0 = tk * kTile;
    const int dbeg = split * dchunk;
    const int dend = min(D, dbeg + dchunk);

    const int lrow = tid >> 2;       // loader: row within tile
    const int lcol = (tid & 3) * 4;  // loader: first of 4 depth slots
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;

    const int qi = q0 + lrow, kj = k0 + lrow;
    const T* qrow = Q + ((size_t)bh * Lq + (qi < Lq ? qi : 0)) * D;
    const T* krow = K + ((size_t)bh * Lk + (kj < Lk ? kj : 0)) * D;
    const bool vec = vec_ok != 0;

    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;

    for (int d0 = dbeg; d0 < dend; d0 += kDepth) {
        float4 qv[2], kv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            qv[h] = make_float4(0.f, 0.f, 0.f, 0.f);
            kv[h] = qv[h];
            const int d = d0 + 16 * h + lcol;
            if (qi < Lq) qv[h] = load_row4_pe<T, PEK>(qrow, qi, d, dend, pq, vec);
            if (kj < Lk) kv[h] = load_row4_pe<T, PEK>(krow, kj, d, dend, pk, vec);
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = 16 * h + lcol;
            Qs[r + 0][lrow] = qv[h].x; Qs[r + 1][lrow] = qv[h].y;
            Qs[r + 2][lrow] = qv[h].z; Qs[r + 3][lrow] = qv[h].w;
            Ks[r + 0][lrow] = kv[h].x; Ks[r + 1][lrow] = kv[h].y;
            Ks[r + 2][lrow] = kv[h].z; Ks[r + 3][lrow] = kv[h].w;
        }
        __syncthreads();
        mfma_slice(Qs, Ks, wm, wn, lane, acc);
    }

    float* Sp = S + ((size_t)split * BH + bh) * (size_t)Lq * Lk;
    const int c = k0 + wn + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = q0 + mfma_row(wm, lane, r);
        if (row < Lq && c < Lk) Sp[(size_t)row * Lk + c] = acc[r];
    }
}

// One workgroup per score row.  Separate LDS slots for the max and the sum
// reductions, so the second reduction never overwrites a slot the first may
// still be reading.
__global__ __launch_bounds__(256) void k_softmax(const float* __restrict__ S, float* P, long rows,
                                                  int Lk, int nsplit, size_t split_stride,
                                                  float scale) {
    __shared__ float red_max[4];
    __shared__ float red_sum[4];
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;

    for (long r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* s = S + (size_t)r * Lk;
        float* p = P + (size_t)r * Lk;
        float m = -INFINITY;
        for (int j = tid; j < Lk; j += 256) {
            float acc = s[j];
            for (int sp = 1; sp < nsplit; ++sp) acc += s[(size_t)sp * split_stride + j];
            acc *= scale;
            p[j] = acc;
            m = fmaxf(m, acc);
        }
        m = wave_max(m);
        if (lane == 0) red_max[wid] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red_max[0], red_max[1]), fmaxf(red_max[2], red_max[3]));

        float l = 0.f;
        for (int j = tid; j < Lk; j += 256) {
            const float e = expf(p[j] - m);
            p[j] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) red_sum[wid] = l;
        __syncthreads();
        l = (red_sum[0] + red_sum[1]) + (red_sum[2] + red_sum[3]);
        const float l15 = l * kPInv;  // P written times 2^15 (exact)
        for (int j = tid; j < Lk; j += 256) p[j] = p[j] / l15;
        __syncthreads();  // red_* reused by the next row
    }
}

// Rows of at most 64 NPL keys: one wave per row, the row in registers (lane
// l holds keys l + 64 u), so the scores are read once and P written once;
// four rows per workgroup.
template <int NPL>
__global__ __launch_bounds__(256) void k_softmax_rows(const float* __restrict__ S, float* P,
                                                      long rows, int Lk, int nsplit,
                                                      size_t split_stride, float scale) {
    const int lane = threadIdx.x & 63;
    const long wave = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    for (long r = wave; r < rows; r += (long)gridDim.x * 4) {
        const float* s = S + (size_t)r * Lk;
        float* p = P + (size_t)r * Lk;
        float v[NPL];
        float m = -INFINITY;
#pragma unroll
        for (int u = 0; u < NPL; ++u) {
            const int j = lane + 64 * u;
            float acc = -INFINITY;
            if (j < Lk) {
                acc = s[j];
                for (int sp = 1; sp < nsplit; ++sp) acc += s[(size_t)sp * split_stride + j];
                acc *= scale;
            }
            v[u] = acc;
            m = fmaxf(m, acc);
        }
        m = wave_max(m);
        float l = 0.f;
#pragma unroll
        for (int u = 0; u < NPL; ++u) {
            v[u] = lane + 64 * u < Lk ? expf(v[u] - m) : 0.f;
            l += v[u];
        }
        l = wave_sum(l) * kPInv;  // P written times 2^15 (exact)
#pragma unroll
        for (int u = 0; u < NPL; ++u) {
            const int j = lane + 64 * u;
            if (j < Lk) p[j] = v[u] / l;
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_pv(const float* __restrict__ P, const T* __restrict__ V,
                                             T* __restrict__ O, int Lq, int Lk, int D,
                                             int tiles_q, int tiles_d, int vec_ok) {
    __shared__ float Ps[kDepth][kTile + kPad];  // [key][row]
    __shared__ float Vs[kDepth][kTile + kPad];  // [key][dim]

    const int tid = threadIdx.x;
    long wg = blockIdx.x;
    const int td = (int)(wg % tiles_d);
    wg /= tiles_d;
    const int tq = (int)(wg % tiles_q);
    const int bh = (int)(wg / tiles_q);
    const int q0 = tq * kTile, d0 = td * kTile;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;

    // P loader: 64 rows x 16 keys, 4 keys per thread
    const int prow = tid >> 2, pk = (tid & 3) * 4;
    // V loader: 16 keys x 64 dims, 4 dims per thread
    const int vkey = tid >> 4, vd = (tid & 15) * 4;
    const bool vec = vec_ok != 0;
    const bool p_vec = (Lk & 3) == 0;

    const float* prow_ptr = P + ((size_t)bh * Lq + (q0 + prow < Lq ? q0 + prow : 0)) * Lk;
    const T* Vh = V + (size_t)bh * Lk * D;

    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;

    for (int k0 = 0; k0 < Lk; k0 += kDepth) {
        float pv[2][4], vv[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int c = 0; c < 4; ++c) pv[h][c] = vv[h][c] = 0.f;
            if (q0 + prow < Lq) {
                const int kk = k0 + 16 * h + pk;
                if (p_vec && kk + 3 < Lk) {
                    const float4 t = *reinterpret_cast<const float4*>(prow_ptr + kk);
                    pv[h][0] = t.x; pv[h][1] = t.y; pv[h][2] = t.z; pv[h][3] = t.w;
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (kk + c < Lk) pv[h][c] = prow_ptr[kk + c];
                }
            }
            const int key = k0 + 16 * h + vkey;
            if (key < Lk) {
                const T* vr = Vh + (size_t)key * D;
                const int dd = d0 + vd;
                if (vec && dd + 3 < D) {
                    const float4 t = Elem<T>::ld4(vr, dd);
                    vv[h][0] = t.x; vv[h][1] = t.y; vv[h][2] = t.z; vv[h][3] = t.w;
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (dd + c < D) vv[h][c] = Elem<T>::ld(vr, dd + c);
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int c = 0; c < 4; ++c) Ps[16 * h + pk + c][prow] = pv[h][c];
            *reinterpret_cast<float4*>(&Vs[16 * h + vkey][vd]) =
                make_float4(vv[h][0], vv[h][1], vv[h][2], vv[h][3]);
        }
        __syncthreads();
        mfma_slice(Ps, Vs, wm, wn, lane, acc);
    }

    const int dd = d0 + wn + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = q0 + mfma_row(wm, lane, r);
        if (row < Lq && dd < D)
            Elem<T>::st(O + ((size_t)bh * Lq + row) * D, dd, acc[r] * kPInv);  // P's 2^15
    }
}

// Positional-encoding pre-pass: out[row] = PE(in[row]) with position
// row % seq_len (the "separate"/"hybrid" pipelines' pre-pass).
template <typename T, int PEK>
__global__ __launch_bounds__(256) void k_pe_apply(const T* __restrict__ in, T* __restrict__ out,
                                                   long n_rows, int seq_len, int D, PeSide pe,
                                                   int vec_ok) {
    const bool vec = vec_ok != 0;
    for (long row = blockIdx.x; row < n_rows; row += gridDim.x) {
        const int pos = (int)(row % seq_len);
        const T* xr = in + (size_t)row * D;
        T* yr = out + (size_t)row * D;
        for (int d = threadIdx.x * 4; d < D; d += 256 * 4) {
            const float4 v = load_row4_pe<T, PEK>(xr, pos, d, D, pe, vec);
            if (vec && d + 3 < D) {
                Elem<T>::st4(yr, d, v);
            } else {
                const float vv[4] = {v.x, v.y, v.z, v.w};
                for (int c = 0; c < 4 && d + c < D; ++c) Elem<T>::st(yr, d + c, vv[c]);
            }
        }
    }
}

template <typename T>
hipError_t qk_partial_t(int pek, const void* Q, const void* K, float* S, int BH, int Lq, int Lk,
                        int D, int dchunk, int nsplit, const PeSide& pq, const PeSide& pk,
                        int vec_ok, hipStream_t st) {
    const int tiles_q = (Lq + kTile - 1) / kTile, tiles_k = (Lk + kTile - 1) / kTile;
    const long nwg = (long)BH * tiles_q * tiles_k * nsplit;
    const T* q = static_cast<const T*>(Q);
    const T* k = static_cast<const T*>(K);
    const dim3 grid((unsigned)nwg), block(256);
    switch (pek) {
        case kPeNone:
            hipLaunchKernelGGL((k_qk_partial<T, kPeNone>), grid, block, 0, st, q, k, S, BH, Lq, Lk,
                               D, dchunk, nsplit, tiles_q, tiles_k, pq, pk, vec_ok);
            break;
        case kPeRopeInterleaved:
            hipLaunchKernelGGL((k_qk_partial<T, kPeRopeInterleaved>), grid, block, 0, st, q, k, S,
                               BH, Lq, Lk, D, dchunk, nsplit, tiles_q, tiles_k, pq, pk, vec_ok);
            break;
        case kPeRopeHalf:
            hipLaunchKernelGGL((k_qk_partial<T, kPeRopeHalf>), grid, block, 0, st, q, k, S, BH, Lq,
                               Lk, D, dchunk, nsplit, tiles_q, tiles_k, pq, pk, vec_ok);
            break;
        case kPeSinusoidal:
            hipLaunchKernelGGL((k_qk_partial<T, kPeSinusoidal>), grid, block, 0, st, q, k, S, BH,
                               Lq, Lk, D, dchunk, nsplit, tiles_q, tiles_k, pq, pk, vec_ok);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t pe_apply_t(int pek, const void* in, void* out, long n_rows, int seq_len, int D,
                      const PeSide& pe, int vec_ok, hipStream_t st) {
    const long nwg = n_rows < 65536 ? n_rows : 65536;
    const T* x = static_cast<const T*>(in);
    T* y = static_cast<T*>(out);
    const dim3 grid((unsigned)nwg), block(256);
    switch (pek) {
        case kPeRopeInterleaved:
            hipLaunchKernelGGL((k_pe_apply<T, kPeRopeInterleaved>), grid, block, 0, st, x, y,
                               n_rows, seq_len, D, pe, vec_ok);
            break;
        case kPeRopeHalf:
            hipLaunchKernelGGL((k_pe_apply<T, kPeRopeHalf>), grid, block, 0, st, x, y, n_rows,
                               seq_len, D, pe, vec_ok);
            break;
        case kPeSinusoidal:
            hipLaunchKernelGGL((k_pe_apply<T, kPeSinusoidal>), grid, block, 0, st, x, y, n_rows,
                               seq_len, D, pe, vec_ok);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

// fp32 with head_d % 4 == 0 and 16-byte aligned bases takes the 16-bit
// MFMA forms (stream16.hip), while every per-head byte offset fits the
// 32-bit buffer offsets they use.
static bool s16_ok(int dtype, int vec_ok, int Lq, int Lk, int D) {
    const long long lim = 1LL << 31;
    return dtype == kDtypeF32 && vec_ok && D % 4 == 0 && (long long)Lq * D * 4 < lim &&
           (long long)Lk * D * 4 < lim && (long long)Lq * Lk * 4 < lim;
}

hipError_t launch_qk_partial(int dtype, int pek, const void* Q, const void* K, float* S, int BH,
                             int Lq, int Lk, int D, int dchunk, int nsplit, const PeSide& pq,
                             const PeSide& pk, int vec_ok, hipStream_t st) {
    if (s16_ok(dtype, vec_ok, Lq, Lk, D))
        return launch_qk_s16(pek, static_cast<const float*>(Q), static_cast<const float*>(K), S,
                             BH, Lq, Lk, D, dchunk, nsplit, pq, pk, st);
    if (dtype == kDtypeF32)
        return qk_partial_t<float>(pek, Q, K, S, BH, Lq, Lk, D, dchunk, nsplit, pq, pk, vec_ok,
                                   st);
    return qk_partial_t<uint16_t>(pek, Q, K, S, BH, Lq, Lk, D, dchunk, nsplit, pq, pk, vec_ok, st);
}

hipError_t launch_softmax(const float* S, float* P, long rows, int Lk, int nsplit,
                          size_t split_stride, float scale, hipStream_t st) {
    // a wave per row pays off where each element is one partial; summing many
    // D-chunks' partials wants more threads per row (the kernel below)
    if (Lk <= 64 * 32 && nsplit == 1) {
        const long nwg = std::min<long>((rows + 3) / 4, 65536);
        const dim3 grid((unsigned)nwg), block(256);
        if (Lk <= 64 * 4)
            hipLaunchKernelGGL(k_softmax_rows<4>, grid, block, 0, st, S, P, rows, Lk, nsplit,
                               split_stride, scale);
        else if (Lk <= 64 * 8)
            hipLaunchKernelGGL(k_softmax_rows<8>, grid, block, 0, st, S, P, rows, Lk, nsplit,
                               split_stride, scale);
        else if (Lk <= 64 * 16)
            hipLaunchKernelGGL(k_softmax_rows<16>, grid, block, 0, st, S, P, rows, Lk, nsplit,
                               split_stride, scale);
        else
            hipLaunchKernelGGL(k_softmax_rows<32>, grid, block, 0, st, S, P, rows, Lk, nsplit,
                               split_stride, scale);
        return hipGetLastError();
    }
    const long nwg = rows < 65536 ? rows : 65536;
    hipLaunchKernelGGL(k_softmax, dim3((unsigned)nwg), dim3(256), 0, st, S, P, rows, Lk, nsplit,
                       split_stride, scale);
    return hipGetLastError();
}

hipError_t launch_pv(int dtype, const float* P, const void* V, void* O, int BH, int Lq, int Lk,
                     int D, int vec_ok, hipStream_t st) {
    if (s16_ok(dtype, vec_ok, Lq, Lk, D))
        return launch_pv_s16(P, static_cast<const float*>(V), static_cast<float*>(O), BH, Lq, Lk,
                             D, st);
    const int tiles_q = (Lq + kTile - 1) / kTile, tiles_d = (D + kTile - 1) / kTile;
    const dim3 grid((unsigned)((long)BH * tiles_q * tiles_d)), block(256);
    if (dtype == kDtypeF32) {
        hipLaunchKernelGGL((k_pv<float>), grid, block, 0, st, P, static_cast<const float*>(V),
                           static_cast<float*>(O), Lq, Lk, D, tiles_q, tiles_d, vec_ok);
    } else {
        hipLaunchKernelGGL((k_pv<uint16_t>), grid, block, 0, st, P,
                           static_cast<const uint16_t*>(V), static_cast<uint16_t*>(O), Lq, Lk, D,
                           tiles_q, tiles_d, vec_ok);
    }
    return hipGetLastError();
}

hipError_t launch_pe_apply(int dtype, int pek, const void* in, void* out, long n_rows,
                           int seq_len, int D, const PeSide& pe, int vec_ok, hipStream_t st) {
    if (dtype == kDtypeF32)
        return pe_apply_t<float>(pek, in, out, n_rows, seq_len, D, pe, vec_ok, st);
    return pe_apply_t<uint16_t>(pek, in, out, n_rows, seq_len, D, pe, vec_ok, st);
}

}  // namespace atn
