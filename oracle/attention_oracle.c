/*
 * CPU oracle for the large-head-dim SDPA path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the reference project's own CPU attention
 * routines so that the HIP kernels can be checked against them on identical
 * inputs.  It is a checker, never part of the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * the product library never links or calls it.
 *
 * Fidelity rules (they make the restatement reproduce the reference's bits):
 *   - float accumulators, loops in the reference's order (d ascending inside
 *     j ascending inside i), libm expf / powf / sinf / cosf / sqrtf;
 *   - built with -O2 -ffp-contract=off and no -ffast-math, so gcc neither
 *     fuses a*b+c nor reorders the float reductions;
 *   - the per-row arithmetic is identical in the serial and the OpenMP entry
 *     points (parallelism is only over independent output rows), so both
 *     produce the same bits.
 *
 * Each function cites the reference file:line it restates.  Functions whose
 * results no reference golden vector or closed form pins say so below.
 *
 * Pinning (checked by tests/test_oracle_*.py):
 *   oracle_attention          golden vectors in pytorch_reference_data (all 6
 *                             shapes) + closed forms (equal V rows, Q = 0,
 *                             Lk = 1, constant inputs) + fp64 brute force.
 *   oracle_rope_cache,
 *   oracle_apply_rope_interleaved,
 *   oracle_attention_rope     pos-0 identity, per-pair norm preservation,
 *                             rotation composition, rope(Q)/rope(K) through
 *                             oracle_attention, and a float64 re-derivation of
 *                             the angle table.
 *   oracle_apply_rope_half    permutation identity rotate_half = P^-1 o
 *                             interleaved o P (no reference vectors exist).
 *   oracle_sinusoidal_table,
 *   oracle_attention_sinusoidal  PE(pos 0) = [0,1,0,1,...], linearity
 *                             attn_sin(Q,K,V) == attn(Q+PE, K+PE, V).
 *   oracle_rope_freqs,
 *   oracle_sinusoidal_freqs   float64 1/base^(2i/r) and 1/1e4^(2(d/2)/D),
 *                             and the pinned tables' position-1 rows hold
 *                             cos/sin of exactly these frequencies.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* Mutation switch used only by the tests that prove the checks can fail:
 * 0 = faithful; 1 = drop the 1/sqrt(D) scale; 2 = swap sin and cos in the
 * PE/rotation tables; 3 = transpose the rotation (sign of sin flipped);
 * 4 = wrong key position (RoPE: keys start at position 1; sinusoidal: keys
 * take the query's position).  Never set outside tests. */
static int g_mutation = 0;
void oracle_set_mutation(int m) { g_mutation = m; }
int oracle_get_mutation(void) { return g_mutation; }

/* ------------------------------------------------------------------------- */
/* One output row of SDPA: final/attention.cu:241-280 (loop body for fixed
 * b, h, i).  q: [D], k/v: [Lk][D], out: [D], scores: scratch [Lk]. */
static void sdpa_row(const float *q, const float *k, const float *v, float *out,
                     int len_k, int head_d, float scale, float *scores) {
    float max_s = -INFINITY;
    for (int j = 0; j < len_k; j++) {
        const float *kr = k + (size_t)j * head_d;
        float s = 0.0f;
        for (int d = 0; d < head_d; d++) s += q[d] * kr[d];
        s *= scale;
        scores[j] = s;
        max_s = fmaxf(max_s, s);
    }
    float exp_total = 0.0f;
    for (int j = 0; j < len_k; j++) {
        scores[j] = expf(scores[j] - max_s);
        exp_total += scores[j];
    }
    for (int j = 0; j < len_k; j++) scores[j] /= exp_total;
    for (int d = 0; d < head_d; d++) {
        float result = 0.0f;
        for (int j = 0; j < len_k; j++) result += scores[j] * v[(size_t)j * head_d + d];
        out[d] = result;
    }
}

static float sdpa_scale(int head_d) {
    /* final/attention.cu:239 */
    return g_mutation == 1 ? 1.0f : 1.0f / sqrtf((float)head_d);
}

/* Rows [row_begin, row_end) of the flattened (b*H + h)*Lq + i index space.
 * Restates attention_cpu, final/attention.cu:228-283.  Inputs contiguous
 * [B][H][L][D].  nthreads <= 1 runs serially. */
void oracle_attention_rows(const float *Q, const float *K, const float *V, float *out,
                           int B, int H, int Lq, int Lk, int D,
                           long row_begin, long row_end, int nthreads) {
    const float scale = sdpa_scale(D);
    const long total = (long)B * H * Lq;
    if (row_begin < 0) row_begin = 0;
    if (row_end > total) row_end = total;
    (void)nthreads;
#ifdef _OPENMP
    int nt = nthreads > 1 ? nthreads : 1;
#pragma omp parallel num_threads(nt)
#endif
    {
        float *scores = (float *)malloc(sizeof(float) * (size_t)(Lk > 0 ? Lk : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (long r = row_begin; r < row_end; r++) {
            long bh = r / Lq;
            const float *q = Q + (size_t)r * D;
            const float *k = K + (size_t)bh * Lk * D;
            const float *v = V + (size_t)bh * Lk * D;
            sdpa_row(q, k, v, out + (size_t)r * D, Lk, D, scale, scores);
        }
        free(scores);
    }
}

/* attention_cpu, final/attention.cu:228-283 (whole tensor, serial). */
void oracle_attention(const float *Q, const float *K, const float *V, float *out,
                      int B, int H, int Lq, int Lk, int D) {
    oracle_attention_rows(Q, K, V, out, B, H, Lq, Lk, D, 0, (long)B * H * Lq, 1);
}

/* ------------------------------------------------------------------------- */
/* precompute_rope_cache, final/rope.cu:20-40: cache[pos][rotary_dim], each
 * (cos, sin) duplicated at 2i and 2i+1; freq_i = 1/powf(base, 2i/rotary_dim). */
void oracle_rope_cache(float *cos_cache, float *sin_cache, int max_seq_len, int rotary_dim,
                       float base) {
    for (int pos = 0; pos < max_seq_len; pos++) {
        for (int i = 0; i < rotary_dim / 2; i++) {
            float freq = 1.0f / powf(base, (2.0f * i) / rotary_dim);
            float theta = pos * freq;
            float c = cosf(theta), s = sinf(theta);
            if (g_mutation == 2) { float t = c; c = s; s = t; }
            cos_cache[(size_t)pos * rotary_dim + 2 * i] = c;
            cos_cache[(size_t)pos * rotary_dim + 2 * i + 1] = c;
            sin_cache[(size_t)pos * rotary_dim + 2 * i] = s;
            sin_cache[(size_t)pos * rotary_dim + 2 * i + 1] = s;
        }
    }
}

/* Frequencies used by every on-the-fly RoPE variant: the value the reference
 * computes per pair, final/rope.cu:96-98 and :132-134
 * (1/powf(base, (2.0f*i)/rotary_dim)).  freq: [rotary_dim/2]. */
void oracle_rope_freqs(float *freq, int rotary_dim, float base) {
    for (int i = 0; i < rotary_dim / 2; i++) freq[i] = 1.0f / powf(base, (2.0f * i) / rotary_dim);
}

/* apply_rope_cpu, final/rope.cu:1418-1435, generalised to a partial rotary
 * width as in the v7 kernel (final/rope.cu:137-154): dims < rotary_dim are
 * rotated in interleaved pairs (2i, 2i+1) with the cache row of the token's
 * position; dims >= rotary_dim pass through.  cache: [pos][rotary_dim].
 * input/output: [seq_len][hdim]; position of row p is pos0 + p. */
void oracle_apply_rope_interleaved(const float *input, float *output, const float *cos_cache,
                                   const float *sin_cache, int seq_len, int hdim, int rotary_dim,
                                   int pos0) {
    for (int p = 0; p < seq_len; p++) {
        const float *x = input + (size_t)p * hdim;
        float *y = output + (size_t)p * hdim;
        const float *cc = cos_cache + (size_t)(pos0 + p) * rotary_dim;
        const float *sc = sin_cache + (size_t)(pos0 + p) * rotary_dim;
        for (int d = 0; d < rotary_dim; d += 2) {
            float xe = x[d], xo = x[d + 1];
            float c = cc[d], s = sc[d];
            if (g_mutation == 3) s = -s;
            y[d] = xe * c - xo * s;
            y[d + 1] = xe * s + xo * c;
        }
        for (int d = rotary_dim; d < hdim; d++) y[d] = x[d];
    }
}

/* Rotate-half RoPE (pairs (i, i + rotary_dim/2)), with the same frequency,
 * angle and float conventions as the interleaved form above.  The reference
 * has no rotate-half code; this function is defined by the identity
 * rotate_half(x) = P^-1 interleaved(P x), where (P x)[2i] = x[i] and
 * (P x)[2i+1] = x[i + rotary_dim/2] -- the tests check exactly that identity
 * against oracle_apply_rope_interleaved.  cache: [pos][rotary_dim] in the
 * interleaved (duplicated-pair) format of oracle_rope_cache. */
void oracle_apply_rope_half(const float *input, float *output, const float *cos_cache,
                            const float *sin_cache, int seq_len, int hdim, int rotary_dim,
                            int pos0) {
    const int half = rotary_dim / 2;
    for (int p = 0; p < seq_len; p++) {
        const float *x = input + (size_t)p * hdim;
        float *y = output + (size_t)p * hdim;
        const float *cc = cos_cache + (size_t)(pos0 + p) * rotary_dim;
        const float *sc = sin_cache + (size_t)(pos0 + p) * rotary_dim;
        for (int i = 0; i < half; i++) {
            float xa = x[i], xb = x[i + half];
            float c = cc[2 * i], s = sc[2 * i];
            if (g_mutation == 3) s = -s;
            y[i] = xa * c - xb * s;
            y[i + half] = xa * s + xb * c;
        }
        for (int d = rotary_dim; d < hdim; d++) y[d] = x[d];
    }
}

/* attention_rope_cpu, final/rope.cu:1439-1499, extended with: a partial
 * rotary width (v7 semantics), a choice of pairing (0 = interleaved as in
 * the reference, 1 = rotate-half), and per-side switches so the v7 hybrid
 * (K already rotated by the caller, final/rope.cu:102-228) is covered.
 * cos/sin caches: [max(Lq,Lk)][rotary_dim]; positions start at 0 for Q and
 * for K independently (final/rope.cu:129, :1126).  Rows restricted to
 * [row_begin, row_end) of the flattened (bh, i) space. */
void oracle_attention_rope_rows(const float *Q, const float *K, const float *V, float *out,
                                const float *cos_cache, const float *sin_cache, int B, int H,
                                int Lq, int Lk, int D, int rotary_dim, int pairing, int rotate_q,
                                int rotate_k, long row_begin, long row_end, int nthreads) {
    const float scale = sdpa_scale(D);
    const long total = (long)B * H * Lq;
    if (row_begin < 0) row_begin = 0;
    if (row_end > total) row_end = total;
    if (row_end <= row_begin || Lq <= 0) return;
    void (*rot)(const float *, float *, const float *, const float *, int, int, int, int) =
        pairing == 1 ? oracle_apply_rope_half : oracle_apply_rope_interleaved;
    /* mutation 4: key positions start at 1 instead of 0 (an index bug); the
     * caches must then hold Lk + 1 rows */
    const int kpos0 = (g_mutation == 4) ? 1 : 0;
    (void)nthreads;
    float *krot = (float *)malloc(sizeof(float) * (size_t)Lk * D + 4);
    for (long bh = row_begin / Lq; bh <= (row_end - 1) / Lq; bh++) {
        /* K rotated once per head, like final/rope.cu:1459-1463 */
        const float *kh = K + (size_t)bh * Lk * D;
        if (rotate_k) rot(kh, krot, cos_cache, sin_cache, Lk, D, rotary_dim, kpos0);
        else memcpy(krot, kh, sizeof(float) * (size_t)Lk * D);
        const long r0 = bh * Lq > row_begin ? bh * Lq : row_begin;
        const long r1 = (bh + 1) * Lq < row_end ? (bh + 1) * Lq : row_end;
#ifdef _OPENMP
        int nt = nthreads > 1 ? nthreads : 1;
#pragma omp parallel num_threads(nt)
#endif
        {
            float *scores = (float *)malloc(sizeof(float) * (size_t)(Lk > 0 ? Lk : 1));
            float *qrot = (float *)malloc(sizeof(float) * (size_t)D + 4);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
            for (long r = r0; r < r1; r++) {
                const int i = (int)(r - bh * Lq);
                const float *q = Q + (size_t)r * D;
                if (rotate_q) rot(q, qrot, cos_cache, sin_cache, 1, D, rotary_dim, i);
                else memcpy(qrot, q, sizeof(float) * (size_t)D);
                sdpa_row(qrot, krot, V + (size_t)bh * Lk * D, out + (size_t)r * D, Lk, D, scale,
                         scores);
            }
            free(qrot);
            free(scores);
        }
    }
    free(krot);
}

/* attention_rope_cpu, final/rope.cu:1439-1499 (whole tensor, serial,
 * interleaved, rotary = D, cache [pos][D]). */
void oracle_attention_rope(const float *Q, const float *K, const float *V, float *out,
                           const float *cos_cache, const float *sin_cache, int B, int H, int Lq,
                           int Lk, int D) {
    oracle_attention_rope_rows(Q, K, V, out, cos_cache, sin_cache, B, H, Lq, Lk, D, D, 0, 1, 1, 0,
                               (long)B * H * Lq, 1);
}

/* ------------------------------------------------------------------------- */
/* generate_sinusoidal_embeddings_cpu, final/sinusoidal.cu:838-855:
 * tables [pos][hdim], freq index d/2, angle pos*freq, sinf and cosf. */
void oracle_sinusoidal_table(float *sin_table, float *cos_table, int max_seq_len, int hdim) {
    const float base = 10000.0f;
    for (int pos = 0; pos < max_seq_len; pos++) {
        for (int i = 0; i < hdim; i++) {
            float freq = 1.0f / powf(base, (2.0f * (i / 2)) / (float)hdim);
            float angle = pos * freq;
            float s = sinf(angle), c = cosf(angle);
            if (g_mutation == 2) { float t = s; s = c; c = t; }
            sin_table[(size_t)pos * hdim + i] = s;
            cos_table[(size_t)pos * hdim + i] = c;
        }
    }
}

/* Frequencies of the sinusoidal PE per dim (final/sinusoidal.cu:112-114):
 * freq[d] = 1/powf(1e4, 2*(d/2)/D). */
void oracle_sinusoidal_freqs(float *freq, int hdim) {
    for (int d = 0; d < hdim; d++) freq[d] = 1.0f / powf(10000.0f, (2.0f * (d / 2)) / (float)hdim);
}

/* X + PE for rows [0, seq_len) with positions pos0.. (the separate path's
 * apply_sinusoidal_embeddings, final/sinusoidal.cu:714-744, in which even d
 * takes sin and odd d takes cos). */
void oracle_add_sinusoidal(const float *input, float *output, const float *sin_table,
                           const float *cos_table, int seq_len, int hdim, int pos0) {
    for (int p = 0; p < seq_len; p++) {
        const float *st = sin_table + (size_t)(pos0 + p) * hdim;
        const float *ct = cos_table + (size_t)(pos0 + p) * hdim;
        for (int d = 0; d < hdim; d++) {
            float val = input[(size_t)p * hdim + d];
            val += (d % 2 == 0) ? st[d] : ct[d];
            output[(size_t)p * hdim + d] = val;
        }
    }
}

/* attention_sinusoidal_cpu, final/sinusoidal.cu:858-928: PE added to q
 * (row i of the tables) and k (row j) inside the score loop; tables sized to
 * max(Lq, Lk) rows.  add_q/add_k switch each side (the hybrid and separate
 * pipelines of kernels/attention_kernel_sinusoidal_hybrid.cu share these
 * semantics).  Rows restricted to [row_begin, row_end). */
void oracle_attention_sinusoidal_rows(const float *Q, const float *K, const float *V,
                                      const float *sin_table, const float *cos_table, float *out,
                                      int B, int H, int Lq, int Lk, int D, int add_q, int add_k,
                                      long row_begin, long row_end, int nthreads) {
    const float scale = sdpa_scale(D);
    const long total = (long)B * H * Lq;
    if (row_begin < 0) row_begin = 0;
    if (row_end > total) row_end = total;
    (void)nthreads;
#ifdef _OPENMP
    int nt = nthreads > 1 ? nthreads : 1;
#pragma omp parallel num_threads(nt)
#endif
    {
        float *scores = (float *)malloc(sizeof(float) * (size_t)(Lk > 0 ? Lk : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (long r = row_begin; r < row_end; r++) {
            long bh = r / Lq;
            int i = (int)(r - bh * Lq);
            const float *q = Q + (size_t)r * D;
            const float *kb = K + (size_t)bh * Lk * D;
            const float *vb = V + (size_t)bh * Lk * D;
            int qpos = i;
            const float *sq = sin_table + (size_t)qpos * D;
            const float *cq = cos_table + (size_t)qpos * D;
            float max_s = -INFINITY;
            for (int j = 0; j < Lk; j++) {
                const float *k = kb + (size_t)j * D;
                int kpos = (g_mutation == 4) ? i : j;
                const float *sk = sin_table + (size_t)kpos * D;
                const float *ck = cos_table + (size_t)kpos * D;
                float s = 0.0f;
                for (int d = 0; d < D; d++) {
                    float q_val = q[d];
                    float k_val = k[d];
                    if (d % 2 == 0) {
                        if (add_q) q_val += sq[d];
                        if (add_k) k_val += sk[d];
                    } else {
                        if (add_q) q_val += cq[d];
                        if (add_k) k_val += ck[d];
                    }
                    s += q_val * k_val;
                }
                s *= scale;
                scores[j] = s;
                max_s = fmaxf(max_s, s);
            }
            float exp_total = 0.0f;
            for (int j = 0; j < Lk; j++) {
                scores[j] = expf(scores[j] - max_s);
                exp_total += scores[j];
            }
            for (int j = 0; j < Lk; j++) scores[j] /= exp_total;
            float *o = out + (size_t)r * D;
            for (int d = 0; d < D; d++) {
                float result = 0.0f;
                for (int j = 0; j < Lk; j++) result += scores[j] * vb[(size_t)j * D + d];
                o[d] = result;
            }
        }
        free(scores);
    }
}

/* attention_sinusoidal_cpu, final/sinusoidal.cu:858-928 (whole tensor). */
void oracle_attention_sinusoidal(const float *Q, const float *K, const float *V,
                                 const float *sin_table, const float *cos_table, float *out,
                                 int B, int H, int Lq, int Lk, int D) {
    oracle_attention_sinusoidal_rows(Q, K, V, sin_table, cos_table, out, B, H, Lq, Lk, D, 1, 1, 0,
                                     (long)B * H * Lq, 1);
}

/* ------------------------------------------------------------------------- */
/* fp32 -> bf16 round-to-nearest-even and back (the closed form the bf16
 * kernels' inputs are built with); NaN is kept quiet. */
void oracle_f32_to_bf16(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint32_t u;
        memcpy(&u, &in[i], 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) {
            out[i] = (uint16_t)((u >> 16) | 0x40);
        } else {
            uint32_t lsb = (u >> 16) & 1u;
            out[i] = (uint16_t)((u + 0x7fffu + lsb) >> 16);
        }
    }
}

void oracle_bf16_to_f32(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint32_t u = (uint32_t)in[i] << 16;
        memcpy(&out[i], &u, 4);
    }
}

int oracle_openmp_enabled(void) {
#ifdef _OPENMP
    return 1;
#else
    return 0;
#endif
}
