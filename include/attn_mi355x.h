/*
 * attn_mi355x.h -- C ABI of the MI355X (gfx950) large-head-dim attention library.
 *
 * Drop-in entry points keep the reference project's names, argument order and
 * semantics (agoel2005/accelerated-final-project, cited as file:line):
 *   - all tensors are device pointers, contiguous [batch][heads][len][head_d];
 *   - scale = 1/sqrtf(head_d) (also for RoPE, final/rope.cu:234); no mask;
 *   - positions run 0..len-1 independently for Q and for K;
 *   - RoPE and sinusoidal bases are 10000;
 *   - the call is synchronous (the reference ends every launcher with
 *     cudaDeviceSynchronize, final/attention.cu:219-220) and, on any error,
 *     prints "attn_mi355x error <code> (<text>) at <entry point>" to stderr
 *     and calls exit(EXIT_FAILURE) like the reference's CUDA_CHECK
 *     (final/attention.cu:12-21) -- except for a timed-out wait of the
 *     single-launch kernel (ATN_ERR_DEVICE_TIMEOUT: other work held CUs its
 *     grid needed), after which an attention call runs once more on kernels
 *     that wait on no other workgroup and exits only if that fails too.
 * The atn_*_ex entry points are the asynchronous, non-exiting forms: they
 * validate every argument before any HIP call, return an ATN_* status and
 * enqueue on the given stream (a hipStream_t passed as void*; NULL = the
 * null stream).
 *
 * bf16 tensors are raw bfloat16 bits (uint16_t), the upper half of an IEEE
 * float32; conversions round to nearest even.  Arithmetic is fp32 throughout
 * (accumulation, softmax), bf16 outputs are rounded once at the end.
 *
 * Buffers are owned by the caller.  `out` must not alias an input.  Pointers
 * need only element alignment; 16-byte (fp32) / 8-byte (bf16) alignment with
 * head_d % 4 == 0 selects the vector-load path.
 */
#ifndef ATTN_MI355X_H
#define ATTN_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t atn_bf16;

/* ---- status codes (returned by every atn_*_ex function) ---- */
#define ATN_OK 0
#define ATN_ERR_NULL_POINTER (-1)   /* a required pointer is NULL */
#define ATN_ERR_BAD_DIMENSION (-2)  /* a size is < 1 */
#define ATN_ERR_BAD_ROTARY (-3)     /* rotary_dim odd, < 2 or > head_d */
#define ATN_ERR_SIZE_OVERFLOW (-4)  /* an element count overflows 63 bits */
#define ATN_ERR_ALIASING (-5)       /* out overlaps an input */
#define ATN_ERR_NO_DEVICE (-6)      /* no HIP device is visible */
#define ATN_ERR_HIP (-7)            /* a HIP runtime call failed */
#define ATN_ERR_WORKSPACE (-8)      /* caller workspace too small */
#define ATN_ERR_BAD_ARGUMENT (-9)   /* enum out of range, bad table size ... */
#define ATN_ERR_MISALIGNED (-10)    /* pointer not aligned to its element size */
#define ATN_ERR_DEVICE_TIMEOUT (-11) /* a kernel's bounded cross-workgroup wait expired */
#define ATN_ERR_CAPTURE (-12)        /* a library allocation was needed during graph capture */
#define ATN_ERR_SCRATCH_LIMIT (-13)  /* shape needs more than the allocation-free scratch */
#define ATN_ERR_NOT_PREPARED (-14)   /* encoding tables not built (atn_prepare_pe_ex) */

/* Text for a status code (static storage). */
const char *atn_status_string(int status);
/* hipError_t of the last failing HIP call in this thread (0 if none). */
int atn_last_hip_error(void);

/* ---- enums of the _ex interface ---- */
#define ATN_DTYPE_F32 0
#define ATN_DTYPE_BF16 1

#define ATN_PE_NONE 0
#define ATN_PE_ROPE 1
#define ATN_PE_SINUSOIDAL 2

#define ATN_ROPE_INTERLEAVED 0 /* pairs (2i, 2i+1): every reference RoPE kernel */
#define ATN_ROPE_HALF 1        /* pairs (i, i + rotary_dim/2) */

/* Positional encoding applied to Q and/or K inside the attention call.
 * Angles: RoPE theta(pos, i) = pos * (1/powf(base, (2i)/rotary_dim));
 * sinusoidal angle(pos, d) = pos * (1/powf(10000, 2*(d/2)/head_d)), even d
 * adds sin, odd d adds cos (final/sinusoidal.cu:838-855).
 * Tables: NULL = the library builds its own (host libm, uploaded once per
 * device and shape, then cached); or the caller's device tables in the
 * reference formats -- RoPE cos/sin caches [pos][rotary_dim] with values
 * duplicated at 2i and 2i+1 (final/rope.cu:20-40), sinusoidal sin/cos
 * tables [pos][head_d] (final/sinusoidal.cu:838-855); they need at least
 * max(len_q, len_k) rows. */
typedef struct atn_pe_desc {
    int kind;          /* ATN_PE_* */
    int pairing;       /* RoPE: ATN_ROPE_* */
    int rotary_dim;    /* RoPE: rotated width (even, <= head_d); 0 = head_d */
    int apply_q;       /* nonzero: encode Q */
    int apply_k;       /* nonzero: encode K */
    float base;        /* RoPE base; 0 = 10000 (sinusoidal is always 10000) */
    const float *table_a; /* RoPE cos cache / sinusoidal sin table, or NULL */
    const float *table_b; /* RoPE sin cache / sinusoidal cos table, or NULL */
} atn_pe_desc;

/* ==================== drop-in entry points (synchronous) ==================== */

/* fp32 fused SDPA.  Replaces attention_forward_optimized,
 * final/attention.cu:195-221 (kernel :84-191); the dispatcher copy in
 * kernels/attention_kernel.cu:304-336 has the same contract. */
void attention_forward_optimized(const float *Q, const float *K, const float *V, float *out,
                                 int batch_sz, int num_heads, int len_q, int len_k, int head_d);

/* Small-head-dim path of the reference dispatcher: attention_forward,
 * kernels/attention_kernel.cu:339-365.  Same results as above. */
void attention_forward(const float *Q, const float *K, const float *V, float *out, int batch_sz,
                       int num_heads, int len_q, int len_k, int head_d);

/* fp32 RoPE, full fusion with caller caches [pos][head_d] (interleaved,
 * rotary = head_d): attention_forward_rope_fused, final/rope.cu:1209-1238
 * (kernel :1058-1207). */
void attention_forward_rope_fused(const float *Q, const float *K, const float *V, float *out,
                                  const float *cos_cache, const float *sin_cache, int batch_sz,
                                  int num_heads, int len_q, int len_k, int head_d);

/* fp32 RoPE v7 hybrid: Q rotated in-kernel (interleaved, partial
 * rotary_dim, base 10000), K already rotated by the caller:
 * attention_forward_rope_fused_v7_hybrid, final/rope.cu:230-247
 * (kernel :102-228). */
void attention_forward_rope_fused_v7_hybrid(const float *Q, const float *K_rotated,
                                            const float *V, float *out, int batch_sz,
                                            int num_heads, int len_q, int len_k, int head_d,
                                            int rotary_dim);

/* fp32 RoPE "separate" pipeline: pre-pass Q->Q_rope, K->K_rope with caller
 * caches [pos][rotary_dim], then plain attention:
 * attention_forward_separate_rope, final/rope.cu:1379-1416.  Position of a
 * token is its row index within its sequence (the reference's rope_kernel
 * uses token % 64, final/rope.cu:1257, correct only for len = 64). */
void attention_forward_separate_rope(const float *Q, const float *K, const float *V,
                                     float *Q_rope, float *K_rope, float *out,
                                     const float *cos_cache, const float *sin_cache, int batch_sz,
                                     int num_heads, int len_q, int len_k, int head_d,
                                     int rotary_dim);

/* RoPE pre-pass over total_tokens rows of head_d (interleaved, dims >=
 * rotary_dim copied), position = token % seq_len: replaces the rope_kernel
 * launch of final/rope.cu:1240-1280 (whose position is token % 64). */
void rope_forward(const float *input, float *output, const float *cos_cache,
                  const float *sin_cache, int total_tokens, int hdim, int rotary_dim,
                  int seq_len);

/* Sinusoidal PE pre-pass: output = input + PE(token % seqlen) with caller
 * tables [pos][hdim]: replaces the apply_sinusoidal_embeddings launch,
 * final/sinusoidal.cu:714-744 (same argument order). */
void apply_sinusoidal_embeddings(const float *input, const float *sin_table,
                                 const float *cos_table, float *output, int total_tokens,
                                 int hdim, int seqlen);

/* fp32 sinusoidal V5 full fusion (PE computed for q and k inside the call):
 * the reference launches attention_fwd_kernel_sinusoidal_fused_v5 directly
 * (final/sinusoidal.cu:82-234, launch :1135-1137); this is its host form. */
void attention_forward_sinusoidal_fused(const float *Q, const float *K, const float *V,
                                        float *out, int batch_sz, int num_heads, int len_q,
                                        int len_k, int head_d);

/* fp32 sinusoidal hybrid: K_emb = K + PE (pre-pass), Q + PE fused, caller
 * tables [pos][head_d]: attention_forward_sinusoidal_hybrid,
 * kernels/attention_kernel_sinusoidal_hybrid.cu:282-315. */
void attention_forward_sinusoidal_hybrid(const float *Q, const float *K, const float *V,
                                         const float *sin_table, const float *cos_table,
                                         float *K_emb, float *out, int batch_sz, int num_heads,
                                         int len_q, int len_k, int head_d);

/* fp32 sinusoidal separate: Q_emb, K_emb pre-passes then plain attention:
 * attention_forward_sinusoidal_separate,
 * kernels/attention_kernel_sinusoidal_hybrid.cu:465-502. */
void attention_forward_sinusoidal_separate(const float *Q, const float *K, const float *V,
                                           const float *sin_table, const float *cos_table,
                                           float *Q_emb, float *K_emb, float *out, int batch_sz,
                                           int num_heads, int len_q, int len_k, int head_d);

/* bf16 SDPA (fp32 math): attention_forward_bf16,
 * kernels/attention_bf16_optimized_fused.cu:493-505 (kernel :80-180). */
void attention_forward_bf16(const atn_bf16 *Q, const atn_bf16 *K, const atn_bf16 *V,
                            atn_bf16 *out, int bs, int nh, int len_q, int len_k, int head_d);

/* bf16 RoPE v7 form (K pre-rotated, Q rotated in-kernel, partial
 * rotary_dim): attention_forward_rope_bf16,
 * kernels/attention_bf16_optimized_fused.cu:507-519 (kernel :186-321). */
void attention_forward_rope_bf16(const atn_bf16 *Q, const atn_bf16 *K_rotated,
                                 const atn_bf16 *V, atn_bf16 *out, int bs, int nh, int len_q,
                                 int len_k, int head_d, int rotary_dim);

/* bf16 RoPE full fusion (Q and K rotated in-kernel, interleaved, rotary =
 * head_d, base 10000).  The reference exports this form under the same name
 * as the v7 one (kernels/attention_bf16_all_kernels.cu:451-466, kernel
 * :211-323); it is exported here under a distinct name. */
void attention_forward_rope_fused_bf16(const atn_bf16 *Q, const atn_bf16 *K, const atn_bf16 *V,
                                       atn_bf16 *out, int bs, int nh, int len_q, int len_k,
                                       int head_d);

/* bf16 sinusoidal V5: attention_forward_sinusoidal_bf16,
 * kernels/attention_bf16_optimized_fused.cu:521-533 (kernel :327-487). */
void attention_forward_sinusoidal_bf16(const atn_bf16 *Q, const atn_bf16 *K, const atn_bf16 *V,
                                       atn_bf16 *out, int bs, int nh, int len_q, int len_k,
                                       int head_d);

/* Host-side table builders in the reference's formats (host memory):
 * precompute_rope_cache, final/rope.cu:20-40; the sinusoidal table of
 * generate_sinusoidal_embeddings_cpu, final/sinusoidal.cu:838-855
 * (= precompute_sinusoidal_table, kernels/attention_kernel_sinusoidal_hybrid.cu:75-87). */
void precompute_rope_cache(float *cos_cache, float *sin_cache, int max_seq_len, int rotary_dim,
                           float base);
void precompute_sinusoidal_table(float *sin_table, float *cos_table, int seqlen, int hdim);

/* ==================== asynchronous, status-returning forms ==================== */

/* General fused attention: dtype ATN_DTYPE_*, optional positional encoding
 * (pe == NULL: plain SDPA).  workspace == NULL: library-managed scratch, one
 * per (device, stream), allocated zero-filled on first use and grown as
 * needed; else caller scratch of at least atn_attention_workspace_bytes(...)
 * bytes that was zero-filled once before its first use (its first 40 KiB
 * then hold synchronization words that stay valid from call to call, so it
 * must not be re-initialized while in use).  Calls that run at the same
 * time must not share a workspace.  Enqueued on stream; asynchronous; the
 * enqueued work may be captured into a HIP graph and replayed (the kernel
 * arguments of a call do not depend on earlier calls, and library memory a
 * call has used is never freed).  A call that needs a library allocation
 * (the first call on a stream with workspace == NULL, a larger shape, or the
 * first use of an encoding's tables) returns ATN_ERR_CAPTURE while its
 * stream is being captured: make one uncaptured call of the shape first, or
 * pass a workspace and call atn_prepare_pe_ex beforehand.
 * Shapes with len_q <= 64 and len_k <= 128 run as one kernel whose
 * workgroups meet at bounded device-side barriers; if such a wait ever
 * expires the outputs of that call are NaN and atn_sync_status_ex reports
 * ATN_ERR_DEVICE_TIMEOUT. */
int atn_attention_fwd_ex(int dtype, const void *Q, const void *K, const void *V, void *out,
                         int batch, int heads, int len_q, int len_k, int head_d,
                         const atn_pe_desc *pe, void *workspace, size_t workspace_bytes,
                         void *stream);

/* Allocation-free form of atn_attention_fwd_ex.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It calls no hipMalloc, hipFree or allocating library routine:
 * its scratch is a file-scope device array of ATN_NOALLOC_SCRATCH_BYTES
 * (64 MiB) on each GPU the library runs on, held until the process ends.
 * Same arguments, results and asynchronous semantics as atn_attention_fwd_ex
 * without the workspace, plus these limits:
 *   - a shape whose scratch exceeds the array runs in chunks of (batch,
 *     head) pairs or of query rows, as atn_attention_fwd_ex does with a
 *     small workspace; a shape that no chunk fits (one head's rows too long
 *     for the array) returns ATN_ERR_SCRATCH_LIMIT;
 *   - an encoding with library tables needs them built beforehand
 *     (atn_prepare_pe_ex), else ATN_ERR_NOT_PREPARED; caller tables need
 *     nothing;
 *   - the first call on a device sets the array up (its address, and a
 *     fill kernel clearing its synchronization words) and must not be
 *     captured (ATN_ERR_CAPTURE); later calls may be;
 *   - every call on one GPU shares that GPU's array, so calls that overlap
 *     in time on one GPU (other streams, other threads) race: serialize
 *     them;
 *   - a device-side wait timeout is reported by atn_sync_status_ex with
 *     workspace == NULL. */
#define ATN_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int atn_attention_fwd_noalloc_ex(int dtype, const void *Q, const void *K, const void *V,
                                 void *out, int batch, int heads, int len_q, int len_k,
                                 int head_d, const atn_pe_desc *pe, void *stream);

/* Scratch bytes atn_attention_fwd_ex needs for this shape (0 on bad input).
 * Scratch is bounded: a call whose scratch would exceed its cap -- the
 * caller's workspace_bytes, or 1 GiB for the library's own workspace -- runs
 * in chunks of consecutive (batch, head) pairs, or of query rows of one head,
 * that fit, and this query then reports the largest chunk's need.  Only a
 * shape whose single query row of one head exceeds the cap reports its full
 * need, above the cap: such a call fails with ATN_ERR_WORKSPACE. */
size_t atn_attention_workspace_bytes(int dtype, int batch, int heads, int len_q, int len_k,
                                     int head_d, const atn_pe_desc *pe);

/* Positional-encoding pre-pass over n_rows rows of head_d, position =
 * row % seq_len (pe->apply_q/apply_k are ignored; the encoding is applied). */
int atn_pe_apply_ex(int dtype, const void *in, void *out, long n_rows, int seq_len, int head_d,
                    const atn_pe_desc *pe, void *stream);

/* Synchronizes `stream` and reports whether a call that used `workspace`
 * (NULL: the library's workspace of that stream and the current device's
 * allocation-free scratch) hit a device-side wait timeout: ATN_OK or
 * ATN_ERR_DEVICE_TIMEOUT (the status word is then cleared).  batch and heads are accepted for interface stability and not
 * used. */
int atn_sync_status_ex(void *workspace, int batch, int heads, void *stream);

/* Prepares the library's angle tables for this encoding and shape on the
 * current device -- the fp32 tables and the fp16 tables of the long-sequence
 * path -- otherwise built on first use, which synchronizes. */
int atn_prepare_pe_ex(const atn_pe_desc *pe, int head_d, int max_positions);

/* Which kernels atn_attention_fwd_ex runs for this shape on the current
 * device (ATN_PATH_*), or a negative status for invalid arguments, assuming
 * vector-aligned tensors (16-byte fp32 / 8-byte bf16 bases; otherwise the
 * split-D pipeline runs).  Without a device the answer assumes 256 compute
 * units. */
#define ATN_PATH_FUSED_SMALL 1 /* one launch: split-D slices + device-side S all-reduce */
#define ATN_PATH_SPLIT_D 2     /* three launches: partial QK^T, softmax, PV */
#define ATN_PATH_FLASH 4       /* outside the single-launch window, head_d % 4 == 0, fp32 and
                                  bf16: head_d <= 256 (128 with an encoding): one launch,
                                  online softmax over key tiles, no scratch; grids that would
                                  leave CUs idle split the keys (parts in the workspace, a
                                  second launch merges them) */
#define ATN_PATH_GEMM 3        /* bf16, D % 8 == 0, head_d > 256 (> 128 with an encoding),
                                  outside the single-launch window: MFMA QK^T GEMM, row
                                  softmax, MFMA PV GEMM */
int atn_attention_path_ex(int dtype, int batch, int heads, int len_q, int len_k, int head_d,
                          const atn_pe_desc *pe);

/* Number of visible HIP devices (0 when none); never aborts. */
int atn_device_count(void);

/* ==================== tuning, test controls and introspection ====================
 * None of these has a counterpart in the reference (whose launchers take no
 * options).  They exist for measurement and tests; a program that never
 * calls them gets the library's own choices.  The library reads no
 * environment variables. */

/* Process-wide overrides, applied to calls made after the change.  Zero
 * fields keep the library's choice. */
typedef struct atn_tuning {
    int fused_rows;        /* single-launch kernel: query rows per row group (16, 32, 48 or 64) */
    int fused_dc;          /* single-launch kernel: D-slice width (a multiple of 32) */
    int fused_exchange;    /* 1: one gather, 2: reduce-scatter + all-gather */
    int fused_xcd;         /* 1: exchange inside one XCD's L2, 2: at device scope */
    int no_fused;          /* nonzero: never the single-launch kernel (the other paths) */
    int no_flash;          /* nonzero: never the flash kernel (calls it would take run on
                              the GEMM path, bf16 with D % 8 == 0, or the split-D pipeline) */
    int gemm_fused_k;      /* long-sequence path: 1 K's encoding inside the QK^T GEMM
                              wherever it can run there, 2 never */
    int workspace_cap_mib; /* cap of the library's own workspace before a call is chunked
                              (default 1024) */
    int model_cus;         /* planning without a device (size and path queries): CU count
                              (default 256) */
    int model_xccs;        /* ... and XCD count (default 8) */
    int preset_status;     /* test only: nonzero makes every single-launch call start with
                              its workspace's status word set, as a timed-out call leaves
                              it, so its workgroups take the fail-closed exit (no wait is
                              entered) */
    int flash_form;        /* flash kernel workgroup: 1 = 4 waves of 16 query rows,
                              2 = 8 waves of 16, 3 = 4 waves of 32, 4 = 8 waves of 32
                              (3 and 4: head_d <= 128; head_d > 128 always runs 2);
                              0: the library's choice */
    int splitd_tile;       /* split-D pipeline, fp32 16-bit kernels: 64 or 128 forces
                              that output tile (128 where both of its sides reach
                              128); 0: 128 x 128 where that grid gives every CU two
                              workgroups, else 64 x 64 */
    int flash_split;       /* flash kernel key splits: 1 never split, n >= 2 split the keys
                              into n parts (fewer for short key lengths: two 64-key chunks
                              at least per part); 0: the library's choice (splits where
                              the grid would leave CUs idle) */
} atn_tuning;
/* Replaces the overrides (NULL: all zero) and drops cached plans.  Plans
 * that a forced setting makes impossible fall back to the library's
 * choice. */
int atn_set_tuning_ex(const atn_tuning *t);
int atn_get_tuning_ex(atn_tuning *t);

/* Plan of the single-launch kernel for this shape on the current device
 * (without a device: the atn_tuning model, default 256 CUs in 8 XCDs).
 * Returns 1 and fills the fields when the shape runs on that kernel, 0 when
 * it does not, or a negative status.  Exchanges inside one XCD's L2 are
 * planned only on a device that reports 8 XCDs and a CU count divisible by
 * 8 (a whole MI355X, not a partition of it). */
typedef struct atn_fused_plan_info {
    int rows;       /* query rows per row group */
    int dc;         /* D-slice width */
    int nchunk;     /* slices per row group */
    int gather1;    /* 1: one-gather exchange, 0: reduce-scatter + all-gather (or none) */
    int xcd;        /* 1: exchange inside one XCD's L2 */
    int workgroups; /* grid size */
    int lds;        /* LDS bytes per workgroup */
} atn_fused_plan_info;
int atn_fused_plan_ex(int dtype, int batch, int heads, int len_q, int len_k, int head_d,
                      const atn_pe_desc *pe, atn_fused_plan_info *info);

/* Synchronous drop-in calls that were run a second time without the
 * single-launch kernel after its wait timed out (each such rerun also
 * prints one line to stderr).  reset != 0 sets the count back to 0. */
long atn_rerun_count(int reset);

/* Device memory the library holds on the current device: live workspaces
 * and tables, and superseded buffers it keeps because work captured into a
 * HIP graph may still use them. */
size_t atn_retained_bytes_ex(void);

/* Synchronizes the current device and frees the superseded buffers.  A HIP
 * graph captured before a workspace or table it used was superseded must
 * not be replayed afterwards.  Buffers that no captured work used are freed
 * as soon as they are superseded. */
int atn_release_ex(void);

#ifdef __cplusplus
}
#endif

#endif /* ATTN_MI355X_H */
