// Host-callable launchers for the HIP kernels.  Every launcher is
// asynchronous on `st`, validates nothing (the C-ABI layer does that before
// any HIP call) and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "common.hpp"

namespace atn {

constexpr int kDtypeF32 = 0;
constexpr int kDtypeBF16 = 1;

// Split-D streaming pipeline (stream.hip).
hipError_t launch_qk_partial(int dtype, int pek, const void* Q, const void* K, float* S, int BH,
                             int Lq, int Lk, int D, int dchunk, int nsplit, const PeSide& pq,
                             const PeSide& pk, int vec_ok, hipStream_t st);
hipError_t launch_softmax(const float* S, float* P, long rows, int Lk, int nsplit,
                          size_t split_stride, float scale, hipStream_t st);
hipError_t launch_pv(int dtype, const float* P, const void* V, void* O, int BH, int Lq, int Lk,
                     int D, int vec_ok, hipStream_t st);
// Stages 1 and 3 for fp32 on 16-bit MFMA (stream16.hip; launch_qk_partial
// and launch_pv choose them for fp32 with head_d % 4 == 0, 16-byte aligned
// bases and per-head byte offsets under 2^31).  Output tiles of 128 x 128
// where both of a tile's sides reach 128 and their grid gives every CU two
// workgroups, else 64 x 64; s16_set_tile(64 or 128) forces a size wherever
// it fits, s16_set_tile(0) restores the rule (a tuning override).
void s16_set_tile(int tile);
// Sides a x b (queries x keys for QK^T, queries x dims for PV) that 128 x
// 128 tiles cover with at most 10 % more padding than 64 x 64 ones, both
// sides reaching 128 (the host's D-chunk plan uses the same test).
inline bool s16_fits_128(int a, int b) {
    if (a < 128 || b < 128) return false;
    const double p128 = (double)((a + 127) / 128 * 128) * ((b + 127) / 128 * 128);
    const double p64 = (double)((a + 63) / 64 * 64) * ((b + 63) / 64 * 64);
    return p128 <= 1.1 * p64;
}
hipError_t launch_qk_s16(int pek, const float* Q, const float* K, float* S, int BH, int Lq, int Lk,
                         int D, int dchunk, int nsplit, const PeSide& pq, const PeSide& pk,
                         hipStream_t st);
hipError_t launch_pv_s16(const float* P, const float* V, float* O, int BH, int Lq, int Lk, int D,
                         hipStream_t st);
// Single-launch split-D kernel for len_q <= 64, len_k <= 128 (fused_small.hip):
// row groups of MB query rows, D slices of dc dims; gather1 selects the
// one-gather exchange (each thread polls (MB*NK/256) * nchunk <= 64 words)
// over reduce-scatter + all-gather; xcd selects the XCD-local exchange
// (every slice of a row group on one XCD, arrival counters in xctr, at most
// kXcdGroupsPerXcd row groups per XCD).
constexpr int kXcdCtrWords = 256;                    // counter words per XCD (1 KiB)
constexpr int kXcdGroupsPerXcd = kXcdCtrWords / 2;  // two counters per row group
int fused_small_lds_bytes(int dtype, int pek, int MB, int Lk, int dc, int nchunk);
// resident workgroups per CU for this LDS size (either exchange)
int fused_small_per_cu(int dtype, int pek, int lds);
hipError_t launch_fused_small(int dtype, int pek, const void* Q, const void* K, const void* V,
                              void* O, float* part, float* red,
                              unsigned* epochs, unsigned* done, int* status, unsigned* xctr,
                              int BH, int Lq, int Lk, int D, int MB, int dc, int nchunk,
                              int gather1, int xcd, float scale, const PeSide& pq,
                              const PeSide& pk, hipStream_t st);
// Long-sequence bf16 path (gemm_path.hip): E = exp(scale Q K^T - tile row
// max) (fp16, rows ldE = Lk rounded up to 8 apart, zero past Lk) with
// per-(row, 256-key tile) max and sum, per-row factors g_t = exp(m_t - m) /
// l, O = (E g) V.  Needs D % 8 == 0 and 16-byte aligned bases.
hipError_t launch_encode_f16(int pek, const uint16_t* in, uint16_t* out, float* inv, long n_rows,
                             int seq_len, int D, const PeSide& pe, hipStream_t st);
hipError_t launch_gemm_qk(int f16, const uint16_t* Q, const uint16_t* K, const float* qinv,
                          const float* kinv, uint16_t* E, int ldE, float* st_m, float* st_l,
                          int BH, int Lq, int Lk, int D, float scale, hipStream_t st);
// QK^T GEMM on fp16 Q~ (row scales qinv) and raw bf16 K, K's encoding
// applied in the kernel from an fp16 table (tab: tab_rows positions x D
// 16-bit units); needs D % 128 == 0.
constexpr int kGemmEncRaw = 1, kGemmEncSin = 2, kGemmEncRope = 3, kGemmEncRopeHalf = 4;
hipError_t launch_gemm_qk_enc(int benc, const uint16_t* Qe, const uint16_t* K, const float* qinv,
                              const uint16_t* tab, int tab_rows, uint16_t* E, int ldE,
                              float* st_m, float* st_l, int BH, int Lq, int Lk, int D,
                              float scale, hipStream_t st);
// O = P V from E and the QK^T epilogue's tile statistics (st_m, st_l); ga
// holds the softmax factors of rows with more than 8 key tiles.
hipError_t launch_gemm_pv(const uint16_t* E, int ldE, float* st_m, float* st_l, float* ga,
                          const uint16_t* V, uint16_t* O, int BH, int Lq, int Lk, int D,
                          hipStream_t st);

// Flash-style attention (flash.hip), fp32 or bf16 storage (dtype): any
// len_q and len_k, head_d <= kFlashMaxD (kFlashMaxDEncoded with a positional
// encoding) with head_d % 4 == 0, 16-byte aligned bases, and every head's Q
// or K/V under 2^31 bytes (32-bit buffer offsets); no scratch.
// `form`: the workgroup -- 4 waves of 16 query rows, 8 of 16, 4 of 32 or 8
// of 32 (head_d <= 128; past 128 every form runs 8 of 16).
constexpr int kFlashMaxD = 256, kFlashMaxDEncoded = 128;
constexpr int kFlashForm4x16 = 1, kFlashForm8x16 = 2, kFlashForm4x32 = 3, kFlashForm8x32 = 4;
// Key split (nsplit > 1): workgroup split s takes keys [s kchunk, (s + 1)
// kchunk) and writes its normalized output and statistics to `part`
// (nsplit BH Lq D floats, then nsplit BH Lq float4s; 16-byte aligned), which
// a second kernel merges into O.  nsplit == 1: no scratch (part unused).
bool flash_supported(int dtype, int pek, int D);
hipError_t launch_flash(int dtype, int pek, int form, const void* Q, const void* K, const void* V,
                        void* O, int BH, int Lq, int Lk, int D, float scale, const PeSide& pq,
                        const PeSide& pk, int nsplit, int kchunk, float* part, hipStream_t st);

// Allocation-free entry point: the per-device scratch array (noalloc.hip),
// kNoAllocScratchBytes long.  noalloc_scratch() returns its device address
// for device `dev` (hipGetSymbolAddress, taken once per device) and, on the
// first call for that device, enqueues a fill kernel on `st` that zeroes its
// first sync_bytes; noalloc_ready() tells whether that set-up has happened.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;  // ATN_NOALLOC_SCRATCH_BYTES
bool noalloc_ready(int dev);
hipError_t noalloc_scratch(int dev, size_t sync_bytes, hipStream_t st, void** ptr);

hipError_t launch_pe_apply(int dtype, int pek, const void* in, void* out, long n_rows,
                           int seq_len, int D, const PeSide& pe, int vec_ok, hipStream_t st);

}  // namespace atn
