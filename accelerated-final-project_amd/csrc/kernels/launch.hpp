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
hipError_t launch_pe_apply(int dtype, int pek, const void* in, void* out, long n_rows,
                           int seq_len, int D, const PeSide& pe, int vec_ok, hipStream_t st);

}  // namespace atn
