// Host side of the single-launch split-D kernel (the kernel itself, its
// design notes and its variants: fused_small_impl.hpp and
// fused_small_{f32,bf16}[_xl].hip): LDS size, occupancy and the launch.
#include "fused_small_impl.hpp"

namespace atn {

int fused_small_lds_bytes(int dtype, int pek, int MB, int Lk, int dc, int nchunk) {
    const bool bf16 = dtype == kDtypeBF16;
    return make_geo(!bf16, pek != kPeNone, nchunk > 1, MB, Lk, dc).bytes;
}

int fused_small_per_cu(int dtype, int pek, int lds) {
    // occupancy depends on LDS and registers; the smallest figure of either
    // exchange scope is safe for every variant
    (void)pek;
    if (dtype == kDtypeF32)
        return std::min(fused_small_per_cu_f32(lds), fused_small_per_cu_f32_xl(lds));
    return std::min(fused_small_per_cu_bf16(lds), fused_small_per_cu_bf16_xl(lds));
}

hipError_t launch_fused_small(int dtype, int pek, const void* Q, const void* K, const void* V,
                              void* O, float* part, float* red,
                              unsigned* epochs, unsigned* done, int* status, unsigned* xctr,
                              int BH, int Lq, int Lk, int D, int MB, int dc, int nchunk,
                              int gather1, int xcd, float scale, const PeSide& pq,
                              const PeSide& pk, hipStream_t st) {
    const int QB = (Lq + MB - 1) / MB;
    const int MQ = (MB + 15) / 16 * 16, NK = (Lk + 31) / 32 * 32;
    const int vpr = dc / 4, rstep = 256 / vpr;
    FusedArgs a{Q, K, V, O, part, red, epochs, done, status, Lq, Lk, D, dc, nchunk,
                MB, QB, gather1, BH * QB, xctr, scale, pq, pk,
                rstep, fused_div_magic(nchunk), fused_div_magic(QB), fused_div_magic(BH),
                fused_div_magic(vpr), fused_div_magic(rstep), fused_div_magic(NK)};
    const int lds = fused_small_lds_bytes(dtype, pek, MB, Lk, dc, nchunk);
    // an XL plan with one slice has no exchange: the plain form does the same
    const bool xl = xcd != 0 && nchunk > 1;
    const int form = fused_load_form(MQ, NK, dc);
    if (dtype == kDtypeF32)
        return xl ? fused_small_launch_f32_xl(a, pek, form, lds, st)
                  : fused_small_launch_f32(a, pek, form, lds, st);
    return xl ? fused_small_launch_bf16_xl(a, pek, form, lds, st)
              : fused_small_launch_bf16(a, pek, form, lds, st);
}

}  // namespace atn
