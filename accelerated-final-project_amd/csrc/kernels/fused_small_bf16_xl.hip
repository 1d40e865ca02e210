// k_fused_small variants for bf16, XCD-local exchange: every encoding and
// load form (a translation unit of its own so that the variants compile in
// parallel).
#include "fused_small_impl.hpp"

namespace atn {

hipError_t fused_small_launch_bf16_xl(const FusedArgs& a, int pek, int form, int lds,
                                hipStream_t st) {
    return fused_dispatch<uint16_t, true>(a, pek, form, lds, st);
}

int fused_small_per_cu_bf16_xl(int lds) { return fused_per_cu_forms<uint16_t, true>(lds); }

}  // namespace atn
