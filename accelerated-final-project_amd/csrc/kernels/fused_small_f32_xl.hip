// k_fused_small variants for fp32, XCD-local exchange: every encoding and
// load form (a translation unit of its own so that the variants compile in
// parallel).
#include "fused_small_impl.hpp"

namespace atn {

hipError_t fused_small_launch_f32_xl(const FusedArgs& a, int pek, int form, int lds,
                                hipStream_t st) {
    return fused_dispatch<float, true>(a, pek, form, lds, st);
}

int fused_small_per_cu_f32_xl(int lds) { return fused_per_cu_forms<float, true>(lds); }

}  // namespace atn
