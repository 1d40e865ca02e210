// k_fused_small variants for bf16, device-scope exchange: every encoding and
// load form (a translation unit of its own so that the variants compile in
// parallel).
#include "fused_small_impl.hpp"

namespace atn {

hipError_t fused_small_launch_bf16(const FusedArgs& a, int pek, int form, int lds,
                                hipStream_t st) {
    return fused_dispatch<uint16_t, false>(a, pek, form, lds, st);
}

int fused_small_per_cu_bf16(int lds) { return fused_per_cu_forms<uint16_t, false>(lds); }

}  // namespace atn
