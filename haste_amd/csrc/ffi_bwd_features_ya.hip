// The backward-to-features main kernels for dY rows that do not all start on
// 16-byte boundaries (the kernel is in bwdf_main.hpp).
#include "bwdf_main.hpp"

namespace haste {

int bwdf_run_main_ya(int32_t dtype, int64_t G, const int* tfeat, const int* meta,
                     const uint16_t* twt, const uint16_t* dY, int64_t lddy, float* ws,
                     const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O,
                     hipStream_t st) {
    switch (G) {
#define HASTE_BWDF_YA(GG)                                                                         \
    case GG:                                                                                      \
        return dtype == HASTE_DTYPE_BF16                                                          \
                   ? run_main<BF16, GG, true>(tfeat, meta, twt, dY, lddy, ws, p, B, D, F, O, st)  \
                   : run_main<F16, GG, true>(tfeat, meta, twt, dY, lddy, ws, p, B, D, F, O, st);
        HASTE_BWDF_YA(16)
        HASTE_BWDF_YA(32)
        HASTE_BWDF_YA(64)
        HASTE_BWDF_YA(128)
#undef HASTE_BWDF_YA
    default:
        set_error("haste_ffi_bwd_features: unsupported group size %lld", (long long)G);
        return HASTE_ERR_UNSUPPORTED;
    }
}

}  // namespace haste
