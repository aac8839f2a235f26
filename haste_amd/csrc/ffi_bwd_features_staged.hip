// The staged backward-to-features main kernel (bwdf_staged.hpp) for every
// group size it is built for (G = 32, 64, 128), batch tile (32, 64 columns),
// element type and dY row alignment, with eight waves of one pipeline tile each
// (measured at config 1: four waves of two tiles each, half the operand reads
// from LDS, took 78 against 72 us, and 3109 against 2643 us at config 4).
#include "bwdf_staged.hpp"

namespace haste {

namespace {
template <typename T, int G, bool YA>
int staged_bt(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
              int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
              hipStream_t st) {
    if (p.BT == 64) return launch_staged<T, G, 64, 8, YA>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
    return launch_staged<T, G, 32, 8, YA>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
}
template <typename T, int G>
int staged_ya(bool ya, const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
              int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
              hipStream_t st) {
    return ya ? staged_bt<T, G, true>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st)
              : staged_bt<T, G, false>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
}
}  // namespace

int bwdf_run_staged(int32_t dtype, int64_t G, bool ya, const int* tfeat, const int* meta,
                    const uint16_t* twt, const uint16_t* dY, int64_t lddy, float* ws,
                    const BwdFPlan& p, int64_t B, int64_t D, int64_t O, hipStream_t st) {
    if (p.BT != 32 && p.BT != 64) {
        set_error("haste_ffi_bwd_features: no staged build for %lld batch columns", (long long)p.BT);
        return HASTE_ERR_UNSUPPORTED;
    }
    switch (G) {
#define HASTE_BWDF_STAGED(GG)                                                                   \
    case GG:                                                                                    \
        return dtype == HASTE_DTYPE_BF16                                                        \
                   ? staged_ya<BF16, GG>(ya, tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st)     \
                   : staged_ya<F16, GG>(ya, tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
        HASTE_BWDF_STAGED(32)
        HASTE_BWDF_STAGED(64)
        HASTE_BWDF_STAGED(128)
#undef HASTE_BWDF_STAGED
    default:
        set_error("haste_ffi_bwd_features: no staged build for group size %lld", (long long)G);
        return HASTE_ERR_UNSUPPORTED;
    }
}

}  // namespace haste
