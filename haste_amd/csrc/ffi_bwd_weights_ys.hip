// The weight-gradient kernels for dY row strides that are not a multiple of 8
// (the kernel is in bwdw_kernel.hpp): the last row of dY may end at label O, so
// its piece across O is loaded early and shifted back.  dY is read with the
// default cache policy at every size.
#include "bwdw_kernel.hpp"

namespace haste {

int bwdw_dispatch_ys(int32_t dtype, bool sgd, const int32_t* idx, const uint16_t* xT,
                     int64_t ldx, const uint16_t* dY, int64_t lddy, void* dW, int dW_dtype,
                     void* dbias, int dbias_dtype, int64_t B, int64_t D, int64_t F, int64_t O,
                     int64_t G, const SgdArgs& sg, hipStream_t st) {
    if (dtype == HASTE_DTYPE_BF16)
        return sgd ? dispatch_g<BF16, true, false, true>(idx, xT, ldx, dY, lddy, dW, dW_dtype,
                                                         dbias, dbias_dtype, B, D, F, O, G, sg, st)
                   : dispatch_g<BF16, false, false, true>(idx, xT, ldx, dY, lddy, dW, dW_dtype,
                                                          dbias, dbias_dtype, B, D, F, O, G, sg,
                                                          st);
    return sgd ? dispatch_g<F16, true, false, true>(idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias,
                                                    dbias_dtype, B, D, F, O, G, sg, st)
               : dispatch_g<F16, false, false, true>(idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias,
                                                     dbias_dtype, B, D, F, O, G, sg, st);
}

}  // namespace haste
