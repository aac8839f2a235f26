// Grouped fixed-fan-in backward to weights (+ bias gradient) and the fused
// weight-gradient + SR-SGD step: the C entry points and the instantiations for
// dY row strides that are multiples of 8 (the kernel is in bwdw_kernel.hpp).
#include "bwdw_kernel.hpp"

namespace haste {
namespace {

template <typename T, bool SGD>
int dispatch(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* dY,
             int64_t lddy, void* dW, int dW_dtype, void* dbias, int dbias_dtype, int64_t B,
             int64_t D, int64_t F, int64_t O, int64_t G, const SgdArgs& sg, hipStream_t st) {
    if (lddy % 8 != 0 || !aligned16(dY))
        return bwdw_dispatch_ys(T::code, SGD, idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias,
                                dbias_dtype, B, D, F, O, G, sg, st);
    if constexpr (std::is_same_v<T, BF16>) {
        if (B * lddy * 2 > kMallBytes)
            return dispatch_g<T, SGD, true, false>(idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias,
                                            dbias_dtype, B, D, F, O, G, sg, st);
    }
    return dispatch_g<T, SGD, false, false>(idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias, dbias_dtype, B,
                                     D, F, O, G, sg, st);
}

int check_bwdw(const char* fn, const int32_t* idx, const void* xT, int64_t ldx, const void* dY,
               int64_t lddy, int32_t dW_dtype, void* dbias, int32_t dbias_dtype, int64_t B,
               int64_t D, int64_t F, int64_t O, int64_t G, int32_t dtype) {
    int rc = check_ffi_shape(fn, B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && xT && dY, "%s: null pointer", fn);
    HASTE_CHECK_ARG(ldx >= B && ldx % 8 == 0,
                    "%s: ldx must be >= B and a multiple of 8 (ldx=%lld B=%lld)", fn,
                    (long long)ldx, (long long)B);
    HASTE_CHECK_ARG(lddy >= O && ((lddy % 8 == 0 && aligned16(dY)) || O >= 16),
                    "%s: lddy must be >= O, and dY's rows must start on 16-byte boundaries "
                    "when O < 16 (lddy=%lld O=%lld)", fn, (long long)lddy, (long long)O);
    HASTE_CHECK_ARG(aligned16(xT) && (reinterpret_cast<uintptr_t>(dY) & 1) == 0,
                    "%s: xT must be 16-byte aligned and dY 2-byte aligned", fn);
    HASTE_CHECK_ARG(dW_dtype == HASTE_DTYPE_F32 || dW_dtype == HASTE_DTYPE_BF16 ||
                        dW_dtype == HASTE_DTYPE_F16,
                    "%s: bad dW dtype %d", fn, (int)dW_dtype);
    HASTE_CHECK_ARG(dbias == nullptr || dbias_dtype == HASTE_DTYPE_F32 ||
                        dbias_dtype == HASTE_DTYPE_BF16 || dbias_dtype == HASTE_DTYPE_F16,
                    "%s: bad dbias dtype %d", fn, (int)dbias_dtype);
    return HASTE_OK;
}

}  // namespace
}  // namespace haste

extern "C" int haste_ffi_bwd_weights(const int32_t* idx, const void* xT, int64_t ldx,
                                     const void* dY, int64_t lddy, void* dW, int32_t dW_dtype,
                                     void* dbias, int32_t dbias_dtype, int64_t B, int64_t D,
                                     int64_t F, int64_t O, int64_t G, int32_t dtype,
                                     void* stream) {
    const char* fn = "haste_ffi_bwd_weights";
    int rc = haste::check_bwdw(fn, idx, xT, ldx, dY, lddy, dW_dtype, dbias, dbias_dtype, B, D, F,
                               O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(dW != nullptr, "%s: null pointer", fn);
    HASTE_CHECK_ARG(haste::aligned16(dW), "%s: dW must be 16-byte aligned", fn);
    auto* x = static_cast<const uint16_t*>(xT);
    auto* y = static_cast<const uint16_t*>(dY);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const haste::SgdArgs none{};
    if (dtype == HASTE_DTYPE_BF16)
        return haste::dispatch<haste::BF16, false>(idx, x, ldx, y, lddy, dW, dW_dtype, dbias,
                                                  dbias_dtype, B, D, F, O, G, none, st);
    return haste::dispatch<haste::F16, false>(idx, x, ldx, y, lddy, dW, dW_dtype, dbias,
                                             dbias_dtype, B, D, F, O, G, none, st);
}

extern "C" int haste_ffi_bwd_weights_dx(const int32_t* idx, const void* xT, int64_t ldx,
                                        const void* dY, int64_t lddy, void* dW, int32_t dW_dtype,
                                        void* dbias, int32_t dbias_dtype, uint16_t* dX,
                                        uint64_t dx_seed, void* bwdf_workspace,
                                        int64_t bwdf_workspace_bytes, int64_t B, int64_t D,
                                        int64_t F, int64_t O, int64_t G, int32_t dtype,
                                        void* stream) {
    const char* fn = "haste_ffi_bwd_weights_dx";
    int rc = haste::check_bwdw(fn, idx, xT, ldx, dY, lddy, dW_dtype, dbias, dbias_dtype, B, D, F,
                               O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(dtype == HASTE_DTYPE_BF16, "%s: dX is bf16: the layer must be bf16", fn);
    HASTE_CHECK_ARG(dW != nullptr && haste::aligned16(dW), "%s: dW must be a 16-byte aligned pointer", fn);
    HASTE_CHECK_ARG(dX != nullptr && bwdf_workspace != nullptr,
                    "%s: dX and the bwd-features workspace are required", fn);
    const haste::BwdFPlan p = haste::make_plan(B, D, F, O, G);
    HASTE_CHECK_ARG(haste::aligned16(bwdf_workspace) &&
                        bwdf_workspace_bytes >= p.prep_bytes + p.ws_bytes,
                    "%s: bwd-features workspace too small or misaligned (%lld bytes, need %lld)",
                    fn, (long long)bwdf_workspace_bytes, (long long)(p.prep_bytes + p.ws_bytes));
    haste::SgdArgs sg{};
    sg.rj = haste::reduce_job(
        p, reinterpret_cast<const float*>(static_cast<const char*>(bwdf_workspace) + p.prep_bytes),
        dX, B, D, dx_seed);
    return haste::dispatch<haste::BF16, false>(idx, static_cast<const uint16_t*>(xT), ldx,
                                              static_cast<const uint16_t*>(dY), lddy, dW,
                                              dW_dtype, dbias, dbias_dtype, B, D, F, O, G, sg,
                                              static_cast<hipStream_t>(stream));
}

namespace haste {
namespace {

// The fused weight-gradient + SGD step; dX != NULL: also the final pass of
// backward to features (the partials a haste_ffi_bwd_features_partials call
// left in bwdf_workspace -> dX), as trailing workgroups of the same launch.
int bwdw_sgd(const char* fn, const int32_t* idx, const void* xT, int64_t ldx, const void* dY,
             int64_t lddy, uint16_t* W, uint16_t* bias, float* m_W, float* m_bias, void* dW,
             int32_t dW_dtype, void* dbias, int32_t dbias_dtype, float lr, float wd, float mu,
             int32_t use_mom, int32_t do_sr, uint64_t seed, uint16_t* dX, uint64_t dx_seed,
             void* bwdf_workspace, int64_t bwdf_workspace_bytes, int64_t B, int64_t D, int64_t F,
             int64_t O, int64_t G, int32_t dtype, void* stream,
             const uint64_t* seed_dev = nullptr) {
    int rc = check_bwdw(fn, idx, xT, ldx, dY, lddy, dW_dtype, dbias, dbias_dtype, B, D, F, O, G,
                        dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(dtype == HASTE_DTYPE_BF16, "%s: the SGD step updates bf16 weights only", fn);
    if (O * F > 0xFFFFFFFFll) {
        set_error("%s: O*F = %lld exceeds 2^32 - 1 elements", fn, (long long)(O * F));
        return HASTE_ERR_UNSUPPORTED;
    }
    HASTE_CHECK_ARG(W != nullptr && aligned16(W), "%s: W must be a 16-byte aligned pointer", fn);
    HASTE_CHECK_ARG(dW == nullptr || aligned16(dW), "%s: dW must be 16-byte aligned", fn);
    HASTE_CHECK_ARG(!use_mom || (m_W != nullptr && aligned16(m_W) &&
                                 (bias == nullptr || m_bias != nullptr)),
                    "%s: momentum buffers missing or misaligned", fn);
    SgdArgs sg{W, bias, m_W, m_bias, lr, wd, mu, use_mom ? 1 : 0, do_sr ? 1 : 0,
               (uint32_t)seed, (uint32_t)(seed >> 32), nullptr, nullptr, nullptr, nullptr,
               0, 0, ReduceJob{}, seed_dev};
    if (bwdf_workspace != nullptr) {
        const BwdFPlan p = make_plan(B, D, F, O, G);
        HASTE_CHECK_ARG(aligned16(bwdf_workspace) &&
                            bwdf_workspace_bytes >= p.prep_bytes + p.ws_bytes,
                        "%s: bwd-features workspace too small or misaligned (%lld bytes, need %lld)",
                        fn, (long long)bwdf_workspace_bytes, (long long)(p.prep_bytes + p.ws_bytes));
        char* base = static_cast<char*>(bwdf_workspace);
        sg.twt = reinterpret_cast<uint16_t*>(base + p.twt_off);
        sg.tsrc = reinterpret_cast<const int*>(base + p.tsrc_off);
        sg.perm = reinterpret_cast<const int*>(base + p.perm_off);
        sg.meta = reinterpret_cast<const int*>(base + p.meta_off);
        sg.ndr = (int)p.ndr;
        sg.Tcap = (int)p.Tcap;
        if (dX != nullptr)
            sg.rj = reduce_job(p, reinterpret_cast<const float*>(base + p.prep_bytes), dX, B, D,
                               dx_seed);
    }
    return dispatch<BF16, true>(idx, static_cast<const uint16_t*>(xT), ldx,
                                static_cast<const uint16_t*>(dY), lddy, dW, dW_dtype, dbias,
                                dbias_dtype, B, D, F, O, G, sg, static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace haste

namespace haste {
namespace {
// seed += 1 on the device (one lane; a vector store, its address from a VGPR)
__global__ void seed_advance_kernel(uint64_t* __restrict__ seed) {
    const int t = (int)threadIdx.x;
    if (t == 0) seed[t] += 1u;
}
}  // namespace
}  // namespace haste

extern "C" int haste_ffi_bwd_weights_sgd_dx_dev_seed(
    const int32_t* idx, const void* xT, int64_t ldx, const void* dY, int64_t lddy, uint16_t* W,
    uint16_t* bias, float* m_W, float* m_bias, float lr, float wd, float mu, int32_t use_mom,
    int32_t do_sr, uint64_t* seed_dev, uint16_t* dX, uint64_t dx_seed, void* bwdf_workspace,
    int64_t bwdf_workspace_bytes, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
    int32_t dtype, void* stream) {
    const char* fn = "haste_ffi_bwd_weights_sgd_dx_dev_seed";
    HASTE_CHECK_ARG(dX != nullptr && bwdf_workspace != nullptr,
                    "%s: dX and the bwd-features workspace are required", fn);
    HASTE_CHECK_ARG(seed_dev != nullptr && reinterpret_cast<uintptr_t>(seed_dev) % 8 == 0,
                    "%s: seed_dev must be an 8-byte aligned device pointer", fn);
    int rc = haste::bwdw_sgd(fn, idx, xT, ldx, dY, lddy, W, bias, m_W, m_bias, nullptr,
                             HASTE_DTYPE_F32, nullptr, HASTE_DTYPE_F32, lr, wd, mu, use_mom,
                             do_sr, 0, dX, dx_seed, bwdf_workspace, bwdf_workspace_bytes, B, D, F,
                             O, G, dtype, stream, seed_dev);
    if (rc != HASTE_OK) return rc;
    haste::seed_advance_kernel<<<dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream)>>>(seed_dev);
    HASTE_CHECK_LAUNCH(fn);
    return HASTE_OK;
}

extern "C" int haste_ffi_bwd_weights_sgd(const int32_t* idx, const void* xT, int64_t ldx,
                                         const void* dY, int64_t lddy, uint16_t* W,
                                         uint16_t* bias, float* m_W, float* m_bias, void* dW,
                                         int32_t dW_dtype, void* dbias, int32_t dbias_dtype,
                                         float lr, float wd, float mu, int32_t use_mom,
                                         int32_t do_sr, uint64_t seed, void* bwdf_workspace,
                                         int64_t bwdf_workspace_bytes, int64_t B, int64_t D,
                                         int64_t F, int64_t O, int64_t G, int32_t dtype,
                                         void* stream) {
    return haste::bwdw_sgd("haste_ffi_bwd_weights_sgd", idx, xT, ldx, dY, lddy, W, bias, m_W,
                           m_bias, dW, dW_dtype, dbias, dbias_dtype, lr, wd, mu, use_mom, do_sr,
                           seed, nullptr, 0, bwdf_workspace, bwdf_workspace_bytes, B, D, F, O, G,
                           dtype, stream);
}

extern "C" int haste_ffi_bwd_weights_sgd_dx(const int32_t* idx, const void* xT, int64_t ldx,
                                            const void* dY, int64_t lddy, uint16_t* W,
                                            uint16_t* bias, float* m_W, float* m_bias, float lr,
                                            float wd, float mu, int32_t use_mom, int32_t do_sr,
                                            uint64_t seed, uint16_t* dX, uint64_t dx_seed,
                                            void* bwdf_workspace, int64_t bwdf_workspace_bytes,
                                            int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                                            int32_t dtype, void* stream) {
    const char* fn = "haste_ffi_bwd_weights_sgd_dx";
    HASTE_CHECK_ARG(dX != nullptr && bwdf_workspace != nullptr,
                    "%s: dX and the bwd-features workspace are required", fn);
    return haste::bwdw_sgd(fn, idx, xT, ldx, dY, lddy, W, bias, m_W, m_bias, nullptr,
                           HASTE_DTYPE_F32, nullptr, HASTE_DTYPE_F32, lr, wd, mu, use_mom, do_sr,
                           seed, dX, dx_seed, bwdf_workspace, bwdf_workspace_bytes, B, D, F, O, G,
                           dtype, stream);
}
