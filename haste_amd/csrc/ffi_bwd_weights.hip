// Grouped fixed-fan-in backward to weights (+ bias gradient), gfx950.
//
//   dW[l, j] = sum_b dY[b, l] * xT[idx[g, j], b]        g = l / G
//   dbias[l] = sum_b dY[b, l]
//
// One workgroup per label group; the contraction runs over the whole batch.
// MFMA orientation: M = labels, N = fan-in slots, K = batch.  dY[b, g*G:(g+1)*G]
// is read once from HBM in 128-row chunks, transposed in registers and staged
// in LDS as Ys[label][batch] (A fragments are 16-byte LDS reads).  The gathered
// features are the B operand and come straight from L2: for a fixed slot j a
// fragment is 8 consecutive batch entries of row xT[idx[g, j]].  The bias
// gradient is one extra MFMA column tile against a constant ones fragment, so
// dY is read once for both outputs (the reference reads it a second time for
// torch.sum, shared_ffi/bindings.py:40).
#include <algorithm>

#include "common.hpp"

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

constexpr int kThreads = 256;
constexpr int kKC = 128;  // batch rows per LDS stage

template <int G, int FP>
struct BwdWCfg {
    static constexpr int MTILES = G / 16;
    static constexpr int NTILES = FP / 16;
    static constexpr int WN = NTILES < 4 ? NTILES : 4;
    static constexpr int WM0 = 4 / WN;
    static constexpr int WM = MTILES < WM0 ? MTILES : WM0;
    static constexpr int MT = MTILES / WM;
    static constexpr int NT = NTILES / WN;
    static constexpr int LDY = kKC + 8;  // LDS pitch (elements) of Ys rows
    static constexpr int ITEMS = (G / 8) * (kKC / 4);
};

__device__ __forceinline__ uint32_t half_of(const u32x4& v, int e) {
    return (e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xFFFFu);
}

template <typename T>
__device__ __forceinline__ uint32_t one_pair();
template <>
__device__ __forceinline__ uint32_t one_pair<BF16>() { return 0x3F803F80u; }
template <>
__device__ __forceinline__ uint32_t one_pair<F16>() { return 0x3C003C00u; }

template <typename T, int G, int FP>
__global__ __launch_bounds__(kThreads) void ffi_bwd_w_kernel(
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ xT, int64_t ldx,
    const uint16_t* __restrict__ dY, int64_t lddy, void* __restrict__ dW, int dW_dtype,
    void* __restrict__ dbias, int dbias_dtype, int B, int D, int F, int64_t O) {
    using C = BwdWCfg<G, FP>;
    __shared__ __attribute__((aligned(16))) uint16_t Ys[G * C::LDY];
    __shared__ int32_t sidx[FP];

    const int64_t g = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave % C::WN;
    const int wm = wave / C::WN;
    const bool active = wm < C::WM;
    const int lrow = lane & 15;
    const int lq = lane >> 4;
    const int64_t l0 = g * G;

    for (int j = tid; j < FP; j += kThreads)
        sidx[j] = j < F ? min(max(idx[g * F + j], 0), D - 1) : 0;

    f32x4 acc[C::MT][C::NT];
    f32x4 accb[C::MT];
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) {
        accb[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const uint32_t op = one_pair<T>();
    const u32x4 ones = u32x4{op, op, op, op};
    const bool do_bias = dbias != nullptr && wn == 0;
    __syncthreads();

    // Row pointers of this lane's B-operand slots.
    const uint16_t* xrow[C::NT];
    bool jvalid[C::NT];
#pragma unroll
    for (int nt = 0; nt < C::NT; ++nt) {
        const int j = (wn * C::NT + nt) * 16 + lrow;
        jvalid[nt] = j < F;
        xrow[nt] = xT + (int64_t)sidx[j < FP ? j : 0] * ldx;
    }

    for (int kc = 0; kc < B; kc += kKC) {
        // ---- stage dY[kc:kc+128, l0:l0+G] transposed into Ys[label][batch] ----
        for (int it = tid; it < C::ITEMS; it += kThreads) {
            const int lo8 = it % (G / 8);
            const int bq = it / (G / 8);
            const int lcol = lo8 * 8;
            const int b0 = kc + bq * 4;
            u32x4 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (b0 + q < B && l0 + lcol < O)
                    v[q] = *reinterpret_cast<const u32x4*>(dY + (int64_t)(b0 + q) * lddy + l0 + lcol);
                else
                    v[q] = u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                uint32_t lo = half_of(v[0], e) | (half_of(v[1], e) << 16);
                uint32_t hi = half_of(v[2], e) | (half_of(v[3], e) << 16);
                if (l0 + lcol + e >= O) { lo = 0u; hi = 0u; }
                *reinterpret_cast<u32x2*>(&Ys[(lcol + e) * C::LDY + bq * 4]) = u32x2{lo, hi};
            }
        }
        __syncthreads();

        if (active) {
#pragma unroll
            for (int ks = 0; ks < kKC / 32; ++ks) {
                const int bk = kc + ks * 32 + lq * 8;  // first batch row of this lane's K chunk
                if (kc + ks * 32 >= B) break;
                u32x4 bf[C::NT];
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt) {
                    if (jvalid[nt] && bk < B) {
                        bf[nt] = *reinterpret_cast<const u32x4*>(xrow[nt] + bk);
                        if (bk + 8 > B) {
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                if (bk + e >= B) bf[nt][e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                        }
                    } else {
                        bf[nt] = u32x4{0u, 0u, 0u, 0u};
                    }
                }
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt) {
                    const int m0 = (wm * C::MT + mt) * 16;
                    const u32x4 af = *reinterpret_cast<const u32x4*>(
                        &Ys[(m0 + lrow) * C::LDY + ks * 32 + lq * 8]);
#pragma unroll
                    for (int nt = 0; nt < C::NT; ++nt) acc[mt][nt] = mfma16x16x32<T>(af, bf[nt], acc[mt][nt]);
                    if (do_bias) accb[mt] = mfma16x16x32<T>(af, ones, accb[mt]);
                }
            }
        }
        __syncthreads();
    }

    if (!active) return;
    // ---- epilogue ----
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) {
        const int64_t lb = l0 + (wm * C::MT + mt) * 16 + lq * 4;
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt) {
            const int j = (wn * C::NT + nt) * 16 + lrow;
            if (j >= F) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t l = lb + i;
                if (l >= O) continue;
                const float v = acc[mt][nt][i];
                if (dW_dtype == HASTE_DTYPE_F32)
                    static_cast<float*>(dW)[l * F + j] = v;
                else if (dW_dtype == HASTE_DTYPE_BF16)
                    static_cast<uint16_t*>(dW)[l * F + j] = (uint16_t)f32_to_bf16_rne(v);
                else
                    static_cast<uint16_t*>(dW)[l * F + j] = (uint16_t)f32_to_f16_rne(v);
            }
        }
        if (do_bias && lrow == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t l = lb + i;
                if (l >= O) continue;
                const float v = accb[mt][i];
                if (dbias_dtype == HASTE_DTYPE_F32)
                    static_cast<float*>(dbias)[l] = v;
                else if (dbias_dtype == HASTE_DTYPE_BF16)
                    static_cast<uint16_t*>(dbias)[l] = (uint16_t)f32_to_bf16_rne(v);
                else
                    static_cast<uint16_t*>(dbias)[l] = (uint16_t)f32_to_f16_rne(v);
            }
        }
    }
}

template <typename T, int G, int FP>
int launch(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* dY, int64_t lddy,
           void* dW, int dW_dtype, void* dbias, int dbias_dtype, int64_t B, int64_t D, int64_t F,
           int64_t O, hipStream_t st) {
    const int64_t Gc = ceil_div(O, G);
    if (Gc > 0x7FFFFFFF) {
        set_error("haste_ffi_bwd_weights: too many groups");
        return HASTE_ERR_UNSUPPORTED;
    }
    ffi_bwd_w_kernel<T, G, FP><<<dim3((unsigned)Gc), dim3(kThreads), 0, st>>>(
        idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias, dbias_dtype, (int)B, (int)D, (int)F, O);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_weights");
    return HASTE_OK;
}

template <typename T, int G>
int dispatch_fp(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* dY,
                int64_t lddy, void* dW, int dW_dtype, void* dbias, int dbias_dtype, int64_t B,
                int64_t D, int64_t F, int64_t O, hipStream_t st) {
#define HASTE_BWDW_ARGS idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias, dbias_dtype, B, D, F, O, st
    if (F <= 32) return launch<T, G, 32>(HASTE_BWDW_ARGS);
    if (F <= 64) return launch<T, G, 64>(HASTE_BWDW_ARGS);
    if (F <= 128) return launch<T, G, 128>(HASTE_BWDW_ARGS);
    return launch<T, G, 256>(HASTE_BWDW_ARGS);
#undef HASTE_BWDW_ARGS
}

template <typename T>
int dispatch_g(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* dY,
               int64_t lddy, void* dW, int dW_dtype, void* dbias, int dbias_dtype, int64_t B,
               int64_t D, int64_t F, int64_t O, int64_t G, hipStream_t st) {
#define HASTE_BWDW_ARGS idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias, dbias_dtype, B, D, F, O, st
    switch (G) {
    case 16: return dispatch_fp<T, 16>(HASTE_BWDW_ARGS);
    case 32: return dispatch_fp<T, 32>(HASTE_BWDW_ARGS);
    case 64: return dispatch_fp<T, 64>(HASTE_BWDW_ARGS);
    default: return dispatch_fp<T, 128>(HASTE_BWDW_ARGS);
    }
#undef HASTE_BWDW_ARGS
}

}  // namespace
}  // namespace haste

extern "C" int haste_ffi_bwd_weights(const int32_t* idx, const void* xT, int64_t ldx,
                                     const void* dY, int64_t lddy, void* dW, int32_t dW_dtype,
                                     void* dbias, int32_t dbias_dtype, int64_t B, int64_t D,
                                     int64_t F, int64_t O, int64_t G, int32_t dtype,
                                     void* stream) {
    int rc = haste::check_ffi_shape("haste_ffi_bwd_weights", B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && xT && dY && dW, "haste_ffi_bwd_weights: null pointer");
    HASTE_CHECK_ARG(ldx >= B && ldx % 8 == 0,
                    "haste_ffi_bwd_weights: ldx must be >= B and a multiple of 8 (ldx=%lld B=%lld)",
                    (long long)ldx, (long long)B);
    HASTE_CHECK_ARG(lddy >= O && lddy % 8 == 0,
                    "haste_ffi_bwd_weights: lddy must be >= O and a multiple of 8 (lddy=%lld O=%lld)",
                    (long long)lddy, (long long)O);
    HASTE_CHECK_ARG(haste::aligned16(xT) && haste::aligned16(dY),
                    "haste_ffi_bwd_weights: xT and dY must be 16-byte aligned");
    HASTE_CHECK_ARG(dW_dtype == HASTE_DTYPE_F32 || dW_dtype == HASTE_DTYPE_BF16 ||
                        dW_dtype == HASTE_DTYPE_F16,
                    "haste_ffi_bwd_weights: bad dW dtype %d", (int)dW_dtype);
    HASTE_CHECK_ARG(dbias == nullptr || dbias_dtype == HASTE_DTYPE_F32 ||
                        dbias_dtype == HASTE_DTYPE_BF16 || dbias_dtype == HASTE_DTYPE_F16,
                    "haste_ffi_bwd_weights: bad dbias dtype %d", (int)dbias_dtype);
    auto* x = static_cast<const uint16_t*>(xT);
    auto* y = static_cast<const uint16_t*>(dY);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == HASTE_DTYPE_BF16)
        return haste::dispatch_g<haste::BF16>(idx, x, ldx, y, lddy, dW, dW_dtype, dbias,
                                              dbias_dtype, B, D, F, O, G, st);
    return haste::dispatch_g<haste::F16>(idx, x, ldx, y, lddy, dW, dW_dtype, dbias, dbias_dtype,
                                         B, D, F, O, G, st);
}
