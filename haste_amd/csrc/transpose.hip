// Feature transpose X [B, D] -> X^T [D, ldt] (2-byte elements), the layout the
// FFI kernels gather from (a feature index selects one contiguous row of B
// values).  64 x 64 tiles staged through LDS; 16-byte loads and stores where a
// row chunk of 8 elements is in bounds and aligned, element accesses otherwise.
// Columns B..ldt-1 of X^T are written as zero, so kernels that read whole
// 8-column chunks never see uninitialised padding.
#include "common.hpp"

namespace haste {
namespace {

constexpr int kT = 64;

__global__ __launch_bounds__(256) void transpose_kernel(const uint16_t* __restrict__ x,
                                                        int64_t ldx, uint16_t* __restrict__ xT,
                                                        int64_t ldt, int64_t B, int64_t D,
                                                        int32_t vec) {
    __shared__ uint16_t tile[kT][kT + 2];
    const int64_t b0 = (int64_t)blockIdx.x * kT;  // output columns (batch)
    const int64_t d0 = (int64_t)blockIdx.y * kT;  // output rows (features)
    const int tid = threadIdx.x;
    // load x[b0 + r][d0 + c .. c+7] -> tile[r][c..c+7]
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r = tid / 8 + 32 * h, c = (tid % 8) * 8;
        const int64_t b = b0 + r, d = d0 + c;
        uint16_t v[8];
        if (vec && b < B && d + 8 <= D) {
            u32x4 q = *reinterpret_cast<const u32x4*>(x + b * ldx + d);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[2 * e] = (uint16_t)(q[e] & 0xFFFFu);
                v[2 * e + 1] = (uint16_t)(q[e] >> 16);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (b < B && d + e < D) ? x[b * ldx + d + e] : 0;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) tile[r][c + e] = v[e];
    }
    __syncthreads();
    // store xT[d0 + r][b0 + c .. c+7] = tile[c..c+7][r]; columns >= B are zero
    const int64_t ncol = ldt;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r = tid / 8 + 32 * h, c = (tid % 8) * 8;
        const int64_t d = d0 + r, b = b0 + c;
        if (d >= D || b >= ncol) continue;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (b + e < B) ? tile[c + e][r] : 0;
        if (vec && b + 8 <= ncol) {
            u32x4 q;
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = (uint32_t)v[2 * e] | ((uint32_t)v[2 * e + 1] << 16);
            *reinterpret_cast<u32x4*>(xT + d * ldt + b) = q;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (b + e < ncol) xT[d * ldt + b + e] = v[e];
        }
    }
}

}  // namespace
}  // namespace haste

extern "C" int haste_transpose_features(const uint16_t* x, int64_t ldx, uint16_t* xT, int64_t ldt,
                                        int64_t B, int64_t D, void* stream) {
    HASTE_CHECK_ARG(B >= 0 && D >= 0, "haste_transpose_features: negative size");
    HASTE_CHECK_ARG(ldx >= D && ldt >= B,
                    "haste_transpose_features: need ldx >= D and ldt >= B (ldx=%lld ldt=%lld)",
                    (long long)ldx, (long long)ldt);
    if (D == 0 || ldt == 0) return HASTE_OK;
    HASTE_CHECK_ARG(xT != nullptr && (B == 0 || x != nullptr),
                    "haste_transpose_features: null pointer");
    const int64_t gx = haste::ceil_div(ldt, (int64_t)haste::kT);
    const int64_t gy = haste::ceil_div(D, (int64_t)haste::kT);
    HASTE_CHECK_ARG(gx < 65536 * 32 && gy < 65536, "haste_transpose_features: matrix too large");
    const int vec = haste::aligned16(x) && haste::aligned16(xT) && ldx % 8 == 0 && ldt % 8 == 0;
    haste::transpose_kernel<<<dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                              static_cast<hipStream_t>(stream)>>>(x, ldx, xT, ldt, B, D, vec);
    HASTE_CHECK_LAUNCH("haste_transpose_features");
    return HASTE_OK;
}
