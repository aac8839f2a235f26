// Grouped fixed-fan-in forward (gfx950).
//
//   out[b, l] = RNE( sum_j xT[idx[g, j], b] * W[l, j] + bias[l] ),  g = l / G
//
// One workgroup = one label group g x a chunk of the batch.  Per batch tile of
// 64 columns, the gathered rows xT[idx[g, :], b0:b0+64] are loaded with 16-byte
// loads (xT is tiny and L2 resident), transposed in registers and stored to LDS
// as Xs[b][j] so each MFMA B-fragment is one 16-byte LDS read.  W fragments
// (MFMA A operand: label rows x 8 contiguous fan-in slots) are loaded straight
// from HBM into VGPRs once per workgroup and reused over the whole batch chunk.
// bf16/f16 MFMA 16x16x32 with fp32 accumulation; bias is added in fp32 and the
// result rounded to nearest even (as dump_and_store_tile,
// shared_ffi/ffi_forward_kernels.cu:85-101).
#include <algorithm>

#include "common.hpp"

namespace haste {
namespace {

constexpr int kBT = 64;       // batch columns per tile
constexpr int kThreads = 256; // 4 waves

template <typename T, int G, int FP>
struct FwdCfg {
    static constexpr int KS = FP / 32;            // MFMA k-steps
    static constexpr int MTILES = G / 16;         // label tiles in the group
    static constexpr int WM = MTILES < 4 ? MTILES : 4;  // waves along labels
    static constexpr int WN = 4 / WM;             // waves along batch
    static constexpr int MT = MTILES / WM;        // label tiles per wave
    static constexpr int NT = (kBT / 16) / WN;    // batch tiles per wave
    static constexpr int LDX = FP + 8;            // LDS row pitch (elements), +16 B vs bank conflicts
    static constexpr int ITEMS = (FP / 4) * (kBT / 8);  // gather items per batch tile
};

__device__ __forceinline__ uint32_t half_of(const u32x4& v, int e) {
    return (e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xFFFFu);
}

template <typename T, int G, int FP>
__global__ __launch_bounds__(kThreads) void ffi_fwd_kernel(
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ xT, int64_t ldx,
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int B, int D, int F, int64_t O, int64_t Gc, int nchunks, int tiles_per_chunk) {
    using C = FwdCfg<T, G, FP>;
    __shared__ __attribute__((aligned(16))) uint16_t Xs[kBT * C::LDX];
    __shared__ int32_t sidx[FP];

    const int64_t work = xcd_remap(blockIdx.x, Gc * nchunks);
    if (work < 0) return;
    const int64_t g = work / nchunks;
    const int chunk = (int)(work % nchunks);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave % C::WM;
    const int wn = wave / C::WM;
    const int lrow = lane & 15;  // row of A / column of B / column of D
    const int lq = lane >> 4;    // quad: K-chunk of A/B, row-quad of D

    // Indices outside [0, D) are clamped (the reference leaves them undefined).
    for (int j = tid; j < FP; j += kThreads)
        sidx[j] = j < F ? min(max(idx[g * F + j], 0), D - 1) : 0;

    // W fragments (A operand) and bias for this wave's label tiles.
    u32x4 wf[C::MT][C::KS];
    float bv[C::MT][4];
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) {
        const int64_t l = g * G + (int64_t)(wm * C::MT + mt) * 16 + lrow;
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
            const int k = ks * 32 + lq * 8;
            if (l < O && k < F)
                wf[mt][ks] = *reinterpret_cast<const u32x4*>(W + l * F + k);
            else
                wf[mt][ks] = u32x4{0u, 0u, 0u, 0u};
        }
        const int64_t lb = g * G + (int64_t)(wm * C::MT + mt) * 16 + lq * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            bv[mt][i] = (bias != nullptr && lb + i < O) ? bits_to_f32<T>(bias[lb + i]) : 0.0f;
    }
    __syncthreads();

    const int b_chunk0 = chunk * tiles_per_chunk * kBT;
    for (int t = 0; t < tiles_per_chunk; ++t) {
        const int b_base = b_chunk0 + t * kBT;
        if (b_base >= B) break;

        // ---- gather xT[idx[j], b_base + 0..63] into Xs[b][j] ----
        for (int it = tid; it < C::ITEMS; it += kThreads) {
            const int jq = it % (FP / 4);
            const int bo = it / (FP / 4);
            const int j0 = jq * 4;
            const int b0 = b_base + bo * 8;
            u32x4 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (j0 + q < F && b0 < B)
                    v[q] = *reinterpret_cast<const u32x4*>(xT + (int64_t)sidx[j0 + q] * ldx + b0);
                else
                    v[q] = u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                uint32_t lo = half_of(v[0], e) | (half_of(v[1], e) << 16);
                uint32_t hi = half_of(v[2], e) | (half_of(v[3], e) << 16);
                if (b0 + e >= B) { lo = 0u; hi = 0u; }
                *reinterpret_cast<u32x2*>(&Xs[(bo * 8 + e) * C::LDX + j0]) = u32x2{lo, hi};
            }
        }
        __syncthreads();

        // ---- MFMA: D[label][batch] = W_tile x Xg^T ----
        f32x4 acc[C::MT][C::NT];
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt) {
            const int n0 = (wn * C::NT + nt) * 16;
#pragma unroll
            for (int ks = 0; ks < C::KS; ++ks) {
                const u32x4 bfrag =
                    *reinterpret_cast<const u32x4*>(&Xs[(n0 + lrow) * C::LDX + ks * 32 + lq * 8]);
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
                    acc[mt][nt] = mfma16x16x32<T>(wf[mt][ks], bfrag, acc[mt][nt]);
            }
        }

        // ---- epilogue: + bias (fp32), RNE, store 4 consecutive labels per lane ----
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt) {
            const int b = b_base + (wn * C::NT + nt) * 16 + lrow;
            if (b >= B) continue;
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt) {
                const int64_t l = g * G + (int64_t)(wm * C::MT + mt) * 16 + lq * 4;
                uint32_t h[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) h[i] = f32_to_bits<T>(acc[mt][nt][i] + bv[mt][i]);
                uint16_t* dst = out + (int64_t)b * ldo + l;
                if (l + 3 < O) {
                    *reinterpret_cast<u32x2*>(dst) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (l + i < O) dst[i] = (uint16_t)h[i];
                }
            }
        }
        __syncthreads();
    }
}

template <typename T, int G, int FP>
int launch_fwd(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* W,
               const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t B, int64_t D, int64_t F,
               int64_t O, hipStream_t st) {
    const int64_t Gc = ceil_div(O, G);
    const int64_t ntiles = ceil_div(B, kBT);
    int64_t tpc = std::max<int64_t>(1, std::min<int64_t>(ntiles, (Gc * ntiles) / 8192));
    const int64_t nchunks = ceil_div(ntiles, tpc);
    const int64_t nlogical = Gc * nchunks;
    const int64_t grid = 8 * ceil_div(nlogical, 8);
    if (grid > 0x7FFFFFFF) {
        set_error("haste_ffi_forward: problem too large (grid %lld)", (long long)grid);
        return HASTE_ERR_UNSUPPORTED;
    }
    ffi_fwd_kernel<T, G, FP><<<dim3((unsigned)grid), dim3(kThreads), 0, st>>>(
        idx, xT, ldx, W, bias, out, ldo, (int)B, (int)D, (int)F, O, Gc, (int)nchunks, (int)tpc);
    HASTE_CHECK_LAUNCH("haste_ffi_forward");
    return HASTE_OK;
}

template <typename T, int G>
int dispatch_fp(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* W,
                const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t B, int64_t D, int64_t F,
                int64_t O, hipStream_t st) {
    if (F <= 32) return launch_fwd<T, G, 32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
    if (F <= 64) return launch_fwd<T, G, 64>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
    if (F <= 128) return launch_fwd<T, G, 128>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
    return launch_fwd<T, G, 256>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
}

template <typename T>
int dispatch_g(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* W,
               const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t B, int64_t D, int64_t F,
               int64_t O, int64_t G, hipStream_t st) {
    switch (G) {
    case 16: return dispatch_fp<T, 16>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
    case 32: return dispatch_fp<T, 32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
    case 64: return dispatch_fp<T, 64>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
    case 128: return dispatch_fp<T, 128>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, st);
    default: break;
    }
    set_error("Unsupported group size for FFI kernel. choose from 16,32,64,128 (got %lld)",
              (long long)G);
    return HASTE_ERR_UNSUPPORTED;
}

}  // namespace

// Shape checks shared by the three FFI entry points.
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype) {
    if (dtype != HASTE_DTYPE_BF16 && dtype != HASTE_DTYPE_F16) {
        set_error("%s: unsupported dtype code %d (bf16 or f16 only)", fn, (int)dtype);
        return HASTE_ERR_UNSUPPORTED;
    }
    if (G != 16 && G != 32 && G != 64 && G != 128) {
        set_error("Unsupported group size for FFI kernel. choose from 16,32,64,128 (got %lld)",
                  (long long)G);
        return HASTE_ERR_UNSUPPORTED;
    }
    if (F % 16 != 0 || F < 16) {
        set_error("FANIN size should be multiple of 16 and >=16 (got %lld)", (long long)F);
        return HASTE_ERR_INVALID_ARG;
    }
    if (F > 256) {
        set_error("FANIN should be <=256 (got %lld)", (long long)F);
        return HASTE_ERR_UNSUPPORTED;
    }
    if (B <= 0) {
        set_error("batch size B must be positive (got %lld)", (long long)B);
        return HASTE_ERR_INVALID_ARG;
    }
    if (B > 0x7FFFFFFF || D <= 0 || D > 0x7FFFFFFF || O <= 0) {
        set_error("%s: invalid sizes B=%lld D=%lld O=%lld", fn, (long long)B, (long long)D,
                  (long long)O);
        return HASTE_ERR_INVALID_ARG;
    }
    (void)fn;
    return HASTE_OK;
}

}  // namespace haste

extern "C" int haste_ffi_forward(const int32_t* idx, const void* xT, int64_t ldx, const void* W,
                                 const void* bias, void* out, int64_t ldo, int64_t B, int64_t D,
                                 int64_t F, int64_t O, int64_t G, int32_t dtype, void* stream) {
    int rc = haste::check_ffi_shape("haste_ffi_forward", B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && xT && W && out, "haste_ffi_forward: null pointer");
    HASTE_CHECK_ARG(ldx >= B && ldx % 8 == 0,
                    "haste_ffi_forward: ldx must be >= B and a multiple of 8 (ldx=%lld B=%lld)",
                    (long long)ldx, (long long)B);
    HASTE_CHECK_ARG(ldo >= O && ldo % 8 == 0,
                    "haste_ffi_forward: ldo must be >= O and a multiple of 8 (ldo=%lld O=%lld)",
                    (long long)ldo, (long long)O);
    HASTE_CHECK_ARG(haste::aligned16(xT) && haste::aligned16(W) && haste::aligned16(out),
                    "haste_ffi_forward: xT, W and out must be 16-byte aligned");
    auto* x = static_cast<const uint16_t*>(xT);
    auto* w = static_cast<const uint16_t*>(W);
    auto* bb = static_cast<const uint16_t*>(bias);
    auto* o = static_cast<uint16_t*>(out);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == HASTE_DTYPE_BF16)
        return haste::dispatch_g<haste::BF16>(idx, x, ldx, w, bb, o, ldo, B, D, F, O, G, st);
    return haste::dispatch_g<haste::F16>(idx, x, ldx, w, bb, o, ldo, B, D, F, O, G, st);
}
