// Grouped fixed-fan-in backward to weights (+ bias gradient), gfx950.
//
//   dW[l, j] = sum_b dY[b, l] * xT[idx[g, j], b]        g = l / G
//   dbias[l] = sum_b dY[b, l]
//
// One workgroup per label group; the contraction runs over the whole batch.
// MFMA orientation: M = fan-in slots, N = labels, K = batch.
//  - A (slots x batch) comes straight from L2: for slot j a fragment is 8
//    consecutive batch entries of row xT[idx[g, j]] (one 16-byte load).
//  - B (batch x labels) is dY[b, g*G:(g+1)*G], copied row-major into LDS in
//    chunks of 64 batch rows (double-buffered, the next chunk's loads in flight
//    during the current chunk's MFMAs) and read back with ds_read_b64_tr_b16,
//    which hands each lane 4 consecutive batch values of one label: dY needs no
//    transposition pass.
//  - D holds 4 consecutive slots of one label per lane: dW rows are written 16
//    bytes (fp32) per lane.
// The bias gradient is one extra MFMA per label tile with A = ones, so dY is
// read once for both outputs (the reference reads it a second time for
// torch.sum, shared_ffi/bindings.py:40).
#include <algorithm>

#include "common.hpp"

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

constexpr int kThreads = 256;
constexpr int kKC = 64;  // batch rows per LDS stage

template <int G, int FP>
struct BwdWCfg {
    static constexpr int MTILES = FP / 16;                    // slot tiles
    static constexpr int NTILES = G / 16;                     // label tiles
    static constexpr int WM = MTILES < 4 ? MTILES : 4;        // waves along slots
    static constexpr int WN0 = 4 / WM;
    static constexpr int WN = NTILES < WN0 ? NTILES : WN0;    // waves along labels
    static constexpr int MT = MTILES / WM;
    static constexpr int NT = NTILES / WN;
    static constexpr int RB = 2 * G + 16;                     // LDS bytes per staged dY row
    static constexpr int PIECES = kKC * G / 8;                // 16-byte pieces per chunk
    static constexpr int PPT = (PIECES + kThreads - 1) / kThreads;
};

template <typename T>
__device__ __forceinline__ uint32_t one_pair();
template <>
__device__ __forceinline__ uint32_t one_pair<BF16>() { return 0x3F803F80u; }
template <>
__device__ __forceinline__ uint32_t one_pair<F16>() { return 0x3C003C00u; }

typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4 of
// the 8-byte rows addressed by lanes 4k + i/4 (k = 0..3) as its element k.
__device__ __forceinline__ u32x2 lds_read_tr16(const char* p) {
    typedef fp16x4_t __attribute__((address_space(3))) * lds_p;
    const fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (lds_p)(__attribute__((address_space(3))) char*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// Two waves per SIMD (at most 256 registers each) hide the chunk pipeline's load
// latency; the largest tile set (G = 128, 256 slots) needs more registers.
template <int G, int FP>
constexpr int bwdw_waves_per_simd() { return G * FP >= 128 * 256 ? 1 : 2; }

template <typename T, int G, int FP>
__global__ __launch_bounds__(kThreads, (bwdw_waves_per_simd<G, FP>())) void ffi_bwd_w_kernel(
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ xT, int64_t ldx,
    const uint16_t* __restrict__ dY, int64_t lddy, void* __restrict__ dW, int dW_dtype,
    void* __restrict__ dbias, int dbias_dtype, int B, int D, int F, int64_t O) {
    using C = BwdWCfg<G, FP>;
    constexpr int MT = C::MT, NT = C::NT, RB = C::RB, PPT = C::PPT;
    __shared__ __attribute__((aligned(16))) char Ys[2][kKC * RB];

    const int64_t g = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % C::WM, wn = wave / C::WM;
    const bool active = wn < C::WN;
    const int col = lane & 15, kq = lane >> 4;
    const int64_t l0 = g * G;
    const int nchunks = (B + kKC - 1) / kKC;

    // A rows: this lane's slots
    const uint16_t* xrow[MT];
    bool jvalid[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int j = (wm * MT + mt) * 16 + col;
        jvalid[mt] = active && j < F;
        const int d = jvalid[mt] ? min(max(idx[g * F + j], 0), D - 1) : 0;
        xrow[mt] = xT + (int64_t)d * ldx;
    }

    // dY chunk c (rows c*64 ..) -> registers; rows >= B and labels >= O are zero
    auto fetch = [&](int c, u32x4 (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int p = tid + q * kThreads;
            const int r = p / (G / 8), cc = p % (G / 8);
            const int64_t b = (int64_t)c * kKC + r;
            const int64_t l = l0 + cc * 8;
            v[q] = u32x4{0u, 0u, 0u, 0u};
            if (p < C::PIECES && b < B) {
                if (l + 8 <= O) {
                    v[q] = *reinterpret_cast<const u32x4*>(dY + b * lddy + l);
                } else if (l < O) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (l + e < O) v[q][e >> 1] |= (uint32_t)dY[b * lddy + l + e] << ((e & 1) * 16);
                }
            }
        }
    };
    auto stash = [&](int buf, const u32x4 (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int p = tid + q * kThreads;
            if (p < C::PIECES) {
                const int r = p / (G / 8), cc = p % (G / 8);
                *reinterpret_cast<u32x4*>(&Ys[buf][r * RB + cc * 16]) = v[q];
            }
        }
    };
    // A fragments of chunk c: 8 consecutive batch entries of each slot row
    // (entries >= B read as zero)
    auto fetch_a = [&](int c, u32x4 (&a)[2][MT]) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int bk = c * kKC + ks * 32 + kq * 8;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                u32x4 v = u32x4{0u, 0u, 0u, 0u};
                if (jvalid[mt] && bk < B) {
                    v = *reinterpret_cast<const u32x4*>(xrow[mt] + bk);
                    if (bk + 8 > B) {
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (bk + e >= B) v[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                    }
                }
                a[ks][mt] = v;
            }
        }
    };

    f32x4 acc[MT][NT];
    f32x4 accb[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        accb[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const uint32_t op = one_pair<T>();
    const u32x4 ones = u32x4{op, op, op, op};
    const bool do_bias = dbias != nullptr && wm == 0 && active;

    u32x4 yv[PPT];
    fetch(0, yv);
    stash(0, yv);
    if (nchunks > 1) fetch(1, yv);
    u32x4 a[2][MT];
    fetch_a(0, a);
    __syncthreads();

    // lane's tr-read address inside a staged chunk: row 8*kq + 4*half + col/4,
    // labels n0 + 4*(col%4)
    const int tr_off = (kq * 8 + col / 4) * RB + (col % 4) * 8;
    for (int c = 0; c < nchunks; ++c) {
        const char* ys = Ys[c & 1];
        u32x4 an[2][MT];
        if (c + 1 < nchunks) fetch_a(c + 1, an);
        if (active) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const char* p = ys + tr_off + ks * 32 * RB + (wn * NT + nt) * 32;
                    const u32x2 lo = lds_read_tr16(p);
                    const u32x2 hi = lds_read_tr16(p + 4 * RB);
                    const u32x4 bf = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[mt][nt] = mfma16x16x32<T>(a[ks][mt], bf, acc[mt][nt]);
                    if (do_bias) accb[nt] = mfma16x16x32<T>(ones, bf, accb[nt]);
                }
            }
        }
        if (c + 1 < nchunks) {
            stash((c + 1) & 1, yv);
            if (c + 2 < nchunks) fetch(c + 2, yv);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) a[ks][mt] = an[ks][mt];
        }
        __syncthreads();
    }

    if (!active) return;
    // ---- epilogue: lane holds slots 4*kq..+3 of label col in each tile ----
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int64_t l = l0 + (wn * NT + nt) * 16 + col;
        if (l >= O) continue;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int j = (wm * MT + mt) * 16 + kq * 4;
            if (j >= F) continue;
            const f32x4 v = acc[mt][nt];
            if (dW_dtype == HASTE_DTYPE_F32) {
                *reinterpret_cast<f32x4*>(static_cast<float*>(dW) + l * F + j) = v;
            } else {
                u32x2 h;
                if (dW_dtype == HASTE_DTYPE_BF16) {
                    h[0] = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
                    h[1] = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
                } else {
                    h[0] = f32_to_f16_rne(v[0]) | (f32_to_f16_rne(v[1]) << 16);
                    h[1] = f32_to_f16_rne(v[2]) | (f32_to_f16_rne(v[3]) << 16);
                }
                *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(dW) + l * F + j) = h;
            }
        }
        if (do_bias && kq == 0) {
            const float v = accb[nt][0];
            if (dbias_dtype == HASTE_DTYPE_F32)
                static_cast<float*>(dbias)[l] = v;
            else if (dbias_dtype == HASTE_DTYPE_BF16)
                static_cast<uint16_t*>(dbias)[l] = (uint16_t)f32_to_bf16_rne(v);
            else
                static_cast<uint16_t*>(dbias)[l] = (uint16_t)f32_to_f16_rne(v);
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
