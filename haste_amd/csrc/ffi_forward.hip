// Grouped fixed-fan-in forward (gfx950).
//
//   out[b, l] = RNE( sum_j xT[idx[g, j], b] * W[l, j] + bias[l] ),  g = l / G
//
// One workgroup = one label group g x a chunk of the batch, in tiles of 64
// batch columns.  MFMA orientation: M = labels, N = batch, K = fan-in slots.
//  - A: W fragments (label rows x 8 contiguous slots) loaded once per
//    workgroup from HBM into VGPRs and reused over the whole batch chunk.
//  - B: the gathered rows xT[idx[g, j], b0:b0+64] are copied row-major into LDS
//    (16-byte copies, Xg[slot][batch]; xT is small and L2 resident) and read
//    back with ds_read_b64_tr_b16, which hands each lane 4 consecutive slots of
//    one batch column.  The next tile's rows are fetched into registers while
//    the current tile's MFMAs run (two LDS buffers).
// bf16/f16 MFMA 16x16x32 with fp32 accumulation; bias is added in fp32 and the
// result rounded to nearest even (as dump_and_store_tile,
// shared_ffi/ffi_forward_kernels.cu:85-101).
#include <algorithm>

#include "common.hpp"

namespace haste {
namespace {

constexpr int kBT = 64;        // batch columns per tile
constexpr int kThreads = 256;  // 4 waves

template <typename T, int G, int FP>
struct FwdCfg {
    static constexpr int KS = FP / 32;                  // MFMA k-steps
    static constexpr int MTILES = G / 16;               // label tiles in the group
    static constexpr int WM = MTILES < 4 ? MTILES : 4;  // waves along labels
    static constexpr int WN = 4 / WM;                   // waves along batch
    static constexpr int MT = MTILES / WM;              // label tiles per wave
    static constexpr int NT = (kBT / 16) / WN;          // batch tiles per wave
    static constexpr int RB = kBT * 2 + 16;             // LDS bytes per gathered row
    static constexpr int PIECES = FP * (kBT / 8);       // 16-byte pieces per tile
    static constexpr int PPT = PIECES / kThreads;       // >= 1 (FP >= 32)
};

typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4 of
// the 8-byte rows addressed by lanes 4k + i/4 (k = 0..3) as its element k.
__device__ __forceinline__ u32x2 lds_read_tr16(const char* p) {
    typedef fp16x4_t __attribute__((address_space(3))) * lds_p;
    const fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (lds_p)(__attribute__((address_space(3))) char*)(p));
    return __builtin_bit_cast(u32x2, v);
}

template <typename T, int G, int FP>
__global__ __launch_bounds__(kThreads, 2) void ffi_fwd_kernel(
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ xT, int64_t ldx,
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int B, int D, int F, int64_t O, int64_t Gc, int nchunks, int tiles_per_chunk) {
    using C = FwdCfg<T, G, FP>;
    constexpr int KS = C::KS, MT = C::MT, NT = C::NT, RB = C::RB, PPT = C::PPT;
    __shared__ __attribute__((aligned(16))) char Xg[2][FP * RB];
    __shared__ int32_t sidx[FP];

    const int64_t work = xcd_remap(blockIdx.x, Gc * nchunks);
    if (work < 0) return;
    const int64_t g = work / nchunks;
    const int chunk = (int)(work % nchunks);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % C::WM, wn = wave / C::WM;
    const int col = lane & 15;  // row of A / column of B / column of D
    const int kq = lane >> 4;   // K-chunk of A/B, row-quad of D

    // Indices outside [0, D) are clamped (the reference leaves them undefined);
    // slots >= F gather row 0 (their W columns are zero).
    for (int j = tid; j < FP; j += kThreads)
        sidx[j] = j < F ? min(max(idx[g * F + j], 0), D - 1) : 0;

    // W fragments (A operand) and bias for this wave's label tiles.
    u32x4 wf[MT][KS];
    float bv[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int64_t l = g * G + (int64_t)(wm * MT + mt) * 16 + col;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int k = ks * 32 + kq * 8;
            if (l < O && k < F)
                wf[mt][ks] = *reinterpret_cast<const u32x4*>(W + l * F + k);
            else
                wf[mt][ks] = u32x4{0u, 0u, 0u, 0u};
        }
        const int64_t lb = g * G + (int64_t)(wm * MT + mt) * 16 + kq * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            bv[mt][i] = (bias != nullptr && lb + i < O) ? bits_to_f32<T>(bias[lb + i]) : 0.0f;
    }
    __syncthreads();

    // piece p of a tile: slot p / 8, batch columns 8 * (p % 8) .. +7
    // (columns >= B read as zero)
    auto fetch = [&](int b_base, u32x4 (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int p = tid + q * kThreads;
            const int j = p / (kBT / 8), b0 = b_base + (p % (kBT / 8)) * 8;
            v[q] = u32x4{0u, 0u, 0u, 0u};
            if (b0 < B) {
                v[q] = *reinterpret_cast<const u32x4*>(xT + (int64_t)sidx[j] * ldx + b0);
                if (b0 + 8 > B) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (b0 + e >= B) v[q][e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                }
            }
        }
    };
    auto stash = [&](int buf, const u32x4 (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int p = tid + q * kThreads;
            *reinterpret_cast<u32x4*>(&Xg[buf][(p / (kBT / 8)) * RB + (p % (kBT / 8)) * 16]) = v[q];
        }
    };

    const int b_chunk0 = chunk * tiles_per_chunk * kBT;
    const int ntiles = min(tiles_per_chunk, (B - b_chunk0 + kBT - 1) / kBT);
    u32x4 xv[PPT];
    fetch(b_chunk0, xv);
    stash(0, xv);
    if (ntiles > 1) fetch(b_chunk0 + kBT, xv);
    __syncthreads();

    // lane's tr-read address: slot 8*kq + col/4 (+4 for the second half), batch
    // columns n0 + 4*(col%4)
    const int tr_off = (kq * 8 + col / 4) * RB + (col % 4) * 8;
    for (int t = 0; t < ntiles; ++t) {
        const int b_base = b_chunk0 + t * kBT;
        const char* xs = Xg[t & 1];
        f32x4 acc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n0 = (wn * NT + nt) * 16;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const char* p = xs + tr_off + ks * 32 * RB + n0 * 2;
                const u32x2 lo = lds_read_tr16(p);
                const u32x2 hi = lds_read_tr16(p + 4 * RB);
                const u32x4 bf = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16x16x32<T>(wf[mt][ks], bf, acc[mt][nt]);
            }
        }
        if (t + 1 < ntiles) {
            stash((t + 1) & 1, xv);
            if (t + 2 < ntiles) fetch(b_base + 2 * kBT, xv);
        }

        // ---- epilogue: + bias (fp32), RNE, store 4 consecutive labels per lane ----
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int b = b_base + (wn * NT + nt) * 16 + col;
            if (b >= B) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int64_t l = g * G + (int64_t)(wm * MT + mt) * 16 + kq * 4;
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
