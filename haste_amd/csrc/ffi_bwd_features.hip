// Grouped fixed-fan-in backward to features, deterministic (gfx950).
//
//   dXT[d, b] = sum_{g, j: idx[g, j] = d} sum_{l in g} W[l, j] * dY[b, l]
//
// The reference scatters with fp32 atomicAdd into global memory
// (shared_ffi/ffi_backward_features.cu:202-212), so its sums depend on timing.
// Here no float atomic ever touches global memory and every sum has a fixed
// order:
//
//  1. prep: per group, the F slots are stably sorted by index.  Equal indices
//     become adjacent; a slot's "colour" is (its rank inside its run of equal
//     indices) / 4.
//  2. main: workgroup (group slice s, feature range dr, batch tile bt) keeps a
//     partial dXT[d in dr, b in bt] in LDS (fp32).  For each group of its slice,
//     in order, it stages W_g transposed in LDS, splits the sorted positions
//     between its 4 waves at run boundaries (so no two waves own the same
//     feature), and each wave computes P = W_g^T dY_g^T for its positions with
//     MFMA (M = sorted positions, N = batch, K = labels) and adds the rows into
//     the LDS partial.  One add instruction covers positions p, p+4, p+8, p+12
//     of one batch column; those can only collide inside a run of >= 5 equal
//     indices, and such lanes are separated into colour passes.  All adds to one
//     LDS word therefore come from one wave, in program order.
//  3. reduce: dXT = sum over slices s = 0..S-1 in ascending order (fp32 out), or
//     fused with the bf16 stochastic rounding of shared_ffi/bindings.py:44-48.
#include <algorithm>

#include "common.hpp"

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

constexpr int kThreads = 256;
constexpr int kBT = 32;  // batch columns per workgroup
constexpr int kLdsBytes = 160 * 1024;
constexpr int kTargetCTAs = 256;

// LDS row pitch of the staged W_g^T (elements) and the largest feature range a
// workgroup can hold in its LDS partial for a given (G, FP).
constexpr int ws_pitch(int G) { return G + 8; }
constexpr int max_dc(int G, int FP) {
    return (kLdsBytes - FP * ws_pitch(G) * 2 - FP * 8 - 256) / 4 / kBT;
}
int max_dc_rt(int64_t G, int64_t F) {
    const int FP = F <= 32 ? 32 : F <= 64 ? 64 : F <= 128 ? 128 : 256;
    return max_dc((int)G, FP);
}

struct BwdFPlan {
    int64_t Gc, nbt, Bp, ndr, Dc, S, gps;  // gps = groups per slice
    int64_t prep_bytes, ws_bytes;
};

BwdFPlan make_plan(int64_t B, int64_t D, int64_t F, int64_t O, int64_t G) {
    BwdFPlan p;
    p.Gc = ceil_div(O, G);
    p.nbt = ceil_div(B, kBT);
    p.Bp = p.nbt * kBT;
    p.ndr = ceil_div(D, max_dc_rt(G, F));
    p.Dc = ceil_div(D, p.ndr);
    int64_t S = std::max<int64_t>(1, kTargetCTAs / (p.nbt * p.ndr));
    S = std::min<int64_t>(S, std::max<int64_t>(1, ceil_div(p.Gc, 8)));
    p.gps = ceil_div(p.Gc, S);
    p.S = ceil_div(p.Gc, p.gps);
    p.prep_bytes = ((p.Gc * F * 8) + 255) / 256 * 256;
    p.ws_bytes = p.S * D * p.Bp * 4;
    return p;
}

// --------------------------------------------------------------- prep ------
// sorted[g*F + p] = {index, slot | colour << 16} for sorted position p.
__global__ __launch_bounds__(kThreads) void bwdf_prep_kernel(const int32_t* __restrict__ idx,
                                                             int2* __restrict__ sorted, int F,
                                                             int D) {
    __shared__ int32_t s[256];
    const int64_t g = blockIdx.x;
    const int j = threadIdx.x;
    if (j < F) s[j] = min(max(idx[g * F + j], 0), D - 1);
    __syncthreads();
    if (j >= F) return;
    const int v = s[j];
    int rank = 0, run = 0;
    for (int q = 0; q < F; ++q) {
        const int u = s[q];
        rank += (u < v) || (u == v && q < j);
        run += (u == v && q < j);
    }
    sorted[g * F + rank] = make_int2(v, j | ((run >> 2) << 16));
}

// --------------------------------------------------------------- main ------
template <typename T, int G, int FP>
struct BwdFCfg {
    static constexpr int KS = G >= 32 ? G / 32 : 1;  // MFMA k-steps over labels
    static constexpr int LDW = ws_pitch(G);          // Ws row pitch (elements)
    static constexpr int ACC = max_dc(G, FP) * kBT;  // LDS partial size (floats)
    static constexpr int NT = kBT / 16;              // batch n-tiles (all owned by each wave)
    static constexpr int ITEMS = (G / 4) * (FP / 8); // W staging items
};

template <typename T, int G, int FP>
__global__ __launch_bounds__(kThreads) void bwdf_main_kernel(
    const int2* __restrict__ sorted, const uint16_t* __restrict__ W,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int F, int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S) {
    using C = BwdFCfg<T, G, FP>;
    __shared__ float acc[C::ACC];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[FP * C::LDW];
    __shared__ int2 ss[FP];
    __shared__ int bounds[5];

    const int64_t work = xcd_remap(blockIdx.x, (int64_t)S * ndr * nbt);
    if (work < 0) return;
    const int bt = (int)(work % nbt);
    const int dr = (int)((work / nbt) % ndr);
    const int s = (int)(work / ((int64_t)nbt * ndr));
    const int d_lo = dr * Dc;
    const int d_hi = min(D, d_lo + Dc);
    const int b_base = bt * kBT;
    const int64_t g_begin = (int64_t)s * gps;
    const int64_t g_end = min(Gc, g_begin + gps);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lrow = lane & 15;
    const int lq = lane >> 4;

    for (int i = tid; i < (d_hi - d_lo) * kBT; i += kThreads) acc[i] = 0.0f;

    for (int64_t g = g_begin; g < g_end; ++g) {
        const int64_t l0 = g * G;
        // ---- sorted slot table + W_g^T staging ----
        for (int p = tid; p < F; p += kThreads) ss[p] = sorted[g * F + p];
        for (int it = tid; it < C::ITEMS; it += kThreads) {
            const int lq4 = it % (G / 4);
            const int jo = it / (G / 4);
            const int lc = lq4 * 4;
            const int j0 = jo * 8;
            u32x4 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (l0 + lc + q < O && j0 < F)
                    v[q] = *reinterpret_cast<const u32x4*>(W + (l0 + lc + q) * F + j0);
                else
                    v[q] = u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int sh = (e & 1) * 16;
                uint32_t a0 = (v[0][e >> 1] >> sh) & 0xFFFFu, a1 = (v[1][e >> 1] >> sh) & 0xFFFFu;
                uint32_t a2 = (v[2][e >> 1] >> sh) & 0xFFFFu, a3 = (v[3][e >> 1] >> sh) & 0xFFFFu;
                *reinterpret_cast<u32x2*>(&Ws[(j0 + e) * C::LDW + lc]) =
                    u32x2{a0 | (a1 << 16), a2 | (a3 << 16)};
            }
        }
        __syncthreads();

        // ---- positions of this workgroup's feature range, split at run starts ----
        if (tid < 5) {
            // lower_bound of d_lo and d_hi in the sorted indices
            int lo = 0, hi = F;
            while (lo < hi) { int m = (lo + hi) >> 1; if (ss[m].x < d_lo) lo = m + 1; else hi = m; }
            const int P0 = lo;
            lo = P0; hi = F;
            while (lo < hi) { int m = (lo + hi) >> 1; if (ss[m].x < d_hi) lo = m + 1; else hi = m; }
            const int P1 = lo;
            int t = P0 + ((P1 - P0) * tid) / 4;
            while (t > P0 && t < P1 && ss[t].x == ss[t - 1].x) ++t;
            bounds[tid] = tid == 4 ? P1 : t;
        }
        __syncthreads();
        const int pb = bounds[wave];
        const int pe = bounds[wave + 1];

        if (pb < pe) {
            // B fragments: dY[b][l0 + k], 8 consecutive labels per lane.
            u32x4 bfr[C::NT][C::KS];
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) {
                const int b = b_base + nt * 16 + lrow;
#pragma unroll
                for (int ks = 0; ks < C::KS; ++ks) {
                    const int k = ks * 32 + lq * 8;
                    if (b < B && k < G && l0 + k < O) {
                        bfr[nt][ks] = *reinterpret_cast<const u32x4*>(dY + (int64_t)b * lddy + l0 + k);
                        if (l0 + k + 8 > O) {
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                if (l0 + k + e >= O) bfr[nt][ks][e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                        }
                    } else {
                        bfr[nt][ks] = u32x4{0u, 0u, 0u, 0u};
                    }
                }
            }
            for (int m0 = pb; m0 < pe; m0 += 16) {
                // A fragments: rows = sorted positions, 8 consecutive labels from Ws.
                const int pa = m0 + lrow;
                const int slot = pa < pe ? (ss[pa].y & 0xFFFF) : 0;
                f32x4 c[C::NT];
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt) c[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < C::KS; ++ks) {
                    const int k = ks * 32 + lq * 8;
                    u32x4 af = u32x4{0u, 0u, 0u, 0u};
                    if (pa < pe && k < G) af = *reinterpret_cast<const u32x4*>(&Ws[slot * C::LDW + k]);
#pragma unroll
                    for (int nt = 0; nt < C::NT; ++nt) c[nt] = mfma16x16x32<T>(af, bfr[nt][ks], c[nt]);
                }
                // Scatter rows of P into the LDS partial.  D row r = 4*lq + i.
                int dl[4], col[4];
                int maxc = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int p = m0 + lq * 4 + i;
                    if (p < pe) {
                        const int2 e = ss[p];
                        dl[i] = e.x - d_lo;
                        col[i] = e.y >> 16;
                    } else {
                        dl[i] = -1;
                        col[i] = 0;
                    }
                    maxc = max(maxc, col[i]);
                }
                // wave-uniform maximum colour
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) maxc = max(maxc, __shfl_xor(maxc, off));
                for (int cc = 0; cc <= maxc; ++cc) {
#pragma unroll
                    for (int nt = 0; nt < C::NT; ++nt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if (dl[i] >= 0 && col[i] == cc)
                                atomicAdd(&acc[dl[i] * kBT + nt * 16 + lrow], c[nt][i]);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    // ---- write the partial: ws[s][d][bt*32 + b] ----
    for (int i = tid; i < (d_hi - d_lo) * kBT; i += kThreads) {
        const int d = i / kBT, b = i % kBT;
        ws[((int64_t)s * D + d_lo + d) * Bp + b_base + b] = acc[i];
    }
}

// ------------------------------------------------------------- reduce ------
__global__ __launch_bounds__(256) void bwdf_reduce_kernel(const float* __restrict__ ws,
                                                          float* __restrict__ dXT, int B, int Bp,
                                                          int D, int S) {
    const int64_t n = (int64_t)D * B;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t d = i / B, b = i % B;
        float v = 0.0f;
        for (int s = 0; s < S; ++s) v += ws[((int64_t)s * D + d) * Bp + b];
        dXT[i] = v;
    }
}

// Sum over slices, transpose [D, B] -> [B, D] and stochastically round to bf16
// with tl.randint(seed, b*D + d).  Tile: 32 features x 32 batch columns.
__global__ __launch_bounds__(256) void bwdf_reduce_sr_kernel(const float* __restrict__ ws,
                                                             uint16_t* __restrict__ dX, int B,
                                                             int Bp, int D, int S, uint32_t k0,
                                                             uint32_t k1) {
    __shared__ float t[32][33];
    const int d0 = blockIdx.x * 32, b0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // ty in 0..7
    for (int r = ty; r < 32; r += 8) {
        const int d = d0 + r, b = b0 + tx;
        float v = 0.0f;
        if (d < D && b < B)
            for (int s = 0; s < S; ++s) v += ws[((int64_t)s * D + d) * Bp + b];
        t[r][tx] = v;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int b = b0 + r, d = d0 + tx;
        if (d < D && b < B) {
            const uint64_t off = (uint64_t)b * D + d;
            dX[(int64_t)b * D + d] =
                (uint16_t)sr_bf16(t[tx][r], philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1));
        }
    }
}

template <typename T, int G, int FP>
int launch_main(const int2* sorted, const uint16_t* W, const uint16_t* dY, int64_t lddy,
                float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O,
                hipStream_t st) {
    const int64_t nlog = p.S * p.ndr * p.nbt;
    const int64_t grid = 8 * ceil_div(nlog, 8);
    bwdf_main_kernel<T, G, FP><<<dim3((unsigned)grid), dim3(kThreads), 0, st>>>(
        sorted, W, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, (int)F, O, p.Gc, (int)p.nbt,
        (int)p.ndr, (int)p.Dc, (int)p.gps, (int)p.S);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

template <typename T, int G>
int dispatch_fp(const int2* sorted, const uint16_t* W, const uint16_t* dY, int64_t lddy, float* ws,
                const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O, hipStream_t st) {
    if (F <= 32) return launch_main<T, G, 32>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
    if (F <= 64) return launch_main<T, G, 64>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
    if (F <= 128) return launch_main<T, G, 128>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
    return launch_main<T, G, 256>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
}

template <typename T>
int dispatch_g(const int2* sorted, const uint16_t* W, const uint16_t* dY, int64_t lddy, float* ws,
               const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
               hipStream_t st) {
    switch (G) {
    case 16: return dispatch_fp<T, 16>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
    case 32: return dispatch_fp<T, 32>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
    case 64: return dispatch_fp<T, 64>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
    default: return dispatch_fp<T, 128>(sorted, W, dY, lddy, ws, p, B, D, F, O, st);
    }
}

// Runs prep + main; leaves the per-slice partials in the workspace.
int run_partials(const char* fn, const int32_t* idx, const void* W, const void* dY, int64_t lddy,
                 void* workspace, int64_t workspace_bytes, int64_t B, int64_t D, int64_t F,
                 int64_t O, int64_t G, int32_t dtype, hipStream_t st, BwdFPlan* plan_out) {
    int rc = check_ffi_shape(fn, B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && W && dY, "%s: null pointer", fn);
    HASTE_CHECK_ARG(lddy >= O && lddy % 8 == 0,
                    "%s: lddy must be >= O and a multiple of 8 (lddy=%lld O=%lld)", fn,
                    (long long)lddy, (long long)O);
    HASTE_CHECK_ARG(aligned16(W) && aligned16(dY) && aligned16(workspace),
                    "%s: W, dY and workspace must be 16-byte aligned", fn);
    const BwdFPlan p = make_plan(B, D, F, O, G);
    if (workspace == nullptr || workspace_bytes < p.prep_bytes + p.ws_bytes) {
        set_error("%s: workspace too small (%lld bytes, need %lld)", fn,
                  (long long)workspace_bytes, (long long)(p.prep_bytes + p.ws_bytes));
        return HASTE_ERR_WORKSPACE;
    }
    int2* sorted = static_cast<int2*>(workspace);
    float* ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.prep_bytes);
    bwdf_prep_kernel<<<dim3((unsigned)p.Gc), dim3(kThreads), 0, st>>>(idx, sorted, (int)F, (int)D);
    HASTE_CHECK_LAUNCH(fn);
    auto* w = static_cast<const uint16_t*>(W);
    auto* y = static_cast<const uint16_t*>(dY);
    rc = dtype == HASTE_DTYPE_BF16 ? dispatch_g<BF16>(sorted, w, y, lddy, ws, p, B, D, F, O, G, st)
                                   : dispatch_g<F16>(sorted, w, y, lddy, ws, p, B, D, F, O, G, st);
    *plan_out = p;
    return rc;
}

}  // namespace
}  // namespace haste

extern "C" int64_t haste_ffi_bwd_features_workspace_size(int64_t B, int64_t D, int64_t F,
                                                         int64_t O, int64_t G, int32_t dtype) {
    int rc = haste::check_ffi_shape("haste_ffi_bwd_features_workspace_size", B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    const haste::BwdFPlan p = haste::make_plan(B, D, F, O, G);
    return p.prep_bytes + p.ws_bytes;
}

extern "C" int haste_ffi_bwd_features(const int32_t* idx, const void* W, const void* dY,
                                      int64_t lddy, float* dXT, void* workspace,
                                      int64_t workspace_bytes, int64_t B, int64_t D, int64_t F,
                                      int64_t O, int64_t G, int32_t dtype, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    HASTE_CHECK_ARG(dXT != nullptr, "haste_ffi_bwd_features: null output");
    haste::BwdFPlan p;
    int rc = haste::run_partials("haste_ffi_bwd_features", idx, W, dY, lddy, workspace,
                                 workspace_bytes, B, D, F, O, G, dtype, st, &p);
    if (rc != HASTE_OK) return rc;
    const float* ws = reinterpret_cast<const float*>(static_cast<const char*>(workspace) + p.prep_bytes);
    const int64_t n = D * B;
    const int64_t blocks = std::min<int64_t>(haste::ceil_div(n, 256), 1 << 16);
    haste::bwdf_reduce_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(ws, dXT, (int)B,
                                                                          (int)p.Bp, (int)D, (int)p.S);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

extern "C" int haste_ffi_bwd_features_sr(const int32_t* idx, const void* W, const void* dY,
                                         int64_t lddy, uint16_t* dX, uint64_t seed,
                                         void* workspace, int64_t workspace_bytes, int64_t B,
                                         int64_t D, int64_t F, int64_t O, int64_t G,
                                         int32_t dtype, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    HASTE_CHECK_ARG(dX != nullptr, "haste_ffi_bwd_features_sr: null output");
    haste::BwdFPlan p;
    int rc = haste::run_partials("haste_ffi_bwd_features_sr", idx, W, dY, lddy, workspace,
                                 workspace_bytes, B, D, F, O, G, dtype, st, &p);
    if (rc != HASTE_OK) return rc;
    const float* ws = reinterpret_cast<const float*>(static_cast<const char*>(workspace) + p.prep_bytes);
    dim3 grid((unsigned)haste::ceil_div(D, 32), (unsigned)haste::ceil_div(B, 32));
    haste::bwdf_reduce_sr_kernel<<<grid, dim3(256), 0, st>>>(ws, dX, (int)B, (int)p.Bp, (int)D,
                                                            (int)p.S, (uint32_t)seed,
                                                            (uint32_t)(seed >> 32));
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features_sr");
    return HASTE_OK;
}
