// Grouped fixed-fan-in backward to features, deterministic (gfx950).
//
//   dXT[d, b] = sum_{g, j: idx[g, j] = d} sum_{l in g} W[l, j] * dY[b, l]
//
// The reference scatters with fp32 atomicAdd into global memory
// (shared_ffi/ffi_backward_features.cu:202-212), so its sums depend on timing.
// Here no float atomic ever touches global memory and every sum has a fixed
// order:
//
//  1. prep: per group, the F slots are stably sorted by index, so equal
//     indices become adjacent runs; the sorted positions of each feature range
//     are split into 4 quarters at run starts.
//  2. main: workgroup (group slice s, feature range dr, batch tile bt) keeps a
//     partial dXT[d in dr, b in bt] in LDS (fp32).  For each group of its slice,
//     in order, it stages W_g transposed in LDS; each of 8 waves (4 position
//     quarters x 2 halves of the 32 batch columns) computes P = W_g^T dY_g^T for
//     its positions with MFMA (M = sorted positions, N = batch, K = labels) and
//     adds the rows into the LDS partial with plain reads and writes (LDS float
//     atomics execute one lane at a time).  No two waves own the same word and
//     no two lanes of one access instruction target the same word (see the
//     scatter note at bwdf_main_kernel), so every word is updated by one wave
//     in program order.
//  3. reduce: dXT = sum over slices s = 0..S-1 in ascending order (fp32 out), or
//     fused with the bf16 stochastic rounding of shared_ffi/bindings.py:44-48.
#include <algorithm>

#include "common.hpp"

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

constexpr int kMainThreads = 512;  // 8 waves
constexpr int kBT = 32;             // batch columns per workgroup
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
    p.prep_bytes = ((p.Gc * F * 8 + p.Gc * p.ndr * 32) + 255) / 256 * 256;
    p.ws_bytes = p.S * D * p.Bp * 4;
    return p;
}

// --------------------------------------------------------------- prep ------
// sorted[g*F + p] = {index, slot | run << 16} for sorted position p, where run
// is the number of earlier positions holding the same index.
// meta[(g*ndr + dr)*8 + w], w = 0..4: position quarter w of feature range dr is
// [meta[w], meta[w+1]); splits are moved to the start of a run of equal
// indices, so no feature is shared by two quarters.  meta[5] bounds the colour
// count of the scatter (see bwdf_main_kernel): ceil((longest run - 1) / 4).
__global__ __launch_bounds__(256) void bwdf_prep_kernel(const int32_t* __restrict__ idx,
                                                        int2* __restrict__ sorted,
                                                        int* __restrict__ meta, int F, int D,
                                                        int ndr, int Dc) {
    __shared__ int32_t s[256];
    __shared__ int32_t sv[256];
    __shared__ int run_max;
    const int64_t g = blockIdx.x;
    const int j = threadIdx.x;
    if (j == 0) run_max = 0;
    if (j < F) s[j] = min(max(idx[g * F + j], 0), D - 1);
    __syncthreads();
    if (j < F) {
        const int v = s[j];
        int rank = 0, run = 0;
        for (int q = 0; q < F; ++q) {
            const int u = s[q];
            rank += (u < v) || (u == v && q < j);
            run += (u == v && q < j);
        }
        sorted[g * F + rank] = make_int2(v, j | (run << 16));
        sv[rank] = v;
        atomicMax(&run_max, run);
    }
    __syncthreads();
    for (int dr = j; dr < ndr; dr += 256) {
        const int d_lo = dr * Dc, d_hi = min(D, d_lo + Dc);
        int lo = 0, hi = F;
        while (lo < hi) { const int m = (lo + hi) >> 1; if (sv[m] < d_lo) lo = m + 1; else hi = m; }
        const int P0 = lo;
        hi = F;
        while (lo < hi) { const int m = (lo + hi) >> 1; if (sv[m] < d_hi) lo = m + 1; else hi = m; }
        const int P1 = lo;
        int* m = meta + (g * ndr + dr) * 8;
        m[0] = P0;
        for (int w = 1; w < 4; ++w) {
            int t = P0 + ((P1 - P0) * w) / 4;
            while (t > P0 && t < P1 && sv[t] == sv[t - 1]) ++t;
            m[w] = t;
        }
        m[4] = P1;
        m[5] = (run_max + 3) / 4;
        m[6] = 0;
        m[7] = 0;
    }
}

// --------------------------------------------------------------- main ------
template <typename T, int G, int FP>
struct BwdFCfg {
    static constexpr int KS = G >= 32 ? G / 32 : 1;  // MFMA k-steps over labels
    static constexpr int LDW = ws_pitch(G);          // Ws row pitch (elements)
    static constexpr int ACC = max_dc(G, FP) * kBT;  // LDS partial size (floats)
    static constexpr int ITEMS = (G / 4) * (FP / 8); // W staging items: 4 labels x 8 slots
    static constexpr int IPT = (ITEMS + kMainThreads - 1) / kMainThreads;
};

// 8 waves: wave = 2 * quarter + half.  `half` selects the 16 batch columns of
// the 32-column tile, `quarter` the sorted-position quarter (its features).
// The next group's W tile, slot table, quarter bounds and dY fragments are
// loaded into registers while the current group is computed.
//
// Scatter of one MFMA tile (rows = 16 sorted positions, lane holds positions
// 4*lq + i, i = 0..3, of one batch column): equal indices are adjacent, so a
// lane first folds each run inside its own 4 positions into the run's first
// position there (the "head").  Heads of one run that sit in different lanes
// get successive colours; pass c reads, adds and writes all heads of colour c
// at once.  Within a pass every lane targets a distinct word, and every word
// is only ever touched by one wave, in program order.
template <typename T, int G, int FP>
__global__ __launch_bounds__(kMainThreads) void bwdf_main_kernel(
    const int2* __restrict__ sorted, const int* __restrict__ meta, const uint16_t* __restrict__ W,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int F, int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S) {
    using C = BwdFCfg<T, G, FP>;
    __shared__ float acc[C::ACC];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[FP * C::LDW];
    __shared__ int2 ss[FP];
    __shared__ int mb[8];

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
    const int half = wave & 1;
    const int quarter = wave >> 1;
    const int lrow = lane & 15;
    const int lq = lane >> 4;
    const int col = half * 16 + lrow;  // batch column of this lane inside the tile

    u32x4 wreg[C::IPT][4];
    int2 ssreg = make_int2(0, 0);
    int mreg = 0;
    u32x4 bnext[C::KS];

    auto load = [&](int64_t g) {
        const int64_t l0 = g * G;
#pragma unroll
        for (int i = 0; i < C::IPT; ++i) {
            const int it = tid + i * kMainThreads;
            const int lc = (it % (G / 4)) * 4;
            const int j0 = (it / (G / 4)) * 8;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (it < C::ITEMS && l0 + lc + q < O && j0 < F)
                    wreg[i][q] = *reinterpret_cast<const u32x4*>(W + (l0 + lc + q) * F + j0);
                else
                    wreg[i][q] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        if (tid < F) ssreg = sorted[g * F + tid];
        if (tid < 8) mreg = meta[(g * ndr + dr) * 8 + tid];
        const int b = b_base + col;
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
            const int k = ks * 32 + lq * 8;
            if (b < B && k < G && l0 + k < O) {
                bnext[ks] = *reinterpret_cast<const u32x4*>(dY + (int64_t)b * lddy + l0 + k);
                if (l0 + k + 8 > O) {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (l0 + k + e >= O) bnext[ks][e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                }
            } else {
                bnext[ks] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };

    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < C::IPT; ++i) {
            const int it = tid + i * kMainThreads;
            if (it >= C::ITEMS) continue;
            const int lc = (it % (G / 4)) * 4;
            const int j0 = (it / (G / 4)) * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int sh = (e & 1) * 16;
                const uint32_t a0 = (wreg[i][0][e >> 1] >> sh) & 0xFFFFu;
                const uint32_t a1 = (wreg[i][1][e >> 1] >> sh) & 0xFFFFu;
                const uint32_t a2 = (wreg[i][2][e >> 1] >> sh) & 0xFFFFu;
                const uint32_t a3 = (wreg[i][3][e >> 1] >> sh) & 0xFFFFu;
                *reinterpret_cast<u32x2*>(&Ws[(j0 + e) * C::LDW + lc]) =
                    u32x2{a0 | (a1 << 16), a2 | (a3 << 16)};
            }
        }
        if (tid < F) ss[tid] = ssreg;
        if (tid < 8) mb[tid] = mreg;
    };

    for (int i = tid; i < (d_hi - d_lo) * kBT; i += kMainThreads) acc[i] = 0.0f;
    if (g_begin < g_end) load(g_begin);

    for (int64_t g = g_begin; g < g_end; ++g) {
        stage();
        u32x4 bcur[C::KS];
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) bcur[ks] = bnext[ks];
        __syncthreads();
        if (g + 1 < g_end) load(g + 1);

        const int pb = mb[quarter];
        const int pe = mb[quarter + 1];
        const int maxc = mb[5];
        for (int m0 = pb; m0 < pe; m0 += 16) {
            // A fragments: rows = sorted positions, 8 consecutive labels from Ws.
            const int pa = m0 + lrow;
            const int slot = pa < pe ? (ss[pa].y & 0xFFFF) : 0;
            // scatter metadata of this lane's 4 positions (and the one before)
            int2 e[4];
            const int p0 = m0 + lq * 4;  // lane-aligned quad: p0 - pb is a multiple of 4
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = (p0 + i < pe) ? ss[p0 + i] : make_int2(-1, 0);
            f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < C::KS; ++ks) {
                const int k = ks * 32 + lq * 8;
                u32x4 af = u32x4{0u, 0u, 0u, 0u};
                if (pa < pe && k < G) af = *reinterpret_cast<const u32x4*>(&Ws[slot * C::LDW + k]);
                c = mfma16x16x32<T>(af, bcur[ks], c);
            }
            // fold runs inside the lane's 4 positions into their heads
            int addr[4], colour[4];
            bool head[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = p0 + i;
                const int rel = p - pb;
                const bool valid = e[i].x >= 0;
                head[i] = valid && (i == 0 || e[i].x != e[i - 1].x);
                const int run = e[i].y >> 16;
                colour[i] = rel / 4 - max(rel - run, 0) / 4;
                addr[i] = (e[i].x - d_lo) * kBT + col;
            }
#pragma unroll
            for (int i = 3; i >= 1; --i)
                if (e[i].x >= 0 && !head[i]) c[i - 1] += c[i];
            for (int cc = 0; cc <= maxc; ++cc) {
                float o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = (head[i] && colour[i] == cc) ? acc[addr[i]] : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (head[i] && colour[i] == cc) acc[addr[i]] = o[i] + c[i];
            }
        }
        __syncthreads();
    }

    // ---- write the partial: ws[s][d][bt*32 + b] ----
    for (int i = tid; i < (d_hi - d_lo) * kBT; i += kMainThreads) {
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
int launch_main(const int2* sorted, const int* meta, const uint16_t* W, const uint16_t* dY, int64_t lddy,
                float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O,
                hipStream_t st) {
    const int64_t nlog = p.S * p.ndr * p.nbt;
    const int64_t grid = 8 * ceil_div(nlog, 8);
    bwdf_main_kernel<T, G, FP><<<dim3((unsigned)grid), dim3(kMainThreads), 0, st>>>(
        sorted, meta, W, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, (int)F, O, p.Gc, (int)p.nbt,
        (int)p.ndr, (int)p.Dc, (int)p.gps, (int)p.S);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

template <typename T, int G>
int dispatch_fp(const int2* sorted, const int* meta, const uint16_t* W, const uint16_t* dY, int64_t lddy, float* ws,
                const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O, hipStream_t st) {
    if (F <= 32) return launch_main<T, G, 32>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
    if (F <= 64) return launch_main<T, G, 64>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
    if (F <= 128) return launch_main<T, G, 128>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
    return launch_main<T, G, 256>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
}

template <typename T>
int dispatch_g(const int2* sorted, const int* meta, const uint16_t* W, const uint16_t* dY, int64_t lddy, float* ws,
               const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
               hipStream_t st) {
    switch (G) {
    case 16: return dispatch_fp<T, 16>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
    case 32: return dispatch_fp<T, 32>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
    case 64: return dispatch_fp<T, 64>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
    default: return dispatch_fp<T, 128>(sorted, meta, W, dY, lddy, ws, p, B, D, F, O, st);
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
    int* meta = reinterpret_cast<int*>(sorted + p.Gc * F);
    float* ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.prep_bytes);
    bwdf_prep_kernel<<<dim3((unsigned)p.Gc), dim3(256), 0, st>>>(idx, sorted, meta, (int)F,
                                                                     (int)D, (int)p.ndr, (int)p.Dc);
    HASTE_CHECK_LAUNCH(fn);
    auto* w = static_cast<const uint16_t*>(W);
    auto* y = static_cast<const uint16_t*>(dY);
    rc = dtype == HASTE_DTYPE_BF16 ? dispatch_g<BF16>(sorted, meta, w, y, lddy, ws, p, B, D, F, O, G, st)
                                   : dispatch_g<F16>(sorted, meta, w, y, lddy, ws, p, B, D, F, O, G, st);
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
