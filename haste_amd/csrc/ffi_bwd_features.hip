// Grouped fixed-fan-in backward to features, deterministic (gfx950).
//
//   dXT[d, b] = sum_{g, j: idx[g, j] = d} sum_{l in g} W[l, j] * dY[b, l]
//
// The reference scatters with fp32 atomicAdd into global memory
// (shared_ffi/ffi_backward_features.cu:202-212), so its sums depend on timing.
// Here no float atomic touches any memory and every sum has a fixed order:
//
//  1. prep (one workgroup per group): the F slots are stably sorted by index,
//     so equal indices become adjacent runs; the sorted table, the bounds of
//     eight value parts of every feature range, and W_g transposed in sorted
//     slot order (WT[g][p][l] = W[g*G + l][slot(p)]) are written to the
//     workspace.
//  2. main: a workgroup (group slice s, feature range dr, 32-column batch tile
//     bt) keeps the partial dXT[d in dr, b in bt] in LDS (fp32).  Its 8 waves
//     own fixed value parts of dr, so they never touch the same LDS word and
//     run through the slice's groups independently (no barriers).  Per group a
//     wave multiplies the WT rows of its positions with dY_g (MFMA, M = sorted
//     positions, N = batch, K = labels) and adds the result rows into the LDS
//     partial with plain reads and writes (LDS float atomics execute one lane
//     at a time).  Operands come straight from global memory into registers,
//     two groups ahead.
//  3. reduce: dXT = sum over slices s = 0..S-1 in ascending order (fp32 out), or
//     fused with the bf16 stochastic rounding of shared_ffi/bindings.py:44-48.
#include <algorithm>

#include "common.hpp"

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

constexpr int kWaves = 4;                 // waves per workgroup, one value part each
constexpr int kMainThreads = 64 * kWaves;
constexpr int kMetaStride = 16;           // ints of meta per (group, feature range)
constexpr int kBT = 32;            // batch columns per workgroup
constexpr int kLdsBytes = 160 * 1024;
constexpr int kTargetCTAs = 256;
constexpr int kMaxDc = (kLdsBytes - 2 * kMainThreads * 4) / 4 / kBT;  // features in the LDS partial
static_assert(kMaxDc * kBT * 4 + 2 * kMainThreads * 4 <= kLdsBytes, "LDS budget");

struct BwdFPlan {
    int64_t Gc, nbt, Bp, ndr, Dc, S, gps;  // gps = groups per slice
    int64_t sorted_off, meta_off, wt_off, prep_bytes, ws_bytes;
};

BwdFPlan make_plan(int64_t B, int64_t D, int64_t F, int64_t O, int64_t G) {
    BwdFPlan p;
    p.Gc = ceil_div(O, G);
    p.nbt = ceil_div(B, kBT);
    p.Bp = p.nbt * kBT;
    p.ndr = ceil_div(D, kMaxDc);
    p.Dc = ceil_div(D, p.ndr);
    int64_t S = std::max<int64_t>(1, kTargetCTAs / (p.nbt * p.ndr));
    S = std::min<int64_t>(S, std::max<int64_t>(1, ceil_div(p.Gc, 8)));
    p.gps = ceil_div(p.Gc, S);
    p.S = ceil_div(p.Gc, p.gps);
    auto r256 = [](int64_t x) { return (x + 255) / 256 * 256; };
    p.sorted_off = 0;
    p.meta_off = r256(p.Gc * F * 4);
    p.wt_off = p.meta_off + r256(p.Gc * p.ndr * kMetaStride * 4);
    p.prep_bytes = p.wt_off + r256(p.Gc * F * G * 2);
    p.ws_bytes = p.S * D * p.Bp * 4;
    return p;
}

// --------------------------------------------------------------- prep ------
// sorted[g*F + p] = (index << 8) | (colour + 1) for sorted position p (an
// arithmetic >> 8 recovers the index; -1 marks an empty entry).  Value part w (of
// kWaves) of feature range dr owns sorted positions [m[w], m[w+1]), m = meta +
// (g*ndr + dr)*kMetaStride (its values lie in [d_lo + (Dc'*w)/kWaves,
// d_lo + (Dc'*(w+1))/kWaves)); m[kWaves + 1] bounds the colour count of the
// scatter: ceil((longest run - 1) / 4).
// colour: with rel = p - (first position of p's part), a position is a
// "head" if rel % 4 == 0 or it starts a run of equal indices; heads get
// colour rel/4 - (rel - run)/4 (run = rank inside the run), others -1.
// wt[(g*F + p)*G + l] = W[g*G + l][slot(p)] (0 for labels >= O).
template <int G>
__global__ __launch_bounds__(256) void bwdf_prep_kernel(const int32_t* __restrict__ idx,
                                                        const uint16_t* __restrict__ W,
                                                        int32_t* __restrict__ sorted,
                                                        int* __restrict__ meta,
                                                        uint16_t* __restrict__ wt, int F, int D,
                                                        int64_t O, int ndr, int Dc) {
    constexpr int LDW = G + 8;
    __shared__ int32_t s[256];
    __shared__ int32_t sv[256];
    __shared__ int32_t srun[256];
    __shared__ int32_t sslot[256];
    __shared__ int run_max;
    __shared__ __attribute__((aligned(16))) uint16_t Wt[256 * LDW];  // Wt[slot][label]
    const int64_t g = blockIdx.x;
    const int64_t l0 = g * G;
    const int tid = threadIdx.x;
    if (tid == 0) run_max = 0;
    if (tid < F) s[tid] = min(max(idx[g * F + tid], 0), D - 1);
    // W_g rows -> LDS transposed: item = (label, 8 slots)
    for (int it = tid; it < G * (F / 8); it += 256) {
        const int l = it / (F / 8);
        const int j0 = (it % (F / 8)) * 8;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (l0 + l < O) v = *reinterpret_cast<const u32x4*>(W + (l0 + l) * F + j0);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            Wt[(j0 + e) * LDW + l] = (uint16_t)((e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xFFFFu));
    }
    __syncthreads();
    if (tid < F) {
        const int v = s[tid];
        int rank = 0, run = 0;
        for (int q = 0; q < F; ++q) {
            const int u = s[q];
            rank += (u < v) || (u == v && q < tid);
            run += (u == v && q < tid);
        }
        sv[rank] = v;
        srun[rank] = run;
        sslot[rank] = tid;
        atomicMax(&run_max, run);
    }
    __syncthreads();
    auto lower_bound = [&](int bound) {
        int lo = 0, hi = F;
        while (lo < hi) {
            const int mm = (lo + hi) >> 1;
            if (sv[mm] < bound) lo = mm + 1; else hi = mm;
        }
        return lo;
    };
    for (int dr = tid; dr < ndr; dr += 256) {
        const int d_lo = dr * Dc, d_hi = min(D, d_lo + Dc);
        int* m = meta + (g * ndr + dr) * kMetaStride;
        for (int w = 0; w <= kWaves; ++w) m[w] = lower_bound(d_lo + ((d_hi - d_lo) * w) / kWaves);
        m[kWaves + 1] = (run_max + 3) / 4;
    }
    if (tid < F) {
        const int p = tid;
        const int x = sv[p];
        const int dr = x / Dc;
        const int d_lo = dr * Dc, d_hi = min(D, d_lo + Dc);
        int w = kWaves - 1;
        while (w > 0 && x < d_lo + ((d_hi - d_lo) * w) / kWaves) --w;
        const int pb = lower_bound(d_lo + ((d_hi - d_lo) * w) / kWaves);
        const int rel = p - pb;
        const int run = srun[p];
        const bool head = (rel % 4 == 0) || run == 0;
        sorted[g * F + p] = (x << 8) | (head ? rel / 4 - (rel - run) / 4 + 1 : 0);
    }
    // sorted rows of W_g^T: item = (position, 8 labels)
    for (int it = tid; it < F * (G / 8); it += 256) {
        const int p = it / (G / 8);
        const int lc = (it % (G / 8)) * 8;
        const u32x4 v = *reinterpret_cast<const u32x4*>(&Wt[sslot[p] * LDW + lc]);
        *reinterpret_cast<u32x4*>(wt + ((g * F + p) * G + lc)) = v;
    }
}

// --------------------------------------------------------------- main ------
template <typename T, int G, int FP>
struct BwdFCfg {
    static constexpr int KS = G >= 32 ? G / 32 : 1;  // MFMA k-steps over labels
    static constexpr int NT = kBT / 16;              // batch n-tiles per wave
    static constexpr int MAXT = FP >= 256 ? 5 : FP >= 128 ? 3 : 2;  // tiles kept in registers
};

typedef int32_t i32x4a __attribute__((ext_vector_type(4), aligned(4)));

template <int KS, int MAXT, int NT>
struct BwdFRegs {
    u32x4 a[MAXT][KS];  // WT rows of the wave's positions (A operand)
    int e[MAXT][4];     // packed slot-table entries of this lane's scatter positions
    u32x4 b[NT][KS];    // dY fragments (B operand)
    int pb, pe, maxc;
};

// Scatter of one MFMA tile (rows = 16 sorted positions; lane holds positions
// 4*lq + i, i = 0..3, of one batch column): equal indices are adjacent, so a
// lane first folds each run inside its own 4 positions into the run's first
// position there (the "head").  Heads of one run that sit in different
// lanes/tiles get successive colours (their quad index relative to the run
// start); pass c reads, adds and writes all heads of colour c at once.  Within
// a pass every lane targets a distinct word, and every word is only ever
// touched by one wave, in program order (the compiler keeps these plain LDS
// accesses in order: as far as it knows they may alias).
template <typename T, int G, int FP>
__global__ __launch_bounds__(kMainThreads) void bwdf_main_kernel(
    const int32_t* __restrict__ sorted, const int* __restrict__ meta,
    const uint16_t* __restrict__ wt, const uint16_t* __restrict__ dY, int64_t lddy,
    float* __restrict__ ws, int B, int Bp, int D, int F, int64_t O, int64_t Gc, int nbt, int ndr,
    int Dc, int gps, int S) {
    using C = BwdFCfg<T, G, FP>;
    constexpr int KS = C::KS, NT = C::NT, MAXT = C::MAXT;
    using R = BwdFRegs<KS, MAXT, NT>;
    __shared__ float acc[kMaxDc * kBT + 2 * kMainThreads];  // + two dummy words per lane

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
    const int part = tid >> 6;  // value part of this wave
    const int lrow = lane & 15;
    const int lq = lane >> 4;

    for (int i = tid; i < (d_hi - d_lo) * kBT; i += kMainThreads) acc[i] = 0.0f;
    __syncthreads();

    // Branch-free loads: addresses are clamped into the group's blocks and
    // out-of-range values replaced by selects (divergent branches around
    // memory operations cost far more than the operations themselves).  The
    // dY masking only runs for the ragged last group / batch tile.
    const bool full_b = b_base + kBT <= B;
    auto load = [&](int64_t g, R& r) {
        const int* m = meta + (g * ndr + dr) * kMetaStride;
        r.pb = m[part];
        r.pe = m[part + 1];
        r.maxc = m[kWaves + 1];
        const int64_t l0 = g * G;
        const uint16_t* wg = wt + g * F * G;
        const int32_t* sg = sorted + g * F;
        const bool clamp_p = r.pb + 16 * MAXT + 4 > F;
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (r.pb + t * 16 >= r.pe) break;  // wave-uniform: no positions left
            int pa = r.pb + t * 16 + lrow;
            if (clamp_p) pa = min(pa, F - 1);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int k = G >= 32 ? ks * 32 + lq * 8 : (lq & 1) * 8;
                r.a[t][ks] = *reinterpret_cast<const u32x4*>(wg + pa * G + k);
            }
            // the lane's 4 consecutive entries with one (4-byte aligned) 16-byte load
            const int p0 = r.pb + t * 16 + lq * 4;
            i32x4a v;
            if (clamp_p && p0 + 4 > F) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = sg[min(p0 + i, F - 1)];
            } else {
                v = *reinterpret_cast<const i32x4a*>(sg + p0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) r.e[t][i] = p0 + i < r.pe ? v[i] : -1;
        }
        const bool full = full_b && l0 + G <= O;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int b = b_base + nt * 16 + lrow;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int k = ks * 32 + lq * 8;
                if (full && k < G) {
                    r.b[nt][ks] = *reinterpret_cast<const u32x4*>(dY + (int64_t)b * lddy + l0 + k);
                } else {
                    const int64_t col = min(l0 + min(k, G - 8), lddy - 8);
                    u32x4 v = *reinterpret_cast<const u32x4*>(dY + (int64_t)min(b, B - 1) * lddy + col);
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const bool ok = b < B && k + q < G && l0 + k + q < O;
                        v[q >> 1] &= ok ? 0xFFFFFFFFu : ((q & 1) ? 0x0000FFFFu : 0xFFFF0000u);
                    }
                    r.b[nt][ks] = v;
                }
            }
        }
    };

    // Multiply + scatter `ntiles` (<= MAXT) tiles of 16 positions.  Lanes
    // without work in a pass read and write a private dummy word (two words,
    // 16 apart, one per batch half), so the LDS accesses need no divergent
    // branches; tile loops use wave-uniform branches only.
    const int dummy = kMaxDc * kBT + part * 128 + lane;
    const int colbase = lrow - d_lo * kBT;
    auto compute = [&](const u32x4 (&a)[MAXT][KS], const int (&e)[MAXT][4],
                       const u32x4 (&b)[NT][KS], int ntiles, int maxc) {
        int addr[MAXT][4], col1[MAXT][4];
        float o[MAXT][NT][4];
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t >= ntiles) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                addr[t][i] = (e[t][i] >> 8) * kBT + colbase;
                col1[t][i] = e[t][i] & 0xFF;  // colour + 1; 0 = not a head
                const int eff = col1[t][i] == 1 ? addr[t][i] : dummy;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) o[t][nt][i] = acc[eff + nt * 16];
            }
        }
        f32x4 c[MAXT][NT];
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t >= ntiles) continue;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                c[t][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) c[t][nt] = mfma16x16x32<T>(a[t][ks], b[nt][ks], c[t][nt]);
                // fold runs inside the lane's 4 positions into their heads
#pragma unroll
                for (int i = 3; i >= 1; --i)
                    if (maxc > 0) c[t][nt][i - 1] += (col1[t][i] == 0 && e[t][i] >= 0) ? c[t][nt][i] : 0.0f;
            }
        }
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t >= ntiles) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int eff = col1[t][i] == 1 ? addr[t][i] : dummy;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[eff + nt * 16] = o[t][nt][i] + c[t][nt][i];
            }
        }
        for (int cc = 1; cc <= maxc; ++cc) {
#pragma unroll
            for (int t = 0; t < MAXT; ++t) {
                if (t >= ntiles) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int eff = col1[t][i] == cc + 1 ? addr[t][i] : dummy;
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) o[t][nt][i] = acc[eff + nt * 16];
                }
            }
#pragma unroll
            for (int t = 0; t < MAXT; ++t) {
                if (t >= ntiles) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int eff = col1[t][i] == cc + 1 ? addr[t][i] : dummy;
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) acc[eff + nt * 16] = o[t][nt][i] + c[t][nt][i];
                }
            }
        }
    };

    // Tiles beyond MAXT (only for heavily duplicated index sets): loaded and
    // processed MAXT at a time, without prefetch.
    auto overflow = [&](int64_t g, const R& r) {
        const int total = (r.pe - r.pb + 15) / 16;
        const uint16_t* wg = wt + g * F * G;
        const int32_t* sg = sorted + g * F;
        for (int t0 = MAXT; t0 < total; t0 += MAXT) {
            u32x4 a[MAXT][KS];
            int e[MAXT][4];
#pragma unroll
            for (int t = 0; t < MAXT; ++t) {
                const int pa = min(r.pb + (t0 + t) * 16 + lrow, F - 1);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int k = G >= 32 ? ks * 32 + lq * 8 : (lq & 1) * 8;
                    a[t][ks] = *reinterpret_cast<const u32x4*>(wg + pa * G + k);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int p = r.pb + (t0 + t) * 16 + lq * 4 + i;
                    const int v = sg[min(p, F - 1)];
                    e[t][i] = p < r.pe ? v : -1;
                }
            }
            compute(a, e, r.b, min(MAXT, total - t0), r.maxc);
        }
    };

    auto process = [&](int64_t g, const R& r) {
        const int total = (r.pe - r.pb + 15) / 16;
        compute(r.a, r.e, r.b, min(MAXT, total), r.maxc);
        if (total > MAXT) overflow(g, r);
    };

    // Three register sets: group g is computed while g+1 and g+2 are in flight.
    if (g_begin < g_end) {
        R r0, r1, r2;
        load(g_begin, r0);
        if (g_begin + 1 < g_end) load(g_begin + 1, r1);
        int64_t g = g_begin;
        while (true) {
            if (g + 2 < g_end) load(g + 2, r2);
            process(g, r0);
            if (++g >= g_end) break;
            if (g + 2 < g_end) load(g + 2, r0);
            process(g, r1);
            if (++g >= g_end) break;
            if (g + 2 < g_end) load(g + 2, r1);
            process(g, r2);
            if (++g >= g_end) break;
        }
    }
    __syncthreads();

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
int launch_main(const int32_t* sorted, const int* meta, const uint16_t* wt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F,
                int64_t O, hipStream_t st) {
    const int64_t nlog = p.S * p.ndr * p.nbt;
    const int64_t grid = 8 * ceil_div(nlog, 8);
    bwdf_main_kernel<T, G, FP><<<dim3((unsigned)grid), dim3(kMainThreads), 0, st>>>(
        sorted, meta, wt, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, (int)F, O, p.Gc, (int)p.nbt,
        (int)p.ndr, (int)p.Dc, (int)p.gps, (int)p.S);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

template <typename T, int G>
int dispatch_fp(const int32_t* sorted, const int* meta, const uint16_t* wt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F,
                int64_t O, hipStream_t st) {
#define HASTE_BWDF_ARGS sorted, meta, wt, dY, lddy, ws, p, B, D, F, O, st
    if (F <= 32) return launch_main<T, G, 32>(HASTE_BWDF_ARGS);
    if (F <= 64) return launch_main<T, G, 64>(HASTE_BWDF_ARGS);
    if (F <= 128) return launch_main<T, G, 128>(HASTE_BWDF_ARGS);
    return launch_main<T, G, 256>(HASTE_BWDF_ARGS);
#undef HASTE_BWDF_ARGS
}

template <int G>
void launch_prep(const int32_t* idx, const uint16_t* W, int32_t* sorted, int* meta, uint16_t* wt,
                 const BwdFPlan& p, int64_t D, int64_t F, int64_t O, hipStream_t st) {
    bwdf_prep_kernel<G><<<dim3((unsigned)p.Gc), dim3(256), 0, st>>>(
        idx, W, sorted, meta, wt, (int)F, (int)D, O, (int)p.ndr, (int)p.Dc);
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
    char* base = static_cast<char*>(workspace);
    int32_t* sorted = reinterpret_cast<int32_t*>(base + p.sorted_off);
    int* meta = reinterpret_cast<int*>(base + p.meta_off);
    uint16_t* wt = reinterpret_cast<uint16_t*>(base + p.wt_off);
    float* ws = reinterpret_cast<float*>(base + p.prep_bytes);
    auto* w = static_cast<const uint16_t*>(W);
    auto* y = static_cast<const uint16_t*>(dY);
    switch (G) {
#define HASTE_BWDF_G(GG)                                                                      \
    case GG:                                                                                  \
        launch_prep<GG>(idx, w, sorted, meta, wt, p, D, F, O, st);                            \
        HASTE_CHECK_LAUNCH(fn);                                                               \
        rc = dtype == HASTE_DTYPE_BF16                                                        \
                 ? dispatch_fp<BF16, GG>(sorted, meta, wt, y, lddy, ws, p, B, D, F, O, st)    \
                 : dispatch_fp<F16, GG>(sorted, meta, wt, y, lddy, ws, p, B, D, F, O, st);    \
        break;
        HASTE_BWDF_G(16)
        HASTE_BWDF_G(32)
        HASTE_BWDF_G(64)
        HASTE_BWDF_G(128)
#undef HASTE_BWDF_G
    default:
        set_error("%s: unsupported group size %lld", fn, (long long)G);
        return HASTE_ERR_UNSUPPORTED;
    }
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
