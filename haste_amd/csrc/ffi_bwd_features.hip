// Grouped fixed-fan-in backward to features, deterministic (gfx950).
//
//   dXT[d, b] = sum_{g, j: idx[g, j] = d} sum_{l in g} W[l, j] * dY[b, l]
//
// The reference scatters with fp32 atomicAdd into global memory
// (shared_ffi/ffi_backward_features.cu:202-212), so its sums depend on timing.
// Here no float atomic touches any memory and every sum has a fixed order:
//
//  1. prep (one workgroup per group g): the distinct indices of the group are
//     split by feature range (Dc features each) and laid out in tiles of 16
//     positions.  A tile row holds the group's weights for that feature,
//     transposed (WT[pos][label]).  An index that occurs k > 1 times in the
//     group gets sum_j W[l, j] (fp32, ascending j) split into a 16-bit "hi"
//     row (layer 0) and the 16-bit rounding of the remainder as a "lo" row
//     (layer 1), so inside a layer every feature occurs once.
//  2. main: a workgroup owns (group slice s, feature range r, batch tile of
//     BT columns) and keeps dXT[range, tile] as an fp32 partial in LDS.  Wave
//     w owns batch rows [w*RPW, (w+1)*RPW) of the tile, so no two waves touch
//     the same LDS word and the waves never synchronise.  Per group a wave
//     multiplies its dY rows with the range's tiles (MFMA, M = batch rows,
//     N = 16 positions, K = labels); a lane then holds four consecutive
//     batch values of one feature and adds them into LDS with one 16-byte
//     read and one 16-byte write.  Reads of all tiles of a layer are issued
//     before their writes (a layer's features are distinct); a wave's LDS
//     accesses execute in program order, so layer 1 and later groups see
//     the earlier writes.  Operands come from global memory into registers,
//     NS groups ahead.
//  3. reduce: dXT = sum over slices s = 0..S-1 in ascending order (fp32 out), or
//     fused with the bf16 stochastic rounding of shared_ffi/bindings.py:44-48.
#include <algorithm>

#include "common.hpp"

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

constexpr int kMainThreads = 256;  // 4 waves
constexpr int kAccPad = 4;         // fp32 words of padding per LDS row (bank spread)
constexpr int kDummyFloats = 4 * kMainThreads;  // one 16-byte dummy slot per lane
constexpr int kAccBytes = 140 * 1024;           // LDS for the partial (incl. dummies)
constexpr int kTargetCTAs = 256;
constexpr int kMaxRanges = 128;  // feature ranges per group handled by prep
constexpr int kMetaStride = 4;   // ints per (group, range): tile begin, layer-1 begin, end

__host__ __device__ constexpr int acc_stride(int bt) { return bt + kAccPad; }
__host__ __device__ constexpr int max_dc(int bt) {
    return (kAccBytes / 4 - kDummyFloats) / acc_stride(bt);
}

struct BwdFPlan {
    int64_t Gc, BT, nbt, Bp, ndr, Dc, S, gps, Tcap;
    int64_t tfeat_off, meta_off, twt_off, prep_bytes, ws_bytes;
};

BwdFPlan make_plan(int64_t B, int64_t D, int64_t F, int64_t O, int64_t G) {
    BwdFPlan p;
    p.Gc = ceil_div(O, G);
    p.BT = B <= 64 ? 64 : 128;
    p.nbt = ceil_div(B, p.BT);
    p.Bp = p.nbt * p.BT;
    p.ndr = ceil_div(D, max_dc((int)p.BT));
    p.Dc = ceil_div(D, p.ndr);
    int64_t S = std::max<int64_t>(1, kTargetCTAs / (p.nbt * p.ndr));
    S = std::min<int64_t>(S, std::max<int64_t>(1, ceil_div(p.Gc, 8)));
    p.gps = ceil_div(p.Gc, S);
    p.S = ceil_div(p.Gc, p.gps);
    // tiles per group: layer 0 holds <= F distinct features, layer 1 <= F/2, and
    // each non-empty range pads its layer to a multiple of 16
    const int64_t r0 = std::min<int64_t>(p.ndr, F), r1 = std::min<int64_t>(p.ndr, F / 2);
    p.Tcap = ceil_div(F + 15 * r0, 16) + ceil_div(F / 2 + 15 * r1, 16);
    auto r256 = [](int64_t x) { return (x + 255) / 256 * 256; };
    p.tfeat_off = 0;
    p.meta_off = r256(p.Gc * p.Tcap * 16 * 4);
    p.twt_off = p.meta_off + r256(p.Gc * p.ndr * kMetaStride * 4);
    p.prep_bytes = p.twt_off + r256(p.Gc * p.Tcap * 16 * G * 2);
    p.ws_bytes = p.S * D * p.Bp * 4;
    return p;
}

// --------------------------------------------------------------- prep ------
// Tiles of group g start at tile g*Tcap.  For range r, meta[(g*ndr + r)*4 + 0..2]
// = (tb, tm, te): layer-0 tiles [tb, tm), layer-1 tiles [tm, te) (relative to
// g*Tcap).  tfeat[t*16 + p] = feature - r*Dc of position p of tile t, or -1 for
// padding; twt[(t*16 + p)*G + l] = weight of label l (0 for padding and for
// labels >= O).  Features within a range's layer are in ascending order.
template <typename T, int G>
__global__ __launch_bounds__(256) void bwdf_prep_kernel(const int32_t* __restrict__ idx,
                                                        const uint16_t* __restrict__ W,
                                                        int* __restrict__ tfeat,
                                                        int* __restrict__ meta,
                                                        uint16_t* __restrict__ twt, int F, int D,
                                                        int64_t O, int ndr, int Dc, int Tcap) {
    __shared__ __attribute__((aligned(16))) uint16_t s_w[G * 256];  // W_g [label][slot]
    __shared__ int s_idx[256];
    __shared__ int s_flag[256];  // bit 0: first occurrence, bit 1: occurs more than once
    __shared__ int s_perm[256];  // slots in (index, slot) order
    __shared__ int s_cnt[2][kMaxRanges];
    __shared__ int s_tile[kMaxRanges][3];
    __shared__ int s_ntiles;
    const int64_t g = blockIdx.x;
    const int64_t l0 = g * G;
    const int tid = threadIdx.x;
    for (int i = tid; i < 2 * kMaxRanges; i += 256) (&s_cnt[0][0])[i] = 0;
    if (tid < F) s_idx[tid] = min(max(idx[g * F + tid], 0), D - 1);
    for (int it = tid; it < G * (F / 8); it += 256) {
        const int l = it / (F / 8), j0 = (it % (F / 8)) * 8;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (l0 + l < O) v = *reinterpret_cast<const u32x4*>(W + (l0 + l) * F + j0);
        *reinterpret_cast<u32x4*>(&s_w[l * F + j0]) = v;
    }
    __syncthreads();
    int f = 0, rank = 0, cnt = 0;
    bool first = false;
    if (tid < F) {
        f = s_idx[tid];
        int before = 0;
        for (int k = 0; k < F; ++k) {
            const int v = s_idx[k];
            rank += v < f;
            before += (v == f) & (k < tid);
            cnt += v == f;
        }
        rank += before;
        first = before == 0;
        s_perm[rank] = tid;
        s_flag[tid] = (first ? 1 : 0) | (cnt > 1 ? 2 : 0);
    }
    __syncthreads();
    const int r = f / Dc;
    const int r_lo = r * Dc;
    int pu = 0, pd = 0;  // rank among the range's distinct / duplicated features
    if (tid < F && first) {
        for (int k = 0; k < F; ++k) {
            const int v = s_idx[k], fl = s_flag[k];
            const bool in = (fl & 1) && v >= r_lo && v < f;
            pu += in;
            pd += in && (fl & 2);
        }
        atomicAdd(&s_cnt[0][r], 1);
        if (cnt > 1) atomicAdd(&s_cnt[1][r], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int t = 0;
        for (int rr = 0; rr < ndr; ++rr) {
            s_tile[rr][0] = t;
            t += (s_cnt[0][rr] + 15) / 16;
            s_tile[rr][1] = t;
            t += (s_cnt[1][rr] + 15) / 16;
            s_tile[rr][2] = t;
        }
        s_ntiles = t;
    }
    __syncthreads();
    for (int rr = tid; rr < ndr; rr += 256) {
        int* m = meta + (g * ndr + rr) * kMetaStride;
        m[0] = s_tile[rr][0];
        m[1] = s_tile[rr][1];
        m[2] = s_tile[rr][2];
        m[3] = 0;
    }
    const int64_t tbase = g * Tcap;
    if (tid < F && first) {
        const int t0 = s_tile[r][0] + pu / 16, p0 = pu % 16;
        const int t1 = s_tile[r][1] + pd / 16, p1 = pd % 16;
        tfeat[(tbase + t0) * 16 + p0] = f - r_lo;
        if (cnt > 1) tfeat[(tbase + t1) * 16 + p1] = f - r_lo;
        uint16_t* hi_row = twt + ((tbase + t0) * 16 + p0) * G;
        uint16_t* lo_row = twt + ((tbase + t1) * 16 + p1) * G;
#pragma unroll 1
        for (int lc = 0; lc < G; lc += 8) {
            u32x4 hv, lv;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int l = lc + e;
                uint32_t hb, lb = 0;
                if (cnt == 1) {
                    hb = s_w[l * F + tid];
                } else {
                    float sum = 0.0f;
                    for (int q = 0; q < cnt; ++q) sum += bits_to_f32<T>(s_w[l * F + s_perm[rank + q]]);
                    hb = f32_to_bits<T>(sum);
                    lb = f32_to_bits<T>(sum - bits_to_f32<T>(hb));
                }
                if (e & 1) {
                    hv[e >> 1] |= hb << 16;
                    lv[e >> 1] |= lb << 16;
                } else {
                    hv[e >> 1] = hb;
                    lv[e >> 1] = lb;
                }
            }
            *reinterpret_cast<u32x4*>(hi_row + lc) = hv;
            if (cnt > 1) *reinterpret_cast<u32x4*>(lo_row + lc) = lv;
        }
    }
    // padding slots of every range's layers
    const int nslots = s_ntiles * 16;
    for (int i = tid; i < nslots; i += 256) {
        const int t = i / 16, p = i % 16;
        int rr = 0;
        while (t >= s_tile[rr][2]) ++rr;  // empty ranges have tb == te and are skipped
        const bool lay1 = t >= s_tile[rr][1];
        const int used = lay1 ? s_cnt[1][rr] : s_cnt[0][rr];
        const int slot = (t - s_tile[rr][lay1 ? 1 : 0]) * 16 + p;
        if (slot < used) continue;
        tfeat[(tbase + t) * 16 + p] = -1;
        uint16_t* row = twt + ((tbase + t) * 16 + p) * G;
        for (int lc = 0; lc < G; lc += 8)
            *reinterpret_cast<u32x4*>(row + lc) = u32x4{0u, 0u, 0u, 0u};
    }
}

// --------------------------------------------------------------- main ------
template <int G, int RPW, int FP>
struct BwdFCfg {
    static constexpr int KS = G >= 32 ? G / 32 : 1;  // MFMA k-steps over labels
    static constexpr int MT = RPW / 16;              // 16-row batch tiles per wave
    static constexpr int BT = 4 * RPW;               // batch columns per workgroup
    static constexpr int AS = acc_stride(BT);
    static constexpr int NS = G >= 128 ? 2 : 3;      // groups in flight per wave
    // tiles per group kept in registers (a range's usual share of F, padded)
    static constexpr int MAXT = FP >= 256 ? 6 : FP >= 128 ? 4 : 3;
};

template <int KS, int MT, int MAXT>
struct BwdFRegs {
    u32x4 a[MT][KS];    // dY rows of the wave (A operand)
    u32x4 b[MAXT][KS];  // tile rows (B operand)
    int f[MAXT];        // feature (relative to the range) of this lane's tile column
    int tb, tm, te;     // tiles of the group's range (relative to the group base)
};

template <typename T, int G, int RPW, int FP>
__global__ __launch_bounds__(kMainThreads) void bwdf_main_kernel(
    const int* __restrict__ tfeat, const int* __restrict__ meta, const uint16_t* __restrict__ twt,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S, int Tcap) {
    using C = BwdFCfg<G, RPW, FP>;
    constexpr int KS = C::KS, MT = C::MT, BT = C::BT, AS = C::AS, NS = C::NS, MAXT = C::MAXT;
    using R = BwdFRegs<KS, MT, MAXT>;
    __shared__ __attribute__((aligned(16))) float acc[max_dc(BT) * AS + kDummyFloats];

    const int64_t work = xcd_remap(blockIdx.x, (int64_t)S * ndr * nbt);
    if (work < 0) return;
    const int bt = (int)(work % nbt);
    const int r = (int)((work / nbt) % ndr);
    const int s = (int)(work / ((int64_t)nbt * ndr));
    const int d_lo = r * Dc;
    const int dn = min(Dc, D - d_lo);
    const int64_t g_lo = (int64_t)s * gps;
    const int64_t g_hi = min<int64_t>(Gc, g_lo + gps);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15;  // A row within an M tile / B column (tile position)
    const int kq = lane >> 4;   // which 8 of the 32 K elements
    const bool kq_ok = G >= 32 || kq < 2;

    for (int i = tid * 4; i < dn * AS; i += kMainThreads * 4)
        *reinterpret_cast<f32x4*>(&acc[i]) = f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();

    // this lane's dY rows (clamped: rows >= B only feed partial columns never read)
    const uint16_t* yrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int b = min(bt * BT + wave * RPW + mt * 16 + col, B - 1);
        yrow[mt] = dY + (int64_t)b * lddy;
    }
    const int kofs = kq_ok ? kq * 8 : 0;
    const int dummy = max_dc(BT) * AS + tid * 4;
    const int bofs = wave * RPW + kq * 4;  // batch column of this lane's first D row

    auto load = [&](R& x, int64_t g) {
        const int* m = meta + (g * ndr + r) * kMetaStride;
        x.tb = m[0];
        x.tm = m[1];
        x.te = m[2];
        const int64_t c0 = g * G;
        if (c0 + G <= O) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    u32x4 v = *reinterpret_cast<const u32x4*>(yrow[mt] + c0 + ks * 32 + kofs);
                    x.a[mt][ks] = kq_ok ? v : u32x4{0u, 0u, 0u, 0u};
                }
        } else {  // last group: labels >= O read as zero
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int64_t c = c0 + ks * 32 + kofs;
                    uint32_t h[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) h[e] = (kq_ok && c + e < O) ? yrow[mt][c + e] : 0u;
#pragma unroll
                    for (int q = 0; q < 4; ++q) x.a[mt][ks][q] = h[2 * q] | (h[2 * q + 1] << 16);
                }
        }
        const int64_t tbase = g * Tcap + x.tb;
        const int nt = x.te - x.tb;
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t >= nt) break;
            const int64_t row = (tbase + t) * 16 + col;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 v = *reinterpret_cast<const u32x4*>(twt + row * G + ks * 32 + kofs);
                x.b[t][ks] = kq_ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
            x.f[t] = tfeat[row];
        }
    };

    auto addr = [&](int f, int mt) { return f >= 0 ? f * AS + bofs + mt * 16 : dummy; };

    // read-add-write of tiles [t0, t1) of one layer (features distinct)
    auto rmw = [&](const R& x, const f32x4 (&c)[MAXT][MT], int t0, int t1) {
        f32x4 old[MAXT][MT];
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t < t0 || t >= t1) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                old[t][mt] = *reinterpret_cast<const f32x4*>(&acc[addr(x.f[t], mt)]);
        }
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t < t0 || t >= t1) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                *reinterpret_cast<f32x4*>(&acc[addr(x.f[t], mt)]) = old[t][mt] + c[t][mt];
        }
    };

    auto compute = [&](const R& x, int64_t g) {
        const int nt = x.te - x.tb;
        const int nreg = min(nt, MAXT);
        const int n0 = min(x.tm - x.tb, nreg);
        f32x4 c[MAXT][MT];
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t >= nreg) break;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(x.a[mt][ks], x.b[t][ks], v);
                c[t][mt] = v;
            }
        }
        rmw(x, c, 0, n0);
        if (n0 < nreg) rmw(x, c, n0, nreg);
        // tiles beyond the register set (ranges holding an unusual share of F)
        for (int t = MAXT; t < nt; ++t) {
            const int64_t row = (g * Tcap + x.tb + t) * 16 + col;
            u32x4 bb[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 v = *reinterpret_cast<const u32x4*>(twt + row * G + ks * 32 + kofs);
                bb[ks] = kq_ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
            const int f = tfeat[row];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(x.a[mt][ks], bb[ks], v);
                f32x4* p = reinterpret_cast<f32x4*>(&acc[addr(f, mt)]);
                *p = *p + v;
            }
        }
    };

    R rg[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k)
        if (g_lo + k < g_hi) load(rg[k], g_lo + k);
    for (int64_t g = g_lo; g < g_hi; g += NS) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            if (g + k >= g_hi) break;
            compute(rg[k], g + k);
            if (g + k + NS < g_hi) load(rg[k], g + k + NS);
        }
    }
    __syncthreads();

    // ---- write the partial: ws[s][d_lo + d][bt*BT + b] ----
    float* out = ws + ((int64_t)s * D + d_lo) * Bp + (int64_t)bt * BT;
    for (int i = tid; i < dn * (BT / 4); i += kMainThreads) {
        const int d = i / (BT / 4), b4 = (i % (BT / 4)) * 4;
        *reinterpret_cast<f32x4*>(out + (int64_t)d * Bp + b4) =
            *reinterpret_cast<const f32x4*>(&acc[d * AS + b4]);
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

template <typename T, int G, int RPW, int FP>
int launch_main(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
                hipStream_t st) {
    const int64_t nlog = p.S * p.ndr * p.nbt;
    const int64_t grid = 8 * ceil_div(nlog, 8);
    bwdf_main_kernel<T, G, RPW, FP><<<dim3((unsigned)grid), dim3(kMainThreads), 0, st>>>(
        tfeat, meta, twt, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, O, p.Gc, (int)p.nbt,
        (int)p.ndr, (int)p.Dc, (int)p.gps, (int)p.S, (int)p.Tcap);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

template <typename T, int G, int RPW>
int dispatch_fp(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F,
                int64_t O, hipStream_t st) {
#define HASTE_BWDF_ARGS tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st
    if (F <= 64) return launch_main<T, G, RPW, 64>(HASTE_BWDF_ARGS);
    if (F <= 128) return launch_main<T, G, RPW, 128>(HASTE_BWDF_ARGS);
    return launch_main<T, G, RPW, 256>(HASTE_BWDF_ARGS);
#undef HASTE_BWDF_ARGS
}

template <typename T, int G>
int run_main(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
             int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F,
             int64_t O, hipStream_t st) {
    if (p.BT == 64) return dispatch_fp<T, G, 16>(tfeat, meta, twt, dY, lddy, ws, p, B, D, F, O, st);
    return dispatch_fp<T, G, 32>(tfeat, meta, twt, dY, lddy, ws, p, B, D, F, O, st);
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
    if (p.ndr > kMaxRanges) {
        set_error("%s: D = %lld is too large (at most %lld features)", fn, (long long)D,
                  (long long)kMaxRanges * max_dc((int)p.BT));
        return HASTE_ERR_UNSUPPORTED;
    }
    if (workspace == nullptr || workspace_bytes < p.prep_bytes + p.ws_bytes) {
        set_error("%s: workspace too small (%lld bytes, need %lld)", fn,
                  (long long)workspace_bytes, (long long)(p.prep_bytes + p.ws_bytes));
        return HASTE_ERR_WORKSPACE;
    }
    char* base = static_cast<char*>(workspace);
    int* tfeat = reinterpret_cast<int*>(base + p.tfeat_off);
    int* meta = reinterpret_cast<int*>(base + p.meta_off);
    uint16_t* twt = reinterpret_cast<uint16_t*>(base + p.twt_off);
    float* ws = reinterpret_cast<float*>(base + p.prep_bytes);
    auto* w = static_cast<const uint16_t*>(W);
    auto* y = static_cast<const uint16_t*>(dY);
    const dim3 pgrid((unsigned)p.Gc);
    switch (G) {
#define HASTE_BWDF_G(GG)                                                                        \
    case GG:                                                                                    \
        if (dtype == HASTE_DTYPE_BF16) {                                                        \
            bwdf_prep_kernel<BF16, GG><<<pgrid, dim3(256), 0, st>>>(                            \
                idx, w, tfeat, meta, twt, (int)F, (int)D, O, (int)p.ndr, (int)p.Dc, (int)p.Tcap); \
            HASTE_CHECK_LAUNCH(fn);                                                             \
            rc = run_main<BF16, GG>(tfeat, meta, twt, y, lddy, ws, p, B, D, F, O, st);          \
        } else {                                                                                \
            bwdf_prep_kernel<F16, GG><<<pgrid, dim3(256), 0, st>>>(                             \
                idx, w, tfeat, meta, twt, (int)F, (int)D, O, (int)p.ndr, (int)p.Dc, (int)p.Tcap); \
            HASTE_CHECK_LAUNCH(fn);                                                             \
            rc = run_main<F16, GG>(tfeat, meta, twt, y, lddy, ws, p, B, D, F, O, st);           \
        }                                                                                       \
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
