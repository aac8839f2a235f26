// Grouped fixed-fan-in backward to features, deterministic (gfx950).
//
//   dXT[d, b] = sum_{g, j: idx[g, j] = d} sum_{l in g} W[l, j] * dY[b, l]
//
// The reference scatters with fp32 atomicAdd into global memory
// (shared_ffi/ffi_backward_features.cu:202-212), so its sums depend on timing.
// Here no float atomic touches any memory and every sum has a fixed order:
//
//  1. plan (depends on idx only; callers may keep it across calls until idx
//     changes): the distinct indices of every group are split by feature
//     range (Dc features each) and laid out in tiles of 16 positions.  An
//     index that occurs k > 1 times in the group gets a "hi" row in layer 0
//     and a "lo" row in layer 1, so inside a layer every feature occurs once.
//     Inside a layer, features are dealt round-robin over the tiles in order
//     of (feature mod 16, feature), so the 16 lanes of a tile mostly hit
//     distinct LDS bank groups in step 2.
//     gather (every call): tile row p of group g = W_g column of p's slot,
//     transposed (WT[pos][label]); a duplicated index gets
//     sum_j W[l, j] (fp32, ascending j) split into its 16-bit rounding (hi)
//     and the 16-bit rounding of the remainder (lo).
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

#include "bwdf_plan.hpp"

#ifndef HASTE_BWDF_STATIC_TILES
#define HASTE_BWDF_STATIC_TILES 0  // 1: always MAXT tile loads per ring slot (measured slower)
#endif

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

constexpr int kMainThreads = 256;  // 4 waves
// --------------------------------------------------------------- plan ------
// Tiles of group g start at tile g*Tcap.  For range r, meta[(g*ndr + r)*4 + 0..2]
// = (tb, tm, te): layer-0 tiles [tb, tm), layer-1 tiles [tm, te) (relative to
// g*Tcap); meta[(g*ndr + ndr-1)*4 + 2] is the group's tile count.  For tile row
// (t, p): tfeat = byte offset of the feature's row in the main kernel's LDS
// partial, (feature - r*Dc) * row_bytes, or (trash_row + p) * row_bytes for
// padding; tsrc = (start << 10) |
// (count << 1) | lo: the row sums W over slots perm[g*F + start ..
// start+count) (count 0 = padding); lo selects the remainder row.
__global__ __launch_bounds__(256) void bwdf_plan_kernel(const int32_t* __restrict__ idx,
                                                        int* __restrict__ tfeat,
                                                        int* __restrict__ tsrc,
                                                        int* __restrict__ perm,
                                                        int* __restrict__ meta, int F, int D,
                                                        int ndr, int Dc, int Tcap, int row_bytes,
                                                        int trash_row) {
    __shared__ int s_idx[256];
    __shared__ int s_flag[256];  // bit 0: first occurrence, bit 1: occurs more than once
    __shared__ int s_cnt[2][kMaxRanges];
    __shared__ int s_tile[kMaxRanges][3];
    __shared__ int s_ntiles;
    const int64_t g = blockIdx.x;
    const int tid = threadIdx.x;
    for (int i = tid; i < 2 * kMaxRanges; i += 256) (&s_cnt[0][0])[i] = 0;
    if (tid < F) s_idx[tid] = min(max(idx[g * F + tid], 0), D - 1);
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
        perm[g * F + rank] = tid;
        s_flag[tid] = (first ? 1 : 0) | (cnt > 1 ? 2 : 0);
    }
    __syncthreads();
    const int r = f / Dc;
    const int r_lo = r * Dc;
    const int key = (((f - r_lo) & 15) << 16) | (f - r_lo);
    int pu = 0, pd = 0;  // order of the feature among the range's distinct / duplicated ones
    if (tid < F && first) {
        for (int k = 0; k < F; ++k) {
            const int v = s_idx[k], fl = s_flag[k];
            const int kk = (((v - r_lo) & 15) << 16) | (v - r_lo);
            const bool in = (fl & 1) && v >= r_lo && v < r_lo + Dc && kk < key;
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
        const int T0 = s_tile[r][1] - s_tile[r][0];
        const int64_t row0 = (tbase + s_tile[r][0] + pu % T0) * 16 + pu / T0;
        tfeat[row0] = (f - r_lo) * row_bytes;
        tsrc[row0] = (rank << 10) | (cnt << 1);
        if (cnt > 1) {
            const int T1 = s_tile[r][2] - s_tile[r][1];
            const int64_t row1 = (tbase + s_tile[r][1] + pd % T1) * 16 + pd / T1;
            tfeat[row1] = (f - r_lo) * row_bytes;
            tsrc[row1] = (rank << 10) | (cnt << 1) | 1;
        }
    }
    // padding rows of every range's layers
    const int nslots = s_ntiles * 16;
    for (int i = tid; i < nslots; i += 256) {
        const int t = i / 16, p = i % 16;
        int rr = 0;
        while (t >= s_tile[rr][2]) ++rr;  // empty ranges have tb == te and are skipped
        const bool lay1 = t >= s_tile[rr][1];
        const int used = lay1 ? s_cnt[1][rr] : s_cnt[0][rr];
        const int tl0 = s_tile[rr][lay1 ? 1 : 0];
        const int nt = (lay1 ? s_tile[rr][2] : s_tile[rr][1]) - tl0;
        if (p * nt + (t - tl0) < used) continue;
        tfeat[(tbase + t) * 16 + p] = (trash_row + p) * row_bytes;
        tsrc[(tbase + t) * 16 + p] = 0;
    }
}

// ------------------------------------------------------------- gather ------
// One workgroup per group: W_g is staged in LDS ([label][slot], row stride
// F + 2 halves so the 8 label rows a wave reads at once sit in distinct banks),
// then each thread writes 8 labels (16 bytes) of one tile row.
template <typename T, int G>
__global__ __launch_bounds__(256) void bwdf_gather_kernel(const uint16_t* __restrict__ W,
                                                          const int* __restrict__ tsrc,
                                                          const int* __restrict__ perm,
                                                          const int* __restrict__ meta,
                                                          uint16_t* __restrict__ twt, int F,
                                                          int64_t O, int ndr, int Tcap) {
    __shared__ uint32_t s_w[G * 129];  // G rows of (F + 2) halves, F <= 256
    __shared__ int s_perm[256];
    const int64_t g = blockIdx.x;
    const int tid = threadIdx.x;
    const int ldw = F / 2 + 1;  // row stride in 32-bit words
    for (int it = tid; it < G * (F / 8); it += 256) {
        const int l = it / (F / 8), j0 = (it % (F / 8)) * 8;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (g * G + l < O) v = *reinterpret_cast<const u32x4*>(W + (g * G + l) * F + j0);
#pragma unroll
        for (int q = 0; q < 4; ++q) s_w[l * ldw + j0 / 2 + q] = v[q];
    }
    if (tid < F) s_perm[tid] = perm[g * F + tid];
    const int nrows = meta[(g * ndr + ndr - 1) * kMetaStride + 2] * 16;
    __syncthreads();
    auto wv = [&](int l, int slot) -> uint32_t {
        const uint32_t w2 = s_w[l * ldw + (slot >> 1)];
        return (slot & 1) ? (w2 >> 16) : (w2 & 0xFFFFu);
    };
    constexpr int CH = G / 8;  // 16-byte chunks per row
    for (int it = tid; it < nrows * CH; it += 256) {
        const int row = it / CH, lc = (it % CH) * 8;
        const u32x4 v = wt_chunk<T>(tsrc[(g * Tcap) * 16 + row], s_perm, wv, lc);
        *reinterpret_cast<u32x4*>(twt + ((g * Tcap) * 16 + row) * G + lc) = v;
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
    int f[MAXT];        // LDS byte offset of this lane's tile column (feature row)
    int tb, tm, te;     // tiles of the group's range (relative to the group base)
};

// Per-wave LDS ring of group tile ranges: kMetaChunk groups per chunk, two chunks.
constexpr int kMetaChunk = 64;
constexpr int kMetaInts = kMainThreads / 64 * 2 * kMetaChunk * 2;

template <typename T, int G, int RPW, int FP>
__global__ __launch_bounds__(kMainThreads) void bwdf_main_kernel(
    const int* __restrict__ tfeat, const int* __restrict__ meta, const uint16_t* __restrict__ twt,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S, int Tcap) {
    using C = BwdFCfg<G, RPW, FP>;
    constexpr int KS = C::KS, MT = C::MT, BT = C::BT, AS = C::AS, NS = C::NS, MAXT = C::MAXT;
    using R = BwdFRegs<KS, MT, MAXT>;
    __shared__ __attribute__((aligned(16))) float acc[(max_dc(BT) + kTrashRows) * AS];
    __shared__ __attribute__((aligned(16))) int s_meta[kMetaInts];

    const int64_t work = xcd_remap(blockIdx.x, (int64_t)S * ndr * nbt);
    if (work < 0) return;
    const int bt = (int)(work % nbt);
    const int r = (int)((work / nbt) % ndr);
    const int s = (int)(work / ((int64_t)nbt * ndr));
    const int d_lo = r * Dc;
    const int dn = min(Dc, D - d_lo);
    const int64_t g_lo = (int64_t)s * gps;
    const int64_t g_hi = min<int64_t>(Gc, g_lo + gps);
    const int64_t g_full = min<int64_t>(g_hi, O / G);  // groups before it have G labels

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
    char* const acc_b = reinterpret_cast<char*>(acc) + (wave * RPW + kq * 4) * 4;

    // Tile ranges (tb, tm, te) of the slice's groups reach the wave through a
    // per-wave LDS ring (lane L loads group c*64 + L of chunk c), so that reading
    // them is an in-order LDS access like the partial's reads and writes.
    // Entries are packed to two ints, (tb | tm << 16, te), both of which are used.
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
    int* const my_meta = s_meta + wave * 2 * kMetaChunk * 2;
    auto meta_chunk = [&](int64_t c) {
        const int64_t g = g_lo + c * kMetaChunk + lane;
        return *reinterpret_cast<const i32x4*>(meta + (min<int64_t>(g, g_hi - 1) * ndr + r) *
                                                           kMetaStride);
    };
    auto put_chunk = [&](int64_t c, i32x4 v) {
        *reinterpret_cast<i32x2*>(my_meta + ((c & 1) * kMetaChunk + lane) * 2) =
            i32x2{v[0] | (v[1] << 16), v[2]};
    };
    auto read_meta = [&](int64_t i) {  // i = g - g_lo
        return *reinterpret_cast<const i32x2*>(
            my_meta + (((i / kMetaChunk) & 1) * kMetaChunk + i % kMetaChunk) * 2);
    };
    auto unpack_meta = [&](R& x, i32x2 m) {
        const int m0 = __builtin_amdgcn_readfirstlane(m[0]);
        x.tb = m0 & 0xFFFF;
        x.tm = m0 >> 16;
        x.te = __builtin_amdgcn_readfirstlane(m[1]);
    };

    // tile rows of a group (tb/te set); slots past the range's last tile point at
    // this lane's trash row (their MFMA results are added there and never read)
    const int trash_f = (max_dc(BT) + col) * AS * 4;
    auto load_tiles = [&](R& x, int64_t g) {
        const int64_t tbase = g * Tcap + x.tb;
        const int nt = x.te - x.tb;
#if HASTE_BWDF_STATIC_TILES
        // always MAXT tile loads (slots past the last tile re-read it: L1 hits), so
        // the compiler knows how many loads follow each ring slot's
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            const int64_t row = (tbase + max(0, min(t, nt - 1))) * 16 + col;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 v = *reinterpret_cast<const u32x4*>(twt + row * G + ks * 32 + kofs);
                x.b[t][ks] = kq_ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
            const int f = tfeat[row];
            x.f[t] = t < nt ? f : trash_f;
        }
#else
#pragma unroll
        for (int t = 0; t < MAXT; ++t) x.f[t] = trash_f;
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
#endif
    };

    auto load = [&](R& x, int64_t g, i32x2 m) {  // g < g_full: all G labels
        unpack_meta(x, m);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 v = *reinterpret_cast<const u32x4*>(yrow[mt] + g * G + ks * 32 + kofs);
                x.a[mt][ks] = kq_ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
        load_tiles(x, g);
    };

    auto mfma_tiles = [&](const R& x, int nreg, f32x4 (&c)[MAXT][MT]) {
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t >= nreg) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(x.a[mt][ks], x.b[t][ks], v);
                c[t][mt] = v;
            }
        }
    };

    // acc[feature rows of tiles t0..t1-1] += c: all reads of the tiles are issued
    // before their writes (the tiles' features are distinct)
    auto rmw = [&](const R& x, const f32x4 (&c)[MAXT][MT], int t0, int t1) {
        f32x4 old[MAXT][MT];
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t < t0 || t >= t1) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                old[t][mt] = *reinterpret_cast<const f32x4*>(acc_b + x.f[t] + mt * 64);
        }
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            if (t < t0 || t >= t1) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                *reinterpret_cast<f32x4*>(acc_b + x.f[t] + mt * 64) = old[t][mt] + c[t][mt];
        }
    };

    // Writes of the second 16-row block (mt = 1) of the previous group, deferred:
    // that block's columns are disjoint from the first block's, so the next group's
    // first-block reads may be issued before them (reads then overlap writes).
    // Every step issues the same LDS operations (unused tile slots go to the trash
    // rows), so each wait covers exactly the operations it needs.
    struct Pend {
        f32x4 old[MAXT], c[MAXT];
        int f[MAXT];
    } pend;
    auto pend_clear = [&]() {
#pragma unroll
        for (int t = 0; t < MAXT; ++t) {
            pend.old[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            pend.c[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            pend.f[t] = trash_f;
        }
    };
    pend_clear();
    auto flush = [&]() {
        if constexpr (MT == 2) {
#pragma unroll
            for (int t = 0; t < MAXT; ++t)
                *reinterpret_cast<f32x4*>(acc_b + pend.f[t] + 64) = pend.old[t] + pend.c[t];
        }
    };
    // the same, re-reading the values (nothing else touches those words before):
    // keeps the fast path's adds next to their writes instead of at the loop head
    auto flush_rmw = [&]() {
        if constexpr (MT == 2) {
#pragma unroll
            for (int t = 0; t < MAXT; ++t) {
                f32x4* q = reinterpret_cast<f32x4*>(acc_b + pend.f[t] + 64);
                *q = *q + pend.c[t];
            }
        }
    };

    auto compute = [&](const R& x, int64_t g) {
        const int nt = x.te - x.tb;
        const int n0 = x.tm - x.tb;
        if (MT == 2 && n0 == nt && nt <= MAXT) {
            // one layer, all tiles in registers: R0(g) W1(g-1) R1(g) W0(g); W1(g) deferred
            f32x4 c[MAXT][MT];
            mfma_tiles(x, MAXT, c);
            f32x4 o0[MAXT];
#pragma unroll
            for (int t = 0; t < MAXT; ++t) o0[t] = *reinterpret_cast<const f32x4*>(acc_b + x.f[t]);
            flush();
#pragma unroll
            for (int t = 0; t < MAXT; ++t) {
                pend.old[t] = *reinterpret_cast<const f32x4*>(acc_b + x.f[t] + 64);
                pend.c[t] = c[t][MT - 1];
                pend.f[t] = x.f[t];
            }
#pragma unroll
            for (int t = 0; t < MAXT; ++t)
                *reinterpret_cast<f32x4*>(acc_b + x.f[t]) = o0[t] + c[t][0];
            return;
        }
        flush_rmw();
        pend_clear();
        const int nreg = min(nt, MAXT);
        const int n0r = min(n0, nreg);
        f32x4 c[MAXT][MT];
        mfma_tiles(x, nreg, c);
        rmw(x, c, 0, n0r);
        if (n0r < nreg) rmw(x, c, n0r, nreg);
        // tiles beyond the register set (ranges holding an unusual share of F)
        for (int t = MAXT; t < nt; ++t) {
            const int64_t row = (g * Tcap + x.tb + t) * 16 + col;
            u32x4 bb[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u32x4 v = *reinterpret_cast<const u32x4*>(twt + row * G + ks * 32 + kofs);
                bb[ks] = kq_ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
            char* p = acc_b + tfeat[row];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = *reinterpret_cast<const f32x4*>(p + mt * 64);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(x.a[mt][ks], bb[ks], v);
                *reinterpret_cast<f32x4*>(p + mt * 64) = v;
            }
        }
    };

    // Meta chunks 0 and 1 in LDS, chunk 2 in registers.  Iteration i looks up
    // groups [i + NS, i + 2NS): chunk (i + NS) / 64 and possibly the next one,
    // so entering a new chunk frees the slot of the one before it.
    put_chunk(0, meta_chunk(0));
    put_chunk(1, meta_chunk(1));
    i32x4 mnext = meta_chunk(2);
    int64_t c_top = 1;  // newest chunk in LDS

    if (g_lo < g_full) {
        // ring of NS groups in flight; slots past the last full group re-load it
        // (never computed)
        const int64_t nfull = g_full - g_lo;
        R rg[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const int64_t ik = min<int64_t>(k, nfull - 1);
            load(rg[k], g_lo + ik, read_meta(ik));
        }
        for (int64_t i = 0; i < nfull; i += NS) {
            if ((i + NS) / kMetaChunk + 1 > c_top) {
                ++c_top;
                put_chunk(c_top, mnext);
                mnext = meta_chunk(c_top + 1);
            }
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const int64_t in = min<int64_t>(i + k + NS, nfull - 1);
                const i32x2 m = read_meta(in);  // issued before compute's LDS traffic
                if (i + k < nfull) compute(rg[k], g_lo + i + k);
                load(rg[k], g_lo + in, m);
            }
        }
    }
    flush_rmw();
    pend_clear();
    if (g_full < g_hi) {  // the last group, holding O % G labels: columns >= O read as 0
        R x;
        const int64_t g = g_full;
        put_chunk((g - g_lo) / kMetaChunk, meta_chunk((g - g_lo) / kMetaChunk));
        unpack_meta(x, read_meta(g - g_lo));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int64_t c = g * G + ks * 32 + kofs;
                uint32_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = (kq_ok && c + e < O) ? yrow[mt][c + e] : 0u;
#pragma unroll
                for (int q = 0; q < 4; ++q) x.a[mt][ks][q] = h[2 * q] | (h[2 * q + 1] << 16);
            }
        load_tiles(x, g);
        compute(x, g);
        flush_rmw();
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
// Both reduce kernels read the partials as 16-byte rows of 4 batch columns
// (Bp is a multiple of 64, so every such read is in bounds and aligned).
__device__ __forceinline__ f32x4 sum_slices(const float* __restrict__ ws, int64_t D, int Bp,
                                            int S, int64_t d, int b4) {
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    const float* p = ws + d * Bp + b4;
    const int64_t step = D * Bp;
#pragma unroll 4
    for (int s = 0; s < S; ++s) v += *reinterpret_cast<const f32x4*>(p + s * step);
    return v;
}

__global__ __launch_bounds__(256) void bwdf_reduce_kernel(const float* __restrict__ ws,
                                                          float* __restrict__ dXT, int B, int Bp,
                                                          int D, int S) {
    const int nb4 = (B + 3) / 4;
    const int64_t n = (int64_t)D * nb4;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t d = i / nb4;
        const int b4 = (int)(i % nb4) * 4;
        const f32x4 v = sum_slices(ws, D, Bp, S, d, b4);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (b4 + e < B) dXT[d * B + b4 + e] = v[e];
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
    {
        const int r = threadIdx.x >> 3, c4 = (threadIdx.x & 7) * 4;
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (d0 + r < D) v = sum_slices(ws, D, Bp, S, d0 + r, b0 + c4);
#pragma unroll
        for (int e = 0; e < 4; ++e) t[r][c4 + e] = v[e];
    }
    __syncthreads();
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // ty in 0..7
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

// Checks the arguments and the workspace size; returns the plan.
int check_bwdf(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
               int32_t dtype, const void* workspace, int64_t workspace_bytes, BwdFPlan* out) {
    int rc = check_ffi_shape(fn, B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    const BwdFPlan p = make_plan(B, D, F, O, G);
    if (p.ndr > kMaxRanges) {
        set_error("%s: D = %lld is too large (at most %lld features)", fn, (long long)D,
                  (long long)kMaxRanges * max_dc((int)p.BT));
        return HASTE_ERR_UNSUPPORTED;
    }
    HASTE_CHECK_ARG(aligned16(workspace), "%s: workspace must be 16-byte aligned", fn);
    if (workspace == nullptr || workspace_bytes < p.prep_bytes + p.ws_bytes) {
        set_error("%s: workspace too small (%lld bytes, need %lld)", fn,
                  (long long)workspace_bytes, (long long)(p.prep_bytes + p.ws_bytes));
        return HASTE_ERR_WORKSPACE;
    }
    *out = p;
    return HASTE_OK;
}

// Runs [plan +] [gather +] main; leaves the per-slice partials in the workspace.
int run_partials(const char* fn, const int32_t* idx, const void* W, const void* dY, int64_t lddy,
                 void* workspace, int64_t workspace_bytes, int64_t B, int64_t D, int64_t F,
                 int64_t O, int64_t G, int32_t dtype, int32_t plan_ready, hipStream_t st,
                 BwdFPlan* plan_out) {
    BwdFPlan p;
    int rc = check_bwdf(fn, B, D, F, O, G, dtype, workspace, workspace_bytes, &p);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && W && dY, "%s: null pointer", fn);
    HASTE_CHECK_ARG(lddy >= O && lddy % 8 == 0,
                    "%s: lddy must be >= O and a multiple of 8 (lddy=%lld O=%lld)", fn,
                    (long long)lddy, (long long)O);
    HASTE_CHECK_ARG(aligned16(W) && aligned16(dY), "%s: W and dY must be 16-byte aligned", fn);
    HASTE_CHECK_ARG(plan_ready >= 0 && plan_ready <= 2, "%s: plan_ready must be 0, 1 or 2 (got %d)",
                    fn, (int)plan_ready);
    char* base = static_cast<char*>(workspace);
    int* tfeat = reinterpret_cast<int*>(base + p.tfeat_off);
    int* tsrc = reinterpret_cast<int*>(base + p.tsrc_off);
    int* perm = reinterpret_cast<int*>(base + p.perm_off);
    int* meta = reinterpret_cast<int*>(base + p.meta_off);
    uint16_t* twt = reinterpret_cast<uint16_t*>(base + p.twt_off);
    float* ws = reinterpret_cast<float*>(base + p.prep_bytes);
    auto* w = static_cast<const uint16_t*>(W);
    auto* y = static_cast<const uint16_t*>(dY);
    const dim3 pgrid((unsigned)p.Gc);
    if (!plan_ready) {
        bwdf_plan_kernel<<<pgrid, dim3(256), 0, st>>>(
            idx, tfeat, tsrc, perm, meta, (int)F, (int)D, (int)p.ndr, (int)p.Dc, (int)p.Tcap,
            acc_stride((int)p.BT) * 4, max_dc((int)p.BT));
        HASTE_CHECK_LAUNCH(fn);
    }
    const bool gather = plan_ready != 2;
    switch (G) {
#define HASTE_BWDF_G(GG)                                                                        \
    case GG:                                                                                    \
        if (dtype == HASTE_DTYPE_BF16) {                                                        \
            if (gather) {                                                                       \
                bwdf_gather_kernel<BF16, GG><<<pgrid, dim3(256), 0, st>>>(                      \
                    w, tsrc, perm, meta, twt, (int)F, O, (int)p.ndr, (int)p.Tcap);              \
                HASTE_CHECK_LAUNCH(fn);                                                         \
            }                                                                                   \
            rc = run_main<BF16, GG>(tfeat, meta, twt, y, lddy, ws, p, B, D, F, O, st);          \
        } else {                                                                                \
            if (gather) {                                                                       \
                bwdf_gather_kernel<F16, GG><<<pgrid, dim3(256), 0, st>>>(                       \
                    w, tsrc, perm, meta, twt, (int)F, O, (int)p.ndr, (int)p.Tcap);              \
                HASTE_CHECK_LAUNCH(fn);                                                         \
            }                                                                                   \
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

extern "C" int haste_ffi_bwd_features_plan(const int32_t* idx, void* workspace,
                                           int64_t workspace_bytes, int64_t B, int64_t D,
                                           int64_t F, int64_t O, int64_t G, int32_t dtype,
                                           void* stream) {
    const char* fn = "haste_ffi_bwd_features_plan";
    haste::BwdFPlan p;
    int rc = haste::check_bwdf(fn, B, D, F, O, G, dtype, workspace, workspace_bytes, &p);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx != nullptr, "%s: null pointer", fn);
    char* base = static_cast<char*>(workspace);
    haste::bwdf_plan_kernel<<<dim3((unsigned)p.Gc), dim3(256), 0,
                              static_cast<hipStream_t>(stream)>>>(
        idx, reinterpret_cast<int*>(base + p.tfeat_off), reinterpret_cast<int*>(base + p.tsrc_off),
        reinterpret_cast<int*>(base + p.perm_off), reinterpret_cast<int*>(base + p.meta_off),
        (int)F, (int)D, (int)p.ndr, (int)p.Dc, (int)p.Tcap, haste::acc_stride((int)p.BT) * 4,
        haste::max_dc((int)p.BT));
    HASTE_CHECK_LAUNCH(fn);
    return HASTE_OK;
}

extern "C" int haste_ffi_bwd_features(const int32_t* idx, const void* W, const void* dY,
                                      int64_t lddy, float* dXT, void* workspace,
                                      int64_t workspace_bytes, int64_t B, int64_t D, int64_t F,
                                      int64_t O, int64_t G, int32_t dtype, int32_t plan_ready,
                                      void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    HASTE_CHECK_ARG(dXT != nullptr, "haste_ffi_bwd_features: null output");
    haste::BwdFPlan p;
    int rc = haste::run_partials("haste_ffi_bwd_features", idx, W, dY, lddy, workspace,
                                 workspace_bytes, B, D, F, O, G, dtype, plan_ready, st, &p);
    if (rc != HASTE_OK) return rc;
    const float* ws = reinterpret_cast<const float*>(static_cast<const char*>(workspace) + p.prep_bytes);
    const int64_t n = D * haste::ceil_div(B, 4);
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
                                         int32_t dtype, int32_t plan_ready, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    HASTE_CHECK_ARG(dX != nullptr, "haste_ffi_bwd_features_sr: null output");
    haste::BwdFPlan p;
    int rc = haste::run_partials("haste_ffi_bwd_features_sr", idx, W, dY, lddy, workspace,
                                 workspace_bytes, B, D, F, O, G, dtype, plan_ready, st, &p);
    if (rc != HASTE_OK) return rc;
    const float* ws = reinterpret_cast<const float*>(static_cast<const char*>(workspace) + p.prep_bytes);
    dim3 grid((unsigned)haste::ceil_div(D, 32), (unsigned)haste::ceil_div(B, 32));
    haste::bwdf_reduce_sr_kernel<<<grid, dim3(256), 0, st>>>(ws, dX, (int)B, (int)p.Bp, (int)D,
                                                            (int)p.S, (uint32_t)seed,
                                                            (uint32_t)(seed >> 32));
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features_sr");
    return HASTE_OK;
}
