// The main kernel of the backward to features (a workgroup per group slice x
// feature range x batch tile, partial sums in LDS) in two builds -- the LDS-ring
// build and the direct build -- and their launch templates.  Instantiated by
// ffi_bwd_features.hip for dY rows that start on 16-byte boundaries and by
// ffi_bwd_features_ya.hip (YA) for any other rows.
#pragma once

#include <type_traits>
#include <utility>

#include "bwdf_plan.hpp"

namespace haste {
namespace {

// --------------------------------------------------------------- main ------
// A workgroup owns (group slice s, feature range r, batch tile of BT = 16*WAVES
// columns) and keeps dXT[range, tile] as an fp32 partial in LDS.  The tile's
// rows are WAVES blocks of 16; a wave owns MT consecutive blocks (MT = 2 for
// the 128-column build of aligned dY rows: four waves, one per SIMD, each
// reading the ring once for two blocks), so no two waves touch the same LDS
// word of the partial.
// Per group:
//  - the group's W^T tiles for the range (and the partial-row offsets of their
//    positions) are staged once into a double-buffered LDS ring, shared by all
//    waves: each thread copies 16-byte chunks loaded two groups ahead;
//  - each wave multiplies its dY rows (MT blocks of 16 x G) with
//    the tiles (MFMA, M = batch rows, N = 16 positions, K = labels); a lane then
//    holds four consecutive batch values of one position and adds them into
//    the partial row of the position's feature with one 16-byte read and one
//    16-byte write.  A layer-1 tile (the second rows of duplicated indices)
//    shares its positions' features with the layer-0 tile it pairs with, so
//    its products are added to that tile's before the update.  Within a layer
//    the tiles' features are distinct, so all reads of the update are issued
//    before its writes; a wave's LDS accesses complete in order, so later
//    groups see the earlier writes.  Padding positions add into trash rows
//    that are never read.
//  - one barrier per group publishes the next group's ring buffer.
// Ranges holding more than RT tiles in a group process the rest in further
// rounds staged synchronously (rare: a range's share of F is usually ~F/ndr),
// layer by layer.
template <int G, int WAVES, int RT_, int MT_>
struct BwdFCfg {
    static constexpr int KS = G >= 32 ? G / 32 : 1;  // MFMA k-steps over labels
    static constexpr int BT = 16 * WAVES;            // batch columns per workgroup
    static constexpr int AS = acc_stride(BT);
    static constexpr int RT = RT_;
    static constexpr int MT = MT_;                   // 16-row M tiles per wave
    static constexpr int RB = ring_row_bytes(G);
    static constexpr int RING = RT * 16 * RB;        // bytes per ring buffer
    static constexpr int THREADS = 64 * WAVES / MT;
    static constexpr int CH = G / 8;                 // 16-byte chunks per W^T row
    static constexpr int SPT = (RT * 16 * CH + THREADS - 1) / THREADS;  // staged chunks per thread
    static constexpr int DCMAX = max_dc(BT, G, RT);
    static_assert(DCMAX > 0, "LDS budget");
};

// YA: the rows of dY need not start on 16-byte boundaries (any lddy, any
// 2-byte aligned dY).  A lane then loads each 8-label fragment as the two
// aligned 16-byte chunks that hold it and funnel-shifts them (unaligned 16-byte
// loads cost the kernel about twice its time); dY's last row, which may end at
// label O, is read by plain (unaligned) loads, its piece across O loaded early
// and shifted back.
template <typename T, int G, int WAVES, int RT_, bool YA, int MT_>
__global__ __launch_bounds__(64 * WAVES / MT_, 1) void bwdf_main_kernel(
    const int* __restrict__ tfeat, const int* __restrict__ meta, const uint16_t* __restrict__ twt,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S, int Tcap) {
    using C = BwdFCfg<G, WAVES, RT_, MT_>;
    constexpr int KS = C::KS, BT = C::BT, AS = C::AS, RT = C::RT, RB = C::RB, CH = C::CH, MT = C::MT;
    constexpr int SPT = C::SPT, NTH = C::THREADS;
    __shared__ __attribute__((aligned(16))) float acc[(C::DCMAX + kTrashRows) * AS];
    __shared__ __attribute__((aligned(16))) char ring[2][C::RING];
    __shared__ int fring[2][RT * 16];

    const int64_t work = xcd_remap(blockIdx.x, (int64_t)S * ndr * nbt);
    if (work < 0) return;
    const int bt = (int)(work % nbt);
    const int r = (int)((work / nbt) % ndr);
    const int s = (int)(work / ((int64_t)nbt * ndr));
    const int d_lo = r * Dc;
    const int dn = min(Dc, D - d_lo);
    const int64_t g_lo = (int64_t)s * gps;
    const int64_t g_hi = min<int64_t>(Gc, g_lo + gps);
    const int ng = (int)(g_hi - g_lo);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15;  // A row within the M tile / B column (tile position)
    const int kq = lane >> 4;   // which 8 of the 32 K elements
    const bool kq_ok = G >= 32 || kq < 2;
    const int kofs = kq_ok ? kq * 8 : 0;
    const int trash_f = (C::DCMAX + (col & (kTrashRows - 1))) * AS * 4;

    // dY of this lane's row (rows >= B read as zero; labels >= O are masked at
    // use).  A row is read up to the 8-label piece boundary past O (YA: 8 more
    // labels), inside the next row when lddy < ceil8(O) + 8; dY's last row is
    // read up to O only (YA), the piece that straddles O loaded early and
    // shifted back (shift_down16; O >= 16 keeps the early load inside the
    // resource).
    const int b0 = bt * BT;
    const int rows = min(BT, B - b0);
    // M tile mt of the wave covers the tile's rows 16 * (wave * MT + mt) ..
    int lrow[MT];
    bool last_row[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        lrow[mt] = (wave * MT + mt) * 16 + col;
        last_row[mt] = YA && b0 + lrow[mt] == B - 1;
    }
    // (YA: the resource starts at the 16-byte boundary at or below the tile's
    // first row, delta bytes before it)
    const uintptr_t tile = reinterpret_cast<uintptr_t>(dY + (int64_t)b0 * lddy);
    const uint32_t delta = YA ? (uint32_t)(tile & 15) : 0u;
    const rsrc_t yr = make_rsrc(reinterpret_cast<const char*>(tile - delta),
                                ((int64_t)(rows - 1) * lddy +
                                 (!YA ? (O + 7) / 8 * 8 : b0 + rows == B ? O : (O + 7) / 8 * 8 + 8)) * 2 +
                                    delta);
    // YA: bytes by which the lane's row starts past a 16-byte boundary
    uint32_t mb[MT];
    // elements the lane's piece ks of group g is loaded early by: 0 unless it
    // straddles O in dY's last row (then g is the last group)
    int sh_last[MT][KS];
    // byte offset of the lane's first label in the tile (32 bits: the tile's
    // resource spans at most kMaxRsrcBytes; g * G * 2 < 2 * lddy for real groups)
    uint32_t yoff2[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        mb[mt] = YA ? (uint32_t)((delta + (uint64_t)lrow[mt] * (uint64_t)lddy * 2) & 15) : 0u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int64_t over = (Gc - 1) * G + kofs + ks * 32 + 8 - O;
            sh_last[mt][ks] = (last_row[mt] && over > 0 && over < 8) ? (int)over : 0;
        }
        yoff2[mt] = delta + (uint32_t)(((int64_t)lrow[mt] * lddy + kofs) * 2);
    }
    auto tail_shift = [&](int64_t g, int mt, int ks) __attribute__((always_inline)) -> int {
        return g == Gc - 1 ? sh_last[mt][ks] : 0;
    };
    // a: the fragment (YA: the aligned chunk holding its start); YA b: the next chunk
    auto load_y = [&](int64_t g, u32x4 (&a)[MT][KS], u32x4 (&b)[MT][KS]) __attribute__((always_inline)) {
        const uint32_t go = (uint32_t)g * (uint32_t)(G * 2);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint32_t o = yoff2[mt] + go + ks * 64;
                if constexpr (YA) {
                    a[mt][ks] = buf_load16(yr, !kq_ok ? kOOB : last_row[mt] ? o - 2 * tail_shift(g, mt, ks) : o - mb[mt]);
                    b[mt][ks] = buf_load16(yr, !kq_ok || last_row[mt] ? kOOB : o - mb[mt] + 16);
                } else {
                    a[mt][ks] = buf_load16(yr, kq_ok ? o : kOOB);
                }
            }
        }
    };
    // The fragments of group g as the MFMA takes them: YA chunks joined; labels
    // >= O zeroed (only the last group has any: a uniform branch)
    auto prep_y = [&](int64_t g, u32x4 (&a)[MT][KS], const u32x4 (&b)[MT][KS]) __attribute__((always_inline)) {
        if constexpr (YA) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    a[mt][ks] = shift_pair16(a[mt][ks], b[mt][ks], last_row[mt] ? 0u : mb[mt]);
        }
        const int64_t rem = O - g * G;  // labels of group g below O
        if (rem >= G) return;
        const int nr = (int)max<int64_t>(rem, 0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int sh = tail_shift(g, mt, ks);
                if (sh) a[mt][ks] = shift_down16(a[mt][ks], sh);
                const int nv = nr - (ks * 32 + kofs);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    a[mt][ks][e] &= (2 * e + 1 < nv) ? 0xFFFFFFFFu : (2 * e < nv ? 0xFFFFu : 0u);
            }
        }
    };

    // Tile range of group g_lo + i in range r: tb | tm << 16, te (layer-0 tiles
    // [tb, tm), layer-1 tiles [tm, te)).  A buffer load, i.e. a vector-memory op
    // consumed DEPTH iterations later: a scalar load would hold up every later
    // LDS wait of the wave until it returns; both words are used, so no register
    // of the load is free for reuse (which would wait for it).  Groups past the
    // slice read as zero (no tiles), so iterations past them do nothing.
    const rsrc_t mr = make_rsrc(meta + (g_lo * ndr + r) * kMetaStride,
                                ((int64_t)(max(ng, 1) - 1) * ndr + 1) * kMetaStride * 4);
    auto load_meta = [&](int i) __attribute__((always_inline)) -> u32x2 {
        return buf_load8(mr, i < ng ? (uint32_t)(i * ndr * kMetaStride * 4) : kOOB);
    };
    // wave-uniform (SGPR) form
    auto uniform_meta = [](const u32x2& m) __attribute__((always_inline)) -> u32x2 {
        return u32x2{(uint32_t)__builtin_amdgcn_readfirstlane((int)m[0]),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)m[1])};
    };
    // Stage tiles [tb + t0, tb + t0 + RT) of group g_lo + i into registers: W^T
    // chunks and the positions' partial-row offsets (past the range's tiles:
    // zero W^T rows, trash offsets).  m is uniform.
    struct Stage {
        u32x4 w[SPT];
        int f;
    };
    auto load_stage = [&](int i, u32x2 m, int t0, Stage& st) __attribute__((always_inline)) {
        // wave-uniform (SGPR) values, so the buffer descriptors below are scalar
        const int tb = __builtin_amdgcn_readfirstlane((int)(m[0] & 0xFFFF) + t0);
        const int nrow = __builtin_amdgcn_readfirstlane(max(0, min(RT, (int)m[1] - tb)) * 16);
        const int64_t row0 = ((g_lo + __builtin_amdgcn_readfirstlane(i)) * Tcap + tb) * 16;
        const rsrc_t wr = make_rsrc_u32(twt + row0 * G, (uint32_t)nrow * G * 2);
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            const int c = tid + k * NTH;
            st.w[k] = buf_load16(wr, c < RT * 16 * CH ? (uint32_t)c * 16 : kOOB);
        }
        const rsrc_t fr = make_rsrc_u32(tfeat + row0, (uint32_t)nrow * 4);
        // used as loaded (rows past nrow are selected away in store_stage): an
        // operation on a pending load would wait for it here
        // only the waves holding threads tid < RT * 16 (the ones that write the
        // offsets into the ring) issue this load: a wave-uniform branch
        if (__builtin_amdgcn_readfirstlane(wave) < (RT * 16 + 63) / 64)
            st.f = (int)buf_load4(fr, tid < RT * 16 ? (uint32_t)tid * 4 : kOOB);
    };
    auto store_stage = [&](int buf, const Stage& st, u32x2 m, int t0) __attribute__((always_inline)) {
        const int tb = (int)(m[0] & 0xFFFF) + t0;
        const int nt = max(0, min(RT, (int)m[1] - tb));  // tiles of this round
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            const int c = tid + k * NTH;
            if (c < RT * 16 * CH)
                // chunk c of the stage in twt storage order
                *reinterpret_cast<u32x4*>(&ring[buf][twt_row_of(c, G) * RB + twt_chunk_of(c, G) * 16]) = st.w[k];
        }
        if (tid < RT * 16) fring[buf][tid] = tid < nt * 16 ? st.f : (C::DCMAX + (tid & (kTrashRows - 1))) * AS * 4;
    };

    // Batch columns of a partial row are permuted: the 4 columns a lane adds (its
    // wave's rows 4kq .. 4kq+3) sit at column (kq & 1) * BT/2 + 8*wave + 4*(kq >> 1),
    // so in one 16-byte RMW instruction the lanes of kq = 0 and 1 are 256 bytes
    // apart: reads (32 lanes, 512-byte bank window) and writes (16 lanes, 256
    // bytes) are conflict-free when a tile's features differ mod 16, which the
    // plan's dealing arranges.
    auto perm_col = [](int w, int q) { return (q & 1) * (BT / 2) + w * 8 + (q >> 1) * 4; };
    // (M tile mt of a wave adds the columns of the 16-row block wave * MT + mt)
    char* acc_b[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc_b[mt] = reinterpret_cast<char*>(acc) + perm_col(wave * MT + mt, kq) * 4;
    // A round is up to RT staged tiles of one group.  Its MFMAs run on all RT
    // ring tiles (rows past the round's tiles are zero) and the products stay
    // in registers; the partial update (read, add, write) of a round runs in
    // the next iteration, in the same code as the next round's MFMAs, so the
    // products' latency and the update's LDS traffic overlap the next group.
    struct Round {
        f32x4 c[MT][RT];  // dY rows of M tile mt x W^T tile t
        int f[RT];    // partial-row byte offset of the lane's position in tile t
        int n0, nt;   // uniform: layer-0 tiles and tiles of the round (nt 0: nothing to add)
    };
    auto round_counts = [](u32x2 m, int t0, Round& r) __attribute__((always_inline)) {
        const int tb = (int)(m[0] & 0xFFFF) + t0;
        r.n0 = max(0, (int)(m[0] >> 16) - tb);
        r.nt = max(0, min(RT, (int)m[1] - tb));
    };
    // ring and offset reads of the round staged in ring[buf]
    auto read_round = [&](int buf, u32x4 (&bf)[RT][KS], Round& r) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            r.f[t] = fring[buf][t * 16 + col];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                bf[t][ks] = *reinterpret_cast<const u32x4*>(&ring[buf][(t * 16 + col) * RB + ks * 64 + kq * 16]);
                if (!kq_ok) bf[t][ks] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto mma_round = [&](const u32x4 (&a)[MT][KS], const u32x4 (&bf)[RT][KS], Round& r) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(a[mt][ks], bf[t][ks], v);
                r.c[mt][t] = v;
            }
        }
    };
    // Partial update of a group's first round pr, whose first N0 tiles are
    // layer 0: layer-1 tile t of the group is the round's tile N0 + t and pairs
    // with its tile t (a round starting at the group's first tile holds
    // layer-1 tiles only when all layer-0 tiles fit), so one pass adds both.
    // Tiles past the range's are zero rows (zero products).  The MFMAs of the
    // next round (mma) are issued between the reads and the writes.
    auto update_first_n = [&](const Round& pr, auto n0, auto mma) __attribute__((always_inline)) {
        constexpr int N0 = decltype(n0)::value;
        f32x4 old[MT][N0 > 0 ? N0 : 1];
#pragma unroll
        for (int t = 0; t < N0; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) old[mt][t] = *reinterpret_cast<const f32x4*>(acc_b[mt] + pr.f[t]);
        mma();
#pragma unroll
        for (int t = 0; t < N0; ++t) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = pr.c[mt][t];
                if (N0 + t < RT) v += pr.c[mt][N0 + t];
                *reinterpret_cast<f32x4*>(acc_b[mt] + pr.f[t]) = old[mt][t] + v;
            }
        }
        // every LDS op of the wave but the MT*N0 writes has completed (a count
        // above the counter's maximum waits for a little more)
        __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(MT * N0 < 15 ? MT * N0 : 15));
    };
    auto update_first = [&](const Round& pr, auto mma) __attribute__((always_inline)) {
        static_assert(RT <= 8, "ring tiles");
        using std::integral_constant;
        switch (min(pr.n0, pr.nt)) {
        case 0: update_first_n(pr, integral_constant<int, 0>{}, mma); break;
        case 1: update_first_n(pr, integral_constant<int, 1>{}, mma); break;
        case 2: update_first_n(pr, integral_constant<int, (RT >= 2 ? 2 : 1)>{}, mma); break;
        case 3: update_first_n(pr, integral_constant<int, (RT >= 3 ? 3 : 1)>{}, mma); break;
        case 4: update_first_n(pr, integral_constant<int, (RT >= 4 ? 4 : 1)>{}, mma); break;
        case 5: update_first_n(pr, integral_constant<int, (RT >= 5 ? 5 : 1)>{}, mma); break;
        case 6: update_first_n(pr, integral_constant<int, (RT >= 6 ? 6 : 1)>{}, mma); break;
        case 7: update_first_n(pr, integral_constant<int, (RT >= 7 ? 7 : 1)>{}, mma); break;
        default: update_first_n(pr, integral_constant<int, RT>{}, mma); break;
        }
    };
    // Partial update of a further round: layer 0 (layer-1 tiles add into trash
    // rows), then layer 1 if any; a pass issues all its reads before its writes
    // (a layer's features are distinct), and a wave's LDS accesses complete in
    // order, so later passes and rounds see the writes.
    auto update_n = [&](const Round& pr, auto ntiles, auto mma) __attribute__((always_inline)) {
        constexpr int NTL = decltype(ntiles)::value;
        f32x4 old[MT][NTL > 0 ? NTL : 1];
        int fa[NTL > 0 ? NTL : 1];
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
            fa[t] = t < pr.n0 ? pr.f[t] : trash_f;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) old[mt][t] = *reinterpret_cast<const f32x4*>(acc_b[mt] + fa[t]);
        }
        mma();
#pragma unroll
        for (int t = 0; t < NTL; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                *reinterpret_cast<f32x4*>(acc_b[mt] + fa[t]) = old[mt][t] + pr.c[mt][t];
        if (pr.n0 < NTL) {
#pragma unroll
            for (int t = 0; t < NTL; ++t) {
                fa[t] = t >= pr.n0 ? pr.f[t] : trash_f;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) old[mt][t] = *reinterpret_cast<const f32x4*>(acc_b[mt] + fa[t]);
            }
#pragma unroll
            for (int t = 0; t < NTL; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    *reinterpret_cast<f32x4*>(acc_b[mt] + fa[t]) = old[mt][t] + pr.c[mt][t];
        }
        // every LDS op of the wave but the last pass's MT*NTL writes has completed
        __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(MT * NTL < 15 ? MT * NTL : 15));
    };
    // update of a further round pr, specialised for its tile count (a uniform switch)
    auto update = [&](const Round& pr, auto mma) __attribute__((always_inline)) {
        static_assert(RT <= 8, "ring tiles");
        using std::integral_constant;
        switch (pr.nt) {
        case 0: update_n(pr, integral_constant<int, 0>{}, mma); break;
        case 1: update_n(pr, integral_constant<int, 1>{}, mma); break;
        case 2: update_n(pr, integral_constant<int, (RT >= 2 ? 2 : 1)>{}, mma); break;
        case 3: update_n(pr, integral_constant<int, (RT >= 3 ? 3 : 1)>{}, mma); break;
        case 4: update_n(pr, integral_constant<int, (RT >= 4 ? 4 : 1)>{}, mma); break;
        case 5: update_n(pr, integral_constant<int, (RT >= 5 ? 5 : 1)>{}, mma); break;
        case 6: update_n(pr, integral_constant<int, (RT >= 6 ? 6 : 1)>{}, mma); break;
        case 7: update_n(pr, integral_constant<int, (RT >= 7 ? 7 : 1)>{}, mma); break;
        default: update_n(pr, integral_constant<int, RT>{}, mma); break;
        }
    };
    auto no_mma = []() __attribute__((always_inline)) {};
    // Further rounds of a group whose range holds more than RT tiles, done
    // synchronously after the group's first round: staged into ring[buf] (not
    // in use by any wave at this point), multiplied and added at once.
    auto extra_rounds = [&](int i, u32x2 m, int buf, const u32x4 (&a)[MT][KS]) __attribute__((always_inline)) {
        const int ntot = (int)m[1] - (int)(m[0] & 0xFFFF);
        for (int t0 = RT; t0 < ntot; t0 += RT) {
            Stage st;
            load_stage(i, m, t0, st);
            store_stage(buf, st, m, t0);
            __syncthreads();
            Round r;
            u32x4 bf[RT][KS];
            read_round(buf, bf, r);
            mma_round(a, bf, r);
            round_counts(m, t0, r);
            update(r, no_mma);
            __syncthreads();
        }
    };

    // ---- pipeline: ring[i % 2] holds group i.  Every global load is issued
    // DEPTH iterations before its use, in the same order every iteration (W^T
    // stage of group i+1+DEPTH, dY of group i+DEPTH, meta of group i+1+2*DEPTH),
    // so the one wait of an iteration (on the meta it converts) covers exactly
    // the loads of iteration i-DEPTH.  Register sets rotate over NS slots
    // (group h in slot h % NS), resolved at compile time by unrolling
    // kGroupUnroll iterations (a multiple of NS and of the 2 ring buffers);
    // the loop runs whole unrolled iterations without guards.  Iteration i
    // stages group i+1 into ring[1 - i % 2] (read by every wave before the
    // last barrier), reads and multiplies group i's first round and adds
    // group i-1's products into the partial. ----
    // G = 128 groups take about twice as long per iteration, so two groups of
    // look-ahead cover the load latency; the shallower pipeline leaves room in
    // the register budget for the larger dY fragments and ring rounds.
    constexpr int DEPTH = G >= 128 ? 2 : 5, NS = DEPTH + 1;
    static_assert(kGroupUnroll % NS == 0 && kGroupUnroll % 2 == 0, "unroll");
    Stage stg[NS];
    u32x4 ya[NS][MT][KS];
    u32x4 yb[YA ? NS : 1][MT][KS];  // YA: the second chunk of each fragment
    u32x2 mraw[NS];
    u32x2 mu[DEPTH + 1];  // uniform meta of groups i .. i+DEPTH
    Round rd[2];          // round of group i in rd[i % 2]
    rd[0].nt = rd[1].nt = 0;
    rd[0].n0 = rd[1].n0 = 0;
    {
        u32x2 m0[DEPTH + 1];
#pragma unroll
        for (int k = 0; k <= DEPTH; ++k) m0[k] = load_meta(k);
        // the partial is cleared while the first tile ranges load
        for (int i = tid * 4; i < dn * AS; i += NTH * 4)
            *reinterpret_cast<f32x4*>(&acc[i]) = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k <= DEPTH; ++k) mu[k] = uniform_meta(m0[k]);
        load_stage(0, mu[0], 0, stg[0]);
        store_stage(0, stg[0], mu[0], 0);
        // iterations -DEPTH .. -1 of the steady-state load sequence, kept in
        // that order (the loop's wait counts assume it)
#pragma unroll
        for (int k = 1; k <= DEPTH; ++k) {
            __builtin_amdgcn_sched_barrier(0);
            load_stage(k, mu[k], 0, stg[k % NS]);
            load_y(g_lo + k - 1, ya[(k - 1) % NS], yb[YA ? (k - 1) % NS : 0]);
            mraw[(k + DEPTH) % NS] = load_meta(k + DEPTH);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    auto body = [&](int i, auto kc) __attribute__((always_inline)) {
        constexpr int K = decltype(kc)::value;  // i % kGroupUnroll
        constexpr int Q = K % NS;               // i % NS
        constexpr int P = K % 2;                // ring buffer of group i
        const u32x2 mn = uniform_meta(mraw[(Q + 1 + DEPTH) % NS]);
        load_stage(i + 1 + DEPTH, mn, 0, stg[(Q + 1 + DEPTH) % NS]);
        load_y(g_lo + i + DEPTH, ya[(Q + DEPTH) % NS], yb[YA ? (Q + DEPTH) % NS : 0]);
        mraw[(Q + 1 + 2 * DEPTH) % NS] = load_meta(i + 1 + 2 * DEPTH);
        store_stage(1 - P, stg[(Q + 1) % NS], mu[1], 0);
        prep_y(g_lo + i, ya[Q], yb[YA ? Q : 0]);
        u32x4 bf[RT][KS];
        read_round(P, bf, rd[P]);
        asm volatile("" ::: "memory");  // the update's LDS ops stay after the stage and reads
        update_first(rd[1 - P], [&]() __attribute__((always_inline)) { mma_round(ya[Q], bf, rd[P]); });
        round_counts(mu[0], 0, rd[P]);
        if ((int)mu[0][1] - (int)(mu[0][0] & 0xFFFF) > RT) {  // uniform, rare
            // add this round now, then the group's further rounds in order
            update_first(rd[P], no_mma);
            rd[P].nt = 0;
            __syncthreads();
            extra_rounds(i, mu[0], P, ya[Q]);
            // the rounds consumed their loads (only some threads use a stage's
            // position offsets); say so, so later code need not wait for them
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        }
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) mu[k] = mu[k + 1];
        mu[DEPTH] = mn;
        // Barrier without draining the wave's LDS queue: other waves next write
        // ring[P] and read ring[1 - P], and this wave's reads of ring[P] and
        // fring[P] and writes of ring[1 - P] have completed (the update's wait);
        // only its last partial writes may still be in flight, and no other
        // wave touches those words.
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    for (int i = 0; i < ng; i += kGroupUnroll) {
        body(i, std::integral_constant<int, 0>{});
        body(i + 1, std::integral_constant<int, 1>{});
        body(i + 2, std::integral_constant<int, 2>{});
        body(i + 3, std::integral_constant<int, 3>{});
        body(i + 4, std::integral_constant<int, 4>{});
        body(i + 5, std::integral_constant<int, 5>{});
    }
    static_assert(kGroupUnroll % 2 == 0, "the last iteration's round is in rd[1]");
    update_first(rd[1], no_mma);
    __syncthreads();

    // ---- write the partial: ws[s][d_lo + d][bt*BT + b] ----
    float* out = ws + ((int64_t)s * D + d_lo) * Bp + (int64_t)bt * BT;
    for (int i = tid; i < dn * (BT / 4); i += NTH) {
        const int d = i / (BT / 4), q = i % (BT / 4);  // natural columns 4q .. 4q+3
        *reinterpret_cast<f32x4*>(out + (int64_t)d * Bp + q * 4) =
            *reinterpret_cast<const f32x4*>(&acc[d * AS + perm_col(q / 4, q % 4)]);
    }
}

// f(integral_constant<int, K>) for K = 0, 1, ..., in order
template <int... K, typename F>
__device__ __forceinline__ void unroll_seq(std::integer_sequence<int, K...>, F&& f) {
    (f(std::integral_constant<int, K>{}), ...);
}

// Direct build: no LDS ring and no barrier per group.  Each wave loads the
// MFMA operand fragments of a group's W^T tiles straight from the workspace
// (one contiguous 1 KB block per tile and k-step in the chunk-major twt
// layout), the positions' partial-row offsets and its dY fragments, two or
// five groups ahead, and adds its products into its own columns of the partial
// (the same update as the ring build: a round of up to RT tiles, layer-1 tiles
// added with their layer-0 pairs, further rounds of large ranges done at
// once).  The waves share nothing until the partial is written out.  Every
// wave reads the tiles itself: four times the ring's W^T reads, from L2.  YA:
// dY rows off 16-byte boundaries; a lane loads the aligned chunk holding its
// fragment's start and takes the next one from a neighbouring lane.
template <typename T, int G, int WAVES, int RT_, int MT_, bool YA>
__global__ __launch_bounds__(64 * WAVES / MT_, 1) void bwdf_direct_kernel(
    const int* __restrict__ tfeat, const int* __restrict__ meta, const uint16_t* __restrict__ twt,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S, int Tcap) {
    using C = BwdFCfg<G, WAVES, RT_, MT_>;
    constexpr int KS = C::KS, BT = C::BT, AS = C::AS, RT = C::RT, MT = C::MT, NTH = C::THREADS;
    static_assert(G >= 32, "direct build: one 32-label k-step per fragment");
    __shared__ __attribute__((aligned(16))) float acc[(C::DCMAX + kTrashRows) * AS];

    const int64_t work = xcd_remap(blockIdx.x, (int64_t)S * ndr * nbt);
    if (work < 0) return;
    const int bt = (int)(work % nbt);
    const int r = (int)((work / nbt) % ndr);
    const int s = (int)(work / ((int64_t)nbt * ndr));
    const int d_lo = r * Dc;
    const int dn = min(Dc, D - d_lo);
    const int64_t g_lo = (int64_t)s * gps;
    const int64_t g_hi = min<int64_t>(Gc, g_lo + gps);
    const int ng = (int)(g_hi - g_lo);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15;  // A row within the M tile / B column (tile position)
    const int kq = lane >> 4;   // which 8 of the 32 K elements
    const int trash_f = (C::DCMAX + (col & (kTrashRows - 1))) * AS * 4;

    // dY fragments: row b0 + lrow[mt], labels g*G + 32*ks + 8*kq .. +7 (rows >=
    // B read as zero, labels >= O masked at use).  A row is read up to the
    // 8-label piece boundary past O (YA: 8 more labels), inside the next row when
    // lddy < ceil8(O) + 8; dY's last row is read up to O only (YA), the piece
    // that straddles O loaded early and shifted back.
    const int b0 = bt * BT;
    const int rows = min(BT, B - b0);
    int lrow[MT];
    bool last_row[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        lrow[mt] = (wave * MT + mt) * 16 + col;
        last_row[mt] = YA && b0 + lrow[mt] == B - 1;
    }
    // (YA: the resource starts at the 16-byte boundary at or below the tile's
    // first row, delta bytes before it)
    const uintptr_t ytile = reinterpret_cast<uintptr_t>(dY + (int64_t)b0 * lddy);
    const uint32_t delta = YA ? (uint32_t)(ytile & 15) : 0u;
    const rsrc_t yr = make_rsrc(reinterpret_cast<const char*>(ytile - delta),
                                ((int64_t)(rows - 1) * lddy +
                                 (!YA ? (O + 7) / 8 * 8 : b0 + rows == B ? O : (O + 7) / 8 * 8 + 8)) * 2 +
                                    delta);
    uint32_t mb[MT];  // YA: bytes by which the lane's row starts past a 16-byte boundary
    int sh_last[MT][KS];
    uint32_t yoff2[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        mb[mt] = YA ? (uint32_t)((delta + (uint64_t)lrow[mt] * (uint64_t)lddy * 2) & 15) : 0u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int64_t over = (Gc - 1) * G + kq * 8 + ks * 32 + 8 - O;
            sh_last[mt][ks] = (last_row[mt] && over > 0 && over < 8) ? (int)over : 0;
        }
        yoff2[mt] = delta + (uint32_t)(((int64_t)lrow[mt] * lddy + kq * 8) * 2);
    }
    auto tail_shift = [&](int64_t g, int mt, int ks) __attribute__((always_inline)) -> int {
        return g == Gc - 1 ? sh_last[mt][ks] : 0;
    };
    // a: the fragment (YA: the aligned chunk holding its start).  YA: the chunk
    // after it is the aligned chunk that lane + 16 (the same row's next 8
    // labels) loaded -- for the lanes of k-chunk 3 that of lane - 48 at the next
    // k-step -- so it is taken across lanes (ds_bpermute) instead of loaded
    // again; only k-chunk 3's last k-step loads its next chunk itself (e, one
    // per M tile; the other lanes' e loads are out of range).
    auto load_y = [&](int64_t g, u32x4 (&a)[MT][KS], u32x4 (&e)[MT][1]) __attribute__((always_inline)) {
        const uint32_t go = (uint32_t)g * (uint32_t)(G * 2);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint32_t o = yoff2[mt] + go + ks * 64;
                if constexpr (YA)
                    a[mt][ks] = buf_load16(yr, last_row[mt] ? o - 2 * tail_shift(g, mt, ks) : o - mb[mt]);
                else
                    a[mt][ks] = buf_load16(yr, o);
            }
            if constexpr (YA) {
                const uint32_t o = yoff2[mt] + go + (KS - 1) * 64;
                e[mt][0] = buf_load16(yr, kq == 3 && !last_row[mt] ? o - mb[mt] + 16 : kOOB);
            }
        }
    };
    const int nb_addr = ((lane + 16) & 63) * 4;  // ds_bpermute source: lane + 16
    auto next_chunk = [&](const u32x4& v) __attribute__((always_inline)) -> u32x4 {
        u32x4 r;
#pragma unroll
        for (int q = 0; q < 4; ++q) r[q] = (uint32_t)__builtin_amdgcn_ds_bpermute(nb_addr, (int)v[q]);
        return r;
    };
    // the fragments as the MFMA takes them: YA chunks joined; labels >= O zeroed
    // (only the last group has any: a uniform branch)
    // the slice's group holding labels past O (its last, in the last slice), and
    // the labels it has
    const int i_tail = (g_hi == Gc && O % G != 0) ? ng - 1 : -1;
    const int nr_tail = (int)(O - (Gc - 1) * G);
    auto prep_y = [&](int i, u32x4 (&a)[MT][KS], const u32x4 (&e)[MT][1]) __attribute__((always_inline)) {
        const int64_t g = g_lo + i;
        if constexpr (YA) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                u32x4 nxt[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    // what this lane offers to lane - 16: its own chunk, or for
                    // k-chunk 0 (read by k-chunk 3 of the previous k-step) the
                    // next k-step's chunk
                    const u32x4 offer = (kq == 0 && ks + 1 < KS) ? a[mt][ks + 1] : a[mt][ks];
                    nxt[ks] = next_chunk(offer);
                    if (ks == KS - 1 && kq == 3) nxt[ks] = e[mt][0];
                }
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    a[mt][ks] = shift_pair16(a[mt][ks], nxt[ks], last_row[mt] ? 0u : mb[mt]);
            }
        }
        if (__builtin_expect(i != i_tail, 1)) return;
        const int nr = nr_tail;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int sh = tail_shift(g, mt, ks);
                if (sh) a[mt][ks] = shift_down16(a[mt][ks], sh);
                const int nv = nr - (ks * 32 + kq * 8);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    a[mt][ks][e] &= (2 * e + 1 < nv) ? 0xFFFFFFFFu : (2 * e < nv ? 0xFFFFu : 0u);
            }
        }
    };
    // tile range of group g_lo + i in range r (tb | tm << 16, te), as a buffer
    // load (a scalar load would hold up the wave's LDS waits); past the slice: zero
    const rsrc_t mr = make_rsrc(meta + (g_lo * ndr + r) * kMetaStride,
                                ng > 0 ? ((int64_t)(ng - 1) * ndr + 1) * kMetaStride * 4 : 0);
    auto load_meta = [&](int i) __attribute__((always_inline)) -> u32x2 {
        return buf_load8(mr, (uint32_t)(i * ndr * kMetaStride * 4));  // i >= ng: past the end
    };
    auto uniform_meta = [](const u32x2& m) __attribute__((always_inline)) -> u32x2 {
        return u32x2{(uint32_t)__builtin_amdgcn_readfirstlane((int)m[0]),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)m[1])};
    };
    // A round: the lane's operand fragments of tiles [tb + t0, tb + t0 + RT) of
    // group g_lo + i (tiles past the range's read as zero) and the partial-row
    // byte offsets of its position in each
    struct Frag {
        u32x4 b[RT][KS];
        int f[RT];
    };
    auto load_frag = [&](int i, u32x2 m, int t0, Frag& fr) __attribute__((always_inline)) {
        const int tb = __builtin_amdgcn_readfirstlane((int)(m[0] & 0xFFFF) + t0);
        const int nt = __builtin_amdgcn_readfirstlane(max(0, min(RT, (int)m[1] - tb)));
        const int64_t row0 = ((g_lo + __builtin_amdgcn_readfirstlane(i)) * Tcap + tb) * 16;
        const rsrc_t wr = make_rsrc_u32(twt + row0 * G, (uint32_t)nt * 16 * G * 2);
        const rsrc_t frr = make_rsrc_u32(tfeat + row0, (uint32_t)nt * 16 * 4);
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                fr.b[t][ks] = buf_load16(wr, (uint32_t)(t * 16 * G + (ks * 64 + lane) * 8) * 2);
#pragma unroll
        for (int t = 0; t < RT; ++t) fr.f[t] = (int)buf_load4(frr, (uint32_t)(t * 16 + col) * 4);
    };

    // The same for the first round of a group, through resources over the
    // slice's tiles: group i's tiles start at row (i*Tcap + tb)*16 of the
    // slice (the host keeps the slice's bytes under kMaxRsrcBytes); tiles past
    // the range read the next range's rows, which the round does not use, and
    // groups past the slice read zero.
    const int64_t srow0 = g_lo * Tcap * 16;
    const rsrc_t wsl = make_rsrc(twt + srow0 * G, (int64_t)ng * Tcap * 16 * G * 2);
    const rsrc_t fsl = make_rsrc(tfeat + srow0, (int64_t)ng * Tcap * 16 * 4);
    auto load_frag_first = [&](int i, u32x2 m, Frag& fr) __attribute__((always_inline)) {
        const uint32_t row = ((uint32_t)i * (uint32_t)Tcap + (m[0] & 0xFFFFu)) * 16u;
        const uint32_t wo = row * (2u * G) + (uint32_t)lane * 16u;
        const uint32_t fo = row * 4u + (uint32_t)col * 4u;
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                fr.b[t][ks] = buf_load16(wsl, wo + (uint32_t)(t * 16 * G + ks * 512) * 2u);
#pragma unroll
        for (int t = 0; t < RT; ++t) fr.f[t] = (int)buf_load4(fsl, fo + (uint32_t)t * 64u);
    };

    auto perm_col = [](int w, int q) { return (q & 1) * (BT / 2) + w * 8 + (q >> 1) * 4; };
    char* acc_b[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc_b[mt] = reinterpret_cast<char*>(acc) + perm_col(wave * MT + mt, kq) * 4;
    struct Res {
        f32x4 c[MT][RT];
    };
    auto mma_round = [&](const u32x4 (&a)[MT][KS], const Frag& fr, Res& rs) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(a[mt][ks], fr.b[t][ks], v);
                rs.c[mt][t] = v;
            }
        }
    };
    // First round of a group with N0 layer-0 and N1 layer-1 tiles (N1 <= N0,
    // N0 + N1 <= RT): layer-1 tile t is the round's tile N0 + t and adds into
    // its pair's rows; the round's other fragments are not used.  The partial
    // rows are read, the MFMAs issued, then the rows written.
    auto first_n = [&](const u32x4 (&a)[MT][KS], const Frag& fr, auto n0, auto n1) __attribute__((always_inline)) {
        constexpr int N0 = decltype(n0)::value, N1 = decltype(n1)::value;
        if constexpr (N0 + N1 <= RT) {
            f32x4 old[MT][N0];
#pragma unroll
            for (int t = 0; t < N0; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) old[mt][t] = *reinterpret_cast<const f32x4*>(acc_b[mt] + fr.f[t]);
            f32x4 c[MT][N0 + N1];
#pragma unroll
            for (int t = 0; t < N0 + N1; ++t) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(a[mt][ks], fr.b[t][ks], v);
                    c[mt][t] = v;
                }
            }
#pragma unroll
            for (int t = 0; t < N0; ++t) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    f32x4 v = c[mt][t];
                    if (t < N1) v += c[mt][N0 + t];
                    *reinterpret_cast<f32x4*>(acc_b[mt] + fr.f[t]) = old[mt][t] + v;
                }
            }
        }
    };
    auto first = [&](const u32x4 (&a)[MT][KS], const Frag& fr, int n0, int n1) __attribute__((always_inline)) {
        static_assert(RT <= 6, "direct build: rounds of at most 6 tiles");
        using std::integral_constant;
#define HASTE_ROUND(A, B)                                                          \
    case (A) * 8 + (B):                                                             \
        first_n(a, fr, integral_constant<int, (A)>{}, integral_constant<int, (B)>{}); \
        break;
        switch (n0 * 8 + n1) {
            HASTE_ROUND(1, 0) HASTE_ROUND(1, 1)
            HASTE_ROUND(2, 0) HASTE_ROUND(2, 1) HASTE_ROUND(2, 2)
            HASTE_ROUND(3, 0) HASTE_ROUND(3, 1) HASTE_ROUND(3, 2) HASTE_ROUND(3, 3)
            HASTE_ROUND(4, 0) HASTE_ROUND(4, 1) HASTE_ROUND(4, 2)
            HASTE_ROUND(5, 0) HASTE_ROUND(5, 1)
            HASTE_ROUND(6, 0)
        default: break;  // no layer-0 tile in the range
        }
#undef HASTE_ROUND
    };
    // Further rounds of a range holding more than RT tiles (rare): loaded and
    // added at once, layer 0 first (layer-1 tiles into trash rows), then layer 1.
    auto extra_rounds = [&](int i, u32x2 m, const u32x4 (&a)[MT][KS]) __attribute__((always_inline)) {
        const int tb = (int)(m[0] & 0xFFFF), tm = (int)(m[0] >> 16), te = (int)m[1];
        for (int t0 = RT; t0 < te - tb; t0 += RT) {
            Frag fr;
            load_frag(i, m, t0, fr);
            Res rs;
            mma_round(a, fr, rs);
            const int n0 = max(0, tm - (tb + t0));
            const int nt = min(RT, te - (tb + t0));
#pragma unroll
            for (int pass = 0; pass < 2; ++pass) {
                if (pass == 1 && n0 >= nt) break;
                f32x4 old[MT][RT];
                int fa[RT];
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    const bool mine = t < nt && (pass == 0 ? t < n0 : t >= n0);
                    fa[t] = mine ? fr.f[t] : trash_f;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) old[mt][t] = *reinterpret_cast<const f32x4*>(acc_b[mt] + fa[t]);
                }
#pragma unroll
                for (int t = 0; t < RT; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        *reinterpret_cast<f32x4*>(acc_b[mt] + fa[t]) = old[mt][t] + rs.c[mt][t];
            }
        }
    };

    // ---- pipeline: slot i % NS holds group i's fragments.  Iteration i
    // converts the meta of group i+DEPTH (loaded DEPTH iterations earlier, after
    // that iteration's fragment loads, so its wait covers the fragments of group
    // i), issues the loads of group i+DEPTH and the meta of group i+2*DEPTH, and
    // processes group i.  kGroupUnroll iterations are unrolled so that every
    // slot index is a constant; the loop runs whole unrolled iterations.  Five
    // groups of look-ahead where a slot is small (rounds of at most 4
    // fragments: short groups need the deeper pipeline), else two. ----
    constexpr int DEPTH = RT * KS <= 4 ? 5 : 2, NS = DEPTH + 1;
    // groups per unrolled iteration, a multiple of NS (groups past the slice
    // read zero metas and do nothing)
    constexpr int U = kGroupUnroll % NS == 0 ? kGroupUnroll : NS;
    Frag fq[NS];
    u32x4 ya[NS][MT][KS];
    u32x4 yb[YA ? NS : 1][MT][1];  // YA: k-chunk 3's chunk past the group
    u32x2 mraw[NS];
    u32x2 mq[DEPTH];  // uniform meta of groups i .. i+DEPTH-1
    {
        u32x2 m0[DEPTH];
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) m0[k] = load_meta(k);
        for (int i = tid * 4; i < dn * AS; i += NTH * 4)
            *reinterpret_cast<f32x4*>(&acc[i]) = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) mq[k] = uniform_meta(m0[k]);
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) {
            __builtin_amdgcn_sched_barrier(0);
            load_frag_first(k, mq[k], fq[k % NS]);
            load_y(g_lo + k, ya[k % NS], yb[YA ? k % NS : 0]);
            mraw[(k + DEPTH) % NS] = load_meta(k + DEPTH);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // the partial is clear
    auto body = [&](int i, auto kc) __attribute__((always_inline)) {
        constexpr int K = decltype(kc)::value;  // i % U
        constexpr int Q = K % NS;
        const u32x2 mn = uniform_meta(mraw[(Q + DEPTH) % NS]);  // group i + DEPTH
        load_frag_first(i + DEPTH, mn, fq[(Q + DEPTH) % NS]);
        load_y(g_lo + i + DEPTH, ya[(Q + DEPTH) % NS], yb[YA ? (Q + DEPTH) % NS : 0]);
        mraw[(Q + 2 * DEPTH) % NS] = load_meta(i + 2 * DEPTH);
        prep_y(i, ya[Q], yb[YA ? Q : 0]);
        const u32x2 m = mq[0];
        const int tb = (int)(m[0] & 0xFFFF), tm = (int)(m[0] >> 16), te = (int)m[1];
        const int n0 = min(tm - tb, RT);
        first(ya[Q], fq[Q], n0, min(te - tb, RT) - n0);
        if (te - tb > RT) extra_rounds(i, m, ya[Q]);  // uniform, rare
#pragma unroll
        for (int k = 0; k + 1 < DEPTH; ++k) mq[k] = mq[k + 1];
        mq[DEPTH - 1] = mn;
    };
    for (int i = 0; i < ng; i += U)
        unroll_seq(std::make_integer_sequence<int, U>{},
                   [&](auto kc) __attribute__((always_inline)) { body(i + decltype(kc)::value, kc); });
    __syncthreads();

    // ---- write the partial: ws[s][d_lo + d][bt*BT + b] ----
    float* out = ws + ((int64_t)s * D + d_lo) * Bp + (int64_t)bt * BT;
    for (int i = tid; i < dn * (BT / 4); i += NTH) {
        const int d = i / (BT / 4), q = i % (BT / 4);  // natural columns 4q .. 4q+3
        *reinterpret_cast<f32x4*>(out + (int64_t)d * Bp + q * 4) =
            *reinterpret_cast<const f32x4*>(&acc[d * AS + perm_col(q / 4, q % 4)]);
    }
}

template <typename T, int G, int WAVES, int RT, bool YA, int MT, bool DIRECT = false>
int launch_main(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
                hipStream_t st) {
    const int64_t nlog = p.S * p.ndr * p.nbt;
    const int64_t grid = 8 * ceil_div(nlog, 8);
    if (((int64_t)p.BT * lddy + 8) * 2 > kMaxRsrcBytes) {
        set_error("haste_ffi_bwd_features: lddy = %lld too large", (long long)lddy);
        return HASTE_ERR_UNSUPPORTED;
    }
    if constexpr (DIRECT)
        bwdf_direct_kernel<T, G, WAVES, RT, MT, YA><<<dim3((unsigned)grid), dim3(64 * WAVES / MT), 0, st>>>(
            tfeat, meta, twt, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, O, p.Gc, (int)p.nbt,
            (int)p.ndr, (int)p.Dc, (int)p.gps, (int)p.S, (int)p.Tcap);
    else
        bwdf_main_kernel<T, G, WAVES, RT, YA, MT><<<dim3((unsigned)grid), dim3(64 * WAVES / MT), 0, st>>>(
            tfeat, meta, twt, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, O, p.Gc, (int)p.nbt,
            (int)p.ndr, (int)p.Dc, (int)p.gps, (int)p.S, (int)p.Tcap);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

// the plan's ring size: 2, 3 or ring_tiles(G) tiles
template <typename T, int G, int WAVES, bool YA, int MT, bool DIRECT = false>
int launch_ring(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
                hipStream_t st) {
    constexpr int R = ring_tiles(G);
    if (p.RT == 2) return launch_main<T, G, WAVES, 2, YA, MT, DIRECT>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
    if constexpr (R > 3) {
        if (p.RT == 3) return launch_main<T, G, WAVES, 3, YA, MT, DIRECT>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
    }
    return launch_main<T, G, WAVES, R, YA, MT, DIRECT>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
}

// 16-row M tiles per wave of the 128-column build: two for 16-byte aligned dY
// rows; one for YA, whose second chunk per fragment would double the dY
// registers (measured: 138 us with one, 169 us with two, config 1)
template <bool YA>
constexpr int bwdf_mt() { return YA ? 1 : 2; }
template <typename T, int G, bool YA>
int run_main(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
             int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F,
             int64_t O, hipStream_t st) {
    (void)F;
    // The direct build where dY fits in the last-level cache (measured: config
    // 1, 104 -> 101 us, YA rows 137 -> 122 us; config 3, 802 -> 611 us).  With a
    // dY of 686 MB (config 2) it was slower than the ring build (305 -> 361 us),
    // which keeps the waves of a workgroup in step on each group's dY and W^T.
    // It addresses a slice's W^T tiles with 32-bit offsets.
    if constexpr (G == 32 || G == 64) {
        const int build = bwdf_build();
        const bool fits = (p.gps + 16) * p.Tcap * 16 * G * 2 <= kMaxRsrcBytes;
        if (fits && (build == 2 || (build == 0 && B * lddy * 2 <= kMallBytes))) {
            if (p.BT == 64) return launch_ring<T, G, 4, YA, 1, true>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
            return launch_ring<T, G, 8, YA, 2, true>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
        }
    }
    if (p.BT == 64) return launch_ring<T, G, 4, YA, 1>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
    return launch_ring<T, G, 8, YA, bwdf_mt<YA>()>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
}

}  // namespace

// run_main for dY rows that do not all start on 16-byte boundaries (defined in
// ffi_bwd_features_ya.hip).
int bwdf_run_main_ya(int32_t dtype, int64_t G, const int* tfeat, const int* meta,
                     const uint16_t* twt, const uint16_t* dY, int64_t lddy, float* ws,
                     const BwdFPlan& p, int64_t B, int64_t D, int64_t F, int64_t O,
                     hipStream_t st);

}  // namespace haste
