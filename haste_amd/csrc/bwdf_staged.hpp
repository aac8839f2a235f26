// The staged main kernel of the backward to features: a workgroup per (group
// slice, feature range, batch tile of BT columns) keeps dX^T[range, tile] as an
// fp32 partial in LDS, as the ring and direct builds do, but moves its
// operands differently.  On gfx950 a 16-byte load in MFMA operand order (the
// 16 lanes of a fragment reading 16 different rows) runs at about a third of
// the rate of a row-major load (about 16 against 40-50 bytes per clock per
// CU), and an out-of-range buffer load costs as much as a real one.  So:
//  - each group's dY tile [BT rows x G labels] is loaded once per workgroup,
//    row-major (every thread one piece of PB bytes), and staged in LDS
//    (a ring of six buffers, filled a plan window ahead; 16-byte chunks XOR-swizzled
//    per row so that the operand reads of 16 rows hit distinct bank groups);
//  - wave w owns W^T tile w of the range (16 positions): it loads that tile's
//    operand fragments (chunk-major twt: one contiguous 1 KB per k-step) and
//    the positions' partial-row offsets, reads the staged dY operands of all
//    BT rows and multiplies (MFMA, M = batch rows, N = positions, K =
//    labels); one group later its lanes add the products into the partial
//    rows of the tile's features (one 16-byte read-modify-write per 16-row
//    block).  Within a layer a group's features are distinct, so the waves of
//    one group never touch the same partial word;
//  - a barrier, after each wave's LDS operations have completed, orders the
//    groups' partial updates and publishes the staged tiles.  The plan lays
//    out windows of kPlanWindow consecutive groups with every feature they
//    share in the tile of the same index -- one wave -- so the window's
//    updates need no barrier between them: one barrier per window.
// A duplicated index's second ("lo") row sits in the same tile as its "hi"
// row (the plan's in-tile mode: no layer-1 tiles, so no wave carries a second
// tile in the pipeline), its partial-row offset marked by bit 0: the wave adds
// the tile's products in two passes, the hi and single rows first, then the lo
// rows, each pass sending the other lanes to a trash row.  A group whose range
// holds more than eight tiles takes the rest in a pass of its own between two
// more barriers, each wave adding tiles whose features no other wave touches
// in that pass.
// YA: dY rows at any 2-byte alignment; pieces are loaded from unaligned
// addresses, and the piece of dY's last row that straddles label O (the end of
// the tensor) is loaded early and shifted back.
#pragma once

#include <type_traits>

#include "bwdf_plan.hpp"

namespace haste {
namespace {

template <int G, int BT, int W>
struct StagedCfg {
    static constexpr int WAVES = W;
    static constexpr int TPW = kStagedTiles / W;  // pipeline tiles per wave
    static constexpr int NTH = 64 * WAVES;
    static constexpr int KS = G / 32;        // MFMA k-steps over the group's labels
    static constexpr int MT = BT / 16;       // 16-row blocks of the batch tile
    static constexpr int RB = 2 * G;         // bytes of a staged dY row
    static constexpr int STG = BT * RB;      // bytes of a staging buffer
    static constexpr int PB = STG / NTH;     // dY bytes each thread loads per group
    static constexpr int PW = PB / 4;        // 32-bit words of a piece
    static constexpr int AS = acc_stride(BT);
    static constexpr int DCMAX = staged_max_dc(BT, G);
    // groups of load look-ahead; G = 128 fragments are four times larger
    static constexpr int DEPTH = G >= 128 ? 2 : 5;
    static constexpr int NS = DEPTH + 1;     // register slots of the pipeline
    static_assert(G >= 32, "staged build: G >= 32");
    static_assert(TPW * W == kStagedTiles, "tiles per wave");
    static_assert(PB == 4 || PB == 8 || PB == 16 || PB == 32, "dY piece");
    static_assert(kGroupUnroll % NS == 0 && kGroupUnroll % 2 == 0 && kGroupUnroll % kStageBufs == 0, "unroll");
    static_assert(DCMAX > 0, "LDS budget");
};

// Byte offset of 16-byte chunk c of staged row r.  A 256-byte bank window
// holds 128 / G rows; chunk c of row r is stored at chunk c ^ (window index),
// so the chunk c of 16 consecutive rows (what the 16 lanes of an operand
// fragment read) lies in 16 distinct 16-byte bank groups.
template <int G>
__device__ __forceinline__ int stg_off(int r, int c) {
    constexpr int RPW = 128 / G;
    return r * (2 * G) + 16 * (c ^ ((r / RPW) & (G / 8 - 1)));
}

template <int PW>
struct PieceT;
template <>
struct PieceT<1> { using type = uint32_t; };
template <>
struct PieceT<2> { using type = u32x2; };
template <>
struct PieceT<4> { using type = u32x4; };
struct Piece32 { u32x4 a, b; };
template <>
struct PieceT<8> { using type = Piece32; };

template <int PW>
__device__ __forceinline__ typename PieceT<PW>::type load_piece(rsrc_t r, uint32_t off) {
    if constexpr (PW == 1) return buf_load4(r, off);
    else if constexpr (PW == 2) return buf_load8(r, off);
    else if constexpr (PW == 4) return buf_load16(r, off);
    else return Piece32{buf_load16(r, off), buf_load16(r, off + 16)};
}
template <int PW>
__device__ __forceinline__ void unpack_piece(const typename PieceT<PW>::type& v, uint32_t (&w)[PW]) {
    if constexpr (PW == 1) {
        w[0] = v;
    } else if constexpr (PW == 8) {
#pragma unroll
        for (int k = 0; k < 4; ++k) { w[k] = v.a[k]; w[4 + k] = v.b[k]; }
    } else {
#pragma unroll
        for (int k = 0; k < PW; ++k) w[k] = v[k];
    }
}

// Elements sh .. 2*PW-1 of the piece (16-bit) move to 0 .. 2*PW-1-sh; the top
// sh elements become zero.  sh in [0, 2*PW), per lane.
template <int PW>
__device__ __forceinline__ void piece_shift_down(uint32_t (&w)[PW], int sh) {
    const int ws = sh >> 1;
    const uint32_t bs = (uint32_t)(sh & 1) * 2;
    uint32_t o[PW];
#pragma unroll
    for (int k = 0; k < PW; ++k) {
        uint32_t lo = 0u, hi = 0u;
#pragma unroll
        for (int j = 0; j < PW; ++j) {
            lo = j == k + ws ? w[j] : lo;
            hi = j == k + ws + 1 ? w[j] : hi;
        }
        o[k] = __builtin_amdgcn_alignbyte(hi, lo, bs);
    }
#pragma unroll
    for (int k = 0; k < PW; ++k) w[k] = o[k];
}

template <typename T, int G, int BT, int W, bool YA>
__global__ __launch_bounds__(64 * W, 1) void bwdf_staged_kernel(
    const int* __restrict__ tfeat, const int* __restrict__ meta, const uint16_t* __restrict__ twt,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S, int Tcap) {
    using C = StagedCfg<G, BT, W>;
    constexpr int KS = C::KS, MT = C::MT, STG = C::STG, PB = C::PB, PW = C::PW, AS = C::AS;
    constexpr int NTH = C::NTH, DEPTH = C::DEPTH, NS = C::NS, WAVES = C::WAVES;
    constexpr int TPW = C::TPW;
    using Piece = typename PieceT<PW>::type;
    __shared__ __attribute__((aligned(16))) float acc[(C::DCMAX + kTrashRows) * AS];
    __shared__ __attribute__((aligned(16))) char stg[kStageBufs][STG];

    const int64_t work = xcd_remap(blockIdx.x, (int64_t)S * ndr * nbt);
    if (work < 0) return;
    const int bt = (int)(work % nbt);
    const int r = (int)((work / nbt) % ndr);
    const int s = (int)(work / ((int64_t)nbt * ndr));
    const int d_lo = r * Dc;
    const int dn = min(Dc, D - d_lo);
    const int64_t g_lo = (int64_t)s * gps;
    const int ng = (int)(min<int64_t>(Gc, g_lo + gps) - g_lo);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15;  // operand row within a 16-row block / tile position
    const int kq = lane >> 4;   // which 8 of an MFMA's 32 labels

    // ---- dY pieces: thread tid loads bytes [pbyte, pbyte + PB) of a group's
    // segment of tile row prow.  Rows >= B read as zero.  A row is read up to the
    // 8-label boundary past O (YA: 8 labels more), inside the next row when the
    // stride leaves no room; dY's last row is read up to O only (YA), its piece
    // across O loaded early and shifted back.  Labels >= O are zeroed when
    // staged (only the last group has any).
    const int b0 = bt * BT;
    const int rows = min(BT, B - b0);
    const int prow = (tid * PB) / C::RB;
    const int pbyte = (tid * PB) % C::RB;
    const int plab = pbyte / 2;
    const bool p_last_row = YA && b0 + prow == B - 1;
    const uintptr_t ytile = reinterpret_cast<uintptr_t>(dY + (int64_t)b0 * lddy);
    const uint32_t delta = YA ? (uint32_t)(ytile & 15) : 0u;
    const rsrc_t yr = make_rsrc(reinterpret_cast<const char*>(ytile - delta),
                                ((int64_t)(rows - 1) * lddy +
                                 (!YA ? (O + 7) / 8 * 8 : b0 + rows == B ? O : (O + 7) / 8 * 8 + 8)) * 2 +
                                    delta);
    // (32 bits: the tile's resource spans at most kMaxRsrcBytes)
    const uint32_t yrow = delta + (uint32_t)((int64_t)prow * lddy * 2) + (uint32_t)pbyte;
    // groups are indexed from the slice's first (i = g - g_lo); the last group
    // of dY is i == last_i
    const int last_i = (int)(Gc - 1 - g_lo);
    // YA: elements by which the last group's piece is loaded early (0 unless it
    // straddles O in dY's last row)
    int sh_last = 0;
    if constexpr (YA) {
        const int64_t over = (Gc - 1) * G + plab + PB / 2 - O;
        sh_last = p_last_row && over > 0 && over < PB / 2 ? (int)over : 0;
    }
    auto load_y = [&](int i) __attribute__((always_inline)) -> Piece {
        const uint32_t sh = YA && i == last_i ? (uint32_t)sh_last : 0u;
        return load_piece<PW>(yr, yrow + (uint32_t)(g_lo + i) * (uint32_t)(G * 2) - 2u * sh);
    };
    // group i's piece into staging buffer buf (labels >= O zeroed)
    const int soff = stg_off<G>(prow, pbyte / 16) + (PB < 16 ? pbyte % 16 : 0);
    auto stage = [&](int i, const Piece& pc, int buf) __attribute__((always_inline)) {
        uint32_t w[PW];
        unpack_piece<PW>(pc, w);
        if (i >= last_i) {  // uniform: the last group (or past the end)
            if constexpr (YA) {
                if (i == last_i && sh_last) piece_shift_down<PW>(w, sh_last);
            }
            const int64_t nv = O - ((g_lo + i) * G + plab);  // labels of the piece below O
#pragma unroll
            for (int k = 0; k < PW; ++k)
                w[k] &= (2 * k + 1 < nv) ? 0xFFFFFFFFu : (2 * k < nv ? 0xFFFFu : 0u);
        }
        char* p = &stg[buf][soff];
        if constexpr (PW == 1) {
            *reinterpret_cast<uint32_t*>(p) = w[0];
        } else if constexpr (PW == 2) {
            *reinterpret_cast<u32x2*>(p) = u32x2{w[0], w[1]};
        } else if constexpr (PW == 4) {
            *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
        } else {
            *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
            *reinterpret_cast<u32x4*>(&stg[buf][stg_off<G>(prow, pbyte / 16 + 1)]) =
                u32x4{w[4], w[5], w[6], w[7]};
        }
    };
    // the dY operand fragments of all BT rows from staging buffer buf
    auto read_a = [&](int buf, u32x4 (&a)[MT][KS]) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                a[mt][ks] = *reinterpret_cast<const u32x4*>(&stg[buf][stg_off<G>(16 * mt + col, 4 * ks + kq)]);
    };

    // ---- per-group metadata: tile range of group g_lo + i in range r, (tb |
    // tm << 16, te): layer-0 tiles [tb, tm), layer-1 tiles [tm, te).  A buffer
    // (vector) load, used DEPTH + 1 iterations later (a scalar load would hold
    // up every LDS wait of the wave until it returns).  Past the slice: zero.
    const rsrc_t mr = make_rsrc(meta + (g_lo * ndr + r) * kMetaStride,
                                ((int64_t)(max(ng, 1) - 1) * ndr + 1) * kMetaStride * 4);
    auto load_meta = [&](int i) __attribute__((always_inline)) -> u32x2 {
        return buf_load8(mr, i < ng ? (uint32_t)(i * ndr * kMetaStride * 4) : kOOB);
    };
    auto uniform_meta = [](const u32x2& m) __attribute__((always_inline)) -> u32x2 {
        return u32x2{(uint32_t)__builtin_amdgcn_readfirstlane((int)m[0]),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)m[1])};
    };

    char* const accb = reinterpret_cast<char*>(acc);
    const int colb = kq * 16;  // bytes: batch rows 4kq .. 4kq+3 of a 16-row block

    // W^T tiles and their partial-row offsets of the slice's groups, addressed by
    // 32-bit offsets from the slice's first tile (the plan keeps a slice's twt
    // under kMaxRsrcBytes).  A wave whose tile a group lacks reads some other
    // tile of the slice (or zeros past its end) and never uses what it read.
    const rsrc_t wr_s = make_rsrc(twt + g_lo * Tcap * 16 * G, (int64_t)ng * Tcap * 16 * G * 2);
    const rsrc_t fr_s = make_rsrc(tfeat + g_lo * Tcap * 16, (int64_t)ng * Tcap * 16 * 4);

    // Partial-row byte offsets of a lane's position for the two passes of an
    // update: pass 1 adds the hi and single rows (lo rows go to a trash row),
    // pass 2 the lo rows (bit 0 of the plan's offset; the others to a trash row).
    const int trash_b = (C::DCMAX + (col & (kTrashRows - 1))) * AS * 4;
    auto pass1 = [&](int fo) __attribute__((always_inline)) { return (fo & 1) ? trash_b : fo; };
    auto pass2 = [&](int fo) __attribute__((always_inline)) { return (fo & 1) ? fo - 1 : trash_b; };
    // whether any lane of the wave holds a lo row (uniform)
    auto any_lo = [](int fo) __attribute__((always_inline)) {
        return __builtin_amdgcn_ballot_w64((fo & 1) != 0) != 0;
    };

    // The pipeline.  Step j's loads -- W^T fragments and partial-row offsets
    // of group j, dY piece of group j+1, metadata of group j+DEPTH+1 -- are
    // issued in iteration j-DEPTH into register slot j % NS, in the same order
    // every iteration, so iteration i waits for exactly the loads of step i.
    // Iteration i stages group i+1's dY, multiplies group i and adds group
    // i-1's products into the partial; kGroupUnroll iterations are unrolled so
    // that every slot and staging buffer index is a constant.
    {
        struct Frag {
            u32x4 b0[TPW][KS];       // tiles wave + WAVES*k
            int fo[TPW];             // the plan's partial-row offsets of the lane's positions
        };
        auto load_frag = [&](int i, u32x2 m, Frag& fr) __attribute__((always_inline)) {
            const uint32_t tb = m[0] & 0xFFFFu;
            // the wave's tile, counted from the slice's first
            const uint32_t t0 = (uint32_t)i * (uint32_t)Tcap + tb + (uint32_t)wave;
            const uint32_t fl = (uint32_t)lane * 16u;  // the lane's 16 bytes of a k-step's 1 KB
#pragma unroll
            for (int k = 0; k < TPW; ++k)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    fr.b0[k][ks] = buf_load16(wr_s, (t0 + k * WAVES) * (16u * G * 2u) + fl + ks * 1024u);
#pragma unroll
            for (int k = 0; k < TPW; ++k)
                fr.fo[k] = (int)buf_load4(fr_s, ((t0 + k * WAVES) * 16u + (uint32_t)col) * 4u);
        };
        auto mma = [&](const u32x4 (&a)[MT][KS], const u32x4 (&b)[KS], f32x4 (&c)[MT])
            __attribute__((always_inline)) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(a[mt][ks], b[ks], v);
                c[mt] = v;
            }
        };
        // products c of a tile added at the lane's plan offset fo (both passes)
        auto add_tile = [&](int fo, const f32x4 (&c)[MT]) __attribute__((always_inline)) {
            const int o1 = pass1(fo);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                f32x4* q = reinterpret_cast<f32x4*>(accb + o1 + mt * 64 + colb);
                *q = *q + c[mt];
            }
            if (any_lo(fo)) {
                const int o2 = pass2(fo);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    f32x4* q = reinterpret_cast<f32x4*>(accb + o2 + mt * 64 + colb);
                    *q = *q + c[mt];
                }
            }
        };
        // Tiles of group g_lo + i beyond the pipeline's (>= kStagedTiles),
        // loaded and added at once by the wave that owns the pipeline tile of
        // the same index modulo WAVES.
        auto extra = [&](int i, u32x2 m, int buf) __attribute__((always_inline)) {
            const int tb = (int)(m[0] & 0xFFFF), te = (int)m[1];
            const int64_t gbase = (g_lo + __builtin_amdgcn_readfirstlane(i)) * Tcap;
            u32x4 a[MT][KS];
            read_a(buf, a);
            // tiles are addressed from the group's first tile (all in range)
            const rsrc_t wr = make_rsrc_u32(twt + gbase * 16 * G, (uint32_t)te * 16u * G * 2u);
            const rsrc_t frr = make_rsrc_u32(tfeat + gbase * 16, (uint32_t)te * 16u * 4u);
            for (int t = wave + kStagedTiles; t < te - tb; t += WAVES) {
                u32x4 b0[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    b0[ks] = buf_load16(wr, (uint32_t)((tb + t) * 16 * G + (ks * 64 + lane) * 8) * 2);
                const int fo = (int)buf_load4(frr, (uint32_t)((tb + t) * 16 + col) * 4);
                f32x4 c0[MT];
                mma(a, b0, c0);
                add_tile(fo, c0);
            }
            // every load of this pass has been used; say so, so that later code
            // need not wait for them
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        };

        Frag fq[NS];
        Piece yq[NS];
        u32x2 mraw[NS];
        u32x2 mu[DEPTH + 1];  // uniform metadata of groups i .. i+DEPTH
        f32x4 pd[TPW][MT];    // products of the previous group
        int fod[TPW];
        int n0d = 0;          // uniform: tiles of the previous group
#pragma unroll
        for (int k = 0; k < TPW; ++k) fod[k] = 0;
        {
            u32x2 m0[DEPTH + 1];
#pragma unroll
            for (int k = 0; k <= DEPTH; ++k) m0[k] = load_meta(k);
            Piece y0[kPlanWindow];
#pragma unroll
            for (int k = 0; k < kPlanWindow; ++k) y0[k] = load_y(k);
            for (int k = tid * 4; k < dn * AS; k += NTH * 4)
                *reinterpret_cast<f32x4*>(&acc[k]) = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k <= DEPTH; ++k) mu[k] = uniform_meta(m0[k]);
#pragma unroll
            for (int k = 0; k < kPlanWindow; ++k) stage(k, y0[k], k);
#pragma unroll
            for (int k = 0; k < DEPTH; ++k) {
                __builtin_amdgcn_sched_barrier(0);
                load_frag(k, mu[k], fq[k % NS]);
                yq[k % NS] = load_y(k + kPlanWindow);
                mraw[k % NS] = load_meta(k + DEPTH + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(0));
        __builtin_amdgcn_s_barrier();
        auto body = [&](int i, auto kc) __attribute__((always_inline)) {
            constexpr int K = decltype(kc)::value;  // i % kGroupUnroll
            constexpr int Q = K % NS;               // slot of step i
            constexpr int QN = (Q + DEPTH) % NS;    // slot of step i + DEPTH
            load_frag(i + DEPTH, mu[DEPTH], fq[QN]);
            yq[QN] = load_y(i + DEPTH + kPlanWindow);
            mraw[QN] = load_meta(i + 2 * DEPTH + 1);
            const u32x2 m = mu[0];
            const int tb = (int)(m[0] & 0xFFFF), te = (int)m[1];
            // The previous group's partial rows (pass 1) are read, and this
            // group's products computed, whether or not the wave has the tile
            // (the offsets always name valid rows; a wave without the tile
            // multiplies some other tile, and neither result is written):
            // branches here would only add register initialisations.
            f32x4 old[TPW][MT];
#pragma unroll
            for (int k = 0; k < TPW; ++k)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    old[k][mt] = *reinterpret_cast<const f32x4*>(accb + pass1(fod[k]) + mt * 64 + colb);
            stage(i + kPlanWindow, yq[Q], (K + kPlanWindow) % kStageBufs);
            f32x4 pc[TPW][MT];
            u32x4 a[MT][KS];
            read_a(K % kStageBufs, a);
#pragma unroll
            for (int k = 0; k < TPW; ++k) mma(a, fq[Q].b0[k], pc[k]);
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
                if (wave + k * WAVES < n0d) {  // uniform: the wave had tile k
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        *reinterpret_cast<f32x4*>(accb + pass1(fod[k]) + mt * 64 + colb) = old[k][mt] + pd[k][mt];
                    if (any_lo(fod[k])) {  // the tile's lo rows, after their hi rows
                        const int o2 = pass2(fod[k]);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            f32x4* q = reinterpret_cast<f32x4*>(accb + o2 + mt * 64 + colb);
                            *q = *q + pd[k][mt];
                        }
                    }
                }
            }
            n0d = te - tb;
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
                fod[k] = fq[Q].fo[k];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) pd[k][mt] = pc[k][mt];
            }
#pragma unroll
            for (int k = 0; k < DEPTH; ++k) mu[k] = mu[k + 1];
            mu[DEPTH] = uniform_meta(mraw[Q]);
            // The barrier orders this iteration's partial updates (group
            // i-1's) before the next one's (group i's) and publishes the
            // staged tiles.  Within a plan window (every feature its groups
            // share in one wave's tile) the updates need none: it runs after
            // the iteration of a window's first group, and of a group the
            // plan could not lay out with its window; a tile staged
            // kPlanWindow groups ahead is published by one of them in time.
            const bool more = te - tb > kStagedTiles;  // uniform, rare
            if (K % kPlanWindow == 0 || (m[0] & kMetaUnpaired) || more) {
                __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(0));
                __builtin_amdgcn_s_barrier();
            }
            if (more) {
                extra(i, m, K % kStageBufs);
                __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(0));
                __builtin_amdgcn_s_barrier();
            }
        };
        for (int i = 0; i < ng; i += kGroupUnroll) {
            body(i, std::integral_constant<int, 0>{});
            body(i + 1, std::integral_constant<int, 1>{});
            body(i + 2, std::integral_constant<int, 2>{});
            body(i + 3, std::integral_constant<int, 3>{});
            body(i + 4, std::integral_constant<int, 4>{});
            body(i + 5, std::integral_constant<int, 5>{});
        }
#pragma unroll
        for (int k = 0; k < TPW; ++k)
            if (wave + k * WAVES < n0d) add_tile(fod[k], pd[k]);
        // every load has been used (the last iterations' look-ahead loads are
        // out of range or unused)
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    }
    __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(0));
    __syncthreads();

    // ---- write the partial: ws[s][d_lo + d][bt*BT + b] ----
    float* out = ws + ((int64_t)s * D + d_lo) * Bp + (int64_t)bt * BT;
    for (int i = tid; i < dn * (BT / 4); i += NTH) {
        const int d = i / (BT / 4), q = i % (BT / 4);
        *reinterpret_cast<f32x4*>(out + (int64_t)d * Bp + q * 4) =
            *reinterpret_cast<const f32x4*>(&acc[d * AS + q * 4]);
    }
}

template <typename T, int G, int BT, int W, bool YA>
int launch_staged(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
                  int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
                  hipStream_t st) {
    const int64_t nlog = p.S * p.ndr * p.nbt;
    const int64_t grid = 8 * ceil_div(nlog, 8);
    if (((int64_t)BT * lddy + 8) * 2 > kMaxRsrcBytes) {
        set_error("haste_ffi_bwd_features: lddy = %lld too large", (long long)lddy);
        return HASTE_ERR_UNSUPPORTED;
    }
    bwdf_staged_kernel<T, G, BT, W, YA><<<dim3((unsigned)grid), dim3(64 * W), 0, st>>>(
        tfeat, meta, twt, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, O, p.Gc, (int)p.nbt, (int)p.ndr,
        (int)p.Dc, (int)p.gps, (int)p.S, (int)p.Tcap);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

}  // namespace

// The staged main kernel for a plan made for it (p.staged), defined in
// ffi_bwd_features_staged.hip.
int bwdf_run_staged(int32_t dtype, int64_t G, bool ya, const int* tfeat, const int* meta,
                    const uint16_t* twt, const uint16_t* dY, int64_t lddy, float* ws,
                    const BwdFPlan& p, int64_t B, int64_t D, int64_t O, hipStream_t st);

}  // namespace haste
