// Layout of the backward-to-features workspace ("plan" + transposed weights),
// shared by the bwd-features kernels and the fused weight-gradient + SGD kernel,
// which can refresh the transposed weights of the updated W for the next step.
//
// Per group g (Gc = ceil(O/G) groups), the distinct indices of idx[g, :] are
// split by feature range (ndr ranges of Dc features) and laid out in tiles of
// 16 positions; an index occurring k > 1 times gets a "hi" row in layer 0 and
// a "lo" row in layer 1 -- or, in the staged build's plan (in-tile mode), the
// lo row right after the hi row in the same layer-0 tile, its tfeat entry
// marked by bit 0, and no layer 1.  Workspace regions (byte offsets in BwdFPlan):
//   tfeat  int32 [Gc, Tcap*16]  LDS byte offset of the position's feature row
//   tsrc   int32 [Gc, Tcap*16]  (start << 10) | (count << 1) | lo: the position
//                               sums W over slots perm[g*F + start .. +count)
//   perm   int32 [Gc, F]        slots of the group sorted by index
//   meta   int32 [Gc, ndr, 2]   tb | tm << 16, te: tiles [tb, tm) layer 0, [tm, te)
//                               layer 1 of the range
//   twt    16-bit [Gc, Tcap*16, G]  W^T: row p = sum of W columns of position p
//                               (tiles of 16 rows, chunk-major: twt_elem)
//   partials fp32 [S, D, Bp]    per-slice partial sums of dX^T
#pragma once

#include <algorithm>
#include <cmath>

#include "common.hpp"

namespace haste {

constexpr int kAccPad = 4;        // fp32 words of padding per LDS partial row (bank spread)
constexpr int kTrashRows = 4;     // LDS partial rows that padding tile columns add into
constexpr int kTargetCTAs = 256;
constexpr int kMaxRanges = 128;   // feature ranges per group handled by the plan kernel
constexpr int kMetaStride = 2;    // ints per (group, range): tb | tm << 16, te
constexpr int kLdsBytes = 160 * 1024;
constexpr int kLdsMisc = 1024;    // LDS the main kernel keeps for other things
constexpr int kGroupUnroll = 6;   // groups per unrolled iteration of the main kernel's loop

// The main kernel stages each group's W^T tiles (and their partial-row offsets)
// in a double-buffered LDS ring of RT tiles of 16 rows; a W^T row is 2G bytes,
// stored with 32 bytes of padding (conflict-free 16-byte reads of 16 rows).
// Ranges with more tiles take the rest from global memory.  Every wave
// multiplies all RT ring tiles of a round, so the kernel is built for RT in
// {2, 3, ring_tiles(G)} and the plan picks the smallest ring that a range's
// tiles fit in 99 % of rounds (ring_overflow below); a smaller ring also
// leaves more LDS for the partial.
__host__ __device__ constexpr int ring_tiles(int G) { return G <= 16 ? 8 : G <= 32 ? 6 : G <= 64 ? 4 : 3; }
__host__ __device__ constexpr int ring_row_bytes(int G) { return 2 * G + 32; }
__host__ __device__ constexpr int ring_bytes(int G, int rt) {
    return 2 * rt * 16 * (ring_row_bytes(G) + 4);
}
__host__ __device__ constexpr int acc_stride(int bt) { return bt + kAccPad; }
// Features per range: the LDS partial holds (Dc + kTrashRows) rows of bt fp32.
__host__ __device__ constexpr int max_dc(int bt, int G, int rt) {
    return (kLdsBytes - kLdsMisc - ring_bytes(G, rt)) / 4 / acc_stride(bt) - kTrashRows;
}

// The staged build (bwdf_staged.hpp): kStagedTiles W^T tiles of a group's
// range in its pipeline, dealt over its waves, and a ring of kStageBufs LDS
// copies of the groups' dY tiles of bt rows x G labels beside the partial
// (group i in buffer i % kStageBufs, staged kPlanWindow groups ahead).  Its
// plan is made in windows of kPlanWindow groups (bwdf_plan_window_kernel) that
// need no barrier between their partial updates; bit 31 of a group's meta
// word 0 says it could not be laid out as part of its window.
constexpr int kStagedTiles = 8;
constexpr int kStagedWaves = 8;  // the model's wave count (pick_staged_bt)
constexpr int kStageBufs = 6;    // kGroupUnroll: a group's buffer is its unrolled step
#ifndef HASTE_PLAN_WINDOW
#define HASTE_PLAN_WINDOW 3
#endif
constexpr int kPlanWindow = HASTE_PLAN_WINDOW;
static_assert(kGroupUnroll % kPlanWindow == 0 && 2 * kPlanWindow <= kStageBufs, "plan window");
constexpr uint32_t kMetaUnpaired = 0x80000000u;
__host__ __device__ constexpr int staged_max_dc(int bt, int G) {
    return (kLdsBytes - kLdsMisc - kStageBufs * bt * 2 * G) / 4 / acc_stride(bt) - kTrashRows;
}

// Probability that a range holds more than rt layer-0 tiles when its share of
// a group's F indices is Binomial(F, q) -- an upper bound for indices drawn
// uniformly without replacement, whose share is hypergeometric.
inline double ring_overflow(int64_t F, double q, int rt) {
    const int64_t cap = 16 * (int64_t)rt;
    if (cap >= F) return 0.0;
    if (q >= 1.0) return 1.0;
    // log pmf by the ratio pmf(n+1) / pmf(n) = (F-n)/(n+1) * q/(1-q), from
    // pmf(0) = (1-q)^F (no lgamma: it writes the global signgam)
    const double lodds = std::log(q) - std::log1p(-q);
    double lp = (double)F * std::log1p(-q), s = 0.0;
    for (int64_t n = 0; n < F; ++n) {
        if (n > cap) s += std::exp(lp);
        lp += std::log((double)(F - n) / (double)(n + 1)) + lodds;
    }
    return s + std::exp(lp);  // n = F
}

// The smallest ring whose rounds overflow for under 1 % of (group, range)
// pairs.  Plans are made on every call, so the last shape's choice is kept
// (per host thread) instead of summing the binomial tail again.
inline int64_t pick_ring(int64_t BT, int64_t D, int64_t F, int64_t G) {
    thread_local int64_t key[4] = {-1, -1, -1, -1};
    thread_local int64_t last = 0;
    if (key[0] == BT && key[1] == D && key[2] == F && key[3] == G) return last;
    int64_t ring = ring_tiles((int)G);
    for (int rt = 2; rt <= 3 && rt < ring; ++rt) {
        const int64_t dc = ceil_div(D, ceil_div(D, (int64_t)max_dc((int)BT, (int)G, rt)));
        if (ring_overflow(F, std::min(1.0, (double)dc / (double)D), rt) < 0.01) {
            ring = rt;
            break;
        }
    }
    key[0] = BT; key[1] = D; key[2] = F; key[3] = G;
    last = ring;
    return ring;
}

// W^T is stored in tiles of 16 rows, chunk-major: the 16-byte chunk k (labels
// 8k .. 8k+7) of row p of a tile is chunk k*16 + p of the tile, so the 16 rows'
// chunk k -- what 16 lanes of an MFMA operand fragment read -- are one
// contiguous 256-byte block.  Element offset of the chunk of labels lc .. lc+7
// of tile row `row` (a group's rows start at a multiple of 16), and the (row,
// chunk) of a group's it-th chunk in storage order.
__host__ __device__ constexpr int64_t twt_elem(int64_t row, int lc, int G) {
    return (row / 16) * 16 * G + ((lc / 8) * 16 + row % 16) * 8;
}
__host__ __device__ constexpr int twt_row_of(int it, int G) { return (it / (2 * G)) * 16 + it % 16; }
__host__ __device__ constexpr int twt_chunk_of(int it, int G) { return (it / 16) % (G / 8); }

struct BwdFPlan {
    int64_t Gc, BT, nbt, Bp, ndr, Dc, S, gps, Tcap;
    int64_t RT, DCMAX;  // ring tiles of the main kernel; its partial's trash rows start at DCMAX
    int64_t staged;     // the plan is for the staged main kernel (RT unused)
    int64_t tfeat_off, tsrc_off, perm_off, meta_off, twt_off, prep_bytes, ws_bytes;
};

// Sum of the S per-slice partials of dX^T (fp32 [S, D, Bp]) at feature d,
// batch columns b4 .. b4+3.
__device__ __forceinline__ f32x4 sum_slices(const float* __restrict__ ws, int64_t D, int Bp,
                                            int S, int64_t d, int b4) {
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    const float* p = ws + d * Bp + b4;
    const int64_t step = D * Bp;
#pragma unroll 4
    for (int s = 0; s < S; ++s) v += *reinterpret_cast<const f32x4*>(p + s * step);
    return v;
}

// The final pass of backward to features with stochastic rounding, as a job of
// ntiles tiles of 32 features x 32 batch columns (nx tiles along D): sum the
// slices, transpose [D, B] -> [B, D] and round to bf16 with
// tl.randint(seed, b*D + d).
struct ReduceJob {
    const float* ws;
    uint16_t* dX;
    int B, Bp, D, S, nx, ntiles;
    uint32_t k0, k1;
};

inline ReduceJob reduce_job(const BwdFPlan& p, const float* ws, uint16_t* dX, int64_t B,
                            int64_t D, uint64_t seed) {
    ReduceJob j{ws, dX, (int)B, (int)p.Bp, (int)D, (int)p.S, (int)ceil_div(D, 32), 0,
                (uint32_t)seed, (uint32_t)(seed >> 32)};
    j.ntiles = j.nx * (int)ceil_div(B, 32);
    return j;
}

// Tile `tile` of the job, by a workgroup of 256 threads; t: 32 x 33 floats of LDS.
__device__ __forceinline__ void reduce_sr_tile(const ReduceJob& j, int tile, float (*t)[33]) {
    const int d0 = (tile % j.nx) * 32, b0 = (tile / j.nx) * 32;
    {
        const int r = threadIdx.x >> 3, c4 = (threadIdx.x & 7) * 4;
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (d0 + r < j.D) v = sum_slices(j.ws, j.D, j.Bp, j.S, d0 + r, b0 + c4);
#pragma unroll
        for (int e = 0; e < 4; ++e) t[r][c4 + e] = v[e];
    }
    __syncthreads();
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // ty in 0..7
    for (int r = ty; r < 32; r += 8) {
        const int b = b0 + r, d = d0 + tx;
        if (d < j.D && b < j.B) {
            const uint64_t off = (uint64_t)b * j.D + d;
            j.dX[(int64_t)b * j.D + d] = (uint16_t)sr_bf16(
                t[tx][r], philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, j.k0, j.k1));
        }
    }
}

// The main-kernel build selected by haste_ffi_bwd_features_set_build (0 by
// shape, 1 LDS ring, 2 direct where built).
int bwdf_build();


// Batch columns per workgroup of the staged build, 32 or 64, by a model of
// the clocks a CU spends per (group, range, batch tile): LDS -- staging the dY
// tile (about 13 clocks per KB written), reading its operands (4.4 per KB) and
// the partial read-modify-writes (17.8 per KB) for each of the range's tiles
// -- against the vector-memory address path (about 45 bytes per clock: the dY
// tile plus every wave's W^T fragment loads, issued whether or not the wave has
// a tile), plus about 150 clocks of per-group overhead; times the number of
// (group, range, batch tile) units.  Measured rates on the pool's MI355X.
inline int64_t pick_staged_bt(int64_t B, int64_t D, int64_t F, int64_t G) {
    int64_t best_bt = 32;
    double best = -1.0;
    for (int64_t bt = 32; bt <= 64; bt *= 2) {
        if (bt > 32 && B <= 32) break;
        const int64_t ndr = ceil_div(D, (int64_t)staged_max_dc((int)bt, (int)G));
        const double tiles = std::ceil((double)F / (double)ndr / 16.0) + 0.5;
        const double stg = (double)(bt * 2 * G) / 1024.0;  // KB
        const double lds = stg * 13.0 + tiles * (stg * 4.4 + 16.0 * bt * 4 / 1024.0 * 17.8);
        const double ta = (stg * 1024.0 + (kStagedWaves + 2) * (G / 32) * 1024.0 +
                           kStagedWaves * 256.0) / 45.0;
        const double cost = (double)(ndr * ceil_div(B, bt)) * (std::max(lds, ta) + 150.0);
        if (best < 0.0 || cost < best) {
            best = cost;
            best_bt = bt;
        }
    }
    return best_bt;
}

// The plan for the staged build (staged = true) or the ring / direct builds.
inline BwdFPlan make_plan_for(int64_t B, int64_t D, int64_t F, int64_t O, int64_t G, bool staged) {
    BwdFPlan p;
    p.Gc = ceil_div(O, G);
    p.staged = staged;
    if (p.staged) {
        p.BT = pick_staged_bt(B, D, F, G);
        p.RT = 0;
        p.DCMAX = staged_max_dc((int)p.BT, (int)G);
    } else {
        // 128 batch columns per workgroup, or 64 when the batch is that small or
        // when a 128-column partial would split D into 8 or more feature ranges
        // (every range re-reads dY; with 64 columns a range holds twice the
        // features: config 3, D = 4096, 15 -> 8 ranges, bwd-features 868 -> 804 us;
        // at 3-4 ranges the 128-column build is faster: config 1 103 vs 149 us)
        p.BT = 128;
        if (B <= 64 || ceil_div(D, (int64_t)max_dc(128, (int)G, (int)pick_ring(128, D, F, G))) >= 8)
            p.BT = 64;
        p.RT = pick_ring(p.BT, D, F, G);
        p.DCMAX = max_dc((int)p.BT, (int)G, (int)p.RT);
    }
    p.nbt = ceil_div(B, p.BT);
    p.Bp = p.nbt * p.BT;
    p.ndr = ceil_div(D, p.DCMAX);
    p.Dc = ceil_div(D, p.ndr);
    int64_t S = std::max<int64_t>(1, kTargetCTAs / (p.nbt * p.ndr));
    S = std::min<int64_t>(S, std::max<int64_t>(1, ceil_div(p.Gc, 8)));
    // the main kernel's group loop is unrolled kGroupUnroll times without
    // guards: only the last slice runs (empty) iterations past its groups
    p.gps = ceil_div(ceil_div(p.Gc, S), kGroupUnroll) * kGroupUnroll;
    p.S = ceil_div(p.Gc, p.gps);
    // tiles per group: layer 0 holds <= F distinct features, layer 1 <= F/2, and
    // each non-empty range pads its layer to a multiple of 16
    const int64_t r0 = std::min<int64_t>(p.ndr, F), r1 = std::min<int64_t>(p.ndr, F / 2);
    p.Tcap = ceil_div(F + 15 * r0, 16) + ceil_div(F / 2 + 15 * r1, 16);
    auto r256 = [](int64_t x) { return (x + 255) / 256 * 256; };
    p.tfeat_off = 0;
    p.tsrc_off = r256(p.Gc * p.Tcap * 16 * 4);
    p.perm_off = p.tsrc_off + r256(p.Gc * p.Tcap * 16 * 4);
    p.meta_off = p.perm_off + r256(p.Gc * F * 4);
    p.twt_off = p.meta_off + r256(p.Gc * p.ndr * kMetaStride * 4);
    p.prep_bytes = p.twt_off + r256(p.Gc * p.Tcap * 16 * G * 2);
    p.ws_bytes = p.S * D * p.Bp * 4;
    return p;
}

// The plan of the build that haste_ffi_bwd_features_set_build selects (1 ring,
// 2 direct, 3 staged; 0: by shape).  By shape, G >= 32 takes the staged build
// where a group's range holds seven or more tiles of 16 positions, so that
// nearly all of its eight waves have a tile (measured, config 1: 86 -> 82 us;
// config 4: 3452 -> 2402 us; with four tiles, configs 2 and 3, it was slower
// than the ring and direct builds: 295 -> 336 and 606 -> 805 us), and where
// the slice's W^T tiles span at most kMaxRsrcBytes (its 32-bit tile offsets).
inline BwdFPlan make_plan(int64_t B, int64_t D, int64_t F, int64_t O, int64_t G) {
    const int build = bwdf_build();
    if (G >= 32 && (build == 0 || build == 3)) {
        const BwdFPlan p = make_plan_for(B, D, F, O, G, true);
        const bool fits = (p.gps + 8) * p.Tcap * 16 * G * 2 <= kMaxRsrcBytes;
        if (fits && (build == 3 || F >= 7 * 16 * p.ndr)) return p;
    }
    return make_plan_for(B, D, F, O, G, false);
}

// One 16-byte chunk (labels lc .. lc+7 of the group) of the W^T row described by
// src (a tsrc entry): a single W column, or for a duplicated index the 16-bit
// rounding of the fp32 sum of its columns (ascending slot order) -- the "hi"
// row -- or the rounding of the remainder -- the "lo" row; padding rows are 0.
// wv(l, slot) returns the 16-bit pattern of W[l0 + l, slot].
template <typename T, typename WV>
__device__ __forceinline__ u32x4 wt_chunk(int src, const int* perm_g, WV wv, int lc) {
    const int start = src >> 10, cnt = (src >> 1) & 511, lo = src & 1;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (cnt == 1) {
        const int slot = perm_g[start];
#pragma unroll
        for (int e = 0; e < 8; e += 2) v[e >> 1] = wv(lc + e, slot) | (wv(lc + e + 1, slot) << 16);
    } else if (cnt > 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float sum = 0.0f;
            for (int q = 0; q < cnt; ++q) sum += bits_to_f32<T>(wv(lc + e, perm_g[start + q]));
            const uint32_t hb = f32_to_bits<T>(sum);
            const uint32_t b = lo ? f32_to_bits<T>(sum - bits_to_f32<T>(hb)) : hb;
            v[e >> 1] |= (e & 1) ? (b << 16) : b;
        }
    }
    return v;
}

}  // namespace haste
