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
//     and a "lo" row in layer 1 at the same (tile, position) of its layer, so
//     inside a layer every feature occurs once and layer-1 tile t pairs with
//     layer-0 tile t.  Features are dealt over the tiles position by position
//     in order of (feature mod 16, feature), so the 16 lanes of a tile mostly
//     hit distinct LDS bank groups in step 2.
//     gather (when W changed since the last call): tile row p of group g = W_g
//     column of p's slot, transposed (WT[pos][label]); a duplicated index gets
//     sum_j W[l, j] (fp32, ascending j) split into its 16-bit rounding (hi)
//     and the 16-bit rounding of the remainder (lo).  The fused weight-gradient
//     + SGD kernel writes the same rows for the weights it updates.
//  2. main: a workgroup owns (group slice s, feature range r, batch tile of BT
//     columns) and keeps dXT[range, tile] as an fp32 partial in LDS; wave w
//     owns batch rows [16w, 16w+16), so no two waves touch one LDS word.  Per
//     group the range's WT tiles are staged once into an LDS ring shared by
//     the waves; each wave multiplies its dY rows with them (MFMA, M = batch
//     rows, N = 16 positions, K = labels) and, one group later, a lane adds
//     four consecutive batch values of one position -- the layer-0 product
//     plus the paired layer-1 product -- into the partial row of the
//     position's feature (one 16-byte read and one 16-byte write).  A wave's
//     LDS accesses complete in program order, so later groups see the
//     earlier writes.
//  3. reduce: dXT = sum over slices s = 0..S-1 in ascending order (fp32 out), or
//     fused with the bf16 stochastic rounding of shared_ffi/bindings.py:44-48.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "bwdf_main.hpp"
#include "bwdf_staged.hpp"


namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

namespace {

// --------------------------------------------------------------- plan ------
// Layer-0 slots of a range with T0 layer-0 tiles, T1 layer-1 tiles and nd
// duplicated features: duplicated feature k sits at (tile k % T1, position
// k / T1), as its layer-1 row does, so at position p the tiles [0,
// dup_tiles_at(p)) hold duplicated features.  The other ("free") slots are
// numbered position by position, tile by tile.
__device__ __forceinline__ int dup_tiles_at(int p, int T1, int nd) {
    return min(max(nd - p * T1, 0), T1);
}
__device__ __forceinline__ int dup_free_index(int t, int p, int T0, int T1, int nd) {
    int n = 0;
    for (int s = 0; s < p; ++s) n += T0 - dup_tiles_at(s, T1, nd);
    return n + t - dup_tiles_at(p, T1, nd);
}
// In-tile mode (the staged build's plan): a range's duplicated features come
// first, feature k's two rows in tile k / 8 at positions 2(k % 8) and
// 2(k % 8) + 1; single features fill the other slots position by position over
// the tiles.  Tiles from in_first_free(p, nd) on have position p free.
__device__ __forceinline__ int in_first_free(int p, int nd) {
    return max(0, (nd - p / 2 + 7) / 8);
}
__device__ __forceinline__ void in_free_slot(int k, int T, int nd, int& t, int& p) {
    for (p = 0; p < 15; ++p) {
        const int fr = T - min(T, in_first_free(p, nd));
        if (k < fr) break;
        k -= fr;
    }
    t = in_first_free(p, nd) + k;
}
__device__ __forceinline__ int in_free_index(int t, int p, int T, int nd) {
    int n = 0;
    for (int q = 0; q < p; ++q) n += T - min(T, in_first_free(q, nd));
    return n + t - in_first_free(p, nd);
}
__device__ __forceinline__ void dup_free_slot(int k, int T0, int T1, int nd, int& t, int& p) {
    for (p = 0; p < 15; ++p) {
        const int fr = T0 - dup_tiles_at(p, T1, nd);
        if (k < fr) break;
        k -= fr;
    }
    t = dup_tiles_at(p, T1, nd) + k;
}

// Tiles of group g start at tile g*Tcap.  For range r, meta[(g*ndr + r)*2 + 0..1]
// = (tb | tm << 16, te): layer-0 tiles [tb, tm), layer-1 tiles [tm, te) (relative
// to g*Tcap); meta[(g*ndr + ndr-1)*2 + 1] is the group's tile count.  The
// staged build's plan is made in the in-tile mode instead (plan_in_tile,
// bwdf_plan_pair_kernel): no layer 1 (tm = te); a duplicated feature's "lo"
// row sits in the same tile as its "hi" row, one position after it, and its
// tfeat entry carries bit 0 (row offsets are multiples of 16).  For tile row
// (t, p): tfeat = byte offset of the feature's row in the main kernel's LDS
// partial, (feature - r*Dc) * row_bytes, or (trash_row + p % kTrashRows) * row_bytes for
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
    int pn = 0, pd = 0;  // order of the feature among the range's single / duplicated ones
    if (tid < F && first) {
        for (int k = 0; k < F; ++k) {
            const int v = s_idx[k], fl = s_flag[k];
            const int kk = (((v - r_lo) & 15) << 16) | (v - r_lo);
            const bool in = (fl & 1) && v >= r_lo && v < r_lo + Dc && kk < key;
            pn += in && !(fl & 2);
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
        m[0] = s_tile[rr][0] | (s_tile[rr][1] << 16);
        m[1] = s_tile[rr][2];
    }
    const int64_t tbase = g * Tcap;
    if (tid < F && first) {
        const int T0 = s_tile[r][1] - s_tile[r][0], T1 = s_tile[r][2] - s_tile[r][1];
        // layer-0 slot: a duplicated feature takes the same (tile, position) as
        // its layer-1 row, so the main kernel can add the two products before
        // one partial update; single features fill the other slots position by
        // position over the tiles
        int t, p;
        if (cnt > 1) {
            t = pd % T1;
            p = pd / T1;
        } else {
            dup_free_slot(pn, T0, T1, s_cnt[1][r], t, p);
        }
        const int64_t row0 = (tbase + s_tile[r][0] + t) * 16 + p;
        tfeat[row0] = (f - r_lo) * row_bytes;
        tsrc[row0] = (rank << 10) | (cnt << 1);
        if (cnt > 1) {
            const int64_t row1 = (tbase + s_tile[r][1] + t) * 16 + p;
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
        const int nd = s_cnt[1][rr];
        const int T0 = s_tile[rr][1] - s_tile[rr][0], T1 = s_tile[rr][2] - s_tile[rr][1];
        bool used;
        if (t >= s_tile[rr][1]) {
            used = p * T1 + (t - s_tile[rr][1]) < nd;
        } else {
            const int tt = t - s_tile[rr][0];
            const int occ = dup_tiles_at(p, T1, nd);
            used = tt < occ || dup_free_index(tt, p, T0, T1, nd) < s_cnt[0][rr] - nd;
        }
        if (used) continue;
        tfeat[(tbase + t) * 16 + p] = (trash_row + (p & (kTrashRows - 1))) * row_bytes;
        tsrc[(tbase + t) * 16 + p] = 0;
    }
}

// -------------------------------------------------------- window plan ------
// The staged build's plan (in-tile mode, see bwdf_plan_kernel) made for
// kPlanWindow consecutive groups at a time: the window's first group is laid
// out on its own; each later one with every feature it shares with the
// window's earlier groups (in the same range) in the tile of the same index as
// the latest of them, so the wave that owns that tile adds all of the
// window's products of the feature and the staged kernel needs no barrier
// between the window's partial updates.  Where that does not fit (pinned rows
// over 16 in a tile, or more tiles than the layout tracks or the workspace
// holds), the group is laid out on its own and bit 31 of its meta word 0
// (every range) tells the kernel to keep the barrier before its update.
constexpr int kPairRanges = 8;     // ranges the pinned layout handles (else: unpaired)
constexpr int kPairRangeTiles = 24;  // tiles of a range it tracks

// One slot of a group's index row, as the plan sees it (thread tid = slot).
struct PlanSlot {
    int f, rank, cnt, r, r_lo, pn, pd;
    bool first;
};

// The analysis of group g's index row by the workgroup's 256 threads: the
// clamped indices in s_idx (padded to a multiple of 4 slots), first-occurrence /
// duplicated flags in s_flag, perm, the per-range counts of distinct (s_c[0])
// and duplicated (s_c[1]) features, and the thread's slot (pn / pd left 0, see
// plan_keys).  s_c must be zero on entry.
__device__ __forceinline__ PlanSlot plan_analyse(const int32_t* __restrict__ idx, int64_t g, int F,
                                                 int D, int Dc, int* s_idx, int* s_flag,
                                                 int (*s_c)[kMaxRanges], int* __restrict__ perm) {
    const int tid = threadIdx.x;
    const int F4 = (F + 3) & ~3;  // the rows are scanned 4 slots per 16-byte read
    PlanSlot ps{0, 0, 0, 0, 0, 0, 0, false};
    if (tid < F) s_idx[tid] = min(max(idx[g * F + tid], 0), D - 1);
    else if (tid < F4) s_idx[tid] = INT_MAX;  // padding: matches and precedes no index
    __syncthreads();
    const int4* idx4 = reinterpret_cast<const int4*>(s_idx);
    if (tid < F) {
        ps.f = s_idx[tid];
        int before = 0;
#pragma unroll 4
        for (int k4 = 0; k4 < F4 / 4; ++k4) {
            const int4 v = idx4[k4];
            const int k = 4 * k4;
            ps.rank += (v.x < ps.f) + (v.y < ps.f) + (v.z < ps.f) + (v.w < ps.f);
            before += ((v.x == ps.f) & (k < tid)) + ((v.y == ps.f) & (k + 1 < tid)) +
                      ((v.z == ps.f) & (k + 2 < tid)) + ((v.w == ps.f) & (k + 3 < tid));
            ps.cnt += (v.x == ps.f) + (v.y == ps.f) + (v.z == ps.f) + (v.w == ps.f);
        }
        ps.rank += before;
        ps.first = before == 0;
        perm[g * F + ps.rank] = tid;
        s_flag[tid] = (ps.first ? 1 : 0) | (ps.cnt > 1 ? 2 : 0);
    } else if (tid < F4) {
        s_flag[tid] = 0;
    }
    __syncthreads();
    ps.r = ps.f / Dc;
    ps.r_lo = ps.r * Dc;
    if (tid < F && ps.first) {
        atomicAdd(&s_c[0][ps.r], 1);
        if (ps.cnt > 1) atomicAdd(&s_c[1][ps.r], 1);
    }
    __syncthreads();
    return ps;
}

// ps.pn / ps.pd of a first occurrence (the single / duplicated features of its
// range with a smaller residue key), which plan_in_tile places by.
__device__ __forceinline__ void plan_keys(PlanSlot& ps, int F, int Dc, const int* s_idx,
                                          const int* s_flag) {
    if (!(threadIdx.x < F && ps.first)) return;
    const int F4 = (F + 3) & ~3;
    const int key = (((ps.f - ps.r_lo) & 15) << 16) | (ps.f - ps.r_lo);
    const int4* idx4 = reinterpret_cast<const int4*>(s_idx);
    const int4* flag4 = reinterpret_cast<const int4*>(s_flag);
    auto count = [&](int v, int fl) {
        const int kk = (((v - ps.r_lo) & 15) << 16) | (v - ps.r_lo);
        const bool in = (fl & 1) && v >= ps.r_lo && v < ps.r_lo + Dc && kk < key;
        ps.pn += in && !(fl & 2);
        ps.pd += in && (fl & 2);
    };
#pragma unroll 4
    for (int k4 = 0; k4 < F4 / 4; ++k4) {
        const int4 v = idx4[k4], fl = flag4[k4];
        count(v.x, fl.x);
        count(v.y, fl.y);
        count(v.z, fl.z);
        count(v.w, fl.w);
    }
}

// The in-tile layout of one group on its own (the staged build's plan): tiles per
// range, meta (tm = te, bit 31 of word 0 = flag), the rows of the thread's
// feature and the padding rows.  *t_rel receives the tile of the thread's
// feature relative to its range's first.
__device__ __forceinline__ void plan_in_tile(const PlanSlot& ps, int64_t g, int F, int ndr, int Tcap,
                                             int row_bytes, int trash_row, uint32_t flag,
                                             int (*s_c)[kMaxRanges], int* s_toff,
                                             int* __restrict__ tfeat, int* __restrict__ tsrc,
                                             int* __restrict__ meta, int* t_rel) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        int t = 0;
        for (int rr = 0; rr < ndr; ++rr) {
            s_toff[rr] = t;
            t += (s_c[0][rr] + s_c[1][rr] + 15) / 16;
        }
        s_toff[ndr] = t;
    }
    __syncthreads();
    for (int rr = tid; rr < ndr; rr += 256) {
        int* m = meta + (g * ndr + rr) * kMetaStride;
        m[0] = (int)((uint32_t)s_toff[rr] | ((uint32_t)s_toff[rr + 1] << 16) | flag);
        m[1] = s_toff[rr + 1];
    }
    const int64_t tbase = g * Tcap;
    if (tid < F && ps.first) {
        const int T = s_toff[ps.r + 1] - s_toff[ps.r];
        int t, p;
        if (ps.cnt > 1) {
            t = ps.pd / 8;
            p = 2 * (ps.pd % 8);
        } else {
            in_free_slot(ps.pn, T, s_c[1][ps.r], t, p);
        }
        *t_rel = t;
        const int64_t row0 = (tbase + s_toff[ps.r] + t) * 16 + p;
        tfeat[row0] = (ps.f - ps.r_lo) * row_bytes;
        tsrc[row0] = (ps.rank << 10) | (ps.cnt << 1);
        if (ps.cnt > 1) {
            tfeat[row0 + 1] = (ps.f - ps.r_lo) * row_bytes | 1;
            tsrc[row0 + 1] = (ps.rank << 10) | (ps.cnt << 1) | 1;
        }
    }
    const int nslots = s_toff[ndr] * 16;
    for (int i = tid; i < nslots; i += 256) {
        const int t = i / 16, p = i % 16;
        int rr = 0;
        while (t >= s_toff[rr + 1]) ++rr;  // empty ranges are skipped
        const int nd = s_c[1][rr];
        const int tt = t - s_toff[rr];
        const bool used = tt < in_first_free(p, nd) ||
                          in_free_index(tt, p, s_toff[rr + 1] - s_toff[rr], nd) < s_c[0][rr] - nd;
        if (used) continue;
        tfeat[(tbase + t) * 16 + p] = (trash_row + (p & (kTrashRows - 1))) * row_bytes;
        tsrc[(tbase + t) * 16 + p] = 0;
    }
}

// The tile table of one range for the pinned layout, made by one thread from the
// pinned rows per tile: unpinned duplicated features fill the tiles in order
// (first fit: a tile takes floor((16 - pinned rows) / 2) of them, appended
// tiles 8), pinned singles follow a tile's duplicated rows, and the other
// singles are dealt over the tiles in turn, round k giving one row to every tile
// with at least k free rows (appended tiles take 16 in order).  Writes the
// range's tile count to *nt (over kPairRangeTiles: the pinned layout fails).
struct PairTables {
    int cb[kPairRanges][kPairRangeTiles];    // first unpinned-dup ordinal of the tile
    int ce[kPairRanges][kPairRangeTiles];    // one past its last
    int base[kPairRanges][kPairRangeTiles];  // rows of the tile's duplicated features
    int fr[kPairRanges][kPairRangeTiles];    // rows free for the dealt singles
    int S[kPairRanges][17];                  // dealt singles in rounds 1..k
    int nt1[kPairRanges];                    // tiles before the dealt singles' appended ones
};

__device__ __forceinline__ void pair_range_table(int r, int c0, int nd, int maxpin,
                                                 const int* __restrict__ pd, const int* __restrict__ rs,
                                                 PairTables& tb, int* nt) {
    int npd = 0, nrs = 0, need_ok = 1;
    int p2[kPairRangeTiles], q1[kPairRangeTiles];
#pragma unroll
    for (int t = 0; t < kPairRangeTiles; ++t) {
        p2[t] = 2 * pd[t];
        q1[t] = rs[t];
        npd += pd[t];
        nrs += rs[t];
        need_ok &= p2[t] + q1[t] <= 16;
    }
    const int nt0 = max((c0 + nd + 15) / 16, maxpin + 1);
    const int M = nd - npd, U = (c0 - nd) - nrs;
    int C = 0, nt1 = nt0;
#pragma unroll
    for (int t = 0; t < kPairRangeTiles; ++t) {
        const int cap = t < nt0 ? (16 - p2[t] - q1[t]) / 2 : 8;
        const int u = min(max(M - C, 0), cap);
        if (t >= nt0 && u > 0) nt1 = t + 1;
        tb.cb[r][t] = C;
        tb.ce[r][t] = C + cap;
        C += cap;
        p2[t] += 2 * u;                                  // rows of duplicated features
        tb.base[r][t] = p2[t];
        q1[t] = t < nt1 ? 16 - p2[t] - q1[t] : 0;        // free rows (after nt1 is final below)
    }
    bool ok = need_ok && nt0 <= kPairRangeTiles && M <= C;
    int S = 0;
    tb.S[r][0] = 0;
#pragma unroll
    for (int k = 1; k <= 16; ++k) {
#pragma unroll
        for (int t = 0; t < kPairRangeTiles; ++t) S += (t < nt1 && q1[t] >= k) ? 1 : 0;
        tb.S[r][k] = S;
    }
#pragma unroll
    for (int t = 0; t < kPairRangeTiles; ++t) tb.fr[r][t] = t < nt1 ? q1[t] : 0;
    tb.nt1[r] = nt1;
    const int nt2 = nt1 + (U > S ? (U - S + 15) / 16 : 0);
    *nt = ok ? nt2 : kPairRangeTiles + 1;
}

__global__ __launch_bounds__(256) void bwdf_plan_window_kernel(const int32_t* __restrict__ idx,
                                                               int* __restrict__ tfeat,
                                                               int* __restrict__ tsrc,
                                                               int* __restrict__ perm,
                                                               int* __restrict__ meta, int F, int D,
                                                               int ndr, int Dc, int Tcap,
                                                               int row_bytes, int trash_row,
                                                               int64_t Gc) {
    __shared__ __align__(16) int s_idx[kPlanWindow][256];
    __shared__ __align__(16) int s_flag[kPlanWindow][256];
    __shared__ __align__(16) int s_ftile[kPlanWindow][256];   // tile of the slot's feature (first occurrences)
    __shared__ int s_c[2][kMaxRanges];
    __shared__ int s_toff[kMaxRanges + 1];
    __shared__ int s_pd[kPairRanges][kPairRangeTiles];        // pinned duplicated features per tile
    __shared__ int s_rs[kPairRanges][kPairRangeTiles];        // pinned single features per tile
    __shared__ int s_used[kPairRanges][kPairRangeTiles];      // rows used per tile
    __shared__ int s_maxpin[kPairRanges];
    __shared__ __align__(16) short s_pin[256];                // the slot's pinned tile, or -1
    __shared__ PairTables s_tb;
    __shared__ int s_nt[kPairRanges];                         // tiles per range
    __shared__ int s_fail;
    const int tid = threadIdx.x;
    for (int j = 0; j < kPlanWindow; ++j) {
        const int64_t g = kPlanWindow * (int64_t)blockIdx.x + j;
        if (g >= Gc) return;  // (uniform)
        for (int i = tid; i < 2 * kMaxRanges; i += 256) (&s_c[0][0])[i] = 0;
        for (int i = tid; i < kPairRanges * kPairRangeTiles; i += 256) {
            (&s_pd[0][0])[i] = 0;
            (&s_rs[0][0])[i] = 0;
            (&s_used[0][0])[i] = 0;
        }
        if (tid < kPairRanges) s_maxpin[tid] = -1;
        if (tid == 0) s_fail = j == 0 || ndr > kPairRanges;
        __syncthreads();
        PlanSlot ps = plan_analyse(idx, g, F, D, Dc, s_idx[j], s_flag[j], s_c, perm);
        const bool mine = tid < F && ps.first;
        const bool dup = ps.cnt > 1;
        // each feature the window's earlier groups hold pinned to the tile of
        // the latest of them that holds it
        int pin = -1;
        if (mine) {
            const int F4 = (F + 3) & ~3;
            for (int jj = j - 1; jj >= 0 && pin < 0; --jj) {
                const int4* v4 = reinterpret_cast<const int4*>(s_idx[jj]);
                const int4* t4 = reinterpret_cast<const int4*>(s_ftile[jj]);
#pragma unroll 4
                for (int k4 = 0; k4 < F4 / 4; ++k4) {
                    const int4 v = v4[k4], t = t4[k4];
                    pin = max(pin, v.x == ps.f ? t.x : -1);  // one slot of a group holds the tile
                    pin = max(pin, v.y == ps.f ? t.y : -1);
                    pin = max(pin, v.z == ps.f ? t.z : -1);
                    pin = max(pin, v.w == ps.f ? t.w : -1);
                }
            }
        }
        s_pin[tid] = (short)pin;
        if (mine && pin >= 0 && !s_fail) {
            if (pin >= kPairRangeTiles) {
                atomicOr(&s_fail, 1);
            } else {
                atomicAdd(dup ? &s_pd[ps.r][pin] : &s_rs[ps.r][pin], 1);
                atomicMax(&s_maxpin[ps.r], pin);
            }
        }
        __syncthreads();
        // the slot's rank in its class: pinned rows by slot among their tile's,
        // unpinned duplicated features by slot, unpinned singles by residue key
        int rank = 0;
        if (mine && !s_fail) {
            const int key = (((ps.f - ps.r_lo) & 15) << 16) | (ps.f - ps.r_lo);
            const bool by_key = pin < 0 && !dup;
            auto count = [&](int k, int v, int fl, int pk) {
                const int kk = (((v - ps.r_lo) & 15) << 16) | (v - ps.r_lo);
                const bool same = (fl & 1) && v >= ps.r_lo && v < ps.r_lo + Dc &&
                                  ((fl & 2) != 0) == dup && pk == pin;
                rank += same && (by_key ? kk < key : k < tid);
            };
            const int4* v4 = reinterpret_cast<const int4*>(s_idx[j]);
            const int4* f4 = reinterpret_cast<const int4*>(s_flag[j]);
            const short4* p4 = reinterpret_cast<const short4*>(s_pin);
            const int F4 = (F + 3) & ~3;
#pragma unroll 4
            for (int k4 = 0; k4 < F4 / 4; ++k4) {
                const int4 v = v4[k4], fl = f4[k4];
                const short4 pk = p4[k4];
                count(4 * k4, v.x, fl.x, pk.x);
                count(4 * k4 + 1, v.y, fl.y, pk.y);
                count(4 * k4 + 2, v.z, fl.z, pk.z);
                count(4 * k4 + 3, v.w, fl.w, pk.w);
            }
        }
        if (tid < ndr && !s_fail) {
            int nt;
            pair_range_table(tid, s_c[0][tid], s_c[1][tid], s_maxpin[tid], s_pd[tid], s_rs[tid], s_tb, &nt);
            s_nt[tid] = nt;
            if (nt > kPairRangeTiles) atomicOr(&s_fail, 1);
        }
        __syncthreads();
        if (tid == 0 && !s_fail) {
            int t = 0;
            for (int rr = 0; rr < ndr; ++rr) {
                s_toff[rr] = t;
                t += s_nt[rr];
            }
            s_toff[ndr] = t;
            if (t > Tcap) s_fail = 1;
        }
        __syncthreads();
        if (s_fail) {  // (uniform) laid out on its own; past the window's first, the barrier kept
            int tr = -1;
            plan_keys(ps, F, Dc, s_idx[j], s_flag[j]);
            plan_in_tile(ps, g, F, ndr, Tcap, row_bytes, trash_row, j == 0 ? 0u : kMetaUnpaired, s_c,
                         s_toff, tfeat, tsrc, meta, &tr);
            s_ftile[j][tid] = mine ? tr : -1;
            __syncthreads();
            continue;
        }
        for (int rr = tid; rr < ndr; rr += 256) {
            int* m = meta + (g * ndr + rr) * kMetaStride;
            m[0] = s_toff[rr] | (s_toff[rr + 1] << 16);
            m[1] = s_toff[rr + 1];
        }
        const int64_t tbase = g * Tcap;
        s_ftile[j][tid] = -1;
        if (mine) {
            const int r = ps.r;
            int t, p;
            if (pin >= 0) {
                t = pin;
                p = dup ? 2 * rank : s_tb.base[r][t] + rank;
            } else if (dup) {
                t = 0;
                while (rank >= s_tb.ce[r][t]) ++t;  // rank < the range's unpinned dups <= ce[nt-1]
                p = s_pd[r][t] * 2 + 2 * (rank - s_tb.cb[r][t]);
            } else if (rank < s_tb.S[r][16]) {
                int k = 1;
                while (rank >= s_tb.S[r][k]) ++k;
                int i = rank - s_tb.S[r][k - 1];
                t = 0;
                for (;; ++t) {
                    if (s_tb.fr[r][t] >= k) {
                        if (i == 0) break;
                        --i;
                    }
                }
                p = 16 - s_tb.fr[r][t] + (k - 1);
            } else {
                const int q = rank - s_tb.S[r][16];
                t = s_tb.nt1[r] + q / 16;
                p = q % 16;
            }
            atomicAdd(&s_used[r][t], dup ? 2 : 1);
            s_ftile[j][tid] = t;
            const int64_t row0 = (tbase + s_toff[r] + t) * 16 + p;
            tfeat[row0] = (ps.f - ps.r_lo) * row_bytes;
            tsrc[row0] = (ps.rank << 10) | (ps.cnt << 1);
            if (dup) {
                tfeat[row0 + 1] = (ps.f - ps.r_lo) * row_bytes | 1;
                tsrc[row0 + 1] = (ps.rank << 10) | (ps.cnt << 1) | 1;
            }
        }
        __syncthreads();
        const int nslots = s_toff[ndr] * 16;
        for (int i = tid; i < nslots; i += 256) {
            const int t = i / 16, p = i % 16;
            int rr = 0;
            while (t >= s_toff[rr + 1]) ++rr;
            if (p < s_used[rr][t - s_toff[rr]]) continue;
            tfeat[(tbase + t) * 16 + p] = (trash_row + (p & (kTrashRows - 1))) * row_bytes;
            tsrc[(tbase + t) * 16 + p] = 0;
        }
        __syncthreads();
    }
}

// The plan of p: the staged build's in windows of groups, the others per group.
void launch_plan(const int32_t* idx, int* tfeat, int* tsrc, int* perm, int* meta, int64_t F,
                 int64_t D, const BwdFPlan& p, hipStream_t st) {
    if (p.staged)
        bwdf_plan_window_kernel<<<dim3((unsigned)ceil_div(p.Gc, (int64_t)kPlanWindow)), dim3(256), 0, st>>>(
            idx, tfeat, tsrc, perm, meta, (int)F, (int)D, (int)p.ndr, (int)p.Dc, (int)p.Tcap,
            acc_stride((int)p.BT) * 4, (int)p.DCMAX, p.Gc);
    else
        bwdf_plan_kernel<<<dim3((unsigned)p.Gc), dim3(256), 0, st>>>(
            idx, tfeat, tsrc, perm, meta, (int)F, (int)D, (int)p.ndr, (int)p.Dc, (int)p.Tcap,
            acc_stride((int)p.BT) * 4, (int)p.DCMAX);
}

// ------------------------------------------------------------- gather ------
// The SGD step that haste_sgd_sr_step_wt applies to W while gathering it: the
// update of haste_sgd_sr_step on the tensor W [O, F] (element offsets l*F + j
// from 0, the same FMA chain and Philox words), so W^T is built from the
// updated weights.
struct GatherSgd {
    const void* g;  // gradient [O, F], g_dtype
    float* m;       // fp32 momentum [O, F] (use_mom)
    int g_dtype, use_mom, do_sr;
    float lr, wd, mu;
    uint32_t k0, k1;
    uint16_t* bias;   // not NULL: also the SGD step on the bias [O] (offsets from 0)
    const void* gb;   // its gradient [O], gb_dtype
    float* mb;        // its fp32 momentum [O] (use_mom)
    int gb_dtype;
};

// haste_sgd_sr_step_wt: the SGD step of GatherSgd on W, then W^T of the updated
// weights as bwdf_gather_block_kernel writes it.  A workgroup takes kWtLabels labels
// (W rows) of one group: it updates those rows, stages them in LDS and writes
// their two 16-byte chunks of every W^T row of the group's tiles (the tiles are
// chunk-major, so a label block's chunks are contiguous runs of 512 bytes).
// Small workgroups keep the tail of the grid short and the occupancy high; the
// work is the Philox arithmetic of the SR words.  Rows >= O read as zeros
// through the buffer resources and are never written.
constexpr int kWtLabels = 16;
constexpr int kWtBatch = 2;  // chunks of 8 weights per thread (F <= 256)

template <int G, int GD>
__global__ __launch_bounds__(256) void sgd_wt_kernel(uint16_t* __restrict__ W,
                                                     const int* __restrict__ tsrc,
                                                     const int* __restrict__ perm,
                                                     uint16_t* __restrict__ twt, int F, int64_t O,
                                                     int Tcap, const int* __restrict__ meta,
                                                     int ndr, GatherSgd sg) {
    constexpr int NB = G / kWtLabels;  // workgroups per group
    constexpr int GB = GD == HASTE_DTYPE_F32 ? 4 : 2;  // gradient bytes per element
    __shared__ uint32_t s_w[kWtLabels * 129];  // kWtLabels rows of (F + 2) halves
    __shared__ int s_perm[256];
    const int64_t g = blockIdx.x / NB;
    const int h = (int)(blockIdx.x % NB);
    const int tid = threadIdx.x;
    const int ldw = F / 2 + 1;
    const int cpr = F / 8;  // chunks per row
    const int64_t l0 = g * G + h * kWtLabels;
    const int rows = (int)max<int64_t>(0, min<int64_t>(kWtLabels, O - l0));
    const int nch = rows * cpr;
    const int64_t e0 = l0 * F;
    const rsrc_t rw = make_rsrc_u32(W + e0, (uint32_t)(rows * F * 2));
    const rsrc_t rg = make_rsrc_u32(static_cast<const char*>(sg.g) + e0 * GB, (uint32_t)(rows * F * GB));
    const rsrc_t rm = make_rsrc_u32(sg.use_mom ? sg.m + e0 : sg.m, sg.use_mom ? (uint32_t)(rows * F * 4) : 0u);
    if (tid < F) s_perm[tid] = perm[g * F + tid];
    // the bias of the workgroup's labels, one per thread, as sgd_sr_kernel steps it
    if (sg.bias != nullptr && tid < rows) {
        const int64_t l = l0 + tid;
        const float gbv = sg.gb_dtype == HASTE_DTYPE_F32
                              ? static_cast<const float*>(sg.gb)[l]
                              : (sg.gb_dtype == HASTE_DTYPE_BF16
                                     ? bf16_bits_to_f32(static_cast<const uint16_t*>(sg.gb)[l])
                                     : f16_bits_to_f32(static_cast<const uint16_t*>(sg.gb)[l]));
        float mv = sg.use_mom ? sg.mb[l] : 0.f;
        sg.bias[l] = (uint16_t)sgd_one(bf16_bits_to_f32(sg.bias[l]), gbv, &mv, sg.use_mom, sg.lr,
                                       sg.wd, sg.mu, sg.do_sr, (uint64_t)l, sg.k0, sg.k1);
        if (sg.use_mom) sg.mb[l] = mv;
    }
    u32x4 wv[kWtBatch], gv0[kWtBatch], gv1[kWtBatch];
    f32x4 mv0[kWtBatch], mv1[kWtBatch];
#pragma unroll
    for (int b = 0; b < kWtBatch; ++b) {
        const int it = b * 256 + tid;
        const uint32_t c = (uint32_t)it;
        wv[b] = buf_load16(rw, it < nch ? c * 16u : kOOB);
        gv0[b] = buf_load16(rg, it < nch ? c * (8u * GB) : kOOB);
        if constexpr (GB == 4) gv1[b] = buf_load16(rg, it < nch ? c * 32u + 16u : kOOB);
        mv0[b] = __builtin_bit_cast(f32x4, buf_load16(rm, it < nch ? c * 32u : kOOB));
        mv1[b] = __builtin_bit_cast(f32x4, buf_load16(rm, it < nch ? c * 32u + 16u : kOOB));
    }
#pragma unroll
    for (int b = 0; b < kWtBatch; ++b) {
        const int it = b * 256 + tid;
        if (b * 256 >= kWtLabels * cpr) break;  // uniform: F <= 128 fills one pass
        const int l = it / cpr, j0 = (it % cpr) * 8;
        float gf[8];
        if constexpr (GB == 4) {
            const f32x4 a = __builtin_bit_cast(f32x4, gv0[b]), c = __builtin_bit_cast(f32x4, gv1[b]);
#pragma unroll
            for (int k = 0; k < 4; ++k) { gf[k] = a[k]; gf[4 + k] = c[k]; }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t lo = gv0[b][q] & 0xFFFFu, hi = gv0[b][q] >> 16;
                gf[2 * q] = GD == HASTE_DTYPE_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
                gf[2 * q + 1] = GD == HASTE_DTYPE_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
            }
        }
        float mv[8] = {mv0[b][0], mv0[b][1], mv0[b][2], mv0[b][3],
                       mv1[b][0], mv1[b][1], mv1[b][2], mv1[b][3]};
        const int64_t e = e0 + (int64_t)it * 8;
        uint32_t ob[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t w16 = (k & 1) ? (wv[b][k >> 1] >> 16) : (wv[b][k >> 1] & 0xFFFFu);
            ob[k] = sgd_one(bf16_bits_to_f32(w16), gf[k], &mv[k], sg.use_mom, sg.lr, sg.wd, sg.mu,
                            sg.do_sr, (uint64_t)(e + k), sg.k0, sg.k1);
        }
        const u32x4 v = u32x4{ob[0] | (ob[1] << 16), ob[2] | (ob[3] << 16), ob[4] | (ob[5] << 16),
                              ob[6] | (ob[7] << 16)};
        buf_store16(v, rw, it < nch ? (uint32_t)it * 16u : kOOB);
        if (sg.use_mom) {
            buf_store16(__builtin_bit_cast(u32x4, f32x4{mv[0], mv[1], mv[2], mv[3]}), rm,
                        it < nch ? (uint32_t)it * 32u : kOOB);
            buf_store16(__builtin_bit_cast(u32x4, f32x4{mv[4], mv[5], mv[6], mv[7]}), rm,
                        it < nch ? (uint32_t)it * 32u + 16u : kOOB);
        }
        if (l < kWtLabels) {  // rows >= O stage zeros
#pragma unroll
            for (int q = 0; q < 4; ++q) s_w[l * ldw + j0 / 2 + q] = it < nch ? v[q] : 0u;
        }
    }
    const int nrows = meta[(g * ndr + ndr - 1) * kMetaStride + 1] * 16;
    __syncthreads();
    const int lb = h * kWtLabels;
    auto wvf = [&](int l, int slot) -> uint32_t {
        const uint32_t w2 = s_w[(l - lb) * ldw + (slot >> 1)];
        return (slot & 1) ? (w2 >> 16) : (w2 & 0xFFFFu);
    };
    // per tile of 16 rows: chunk 2h of its rows, then chunk 2h + 1 (32 chunks, 512 bytes)
    for (int it = tid; it < nrows * 2; it += 256) {
        const int row = (it >> 5) * 16 + (it & 15);
        const int lc = lb + ((it >> 4) & 1) * 8;
        const u32x4 v = wt_chunk<BF16>(tsrc[(g * Tcap) * 16 + row], s_perm, wvf, lc);
        *reinterpret_cast<u32x4*>(twt + twt_elem((g * Tcap) * 16 + row, lc, G)) = v;
    }
}

// W^T of the current weights, in the label blocks of sgd_wt_kernel (no update):
// a workgroup loads kWtLabels rows of one group (8 KB of LDS at F = 256, so
// many workgroups share a CU and the loads of one overlap the stores of
// another) and writes their chunks of every W^T row of the group's tiles.
template <typename T, int G>
__global__ __launch_bounds__(256) void bwdf_gather_block_kernel(const uint16_t* __restrict__ W,
                                                                const int* __restrict__ tsrc,
                                                                const int* __restrict__ perm,
                                                                const int* __restrict__ meta,
                                                                uint16_t* __restrict__ twt, int F,
                                                                int64_t O, int ndr, int Tcap) {
    constexpr int NB = G / kWtLabels;  // workgroups per group
    __shared__ uint32_t s_w[kWtLabels * 129];  // kWtLabels rows of (F + 2) halves
    __shared__ int s_perm[256];
    const int64_t g = blockIdx.x / NB;
    const int h = (int)(blockIdx.x % NB);
    const int tid = threadIdx.x;
    const int ldw = F / 2 + 1;
    const int cpr = F / 8;  // chunks per row
    const int64_t l0 = g * G + h * kWtLabels;
    const int rows = (int)max<int64_t>(0, min<int64_t>(kWtLabels, O - l0));
    const int nch = rows * cpr;
    const rsrc_t rw = make_rsrc_u32(W + l0 * F, (uint32_t)(rows * F * 2));
    if (tid < F) s_perm[tid] = perm[g * F + tid];
    u32x4 wv[kWtBatch];
#pragma unroll
    for (int b = 0; b < kWtBatch; ++b) {
        const int it = b * 256 + tid;
        wv[b] = buf_load16(rw, it < nch ? (uint32_t)it * 16u : kOOB);  // rows >= O read zeros
    }
#pragma unroll
    for (int b = 0; b < kWtBatch; ++b) {
        const int it = b * 256 + tid;
        if (b * 256 >= kWtLabels * cpr) break;  // uniform: F <= 128 fills one pass
        const int l = it / cpr, j0 = (it % cpr) * 8;
        if (l < kWtLabels) {
#pragma unroll
            for (int q = 0; q < 4; ++q) s_w[l * ldw + j0 / 2 + q] = wv[b][q];
        }
    }
    const int nrows = meta[(g * ndr + ndr - 1) * kMetaStride + 1] * 16;
    __syncthreads();
    const int lb = h * kWtLabels;
    auto wvf = [&](int l, int slot) -> uint32_t {
        const uint32_t w2 = s_w[(l - lb) * ldw + (slot >> 1)];
        return (slot & 1) ? (w2 >> 16) : (w2 & 0xFFFFu);
    };
    // per tile of 16 rows: chunk 2h of its rows, then chunk 2h + 1 (32 chunks, 512 bytes)
    for (int it = tid; it < nrows * 2; it += 256) {
        const int row = (it >> 5) * 16 + (it & 15);
        const int lc = lb + ((it >> 4) & 1) * 8;
        const u32x4 v = wt_chunk<T>(tsrc[(g * Tcap) * 16 + row], s_perm, wvf, lc);
        *reinterpret_cast<u32x4*>(twt + twt_elem((g * Tcap) * 16 + row, lc, G)) = v;
    }
}

// ------------------------------------------------------------- reduce ------
// Both reduce kernels read the partials as 16-byte rows of 4 batch columns
// (Bp is a multiple of 64, so every such read is in bounds and aligned).
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
__global__ __launch_bounds__(256) void bwdf_reduce_sr_kernel(ReduceJob job) {
    __shared__ float t[32][33];
    reduce_sr_tile(job, blockIdx.x, t);
}

// Checks the arguments and the workspace size; returns the plan.
int check_bwdf(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
               int32_t dtype, const void* workspace, int64_t workspace_bytes, BwdFPlan* out) {
    int rc = check_ffi_shape(fn, B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    const BwdFPlan p = make_plan(B, D, F, O, G);
    if (p.ndr > kMaxRanges) {
        set_error("%s: D = %lld is too large (at most %lld features)", fn, (long long)D,
                  (long long)kMaxRanges * p.DCMAX);
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
    // rows that all start on 16-byte boundaries take the plain build, any other
    // rows the YA build (which needs O >= 16)
    const bool ya = lddy % 8 != 0 || !aligned16(dY);
    HASTE_CHECK_ARG(lddy >= O && (!ya || O >= 16),
                    "%s: lddy must be >= O, and dY's rows must start on 16-byte boundaries "
                    "when O < 16 (lddy=%lld O=%lld)", fn, (long long)lddy, (long long)O);
    HASTE_CHECK_ARG(aligned16(W) && (reinterpret_cast<uintptr_t>(dY) & 1) == 0,
                    "%s: W must be 16-byte aligned and dY 2-byte aligned", fn);
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
    const dim3 ggrid((unsigned)(p.Gc * (G / kWtLabels)));  // label blocks of the W^T gather
    if (!plan_ready) {
        launch_plan(idx, tfeat, tsrc, perm, meta, F, D, p, st);
        HASTE_CHECK_LAUNCH(fn);
    }
    const bool gather = plan_ready != 2;
    switch (G) {
#define HASTE_BWDF_G(GG)                                                                        \
    case GG:                                                                                    \
        if (dtype == HASTE_DTYPE_BF16) {                                                        \
            if (gather) {                                                                       \
                bwdf_gather_block_kernel<BF16, GG><<<ggrid, dim3(256), 0, st>>>( \
                    w, tsrc, perm, meta, twt, (int)F, O, (int)p.ndr, (int)p.Tcap); \
                HASTE_CHECK_LAUNCH(fn);                                                         \
            }                                                                                   \
            rc = p.staged ? bwdf_run_staged(dtype, G, ya, tfeat, meta, twt, y, lddy, ws, p, B, D, O, st) \
                 : ya ? bwdf_run_main_ya(dtype, G, tfeat, meta, twt, y, lddy, ws, p, B, D, F, O, st)  \
                      : run_main<BF16, GG, false>(tfeat, meta, twt, y, lddy, ws, p, B, D, F, O, st); \
        } else {                                                                                \
            if (gather) {                                                                       \
                bwdf_gather_block_kernel<F16, GG><<<ggrid, dim3(256), 0, st>>>( \
                    w, tsrc, perm, meta, twt, (int)F, O, (int)p.ndr, (int)p.Tcap); \
                HASTE_CHECK_LAUNCH(fn);                                                         \
            }                                                                                   \
            rc = p.staged ? bwdf_run_staged(dtype, G, ya, tfeat, meta, twt, y, lddy, ws, p, B, D, O, st) \
                 : ya ? bwdf_run_main_ya(dtype, G, tfeat, meta, twt, y, lddy, ws, p, B, D, F, O, st)  \
                      : run_main<F16, GG, false>(tfeat, meta, twt, y, lddy, ws, p, B, D, F, O, st);  \
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

extern "C" int haste_ffi_bwd_features_config(int64_t B, int64_t D, int64_t F, int64_t O,
                                             int64_t G, int32_t dtype, int64_t* cfg) {
    int rc = haste::check_ffi_shape("haste_ffi_bwd_features_config", B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(cfg != nullptr, "haste_ffi_bwd_features_config: null pointer");
    const haste::BwdFPlan p = haste::make_plan(B, D, F, O, G);
    cfg[0] = p.BT;
    cfg[1] = p.RT;
    cfg[2] = p.ndr;
    cfg[3] = p.S;
    return HASTE_OK;
}

namespace haste {
static std::atomic<int> g_bwdf_build{0};
int bwdf_build() { return g_bwdf_build.load(std::memory_order_relaxed); }
}  // namespace haste

extern "C" int haste_ffi_bwd_features_set_build(int32_t build) {
    HASTE_CHECK_ARG(build >= 0 && build <= 3,
                    "haste_ffi_bwd_features_set_build: build must be 0, 1, 2 or 3 (got %d)", (int)build);
    return haste::g_bwdf_build.exchange(build);
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
    haste::launch_plan(idx, reinterpret_cast<int*>(base + p.tfeat_off),
                       reinterpret_cast<int*>(base + p.tsrc_off),
                       reinterpret_cast<int*>(base + p.perm_off),
                       reinterpret_cast<int*>(base + p.meta_off), F, D, p,
                       static_cast<hipStream_t>(stream));
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
    const haste::ReduceJob job = haste::reduce_job(p, ws, dX, B, D, seed);
    haste::bwdf_reduce_sr_kernel<<<dim3((unsigned)job.ntiles), dim3(256), 0, st>>>(job);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features_sr");
    return HASTE_OK;
}

extern "C" int haste_ffi_bwd_features_partials(const int32_t* idx, const void* W, const void* dY,
                                               int64_t lddy, void* workspace,
                                               int64_t workspace_bytes, int64_t B, int64_t D,
                                               int64_t F, int64_t O, int64_t G, int32_t dtype,
                                               int32_t plan_ready, void* stream) {
    haste::BwdFPlan p;
    return haste::run_partials("haste_ffi_bwd_features_partials", idx, W, dY, lddy, workspace,
                               workspace_bytes, B, D, F, O, G, dtype, plan_ready,
                               static_cast<hipStream_t>(stream), &p);
}

namespace haste {
namespace {
int sgd_step_wt(const char* fn, uint16_t* W, const void* g, int32_t g_dtype, float* m,
                uint16_t* bias, const void* gb, int32_t gb_dtype, float* m_bias, float lr,
                float wd, float mu, int32_t use_mom, int32_t do_sr, uint64_t seed,
                void* workspace, int64_t workspace_bytes, int64_t B, int64_t D, int64_t F,
                int64_t O, int64_t G, int32_t dtype, void* stream) {
    BwdFPlan p;
    int rc = check_bwdf(fn, B, D, F, O, G, dtype, workspace, workspace_bytes, &p);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(dtype == HASTE_DTYPE_BF16, "%s: weights must be bf16", fn);
    HASTE_CHECK_ARG(W && g && aligned16(W) && aligned16(g),
                    "%s: W and g must be 16-byte aligned pointers", fn);
    HASTE_CHECK_ARG(g_dtype == HASTE_DTYPE_BF16 || g_dtype == HASTE_DTYPE_F16 ||
                        g_dtype == HASTE_DTYPE_F32,
                    "%s: bad gradient dtype %d", fn, (int)g_dtype);
    HASTE_CHECK_ARG(!use_mom || (m != nullptr && aligned16(m)),
                    "%s: momentum buffer must be a 16-byte aligned pointer", fn);
    if (bias != nullptr) {
        HASTE_CHECK_ARG(gb != nullptr && (!use_mom || m_bias != nullptr),
                        "%s: the bias needs its gradient (and momentum buffer)", fn);
        HASTE_CHECK_ARG(gb_dtype == HASTE_DTYPE_BF16 || gb_dtype == HASTE_DTYPE_F16 ||
                            gb_dtype == HASTE_DTYPE_F32,
                        "%s: bad bias gradient dtype %d", fn, (int)gb_dtype);
    }
    char* base = static_cast<char*>(workspace);
    const GatherSgd sg{g, m, (int)g_dtype, use_mom ? 1 : 0, do_sr ? 1 : 0, lr, wd, mu,
                       (uint32_t)seed, (uint32_t)(seed >> 32), bias, gb, m_bias, (int)gb_dtype};
    const int* tsrc = reinterpret_cast<const int*>(base + p.tsrc_off);
    const int* perm = reinterpret_cast<const int*>(base + p.perm_off);
    const int* meta = reinterpret_cast<const int*>(base + p.meta_off);
    uint16_t* twt = reinterpret_cast<uint16_t*>(base + p.twt_off);
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto launch = [&](auto gc) {
        constexpr int GG = decltype(gc)::value;
        const dim3 grid((unsigned)(p.Gc * (GG / kWtLabels)));
#define HASTE_SGD_WT(GD)                                                                    \
    sgd_wt_kernel<GG, GD><<<grid, dim3(256), 0, st>>>(W, tsrc, perm, twt, (int)F, O,        \
                                                      (int)p.Tcap, meta, (int)p.ndr, sg)
        if (g_dtype == HASTE_DTYPE_F32) HASTE_SGD_WT(HASTE_DTYPE_F32);
        else if (g_dtype == HASTE_DTYPE_BF16) HASTE_SGD_WT(HASTE_DTYPE_BF16);
        else HASTE_SGD_WT(HASTE_DTYPE_F16);
#undef HASTE_SGD_WT
    };
    switch (G) {
    case 16: launch(std::integral_constant<int, 16>{}); break;
    case 32: launch(std::integral_constant<int, 32>{}); break;
    case 64: launch(std::integral_constant<int, 64>{}); break;
    case 128: launch(std::integral_constant<int, 128>{}); break;
    default:
        set_error("%s: unsupported group size %lld", fn, (long long)G);
        return HASTE_ERR_UNSUPPORTED;
    }
    HASTE_CHECK_LAUNCH(fn);
    return HASTE_OK;
}
}  // namespace
}  // namespace haste

extern "C" int haste_sgd_sr_step_wt(uint16_t* W, const void* g, int32_t g_dtype, float* m,
                                    float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                                    uint64_t seed, void* workspace, int64_t workspace_bytes,
                                    int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                                    int32_t dtype, void* stream) {
    return haste::sgd_step_wt("haste_sgd_sr_step_wt", W, g, g_dtype, m, nullptr, nullptr,
                              HASTE_DTYPE_F32, nullptr, lr, wd, mu, use_mom, do_sr, seed,
                              workspace, workspace_bytes, B, D, F, O, G, dtype, stream);
}

extern "C" int haste_sgd_sr_step_wt_bias(uint16_t* W, const void* g, int32_t g_dtype, float* m,
                                         uint16_t* bias, const void* gb, int32_t gb_dtype,
                                         float* m_bias, float lr, float wd, float mu,
                                         int32_t use_mom, int32_t do_sr, uint64_t seed,
                                         void* workspace, int64_t workspace_bytes, int64_t B,
                                         int64_t D, int64_t F, int64_t O, int64_t G,
                                         int32_t dtype, void* stream) {
    const char* fn = "haste_sgd_sr_step_wt_bias";
    HASTE_CHECK_ARG(bias != nullptr, "%s: null bias", fn);
    return haste::sgd_step_wt(fn, W, g, g_dtype, m, bias, gb, gb_dtype, m_bias, lr, wd, mu,
                              use_mom, do_sr, seed, workspace, workspace_bytes, B, D, F, O, G,
                              dtype, stream);
}
