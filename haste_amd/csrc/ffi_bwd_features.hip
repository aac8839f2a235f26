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

#include <type_traits>

#include "bwdf_plan.hpp"


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
// to g*Tcap); meta[(g*ndr + ndr-1)*2 + 1] is the group's tile count.  For tile row
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
    const int nrows = meta[(g * ndr + ndr - 1) * kMetaStride + 1] * 16;
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
// A workgroup owns (group slice s, feature range r, batch tile of BT = 16*WAVES
// columns) and keeps dXT[range, tile] as an fp32 partial in LDS.  Wave w owns
// batch rows [16w, 16w+16) of the tile, so no two waves touch the same LDS
// word of the partial.  Per group:
//  - the group's W^T tiles for the range (and the partial-row offsets of their
//    positions) are staged once into a double-buffered LDS ring, shared by all
//    waves: each thread copies 16-byte chunks loaded two groups ahead;
//  - each wave multiplies its dY rows (16 x G, loaded one group ahead) with
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
template <int G, int WAVES, int RT_>
struct BwdFCfg {
    static constexpr int KS = G >= 32 ? G / 32 : 1;  // MFMA k-steps over labels
    static constexpr int BT = 16 * WAVES;            // batch columns per workgroup
    static constexpr int AS = acc_stride(BT);
    static constexpr int RT = RT_;
    static constexpr int RB = ring_row_bytes(G);
    static constexpr int RING = RT * 16 * RB;        // bytes per ring buffer
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int CH = G / 8;                 // 16-byte chunks per W^T row
    static constexpr int SPT = (RT * 16 * CH + THREADS - 1) / THREADS;  // staged chunks per thread
    static constexpr int DCMAX = max_dc(BT, G, RT);
    static_assert(DCMAX > 0, "LDS budget");
};

template <typename T, int G, int WAVES, int RT_>
__global__ __launch_bounds__(64 * WAVES, 1) void bwdf_main_kernel(
    const int* __restrict__ tfeat, const int* __restrict__ meta, const uint16_t* __restrict__ twt,
    const uint16_t* __restrict__ dY, int64_t lddy, float* __restrict__ ws, int B, int Bp, int D,
    int64_t O, int64_t Gc, int nbt, int ndr, int Dc, int gps, int S, int Tcap, int yshort) {
    using C = BwdFCfg<G, WAVES, RT_>;
    constexpr int KS = C::KS, BT = C::BT, AS = C::AS, RT = C::RT, RB = C::RB, CH = C::CH;
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
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15;  // A row within the M tile / B column (tile position)
    const int kq = lane >> 4;   // which 8 of the 32 K elements
    const bool kq_ok = G >= 32 || kq < 2;
    const int kofs = kq_ok ? kq * 8 : 0;
    const int trash_f = (C::DCMAX + (col & (kTrashRows - 1))) * AS * 4;

    for (int i = tid * 4; i < dn * AS; i += NTH * 4)
        *reinterpret_cast<f32x4*>(&acc[i]) = f32x4{0.f, 0.f, 0.f, 0.f};

    // dY of this lane's row (rows >= B read as zero; labels >= O are masked at
    // use).  A row is read up to the 8-label piece boundary past O: inside the
    // row when lddy >= O is a multiple of 8, else inside the next row.  dY's
    // last row may end at label O (yshort): there the resource ends at O and
    // the piece that straddles O is loaded early and shifted back
    // (shift_down16; O >= 8 keeps the early load inside the resource).
    const int b0 = bt * BT;
    const int rows = min(BT, B - b0);
    const rsrc_t yr = make_rsrc(dY + (int64_t)b0 * lddy,
                                ((int64_t)(rows - 1) * lddy +
                                 ((yshort && b0 + rows == B) ? O : (O + 7) / 8 * 8)) * 2);
    // elements the lane's piece ks of group g is loaded early by: 0 unless it
    // straddles O in dY's last row (then g is the last group)
    int sh_last[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int64_t over = (Gc - 1) * G + kofs + ks * 32 + 8 - O;
        sh_last[ks] = (yshort && b0 + wave * 16 + col == B - 1 && over > 0 && over < 8) ? (int)over : 0;
    }
    auto tail_shift = [&](int64_t g, int ks) __attribute__((always_inline)) -> int {
        return g == Gc - 1 ? sh_last[ks] : 0;
    };
    // byte offset of the lane's first label in the tile (32 bits: the tile's
    // resource spans at most kMaxRsrcBytes; g * G * 2 < 2 * lddy for real groups)
    const uint32_t yoff2 = (uint32_t)(((int64_t)(wave * 16 + col) * lddy + kofs) * 2);
    auto load_y = [&](int64_t g, u32x4 (&a)[KS]) __attribute__((always_inline)) {
        const uint32_t go = (uint32_t)g * (uint32_t)(G * 2);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            a[ks] = buf_load16(yr, kq_ok ? yoff2 + go + ks * 64 - 2 * tail_shift(g, ks) : kOOB);
    };
    // labels >= O read as zero: only the last group has any (a uniform branch)
    auto mask_y = [&](int64_t g, u32x4 (&a)[KS]) __attribute__((always_inline)) {
        const int64_t rem = O - g * G;  // labels of group g below O
        if (rem >= G) return;
        const int nr = (int)max<int64_t>(rem, 0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int sh = tail_shift(g, ks);
            if (sh) a[ks] = shift_down16(a[ks], sh);
            const int nv = nr - (ks * 32 + kofs);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                a[ks][e] &= (2 * e + 1 < nv) ? 0xFFFFFFFFu : (2 * e < nv ? 0xFFFFu : 0u);
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
        st.f = (int)buf_load4(fr, tid < RT * 16 ? (uint32_t)tid * 4 : kOOB);
    };
    auto store_stage = [&](int buf, const Stage& st, u32x2 m, int t0) __attribute__((always_inline)) {
        const int tb = (int)(m[0] & 0xFFFF) + t0;
        const int nt = max(0, min(RT, (int)m[1] - tb));  // tiles of this round
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            const int c = tid + k * NTH;
            if (c < RT * 16 * CH)
                *reinterpret_cast<u32x4*>(&ring[buf][(c / CH) * RB + (c % CH) * 16]) = st.w[k];
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
    char* const acc_b = reinterpret_cast<char*>(acc) + perm_col(wave, kq) * 4;
    // A round is up to RT staged tiles of one group.  Its MFMAs run on all RT
    // ring tiles (rows past the round's tiles are zero) and the products stay
    // in registers; the partial update (read, add, write) of a round runs in
    // the next iteration, in the same code as the next round's MFMAs, so the
    // products' latency and the update's LDS traffic overlap the next group.
    struct Round {
        f32x4 c[RT];  // dY rows x W^T tile t
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
    auto mma_round = [&](const u32x4 (&a)[KS], const u32x4 (&bf)[RT][KS], Round& r) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) v = mfma16x16x32<T>(a[ks], bf[t][ks], v);
            r.c[t] = v;
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
        f32x4 old[N0 > 0 ? N0 : 1];
#pragma unroll
        for (int t = 0; t < N0; ++t) old[t] = *reinterpret_cast<const f32x4*>(acc_b + pr.f[t]);
        mma();
#pragma unroll
        for (int t = 0; t < N0; ++t) {
            f32x4 v = pr.c[t];
            if (N0 + t < RT) v += pr.c[N0 + t];
            *reinterpret_cast<f32x4*>(acc_b + pr.f[t]) = old[t] + v;
        }
        // every LDS op of the wave but the N0 writes has completed
        __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(N0));
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
        f32x4 old[NTL > 0 ? NTL : 1];
        int fa[NTL > 0 ? NTL : 1];
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
            fa[t] = t < pr.n0 ? pr.f[t] : trash_f;
            old[t] = *reinterpret_cast<const f32x4*>(acc_b + fa[t]);
        }
        mma();
#pragma unroll
        for (int t = 0; t < NTL; ++t) *reinterpret_cast<f32x4*>(acc_b + fa[t]) = old[t] + pr.c[t];
        if (pr.n0 < NTL) {
#pragma unroll
            for (int t = 0; t < NTL; ++t) {
                fa[t] = t >= pr.n0 ? pr.f[t] : trash_f;
                old[t] = *reinterpret_cast<const f32x4*>(acc_b + fa[t]);
            }
#pragma unroll
            for (int t = 0; t < NTL; ++t) *reinterpret_cast<f32x4*>(acc_b + fa[t]) = old[t] + pr.c[t];
        }
        // every LDS op of the wave but the last pass's NTL writes has completed
        __builtin_amdgcn_s_waitcnt(wait_lgkmcnt(NTL));
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
    auto extra_rounds = [&](int i, u32x2 m, int buf, const u32x4 (&a)[KS]) __attribute__((always_inline)) {
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
    u32x4 ya[NS][KS];
    u32x2 mraw[NS];
    u32x2 mu[DEPTH + 1];  // uniform meta of groups i .. i+DEPTH
    Round rd[2];          // round of group i in rd[i % 2]
    rd[0].nt = rd[1].nt = 0;
    rd[0].n0 = rd[1].n0 = 0;
    {
        u32x2 m0[DEPTH + 1];
#pragma unroll
        for (int k = 0; k <= DEPTH; ++k) m0[k] = load_meta(k);
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
            load_y(g_lo + k - 1, ya[(k - 1) % NS]);
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
        load_y(g_lo + i + DEPTH, ya[(Q + DEPTH) % NS]);
        mraw[(Q + 1 + 2 * DEPTH) % NS] = load_meta(i + 1 + 2 * DEPTH);
        store_stage(1 - P, stg[(Q + 1) % NS], mu[1], 0);
        mask_y(g_lo + i, ya[Q]);
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

template <typename T, int G, int WAVES, int RT>
int launch_main(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
                hipStream_t st) {
    const int64_t nlog = p.S * p.ndr * p.nbt;
    const int64_t grid = 8 * ceil_div(nlog, 8);
    if (((int64_t)p.BT * lddy + 8) * 2 > kMaxRsrcBytes) {
        set_error("haste_ffi_bwd_features: lddy = %lld too large", (long long)lddy);
        return HASTE_ERR_UNSUPPORTED;
    }
    bwdf_main_kernel<T, G, WAVES, RT><<<dim3((unsigned)grid), dim3(64 * WAVES), 0, st>>>(
        tfeat, meta, twt, dY, lddy, ws, (int)B, (int)p.Bp, (int)D, O, p.Gc, (int)p.nbt,
        (int)p.ndr, (int)p.Dc, (int)p.gps, (int)p.S, (int)p.Tcap, lddy % 8 != 0);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_features");
    return HASTE_OK;
}

// the plan's ring size: 2, 3 or ring_tiles(G) tiles
template <typename T, int G, int WAVES>
int launch_ring(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
                int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t O,
                hipStream_t st) {
    constexpr int R = ring_tiles(G);
    if (p.RT == 2) return launch_main<T, G, WAVES, 2>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
    if constexpr (R > 3) {
        if (p.RT == 3) return launch_main<T, G, WAVES, 3>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
    }
    return launch_main<T, G, WAVES, R>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
}

template <typename T, int G>
int run_main(const int* tfeat, const int* meta, const uint16_t* twt, const uint16_t* dY,
             int64_t lddy, float* ws, const BwdFPlan& p, int64_t B, int64_t D, int64_t F,
             int64_t O, hipStream_t st) {
    (void)F;
    if (p.BT == 64) return launch_ring<T, G, 4>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
    return launch_ring<T, G, 8>(tfeat, meta, twt, dY, lddy, ws, p, B, D, O, st);
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
    HASTE_CHECK_ARG(lddy >= O && (lddy % 8 == 0 || O >= 8),
                    "%s: lddy must be >= O, and a multiple of 8 when O < 8 (lddy=%lld O=%lld)",
                    fn, (long long)lddy, (long long)O);
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
    const dim3 pgrid((unsigned)p.Gc);
    if (!plan_ready) {
        bwdf_plan_kernel<<<pgrid, dim3(256), 0, st>>>(
            idx, tfeat, tsrc, perm, meta, (int)F, (int)D, (int)p.ndr, (int)p.Dc, (int)p.Tcap,
            acc_stride((int)p.BT) * 4, (int)p.DCMAX);
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
        (int)p.DCMAX);
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
