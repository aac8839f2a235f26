#pragma once
// Grouped fixed-fan-in backward to weights (+ bias gradient), gfx950, optionally
// fused with the SR-SGD update of the weights and bias: the kernel and its
// launch templates, instantiated by ffi_bwd_weights.hip (dY rows of any
// length at a stride that is a multiple of 8) and ffi_bwd_weights_ys.hip (any
// other stride: the last row of dY may end at label O).
//
//   dW[l, j] = sum_b dY[b, l] * xT[idx[g, j], b]        g = l / G
//   dbias[l] = sum_b dY[b, l]
//
// One workgroup per label group; the contraction runs over the whole batch.
// MFMA orientation: M = fan-in slots, N = labels, K = batch.
//  - A (slots x batch): the gathered rows xT[idx[g, j], chunk] are copied
//    row-major into LDS (one 128-byte line per slot and 64-row chunk, eight
//    lines per load instruction) and read back as fragments of 8 consecutive
//    batch entries (ds_read_b128); loaded in MFMA fragment order instead, every
//    instruction touches 16 lines, each half used.  At G = 128, and at G = 64
//    with F = 128, a fragment comes straight from L2 (one 16-byte load of row
//    xT[idx[g, j]]; see BwdWCfg::XS).
//  - B (batch x labels) is dY[b, g*G:(g+1)*G], copied row-major into LDS in
//    chunks of 64 batch rows (double-buffered, the chunk after next in flight
//    in registers) and read back with ds_read_b64_tr_b16, which hands each lane
//    4 consecutive batch values of one label: dY needs no transposition pass.
//  - Every load of the batch loop is a raw buffer access (rows past B, labels
//    past O and slots past F read as zero by the hardware's range check), so
//    the loop has no branches around memory operations.
//  - The bias gradient is one extra MFMA per label tile with A = ones, so dY is
//    read once for both outputs (the reference reads it a second time for
//    torch.sum, shared_ffi/bindings.py:40).
//  - Epilogue: the fp32 gradient tile is staged in LDS and processed as whole
//    rows, 8 consecutive slots per thread: it is stored (fp32 or RNE 16-bit)
//    and/or, in the fused mode, applied to W in place by the SGD step of
//    haste_sgd_sr_step (same FMA chain, same Philox offsets l*F + j for W and l
//    for the bias), so the fp32 gradient need not make a round trip to HBM.
#include <algorithm>
#include <type_traits>

#include "bwdf_plan.hpp"

namespace haste {
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype);

// Parameters of the fused SGD epilogue (unused when SGD == false; rj is used in
// either mode).  twt != NULL:
// also write W^T of the updated weights into the bwd-features workspace
// (tsrc / perm / meta of its plan, Tcap tile rows per group).
struct SgdArgs {
    uint16_t* W;
    uint16_t* bias;
    float* mW;
    float* mb;
    float lr, wd, mu;
    int use_mom, do_sr;
    uint32_t k0, k1;
    uint16_t* twt;
    const int* tsrc;
    const int* perm;
    const int* meta;
    int ndr, Tcap;
    ReduceJob rj;  // ntiles > 0: workgroups Gc .. Gc + ntiles - 1 run this job's tiles
    const uint64_t* seed_dev;  // not NULL: the Philox seed is read here (k0, k1 unused)
};

namespace {

constexpr int kThreads = 256;
constexpr int kStgBytes = 34 * 1024;  // LDS for one pass of the staged gradient tile

template <int G, int FP>
struct BwdWCfg {
    // batch rows per LDS stage: 32 at G = 32, F = 256, whose smaller stages then
    // fit four workgroups per CU (LDS and registers), else 64
    static constexpr int KC = (G == 32 && FP == 256) ? 32 : 64;
    static constexpr int MTILES = FP / 16;                    // slot tiles
    static constexpr int NTILES = G / 16;                     // label tiles
    static constexpr int WM = MTILES < 4 ? MTILES : 4;        // waves along slots
    static constexpr int WN0 = 4 / WM;
    static constexpr int WN = NTILES < WN0 ? NTILES : WN0;    // waves along labels
    static constexpr int MT = MTILES / WM;
    static constexpr int NT = NTILES / WN;
    static constexpr int RB = 2 * G + 16;                     // LDS bytes per staged dY row
    static constexpr int PIECES = KC * G / 8;                // 16-byte pieces per chunk
    static constexpr int PPT = (PIECES + kThreads - 1) / kThreads;
    static constexpr int SP = FP + 4;                         // staged gradient row (floats)
    static constexpr int PR0 = kStgBytes / (SP * 4) / 16 * 16;
    static constexpr int PR = PR0 < G ? PR0 : G;              // labels per epilogue pass
    static constexpr int YS_BYTES = 2 * KC * RB;
    // X^T staged through LDS: measured 487 -> 467 us at config 3 (G = 32,
    // F = 256) and 212 -> 209 at config 2 (G = 64, F = 64); unchanged at config 1
    // (G = 64, F = 128, whose four waves per SIMD leave 128 registers: the
    // staging there spilled one), and 2132 -> 2164 at config 4 (G = 128).  Those
    // two keep the fragment loads.
    static constexpr bool XS = G <= 64 && !(G == 64 && FP == 128);
    static constexpr int RBX = KC * 2 + 16;                  // LDS bytes per staged X^T row
    static constexpr int XS_BYTES = XS ? FP * RBX : 0;        // one chunk of the gathered rows
    static constexpr int PPTX = FP * (KC / 8) / kThreads;    // X^T pieces per thread
    static constexpr int STG_BYTES = PR * SP * 4;
    static constexpr int LDS_BYTES = YS_BYTES + XS_BYTES > STG_BYTES ? YS_BYTES + XS_BYTES : STG_BYTES;
    static constexpr int CPR = FP / 8;                        // 8-slot chunks per staged row
    static constexpr int WPT = (PR * CPR + kThreads - 1) / kThreads;  // chunks per thread, pass 0
    static_assert(PR >= 16 && G % PR == 0, "epilogue pass shape");
    static_assert(PPTX >= 1 && FP * (KC / 8) % kThreads == 0, "X^T pieces");
};

template <typename T>
__device__ __forceinline__ uint32_t one_pair();
template <>
__device__ __forceinline__ uint32_t one_pair<BF16>() { return 0x3F803F80u; }
template <>
__device__ __forceinline__ uint32_t one_pair<F16>() { return 0x3C003C00u; }

// Keep the first nv 16-bit elements of an 8-element fragment (nv >= 8: all).
__device__ __forceinline__ u32x4 keep_first(u32x4 v, int nv) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] &= (2 * e + 1 < nv) ? 0xFFFFFFFFu : (2 * e < nv ? 0xFFFFu : 0u);
    return v;
}



// Two waves per SIMD (at most 256 registers each) hide the chunk pipeline's load
// latency; the largest tile set (G = 128, 256 slots) needs more registers.  At
// G = 64, FP = 128 four fit (the fused update then loads W in its epilogue):
// the 2049 groups of a 131K-label layer run in two rounds of 1024, not three
// of 768.
template <int G, int FP>
constexpr int bwdw_waves_per_simd() {
    return (G == 64 && FP == 128) || (G == 32 && FP == 256) ? 4 : G * FP >= 128 * 256 ? 1 : 2;
}

// dY larger than the last-level cache (kMallBytes): this kernel, its last
// reader in a training step, streams it with non-temporal loads (YNT), so it
// does not evict the weights that the next step's forward reads.
constexpr int kLoadNT = 2;  // buffer-load cache policy: nt on gfx950

template <typename T, int G, int FP, bool SGD, bool YNT, bool YS>
__global__ __launch_bounds__(kThreads, (bwdw_waves_per_simd<G, FP>())) void ffi_bwd_w_kernel(
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ xT, int64_t ldx,
    const uint16_t* __restrict__ dY, int64_t lddy, void* __restrict__ dW, int dW_dtype,
    void* __restrict__ dbias, int dbias_dtype, int B, int D, int F, int64_t O, SgdArgs sg) {
    constexpr bool yshort = YS;
    using C = BwdWCfg<G, FP>;
    constexpr int MT = C::MT, NT = C::NT, RB = C::RB, PPT = C::PPT, SP = C::SP, PR = C::PR;
    constexpr bool XS = C::XS;
    constexpr int RBX = C::RBX, PPTX = XS ? C::PPTX : 1, KC = C::KC, KSC = KC / 32;
    __shared__ __attribute__((aligned(16))) char lds[C::LDS_BYTES];
    __shared__ int s_perm[SGD ? FP : 1];
    __shared__ float s_bg[SGD ? G : 1];  // fused step: the bias gradient of the group
    char (*Ys)[KC * RB] = reinterpret_cast<char (*)[KC * RB]>(lds);
    char* Xs = lds + C::YS_BYTES;
    float* stg = reinterpret_cast<float*>(lds);

    // the last group (partial when O % G != 0, the shortest workgroup) is
    // dispatched first: with Gc = 8k + 1 groups, XCD 0 holds one workgroup
    // more than the others, and it is then that one
    const int64_t Gc = (O + G - 1) / G;
    if (blockIdx.x >= Gc) {  // the reduce job's tiles (sg.rj.ntiles > 0)
        reduce_sr_tile(sg.rj, (int)(blockIdx.x - Gc), reinterpret_cast<float (*)[33]>(lds));
        return;
    }
    const int64_t g = blockIdx.x == 0 ? Gc - 1 : (int64_t)blockIdx.x - 1;
    const int tid = threadIdx.x;
    // the SGD step's Philox key: the launch's seed, or the device-side seed
    uint32_t sk0 = sg.k0, sk1 = sg.k1;
    if constexpr (SGD) {
        if (sg.seed_dev != nullptr) {
            const uint64_t s = *sg.seed_dev;
            sk0 = (uint32_t)s;
            sk1 = (uint32_t)(s >> 32);
        }
    }
    // the wave index as a scalar: branches on wm / wn / active are then scalar
    // branches that skip their MFMAs (an MFMA under an EXEC mask still runs and
    // writes every lane)
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % C::WM, wn = wave / C::WM;
    const bool active = wn < C::WN;
    const int col = lane & 15, kq = lane >> 4;
    const int64_t l0 = g * G;
    const int nl = (int)std::min<int64_t>(G, O - l0);  // labels of this group
    const int nchunks = (B + KC - 1) / KC;

    // Gathered rows (indices outside [0, D) are clamped).  XS: a chunk row is
    // XPR pieces of 8 batch entries; piece tid + q*256 of a chunk is slot
    // tid/XPR + q*256/XPR, batch entries xbc .. xbc+7 of the chunk; xrow = byte
    // offset of the slot's row, kOOB for slots >= F.  Otherwise: the lane's A
    // rows (slots >= F, and inactive waves, read as zero).
    constexpr int XPR = KC / 8;
    const rsrc_t xr = make_rsrc(xT, (int64_t)D * ldx * 2);
    const int xbc = (tid % XPR) * 8;
    uint32_t xrow[PPTX];
    int64_t xoff[XS ? 1 : MT];
    bool jvalid[XS ? 1 : MT];
    if constexpr (XS) {
#pragma unroll
        for (int q = 0; q < PPTX; ++q) {
            const int j = tid / XPR + q * (kThreads / XPR);
            xrow[q] = j < F ? (uint32_t)((int64_t)min(max(idx[g * F + j], 0), D - 1) * ldx * 2) : kOOB;
        }
    } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int j = (wm * MT + mt) * 16 + col;
            jvalid[mt] = active && j < F;
            const int d = jvalid[mt] ? min(max(idx[g * F + j], 0), D - 1) : 0;
            xoff[mt] = (int64_t)d * ldx;
        }
    }

    // dY chunk c (rows c*64 ..) -> registers; rows >= B and labels >= O read as
    // zero (labels of a partial 8-label piece are masked when stashed).  An
    // access that crosses the end of a resource reads as zero as a whole, so the
    // resource covers a row up to the 8-label piece boundary: inside the row
    // when lddy >= O is a multiple of 8, else inside the next row.  dY's last
    // row may end at label O (yshort): there the resource ends at O and the
    // piece that straddles O is loaded early and shifted back (shift_down16).
    int pr[PPT], pcc[PPT];
#pragma unroll
    for (int q = 0; q < PPT; ++q) {
        const int p = tid + q * kThreads;
        pr[q] = p / (G / 8);
        pcc[q] = (p % (G / 8)) * 8;
    }
    // elements piece q of chunk c is loaded early by: 0 unless it straddles O in
    // row B-1 (then c is the last chunk)
    int sh_last[PPT];
#pragma unroll
    for (int q = 0; q < PPT; ++q) {
        const int over = pcc[q] + 8 - nl;  // > 0 only in the last group
        sh_last[q] = (yshort && over > 0 && over < 8 && pr[q] == (B - 1) % KC) ? over : 0;
    }
    const int c_last = (B - 1) / KC;
    auto tail_shift = [&](int c, int q) -> int { return c == c_last ? sh_last[q] : 0; };
    // (the resource starts up to 8 labels before l0, so that an early load of the
    // last group stays inside it: l0 + pcc - sh >= O - 8 >= 0)
    const int pre = yshort ? (int)std::min<int64_t>(l0, 8) : 0;
    auto fetch = [&](int c, u32x4 (&v)[PPT]) {
        const int b0 = c * KC;
        const int rows = std::min(KC, B - b0);
        const int lend = pre + ((yshort && b0 + rows == B) ? nl : (nl + 7) / 8 * 8);
        const rsrc_t yr = make_rsrc(dY + (int64_t)b0 * lddy + l0 - pre,
                                    ((int64_t)(rows - 1) * lddy + lend) * 2);
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const bool ok = tid + q * kThreads < C::PIECES && pcc[q] < nl;
            const int sh = tail_shift(c, q);
            v[q] = __builtin_amdgcn_raw_buffer_load_b128(
                yr, ok ? (uint32_t)(pr[q] * (uint32_t)lddy + pcc[q] + pre - sh) * 2 : kOOB, 0,
                YNT ? kLoadNT : 0);
        }
    };
    auto stash = [&](int c, int buf, const u32x4 (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            if (tid + q * kThreads < C::PIECES) {
                const int sh = tail_shift(c, q);
                *reinterpret_cast<u32x4*>(&Ys[buf][pr[q] * RB + pcc[q] * 2]) =
                    keep_first(sh ? shift_down16(v[q], sh) : v[q], nl - pcc[q]);
            }
        }
    };
    // XS: the X^T pieces of chunk c (entries >= B read as zero, those of a
    // partial piece are masked when stashed)
    auto fetch_x = [&](int c, u32x4 (&v)[PPTX]) {
        const int b0 = c * KC + xbc;
#pragma unroll
        for (int q = 0; q < PPTX; ++q)
            v[q] = buf_load16(xr, xrow[q] != kOOB && b0 < B ? xrow[q] + (uint32_t)b0 * 2 : kOOB);
    };
    auto stash_x = [&](int c, const u32x4 (&v)[PPTX]) {
        const int nv = B - (c * KC + xbc);
#pragma unroll
        for (int q = 0; q < PPTX; ++q)
            *reinterpret_cast<u32x4*>(&Xs[(tid / XPR + q * (kThreads / XPR)) * RBX + xbc * 2]) =
                keep_first(v[q], nv);
    };
    // Otherwise: the A fragments of chunk c, 8 consecutive batch entries of each
    // slot row (entries >= B read as zero; a partial 8-entry piece is masked at use)
    auto fetch_a = [&](int c, u32x4 (&a)[KSC][MT]) {
#pragma unroll
        for (int ks = 0; ks < KSC; ++ks) {
            const int bk = c * KC + ks * 32 + kq * 8;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                a[ks][mt] = buf_load16(xr, jvalid[mt] && bk < B ? (uint32_t)(xoff[mt] + bk) * 2 : kOOB);
        }
    };

    // The bias MFMA of label tile nt runs on the wave with wm == nt % WM, into
    // its accumulator accb[nt / WM]: the waves share the work and hold
    // ceil(NT / WM) accumulators each, not NT.
    constexpr int NBW = (NT + C::WM - 1) / C::WM;
    f32x4 acc[MT][NT];
    f32x4 accb[NBW];
#pragma unroll
    for (int k = 0; k < NBW; ++k) accb[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const uint32_t op = one_pair<T>();
    const u32x4 ones = u32x4{op, op, op, op};
    const bool do_bias = (dbias != nullptr || (SGD && sg.bias != nullptr)) && active;

    const rsrc_t wr = make_rsrc(SGD ? sg.W + l0 * F : nullptr, SGD ? (int64_t)nl * F * 2 : 0);
    constexpr int CPR = C::CPR, WPT = C::WPT;
    // Fused step: the weights and bias the epilogue updates are loaded now, so
    // their latency hides behind the batch loop (the thread's chunks are known:
    // in pass pp, chunk tid + q*256 is row pp*PR + it / CPR, slots (it % CPR) * 8
    // .. +7).  For at most two passes and F <= 128: beyond that the extra
    // registers would cost a wave per SIMD (so would they at four waves).
    constexpr int NPASS = G / PR;
    constexpr bool kWPre = SGD && NPASS <= 2 && FP <= 128 && bwdw_waves_per_simd<G, FP>() < 4;
    u32x4 wpre[kWPre ? NPASS * WPT : 1];
    uint32_t bpre = 0;  // fused step: bias bits of label tid (tid < nl)
    if constexpr (SGD) {
#pragma unroll
        for (int pp = 0; pp < (kWPre ? NPASS : 0); ++pp) {
#pragma unroll
            for (int q = 0; q < WPT; ++q) {
                const int it = tid + q * kThreads;
                const int j0 = (it % CPR) * 8;
                wpre[pp * WPT + q] = buf_load16(
                    wr, it < PR * CPR && j0 < F ? (uint32_t)((pp * PR + it / CPR) * F + j0) * 2 : kOOB);
            }
        }
        const rsrc_t bbr = make_rsrc(sg.bias != nullptr ? sg.bias + l0 : nullptr,
                                     sg.bias != nullptr ? (int64_t)nl * 2 : 0);
        bpre = __builtin_amdgcn_raw_buffer_load_b16(bbr, (tid < G ? tid * 2 : (int)kOOB), 0, 0);
    }

    // Ping-pong register sets by chunk parity (the loop body is unrolled twice),
    // so no register copy waits on a load: dY pieces are fetched two chunks
    // ahead, A fragments one chunk ahead (XS: X^T pieces one chunk ahead, into
    // the one LDS buffer once every wave has read it).  Chunks past the end load
    // nothing (every offset is out of range), so each body issues the same loads.
    u32x4 yr[2][PPT];
    u32x4 ar[XS ? 1 : 2][KSC][MT];
    u32x4 xv[PPTX];
    fetch(0, yr[0]);
    fetch(1, yr[1]);
    if constexpr (XS) fetch_x(0, xv);
    else fetch_a(0, ar[0]);
    stash(0, 0, yr[0]);
    fetch(2, yr[0]);
    if constexpr (XS) {
        stash_x(0, xv);
        fetch_x(1, xv);
    }
    __syncthreads();

    // lane's tr-read address inside a staged chunk: row 8*kq + 4*half + col/4,
    // labels n0 + 4*(col%4)
    const int tr_off = (kq * 8 + col / 4) * RB + (col % 4) * 8;
    auto body = [&](int c, auto parity) {
        constexpr int P = decltype(parity)::value;
        if constexpr (!XS) fetch_a(c + 1, ar[1 - P]);
        if (active && c < nchunks) {
            const char* ys = Ys[P];
#pragma unroll
            for (int ks = 0; ks < KSC; ++ks) {
                u32x4 af[MT];
                if constexpr (XS) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        af[mt] = *reinterpret_cast<const u32x4*>(
                            &Xs[((wm * MT + mt) * 16 + col) * RBX + (ks * 32 + kq * 8) * 2]);
                } else {
                    const int nv = B - (c * KC + ks * 32 + kq * 8);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) af[mt] = keep_first(ar[XS ? 0 : P][ks][mt], nv);
                }
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const char* p = ys + tr_off + ks * 32 * RB + (wn * NT + nt) * 32;
                    const u32x2 lo = lds_read_tr16(p);
                    const u32x2 hi = lds_read_tr16(p + 4 * RB);
                    const u32x4 bf = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[mt][nt] = mfma16x16x32<T>(af[mt], bf, acc[mt][nt]);
                    if (do_bias && nt % C::WM == wm) accb[nt / C::WM] = mfma16x16x32<T>(ones, bf, accb[nt / C::WM]);
                }
            }
        }
        if constexpr (XS) {
            __syncthreads();  // every wave has read the X^T buffer
            stash_x(c + 1, xv);
            fetch_x(c + 2, xv);
        }
        stash(c + 1, 1 - P, yr[1 - P]);  // chunk c + 1 (zeros past the end)
        fetch(c + 3, yr[1 - P]);
        __syncthreads();
    };
    for (int c = 0; c < nchunks; c += 2) {
        body(c, std::integral_constant<int, 0>{});
        body(c + 1, std::integral_constant<int, 1>{});
    }

    // ---- bias: lane (col, kq = 0) of the wave with wm == nt % WM holds the
    // column sum of label (wn*NT + nt)*16 + col in accb[nt / WM][0] ----
    if (do_bias && kq == 0) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int ll = (wn * NT + nt) * 16 + col;
            if (nt % C::WM != wm || ll >= nl) continue;
            const int64_t l = l0 + ll;
            const float v = accb[nt / C::WM][0];
            if (dbias != nullptr) {
                if (dbias_dtype == HASTE_DTYPE_F32)
                    static_cast<float*>(dbias)[l] = v;
                else if (dbias_dtype == HASTE_DTYPE_BF16)
                    static_cast<uint16_t*>(dbias)[l] = (uint16_t)f32_to_bf16_rne(v);
                else
                    static_cast<uint16_t*>(dbias)[l] = (uint16_t)f32_to_f16_rne(v);
            }
            // fused step: staged, and applied below by thread ll (in parallel with
            // the weights, instead of by these 16 lanes while the other waves wait)
            if constexpr (SGD) s_bg[ll] = v;
        }
    }

    // ---- gradient tile: staged in LDS (labels [p0, p0+PR) per pass), then
    // processed as rows of 8 consecutive slots per thread ----
    const int esz = dW_dtype == HASTE_DTYPE_F32 ? 4 : 2;
    const rsrc_t gr = make_rsrc(dW != nullptr ? static_cast<char*>(dW) + l0 * F * esz : nullptr,
                                dW != nullptr ? (int64_t)nl * F * esz : 0);
    const rsrc_t mr = make_rsrc(SGD && sg.use_mom ? sg.mW + l0 * F : nullptr,
                                SGD && sg.use_mom ? (int64_t)nl * F * 4 : 0);
    const bool do_wt = SGD && sg.twt != nullptr;
    if constexpr (SGD) {
        if (do_wt)
            for (int j = tid; j < F; j += kThreads) s_perm[j] = sg.perm[g * F + j];
    }
    // The W^T pass of labels [p0, p0 + PR) writes chunk it (of the group's
    // rows x PR/8 chunks) in twt storage order, so consecutive threads write
    // consecutive 16 bytes: tile row wt_row(it), chunk p0/8 + wt_chk(it).
    // Chunk it = tid + k*256 (k < kWtPre) has its tsrc entry loaded here, long
    // before the pass needs it.
    constexpr int CHP = PR / 8;
    auto wt_row = [](int it) { return (it / (16 * CHP)) * 16 + it % 16; };
    auto wt_chk = [](int it) { return (it / 16) % CHP; };
    constexpr int kWtPre = 8;
    int wsrc[SGD ? kWtPre : 1];
    int wt_rows = 0;
    if constexpr (SGD) {
        if (do_wt) {
            wt_rows = sg.meta[(g * sg.ndr + sg.ndr - 1) * kMetaStride + 1] * 16;
            const rsrc_t tr = make_rsrc(sg.tsrc + g * sg.Tcap * 16, (int64_t)sg.Tcap * 16 * 4);
#pragma unroll
            for (int k = 0; k < kWtPre; ++k)
                wsrc[k] = (int)buf_load4(tr, (uint32_t)wt_row(tid + k * kThreads) * 4);
        }
    }
#pragma unroll 1
    for (int p0 = 0; p0 < G; p0 += PR) {
        if (active) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int ll = (wn * NT + nt) * 16;
                if (ll < p0 || ll >= p0 + PR) continue;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    *reinterpret_cast<f32x4*>(&stg[(ll - p0 + col) * SP + (wm * MT + mt) * 16 + kq * 4]) =
                        acc[mt][nt];
            }
        }
        __syncthreads();
        if constexpr (SGD) {
            if (p0 == 0 && sg.bias != nullptr && tid < nl) {
                const int64_t l = l0 + tid;
                float mv = sg.use_mom ? sg.mb[l] : 0.f;
                sg.bias[l] = (uint16_t)sgd_one(bf16_bits_to_f32(bpre), s_bg[tid], &mv, sg.use_mom,
                                               sg.lr, sg.wd, sg.mu, sg.do_sr, (uint64_t)l, sk0,
                                               sk1);
                if (sg.use_mom) sg.mb[l] = mv;
            }
        }
#pragma unroll
        for (int q = 0; q < WPT; ++q) {
            const int it = tid + q * kThreads;
            if (it >= PR * CPR) break;
            const int lr = p0 + it / CPR, j0 = (it % CPR) * 8;
            const f32x4 g0 = *reinterpret_cast<const f32x4*>(&stg[(lr - p0) * SP + j0]);
            const f32x4 g1 = *reinterpret_cast<const f32x4*>(&stg[(lr - p0) * SP + j0 + 4]);
            const bool in = j0 < F;  // rows >= nl fall outside every resource
            const uint32_t e = (uint32_t)(lr * F + j0);
            if (dW != nullptr) {
                if (dW_dtype == HASTE_DTYPE_F32) {
                    buf_store16(__builtin_bit_cast(u32x4, g0), gr, in ? e * 4 : kOOB);
                    buf_store16(__builtin_bit_cast(u32x4, g1), gr, in ? e * 4 + 16 : kOOB);
                } else {
                    const u32x4 h = dW_dtype == HASTE_DTYPE_BF16
                        ? u32x4{pack2_rne<BF16>(g0[0], g0[1]), pack2_rne<BF16>(g0[2], g0[3]),
                                pack2_rne<BF16>(g1[0], g1[1]), pack2_rne<BF16>(g1[2], g1[3])}
                        : u32x4{pack2_rne<F16>(g0[0], g0[1]), pack2_rne<F16>(g0[2], g0[3]),
                                pack2_rne<F16>(g1[0], g1[1]), pack2_rne<F16>(g1[2], g1[3])};
                    buf_store16(h, gr, in ? e * 2 : kOOB);
                }
            }
            if constexpr (SGD) {
                u32x4 wv;
                if constexpr (kWPre) wv = p0 == 0 ? wpre[q] : wpre[(NPASS - 1) * WPT + q];
                else wv = buf_load16(wr, in ? e * 2 : kOOB);
                float gv[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
                float mv[8];
                if (sg.use_mom) {
                    const f32x4 m0 = __builtin_bit_cast(f32x4, buf_load16(mr, in ? e * 4 : kOOB));
                    const f32x4 m1 = __builtin_bit_cast(f32x4, buf_load16(mr, in ? e * 4 + 16 : kOOB));
#pragma unroll
                    for (int k = 0; k < 4; ++k) { mv[k] = m0[k]; mv[4 + k] = m1[k]; }
                }
                const uint32_t off = (uint32_t)((l0 + lr) * F + j0);
                uint32_t ob[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint32_t wb = (k & 1) ? (wv[k >> 1] >> 16) : (wv[k >> 1] & 0xFFFFu);
                    const uint32_t r = sg.do_sr ? philox_w0_32(off + k, sk0, sk1) : 0u;
                    ob[k] = sgd_one_r(bf16_bits_to_f32(wb), gv[k], &mv[k], sg.use_mom, sg.lr,
                                      sg.wd, sg.mu, sg.do_sr, r);
                }
                const u32x4 wn = u32x4{ob[0] | (ob[1] << 16), ob[2] | (ob[3] << 16),
                                       ob[4] | (ob[5] << 16), ob[6] | (ob[7] << 16)};
                buf_store16(wn, wr, in ? e * 2 : kOOB);
                // the updated weights replace this thread's own staged gradients
                // (the first 16 of its 32 bytes), for the W^T pass below
                if (do_wt) *reinterpret_cast<u32x4*>(&stg[(lr - p0) * SP + j0]) = wn;
                if (sg.use_mom) {
                    buf_store16(__builtin_bit_cast(u32x4, f32x4{mv[0], mv[1], mv[2], mv[3]}), mr,
                                in ? e * 4 : kOOB);
                    buf_store16(__builtin_bit_cast(u32x4, f32x4{mv[4], mv[5], mv[6], mv[7]}), mr,
                                in ? e * 4 + 16 : kOOB);
                }
            }
        }
        if constexpr (SGD) {
            if (do_wt) {
                // W^T tile rows of this group, labels [p0, p0 + PR): 16-byte chunks
                // of 8 labels, as the bwd-features gather kernel builds them
                __syncthreads();
                auto wv = [&](int l, int slot) -> uint32_t {
                    return reinterpret_cast<const uint16_t*>(
                        &stg[(l - p0) * SP + (slot >> 3) * 8])[slot & 7];
                };
                const int64_t rbase = g * sg.Tcap * 16;
                const int nch = wt_rows * CHP;
#pragma unroll
                for (int k = 0; k < kWtPre; ++k) {
                    const int it = tid + k * kThreads;
                    if (it < nch) {
                        const int row = wt_row(it), lc = p0 + wt_chk(it) * 8;
                        const u32x4 v = wt_chunk<BF16>(wsrc[k], s_perm, wv, lc);
                        *reinterpret_cast<u32x4*>(sg.twt + twt_elem(rbase + row, lc, G)) = v;
                    }
                }
                for (int it = tid + kWtPre * kThreads; it < nch; it += kThreads) {
                    const int row = wt_row(it), lc = p0 + wt_chk(it) * 8;
                    const u32x4 v = wt_chunk<BF16>(sg.tsrc[rbase + row], s_perm, wv, lc);
                    *reinterpret_cast<u32x4*>(sg.twt + twt_elem(rbase + row, lc, G)) = v;
                }
            }
        }
        if (p0 + PR < G) __syncthreads();
    }
}

template <typename T, int G, int FP, bool SGD, bool YNT, bool YS>
int launch(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* dY, int64_t lddy,
           void* dW, int dW_dtype, void* dbias, int dbias_dtype, int64_t B, int64_t D, int64_t F,
           int64_t O, const SgdArgs& sg, hipStream_t st) {
    const int64_t Gc = ceil_div(O, G);
    if (Gc + sg.rj.ntiles > 0x7FFFFFFF || D * ldx * 2 > kMaxRsrcBytes ||
        ((int64_t)BwdWCfg<G, FP>::KC * lddy + 8) * 2 > kMaxRsrcBytes || (int64_t)G * F * 4 > kMaxRsrcBytes) {
        set_error("haste_ffi_bwd_weights: problem too large (Gc %lld, lddy %lld, D*ldx %lld)",
                  (long long)Gc, (long long)lddy, (long long)(D * ldx));
        return HASTE_ERR_UNSUPPORTED;
    }
    ffi_bwd_w_kernel<T, G, FP, SGD, YNT, YS><<<dim3((unsigned)(Gc + sg.rj.ntiles)), dim3(kThreads), 0, st>>>(
        idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias, dbias_dtype, (int)B, (int)D, (int)F, O, sg);
    HASTE_CHECK_LAUNCH("haste_ffi_bwd_weights");
    return HASTE_OK;
}

template <typename T, bool SGD, bool YNT, bool YS>
int dispatch_g(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* dY,
             int64_t lddy, void* dW, int dW_dtype, void* dbias, int dbias_dtype, int64_t B,
             int64_t D, int64_t F, int64_t O, int64_t G, const SgdArgs& sg, hipStream_t st) {
#define HASTE_BWDW_FP(GG)                                                                        \
    do {                                                                                         \
        if (F <= 32) return launch<T, GG, 32, SGD, YNT, YS>(idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias,  \
                                                   dbias_dtype, B, D, F, O, sg, st);             \
        if (F <= 64) return launch<T, GG, 64, SGD, YNT, YS>(idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias,  \
                                                   dbias_dtype, B, D, F, O, sg, st);             \
        if (F <= 128) return launch<T, GG, 128, SGD, YNT, YS>(idx, xT, ldx, dY, lddy, dW, dW_dtype,       \
                                                     dbias, dbias_dtype, B, D, F, O, sg, st);    \
        return launch<T, GG, 256, SGD, YNT, YS>(idx, xT, ldx, dY, lddy, dW, dW_dtype, dbias, dbias_dtype, \
                                       B, D, F, O, sg, st);                                      \
    } while (0)
    switch (G) {
    case 16: HASTE_BWDW_FP(16);
    case 32: HASTE_BWDW_FP(32);
    case 64: HASTE_BWDW_FP(64);
    case 128: HASTE_BWDW_FP(128);
    default: break;
    }
#undef HASTE_BWDW_FP
    set_error("haste_ffi_bwd_weights: unsupported group size %lld", (long long)G);
    return HASTE_ERR_UNSUPPORTED;
}

}  // namespace

// dY rows at a stride that is not a multiple of 8 (YS kernels; defined in
// ffi_bwd_weights_ys.hip).  Same arguments as the dispatch of ffi_bwd_weights.hip.
int bwdw_dispatch_ys(int32_t dtype, bool sgd, const int32_t* idx, const uint16_t* xT,
                     int64_t ldx, const uint16_t* dY, int64_t lddy, void* dW, int dW_dtype,
                     void* dbias, int dbias_dtype, int64_t B, int64_t D, int64_t F, int64_t O,
                     int64_t G, const SgdArgs& sg, hipStream_t st);

}  // namespace haste
