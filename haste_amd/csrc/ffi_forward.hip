// Grouped fixed-fan-in forward (gfx950).
//
//   out[b, l] = RNE( sum_j xT[idx[g, j], b] * W[l, j] + bias[l] ),  g = l / G
//
// One workgroup = one label group g x a chunk of the batch (the whole batch
// up to 512 columns), walked in tiles of 64 batch columns.  MFMA orientation:
// M = labels, N = batch, K = fan-in slots.
//  - A: W fragments (label rows x 8 contiguous slots) loaded once per
//    workgroup into VGPRs and reused over the whole batch chunk.  A wave holds
//    the fragments of MT label tiles (all G labels when they fit in 64
//    registers), so the waves split the batch columns of a tile.
//  - B: the gathered rows xT[idx[g, j], b0:b0+64] are copied row-major into LDS
//    (16-byte copies, Xg[slot][batch]; xT is small and L2 resident) and read
//    back with ds_read_b64_tr_b16, which hands each lane 4 consecutive slots of
//    one batch column.  Tile t+2's rows are fetched into registers while tile
//    t's MFMAs run (two LDS buffers, or one where LDS limits the workgroups
//    per CU).
//  - Epilogue: results are staged per wave in LDS and stored as whole 128-byte
//    row segments (a lane's MFMA output covers only 8 bytes of a row; 8-byte
//    stores spread over 16 rows cost four times the L2 write requests).
//  - Every load and store of the tile loop is a raw buffer access: rows past B,
//    labels past O and slots past F are range-checked by the hardware instead
//    of branched around, so the loop issues a fixed number of memory
//    instructions and each wait covers only the loads it needs.
// bf16/f16 MFMA 16x16x32 with fp32 accumulation; bias is added in fp32 and the
// result rounded to nearest even (as dump_and_store_tile,
// shared_ffi/ffi_forward_kernels.cu:85-101).
#include <algorithm>
#include <mutex>

#include "common.hpp"

namespace haste {
namespace {

constexpr int kBT = 64;        // batch columns per tile
constexpr int kStoreNT = 2;    // buffer-store cache policy: nt (non-temporal) on gfx950
constexpr int kThreads = 256;  // 4 waves
constexpr int kMaxTilesPerWG = 8;

// ESZ: bytes per output element (2: logits in the inputs' 16-bit type, 4: fp32
// logits of the fp32 layer).
template <int G, int FP, int ESZ = 2>
struct FwdCfg {
    static constexpr int KS = FP / 32;     // MFMA k-steps
    static constexpr int MTILES = G / 16;  // label tiles in the group
    // Gathered-row LDS buffers: two (tile t+1 is stashed while tile t is read)
    // unless their size caps the workgroups per CU below what the registers
    // allow; with one, a barrier separates a tile's reads from the next stash.
    static constexpr int NB = (FP == 256 || (FP == 128 && (G == 32 || G == 64))) ? 1 : 2;
    // Waves along labels: a wave keeps MT*KS W fragments (<= 16, 64 VGPRs).  At
    // G = 64, FP = 128 two waves share the labels (32 W registers each, twice
    // the LDS reads of the gathered rows), so that four workgroups fit a CU:
    // the 2049 groups of a 131K-label layer then run in two rounds, not three.
    // At G = 32, FP = 256 two label waves halve the W fragment loads (every
    // wave of a label row loads all of its fragments): those loads were a third
    // of the kernel's vector-memory instructions, whose address path bounds it.
    static constexpr int WM = ((G == 64 && FP == 128) || (G == 32 && FP == 256)) ? 2
                              : MTILES * KS <= 16 ? 1 : (MTILES * KS <= 32 ? 2 : 4);
    static constexpr int WN = 4 / WM;             // waves along the batch
    static constexpr int MT = MTILES / WM;        // label tiles per wave
    static constexpr int NT = (kBT / 16) / WN;    // 16-column batch tiles per wave
    static constexpr int RB = kBT * 2 + 16;       // LDS bytes per gathered row
    static constexpr int PIECES = FP * (kBT / 8); // 16-byte pieces per tile
    static constexpr int PPT = PIECES / kThreads; // >= 1 (FP >= 32)
    static constexpr int SRB = MT * 16 * ESZ + 16;  // LDS bytes per staged output row
    static constexpr int STG = NT * 16 * SRB;     // staged output bytes per wave
    static_assert(MTILES % WM == 0 && PPT >= 1, "tile shape");
};

// Fused sparse-BCE epilogue (BCE = true): out receives dY = sigma(x) - y instead of
// the logits x, where x is the bf16-rounded logit and y the label bit; logits,
// when not null, receives x as well.  part[w] = workgroup w's sum over its valid
// elements of max(x, 0) - y*x + log(1 + exp(-|x|)) (the loss of
// src/runner.py:469-478, whose gradient in x is sigma(x) - y).  ybits holds one
// bit per (row, label), ldyw 32-bit words per row.
struct BceArgs {
    const uint32_t* ybits;
    int64_t ldyw;
    uint16_t* logits;
    float* part;
};

// dY = sigma(x) - y of one element, in fp32 from the hardware exp2 and reciprocal
// (about 1 ulp each).  With e = exp(-|x|) and r = 1 / (1 + e), sigma(x) and
// 1 - sigma(x) are r and e*r in some order, so sigma(x) - 1 needs no cancelling
// subtraction.  bce_sigma is the label-free case (y = 0) and also returns
// d = 1 + e, whose log is the element's softplus term; bce_dy_pos is y = 1.
__device__ __forceinline__ float bce_sigma(float x, float* d) {
    const float e = __builtin_amdgcn_exp2f(-__builtin_fabsf(x) * 1.44269504088896341f);
    *d = 1.0f + e;
    const float r = __builtin_amdgcn_rcpf(*d);
    return x >= 0.0f ? r : e * r;
}
__device__ __forceinline__ float bce_dy_pos(float x) {
    const float e = __builtin_amdgcn_exp2f(-__builtin_fabsf(x) * 1.44269504088896341f);
    const float r = __builtin_amdgcn_rcpf(1.0f + e);
    return -(x >= 0.0f ? e * r : r);
}

// LAST: the workgroup's group is the last one and holds fewer than G labels;
// its stores are per element so that no column >= O is written.
// O32: fp32 bias and fp32 logits (the fp32 layer, whose features and weights the
// caller has rounded to fp16); otherwise bias and logits are T.
template <typename T, int G, int FP, bool LAST, bool BCE, bool O32>
__device__ __forceinline__ void fwd_group(const int32_t* __restrict__ idx,
                                          const uint16_t* __restrict__ xT, int64_t ldx,
                                          const uint16_t* __restrict__ W,
                                          const uint16_t* __restrict__ bias,
                                          uint16_t* __restrict__ out, int64_t ldo, int B, int D,
                                          int F, int64_t O, int64_t g, int b_chunk0, int ntiles,
                                          char (*Xg)[FP * FwdCfg<G, FP>::RB],
                                          char (*stg)[FwdCfg<G, FP, O32 ? 4 : 2>::STG],
                                          const BceArgs& bce,
                                          float* s_red) {
    static_assert(!(BCE && O32), "the BCE epilogue writes 16-bit dY");
    constexpr int ESZ = O32 ? 4 : 2;
    using C = FwdCfg<G, FP, ESZ>;
    constexpr int KS = C::KS, MT = C::MT, NT = C::NT, RB = C::RB, PPT = C::PPT, SRB = C::SRB;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % C::WM, wn = wave / C::WM;
    const int col = lane & 15;  // row of A / column of B / column of D
    const int kq = lane >> 4;   // K-chunk of A/B, row-quad of D
    const int64_t l0 = g * G;
    const int nl = (int)std::min<int64_t>(G, O - l0);  // labels of this group

    // piece p of a tile: slot p / 8, batch columns 8 * (p % 8) .. +7.  The
    // thread's slots' indices are loaded first, straight into registers (they
    // start the gather chain); indices outside [0, D) are clamped (the
    // reference leaves them undefined), slots >= F gather row 0 (their W
    // columns read as zero).
    int pj[PPT], pc[PPT], pidx[PPT];
    {
        const rsrc_t ir = make_rsrc(idx + g * F, (int64_t)F * 4);
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int p = tid + q * kThreads;
            pj[q] = p / (kBT / 8);
            pc[q] = (p % (kBT / 8)) * 8;
            pidx[q] = (int)buf_load4(ir, pj[q] < F ? (uint32_t)pj[q] * 4 : kOOB);
        }
    }

    // W fragments (A operand) and bias of this wave's label tiles; rows >= O and
    // slots >= F are outside the resources and read as zero.
    const rsrc_t wr = make_rsrc(W + l0 * F, (int64_t)nl * F * 2);
    const rsrc_t br = bias != nullptr
        ? make_rsrc(reinterpret_cast<const char*>(bias) + l0 * ESZ, (int64_t)nl * ESZ)
        : make_rsrc(W, 0);
    u32x4 wf[MT][KS];
    float bv[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int lr = (wm * MT + mt) * 16 + col;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int k = ks * 32 + kq * 8;
            wf[mt][ks] = buf_load16(wr, k < F ? (uint32_t)(lr * F + k) * 2 : kOOB);
        }
        // labels past the group get the out-of-range offset rather than being
        // left to the range check: loads at consecutive offsets may be merged
        // into one wider load, which a label past the end would zero as a whole
        const int lb = (wm * MT + mt) * 16 + kq * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool in = lb + i < nl;
            bv[mt][i] = O32 ? __builtin_bit_cast(float, buf_load4(br, in ? (uint32_t)(lb + i) * 4 : kOOB))
                            : bits_to_f32<T>(__builtin_amdgcn_raw_buffer_load_b16(
                                  br, in ? (lb + i) * 2 : (int)kOOB, 0, 0));
        }
    }

    // chunks starting at or past B read as zero, columns >= B of a partial chunk
    // are masked when stashed
    const rsrc_t xr = make_rsrc(xT, (int64_t)D * ldx * 2);
    int64_t prow[PPT];
#pragma unroll
    for (int q = 0; q < PPT; ++q) prow[q] = (int64_t)min(max(pidx[q], 0), D - 1) * ldx;
    auto fetch = [&](int b_base, u32x4 (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int b0 = b_base + pc[q];
            v[q] = buf_load16(xr, b0 < B ? (uint32_t)(prow[q] + b0) * 2 : kOOB);
        }
    };
    auto stash = [&](int buf, int b_base, const u32x4 (&v)[PPT]) {
#pragma unroll
        for (int q = 0; q < PPT; ++q) {
            const int nv = B - (b_base + pc[q]);  // valid columns in this chunk
            u32x4 m = v[q];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                m[e] &= (2 * e + 1 < nv) ? 0xFFFFFFFFu : (2 * e < nv ? 0xFFFFu : 0u);
            *reinterpret_cast<u32x4*>(&Xg[buf][pj[q] * RB + pc[q] * 2]) = m;
        }
    };

    u32x4 xv[PPT];
    fetch(b_chunk0, xv);
    stash(0, b_chunk0, xv);
    if (ntiles > 1) fetch(b_chunk0 + kBT, xv);
    __syncthreads();

    // lane's tr-read address: slot 8*kq + col/4 (+4 for the second half), batch
    // columns n0 + 4*(col%4)
    const int tr_off = (kq * 8 + col / 4) * RB + (col % 4) * 8;
    // BCE: label words of the group for each of the lane's rows (the words
    // holding labels l0 .. l0+G-1 start at word l0/32, bit l0 % 32)
    constexpr int YW = G >= 64 ? G / 32 : 2;
    const uint32_t ybit0 = (uint32_t)(l0 % 32);
    // loss of the lane's elements: the max(x, 0) - y*x parts are summed, the
    // d = 1 + exp(-|x|) factors (each in (1, 2]) multiplied over a tile -- at most
    // 64 per lane, so the product stays below 2^64 -- and one log2 is taken per
    // tile instead of one per element
    float lsum = 0.0f;
    static_assert(C::MT * C::NT * 4 <= 64, "loss product range");
    for (int t = 0; t < ntiles; ++t) {
        const int b_base = b_chunk0 + t * kBT;
        const char* xs = Xg[C::NB == 1 ? 0 : t & 1];
        uint32_t yw[NT][YW];
        if constexpr (BCE) {
            const rsrc_t yr = make_rsrc(bce.ybits + (int64_t)b_base * bce.ldyw,
                                        (int64_t)std::min(kBT, B - b_base) * bce.ldyw * 4);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t o = (uint32_t)(((wn * NT + nt) * 16 + col) * bce.ldyw + l0 / 32) * 4;
                if constexpr (YW == 2) {
                    const u32x2 v = buf_load8(yr, o);
                    yw[nt][0] = v[0];
                    yw[nt][1] = v[1];
                } else {
                    const u32x4 v = buf_load16(yr, o);
#pragma unroll
                    for (int k = 0; k < 4; ++k) yw[nt][k] = v[k];
                }
            }
        }
        f32x4 acc[MT][NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int n0 = (wn * NT + nt) * 16;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const char* p = xs + tr_off + ks * 32 * RB + n0 * 2;
                const u32x2 lo = lds_read_tr16(p);
                const u32x2 hi = lds_read_tr16(p + 4 * RB);
                const u32x4 bf = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16x16x32<T>(wf[mt][ks], bf, acc[mt][nt]);
            }
        }
        if (C::NB == 1) __syncthreads();  // every wave is done reading the buffer
        if (t + 1 < ntiles) {
            stash(C::NB == 1 ? 0 : (t + 1) & 1, b_base + kBT, xv);
            if (t + 2 < ntiles) fetch(b_base + 2 * kBT, xv);
        }

        // ---- epilogue: + bias (fp32), RNE (O32: kept in fp32).  A lane holds 4
        // consecutive labels of one batch row; they are staged in LDS and written
        // as row segments.
        // Rows >= B fall outside the tile's resource.  The last (partial) group
        // stores per element instead, so no column >= O is written. ----
        float dprod = 1.0f;  // BCE: the tile's d factors of this lane
        const rsrc_t orr = make_rsrc(reinterpret_cast<char*>(out) + ((int64_t)b_base * ldo + l0) * ESZ,
                                     ((int64_t)(std::min(kBT, B - b_base) - 1) * ldo + nl) * ESZ);
        // BCE with logits wanted: the rounded logits go out directly, 8 bytes per
        // lane (rows past B and labels past O outside the resource)
        const rsrc_t lgr = BCE && bce.logits != nullptr
            ? make_rsrc(bce.logits + (int64_t)b_base * ldo + l0,
                        (int64_t)(std::min(kBT, B - b_base) - 1) * ldo * 2 + nl * 2)
            : make_rsrc(out, 0);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int rb = (wn * NT + nt) * 16 + col;  // row within the tile
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int ll = (wm * MT + mt) * 16 + kq * 4;  // label within the group
                const f32x4 v = acc[mt][nt];
                if constexpr (O32) {
                    const u32x4 h4 = __builtin_bit_cast(
                        u32x4, (f32x4{v[0] + bv[mt][0], v[1] + bv[mt][1], v[2] + bv[mt][2],
                                      v[3] + bv[mt][3]}));
                    const uint32_t off4 = (uint32_t)((int64_t)rb * ldo + ll) * 4;
                    if constexpr (!LAST) {
                        *reinterpret_cast<u32x4*>(&stg[wave][(nt * 16 + col) * SRB + (mt * 16 + kq * 4) * 4]) = h4;
                    } else {
                        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // as the 16-bit LAST stores below
#pragma unroll
                        for (int i = 0; i < 4; ++i) buf_store4(h4[i], orr, ll + i < nl ? off4 + 4 * i : kOOB);
                    }
                    continue;
                }
                u32x2 h = u32x2{pack2_rne<T>(v[0] + bv[mt][0], v[1] + bv[mt][1]),
                                pack2_rne<T>(v[2] + bv[mt][2], v[3] + bv[mt][3])};
                if constexpr (BCE) {
                    if (bce.logits != nullptr) {
                        const uint32_t lo = (uint32_t)((int64_t)rb * ldo + ll) * 2;
                        if (ll + 4 <= nl) {
                            buf_store8(h, lgr, lo);
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                buf_store2((uint16_t)(h[i >> 1] >> ((i & 1) * 16)), lgr,
                                           ll + i < nl ? lo + 2 * i : kOOB);
                        }
                    }
                    const uint32_t bit = ybit0 + (uint32_t)ll;
                    const uint32_t y4 = (yw[nt][bit >> 5] >> (bit & 31)) & 0xFu;
                    const bool row_ok = b_base + rb < B;
                    float x[4], dy[4], lin = 0.0f, dp = 1.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        x[i] = bits_to_f32<T>((h[i >> 1] >> ((i & 1) * 16)) & 0xFFFFu);
                        float d;
                        dy[i] = bce_sigma(x[i], &d);
                        const bool ok = !LAST || ll + i < nl;
                        // max(x, 0) as a select on the compare sigma already made
                        // (fmaxf adds a canonicalising max per element)
                        lin += ok && x[i] >= 0.0f ? x[i] : 0.0f;
                        dp *= ok ? d : 1.0f;
                    }
                    // positive labels are sparse: a wave takes this branch only
                    // when one of its lanes holds one among these 4 elements
                    if (__builtin_amdgcn_ballot_w64(y4 != 0u) != 0) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if ((y4 >> i) & 1u) {
                                dy[i] = bce_dy_pos(x[i]);
                                lin -= (!LAST || ll + i < nl) ? x[i] : 0.0f;
                            }
                        }
                    }
                    lsum += row_ok ? lin : 0.0f;
                    dprod *= row_ok ? dp : 1.0f;
                    h = u32x2{pack2_rne<T>(dy[0], dy[1]), pack2_rne<T>(dy[2], dy[3])};
                }
                const uint32_t off = (uint32_t)((int64_t)rb * ldo + ll) * 2;
                if constexpr (!LAST) {
                    *reinterpret_cast<u32x2*>(&stg[wave][(nt * 16 + col) * SRB + (mt * 16 + kq * 4) * 2]) = h;
                } else {
                    // a store whose lanes are all out of range may retire ahead
                    // of older loads (the next tile's gathered rows); later
                    // counted waits must not rely on it
                    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        buf_store2((uint16_t)(h[i >> 1] >> ((i & 1) * 16)), orr,
                                   ll + i < nl ? off + 2 * i : kOOB);
                }
            }
        }
        if constexpr (BCE) lsum += __builtin_amdgcn_logf(dprod) * 0.693147180559945309f;
        // staged rows go out as 16-byte stores, whole row segments per
        // instruction (full 128-byte lines at MT = 4); the wave reads back only
        // what it wrote, and a wave's LDS accesses complete in order
        auto flush = [&](const rsrc_t& dst) {
            constexpr int LPR = MT * ESZ;   // lanes per staged row (MT*16*ESZ bytes)
            constexpr int RPI = 64 / LPR;   // rows per instruction
#pragma unroll
            for (int r0 = 0; r0 < NT * 16; r0 += RPI) {
                // at G = 16 an instruction spans more rows than the wave staged
                // (RPI = 32 > 16): the lanes past them store nothing
                const int rr = r0 + lane / LPR, cb = (lane % LPR) * 16;
                const bool own = RPI <= NT * 16 || rr < NT * 16;
                const int rs = own ? rr : 0;
                const u32x4 v = *reinterpret_cast<const u32x4*>(&stg[wave][rs * SRB + cb]);
                const int rb = wn * NT * 16 + rs;
                // logits and dY are non-temporal stores (cache-policy bit nt),
                // so the stream of them does not evict the gathered rows and
                // weights (for dY this measured 2.6 us faster over the fused-loss
                // step at config 1, although the backward kernels read it next)
                __builtin_amdgcn_raw_buffer_store_b128(
                    v, dst, own ? (uint32_t)(((int64_t)rb * ldo + wm * MT * 16) * ESZ + cb) : kOOB, 0,
                    kStoreNT);
            }
        };
        // Several waves along the labels whose staged rows are less than a
        // 128-byte line each (G = 64 at F >= 128: two waves of 64 bytes; G = 128
        // at F >= 128: four of 64): after a barrier the group's rows go out as
        // whole lines, wave (wm, wn) writing rows [wm, wm+1) * NT*16/WM of the
        // NT*16 rows its wn block staged, with every wave's labels, so no line is
        // written in parts by different waves at different times.
        constexpr int SEG = MT * 16 * ESZ;  // bytes of a row that one wave staged
        constexpr bool kGroupFlush = C::WM > 1 && SEG < 128;
        auto flush_group = [&](const rsrc_t& dst) {
            constexpr int LPRG = C::WM * SEG / 16;  // lanes per whole group row
            constexpr int RPIG = 64 / LPRG;         // rows per instruction
            constexpr int ROWS = NT * 16 / C::WM;   // rows this wave writes
            static_assert(!kGroupFlush || (LPRG <= 64 && ROWS % RPIG == 0),
                          "whole rows per instruction");
#pragma unroll
            for (int r0 = 0; r0 < ROWS; r0 += RPIG) {
                const int rs = wm * ROWS + r0 + lane / LPRG;  // staged row of the block
                const int cb = (lane % LPRG) * 16;            // byte within the group row
                const int src = cb / SEG + C::WM * wn;        // the wave that staged it
                const u32x4 v = *reinterpret_cast<const u32x4*>(&stg[src][rs * SRB + cb % SEG]);
                const int rb = wn * NT * 16 + rs;
                __builtin_amdgcn_raw_buffer_store_b128(
                    v, dst, (uint32_t)((int64_t)rb * ldo * ESZ + cb), 0, kStoreNT);
            }
        };
        if constexpr (!LAST) {
            if constexpr (kGroupFlush) {
                __syncthreads();  // every wave's labels are staged
                flush_group(orr);
            } else {
                flush(orr);
            }
        }
        __syncthreads();
    }
    if constexpr (BCE) {
        // workgroup sum of the loss terms in a fixed order: lanes by xor
        // butterfly, then the four waves in order
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) lsum += __shfl_xor(lsum, m, 64);
        if (lane == 0) s_red[wave] = lsum;
        __syncthreads();
        if (tid == 0) *bce.part = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    }
}

// Register bound: four waves per SIMD at G = 64, FP = 128 (the split labels
// above), three there for the BCE epilogue, whose extra registers would
// otherwise cost a wave; two elsewhere.
template <int G, int FP, bool BCE, bool O32>
constexpr int fwd_waves_per_simd() { return G == 64 && FP == 128 && !O32 ? (BCE ? 3 : 4) : 2; }

template <typename T, int G, int FP, bool BCE, bool O32>
__global__ __launch_bounds__(kThreads, (fwd_waves_per_simd<G, FP, BCE, O32>())) void ffi_fwd_kernel(
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ xT, int64_t ldx,
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int B, int D, int F, int64_t O, int64_t Gc, int nchunks, int tiles_per_chunk,
    BceArgs bce) {
    using C = FwdCfg<G, FP, O32 ? 4 : 2>;
    __shared__ __attribute__((aligned(16))) char Xg[C::NB][FP * C::RB];
    __shared__ __attribute__((aligned(16))) char stg[4][C::STG];
    __shared__ float s_red[4];

    const int64_t work = xcd_remap(blockIdx.x, Gc * nchunks);
    if (work < 0) return;
    // the last group's chunks are the first work items: when the work does not
    // split evenly over the XCDs, XCD 0 holds one item more than the others,
    // and it is then the last group, the smallest one when O % G != 0
    const int64_t wr = work < nchunks ? work + (Gc - 1) * nchunks : work - nchunks;
    const int64_t g = wr / nchunks;
    const int chunk = (int)(wr % nchunks);
    const int b_chunk0 = chunk * tiles_per_chunk * kBT;
    const int ntiles = min(tiles_per_chunk, (B - b_chunk0 + kBT - 1) / kBT);
    if constexpr (BCE) bce.part += work;
    if ((g + 1) * G > O)
        fwd_group<T, G, FP, true, BCE, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, g,
                                            b_chunk0, ntiles, Xg, stg, bce, s_red);
    else
        fwd_group<T, G, FP, false, BCE, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, g,
                                             b_chunk0, ntiles, Xg, stg, bce, s_red);
}

// Batch chunks per group: the whole batch per workgroup (up to kMaxTilesPerWG
// tiles), split further only when there are too few groups to fill the GPU.
// Returns the chunk count; *tpc = tiles per chunk.
int64_t fwd_chunks(int64_t B, int64_t Gc, int64_t* tpc) {
    const int64_t ntiles = ceil_div(B, kBT);
    int64_t nchunks = ceil_div(ntiles, kMaxTilesPerWG);
    while (Gc * nchunks < 2048 && nchunks < ntiles) ++nchunks;
    *tpc = ceil_div(ntiles, nchunks);
    return ceil_div(ntiles, *tpc);
}

// The host-side limits of launch_fwd: the grid and the 32-bit buffer offsets.
// haste_ffi_forward_bce checks them before it marks any label bits, so a call
// that fails here leaves the workspace zero.
int check_fwd_size(int64_t B, int64_t D, int64_t ldx, int64_t ldo, int64_t O, int64_t G,
                   int64_t out_esz = 2) {
    const int64_t Gc = ceil_div(O, G);
    int64_t tpc = 1;
    const int64_t grid = 8 * ceil_div(Gc * fwd_chunks(B, Gc, &tpc), 8);
    if (grid > 0x7FFFFFFF || (int64_t)kBT * ldo * out_esz > kMaxRsrcBytes ||
        D * ldx * 2 > kMaxRsrcBytes) {
        set_error("haste_ffi_forward: problem too large (grid %lld, ldo %lld, D*ldx %lld)",
                  (long long)grid, (long long)ldo, (long long)(D * ldx));
        return HASTE_ERR_UNSUPPORTED;
    }
    return HASTE_OK;
}

// O32 (fp16 inputs, fp32 bias and logits) is launched without the BCE epilogue.
template <typename T, int G, int FP, bool O32>
int launch_fwd(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* W,
               const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t B, int64_t D, int64_t F,
               int64_t O, const BceArgs* bce, hipStream_t st) {
    const int rc = check_fwd_size(B, D, ldx, ldo, O, G, O32 ? 4 : 2);
    if (rc != HASTE_OK) return rc;
    const int64_t Gc = ceil_div(O, G);
    int64_t tpc = 1;
    const int64_t nchunks = fwd_chunks(B, Gc, &tpc);
    const int64_t grid = 8 * ceil_div(Gc * nchunks, 8);
    if constexpr (!O32) {
        if (bce != nullptr) {
            ffi_fwd_kernel<T, G, FP, true, false><<<dim3((unsigned)grid), dim3(kThreads), 0, st>>>(
                idx, xT, ldx, W, bias, out, ldo, (int)B, (int)D, (int)F, O, Gc, (int)nchunks,
                (int)tpc, *bce);
            HASTE_CHECK_LAUNCH("haste_ffi_forward");
            return HASTE_OK;
        }
    }
    ffi_fwd_kernel<T, G, FP, false, O32><<<dim3((unsigned)grid), dim3(kThreads), 0, st>>>(
        idx, xT, ldx, W, bias, out, ldo, (int)B, (int)D, (int)F, O, Gc, (int)nchunks, (int)tpc,
        BceArgs{nullptr, 0, nullptr, nullptr});
    HASTE_CHECK_LAUNCH("haste_ffi_forward");
    return HASTE_OK;
}

template <typename T, int G, bool O32>
int dispatch_fp(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* W,
                const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t B, int64_t D, int64_t F,
                int64_t O, const BceArgs* bce, hipStream_t st) {
    if (F <= 32) return launch_fwd<T, G, 32, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
    if (F <= 64) return launch_fwd<T, G, 64, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
    if (F <= 128) return launch_fwd<T, G, 128, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
    return launch_fwd<T, G, 256, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
}

template <typename T, bool O32 = false>
int dispatch_g(const int32_t* idx, const uint16_t* xT, int64_t ldx, const uint16_t* W,
               const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t B, int64_t D, int64_t F,
               int64_t O, int64_t G, const BceArgs* bce, hipStream_t st) {
    switch (G) {
    case 16: return dispatch_fp<T, 16, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
    case 32: return dispatch_fp<T, 32, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
    case 64: return dispatch_fp<T, 64, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
    case 128: return dispatch_fp<T, 128, O32>(idx, xT, ldx, W, bias, out, ldo, B, D, F, O, bce, st);
    default: break;
    }
    set_error("Unsupported group size for FFI kernel. choose from 16,32,64,128 (got %lld)",
              (long long)G);
    return HASTE_ERR_UNSUPPORTED;
}

// Label bits of the COO positives (row, label) pairs, ored into the (all zero)
// bitmap; loss_sum_kernel clears the words again after the forward.  Pairs
// outside [0, B) x [0, O) are ignored.
__global__ __launch_bounds__(256) void label_bits_kernel(const int32_t* __restrict__ labels,
                                                         int64_t nnz, uint32_t* __restrict__ ybits,
                                                         int64_t ldyw, int B, int64_t O) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nnz) return;
    const int r = labels[2 * i], c = labels[2 * i + 1];
    if (r < 0 || r >= B || c < 0 || c >= O) return;
    atomicOr(ybits + (int64_t)r * ldyw + c / 32, 1u << (c % 32));
}

// loss = sum of the n workgroup partials (workgroup 0): each thread sums a
// strided subset in order, then a fixed tree over the threads.  Every
// workgroup also clears the label words of 256 of the call's pairs (one launch
// instead of two small ones).
__global__ __launch_bounds__(256) void loss_sum_kernel(const float* __restrict__ part, int64_t n,
                                                       float* __restrict__ loss,
                                                       const int32_t* __restrict__ labels,
                                                       int64_t nnz, uint32_t* __restrict__ ybits,
                                                       int64_t ldyw, int B, int64_t O) {
    __shared__ float s[256];
    const int64_t li = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (li < nnz) {
        const int r = labels[2 * li], c = labels[2 * li + 1];
        if (r >= 0 && r < B && c >= 0 && c < O) ybits[(int64_t)r * ldyw + c / 32] = 0u;
    }
    if (blockIdx.x != 0) return;
    // the partials in batches of 8 loads in flight, summed in index order
    float v = 0.0f;
    for (int64_t i0 = threadIdx.x; i0 < n; i0 += 8 * 256) {
        float pv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) pv[k] = i0 + k * 256 < n ? part[i0 + k * 256] : 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) v += pv[k];
    }
    s[threadIdx.x] = v;
    __syncthreads();
    for (int m = 128; m >= 1; m >>= 1) {
        if ((int)threadIdx.x < m) s[threadIdx.x] += s[threadIdx.x + m];
        __syncthreads();
    }
    if (threadIdx.x == 0) *loss = s[0];
}

struct BceLayout {
    int64_t ldyw, bits_bytes, nparts, bytes;
};
BceLayout bce_layout(int64_t B, int64_t O, int64_t G) {
    BceLayout L;
    const int64_t Gc = ceil_div(O, G);
    int64_t tpc = 1;
    L.ldyw = ceil_div(Gc * G, 32);
    L.bits_bytes = (B * L.ldyw * 4 + 255) / 256 * 256;
    L.nparts = Gc * fwd_chunks(B, Gc, &tpc);
    L.bytes = L.bits_bytes + L.nparts * 4;
    return L;
}

}  // namespace

// Shape checks shared by the three FFI entry points.
int check_ffi_shape(const char* fn, int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                    int32_t dtype) {
    if (dtype != HASTE_DTYPE_BF16 && dtype != HASTE_DTYPE_F16) {
        set_error("%s: unsupported dtype code %d (bf16 or f16 only)", fn, (int)dtype);
        return HASTE_ERR_UNSUPPORTED;
    }
    if (G != 16 && G != 32 && G != 64 && G != 128) {
        set_error("Unsupported group size for FFI kernel. choose from 16,32,64,128 (got %lld)",
                  (long long)G);
        return HASTE_ERR_UNSUPPORTED;
    }
    if (F % 16 != 0 || F < 16) {
        set_error("FANIN size should be multiple of 16 and >=16 (got %lld)", (long long)F);
        return HASTE_ERR_INVALID_ARG;
    }
    if (F > 256) {
        set_error("FANIN should be <=256 (got %lld)", (long long)F);
        return HASTE_ERR_UNSUPPORTED;
    }
    if (B <= 0) {
        set_error("batch size B must be positive (got %lld)", (long long)B);
        return HASTE_ERR_INVALID_ARG;
    }
    if (B > 0x7FFFFFFF || D <= 0 || D > 0x7FFFFFFF || O <= 0) {
        set_error("%s: invalid sizes B=%lld D=%lld O=%lld", fn, (long long)B, (long long)D,
                  (long long)O);
        return HASTE_ERR_INVALID_ARG;
    }
    (void)fn;
    return HASTE_OK;
}

}  // namespace haste

extern "C" int haste_ffi_forward(const int32_t* idx, const void* xT, int64_t ldx, const void* W,
                                 const void* bias, void* out, int64_t ldo, int64_t B, int64_t D,
                                 int64_t F, int64_t O, int64_t G, int32_t dtype, void* stream) {
    int rc = haste::check_ffi_shape("haste_ffi_forward", B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && xT && W && out, "haste_ffi_forward: null pointer");
    HASTE_CHECK_ARG(ldx >= B && ldx % 8 == 0,
                    "haste_ffi_forward: ldx must be >= B and a multiple of 8 (ldx=%lld B=%lld)",
                    (long long)ldx, (long long)B);
    HASTE_CHECK_ARG(ldo >= O && ldo % 8 == 0,
                    "haste_ffi_forward: ldo must be >= O and a multiple of 8 (ldo=%lld O=%lld)",
                    (long long)ldo, (long long)O);
    HASTE_CHECK_ARG(haste::aligned16(xT) && haste::aligned16(W) && haste::aligned16(out),
                    "haste_ffi_forward: xT, W and out must be 16-byte aligned");
    auto* x = static_cast<const uint16_t*>(xT);
    auto* w = static_cast<const uint16_t*>(W);
    auto* bb = static_cast<const uint16_t*>(bias);
    auto* o = static_cast<uint16_t*>(out);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == HASTE_DTYPE_BF16)
        return haste::dispatch_g<haste::BF16>(idx, x, ldx, w, bb, o, ldo, B, D, F, O, G, nullptr, st);
    return haste::dispatch_g<haste::F16>(idx, x, ldx, w, bb, o, ldo, B, D, F, O, G, nullptr, st);
}

extern "C" int haste_ffi_forward_f16_f32out(const int32_t* idx, const void* xT, int64_t ldx,
                                            const void* W, const float* bias, float* out,
                                            int64_t ldo, int64_t B, int64_t D, int64_t F,
                                            int64_t O, int64_t G, void* stream) {
    int rc = haste::check_ffi_shape("haste_ffi_forward_f16_f32out", B, D, F, O, G, HASTE_DTYPE_F16);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && xT && W && out, "haste_ffi_forward_f16_f32out: null pointer");
    HASTE_CHECK_ARG(ldx >= B && ldx % 8 == 0,
                    "haste_ffi_forward_f16_f32out: ldx must be >= B and a multiple of 8 (ldx=%lld B=%lld)",
                    (long long)ldx, (long long)B);
    HASTE_CHECK_ARG(ldo >= O && ldo % 8 == 0,
                    "haste_ffi_forward_f16_f32out: ldo must be >= O and a multiple of 8 (ldo=%lld O=%lld)",
                    (long long)ldo, (long long)O);
    HASTE_CHECK_ARG(haste::aligned16(xT) && haste::aligned16(W) && haste::aligned16(out) &&
                        (bias == nullptr || reinterpret_cast<uintptr_t>(bias) % 4 == 0),
                    "haste_ffi_forward_f16_f32out: xT, W and out must be 16-byte aligned, bias 4-byte");
    return haste::dispatch_g<haste::F16, true>(
        idx, static_cast<const uint16_t*>(xT), ldx, static_cast<const uint16_t*>(W),
        reinterpret_cast<const uint16_t*>(bias), reinterpret_cast<uint16_t*>(out), ldo, B, D, F, O,
        G, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int64_t haste_ffi_forward_bce_workspace_size(int64_t B, int64_t O, int64_t G) {
    if (B <= 0 || O <= 0 || (G != 16 && G != 32 && G != 64 && G != 128)) return -1;
    return haste::bce_layout(B, O, G).bytes;
}

namespace haste {
namespace {

// Launches of haste_ffi_forward_bce on a checked workspace: label bits, the
// forward with the BCE epilogue, the loss sum (which clears the label bits).
int run_forward_bce(const int32_t* idx, const void* xT, int64_t ldx, const void* W,
                    const void* bias, const int32_t* labels, int64_t nnz, void* dY, int64_t ldo,
                    void* logits, float* loss, void* workspace, const BceLayout& L, int64_t B,
                    int64_t D, int64_t F, int64_t O, int64_t G, int32_t dtype, hipStream_t st) {
    auto* ybits = static_cast<uint32_t*>(workspace);
    float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + L.bits_bytes);
    const int64_t lblocks = (nnz + 255) / 256;
    if (lblocks > 0) {
        label_bits_kernel<<<dim3((unsigned)lblocks), dim3(256), 0, st>>>(labels, nnz, ybits,
                                                                          L.ldyw, (int)B, O);
        HASTE_CHECK_LAUNCH("haste_ffi_forward_bce");
    }
    const BceArgs bce{ybits, L.ldyw, static_cast<uint16_t*>(logits), part};
    auto* x = static_cast<const uint16_t*>(xT);
    auto* w = static_cast<const uint16_t*>(W);
    auto* bb = static_cast<const uint16_t*>(bias);
    auto* o = static_cast<uint16_t*>(dY);
    int rc = dtype == HASTE_DTYPE_BF16
                 ? dispatch_g<BF16>(idx, x, ldx, w, bb, o, ldo, B, D, F, O, G, &bce, st)
                 : dispatch_g<F16>(idx, x, ldx, w, bb, o, ldo, B, D, F, O, G, &bce, st);
    if (rc != HASTE_OK) return rc;
    loss_sum_kernel<<<dim3((unsigned)std::max<int64_t>(1, ceil_div(nnz, 256))), dim3(256), 0, st>>>(
        part, L.nparts, loss, labels, nnz, ybits, L.ldyw, (int)B, O);
    HASTE_CHECK_LAUNCH("haste_ffi_forward_bce");
    return HASTE_OK;
}

// Host-side checks of haste_ffi_forward_bce[_noalloc] except the workspace.
int check_forward_bce(const char* fn, const int32_t* idx, const void* xT, int64_t ldx,
                      const void* W, const int32_t* labels, int64_t nnz, const void* dY,
                      int64_t ldo, const void* logits, const float* loss, int64_t B, int64_t D,
                      int64_t F, int64_t O, int64_t G, int32_t dtype) {
    int rc = check_ffi_shape(fn, B, D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx && xT && W && dY && loss && (labels || nnz == 0) && nnz >= 0,
                    "%s: null pointer or negative nnz", fn);
    HASTE_CHECK_ARG(ldx >= B && ldx % 8 == 0,
                    "%s: ldx must be >= B and a multiple of 8 (ldx=%lld B=%lld)", fn,
                    (long long)ldx, (long long)B);
    HASTE_CHECK_ARG(ldo >= O && ldo % 8 == 0,
                    "%s: ldo must be >= O and a multiple of 8 (ldo=%lld O=%lld)", fn,
                    (long long)ldo, (long long)O);
    HASTE_CHECK_ARG(aligned16(xT) && aligned16(W) && aligned16(dY) &&
                        (logits == nullptr || aligned16(logits)),
                    "%s: xT, W, dY and logits must be 16-byte aligned", fn);
    return check_fwd_size(B, D, ldx, ldo, O, G);
}

// Zeroes n16 16-byte words (a fill kernel: no memset node, so a caller may
// capture the call in a HIP graph).
__global__ __launch_bounds__(256) void zero16_kernel(u32x4* __restrict__ p, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
        p[i] = u32x4{0u, 0u, 0u, 0u};
}

constexpr int kMaxDevices = 64;

}  // namespace
}  // namespace haste

// The workspace of haste_ffi_forward_bce_noalloc: one array per GPU (every
// device that runs the library holds its own copy, at its own address, until
// the process ends).  Host code never passes this name to a kernel: it is a
// host-side stand-in, not the device address; the per-device address comes
// from hipGetSymbolAddress below.
static __device__ __align__(256) uint8_t scratch[HASTE_FORWARD_BCE_SCRATCH_BYTES];

namespace haste {
namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the device of stream st (looked up once per
// device, with that device current).
int scratch_for(hipStream_t st, void** out) {
    int dev = -1;
    if (st != nullptr)
        HASTE_HIP_TRY(hipStreamGetDevice(st, &dev), "haste_ffi_forward_bce_noalloc: stream device");
    else
        HASTE_HIP_TRY(hipGetDevice(&dev), "haste_ffi_forward_bce_noalloc: current device");
    HASTE_CHECK_ARG(dev >= 0 && dev < kMaxDevices,
                    "haste_ffi_forward_bce_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = -1;
        HASTE_HIP_TRY(hipGetDevice(&cur), "haste_ffi_forward_bce_noalloc: current device");
        if (cur != dev) HASTE_HIP_TRY(hipSetDevice(dev), "haste_ffi_forward_bce_noalloc: set device");
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) HASTE_HIP_TRY(hipSetDevice(cur), "haste_ffi_forward_bce_noalloc: set device");
        HASTE_HIP_TRY(e, "haste_ffi_forward_bce_noalloc: hipGetSymbolAddress(scratch)");
        HASTE_CHECK_ARG(p != nullptr && aligned16(p),
                        "haste_ffi_forward_bce_noalloc: bad scratch address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return HASTE_OK;
}

}  // namespace
}  // namespace haste

extern "C" int haste_ffi_forward_bce(const int32_t* idx, const void* xT, int64_t ldx,
                                     const void* W, const void* bias, const int32_t* labels,
                                     int64_t nnz, void* dY, int64_t ldo, void* logits,
                                     float* loss, void* workspace, int64_t ws_bytes, int64_t B,
                                     int64_t D, int64_t F, int64_t O, int64_t G, int32_t dtype,
                                     void* stream) {
    const char* fn = "haste_ffi_forward_bce";
    int rc = haste::check_forward_bce(fn, idx, xT, ldx, W, labels, nnz, dY, ldo, logits, loss, B,
                                      D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(workspace != nullptr && haste::aligned16(workspace),
                    "%s: workspace must be a 16-byte aligned pointer", fn);
    const haste::BceLayout L = haste::bce_layout(B, O, G);
    HASTE_CHECK_ARG(ws_bytes >= L.bytes, "%s: workspace too small (%lld < %lld bytes)", fn,
                    (long long)ws_bytes, (long long)L.bytes);
    return haste::run_forward_bce(idx, xT, ldx, W, bias, labels, nnz, dY, ldo, logits, loss,
                                  workspace, L, B, D, F, O, G, dtype,
                                  static_cast<hipStream_t>(stream));
}

extern "C" int haste_ffi_forward_bce_noalloc(const int32_t* idx, const void* xT, int64_t ldx,
                                             const void* W, const void* bias,
                                             const int32_t* labels, int64_t nnz, void* dY,
                                             int64_t ldo, void* logits, float* loss, int64_t B,
                                             int64_t D, int64_t F, int64_t O, int64_t G,
                                             int32_t dtype, void* stream) {
    const char* fn = "haste_ffi_forward_bce_noalloc";
    int rc = haste::check_forward_bce(fn, idx, xT, ldx, W, labels, nnz, dY, ldo, logits, loss, B,
                                      D, F, O, G, dtype);
    if (rc != HASTE_OK) return rc;
    const haste::BceLayout L = haste::bce_layout(B, O, G);
    if (L.bytes > HASTE_FORWARD_BCE_SCRATCH_BYTES) {
        haste::set_error("%s: B = %lld, O = %lld need %lld bytes of scratch, above the "
                         "library's %lld (use haste_ffi_forward_bce with a workspace)",
                         fn, (long long)B, (long long)O, (long long)L.bytes,
                         (long long)HASTE_FORWARD_BCE_SCRATCH_BYTES);
        return HASTE_ERR_WORKSPACE;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = nullptr;
    rc = haste::scratch_for(st, &ws);
    if (rc != HASTE_OK) return rc;
    // the label bitmap must start at zero; the previous call on this GPU left
    // its own layout in the scratch, so this call's part is cleared here
    const int64_t n16 = L.bits_bytes / 16;
    haste::zero16_kernel<<<dim3((unsigned)std::min<int64_t>(haste::ceil_div(n16, 256), 2048)),
                           dim3(256), 0, st>>>(static_cast<haste::u32x4*>(ws), n16);
    HASTE_CHECK_LAUNCH(fn);
    return haste::run_forward_bce(idx, xT, ldx, W, bias, labels, nnz, dY, ldo, logits, loss, ws,
                                  L, B, D, F, O, G, dtype, st);
}
