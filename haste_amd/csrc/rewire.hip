// On-device rewire (prune + regrow) of a grouped FFI layer (bf16, fp16 or fp32
// weights), gfx950.
//
// Restates GroupFixedFanIn.rewire (shared_ffi/rewire.py:143-239) as one or two
// kernel launches with no host synchronisation.  The
// reference's random draws (torch.randint / uniform_ on the device generator)
// and its topk(sorted=False) tie order cannot be reproduced, so the contract
// is fixed here (and restated bit-for-bit by the CPU oracle):
//   score[g, j] = (fp32 sum over rows l of g, ascending, of |W[l, j]|) / rows
//   prune:  THRESHOLD -> score < threshold;  FRACTION -> k smallest (score, j)
// haste_rewire_scores / haste_rewire_ex add the application's variant
// (GroupFixedFanInReal.rewire, src/group_fanin_real.py:150-286):
//   value v[l, j] = |W| or, with a gradient, the saliency |W * grad| in torch's
//           promoted dtype of the two (group_fanin_real.py:199-204): the exact
//           fp32 product rounded to bf16 / fp16 when both are that format, else
//           the fp32 product
//   score  MEAN -> fp32 sum over rows (ascending) / rows;  MAX -> max over rows
//   prune  GLOBAL_FRACTION -> the k smallest keys (bits(score) << 32 | g*F + j)
//           over all slots of the layer, i.e. key <= the k-th smallest key,
//           which the caller selects on the device from the scores
//   regrow: RANDOM -> d = (philox(seed; g*F+j, 1, 0).w0 * D) >> 32
//           UNUSED -> attempts t = 0..63 with counter (g*F+j, 1, t); first
//           candidate not used by the group (kept slots and slots regrown
//           earlier in ascending j); else the last candidate
//   weights at pruned slots, every row: ZERO -> 0; RANDOM ->
//           fma((w0 >> 8) * 2^-24, 2*bound, -bound), w0 = philox(seed; l*F+j, 2, 0).w0,
//           stored in W's dtype (RNE to bf16 / fp16; as is for fp32: the
//           reference draws uniform_ in the weights' dtype, rewire.py:224-237)
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"

// Layout and schedule.  A group g holds rows [g*G, min(O, g*G + G)) of W,
// contiguous in HBM; 256-thread workgroups, a persistent grid (as many
// workgroups as fit on the device, each taking groups b, b + gridDim.x, ...,
// one atomic per workgroup for the pruned count):
//   1. score: the group's rows are copied into LDS with 16-byte loads (in row
//      chunks of up to kStageMax bytes; with a gradient W and grad take half
//      each); thread j then sums / maxes column j in ascending row order;
//   2. prune mask: FRACTION ranks each slot's score with kThreads / F threads
//      per slot;
//   3. new weights: where every group fits one LDS stage with its rows on
//      16-byte boundaries (rewire_whole_kernel), the next group's rows are
//      loaded while the current one is scored, and the pruned columns take
//      their new values as the staged group goes back with 16-byte stores;
//      otherwise (rewire_kernel) each pruned slot's column is stored element
//      by element;
//   4. regrow: RANDOM in the same pass; UNUSED in rewire_regrow_kernel, one
//      wave per group, the pass above having marked the pruned slots -1.
namespace haste {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnusedTries = 64;
constexpr int kStagePieces = 9;                          // 16-byte loads per thread per chunk
constexpr int kStageMax = kStagePieces * kThreads * 16;  // 36 KiB
constexpr int kMiscBytes = 3 * kThreads * 4;             // scores, rank counts, prune mask
constexpr int kSlotsPerLane = 4;                         // F <= 256 slots over one wave

// Element access by dtype code: S the storage word, f() exact to fp32, t() from
// fp32 (RNE to the 16-bit formats, as is for fp32); rp() rounds an exact
// product of two values of the format to the format (one rounding, so the
// compiler may fuse it with the multiply).
template <int DT>
struct El;
template <>
struct El<HASTE_DTYPE_BF16> {
    static constexpr int es = 2;
    using S = uint16_t;
    __device__ static float f(S h) { return bf16_bits_to_f32(h); }
    __device__ static S t(float v) { return (S)f32_to_bf16_rne(v); }
    __device__ static float rp(float p) { return bf16_bits_to_f32(f32_to_bf16_rne(p)); }
};
template <>
struct El<HASTE_DTYPE_F16> {
    static constexpr int es = 2;
    using S = uint16_t;
    __device__ static float f(S h) { return f16_bits_to_f32(h); }
    __device__ static S t(float v) { return (S)f32_to_f16_rne(v); }
    __device__ static float rp(float p) { return (float)(_Float16)p; }
};
template <>
struct El<HASTE_DTYPE_F32> {
    static constexpr int es = 4;
    using S = uint32_t;
    __device__ static float f(S h) { return __uint_as_float(h); }
    __device__ static S t(float v) { return __float_as_uint(v); }
};

// Copies bytes [off, off + n) of a tensor of tot bytes at base into LDS at
// dst + (off & 15), with 16-byte loads from the 16-byte multiple below off
// (n <= kStageMax - 30); returns off & 15.  The one piece that runs past the
// tensor's end (tot - (off & ~15) not a multiple of 16) reads as zeros from the
// buffer resource and is then filled element by element.
__device__ __forceinline__ int stage_bytes(char* dst, const void* base, int64_t tot, int64_t off,
                                           int n, int tid) {
    const int64_t a = off & ~(int64_t)15;
    const int head = (int)(off - a);
    const int np = (head + n + 15) >> 4;
    const char* src = static_cast<const char*>(base) + a;
    const int64_t avail = tot - a;
    const rsrc_t rs = make_rsrc(src, avail);
    const int pe = ((avail & 15) != 0 && (avail >> 4) < np) ? (int)(avail >> 4) : -1;
    u32x4 v[kStagePieces];
#pragma unroll
    for (int i = 0; i < kStagePieces; ++i) {
        if (i * kThreads < np) {
            const int p = tid + i * kThreads;
            v[i] = buf_load16(rs, p < np ? (uint32_t)p * 16u : kOOB);
        }
    }
#pragma unroll
    for (int i = 0; i < kStagePieces; ++i) {
        if (i * kThreads < np) {
            const int p = tid + i * kThreads;
            if (p == pe) {
                const uint16_t* s = reinterpret_cast<const uint16_t*>(src + 16 * (int64_t)p);
                const int nh = (int)(avail & 15) >> 1;
                uint32_t h[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = e < nh ? (uint32_t)s[e] : 0u;
                v[i] = u32x4{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16,
                             h[6] | h[7] << 16};
            }
            if (p < np) *reinterpret_cast<u32x4*>(dst + 16 * p) = v[i];
        }
    }
    return head;
}

// Sum (or max) over `rows` staged rows of column j of |W| or of the saliency
// |W * grad| (GD < 0: no gradient).  The product takes torch's promoted dtype
// of the two: the shared 16-bit format when both have it (the exact fp32
// product rounded once), else fp32.
template <int WD, int GD, bool MAX>
__device__ __forceinline__ float column_score(const char* ws, const char* gs, int rows, int F,
                                              int j, float acc) {
    using Wt = El<WD>;
    const typename Wt::S* wp = reinterpret_cast<const typename Wt::S*>(ws) + j;
#pragma unroll 8
    for (int r = 0; r < rows; ++r) {
        const float w = Wt::f(wp[r * F]);
        float v;
        if constexpr (GD < 0) {
            v = fabsf(w);
        } else {
            using Gt = El<GD < 0 ? HASTE_DTYPE_F32 : GD>;
            const float p = w * Gt::f(reinterpret_cast<const typename Gt::S*>(gs)[r * F + j]);
            if constexpr (GD == WD && WD != HASTE_DTYPE_F32)
                v = fabsf(Wt::rp(p));
            else
                v = fabsf(p);
        }
        acc = MAX ? fmaxf(acc, v) : acc + v;
    }
    return acc;
}

template <int WD, bool MAX>
__device__ __forceinline__ float column_score_g(const char* ws, const char* gs, int gd, bool has_g,
                                                int rows, int F, int j, float acc) {
    if (!has_g) return column_score<WD, -1, MAX>(ws, gs, rows, F, j, acc);
    if (gd == HASTE_DTYPE_BF16) return column_score<WD, HASTE_DTYPE_BF16, MAX>(ws, gs, rows, F, j, acc);
    if (gd == HASTE_DTYPE_F16) return column_score<WD, HASTE_DTYPE_F16, MAX>(ws, gs, rows, F, j, acc);
    return column_score<WD, HASTE_DTYPE_F32, MAX>(ws, gs, rows, F, j, acc);
}

// Score of slot j (threads j >= F return 0) of the group with rows [l0, l1),
// in row chunks of R rows staged at stw (and stg for grad).
template <int WD>
__device__ __forceinline__ float group_score(char* stw, char* stg, const void* W, int64_t wtot, const void* grad,
                             int gd, int64_t gtot, int score_mode, int64_t l0, int64_t l1, int F,
                             int R, int tid) {
    const bool mx = score_mode == HASTE_SCORE_MAX;
    const bool has_g = grad != nullptr;
    const int esg = gd == HASTE_DTYPE_F32 ? 4 : 2;
    float acc = mx ? -__builtin_inff() : 0.0f;
    for (int64_t r0 = l0; r0 < l1; r0 += R) {
        const int rows = (int)min((int64_t)R, l1 - r0);
        if (r0 != l0) __syncthreads();  // readers of the previous chunk are done
        const int hw = stage_bytes(stw, W, wtot, r0 * F * El<WD>::es, rows * F * El<WD>::es, tid);
        int hg = 0;
        if (has_g) hg = stage_bytes(stg, grad, gtot, r0 * F * esg, rows * F * esg, tid);
        __syncthreads();
        if (tid < F)
            acc = mx ? column_score_g<WD, true>(stw + hw, stg + hg, gd, has_g, rows, F, tid, acc)
                     : column_score_g<WD, false>(stw + hw, stg + hg, gd, has_g, rows, F, tid, acc);
    }
    return mx ? acc : acc / (float)(l1 - l0);
}

// New value of W[l, j] at a pruned slot.
__device__ __forceinline__ float init_value(int init_mode, int64_t l, int F, int j, float bound,
                                            uint32_t k0, uint32_t k1) {
    if (init_mode != HASTE_INIT_RANDOM) return 0.0f;
    const uint32_t w0 = philox_w0((uint32_t)(l * F + j), 2u, 0u, k0, k1);
    const float u01 = (float)(w0 >> 8) * 0x1p-24f;
    return __builtin_fmaf(u01, 2.0f * bound, -bound);
}

// Rank of slot j's score among the group's F scores in sc (ties go to the
// lower slot), counted by P = kThreads / F threads per slot (thread t: slot
// t % F, share t / F of the slots compared against); part: kThreads ints of
// LDS.  Every thread calls it (it holds a barrier); threads t < F get the rank.
__device__ __forceinline__ int slot_rank(const float* sc, int* part, int F, int tid) {
    const int P = kThreads / F;
    const int j = tid % F, share = tid / F;
    int cnt = 0;
    if (share < P) {
        const float s = sc[j];
        const int q1 = (share + 1) * F / P;
#pragma unroll 8
        for (int q = share * F / P; q < q1; ++q) {
            const float u = sc[q];
            cnt += (u < s) || (u == s && q < j);
        }
    }
    part[tid] = cnt;
    __syncthreads();
    int rank = 0;
    if (tid < F)
        for (int sh = 0; sh < P; ++sh) rank += part[tid + sh * F];
    return rank;
}

// A 16-byte piece holding W[l, c .. c + 16/es - 1] with its pruned elements
// (bit e of bits: element c + e) set to their new values.
template <int WD>
__device__ __forceinline__ u32x4 reset_piece(u32x4 x, uint32_t bits, int init_mode, int64_t l,
                                             int F, int c, float bound, uint32_t k0,
                                             uint32_t k1) {
    using Wt = El<WD>;
    constexpr int EPP = 16 / Wt::es;
    if (init_mode != HASTE_INIT_RANDOM) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t clear;
            if constexpr (Wt::es == 2)
                clear = ((bits >> (2 * w)) & 1u ? 0xFFFFu : 0u) |
                        ((bits >> (2 * w + 1)) & 1u ? 0xFFFF0000u : 0u);
            else
                clear = (bits >> w) & 1u ? 0xFFFFFFFFu : 0u;
            x[w] &= ~clear;
        }
        return x;
    }
#pragma unroll
    for (int e = 0; e < EPP; ++e) {
        if ((bits >> e) & 1u) {
            const uint32_t h = Wt::t(init_value(init_mode, l, F, c + e, bound, k0, k1));
            if constexpr (Wt::es == 2)
                x[e >> 1] = (e & 1) ? (x[e >> 1] & 0xFFFFu) | (h << 16)
                                    : (x[e >> 1] & 0xFFFF0000u) | h;
            else
                x[e] = h;
        }
    }
    return x;
}

// The thread's pieces p = tid + kThreads*i (i < NPT, p < np) of a staged group
// back to the group's range rw, the pruned slots (mw: the prune mask bits of
// slots 0..255) with their new values.  Every piece goes back, not only those
// that hold pruned slots: whole cache lines are written that way (skipping the
// others measured 8 % slower at config 4, where every line holds some pruned
// slot anyway).  (r, cb): row and byte-in-row of piece i, advanced by
// (step_r, step_b) per piece.
template <int WD, int NPT, bool RANDOM>
__device__ __forceinline__ void write_pieces(const char* stw, rsrc_t rw, const uint64_t (&mw)[4],
                                             int np, int r, int cb, int step_r, int step_b,
                                             int rowb, int tid, int64_t l0, int F, float bound,
                                             uint32_t k0, uint32_t k1) {
    using Wt = El<WD>;
    constexpr int EPP = 16 / Wt::es;
    constexpr int kUnroll = RANDOM ? 1 : NPT;
#pragma unroll kUnroll
    for (int i = 0; i < NPT; ++i) {
        const int p = tid + i * kThreads;
        const int c = cb / Wt::es;
        const uint64_t word = c < 64 ? mw[0] : c < 128 ? mw[1] : c < 192 ? mw[2] : mw[3];
        const uint32_t bits = (uint32_t)(word >> (c & 63)) & ((1u << EPP) - 1u);
        const bool wr = p < np;
        u32x4 x = {0u, 0u, 0u, 0u};
        if (wr)
            x = reset_piece<WD>(*reinterpret_cast<const u32x4*>(stw + 16 * p), bits,
                                RANDOM ? HASTE_INIT_RANDOM : HASTE_INIT_ZERO, l0 + r, F, c, bound,
                                k0, k1);
        buf_store16(x, rw, wr ? (uint32_t)p * 16u : kOOB);
        r += step_r;
        cb += step_b;
        if (cb >= rowb) {
            cb -= rowb;
            ++r;
        }
    }
}

// 16-byte pieces p = tid + kThreads*i (i < NPT) of the byte range of rs;
// pieces past its end read as zeros.
template <int NPT>
__device__ __forceinline__ void load_pieces(u32x4 (&v)[NPT], rsrc_t rs, int tid) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) v[i] = buf_load16(rs, (uint32_t)(tid + i * kThreads) * 16u);
}

// Whole groups: every group's rows fit one LDS stage (NPT pieces of 16 bytes
// per thread) and start and end on 16-byte boundaries, no gradient, scores
// computed here.  A persistent grid: workgroup b takes groups b, b + gridDim.x,
// ...; the next group's rows and indices are loaded into registers while the
// current group is scored from LDS; a group with pruned slots goes back whole
// with 16-byte stores; one atomic per workgroup adds its pruned count.  Pruned
// slots of idx get their RANDOM regrow index here, or -1 for the UNUSED pass
// (rewire_regrow_kernel).  All global accesses go through buffer
// resources with out-of-range offsets for the ones a lane skips, so that the
// loads of the next group are waited for by count.
template <int WD, int NPT>
__global__ __launch_bounds__(kThreads, 4) void rewire_whole_kernel(
    void* __restrict__ W, int32_t* __restrict__ idx, float* __restrict__ scores_out,
    int32_t* __restrict__ n_pruned, int64_t O, int F, int G, int D, int prune_mode, float thr,
    int k, int regrow_mode, int init_mode, float bound, uint32_t k0, uint32_t k1, int score_mode,
    int64_t Gc) {
    using Wt = El<WD>;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    float* sc = reinterpret_cast<float*>(smem);
    int* part = reinterpret_cast<int*>(smem + kThreads * 4);
    uint64_t* mb = reinterpret_cast<uint64_t*>(smem + 2 * kThreads * 4);
    char* stw = smem + kMiscBytes;
    const int tid = threadIdx.x;
    const bool jv = tid < F;
    const int rowb = F * Wt::es;  // a multiple of 16
    char* Wc = static_cast<char*>(W);
    const bool mx = score_mode == HASTE_SCORE_MAX;

    auto w_rsrc = [&](int64_t gg) {
        const int64_t rows = gg < Gc ? min((int64_t)G, O - gg * G) : 0;
        return make_rsrc_u32(Wc + (gg < Gc ? gg : 0) * G * rowb, (uint32_t)(rows * rowb));
    };

    // row and byte-in-row of the thread's first piece; the next piece is
    // step_r rows and step_b bytes on (the same in every group)
    const int step_r = 16 * kThreads / rowb, step_b = 16 * kThreads % rowb;
    const int r_first = 16 * tid / rowb, cb_first = 16 * tid % rowb;

    int total = 0;
    int64_t g = blockIdx.x;
    u32x4 v[NPT];
    load_pieces(v, w_rsrc(g), tid);
    for (; g < Gc; g += gridDim.x) {
        const int64_t l0 = g * G;
        const int rows = (int)min((int64_t)G, O - l0);
        const int np = rows * rowb / 16;
        __syncthreads();  // the previous group's readers of LDS are done
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
            const int p = tid + i * kThreads;
            if (p < np) *reinterpret_cast<u32x4*>(stw + 16 * p) = v[i];
        }
        __syncthreads();
        load_pieces(v, w_rsrc(g + gridDim.x), tid);

        float score = 0.0f;
        if (jv) {
            score = mx ? column_score<WD, -1, true>(stw, nullptr, rows, F, tid, -__builtin_inff())
                       : column_score<WD, -1, false>(stw, nullptr, rows, F, tid, 0.0f) /
                             (float)rows;
            sc[tid] = score;
        }
        buf_store4(__float_as_uint(score),
                   make_rsrc_u32(scores_out + (scores_out ? g * F : 0), scores_out ? F * 4u : 0u),
                   (uint32_t)tid * 4u);
        int m;
        if (prune_mode == HASTE_PRUNE_FRACTION) {
            __syncthreads();
            m = slot_rank(sc, part, F, tid) < k && jv;
        } else {
            m = jv && score < thr;
        }
        const uint64_t bal = __ballot(m);
        if ((tid & 63) == 0) mb[tid >> 6] = bal;
        __syncthreads();
        const uint64_t m0 = mb[0], m1 = mb[1], m2 = mb[2], m3 = mb[3];
        total += __popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3);

        const rsrc_t rw = w_rsrc(g);
        const uint64_t mw[4] = {m0, m1, m2, m3};
        const int npw = (m0 | m1 | m2 | m3) != 0 ? np : 0;  // a group with nothing pruned stays
        if (init_mode == HASTE_INIT_RANDOM)  // a Philox draw per element: one piece at a time
            write_pieces<WD, NPT, true>(stw, rw, mw, npw, r_first, cb_first, step_r, step_b, rowb,
                                        tid, l0, F, bound, k0, k1);
        else
            write_pieces<WD, NPT, false>(stw, rw, mw, npw, r_first, cb_first, step_r, step_b,
                                         rowb, tid, l0, F, bound, k0, k1);
        int32_t ni = -1;
        if (m && regrow_mode == HASTE_REGROW_RANDOM)
            ni = (int32_t)(((uint64_t)philox_w0((uint32_t)(g * F + tid), 1u, 0u, k0, k1) *
                            (uint64_t)D) >> 32);
        buf_store4((uint32_t)ni, make_rsrc_u32(idx + g * F, (uint32_t)F * 4u),
                   m ? (uint32_t)tid * 4u : kOOB);
    }
    if (tid == 0 && total != 0 && n_pruned != nullptr) atomicAdd(n_pruned, total);
}

template <int WD>
__global__ __launch_bounds__(kThreads) void rewire_scores_kernel(
    const void* __restrict__ W, const void* grad, int grad_dtype, int score_mode,
    float* __restrict__ scores, int64_t O, int F, int G, int R, int stage_w) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* stw = smem + kMiscBytes;
    char* stg = stw + stage_w;
    const int64_t g = blockIdx.x;
    const int64_t l0 = g * G, l1 = min(O, l0 + G);
    const int esg = grad_dtype == HASTE_DTYPE_F32 ? 4 : 2;
    const float s = group_score<WD>(stw, stg, W, O * F * El<WD>::es, grad, grad_dtype,
                                    O * F * esg, score_mode, l0, l1, F, R, threadIdx.x);
    if ((int)threadIdx.x < F) scores[g * F + threadIdx.x] = s;
}

// Every other case (rows over several LDS chunks, rows off 16-byte boundaries,
// a gradient, or the layer's scores given): a persistent grid over the groups,
// each scored in row chunks (or read from scores_in), the pruned slots' new
// weights stored element by element down their columns, one atomic per
// workgroup.  scores_in: the layer's scores (GLOBAL_FRACTION, written by
// rewire_scores_kernel with the same value and score modes); key_thr: the k-th
// smallest key.  Pruned slots of idx as in rewire_whole_kernel.
template <int WD>
__global__ __launch_bounds__(kThreads) void rewire_kernel(
    void* __restrict__ W, int32_t* __restrict__ idx, float* __restrict__ scores_out,
    int32_t* __restrict__ n_pruned, int64_t O, int F, int G, int D, int prune_mode, float thr,
    int k, int regrow_mode, int init_mode, float bound, uint32_t k0, uint32_t k1,
    const void* grad, int grad_dtype, int score_mode, const float* __restrict__ scores_in,
    const int64_t* __restrict__ key_thr, int R, int stage_w, int64_t Gc) {
    using Wt = El<WD>;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    float* sc = reinterpret_cast<float*>(smem);
    int* part = reinterpret_cast<int*>(smem + kThreads * 4);
    char* stw = smem + kMiscBytes;
    char* stg = stw + stage_w;
    const int j = threadIdx.x;
    const bool jv = j < F;
    const int esg = grad_dtype == HASTE_DTYPE_F32 ? 4 : 2;

    int total = 0;
    for (int64_t g = blockIdx.x; g < Gc; g += gridDim.x) {
        const int64_t l0 = g * G;
        const int64_t l1 = min(O, l0 + G);
        const int rows = (int)(l1 - l0);
        __syncthreads();  // the previous group's readers of LDS are done
        float score = 0.0f;
        if (scores_in != nullptr) {
            if (jv) score = scores_in[g * F + j];
        } else {
            score = group_score<WD>(stw, stg, W, O * F * Wt::es, grad, grad_dtype, O * F * esg,
                                    score_mode, l0, l1, F, R, j);
        }
        if (jv) {
            sc[j] = score;
            if (scores_out) scores_out[g * F + j] = score;
        }
        int m = 0;
        if (prune_mode == HASTE_PRUNE_FRACTION) {
            __syncthreads();
            m = slot_rank(sc, part, F, j) < k && jv;
        } else if (prune_mode == HASTE_PRUNE_GLOBAL_FRACTION) {
            const int64_t key =
                ((int64_t)__float_as_uint(score) << 32) | (int64_t)(uint32_t)(g * F + j);
            m = jv && key <= *key_thr;
        } else {
            m = jv && score < thr;
        }
        total += __syncthreads_count(m);
        if (m) {
            typename Wt::S* col = static_cast<typename Wt::S*>(W) + l0 * F + j;
            for (int r = 0; r < rows; ++r)
                col[(int64_t)r * F] = Wt::t(init_value(init_mode, l0 + r, F, j, bound, k0, k1));
            idx[g * F + j] =
                regrow_mode == HASTE_REGROW_RANDOM
                    ? (int32_t)(((uint64_t)philox_w0((uint32_t)(g * F + j), 1u, 0u, k0, k1) *
                                 (uint64_t)D) >> 32)
                    : -1;
        }
    }
    if (j == 0 && total != 0 && n_pruned != nullptr) atomicAdd(n_pruned, total);
}

// UNUSED regrow, after a prune pass left -1 at the pruned slots of idx (their
// old indices take no part in it): one wave per group (kWaves groups per workgroup), the group's slots in
// registers (slot lane + 64*s in register s).  Each pruned slot jj, ascending,
// takes the first of its candidates (attempt t: counter (g*F + jj, 1, t)) that
// no kept slot and no pruned slot below jj holds, else its last candidate;
// every first candidate is drawn up front in parallel, one wave ballot per
// candidate checked.
__global__ __launch_bounds__(kThreads) void rewire_regrow_kernel(int32_t* __restrict__ idx,
                                                                 int64_t Gc, int F, int D,
                                                                 uint32_t k0, uint32_t k1) {
    const int64_t g = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (g >= Gc) return;
    const int lane = threadIdx.x & 63;
    const uint32_t gF = (uint32_t)(g * F);
    int32_t cur[kSlotsPerLane];
    bool pr[kSlotsPerLane];
    uint32_t c0[kSlotsPerLane];
#pragma unroll
    for (int s = 0; s < kSlotsPerLane; ++s) {
        const int j2 = lane + 64 * s;
        cur[s] = j2 < F ? idx[g * F + j2] : 0;
        pr[s] = cur[s] < 0;
        c0[s] = 0;
        if (pr[s])
            c0[s] = (uint32_t)(((uint64_t)philox_w0(gF + j2, 1u, 0u, k0, k1) * (uint64_t)D) >> 32);
    }
#pragma unroll
    for (int s = 0; s < kSlotsPerLane; ++s) {
        if (64 * s >= F) break;
        uint64_t bits = __ballot(pr[s]);
        while (bits != 0) {
            const int ln = __builtin_ctzll(bits);
            bits &= bits - 1;
            const int jj = 64 * s + ln;
            uint32_t cand = __builtin_amdgcn_readlane(c0[s], ln);
            for (int t = 1; t < kUnusedTries; ++t) {
                bool used = false;
#pragma unroll
                for (int s2 = 0; s2 < kSlotsPerLane; ++s2) {
                    const int j2 = lane + 64 * s2;
                    used |= j2 < F && (!pr[s2] || j2 < jj) && cur[s2] == (int32_t)cand;
                }
                if (__ballot(used) == 0) break;
                cand = (uint32_t)(((uint64_t)philox_w0(gF + jj, 1u, (uint32_t)t, k0, k1) *
                                   (uint64_t)D) >> 32);
            }
            if (lane == ln) cur[s] = (int32_t)cand;
        }
    }
#pragma unroll
    for (int s = 0; s < kSlotsPerLane; ++s)
        if (pr[s]) idx[g * F + lane + 64 * s] = cur[s];
}

}  // namespace
}  // namespace haste

namespace haste {
namespace {
bool weight_dtype_ok(int32_t wd) {
    return wd == HASTE_DTYPE_BF16 || wd == HASTE_DTYPE_F16 || wd == HASTE_DTYPE_F32;
}
int elem_bytes(int32_t dt) { return dt == HASTE_DTYPE_F32 ? 4 : 2; }

// Row chunk (R rows) and LDS stage sizes for a launch: with a gradient W and
// grad get half of kStageMax each.
struct StagePlan {
    int R, stage_w, lds;
};
StagePlan stage_plan(int32_t wd, const void* grad, int32_t gd, int64_t F, int64_t G) {
    const int esw = elem_bytes(wd), esg = grad ? elem_bytes(gd) : 0;
    const int cap = grad ? kStageMax / 2 : kStageMax;
    const int64_t R = std::min<int64_t>(G, (cap - 16) / (F * std::max(esw, esg)));
    auto stage = [&](int es) { return (int)((R * F * es + 30) / 16 * 16); };
    StagePlan p;
    p.R = (int)R;
    p.stage_w = stage(esw);
    p.lds = kMiscBytes + p.stage_w + (grad ? stage(esg) : 0);
    return p;
}

// Workgroups of a persistent launch: as many as can be resident at once, at
// most one per group.  The answers are kept per (device, kernel, LDS bytes):
// the occupancy query costs more host time than the launch itself.
int64_t persistent_grid(const void* fn, int lds, int64_t Gc) {
    struct Entry {
        int dev;
        const void* fn;
        int lds;
        int64_t blocks;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return std::min<int64_t>(Gc, 1024);
    {
        std::lock_guard<std::mutex> lock(mu);
        for (const Entry& e : cache)
            if (e.dev == dev && e.fn == fn && e.lds == lds) return std::min(Gc, e.blocks);
    }
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, lds) != hipSuccess)
        return std::min<int64_t>(Gc, 1024);
    const int64_t blocks = (int64_t)std::max(cus, 1) * std::max(per_cu, 1);
    std::lock_guard<std::mutex> lock(mu);
    cache.push_back({dev, fn, lds, blocks});
    return std::min(Gc, blocks);
}

struct RewireArgs {
    void* W;
    int32_t wd;
    int32_t* idx;
    float* scores_out;
    int32_t* n_pruned;
    int64_t O, F, G, D;
    int prune_mode;
    float thr;
    int64_t k;
    int regrow_mode, init_mode;
    float bound;
    uint64_t seed;
    const void* grad;
    int gd, score_mode;
    const float* scores_in;
    const int64_t* key_thr;
};

template <int WD, int NPT>
void launch_whole(const RewireArgs& a, int64_t Gc, hipStream_t st) {
    const void* fn = reinterpret_cast<const void*>(&rewire_whole_kernel<WD, NPT>);
    const int lds = kMiscBytes + (int)(a.G * a.F * El<WD>::es);
    rewire_whole_kernel<WD, NPT><<<dim3((unsigned)persistent_grid(fn, lds, Gc)), dim3(kThreads),
                                   lds, st>>>(
        a.W, a.idx, a.scores_out, a.n_pruned, a.O, (int)a.F, (int)a.G, (int)a.D, a.prune_mode,
        a.thr, (int)a.k, a.regrow_mode, a.init_mode, a.bound, (uint32_t)a.seed,
        (uint32_t)(a.seed >> 32), a.score_mode, Gc);
}

template <int WD>
void launch_rewire(const RewireArgs& a, int64_t Gc, hipStream_t st) {
    const int es = El<WD>::es;
    if (a.scores_in == nullptr && a.grad == nullptr && (a.F * es) % 16 == 0 &&
        a.G * a.F * es <= kStageMax && aligned16(a.W)) {
        switch ((int)((a.G * a.F * es + 16 * kThreads - 1) / (16 * kThreads))) {
            case 1: launch_whole<WD, 1>(a, Gc, st); break;
            case 2: launch_whole<WD, 2>(a, Gc, st); break;
            case 3: launch_whole<WD, 3>(a, Gc, st); break;
            case 4: launch_whole<WD, 4>(a, Gc, st); break;
            case 5: launch_whole<WD, 5>(a, Gc, st); break;
            case 6: launch_whole<WD, 6>(a, Gc, st); break;
            case 7: launch_whole<WD, 7>(a, Gc, st); break;
            case 8: launch_whole<WD, 8>(a, Gc, st); break;
            default: launch_whole<WD, kStagePieces>(a, Gc, st); break;
        }
        return;
    }
    const StagePlan sp = stage_plan(WD, a.grad, a.gd, a.F, a.G);
    const int lds = a.scores_in != nullptr ? kMiscBytes : sp.lds;
    const void* fn = reinterpret_cast<const void*>(&rewire_kernel<WD>);
    rewire_kernel<WD><<<dim3((unsigned)persistent_grid(fn, lds, Gc)), dim3(kThreads), lds, st>>>(
        a.W, a.idx, a.scores_out, a.n_pruned, a.O, (int)a.F, (int)a.G, (int)a.D, a.prune_mode,
        a.thr, (int)a.k, a.regrow_mode, a.init_mode, a.bound, (uint32_t)a.seed,
        (uint32_t)(a.seed >> 32), a.grad, a.gd, a.score_mode, a.scores_in, a.key_thr, sp.R,
        sp.stage_w, Gc);
}

// The prune pass (whole-group or general kernel), then the UNUSED regrow pass.
int rewire_dispatch(const RewireArgs& a, hipStream_t st) {
    const int64_t Gc = ceil_div(a.O, a.G);
    if (a.wd == HASTE_DTYPE_BF16)
        launch_rewire<HASTE_DTYPE_BF16>(a, Gc, st);
    else if (a.wd == HASTE_DTYPE_F16)
        launch_rewire<HASTE_DTYPE_F16>(a, Gc, st);
    else
        launch_rewire<HASTE_DTYPE_F32>(a, Gc, st);
    if (a.regrow_mode == HASTE_REGROW_UNUSED)
        rewire_regrow_kernel<<<dim3((unsigned)ceil_div(Gc, kWaves)), dim3(kThreads), 0, st>>>(
            a.idx, Gc, (int)a.F, (int)a.D, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
    return HASTE_OK;
}
}  // namespace
}  // namespace haste

extern "C" int haste_rewire(void* W, int32_t w_dtype, int32_t* idx, float* scores_out,
                            int32_t* n_pruned,
                            int64_t O, int64_t F, int64_t G, int64_t D, int32_t prune_mode,
                            float threshold, int64_t k, int32_t regrow_mode, int32_t init_mode,
                            float bound, uint64_t seed, void* stream) {
    HASTE_CHECK_ARG(W && idx, "haste_rewire: null pointer");
    HASTE_CHECK_ARG(haste::weight_dtype_ok(w_dtype),
                    "haste_rewire: weights must be bf16, fp16 or fp32 (dtype code %d)",
                    (int)w_dtype);
    HASTE_CHECK_ARG(F >= 1 && F <= 256, "haste_rewire: fan_in must be in [1, 256] (got %lld)",
                    (long long)F);
    HASTE_CHECK_ARG(G >= 1 && O >= 1 && D >= 1 && D <= 0x7FFFFFFF,
                    "haste_rewire: invalid sizes O=%lld G=%lld D=%lld", (long long)O,
                    (long long)G, (long long)D);
    HASTE_CHECK_ARG(O * F < ((int64_t)1 << 32),
                    "haste_rewire: O*F must be < 2^32 (Philox counter width)");
    HASTE_CHECK_ARG(prune_mode == HASTE_PRUNE_THRESHOLD || prune_mode == HASTE_PRUNE_FRACTION,
                    "haste_rewire: bad prune mode %d", (int)prune_mode);
    HASTE_CHECK_ARG(regrow_mode == HASTE_REGROW_RANDOM || regrow_mode == HASTE_REGROW_UNUSED,
                    "haste_rewire: bad regrow mode %d", (int)regrow_mode);
    HASTE_CHECK_ARG(init_mode == HASTE_INIT_ZERO || init_mode == HASTE_INIT_RANDOM,
                    "haste_rewire: bad init mode %d", (int)init_mode);
    HASTE_CHECK_ARG(k >= 0 && k <= F, "haste_rewire: k must be in [0, F] (got %lld)", (long long)k);
    const haste::RewireArgs a{W,         w_dtype,   idx,         scores_out, n_pruned,
                              O,         F,         G,           D,          prune_mode,
                              threshold, k,         regrow_mode, init_mode,  bound,
                              seed,      nullptr,   HASTE_DTYPE_F32, HASTE_SCORE_MEAN,
                              nullptr,   nullptr};
    haste::rewire_dispatch(a, static_cast<hipStream_t>(stream));
    HASTE_CHECK_LAUNCH("haste_rewire");
    return HASTE_OK;
}

namespace {
int check_scores_args(const char* fn, const void* W, int32_t w_dtype, int64_t O, int64_t F,
                      int64_t G, const void* grad, int32_t grad_dtype, int32_t score_mode) {
    HASTE_CHECK_ARG(W != nullptr, "%s: null pointer", fn);
    HASTE_CHECK_ARG(haste::weight_dtype_ok(w_dtype),
                    "%s: weights must be bf16, fp16 or fp32 (dtype code %d)", fn, (int)w_dtype);
    HASTE_CHECK_ARG(F >= 1 && F <= 256, "%s: fan_in must be in [1, 256] (got %lld)", fn,
                    (long long)F);
    HASTE_CHECK_ARG(G >= 1 && O >= 1, "%s: invalid sizes O=%lld G=%lld", fn, (long long)O,
                    (long long)G);
    HASTE_CHECK_ARG(O * F < ((int64_t)1 << 32), "%s: O*F must be < 2^32", fn);
    HASTE_CHECK_ARG(score_mode == HASTE_SCORE_MEAN || score_mode == HASTE_SCORE_MAX,
                    "%s: bad score mode %d", fn, (int)score_mode);
    HASTE_CHECK_ARG(grad == nullptr || haste::weight_dtype_ok(grad_dtype),
                    "%s: grad dtype must be bf16, fp16 or fp32 (got %d)", fn, (int)grad_dtype);
    return HASTE_OK;
}
}  // namespace

extern "C" int haste_rewire_scores(const void* W, int32_t w_dtype, const void* grad,
                                   int32_t grad_dtype, int32_t score_mode, float* scores,
                                   int64_t O, int64_t F, int64_t G, void* stream) {
    int rc = check_scores_args("haste_rewire_scores", W, w_dtype, O, F, G, grad, grad_dtype,
                               score_mode);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(scores != nullptr, "haste_rewire_scores: null scores");
    const int64_t Gc = haste::ceil_div(O, G);
    const haste::StagePlan sp = haste::stage_plan(w_dtype, grad, grad_dtype, F, G);
    hipStream_t st = static_cast<hipStream_t>(stream);
#define HASTE_RS_LAUNCH(WD)                                                                     \
    haste::rewire_scores_kernel<WD><<<dim3((unsigned)Gc), dim3(haste::kThreads), sp.lds, st>>>( \
        W, grad, grad_dtype, score_mode, scores, O, (int)F, (int)G, sp.R, sp.stage_w)
    if (w_dtype == HASTE_DTYPE_BF16)
        HASTE_RS_LAUNCH(HASTE_DTYPE_BF16);
    else if (w_dtype == HASTE_DTYPE_F16)
        HASTE_RS_LAUNCH(HASTE_DTYPE_F16);
    else
        HASTE_RS_LAUNCH(HASTE_DTYPE_F32);
#undef HASTE_RS_LAUNCH
    HASTE_CHECK_LAUNCH("haste_rewire_scores");
    return HASTE_OK;
}

extern "C" int haste_rewire_ex(void* W, int32_t w_dtype, int32_t* idx, const void* grad,
                               int32_t grad_dtype,
                               int32_t score_mode, const float* scores_in,
                               const int64_t* key_thr, float* scores_out, int32_t* n_pruned,
                               int64_t O, int64_t F, int64_t G, int64_t D, int32_t prune_mode,
                               float threshold, int64_t k, int32_t regrow_mode,
                               int32_t init_mode, float bound, uint64_t seed, void* stream) {
    int rc = check_scores_args("haste_rewire_ex", W, w_dtype, O, F, G, grad, grad_dtype,
                               score_mode);
    if (rc != HASTE_OK) return rc;
    HASTE_CHECK_ARG(idx != nullptr, "haste_rewire_ex: null idx");
    HASTE_CHECK_ARG(D >= 1 && D <= 0x7FFFFFFF, "haste_rewire_ex: invalid D=%lld", (long long)D);
    HASTE_CHECK_ARG(prune_mode == HASTE_PRUNE_THRESHOLD || prune_mode == HASTE_PRUNE_FRACTION ||
                        prune_mode == HASTE_PRUNE_GLOBAL_FRACTION,
                    "haste_rewire_ex: bad prune mode %d", (int)prune_mode);
    HASTE_CHECK_ARG(prune_mode != HASTE_PRUNE_GLOBAL_FRACTION ||
                        (scores_in != nullptr && key_thr != nullptr),
                    "haste_rewire_ex: GLOBAL_FRACTION needs scores_in and key_thr");
    HASTE_CHECK_ARG(regrow_mode == HASTE_REGROW_RANDOM || regrow_mode == HASTE_REGROW_UNUSED,
                    "haste_rewire_ex: bad regrow mode %d", (int)regrow_mode);
    HASTE_CHECK_ARG(init_mode == HASTE_INIT_ZERO || init_mode == HASTE_INIT_RANDOM,
                    "haste_rewire_ex: bad init mode %d", (int)init_mode);
    HASTE_CHECK_ARG(prune_mode != HASTE_PRUNE_FRACTION || (k >= 0 && k <= F),
                    "haste_rewire_ex: k must be in [0, F] (got %lld)", (long long)k);
    const haste::RewireArgs a{W,         w_dtype,   idx,         scores_out, n_pruned,
                              O,         F,         G,           D,          prune_mode,
                              threshold, k,         regrow_mode, init_mode,  bound,
                              seed,      grad,      grad_dtype,  score_mode, scores_in,
                              key_thr};
    haste::rewire_dispatch(a, static_cast<hipStream_t>(stream));
    HASTE_CHECK_LAUNCH("haste_rewire_ex");
    return HASTE_OK;
}
