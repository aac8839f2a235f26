// On-device rewire (prune + regrow) of a grouped FFI layer (bf16, fp16 or fp32
// weights), gfx950.
//
// Restates GroupFixedFanIn.rewire (shared_ffi/rewire.py:143-239) as one kernel
// with one workgroup per label group and no host synchronisation.  The
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
#include "common.hpp"

namespace haste {
namespace {

constexpr int kThreads = 256;
constexpr int kUnusedTries = 64;

// element i of a tensor of dtype code dt (bf16 / fp16 bit patterns or fp32) as
// fp32 (exact), and stored from fp32 (RNE to the 16-bit formats)
__device__ __forceinline__ float elem_f32(const void* p, int dt, int64_t i) {
    if (dt == HASTE_DTYPE_F32) return static_cast<const float*>(p)[i];
    const uint32_t h = static_cast<const uint16_t*>(p)[i];
    return dt == HASTE_DTYPE_F16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}
__device__ __forceinline__ void store_elem(void* p, int dt, int64_t i, float v) {
    if (dt == HASTE_DTYPE_F32)
        static_cast<float*>(p)[i] = v;
    else
        static_cast<uint16_t*>(p)[i] =
            (uint16_t)(dt == HASTE_DTYPE_F16 ? f32_to_f16_rne(v) : f32_to_bf16_rne(v));
}

// score of slot j of group g over rows [l0, l1): mean or max of |W| or of the
// saliency |W * grad| (grad may be null); pd: dtype of the product (the
// weights' 16-bit format when grad has it too, else fp32: a product of two
// 16-bit values is exact in fp32 and the tensor product rounds it once)
__device__ __forceinline__ float slot_score(const void* __restrict__ W, int wd, const void* grad,
                                            int grad_dtype, int pd, int score_mode, int64_t l0,
                                            int64_t l1, int F, int j) {
    float acc = score_mode == HASTE_SCORE_MAX ? -__builtin_inff() : 0.0f;
    for (int64_t l = l0; l < l1; ++l) {
        const float w = elem_f32(W, wd, l * F + j);
        float v;
        if (grad == nullptr) {
            v = fabsf(w);
        } else {
            const float p = w * elem_f32(grad, grad_dtype, l * F + j);
            v = fabsf(pd == HASTE_DTYPE_BF16 ? bf16_bits_to_f32(f32_to_bf16_rne(p))
                      : pd == HASTE_DTYPE_F16 ? f16_bits_to_f32(f32_to_f16_rne(p))
                                              : p);
        }
        acc = score_mode == HASTE_SCORE_MAX ? fmaxf(acc, v) : acc + v;
    }
    return score_mode == HASTE_SCORE_MAX ? acc : acc / (float)(l1 - l0);
}

__global__ __launch_bounds__(kThreads) void rewire_scores_kernel(
    const void* __restrict__ W, int wd, const void* grad, int grad_dtype, int pd, int score_mode,
    float* __restrict__ scores, int64_t O, int F, int G) {
    const int64_t g = blockIdx.x;
    const int j = threadIdx.x;
    if (j >= F) return;
    const int64_t l0 = g * G, l1 = min(O, l0 + G);
    scores[g * F + j] = slot_score(W, wd, grad, grad_dtype, pd, score_mode, l0, l1, F, j);
}

// scores_in: the layer's scores (GLOBAL_FRACTION, written by rewire_scores_kernel
// with the same value and score modes); key_thr: the k-th smallest key.
__global__ __launch_bounds__(kThreads) void rewire_kernel(
    void* __restrict__ W, int wd, int32_t* __restrict__ idx, float* __restrict__ scores_out,
    int32_t* __restrict__ n_pruned, int64_t O, int F, int G, int D, int prune_mode, float thr,
    int k, int regrow_mode, int init_mode, float bound, uint32_t k0, uint32_t k1,
    const void* grad, int grad_dtype, int pd, int score_mode, const float* __restrict__ scores_in,
    const int64_t* __restrict__ key_thr) {
    __shared__ float sc[256];
    __shared__ int32_t sidx[256];
    __shared__ int mask[256];

    const int64_t g = blockIdx.x;
    const int j = threadIdx.x;
    const int64_t l0 = g * G;
    const int64_t l1 = min(O, l0 + G);
    const bool jv = j < F;

    float score = 0.0f;
    if (jv) {
        score = scores_in != nullptr ? scores_in[g * F + j]
                                     : slot_score(W, wd, grad, grad_dtype, pd, score_mode, l0,
                                                  l1, F, j);
        sc[j] = score;
        sidx[j] = idx[g * F + j];
        if (scores_out) scores_out[g * F + j] = score;
    }
    __syncthreads();

    int m = 0;
    if (jv) {
        if (prune_mode == HASTE_PRUNE_THRESHOLD) {
            m = score < thr;
        } else if (prune_mode == HASTE_PRUNE_GLOBAL_FRACTION) {
            const int64_t key = ((int64_t)__float_as_uint(score) << 32) | (int64_t)(uint32_t)(g * F + j);
            m = key <= *key_thr;
        } else {
            int rank = 0;
            for (int q = 0; q < F; ++q) {
                const float u = sc[q];
                rank += (u < score) || (u == score && q < j);
            }
            m = rank < k;
        }
        mask[j] = m;
    }
    const int count = __syncthreads_count(m);

    if (regrow_mode == HASTE_REGROW_RANDOM) {
        if (m) {
            const uint32_t w0 = philox_w0((uint32_t)(g * F + j), 1u, 0u, k0, k1);
            sidx[j] = (int32_t)(((uint64_t)w0 * (uint64_t)D) >> 32);
        }
    } else {
        for (int jj = 0; jj < F; ++jj) {
            if (!mask[jj]) continue;  // uniform
            uint32_t cand = 0;
            for (int t = 0; t < kUnusedTries; ++t) {
                const uint32_t w0 = philox_w0((uint32_t)(g * F + jj), 1u, (uint32_t)t, k0, k1);
                cand = (uint32_t)(((uint64_t)w0 * (uint64_t)D) >> 32);
                const int used = jv && (!mask[j] || j < jj) && sidx[j] == (int32_t)cand;
                if (!__syncthreads_or(used)) break;
            }
            if (j == 0) sidx[jj] = (int32_t)cand;
            __syncthreads();
        }
    }
    __syncthreads();

    if (m) {
        idx[g * F + j] = sidx[j];
        for (int64_t l = l0; l < l1; ++l) {
            float v = 0.0f;
            if (init_mode == HASTE_INIT_RANDOM) {
                const uint32_t w0 = philox_w0((uint32_t)(l * F + j), 2u, 0u, k0, k1);
                const float u01 = (float)(w0 >> 8) * 0x1p-24f;
                v = __builtin_fmaf(u01, 2.0f * bound, -bound);
            }
            store_elem(W, wd, l * F + j, v);
        }
    }
    if (j == 0 && n_pruned != nullptr && count > 0) atomicAdd(n_pruned, count);
}

}  // namespace
}  // namespace haste

namespace haste {
namespace {
bool weight_dtype_ok(int32_t wd) {
    return wd == HASTE_DTYPE_BF16 || wd == HASTE_DTYPE_F16 || wd == HASTE_DTYPE_F32;
}
// dtype of W * grad in torch's promotion: one 16-bit format for both, else fp32
int product_dtype(int32_t wd, const void* grad, int32_t gd) {
    return grad != nullptr && gd == wd ? wd : HASTE_DTYPE_F32;
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
    const int64_t Gc = haste::ceil_div(O, G);
    hipStream_t st = static_cast<hipStream_t>(stream);
    haste::rewire_kernel<<<dim3((unsigned)Gc), dim3(haste::kThreads), 0, st>>>(
        W, w_dtype, idx, scores_out, n_pruned, O, (int)F, (int)G, (int)D, prune_mode, threshold,
        (int)k, regrow_mode, init_mode, bound, (uint32_t)seed, (uint32_t)(seed >> 32), nullptr,
        HASTE_DTYPE_F32, HASTE_DTYPE_F32, HASTE_SCORE_MEAN, nullptr, nullptr);
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
    haste::rewire_scores_kernel<<<dim3((unsigned)Gc), dim3(haste::kThreads), 0,
                                  static_cast<hipStream_t>(stream)>>>(
        W, w_dtype, grad, grad_dtype, haste::product_dtype(w_dtype, grad, grad_dtype), score_mode,
        scores, O, (int)F, (int)G);
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
    const int64_t Gc = haste::ceil_div(O, G);
    haste::rewire_kernel<<<dim3((unsigned)Gc), dim3(haste::kThreads), 0,
                           static_cast<hipStream_t>(stream)>>>(
        W, w_dtype, idx, scores_out, n_pruned, O, (int)F, (int)G, (int)D, prune_mode, threshold,
        (int)k, regrow_mode, init_mode, bound, (uint32_t)seed, (uint32_t)(seed >> 32), grad,
        grad_dtype, haste::product_dtype(w_dtype, grad, grad_dtype), score_mode, scores_in,
        key_thr);
    HASTE_CHECK_LAUNCH("haste_rewire_ex");
    return HASTE_OK;
}
