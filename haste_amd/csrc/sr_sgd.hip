// Stochastic rounding and the fused SGD(+momentum, +weight decay) step.
//
// Both are single HBM passes over contiguous tensors.  Random bits follow
// Triton's tl.randint(seed, offset) (Philox4x32-10, word 0, counter = offset),
// so results are bit-identical to the reference's Triton kernels
// (shared_ffi/sr_triton.py:9-16, 27-59, 109-213) under the FMA contract
//   g' = fma(wd, w, g);  m' = fma(mu, m, g');  w' = fma(-lr, m' or g', w).
#include <algorithm>

#include "common.hpp"

namespace haste {
namespace {

constexpr int kVec = 8;  // elements per thread per iteration (16 B of bf16)

template <int GD>
__device__ __forceinline__ void load_grad8(const void* g, int64_t i, float out[kVec]) {
    if constexpr (GD == HASTE_DTYPE_F32) {
        const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(g) + i);
        f32x4 a = __builtin_nontemporal_load(p);
        f32x4 b = __builtin_nontemporal_load(p + 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) { out[e] = a[e]; out[4 + e] = b[e]; }
    } else {
        const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(g) + i);
        u32x4 v = __builtin_nontemporal_load(p);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t lo = v[q] & 0xFFFFu, hi = v[q] >> 16;
            out[2 * q] = GD == HASTE_DTYPE_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
            out[2 * q + 1] = GD == HASTE_DTYPE_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
    }
}

template <int GD>
__device__ __forceinline__ float load_grad1(const void* g, int64_t i) {
    if constexpr (GD == HASTE_DTYPE_F32) {
        return static_cast<const float*>(g)[i];
    } else {
        uint32_t h = static_cast<const uint16_t*>(g)[i];
        return GD == HASTE_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    }
}

// One launch updates up to kMaxSegs tensors ("segments"), each with its own
// offset base; every thread handles kVec consecutive elements of one segment
// (16-byte vector loads when the segment is aligned, element loads for the
// segment's tail or an unaligned segment), so a tensor needs no second launch
// for its tail and several small tensors (weights + bias) share one launch.
constexpr int kMaxSegs = 8;
constexpr int kSgdThreads = 256;
constexpr int64_t kSegBlockElems = (int64_t)kSgdThreads * kVec;

struct SgdSeg {
    uint16_t* w;
    const void* g;
    float* m;
    int64_t n;
    uint64_t off0;
    int64_t blk0;  // first block of this segment
    int32_t vec;   // 16-byte aligned w, g (and m)
};
struct SgdBatch {
    SgdSeg s[kMaxSegs];
    int32_t count;
};

// WF16: fp16 weights (an fp16 w_ptr in _sgd_m_wd_sr): read as fp16, and the
// bf16 result of the update stored as fp16 (round to nearest even).
template <bool WF16>
__device__ __forceinline__ float w_to_f32(uint32_t h) {
    return WF16 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}
template <bool WF16>
__device__ __forceinline__ uint32_t w_store_bits(uint32_t bf) {
    return WF16 ? f32_to_f16_rne(bf16_bits_to_f32(bf)) : bf;
}

template <int GD, bool USE_MOM, bool DO_SR, bool WF16>
__global__ __launch_bounds__(kSgdThreads) void sgd_sr_kernel(const SgdBatch b, float lr, float wd,
                                                             float mu, uint64_t seed) {
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    int t = 0;
#pragma unroll
    for (int k = 1; k < kMaxSegs; ++k)
        if (k < b.count && (int64_t)blockIdx.x >= b.s[k].blk0) t = k;
    uint16_t* __restrict__ w = b.s[t].w;
    const void* __restrict__ g = b.s[t].g;
    float* __restrict__ m = b.s[t].m;
    const int64_t n = b.s[t].n;
    const uint64_t offset0 = b.s[t].off0;
    const int64_t i = ((int64_t)blockIdx.x - b.s[t].blk0) * kSegBlockElems +
                      (int64_t)threadIdx.x * kVec;
    if (b.s[t].vec && i + kVec <= n) {
        u32x4 wv = *reinterpret_cast<const u32x4*>(w + i);
        float gf[kVec];
        load_grad8<GD>(g, i, gf);
        float mv[kVec];
        if constexpr (USE_MOM) {
            f32x4 a = reinterpret_cast<const f32x4*>(m + i)[0];
            f32x4 c = reinterpret_cast<const f32x4*>(m + i)[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) { mv[e] = a[e]; mv[4 + e] = c[e]; }
        }
        uint32_t outb[kVec];
#pragma unroll
        for (int e = 0; e < kVec; ++e) {
            uint32_t wb = (e & 1) ? (wv[e >> 1] >> 16) : (wv[e >> 1] & 0xFFFFu);
            outb[e] = w_store_bits<WF16>(sgd_one(w_to_f32<WF16>(wb), gf[e], &mv[e], USE_MOM, lr,
                                                 wd, mu, DO_SR, offset0 + (uint64_t)(i + e), k0, k1));
        }
        u32x4 ov;
#pragma unroll
        for (int q = 0; q < 4; ++q) ov[q] = outb[2 * q] | (outb[2 * q + 1] << 16);
        *reinterpret_cast<u32x4*>(w + i) = ov;
        if constexpr (USE_MOM) {
            f32x4 a, c;
#pragma unroll
            for (int e = 0; e < 4; ++e) { a[e] = mv[e]; c[e] = mv[4 + e]; }
            reinterpret_cast<f32x4*>(m + i)[0] = a;
            reinterpret_cast<f32x4*>(m + i)[1] = c;
        }
    } else {
        for (int e = 0; e < kVec; ++e) {
            const int64_t j = i + e;
            if (j >= n) break;
            float mv = USE_MOM ? m[j] : 0.f;
            w[j] = (uint16_t)w_store_bits<WF16>(sgd_one(w_to_f32<WF16>(w[j]), load_grad1<GD>(g, j),
                                                        &mv, USE_MOM, lr, wd, mu, DO_SR,
                                                        offset0 + (uint64_t)j, k0, k1));
            if (USE_MOM) m[j] = mv;
        }
    }
}

struct SgdTensor {
    uint16_t* w;
    const void* g;
    float* m;
    int64_t n;
    uint64_t offset0;
};

template <int GD, bool WF16>
int launch_sgd(const SgdTensor* ts, int count, float lr, float wd, float mu, int use_mom,
               int do_sr, uint64_t seed, hipStream_t st) {
    for (int base = 0; base < count; base += kMaxSegs) {
        SgdBatch b{};
        int64_t blocks = 0;
        int c = 0;
        for (int k = base; k < count && c < kMaxSegs; ++k) {
            if (ts[k].n == 0) continue;
            SgdSeg& s = b.s[c++];
            s.w = ts[k].w;
            s.g = ts[k].g;
            s.m = ts[k].m;
            s.n = ts[k].n;
            s.off0 = ts[k].offset0;
            s.blk0 = blocks;
            s.vec = aligned16(s.w) && aligned16(s.g) && (!use_mom || aligned16(s.m));
            blocks += ceil_div(s.n, kSegBlockElems);
        }
        b.count = c;
        if (c == 0) continue;
        HASTE_CHECK_ARG(blocks < (int64_t)1 << 31, "haste_sgd_sr_step: tensors too large");
#define HASTE_SGD_LAUNCH(UM, SR)                                                               \
    sgd_sr_kernel<GD, UM, SR, WF16><<<dim3((unsigned)blocks), dim3(kSgdThreads), 0, st>>>(   \
        b, lr, wd, mu, seed)
        if (use_mom && do_sr) HASTE_SGD_LAUNCH(true, true);
        else if (use_mom) HASTE_SGD_LAUNCH(true, false);
        else if (do_sr) HASTE_SGD_LAUNCH(false, true);
        else HASTE_SGD_LAUNCH(false, false);
#undef HASTE_SGD_LAUNCH
        HASTE_CHECK_LAUNCH("haste_sgd_sr_step");
    }
    return HASTE_OK;
}

// SR fp32 -> bf16 over one tensor; vector loads when aligned, element loads for the tail.
__global__ __launch_bounds__(256) void sr_round_kernel(const float* __restrict__ x,
                                                       uint16_t* __restrict__ out, int64_t n,
                                                       int32_t vec, uint32_t k0, uint32_t k1,
                                                       uint64_t offset0) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kVec;
    if (vec && i + kVec <= n) {
        f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + i));
        f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + i) + 1);
        float xf[kVec] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        uint32_t ob[kVec];
#pragma unroll
        for (int e = 0; e < kVec; ++e) {
            uint64_t off = offset0 + (uint64_t)(i + e);
            ob[e] = sr_bf16(xf[e], philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1));
        }
        u32x4 ov;
#pragma unroll
        for (int q = 0; q < 4; ++q) ov[q] = ob[2 * q] | (ob[2 * q + 1] << 16);
        *reinterpret_cast<u32x4*>(out + i) = ov;
    } else {
        for (int e = 0; e < kVec; ++e) {
            const int64_t j = i + e;
            if (j >= n) break;
            uint64_t off = offset0 + (uint64_t)j;
            out[j] = (uint16_t)sr_bf16(x[j], philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u,
                                                       k0, k1));
        }
    }
}

// ---- fp16 and fp8 outputs, fp8 weights (sr_triton.py:18-25,43-46,146,167-168)
// OCP fp8: E4M3 "fn" (bias 7, no infinities, S.1111.111 NaN, largest finite
// 448 = 0x7E) and E5M2 (bias 15, IEEE infinities / NaNs, largest finite
// 57344 = 0x7B).
template <int FMT>
struct F8Fmt {
    static constexpr int M = FMT == HASTE_DTYPE_F8E4M3 ? 3 : 2;
    static constexpr int bias = FMT == HASTE_DTYPE_F8E4M3 ? 7 : 15;
    static constexpr uint32_t maxcode = FMT == HASTE_DTYPE_F8E4M3 ? 0x7Eu : 0x7Bu;
    // 2^(M - emin): the smallest subnormal is 1 / sub_scale
    static constexpr float sub_scale = FMT == HASTE_DTYPE_F8E4M3 ? 512.0f : 65536.0f;
};

// fp8 code -> fp32, exact.
template <int FMT>
__device__ __forceinline__ float f8_to_f32(uint32_t c) {
    using F = F8Fmt<FMT>;
    const uint32_t s = (c & 0x80u) << 24;
    const uint32_t e = (c & 0x7Fu) >> F::M, m = c & ((1u << F::M) - 1u);
    const uint32_t normal = s | ((e + 127u - F::bias) << 23) | (m << (23 - F::M));
    const float sub = (float)m * (1.0f / F::sub_scale);
    float v = e == 0 ? __uint_as_float(s | __float_as_uint(sub)) : __uint_as_float(normal);
    if constexpr (FMT == HASTE_DTYPE_F8E4M3)
        v = (c & 0x7Fu) == 0x7Fu ? __uint_as_float(s | 0x7FC00000u) : v;
    else
        v = e == 31u ? __uint_as_float(s | 0x7F800000u | (m ? 0x400000u : 0u)) : v;
    return v;
}

// fp32 -> fp8, round to nearest even, saturating: finite overflow and
// infinities give the largest finite value with the sign kept; NaN gives
// sign | 0x7F.  Below the smallest normal the code is the value in units of the
// smallest subnormal, rounded to nearest even (2^M being the smallest normal).
template <int FMT>
__device__ __forceinline__ uint32_t f32_to_f8(float f) {
    using F = F8Fmt<FMT>;
    constexpr int rb = 23 - F::M;
    const uint32_t u = __float_as_uint(f), s = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
    const uint32_t sub = (uint32_t)__builtin_rintf(__uint_as_float(a) * F::sub_scale);
    const uint32_t nrm = ((a + ((1u << (rb - 1)) - 1u) + ((a >> rb) & 1u)) >> rb) -
                         ((uint32_t)(127 - F::bias) << F::M);
    uint32_t code = a < (uint32_t)(128 - F::bias) << 23 ? sub : min(nrm, F::maxcode);
    code = a >= 0x7F800000u ? (a == 0x7F800000u ? F::maxcode : 0x7Fu) : code;
    return s | code;
}

// The output code of stochastic_rounding for output dtype OUT.
template <int OUT>
__device__ __forceinline__ uint32_t sr_code(float x, uint32_t r) {
    if constexpr (OUT == HASTE_DTYPE_F8E4M3) {
        const uint32_t u = __float_as_uint(x);
        const uint32_t nan = ((u >> 24) & 0x80u) | 0x7Fu;
        const uint32_t c = f32_to_f8<HASTE_DTYPE_F8E4M3>(__uint_as_float((u + (r & 0xFFFFFu)) & 0xFFF00000u));
        return (u & 0x7FFFFFFFu) > 0x7F800000u ? nan : c;
    } else {
        const uint32_t b = sr_bf16(x, r);
        if constexpr (OUT == HASTE_DTYPE_F16) return f32_to_f16_rne(bf16_bits_to_f32(b));
        else if constexpr (OUT == HASTE_DTYPE_F8E5M2) return f32_to_f8<OUT>(bf16_bits_to_f32(b));
        else return b;
    }
}

// SR of one tensor to output dtype OUT (2- or 1-byte codes), 8 elements per thread.
template <int OUT>
__global__ __launch_bounds__(256) void sr_round_any_kernel(const float* __restrict__ x,
                                                           void* __restrict__ out, int64_t n,
                                                           int32_t vec, uint32_t k0, uint32_t k1,
                                                           uint64_t offset0) {
    constexpr bool B1 = OUT == HASTE_DTYPE_F8E4M3 || OUT == HASTE_DTYPE_F8E5M2;
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kVec;
    if (vec && i + kVec <= n) {
        const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + i));
        const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + i) + 1);
        const float xf[kVec] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        uint32_t c[kVec];
#pragma unroll
        for (int e = 0; e < kVec; ++e) {
            const uint64_t off = offset0 + (uint64_t)(i + e);
            c[e] = sr_code<OUT>(xf[e], philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1));
        }
        if constexpr (B1) {
            *reinterpret_cast<u32x2*>(static_cast<uint8_t*>(out) + i) =
                u32x2{c[0] | c[1] << 8 | c[2] << 16 | c[3] << 24,
                      c[4] | c[5] << 8 | c[6] << 16 | c[7] << 24};
        } else {
            *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + i) =
                u32x4{c[0] | c[1] << 16, c[2] | c[3] << 16, c[4] | c[5] << 16, c[6] | c[7] << 16};
        }
    } else {
        for (int e = 0; e < kVec; ++e) {
            const int64_t j = i + e;
            if (j >= n) break;
            const uint64_t off = offset0 + (uint64_t)j;
            const uint32_t c =
                sr_code<OUT>(x[j], philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1));
            if constexpr (B1) static_cast<uint8_t*>(out)[j] = (uint8_t)c;
            else static_cast<uint16_t*>(out)[j] = (uint16_t)c;
        }
    }
}

// The SGD step of sgd_sr_kernel on one tensor of fp8 weights: loaded exactly,
// the bf16 result stored as fp8 (f32_to_f8).
template <int GD, bool USE_MOM, bool DO_SR, int FMT>
__global__ __launch_bounds__(kSgdThreads) void sgd_sr_f8_kernel(
    uint8_t* __restrict__ w, const void* __restrict__ g, float* __restrict__ m, int64_t n,
    int32_t vec, float lr, float wd, float mu, uint64_t seed, uint64_t offset0) {
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    const int64_t i = ((int64_t)blockIdx.x * kSgdThreads + threadIdx.x) * kVec;
    auto one = [&](uint32_t wc, float gf, float* mv, int64_t j) __attribute__((always_inline)) {
        return f32_to_f8<FMT>(bf16_bits_to_f32(sgd_one(f8_to_f32<FMT>(wc), gf, mv, USE_MOM, lr, wd,
                                                      mu, DO_SR, offset0 + (uint64_t)j, k0, k1)));
    };
    if (vec && i + kVec <= n) {
        const u32x2 wv = *reinterpret_cast<const u32x2*>(w + i);
        float gf[kVec];
        load_grad8<GD>(g, i, gf);
        float mv[kVec];
        if constexpr (USE_MOM) {
            const f32x4 a = reinterpret_cast<const f32x4*>(m + i)[0];
            const f32x4 c = reinterpret_cast<const f32x4*>(m + i)[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) { mv[e] = a[e]; mv[4 + e] = c[e]; }
        }
        uint32_t oc[kVec];
#pragma unroll
        for (int e = 0; e < kVec; ++e) oc[e] = one((wv[e >> 2] >> (8 * (e & 3))) & 0xFFu, gf[e], &mv[e], i + e);
        *reinterpret_cast<u32x2*>(w + i) = u32x2{oc[0] | oc[1] << 8 | oc[2] << 16 | oc[3] << 24,
                                                 oc[4] | oc[5] << 8 | oc[6] << 16 | oc[7] << 24};
        if constexpr (USE_MOM) {
            reinterpret_cast<f32x4*>(m + i)[0] = f32x4{mv[0], mv[1], mv[2], mv[3]};
            reinterpret_cast<f32x4*>(m + i)[1] = f32x4{mv[4], mv[5], mv[6], mv[7]};
        }
    } else {
        for (int e = 0; e < kVec; ++e) {
            const int64_t j = i + e;
            if (j >= n) break;
            float mv = USE_MOM ? m[j] : 0.f;
            w[j] = (uint8_t)one(w[j], load_grad1<GD>(g, j), &mv, j);
            if (USE_MOM) m[j] = mv;
        }
    }
}

// The tl.randint words of the SR and SR-SGD kernels alone: thread t draws the
// words of offsets 64t .. 64t+63 (those below n) and writes their XOR, so the
// kernel is bound by the Philox arithmetic (4 bytes written per 64 words).
constexpr int kFoldWords = 64;
__global__ __launch_bounds__(256) void sr_words_fold_kernel(uint32_t* __restrict__ fold, int64_t n,
                                                            uint32_t k0, uint32_t k1) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t i0 = t * kFoldWords;
    if (i0 >= n) return;
    uint32_t acc = 0u;
    if (i0 + kFoldWords <= n) {
#pragma unroll 4
        for (int e = 0; e < kFoldWords; ++e) {
            const uint64_t off = (uint64_t)(i0 + e);
            acc ^= philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1);
        }
    } else {
        for (int64_t i = i0; i < n; ++i)
            acc ^= philox_w0((uint32_t)i, (uint32_t)((uint64_t)i >> 32), 0u, k0, k1);
    }
    fold[t] = acc;
}

}  // namespace

int sr_round_bf16(const float* x, uint16_t* out, int64_t n, uint64_t seed, uint64_t offset0,
                  hipStream_t st) {
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    const int64_t blocks = ceil_div(n, (int64_t)256 * kVec);
    HASTE_CHECK_ARG(blocks < (int64_t)1 << 31, "haste_sr_round_bf16: tensor too large");
    sr_round_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        x, out, n, aligned16(x) && aligned16(out), k0, k1, offset0);
    HASTE_CHECK_LAUNCH("haste_sr_round_bf16");
    return HASTE_OK;
}

}  // namespace haste

extern "C" int haste_sr_words_fold(uint32_t* fold, int64_t n, uint64_t seed, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sr_words_fold: n must be >= 0 (got %lld)", (long long)n);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(fold != nullptr, "haste_sr_words_fold: null pointer");
    const int64_t threads = haste::ceil_div(n, (int64_t)haste::kFoldWords);
    const int64_t blocks = haste::ceil_div(threads, (int64_t)256);
    HASTE_CHECK_ARG(blocks < (int64_t)1 << 31, "haste_sr_words_fold: n too large");
    haste::sr_words_fold_kernel<<<dim3((unsigned)blocks), dim3(256), 0,
                                  static_cast<hipStream_t>(stream)>>>(fold, n, (uint32_t)seed,
                                                                      (uint32_t)(seed >> 32));
    HASTE_CHECK_LAUNCH("haste_sr_words_fold");
    return HASTE_OK;
}

extern "C" int haste_sr_round_bf16(const float* x, uint16_t* out, int64_t n, uint64_t seed,
                                   uint64_t offset0, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sr_round_bf16: n must be >= 0 (got %lld)", (long long)n);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(x != nullptr && out != nullptr, "haste_sr_round_bf16: null pointer");
    return haste::sr_round_bf16(x, out, n, seed, offset0, static_cast<hipStream_t>(stream));
}

extern "C" int haste_sr_round(const float* x, void* out, int32_t out_dtype, int64_t n,
                              uint64_t seed, uint64_t offset0, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sr_round: n must be >= 0 (got %lld)", (long long)n);
    HASTE_CHECK_ARG(out_dtype == HASTE_DTYPE_BF16 || out_dtype == HASTE_DTYPE_F16 ||
                        out_dtype == HASTE_DTYPE_F8E4M3 || out_dtype == HASTE_DTYPE_F8E5M2,
                    "haste_sr_round: output dtype must be bf16, fp16, fp8 e4m3 or fp8 e5m2 "
                    "(dtype code %d)", (int)out_dtype);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(x != nullptr && out != nullptr, "haste_sr_round: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (out_dtype == HASTE_DTYPE_BF16)
        return haste::sr_round_bf16(x, static_cast<uint16_t*>(out), n, seed, offset0, st);
    const int64_t blocks = haste::ceil_div(n, (int64_t)256 * haste::kVec);
    HASTE_CHECK_ARG(blocks < (int64_t)1 << 31, "haste_sr_round: tensor too large");
    const bool b1 = out_dtype != HASTE_DTYPE_F16;
    const int32_t vec = haste::aligned16(x) &&
                        (reinterpret_cast<uintptr_t>(out) & (b1 ? 7u : 15u)) == 0;
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#define HASTE_SR_LAUNCH(OUT)                                                             \
    haste::sr_round_any_kernel<OUT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, out, n, \
                                                                              vec, k0, k1, \
                                                                              offset0)
    if (out_dtype == HASTE_DTYPE_F16) HASTE_SR_LAUNCH(HASTE_DTYPE_F16);
    else if (out_dtype == HASTE_DTYPE_F8E4M3) HASTE_SR_LAUNCH(HASTE_DTYPE_F8E4M3);
    else HASTE_SR_LAUNCH(HASTE_DTYPE_F8E5M2);
#undef HASTE_SR_LAUNCH
    HASTE_CHECK_LAUNCH("haste_sr_round");
    return HASTE_OK;
}

namespace {
template <int FMT, int GD>
void launch_sgd_f8(uint8_t* w, const void* g, float* m, int64_t n, int64_t blocks, int32_t vec,
                   float lr, float wd, float mu, int32_t use_mom, int32_t do_sr, uint64_t seed,
                   uint64_t offset0, hipStream_t st) {
#define HASTE_SGD8_LAUNCH(UM, SR)                                                           \
    haste::sgd_sr_f8_kernel<GD, UM, SR, FMT><<<dim3((unsigned)blocks),                    \
                                               dim3(haste::kSgdThreads), 0, st>>>(         \
        w, g, m, n, vec, lr, wd, mu, seed, offset0)
    if (use_mom && do_sr) HASTE_SGD8_LAUNCH(true, true);
    else if (use_mom) HASTE_SGD8_LAUNCH(true, false);
    else if (do_sr) HASTE_SGD8_LAUNCH(false, true);
    else HASTE_SGD8_LAUNCH(false, false);
#undef HASTE_SGD8_LAUNCH
}
template <int FMT>
int sgd_f8_dispatch(uint8_t* w, const void* g, int32_t g_dtype, float* m, int64_t n,
                    int64_t blocks, int32_t vec, float lr, float wd, float mu, int32_t use_mom,
                    int32_t do_sr, uint64_t seed, uint64_t offset0, hipStream_t st) {
    switch (g_dtype) {
    case HASTE_DTYPE_BF16:
        launch_sgd_f8<FMT, HASTE_DTYPE_BF16>(w, g, m, n, blocks, vec, lr, wd, mu, use_mom, do_sr, seed, offset0, st);
        break;
    case HASTE_DTYPE_F16:
        launch_sgd_f8<FMT, HASTE_DTYPE_F16>(w, g, m, n, blocks, vec, lr, wd, mu, use_mom, do_sr, seed, offset0, st);
        break;
    case HASTE_DTYPE_F32:
        launch_sgd_f8<FMT, HASTE_DTYPE_F32>(w, g, m, n, blocks, vec, lr, wd, mu, use_mom, do_sr, seed, offset0, st);
        break;
    default:
        haste::set_error("haste_sgd_sr_step_f8: unsupported gradient dtype code %d", (int)g_dtype);
        return HASTE_ERR_UNSUPPORTED;
    }
    HASTE_CHECK_LAUNCH("haste_sgd_sr_step_f8");
    return HASTE_OK;
}
}  // namespace

extern "C" int haste_sgd_sr_step_f8(uint8_t* w, int32_t w_dtype, const void* g, int32_t g_dtype,
                                    float* m, int64_t n, float lr, float wd, float mu,
                                    int32_t use_mom, int32_t do_sr, uint64_t seed,
                                    uint64_t offset0, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sgd_sr_step_f8: n must be >= 0 (got %lld)", (long long)n);
    HASTE_CHECK_ARG(w_dtype == HASTE_DTYPE_F8E4M3 || w_dtype == HASTE_DTYPE_F8E5M2,
                    "haste_sgd_sr_step_f8: weights must be fp8 e4m3 or e5m2 (dtype code %d)",
                    (int)w_dtype);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(w != nullptr && g != nullptr, "haste_sgd_sr_step_f8: null pointer");
    HASTE_CHECK_ARG(!use_mom || m != nullptr, "haste_sgd_sr_step_f8: momentum buffer is NULL");
    const int64_t blocks = haste::ceil_div(n, haste::kSegBlockElems);
    HASTE_CHECK_ARG(blocks < (int64_t)1 << 31, "haste_sgd_sr_step_f8: tensor too large");
    const int32_t vec = (reinterpret_cast<uintptr_t>(w) & 7u) == 0 && haste::aligned16(g) &&
                        (!use_mom || haste::aligned16(m));
    hipStream_t st = static_cast<hipStream_t>(stream);
    return w_dtype == HASTE_DTYPE_F8E4M3
               ? sgd_f8_dispatch<HASTE_DTYPE_F8E4M3>(w, g, g_dtype, m, n, blocks, vec, lr, wd,
                                                     mu, use_mom, do_sr, seed, offset0, st)
               : sgd_f8_dispatch<HASTE_DTYPE_F8E5M2>(w, g, g_dtype, m, n, blocks, vec, lr, wd,
                                                     mu, use_mom, do_sr, seed, offset0, st);
}

namespace {
template <bool WF16 = false>
int sgd_dispatch(const haste::SgdTensor* ts, int count, int32_t g_dtype, float lr, float wd,
                 float mu, int32_t use_mom, int32_t do_sr, uint64_t seed, hipStream_t st,
                 const char* fn) {
    switch (g_dtype) {
    case HASTE_DTYPE_BF16:
        return haste::launch_sgd<HASTE_DTYPE_BF16, WF16>(ts, count, lr, wd, mu, use_mom, do_sr, seed, st);
    case HASTE_DTYPE_F16:
        return haste::launch_sgd<HASTE_DTYPE_F16, WF16>(ts, count, lr, wd, mu, use_mom, do_sr, seed, st);
    case HASTE_DTYPE_F32:
        return haste::launch_sgd<HASTE_DTYPE_F32, WF16>(ts, count, lr, wd, mu, use_mom, do_sr, seed, st);
    default:
        haste::set_error("%s: unsupported gradient dtype code %d", fn, (int)g_dtype);
        return HASTE_ERR_UNSUPPORTED;
    }
}
}  // namespace

extern "C" int haste_sgd_sr_step(uint16_t* w, const void* g, int32_t g_dtype, float* m, int64_t n,
                                 float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                                 uint64_t seed, uint64_t offset0, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sgd_sr_step: n must be >= 0 (got %lld)", (long long)n);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(w != nullptr && g != nullptr, "haste_sgd_sr_step: null pointer");
    HASTE_CHECK_ARG(!use_mom || m != nullptr, "haste_sgd_sr_step: momentum buffer is NULL");
    const haste::SgdTensor t{w, g, m, n, offset0};
    return sgd_dispatch(&t, 1, g_dtype, lr, wd, mu, use_mom, do_sr, seed,
                        static_cast<hipStream_t>(stream), "haste_sgd_sr_step");
}

extern "C" int haste_sgd_sr_step_f16(uint16_t* w, const void* g, int32_t g_dtype, float* m,
                                     int64_t n, float lr, float wd, float mu, int32_t use_mom,
                                     int32_t do_sr, uint64_t seed, uint64_t offset0, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sgd_sr_step_f16: n must be >= 0 (got %lld)", (long long)n);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(w != nullptr && g != nullptr, "haste_sgd_sr_step_f16: null pointer");
    HASTE_CHECK_ARG(!use_mom || m != nullptr, "haste_sgd_sr_step_f16: momentum buffer is NULL");
    const haste::SgdTensor t{w, g, m, n, offset0};
    return sgd_dispatch<true>(&t, 1, g_dtype, lr, wd, mu, use_mom, do_sr, seed,
                              static_cast<hipStream_t>(stream), "haste_sgd_sr_step_f16");
}

extern "C" int haste_sgd_sr_step_multi(const haste_sgd_tensor* tensors, int32_t count,
                                       int32_t g_dtype, float lr, float wd, float mu,
                                       int32_t use_mom, int32_t do_sr, uint64_t seed,
                                       void* stream) {
    HASTE_CHECK_ARG(count >= 0, "haste_sgd_sr_step_multi: count must be >= 0 (got %d)",
                    (int)count);
    if (count == 0) return HASTE_OK;
    HASTE_CHECK_ARG(tensors != nullptr, "haste_sgd_sr_step_multi: null tensor list");
    haste::SgdTensor ts[64];
    for (int base = 0; base < count; base += 64) {
        const int c = std::min<int>(64, count - base);
        for (int k = 0; k < c; ++k) {
            const haste_sgd_tensor& t = tensors[base + k];
            HASTE_CHECK_ARG(t.n >= 0, "haste_sgd_sr_step_multi: tensor %d: n must be >= 0",
                            base + k);
            HASTE_CHECK_ARG(t.n == 0 || (t.w != nullptr && t.g != nullptr),
                            "haste_sgd_sr_step_multi: tensor %d: null pointer", base + k);
            HASTE_CHECK_ARG(t.n == 0 || !use_mom || t.m != nullptr,
                            "haste_sgd_sr_step_multi: tensor %d: momentum buffer is NULL",
                            base + k);
            ts[k] = haste::SgdTensor{t.w, t.g, t.m, t.n, t.offset0};
        }
        int rc = sgd_dispatch(ts, c, g_dtype, lr, wd, mu, use_mom, do_sr, seed,
                              static_cast<hipStream_t>(stream), "haste_sgd_sr_step_multi");
        if (rc != HASTE_OK) return rc;
    }
    return HASTE_OK;
}
