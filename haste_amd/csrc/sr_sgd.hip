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

__device__ __forceinline__ uint32_t sgd_one(float w, float g, float* m, bool use_mom, float lr,
                                            float wd, float mu, bool do_sr, uint64_t off,
                                            uint32_t k0, uint32_t k1) {
    g = __builtin_fmaf(wd, w, g);
    float upd = g;
    if (use_mom) {
        float mv = __builtin_fmaf(mu, *m, g);
        *m = mv;
        upd = mv;
    }
    float nw = __builtin_fmaf(-lr, upd, w);
    if (do_sr) return sr_bf16(nw, philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1));
    return f32_to_bf16_rne(nw);
}

// Vector path: requires 16-byte aligned w, g (and m) and n_vec = n / 8 items.
template <int GD, bool USE_MOM, bool DO_SR>
__global__ __launch_bounds__(256) void sgd_sr_vec_kernel(uint16_t* __restrict__ w,
                                                         const void* __restrict__ g,
                                                         float* __restrict__ m, int64_t n_vec,
                                                         float lr, float wd, float mu,
                                                         uint64_t seed, uint64_t offset0) {
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < n_vec; v += stride) {
        const int64_t i = v * kVec;
        u32x4 wv = *reinterpret_cast<const u32x4*>(w + i);
        float gf[kVec];
        load_grad8<GD>(g, i, gf);
        float mv[kVec];
        if constexpr (USE_MOM) {
            float4 a = reinterpret_cast<const float4*>(m + i)[0];
            float4 b = reinterpret_cast<const float4*>(m + i)[1];
            mv[0] = a.x; mv[1] = a.y; mv[2] = a.z; mv[3] = a.w;
            mv[4] = b.x; mv[5] = b.y; mv[6] = b.z; mv[7] = b.w;
        }
        uint32_t outb[kVec];
#pragma unroll
        for (int e = 0; e < kVec; ++e) {
            uint32_t wb = (e & 1) ? (wv[e >> 1] >> 16) : (wv[e >> 1] & 0xFFFFu);
            outb[e] = sgd_one(bf16_bits_to_f32(wb), gf[e], &mv[e], USE_MOM, lr, wd, mu, DO_SR,
                              offset0 + (uint64_t)(i + e), k0, k1);
        }
        u32x4 ov;
#pragma unroll
        for (int q = 0; q < 4; ++q) ov[q] = outb[2 * q] | (outb[2 * q + 1] << 16);
        *reinterpret_cast<u32x4*>(w + i) = ov;
        if constexpr (USE_MOM) {
            reinterpret_cast<float4*>(m + i)[0] = make_float4(mv[0], mv[1], mv[2], mv[3]);
            reinterpret_cast<float4*>(m + i)[1] = make_float4(mv[4], mv[5], mv[6], mv[7]);
        }
    }
}

// Scalar path for the tail (or unaligned tensors): elements [i0, n).
template <int GD>
__global__ __launch_bounds__(256) void sgd_sr_scalar_kernel(uint16_t* __restrict__ w,
                                                            const void* __restrict__ g,
                                                            float* __restrict__ m, int64_t i0,
                                                            int64_t n, float lr, float wd,
                                                            float mu, int use_mom, int do_sr,
                                                            uint64_t seed, uint64_t offset0) {
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = i0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float dummy = 0.f;
        float* mp = use_mom ? (m + i) : &dummy;
        w[i] = (uint16_t)sgd_one(bf16_bits_to_f32(w[i]), load_grad1<GD>(g, i), mp, use_mom != 0,
                                 lr, wd, mu, do_sr != 0, offset0 + (uint64_t)i, k0, k1);
    }
}

template <int GD>
int launch_sgd(uint16_t* w, const void* g, float* m, int64_t n, float lr, float wd, float mu,
               int use_mom, int do_sr, uint64_t seed, uint64_t offset0, hipStream_t st) {
    const bool vec_ok = aligned16(w) && aligned16(g) && (!use_mom || aligned16(m));
    int64_t n_vec = vec_ok ? n / kVec : 0;
    if (n_vec > 0) {
        const int64_t blocks = std::min<int64_t>(ceil_div(n_vec, 256), 1 << 20);
#define HASTE_SGD_LAUNCH(UM, SR)                                                               \
    sgd_sr_vec_kernel<GD, UM, SR><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(              \
        w, g, m, n_vec, lr, wd, mu, seed, offset0)
        if (use_mom && do_sr) HASTE_SGD_LAUNCH(true, true);
        else if (use_mom) HASTE_SGD_LAUNCH(true, false);
        else if (do_sr) HASTE_SGD_LAUNCH(false, true);
        else HASTE_SGD_LAUNCH(false, false);
#undef HASTE_SGD_LAUNCH
        HASTE_CHECK_LAUNCH("haste_sgd_sr_step");
    }
    const int64_t i0 = n_vec * kVec;
    if (i0 < n) {
        const int64_t blocks = std::min<int64_t>(ceil_div(n - i0, 256), 1 << 20);
        sgd_sr_scalar_kernel<GD><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            w, g, m, i0, n, lr, wd, mu, use_mom, do_sr, seed, offset0);
        HASTE_CHECK_LAUNCH("haste_sgd_sr_step");
    }
    return HASTE_OK;
}

__global__ __launch_bounds__(256) void sr_round_vec_kernel(const float* __restrict__ x,
                                                           uint16_t* __restrict__ out,
                                                           int64_t n_vec, uint32_t k0,
                                                           uint32_t k1, uint64_t offset0) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < n_vec; v += stride) {
        const int64_t i = v * kVec;
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
    }
}

__global__ __launch_bounds__(256) void sr_round_scalar_kernel(const float* __restrict__ x,
                                                              uint16_t* __restrict__ out,
                                                              int64_t i0, int64_t n, uint32_t k0,
                                                              uint32_t k1, uint64_t offset0) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = i0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t off = offset0 + (uint64_t)i;
        out[i] = (uint16_t)sr_bf16(x[i], philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1));
    }
}

}  // namespace

int sr_round_bf16(const float* x, uint16_t* out, int64_t n, uint64_t seed, uint64_t offset0,
                  hipStream_t st) {
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    const bool vec_ok = aligned16(x) && aligned16(out);
    int64_t n_vec = vec_ok ? n / kVec : 0;
    if (n_vec > 0) {
        const int64_t blocks = std::min<int64_t>(ceil_div(n_vec, 256), 1 << 20);
        sr_round_vec_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, out, n_vec, k0, k1,
                                                                        offset0);
        HASTE_CHECK_LAUNCH("haste_sr_round_bf16");
    }
    const int64_t i0 = n_vec * kVec;
    if (i0 < n) {
        const int64_t blocks = std::min<int64_t>(ceil_div(n - i0, 256), 1 << 20);
        sr_round_scalar_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, out, i0, n, k0,
                                                                           k1, offset0);
        HASTE_CHECK_LAUNCH("haste_sr_round_bf16");
    }
    return HASTE_OK;
}

}  // namespace haste

extern "C" int haste_sr_round_bf16(const float* x, uint16_t* out, int64_t n, uint64_t seed,
                                   uint64_t offset0, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sr_round_bf16: n must be >= 0 (got %lld)", (long long)n);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(x != nullptr && out != nullptr, "haste_sr_round_bf16: null pointer");
    return haste::sr_round_bf16(x, out, n, seed, offset0, static_cast<hipStream_t>(stream));
}

extern "C" int haste_sgd_sr_step(uint16_t* w, const void* g, int32_t g_dtype, float* m, int64_t n,
                                 float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                                 uint64_t seed, uint64_t offset0, void* stream) {
    HASTE_CHECK_ARG(n >= 0, "haste_sgd_sr_step: n must be >= 0 (got %lld)", (long long)n);
    if (n == 0) return HASTE_OK;
    HASTE_CHECK_ARG(w != nullptr && g != nullptr, "haste_sgd_sr_step: null pointer");
    HASTE_CHECK_ARG(!use_mom || m != nullptr, "haste_sgd_sr_step: momentum buffer is NULL");
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (g_dtype) {
    case HASTE_DTYPE_BF16:
        return haste::launch_sgd<HASTE_DTYPE_BF16>(w, g, m, n, lr, wd, mu, use_mom, do_sr, seed,
                                                   offset0, st);
    case HASTE_DTYPE_F16:
        return haste::launch_sgd<HASTE_DTYPE_F16>(w, g, m, n, lr, wd, mu, use_mom, do_sr, seed,
                                                  offset0, st);
    case HASTE_DTYPE_F32:
        return haste::launch_sgd<HASTE_DTYPE_F32>(w, g, m, n, lr, wd, mu, use_mom, do_sr, seed,
                                                  offset0, st);
    default:
        haste::set_error("haste_sgd_sr_step: unsupported gradient dtype code %d", (int)g_dtype);
        return HASTE_ERR_UNSUPPORTED;
    }
}
