// Shared device/host helpers for the HASTE FFI HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

#include "../../include/haste_ffi.h"

namespace haste {

// The last-level cache (MALL, Infinity Cache) of an MI355X: 256 MB.
constexpr int64_t kMallBytes = 256ll << 20;

// ---------------------------------------------------------------- errors ----
// Thread-local last error, returned by haste_last_error().
void set_error(const char* fmt, ...);
void clear_error();

#define HASTE_CHECK_ARG(cond, ...)                 \
    do {                                           \
        if (!(cond)) {                             \
            ::haste::set_error(__VA_ARGS__);       \
            return HASTE_ERR_INVALID_ARG;          \
        }                                          \
    } while (0)

#define HASTE_CHECK_LAUNCH(what)                                                  \
    do {                                                                          \
        hipError_t e_ = hipGetLastError();                                        \
        if (e_ != hipSuccess) {                                                   \
            ::haste::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
            return HASTE_ERR_HIP;                                                 \
        }                                                                         \
    } while (0)

#define HASTE_HIP_TRY(expr, what)                                                 \
    do {                                                                          \
        hipError_t e_ = (expr);                                                   \
        if (e_ != hipSuccess) {                                                   \
            ::haste::set_error("%s: %s", what, hipGetErrorString(e_));            \
            return HASTE_ERR_HIP;                                                 \
        }                                                                         \
    } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// --------------------------------------------------------------- vectors ----
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16-bit element type tags.
struct BF16 {
    static constexpr int code = HASTE_DTYPE_BF16;
};
struct F16 {
    static constexpr int code = HASTE_DTYPE_F16;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}

template <typename T>
__device__ __forceinline__ float bits_to_f32(uint32_t h);
template <>
__device__ __forceinline__ float bits_to_f32<BF16>(uint32_t h) { return bf16_bits_to_f32(h); }
template <>
__device__ __forceinline__ float bits_to_f32<F16>(uint32_t h) { return f16_bits_to_f32(h); }

// fp32 -> bf16 round-to-nearest-even (quiet NaN keeps the sign).
// (NaN -> quiet NaN; a select, not a branch, so a loop over elements stays
// straight-line code)
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t qnan = ((u >> 16) | 0x40u) & 0xFFFFu;
    const uint32_t v = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    return (u & 0x7FFFFFFFu) > 0x7F800000u ? qnan : v;
}

// fp32 -> fp16 round-to-nearest-even of the fp32 value f itself: the empty asm
// keeps the compiler from folding the conversion into the operation that made
// f (an fma followed by it would become v_fma_mixlo_f16, which rounds the exact
// result to fp16 once instead of rounding it to fp32 first).
__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
    asm volatile("" : "+v"(f));
    _Float16 h = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Two floats -> two packed 16-bit values (low half = a), round to nearest even
// by the hardware conversion (v_cvt_pk_bf16_f32 / v_cvt_f16_f32); NaN stays NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ uint32_t pack2_rne(float a, float b);

template <typename T>
__device__ __forceinline__ uint32_t f32_to_bits(float f);
template <>
__device__ __forceinline__ uint32_t f32_to_bits<BF16>(float f) { return f32_to_bf16_rne(f); }
template <>
__device__ __forceinline__ uint32_t f32_to_bits<F16>(float f) { return f32_to_f16_rne(f); }
template <>
__device__ __forceinline__ uint32_t pack2_rne<BF16>(float a, float b) {
    return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)a, (__bf16)b});
}
template <>
__device__ __forceinline__ uint32_t pack2_rne<F16>(float a, float b) {
    return __builtin_bit_cast(uint32_t, f16x2_t{(_Float16)a, (_Float16)b});
}

// ---------------------------------------------------------------- MFMA ------
// D(16x16 f32) += A(16x32) * B(32x16); lane L supplies A row L%16 and B column
// L%16, eight K-elements each (the same K positions for A and B), and holds
// D rows 4*(L/16)+0..3 of column L%16.
template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<BF16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<F16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// -------------------------------------------------------------- Philox ------
// Philox4x32-10 (Salmon et al., SC'11) with the round function of Triton's
// philox_impl; returns word 0 for counter (c0, c1, c2, 0) and key (k0, k1).
// tl.randint(seed, off) == philox_w0(off_lo, off_hi, 0, seed_lo, seed_hi).
__device__ __forceinline__ uint32_t philox_w0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t k0,
                                              uint32_t k1) {
    uint32_t c3 = 0u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        // three-input XOR in one instruction (truth table 0x96 = odd parity)
        uint32_t n0 = __builtin_amdgcn_bitop3_b32((uint32_t)(p1 >> 32), c1, k0, 0x96);
        uint32_t n2 = __builtin_amdgcn_bitop3_b32((uint32_t)(p0 >> 32), c3, k1, 0x96);
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

// The same for offsets below 2^32 (counter words 1..3 zero): with the zeros
// folded the first round needs one vector multiply and the second round's
// other product is wave-uniform.
__device__ __forceinline__ uint32_t philox_w0_32(uint32_t c0, uint32_t k0, uint32_t k1) {
    return philox_w0(c0, 0u, 0u, k0, k1);
}

// Stochastic rounding fp32 -> bf16 bits (random low 16 bits added to the fp32
// pattern, upper half kept); NaN -> quiet NaN.
__device__ __forceinline__ uint32_t sr_bf16(float x, uint32_t r) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t qnan = ((u >> 16) | 0x40u) & 0xFFFFu;
    const uint32_t v = (u + (r & 0xFFFFu)) >> 16;
    return (u & 0x7FFFFFFFu) > 0x7F800000u ? qnan : v;
}

// One element of the fused SGD step (shared_ffi/sr_triton.py:109-168) under the
// FMA contract g' = fma(wd, w, g); m' = fma(mu, m, g'); w' = fma(-lr, m' or g', w),
// then SR with the random word r (only its low 16 bits are used) or RNE.
// Returns the new bf16 bits; *m is updated when use_mom.
__device__ __forceinline__ uint32_t sgd_one_r(float w, float g, float* m, bool use_mom, float lr,
                                              float wd, float mu, bool do_sr, uint32_t r) {
    g = __builtin_fmaf(wd, w, g);
    float upd = g;
    if (use_mom) {
        float mv = __builtin_fmaf(mu, *m, g);
        *m = mv;
        upd = mv;
    }
    float nw = __builtin_fmaf(-lr, upd, w);
    return do_sr ? sr_bf16(nw, r) : f32_to_bf16_rne(nw);
}

// The same with r = tl.randint(seed, off).
__device__ __forceinline__ uint32_t sgd_one(float w, float g, float* m, bool use_mom, float lr,
                                            float wd, float mu, bool do_sr, uint64_t off,
                                            uint32_t k0, uint32_t k1) {
    const uint32_t r = do_sr ? philox_w0((uint32_t)off, (uint32_t)(off >> 32), 0u, k0, k1) : 0u;
    return sgd_one_r(w, g, m, use_mom, lr, wd, mu, do_sr, r);
}

// ------------------------------------------------------- buffer access ------
// Raw buffer resources (stride 0): the hardware range-checks every access
// against num_records, returning 0 for loads and dropping stores that fall
// outside.  Kernels use this instead of branches around memory operations, so
// every path issues the same number of vector-memory instructions and the
// compiler can wait for exactly the loads it needs (a branch around a store
// makes it wait for all outstanding stores instead).  An offset of kOOB is
// outside every resource built here (num_records is kept below 2^31).  An
// access that crosses num_records is out of range as a whole.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;
constexpr int64_t kMaxRsrcBytes = 0x7FFFFF00;
// s_waitcnt operand (gfx9 encoding) that waits for every vector-memory op and
// for nothing else: vmcnt 0, expcnt 7 and lgkmcnt 15 (no wait)
constexpr int kWaitVmcnt0 = (7 << 4) | (15 << 8);
// s_waitcnt operand that waits until at most n LDS/scalar-memory ops are
// outstanding (n <= 15) and for nothing else (vmcnt 63, expcnt 7)
__host__ __device__ constexpr int wait_lgkmcnt(int n) { return 0xF | (7 << 4) | (n << 8) | (3 << 14); }

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
    const int64_t n = bytes < 0 ? 0 : (bytes > kMaxRsrcBytes ? kMaxRsrcBytes : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n,
                                             0x00020000);
}
// The same for a size the caller knows to lie in [0, kMaxRsrcBytes] (no clamp).
__device__ __forceinline__ rsrc_t make_rsrc_u32(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ u32x2 buf_load8(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ void buf_store16(u32x4 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}
__device__ __forceinline__ void buf_store8(u32x2 v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}
__device__ __forceinline__ void buf_store4(uint32_t v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}
__device__ __forceinline__ void buf_store2(uint16_t v, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 0);
}

// Rows of a [rows, ld] 16-bit matrix with any ld start on 2-byte boundaries;
// 16-byte loads of 8 elements need no more alignment than that on gfx950
// (unaligned buffer access).  The 8-element piece that straddles the end of
// the matrix's last row is the one exception: it would cross the end of the
// tensor, so it is loaded sh elements early (ending at the row's end) and moved
// back into place with shift_down16.  Elements sh .. 7 of v go to positions
// 0 .. 7 - sh; the top sh positions are unspecified.  sh in [0, 7], per lane.
__device__ __forceinline__ u32x4 shift_down16(u32x4 v, int sh) {
    const int ws = sh >> 1;
    const uint32_t w0 = ws == 0 ? v[0] : ws == 1 ? v[1] : ws == 2 ? v[2] : v[3];
    const uint32_t w1 = ws == 0 ? v[1] : ws == 1 ? v[2] : v[3];
    const uint32_t w2 = ws == 0 ? v[2] : v[3];
    const uint32_t w3 = v[3];
    const uint32_t bs = (uint32_t)(sh & 1) * 2;  // bytes
    return u32x4{__builtin_amdgcn_alignbyte(w1, w0, bs), __builtin_amdgcn_alignbyte(w2, w1, bs),
                 __builtin_amdgcn_alignbyte(w3, w2, bs), __builtin_amdgcn_alignbyte(0u, w3, bs)};
}

// Bytes mb .. mb+15 of the 32 bytes a || b (mb even, per lane, in [0, 14]): an
// 8-element piece that starts mb bytes into the aligned chunk a.
__device__ __forceinline__ u32x4 shift_pair16(u32x4 a, u32x4 b, uint32_t mb) {
    const uint32_t ws = mb >> 2;
    const uint32_t x0 = ws == 0 ? a[0] : ws == 1 ? a[1] : ws == 2 ? a[2] : a[3];
    const uint32_t x1 = ws == 0 ? a[1] : ws == 1 ? a[2] : ws == 2 ? a[3] : b[0];
    const uint32_t x2 = ws == 0 ? a[2] : ws == 1 ? a[3] : ws == 2 ? b[0] : b[1];
    const uint32_t x3 = ws == 0 ? a[3] : ws == 1 ? b[0] : ws == 2 ? b[1] : b[2];
    const uint32_t x4 = ws == 0 ? b[0] : ws == 1 ? b[1] : ws == 2 ? b[2] : b[3];
    const uint32_t bs = mb & 3u;
    return u32x4{__builtin_amdgcn_alignbyte(x1, x0, bs), __builtin_amdgcn_alignbyte(x2, x1, bs),
                 __builtin_amdgcn_alignbyte(x3, x2, bs), __builtin_amdgcn_alignbyte(x4, x3, bs)};
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4 of
// the 8-byte rows addressed by lanes 4k + i/4 (k = 0..3) as its element k.
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
__device__ __forceinline__ u32x2 lds_read_tr16(const char* p) {
    typedef fp16x4_t __attribute__((address_space(3))) * lds_p;
    const fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (lds_p)(__attribute__((address_space(3))) char*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// Workgroup-id remap so that consecutive logical ids land on the same XCD
// (the hardware dispatches workgroup i to XCD i % 8), the ids split as evenly
// as the count allows (XCD x holds nlogical / 8 ids, one more when x <
// nlogical % 8).  Returns -1 for the padding ids of a grid rounded up to a
// multiple of 8.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nlogical) {
    const int64_t lo = nlogical / 8, rem = nlogical % 8;
    const int64_t x = bid % 8, k = bid / 8;
    return k < lo + (x < rem ? 1 : 0) ? x * lo + min(x, rem) + k : -1;
}

}  // namespace haste
