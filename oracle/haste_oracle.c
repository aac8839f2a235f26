/*
 * haste_oracle.c -- CPU restatement of the integer/bit-level parts of HASTE's
 * FFI hot path.  TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (haste_amd/) never links it.
 *
 * What it restates (reference paths relative to the xmc-aalto/haste tree):
 *   - Philox4x32-10 exactly as Triton's tl.randint(seed, offset) evaluates it
 *     (Triton 3.x triton/language/random.py philox_impl/randint4x; called from
 *     shared_ffi/sr_triton.py:11).  Pinned by Random123 KATs and by tl.randint
 *     vectors produced with the installed Triton 3.6.0 interpreter
 *     (tests/golden/randint_vectors.json).
 *   - stochastic_rounding_to_bf16, shared_ffi/sr_triton.py:9-16.
 *   - _seeded_stochastic_rounding / stochastic_rounding, sr_triton.py:27-59.
 *   - _sgd_m_wd_sr / sgd_update, sr_triton.py:109-213, with the FMA contract
 *     g' = fma(wd, w, g); m' = fma(mu, m, g'); w' = fma(-lr, m' or g', w)
 *     (Triton compiles with fp fusion on, so these products are contracted).
 *   - GroupFixedFanIn.rewire, shared_ffi/rewire.py:143-239, with the random
 *     draws replaced by documented Philox streams (torch.randint/uniform_ device
 *     streams cannot be reproduced) and topk ties broken by (score, slot).
 *
 * Parity status of each function is stated in the function's comment.
 * Built with -ffp-contract=off: every fused multiply-add here is an explicit
 * fmaf(), nothing else is contracted.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u

/* Philox4x32 with R rounds (Salmon et al., SC'11, "Parallel random numbers:
 * as easy as 1, 2, 3"; round function as in Triton's philox_impl).
 * Pinned: Random123 known-answer vectors + tl.randint vectors. */
void ho_philox4x32(const uint32_t ctr[4], const uint32_t key[2], int rounds, uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < rounds; ++r) {
        uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
        uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += PHILOX_W0;
        k1 += PHILOX_W1;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* tl.randint(seed, offset): word 0 of Philox4x32-10 with key = (seed lo, seed hi)
 * and counter = (offset lo, offset hi, 0, 0).  Pinned as above. */
uint32_t ho_randint(uint64_t seed, uint64_t offset) {
    uint32_t ctr[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), 0u, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    ho_philox4x32(ctr, key, 10, out);
    return out[0];
}

void ho_randint_array(uint64_t seed, uint64_t offset0, int64_t n, uint32_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = ho_randint(seed, offset0 + (uint64_t)i);
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float ho_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }
float ho_f16_to_f32(uint16_t h);

/* fp32 -> bf16 round-to-nearest-even; NaN -> quiet NaN with the input sign. */
uint16_t ho_f32_to_bf16_rne(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

/* stochastic_rounding_to_bf16 (sr_triton.py:9-16): add the low 16 random bits to
 * the fp32 bit pattern (32-bit wrap-around add) and keep the upper half.
 * NaN inputs give a quiet NaN (the bit trick would otherwise make the payload
 * depend on the random bits; the reference's NaN result is not pinned).
 * Pinned: closed form checks (exact values unchanged, round-up probability,
 * brute-force interval check) in tests/test_oracle_sr.py. */
uint16_t ho_sr_bf16(float x, uint32_t r) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u = u + (r & 0xFFFFu);
    return (uint16_t)(u >> 16);
}

/* stochastic_rounding(x, output, seed) (sr_triton.py:51-59): element i uses
 * offset offset0 + i under `seed`. */
void ho_sr_round_bf16(const float* x, uint16_t* out, int64_t n, uint64_t seed, uint64_t offset0) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = ho_sr_bf16(x[i], ho_randint(seed, offset0 + (uint64_t)i));
}

/* IEEE binary16 -> fp32 (exact). */
float ho_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(s);
        float v = ldexpf((float)m, -24);
        return s ? -v : v;
    }
    if (e == 31) return u2f(s | 0x7F800000u | (m << 13));
    return u2f(s | ((e + 112u) << 23) | (m << 13));
}

/* fp32 -> IEEE binary16, round to nearest even (overflow to infinity, NaN to a
 * quiet NaN with the sign kept).  Pinned against numpy's float16 conversion. */
uint16_t ho_f32_to_f16_rne(float f) {
    uint32_t u = f2u(f);
    uint32_t s = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(s | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x47800000u) {  /* >= 65536: infinity, or the largest values round up to it */
        return (uint16_t)(s | 0x7C00u);
    }
    if (a < 0x38800000u) {  /* below 2^-14: a subnormal (or zero) result */
        /* value = a_float; result = round(value / 2^-24) as an integer mantissa */
        float v = u2f(a);
        double q = ldexp((double)v, 24);  /* exact: v has 24 significant bits */
        double r = nearbyint(q);          /* round to nearest even (default mode) */
        return (uint16_t)(s | (uint32_t)r);
    }
    /* normal range: keep 10 mantissa bits, round the dropped 13 to nearest even */
    uint32_t e = (a >> 23) - 112u;
    uint32_t m = a & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rest = m & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;  /* may carry into e */
    return (uint16_t)(s | h);
}

enum { HO_BF16 = 0, HO_F16 = 1, HO_F32 = 2 };

static inline float load_any(const void* p, int dtype, int64_t i) {
    switch (dtype) {
    case HO_BF16: return ho_bf16_to_f32(((const uint16_t*)p)[i]);
    case HO_F16: return ho_f16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
    }
}

/* Fused SGD step (_sgd_m_wd_sr, sr_triton.py:109-168) on bf16 weights, in place.
 *   g  = float(grad[i]);  w = float(W[i])
 *   g' = fma(wd, w, g)
 *   use_mom: m' = fma(mu, m[i], g'); m[i] = m'; w' = fma(-lr, m', w)
 *   else:    w' = fma(-lr, g', w)
 *   W[i] = do_sr ? SR(w', randint(seed, offset0 + i)) : RNE(w')
 * lr, wd, mu are fp32 (Triton passes Python floats as fp32 scalars).
 * Pinned: exact-rational brute force of the FMA chain on small arrays,
 * closed-form special cases (lr = 0, wd = 0), tests/test_oracle_sgd.py. */
void ho_sgd_sr_step(uint16_t* w, const void* g, int g_dtype, float* m, int64_t n,
                    float lr, float wd, float mu, int use_mom, int do_sr,
                    uint64_t seed, uint64_t offset0) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float wf = ho_bf16_to_f32(w[i]);
        float gf = load_any(g, g_dtype, i);
        gf = fmaf(wd, wf, gf);
        float upd = gf;
        if (use_mom) {
            float mv = fmaf(mu, m[i], gf);
            m[i] = mv;
            upd = mv;
        }
        float nw = fmaf(-lr, upd, wf);
        w[i] = do_sr ? ho_sr_bf16(nw, ho_randint(seed, offset0 + (uint64_t)i))
                     : ho_f32_to_bf16_rne(nw);
    }
}

/* The same step on fp16 weights (an fp16 w_ptr in _sgd_m_wd_sr): w is read as
 * fp16, the update rounded to bf16 as above (SR or RNE), and the bf16 value
 * stored as fp16 (round to nearest even, the store's conversion). */
void ho_sgd_sr_step_f16w(uint16_t* w, const void* g, int g_dtype, float* m, int64_t n,
                         float lr, float wd, float mu, int use_mom, int do_sr,
                         uint64_t seed, uint64_t offset0) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float wf = ho_f16_to_f32(w[i]);
        float gf = load_any(g, g_dtype, i);
        gf = fmaf(wd, wf, gf);
        float upd = gf;
        if (use_mom) {
            float mv = fmaf(mu, m[i], gf);
            m[i] = mv;
            upd = mv;
        }
        float nw = fmaf(-lr, upd, wf);
        uint16_t b = do_sr ? ho_sr_bf16(nw, ho_randint(seed, offset0 + (uint64_t)i))
                           : ho_f32_to_bf16_rne(nw);
        w[i] = ho_f32_to_f16_rne(ho_bf16_to_f32(b));
    }
}

/* ---- fp16 and fp8 outputs (sr_triton.py:18-25,43-46,146,167-168) ----
 * The reference's stochastic_rounding writes float8_e4m3fn outputs through
 * stochastic_rounding_to_fp8 (20 random bits, the fp32 pattern cut to 12 bits,
 * then converted), and every other output dtype through the bf16 rounding
 * followed by the store's conversion to the output dtype; _sgd_m_wd_sr stores
 * its bf16 result into fp16 / fp8 weights the same way.  The conversions:
 *   fp16: round to nearest even (ho_f32_to_f16_rne);
 *   fp8:  round to nearest even, saturating: finite values beyond the largest
 *         finite one and infinities become the largest finite value with the
 *         input's sign (Triton's conversion for float8 stores on NVIDIA GPUs is
 *         cvt.rn.satfinite); NaN becomes sign | 0x7F.
 * Pinned: every fp8 code decodes as torch's float8 types do; in-range
 * encodings equal torch's conversions (which round to nearest even); the
 * saturation and the 20-bit rounding by closed forms (exact unbiasedness over
 * all 2^20 random words) in tests/test_oracle_fp8.py.  The NaN and overflow
 * results of the reference are not pinned (Triton is not runnable here). */
enum { HO_F8E4M3 = 3, HO_F8E5M2 = 4 };

static int f8_mant(int fmt) { return fmt == HO_F8E4M3 ? 3 : 2; }
static int f8_bias(int fmt) { return fmt == HO_F8E4M3 ? 7 : 15; }
static uint32_t f8_maxcode(int fmt) { return fmt == HO_F8E4M3 ? 0x7Eu : 0x7Bu; }

/* OCP E4M3 ("fn": bias 7, no infinities, S.1111.111 NaN) or E5M2 (bias 15,
 * IEEE infinities and NaNs) -> fp32, exact. */
float ho_f8_to_f32(uint8_t c, int fmt) {
    const int M = f8_mant(fmt), bias = f8_bias(fmt);
    const uint32_t s = (uint32_t)(c & 0x80u) << 24;
    const uint32_t e = (c & 0x7Fu) >> M, m = c & ((1u << M) - 1u);
    if (fmt == HO_F8E4M3 && (c & 0x7Fu) == 0x7Fu) return u2f(s | 0x7FC00000u);
    if (fmt == HO_F8E5M2 && e == 31u) return u2f(s | 0x7F800000u | (m ? 0x400000u : 0u));
    float v = e == 0 ? ldexpf((float)m, 1 - bias - M) : ldexpf((float)((1u << M) | m), (int)e - bias - M);
    return s ? -v : v;
}

uint8_t ho_f32_to_f8(float f, int fmt) {
    const int M = f8_mant(fmt), bias = f8_bias(fmt), emin = 1 - bias;
    const uint32_t maxcode = f8_maxcode(fmt);
    const uint32_t u = f2u(f), s = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint8_t)(s | 0x7Fu);
    if (a == 0x7F800000u) return (uint8_t)(s | maxcode);
    if (a < (uint32_t)(emin + 127) << 23) {
        /* below the smallest normal: an integer count of the smallest subnormal,
         * rounded to nearest even (2^M is the smallest normal's code) */
        const float q = rintf(ldexpf(u2f(a), M - emin));
        return (uint8_t)(s | (uint32_t)q);
    }
    const int rb = 23 - M;
    uint32_t code = ((a + ((1u << (rb - 1)) - 1u) + ((a >> rb) & 1u)) >> rb) -
                    ((uint32_t)(127 - bias) << M);
    if (code > maxcode) code = maxcode;
    return (uint8_t)(s | code);
}

/* stochastic_rounding_to_fp8 (sr_triton.py:18-25): add the low 20 random bits
 * to the fp32 pattern (32-bit wrap), clear the low 20 bits, convert.  NaN
 * inputs give NaN (not pinned, as for bf16). */
uint8_t ho_sr_e4m3(float x, uint32_t r) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint8_t)(((u >> 24) & 0x80u) | 0x7Fu);
    u = (u + (r & 0xFFFFFu)) & 0xFFF00000u;
    return ho_f32_to_f8(u2f(u), HO_F8E4M3);
}

/* stochastic_rounding(x, output, seed) for an output of dtype out_dtype
 * (HO_BF16, HO_F16, HO_F8E4M3, HO_F8E5M2): 2-byte or 1-byte codes. */
void ho_sr_round(const float* x, void* out, int out_dtype, int64_t n, uint64_t seed,
                 uint64_t offset0) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t r = ho_randint(seed, offset0 + (uint64_t)i);
        if (out_dtype == HO_F8E4M3) {
            ((uint8_t*)out)[i] = ho_sr_e4m3(x[i], r);
            continue;
        }
        const uint16_t b = ho_sr_bf16(x[i], r);
        if (out_dtype == HO_F8E5M2)
            ((uint8_t*)out)[i] = ho_f32_to_f8(ho_bf16_to_f32(b), HO_F8E5M2);
        else if (out_dtype == HO_F16)
            ((uint16_t*)out)[i] = ho_f32_to_f16_rne(ho_bf16_to_f32(b));
        else
            ((uint16_t*)out)[i] = b;
    }
}

/* _sgd_m_wd_sr on fp8 weights (w_fmt HO_F8E4M3 / HO_F8E5M2): loaded exactly,
 * updated as ho_sgd_sr_step, the bf16 result stored as fp8. */
void ho_sgd_sr_step_f8w(uint8_t* w, int w_fmt, const void* g, int g_dtype, float* m, int64_t n,
                        float lr, float wd, float mu, int use_mom, int do_sr, uint64_t seed,
                        uint64_t offset0) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float wf = ho_f8_to_f32(w[i], w_fmt);
        float gf = load_any(g, g_dtype, i);
        gf = fmaf(wd, wf, gf);
        float upd = gf;
        if (use_mom) {
            float mv = fmaf(mu, m[i], gf);
            m[i] = mv;
            upd = mv;
        }
        float nw = fmaf(-lr, upd, wf);
        uint16_t b = do_sr ? ho_sr_bf16(nw, ho_randint(seed, offset0 + (uint64_t)i))
                           : ho_f32_to_bf16_rne(nw);
        w[i] = ho_f32_to_f8(ho_bf16_to_f32(b), w_fmt);
    }
}

void ho_f8_to_f32_arr(const uint8_t* c, int fmt, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ho_f8_to_f32(c[i], fmt);
}

void ho_f32_to_f8_arr(const float* x, int fmt, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ho_f32_to_f8(x[i], fmt);
}

/* SR to e4m3 of one value under each of n random words (for closed-form checks). */
void ho_sr_e4m3_words(float x, const uint32_t* r, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ho_sr_e4m3(x, r[i]);
}

void ho_f32_to_f16_rne_arr(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ho_f32_to_f16_rne(x[i]);
}

void ho_f32_to_bf16_rne_arr(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ho_f32_to_bf16_rne(x[i]);
}

int ho_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void ho_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ---------------------------------------------------------------------------
 * Rewire (GroupFixedFanIn.rewire, shared_ffi/rewire.py:143-239).
 *
 * Contract (deterministic; the reference's random draws come from torch
 * generators, so this build fixes its own Philox streams):
 *  1. score[g][j] = (sum over rows l of group g, in ascending l, of fp32 |W[l][j]|)
 *                   / (float)rows_in_group            (rewire.py:169-185)
 *  2. prune mask:  threshold mode: score < thr        (rewire.py:188-189)
 *                  fraction mode:  the k slots with the smallest (score, slot)
 *                  pairs, k = int(F * fraction)      (rewire.py:190-204)
 *  3. regrow index for pruned slot (g, j):
 *       RANDOM (with replacement, as rewire.py:211):
 *         u = philox(key = seed, ctr = (g*F + j, 1, 0, 0)).w0;  d = (u * D) >> 32
 *       UNUSED (never an index already present in the group): slots are visited
 *         in ascending j; attempt t uses ctr = (g*F + j, 1, t, 0); a candidate
 *         is accepted if it is not among the group's current indices (kept
 *         slots plus indices regrown earlier in this call); after
 *         HO_UNUSED_MAX_TRIES failed attempts the last candidate is taken.
 *  4. weights of every row of the group at a pruned slot:
 *       ZERO: 0.   RANDOM: u = philox(key = seed, ctr = (l*F + j, 2, 0, 0)).w0,
 *       v = fma((float)(u >> 8) * 2^-24, 2*bound, -bound), bound = 1/sqrt(F)
 *       (fp32, passed in), stored in W's dtype: RNE to bf16 / fp16, or as is
       for fp32 weights (uniform_ in the weights' dtype, rewire.py:226-237).
 * W: bf16 or fp16 bit patterns, or fp32 values (w_dtype HO_BF16 / HO_F16 / HO_F32).
 * Returns the number of pruned slots.  Scores and mask are optional outputs.
 * Pinned: invariants and brute-force selection in tests/test_oracle_rewire.py.
 * --------------------------------------------------------------------------- */
#define HO_UNUSED_MAX_TRIES 64

enum { HO_PRUNE_THRESHOLD = 0, HO_PRUNE_FRACTION = 1 };
enum { HO_REGROW_RANDOM = 0, HO_REGROW_UNUSED = 1 };
enum { HO_INIT_ZERO = 0, HO_INIT_RANDOM = 1 };

static uint32_t philox_w0(uint64_t seed, uint32_t c0, uint32_t c1, uint32_t c2) {
    uint32_t ctr[4] = {c0, c1, c2, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    ho_philox4x32(ctr, key, 10, out);
    return out[0];
}

/* W of dtype w_dtype (HO_BF16 / HO_F16 bit patterns, or HO_F32 values): element i
 * as fp32 (exact), and stored from fp32 (RNE to the 16-bit formats) -- the
 * reference's rewire works in the weights' own dtype (rewire.py:155,224-237). */
static float w_get(const void* W, int w_dtype, int64_t i) {
    if (w_dtype == HO_F32) return ((const float*)W)[i];
    uint16_t h = ((const uint16_t*)W)[i];
    return w_dtype == HO_F16 ? ho_f16_to_f32(h) : ho_bf16_to_f32(h);
}
static void w_set(void* W, int w_dtype, int64_t i, float v) {
    if (w_dtype == HO_F32)
        ((float*)W)[i] = v;
    else
        ((uint16_t*)W)[i] = w_dtype == HO_F16 ? ho_f32_to_f16_rne(v) : ho_f32_to_bf16_rne(v);
}
/* v rounded to dtype dt (RNE) and back: the value of a tensor product in dt */
static float round_as(float v, int dt) {
    if (dt == HO_BF16) return ho_bf16_to_f32(ho_f32_to_bf16_rne(v));
    if (dt == HO_F16) return ho_f16_to_f32(ho_f32_to_f16_rne(v));
    return v;
}

void ho_rewire_scores(const void* W, int w_dtype, float* scores, int64_t O, int64_t F,
                      int64_t G) {
    int64_t Gc = (O + G - 1) / G;
    for (int64_t g = 0; g < Gc; ++g) {
        int64_t l0 = g * G, l1 = l0 + G < O ? l0 + G : O;
        float cnt = (float)(l1 - l0);
        for (int64_t j = 0; j < F; ++j) {
            float s = 0.0f;
            for (int64_t l = l0; l < l1; ++l) s += fabsf(w_get(W, w_dtype, l * F + j));
            scores[g * F + j] = s / cnt;
        }
    }
}

/* ---------------------------------------------------------------------------
 * The application's variant, GroupFixedFanInReal.rewire
 * (src/group_fanin_real.py:150-286):
 *  value v[l][j] = |W| or, with grad, the saliency |W * grad|
 *          (group_fanin_real.py:199-204): the product in prod_dtype, torch's
 *          promoted dtype of (W, grad) -- for two 16-bit values of one format
 *          the (exact) fp32 product rounded to that format, else the fp32
 *          product; grad is passed as its fp32 values.
 *  score  MEAN: fp32 sum over the group's rows in ascending order / rows
 *         (group_fanin_real.py:206-212,226-228); MAX: max over the rows
 *         (group_fanin_real.py:213-220).
 *  prune  GLOBAL_FRACTION: the k slots of the whole layer with the smallest
 *         (score, g*F + j) pairs (group_fanin_real.py:234-251, topk over all
 *         slots; its tie order is unspecified, fixed here to the lower slot).
 * --------------------------------------------------------------------------- */
enum { HO_PRUNE_GLOBAL_FRACTION = 2 };
enum { HO_SCORE_MEAN = 0, HO_SCORE_MAX = 1 };

void ho_rewire_scores_ex(const void* W, int w_dtype, const float* grad, int prod_dtype,
                         int score_mode, float* scores, int64_t O, int64_t F, int64_t G) {
    int64_t Gc = (O + G - 1) / G;
    for (int64_t g = 0; g < Gc; ++g) {
        int64_t l0 = g * G, l1 = l0 + G < O ? l0 + G : O;
        for (int64_t j = 0; j < F; ++j) {
            float acc = score_mode == HO_SCORE_MAX ? -INFINITY : 0.0f;
            for (int64_t l = l0; l < l1; ++l) {
                float w = w_get(W, w_dtype, l * F + j);
                float v = grad ? fabsf(round_as(w * grad[l * F + j], prod_dtype)) : fabsf(w);
                acc = score_mode == HO_SCORE_MAX ? (v > acc ? v : acc) : acc + v;
            }
            scores[g * F + j] = score_mode == HO_SCORE_MAX ? acc : acc / (float)(l1 - l0);
        }
    }
}

static int cmp_u64(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

static int64_t rewire_apply(void* W, int w_dtype, int32_t* idx, int64_t O, int64_t F,
                            int64_t G, int64_t D, int prune_mode, float thr, int64_t k,
                            int regrow_mode, int init_mode, float bound, uint64_t seed,
                            const float* scores, uint8_t* mask);

int64_t ho_rewire_ex(void* W, int w_dtype, int32_t* idx, const float* grad, int prod_dtype,
                     int score_mode, int64_t O, int64_t F, int64_t G, int64_t D,
                     int prune_mode, float thr, int64_t k, int regrow_mode, int init_mode,
                     float bound, uint64_t seed, float* scores_out, uint8_t* mask_out) {
    int64_t Gc = (O + G - 1) / G, n = Gc * F;
    float* scores = (float*)malloc(sizeof(float) * (size_t)n);
    uint8_t* mask = (uint8_t*)calloc((size_t)n, 1);
    ho_rewire_scores_ex(W, w_dtype, grad, prod_dtype, score_mode, scores, O, F, G);
    if (prune_mode == HO_PRUNE_GLOBAL_FRACTION) {
        /* keys (bits(score) << 32 | slot) order the scores (>= 0) with ties to the lower slot */
        uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)n);
        for (int64_t i = 0; i < n; ++i) {
            uint32_t b;
            memcpy(&b, &scores[i], 4);
            keys[i] = ((uint64_t)b << 32) | (uint64_t)i;
        }
        qsort(keys, (size_t)n, sizeof(uint64_t), cmp_u64);
        for (int64_t r = 0; r < k && r < n; ++r) mask[keys[r] & 0xFFFFFFFFu] = 1;
        free(keys);
    }
    int64_t total = rewire_apply(W, w_dtype, idx, O, F, G, D, prune_mode, thr, k, regrow_mode,
                                 init_mode, bound, seed, scores, mask);
    if (scores_out) memcpy(scores_out, scores, sizeof(float) * (size_t)n);
    if (mask_out) memcpy(mask_out, mask, (size_t)n);
    free(scores);
    free(mask);
    return total;
}

int64_t ho_rewire(void* W, int w_dtype, int32_t* idx, int64_t O, int64_t F, int64_t G,
                  int64_t D, int prune_mode, float thr, int64_t k, int regrow_mode,
                  int init_mode, float bound, uint64_t seed, float* scores_out,
                  uint8_t* mask_out) {
    return ho_rewire_ex(W, w_dtype, idx, NULL, HO_F32, HO_SCORE_MEAN, O, F, G, D, prune_mode,
                        thr, k, regrow_mode, init_mode, bound, seed, scores_out, mask_out);
}

/* prune (threshold / per-group fraction into mask; global fraction: mask given),
 * regrow and re-initialise; returns the number of pruned slots */
static int64_t rewire_apply(void* W, int w_dtype, int32_t* idx, int64_t O, int64_t F,
                            int64_t G, int64_t D, int prune_mode, float thr, int64_t k,
                            int regrow_mode, int init_mode, float bound, uint64_t seed,
                            const float* scores, uint8_t* mask) {
    int64_t Gc = (O + G - 1) / G;
    int64_t total = 0;
    for (int64_t g = 0; g < Gc; ++g) {
        const float* s = scores + g * F;
        uint8_t* mk = mask + g * F;
        if (prune_mode == HO_PRUNE_GLOBAL_FRACTION) {
            /* mask already set */
        } else if (prune_mode == HO_PRUNE_THRESHOLD) {
            for (int64_t j = 0; j < F; ++j) mk[j] = s[j] < thr;
        } else {
            /* rank of slot j = #slots with (score, slot) lexicographically smaller */
            for (int64_t j = 0; j < F; ++j) {
                int64_t rank = 0;
                for (int64_t q = 0; q < F; ++q)
                    if (s[q] < s[j] || (s[q] == s[j] && q < j)) ++rank;
                mk[j] = rank < k;
            }
        }
        int32_t* gi = idx + g * F;
        for (int64_t j = 0; j < F; ++j) {
            if (!mk[j]) continue;
            ++total;
            uint32_t slot = (uint32_t)(g * F + j);
            uint32_t cand = (uint32_t)(((uint64_t)philox_w0(seed, slot, 1u, 0u) * (uint64_t)D) >> 32);
            if (regrow_mode == HO_REGROW_UNUSED) {
                for (uint32_t t = 0; t < HO_UNUSED_MAX_TRIES; ++t) {
                    cand = (uint32_t)(((uint64_t)philox_w0(seed, slot, 1u, t) * (uint64_t)D) >> 32);
                    int used = 0;
                    for (int64_t q = 0; q < F; ++q) {
                        /* current index set: kept slots, and pruned slots already regrown (q < j) */
                        if ((!mk[q] || q < j) && gi[q] == (int32_t)cand) { used = 1; break; }
                    }
                    if (!used) break;
                }
            }
            gi[j] = (int32_t)cand;
        }
        int64_t l0 = g * G, l1 = l0 + G < O ? l0 + G : O;
        for (int64_t l = l0; l < l1; ++l) {
            for (int64_t j = 0; j < F; ++j) {
                if (!mk[j]) continue;
                if (init_mode == HO_INIT_ZERO) {
                    w_set(W, w_dtype, l * F + j, 0.0f);
                } else {
                    uint32_t u = philox_w0(seed, (uint32_t)(l * F + j), 2u, 0u);
                    float u01 = (float)(u >> 8) * 0x1p-24f;
                    w_set(W, w_dtype, l * F + j, fmaf(u01, 2.0f * bound, -bound));
                }
            }
        }
    }
    return total;
}
