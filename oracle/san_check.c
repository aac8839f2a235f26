/*
 * san_check.c -- drives every function of haste_oracle.c on small inputs and
 * their edge cases (empty and one-element arrays, ragged tails, NaN and
 * infinities, sizes that leave a partial last group, every dtype and mode), for
 * the AddressSanitizer / UndefinedBehaviorSanitizer build of `make -C oracle
 * sanitize`.  Test infrastructure only, like the oracle.  Prints "san_check OK"
 * and exits 0 when every call returned; a sanitizer report aborts the run.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void ho_philox4x32(const uint32_t ctr[4], const uint32_t key[2], int rounds, uint32_t out[4]);
uint32_t ho_randint(uint64_t seed, uint64_t offset);
void ho_randint_array(uint64_t seed, uint64_t offset0, int64_t n, uint32_t* out);
uint16_t ho_f32_to_bf16_rne(float f);
uint16_t ho_sr_bf16(float x, uint32_t r);
void ho_sr_round_bf16(const float* x, uint16_t* out, int64_t n, uint64_t seed, uint64_t offset0);
float ho_f16_to_f32(uint16_t h);
uint16_t ho_f32_to_f16_rne(float f);
void ho_sgd_sr_step(uint16_t* w, const void* g, int g_dtype, float* m, int64_t n, float lr,
                    float wd, float mu, int use_mom, int do_sr, uint64_t seed, uint64_t offset0);
void ho_sgd_sr_step_f16w(uint16_t* w, const void* g, int g_dtype, float* m, int64_t n, float lr,
                         float wd, float mu, int use_mom, int do_sr, uint64_t seed,
                         uint64_t offset0);
float ho_f8_to_f32(uint8_t c, int fmt);
uint8_t ho_f32_to_f8(float f, int fmt);
uint8_t ho_sr_e4m3(float x, uint32_t r);
void ho_sr_round(const float* x, void* out, int out_dtype, int64_t n, uint64_t seed,
                 uint64_t offset0);
void ho_sgd_sr_step_f8w(uint8_t* w, int w_fmt, const void* g, int g_dtype, float* m, int64_t n,
                        float lr, float wd, float mu, int use_mom, int do_sr, uint64_t seed,
                        uint64_t offset0);
void ho_f8_to_f32_arr(const uint8_t* c, int fmt, float* out, int64_t n);
void ho_f32_to_f8_arr(const float* x, int fmt, uint8_t* out, int64_t n);
void ho_sr_e4m3_words(float x, const uint32_t* r, uint8_t* out, int64_t n);
void ho_f32_to_f16_rne_arr(const float* x, uint16_t* out, int64_t n);
void ho_f32_to_bf16_rne_arr(const float* x, uint16_t* out, int64_t n);
void ho_rewire_scores(const void* W, int w_dtype, float* scores, int64_t O, int64_t F, int64_t G);
void ho_rewire_scores_ex(const void* W, int w_dtype, const float* grad, int prod_dtype,
                         int score_mode, float* scores, int64_t O, int64_t F, int64_t G);
int64_t ho_rewire_ex(void* W, int w_dtype, int32_t* idx, const float* grad, int prod_dtype,
                     int score_mode, int64_t O, int64_t F, int64_t G, int64_t D, int prune_mode,
                     float thr, int64_t k, int regrow_mode, int init_mode, float bound,
                     uint64_t seed, float* scores_out, uint8_t* mask_out);
int64_t ho_rewire(void* W, int w_dtype, int32_t* idx, int64_t O, int64_t F, int64_t G, int64_t D,
                  int prune_mode, float thr, int64_t k, int regrow_mode, int init_mode,
                  float bound, uint64_t seed, float* scores_out, uint8_t* mask_out);

enum { BF16 = 0, F16 = 1, F32 = 2, E4M3 = 3, E5M2 = 4 };

static uint32_t lcg = 12345u;
static float frand(void) {
    lcg = lcg * 1664525u + 1013904223u;
    return ((float)(lcg >> 8) * 0x1p-24f) * 2.0f - 1.0f;
}

/* exactly-sized heap buffers, so that an access one past the end is reported */
static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) abort();
    return p;
}

static float* values(int64_t n) {
    float* x = (float*)xmalloc(sizeof(float) * (size_t)n);
    for (int64_t i = 0; i < n; ++i) x[i] = frand() * (i % 7 == 0 ? 500.0f : 1.0f);
    if (n > 3) { x[1] = INFINITY; x[2] = -INFINITY; x[3] = NAN; }
    if (n > 5) { x[4] = 3e-40f; x[5] = -0.0f; }
    return x;
}

static void check_sr_and_sgd(void) {
    const int64_t sizes[] = {0, 1, 7, 100};
    for (size_t si = 0; si < sizeof(sizes) / sizeof(sizes[0]); ++si) {
        const int64_t n = sizes[si];
        float* x = values(n);
        uint16_t* o16 = (uint16_t*)xmalloc(2 * (size_t)n);
        uint8_t* o8 = (uint8_t*)xmalloc((size_t)n);
        uint32_t* r = (uint32_t*)xmalloc(4 * (size_t)n);
        float* f = (float*)xmalloc(4 * (size_t)n);
        ho_randint_array(7, (uint64_t)1 << 32, n, r);
        ho_sr_round_bf16(x, o16, n, 3, 5);
        ho_sr_round(x, o16, BF16, n, 3, 5);
        ho_sr_round(x, o16, F16, n, 3, 5);
        ho_sr_round(x, o8, E4M3, n, 3, 5);
        ho_sr_round(x, o8, E5M2, n, 3, 5);
        ho_f32_to_f16_rne_arr(x, o16, n);
        ho_f32_to_bf16_rne_arr(x, o16, n);
        ho_f32_to_f8_arr(x, E4M3, o8, n);
        ho_f8_to_f32_arr(o8, E4M3, f, n);
        ho_f32_to_f8_arr(x, E5M2, o8, n);
        ho_f8_to_f32_arr(o8, E5M2, f, n);
        if (n > 0) ho_sr_e4m3_words(x[0], r, o8, n);
        for (int gd = BF16; gd <= F32; ++gd) {
            void* g = xmalloc((gd == F32 ? 4 : 2) * (size_t)n);
            for (int64_t i = 0; i < n; ++i) {
                if (gd == F32) ((float*)g)[i] = frand();
                else ((uint16_t*)g)[i] = gd == BF16 ? ho_f32_to_bf16_rne(frand()) : ho_f32_to_f16_rne(frand());
            }
            for (int mode = 0; mode < 4; ++mode) {
                const int use_mom = mode & 1, do_sr = mode >> 1;
                float* m = (float*)xmalloc(4 * (size_t)n);
                for (int64_t i = 0; i < n; ++i) m[i] = frand() * 0.01f;
                for (int64_t i = 0; i < n; ++i) o16[i] = ho_f32_to_bf16_rne(x[i]);
                ho_sgd_sr_step(o16, g, gd, use_mom ? m : NULL, n, 0.05f, 1e-4f, 0.9f, use_mom,
                               do_sr, 42, 0);
                for (int64_t i = 0; i < n; ++i) o16[i] = ho_f32_to_f16_rne(x[i]);
                ho_sgd_sr_step_f16w(o16, g, gd, use_mom ? m : NULL, n, 0.05f, 1e-4f, 0.9f,
                                    use_mom, do_sr, 42, 0);
                for (int fmt = E4M3; fmt <= E5M2; ++fmt) {
                    ho_f32_to_f8_arr(x, fmt, o8, n);
                    ho_sgd_sr_step_f8w(o8, fmt, g, gd, use_mom ? m : NULL, n, 0.05f, 1e-4f, 0.9f,
                                       use_mom, do_sr, 42, 0);
                }
                free(m);
            }
            free(g);
        }
        free(x); free(o16); free(o8); free(r); free(f);
    }
    uint32_t c[4] = {1, 2, 3, 4}, k[2] = {5, 6}, out[4];
    for (int rounds = 0; rounds <= 10; ++rounds) ho_philox4x32(c, k, rounds, out);
    (void)ho_randint(~(uint64_t)0, ~(uint64_t)0);
    for (int code = 0; code < 256; ++code) {
        (void)ho_f8_to_f32((uint8_t)code, E4M3);
        (void)ho_f8_to_f32((uint8_t)code, E5M2);
        (void)ho_f16_to_f32((uint16_t)(code * 257));
    }
    (void)ho_sr_bf16(NAN, 0xFFFFFFFFu);
    (void)ho_sr_e4m3(-INFINITY, 0xFFFFFFFFu);
    (void)ho_f32_to_f8(3.4e38f, E4M3);
}

static void check_rewire(void) {
    /* (O, F, G, D): a partial last group, one-label groups, F = 1, one group */
    const int64_t shapes[][4] = {{37, 8, 16, 20}, {5, 3, 1, 4}, {9, 1, 4, 2}, {16, 16, 16, 64}};
    for (size_t si = 0; si < sizeof(shapes) / sizeof(shapes[0]); ++si) {
        const int64_t O = shapes[si][0], F = shapes[si][1], G = shapes[si][2], D = shapes[si][3];
        const int64_t Gc = (O + G - 1) / G;
        for (int wd = BF16; wd <= F32; ++wd) {
            const size_t es = wd == F32 ? 4 : 2;
            void* W = xmalloc(es * (size_t)(O * F));
            float* grad = (float*)xmalloc(4 * (size_t)(O * F));
            int32_t* idx = (int32_t*)xmalloc(4 * (size_t)(Gc * F));
            float* scores = (float*)xmalloc(4 * (size_t)(Gc * F));
            uint8_t* mask = (uint8_t*)xmalloc((size_t)(Gc * F));
            for (int rep = 0; rep < 8; ++rep) {
                for (int64_t i = 0; i < O * F; ++i) {
                    const float v = frand() * 0.3f;
                    grad[i] = frand();
                    if (wd == F32) ((float*)W)[i] = v;
                    else ((uint16_t*)W)[i] = wd == BF16 ? ho_f32_to_bf16_rne(v) : ho_f32_to_f16_rne(v);
                }
                for (int64_t i = 0; i < Gc * F; ++i) idx[i] = (int32_t)((uint32_t)(i * 7919) % (uint32_t)D);
                const int prune = rep % 3, regrow = (rep >> 1) & 1, init = (rep >> 2) & 1;
                const int64_t k = prune == 1 ? F / 2 : prune == 2 ? Gc * F / 3 : 0;
                ho_rewire_scores(W, wd, scores, O, F, G);
                ho_rewire_scores_ex(W, wd, rep & 1 ? grad : NULL, wd == F32 ? F32 : wd, rep & 1,
                                    scores, O, F, G);
                if (prune == 2) {  /* global fraction over the layer */
                    (void)ho_rewire_ex(W, wd, idx, rep & 1 ? grad : NULL, F32, rep & 1, O, F, G, D,
                                       prune, 0.0f, k, regrow, init, 0.1f, 9, scores, mask);
                } else {
                    (void)ho_rewire(W, wd, idx, O, F, G, D, prune, 0.1f, k, regrow, init, 0.1f,
                                    9, scores, mask);
                }
            }
            free(W); free(grad); free(idx); free(scores); free(mask);
        }
    }
}

int main(void) {
    check_sr_and_sgd();
    check_rewire();
    printf("san_check OK\n");
    return 0;
}
