// host_check.cpp -- drives the host-side code of libhaste_ffi (argument
// checks, workspace sizing, the bwd-features plan and build choice) without a
// GPU, for the AddressSanitizer / UndefinedBehaviorSanitizer build of
// `make -C haste_amd sanitize` (host code only; no kernel is launched).  Test
// infrastructure.  Prints "host_check OK" and exits 0 when every check held; a
// sanitizer report aborts the run.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/haste_ffi.h"

static int failures = 0;
#define EXPECT(cond)                                                        \
    do {                                                                    \
        if (!(cond)) {                                                      \
            std::fprintf(stderr, "host_check: %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                     \
        }                                                                   \
    } while (0)

// an argument error: a negative code and a message
static void expect_rejected(int rc) {
    EXPECT(rc < 0);
    EXPECT(std::strlen(haste_last_error()) > 0);
}

static void sizes_and_plans() {
    const int64_t Bs[] = {1, 7, 64, 256, 512, 1024};
    const int64_t Ds[] = {1, 300, 768, 4096};
    const int64_t Fs[] = {16, 32, 48, 128, 256, 8, 300};
    const int64_t Os[] = {1, 17, 4096, 131073, 670091, 3000000};
    const int64_t Gs[] = {16, 32, 64, 128, 8};
    int ok = 0;
    for (int build = 0; build <= 3; ++build) {
        haste_ffi_bwd_features_set_build(build);
        for (int64_t B : Bs)
            for (int64_t D : Ds)
                for (int64_t F : Fs)
                    for (int64_t O : Os)
                        for (int64_t G : Gs)
                            for (int32_t dt = 0; dt <= 2; ++dt) {
                                const int64_t ws = haste_ffi_bwd_features_workspace_size(B, D, F, O, G, dt);
                                int64_t cfg[16];
                                std::memset(cfg, 0xFF, sizeof(cfg));
                                const int rc = haste_ffi_bwd_features_config(B, D, F, O, G, dt, cfg);
                                EXPECT((ws > 0) == (rc == HASTE_OK));
                                if (rc == HASTE_OK) {
                                    ++ok;
                                    EXPECT(cfg[0] > 0 && cfg[2] >= 1 && cfg[3] >= 1);
                                    EXPECT(cfg[2] * 1 <= D + 1);
                                }
                                if (build == 0 && dt == 0) {
                                    const int64_t bw = haste_ffi_forward_bce_workspace_size(B, O, G);
                                    EXPECT(bw != 0);
                                }
                            }
    }
    haste_ffi_bwd_features_set_build(0);
    EXPECT(ok > 0);
    EXPECT(haste_ffi_bwd_features_set_build(7) == HASTE_ERR_INVALID_ARG);
    EXPECT(haste_ffi_bwd_features_set_build(-1) == HASTE_ERR_INVALID_ARG);
}

static void argument_checks() {
    const int64_t B = 64, D = 768, F = 32, O = 4096, G = 32;
    expect_rejected(haste_ffi_forward(nullptr, nullptr, 64, nullptr, nullptr, nullptr, O, B, D, F, O, G, 0, nullptr));
    expect_rejected(haste_ffi_forward_f16_f32out(nullptr, nullptr, 64, nullptr, nullptr, nullptr, O, B, D, F, O, G, nullptr));
    expect_rejected(haste_ffi_forward_bce(nullptr, nullptr, 64, nullptr, nullptr, nullptr, 0, nullptr, O, nullptr,
                                          nullptr, nullptr, 0, B, D, F, O, G, 0, nullptr));
    expect_rejected(haste_ffi_forward_bce_noalloc(nullptr, nullptr, 64, nullptr, nullptr, nullptr, 0, nullptr, O,
                                                  nullptr, nullptr, B, D, F, O, G, 0, nullptr));
    expect_rejected(haste_ffi_forward_bce_noalloc(nullptr, nullptr, 1024, nullptr, nullptr, nullptr, 0, nullptr,
                                                  3000000, nullptr, nullptr, 1024, 768, 128, 3000000, 128, 0,
                                                  nullptr));
    expect_rejected(haste_ffi_bwd_features_plan(nullptr, nullptr, 0, B, D, F, O, G, 0, nullptr));
    expect_rejected(haste_ffi_bwd_features(nullptr, nullptr, nullptr, O, nullptr, nullptr, 0, B, D, F, O, G, 0, 0,
                                           nullptr));
    expect_rejected(haste_ffi_bwd_features_sr(nullptr, nullptr, nullptr, O, nullptr, 1, nullptr, 0, B, D, F, O, G,
                                              0, 0, nullptr));
    expect_rejected(haste_ffi_bwd_features_partials(nullptr, nullptr, nullptr, O, nullptr, 0, B, D, F, O, G, 0, 0,
                                                    nullptr));
    expect_rejected(haste_ffi_bwd_weights(nullptr, nullptr, 64, nullptr, O, nullptr, 2, nullptr, 2, B, D, F, O, G,
                                          0, nullptr));
    expect_rejected(haste_ffi_bwd_weights_sgd(nullptr, nullptr, 64, nullptr, O, nullptr, nullptr, nullptr, nullptr,
                                              nullptr, 2, nullptr, 2, 0.1f, 0.f, 0.f, 0, 1, 1, nullptr, 0, B, D,
                                              F, O, G, 0, nullptr));
    expect_rejected(haste_ffi_bwd_weights_sgd_dx(nullptr, nullptr, 64, nullptr, O, nullptr, nullptr, nullptr,
                                                 nullptr, 0.1f, 0.f, 0.f, 0, 1, 1, nullptr, 123, nullptr, 0, B,
                                                 D, F, O, G, 0, nullptr));
    expect_rejected(haste_ffi_bwd_weights_sgd_dx_dev_seed(nullptr, nullptr, 64, nullptr, O, nullptr, nullptr,
                                                          nullptr, nullptr, 0.1f, 0.f, 0.f, 0, 1, nullptr,
                                                          nullptr, 123, nullptr, 0, B, D, F, O, G, 0, nullptr));
    expect_rejected(haste_sgd_sr_step_wt(nullptr, nullptr, 2, nullptr, 0.1f, 0.f, 0.f, 0, 1, 1, nullptr, 0, B, D,
                                         F, O, G, 0, nullptr));
    expect_rejected(haste_sr_words_fold(nullptr, 10, 1, nullptr));
    expect_rejected(haste_sr_round_bf16(nullptr, nullptr, 10, 1, 0, nullptr));
    expect_rejected(haste_sr_round(nullptr, nullptr, 2, 10, 1, 0, nullptr));
    expect_rejected(haste_sgd_sr_step(nullptr, nullptr, 2, nullptr, 10, 0.1f, 0.f, 0.f, 0, 1, 1, 0, nullptr));
    expect_rejected(haste_sgd_sr_step_f16(nullptr, nullptr, 2, nullptr, 10, 0.1f, 0.f, 0.f, 0, 1, 1, 0, nullptr));
    expect_rejected(haste_sgd_sr_step_f8(nullptr, 3, nullptr, 2, nullptr, 10, 0.1f, 0.f, 0.f, 0, 1, 1, 0, nullptr));
    haste_sgd_tensor t[3] = {{nullptr, nullptr, nullptr, 10, 0}, {nullptr, nullptr, nullptr, 0, 0},
                             {nullptr, nullptr, nullptr, -1, 0}};
    expect_rejected(haste_sgd_sr_step_multi(t, 3, 2, 0.1f, 0.f, 0.f, 0, 1, 1, nullptr));
    expect_rejected(haste_sgd_sr_step_multi(nullptr, 2, 2, 0.1f, 0.f, 0.f, 0, 1, 1, nullptr));
    expect_rejected(haste_transpose_features(nullptr, 768, nullptr, 64, B, D, nullptr));
    expect_rejected(haste_rewire(nullptr, 0, nullptr, nullptr, nullptr, O, F, G, D, 1, 0.f, 4, 1, 0, 0.1f, 1,
                                 nullptr));
    expect_rejected(haste_rewire_scores(nullptr, 0, nullptr, 0, 0, nullptr, O, F, G, nullptr));
    expect_rejected(haste_rewire_ex(nullptr, 0, nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr, nullptr, O, F,
                                    G, D, 2, 0.f, 4, 1, 0, 0.1f, 1, nullptr));
    // zero-sized calls that are no-ops
    EXPECT(haste_sr_words_fold(nullptr, 0, 1, nullptr) == HASTE_OK);
    EXPECT(haste_sr_round(nullptr, nullptr, 3, 0, 1, 0, nullptr) == HASTE_OK);
    EXPECT(haste_sgd_sr_step_multi(nullptr, 0, 2, 0.1f, 0.f, 0.f, 0, 1, 1, nullptr) == HASTE_OK);
}

int main() {
    EXPECT(haste_abi_version() > 0);
    sizes_and_plans();
    argument_checks();
    if (failures) {
        std::fprintf(stderr, "host_check: %d failed checks\n", failures);
        return 1;
    }
    std::printf("host_check OK\n");
    return 0;
}
