/*
 * haste_ffi.h -- C ABI of the MI355X (gfx950) HASTE fixed-fan-in (FFI) layer.
 *
 * Drop-in boundary for HASTE's shared_ffi hot path.  Every pointer is a device
 * pointer unless stated otherwise; `stream` is a hipStream_t passed as void*
 * (NULL = the null stream).  Calls are asynchronous on `stream` and never
 * allocate device memory; scratch space is passed in as `workspace`.
 * Return value: HASTE_OK (0) or a negative HASTE_ERR_* code; the message for
 * the calling thread is in haste_last_error().
 *
 * Layouts (row-major, element strides):
 *   idx   int32 [Gc, F]   group_locations, Gc = ceil(O / G); label l uses row l / G
 *   xT    [D, ldx]        features transposed, columns 0..B-1 used, ldx % 8 == 0
 *   W     [O, F]          weights
 *   out   [B, ldo]        logits, columns 0..O-1 written, ldo % 8 == 0
 *   dY    [B, lddy]       grad of logits, lddy >= O, 2-byte aligned.  Rows that do
 *                         not all start on 16-byte boundaries (lddy % 8 != 0, or dY
 *                         not 16-byte aligned) need O >= 16, and then the last row
 *                         need only hold O elements (a [B, O] tensor, or a column
 *                         block of a wider one); they are read at some extra cost
 * Element types are HASTE_DTYPE_* codes; other 16-bit tensors must be 16-byte aligned.
 * Supported: dtype bf16 or f16 (fp32 layers: haste_ffi_forward_f16_f32out, and the
 * fp16 entry points on fp16 copies, as the reference's fp32 kernels compute);
 * G in {16, 32, 64, 128}; F % 16 == 0, 16 <= F <= 256.
 * The reference envelope is G in {16,32,64}, F <= 128 (F <= 256 for G = 16);
 * this library accepts the wider set.
 */
#ifndef HASTE_FFI_H
#define HASTE_FFI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    HASTE_OK = 0,
    HASTE_ERR_INVALID_ARG = -1,
    HASTE_ERR_UNSUPPORTED = -2,
    HASTE_ERR_WORKSPACE = -3,
    HASTE_ERR_HIP = -4
};

enum { HASTE_DTYPE_BF16 = 0, HASTE_DTYPE_F16 = 1, HASTE_DTYPE_F32 = 2 };
/* OCP float8 formats (torch.float8_e4m3fn, torch.float8_e5m2), for the outputs
 * of haste_sr_round and the weights of haste_sgd_sr_step_f8 only. */
enum { HASTE_DTYPE_F8E4M3 = 3, HASTE_DTYPE_F8E5M2 = 4 };

enum { HASTE_PRUNE_THRESHOLD = 0, HASTE_PRUNE_FRACTION = 1, HASTE_PRUNE_GLOBAL_FRACTION = 2 };
enum { HASTE_SCORE_MEAN = 0, HASTE_SCORE_MAX = 1 };
enum { HASTE_REGROW_RANDOM = 0, HASTE_REGROW_UNUSED = 1 };
enum { HASTE_INIT_ZERO = 0, HASTE_INIT_RANDOM = 1 };

/* Message for the last failed call on this thread ("" if none). */
const char* haste_last_error(void);

/* ABI version of this library (increments on incompatible changes). */
int haste_abi_version(void);

/*
 * Grouped FFI forward:
 *   out[b, l] = RNE( sum_j xT[idx[l/G, j], b] * W[l, j]  (+ bias[l]) ),  fp32 accumulation.
 * bias may be NULL.  Replaces ffi_forward_cuda (shared_ffi/ffi_forward_kernels.cu:492-719,
 * bound at shared_ffi/ffi_wrapper.cpp:22-26,32-44), whose output is [B, ceil8(O)].
 */
int haste_ffi_forward(const int32_t* idx, const void* xT, int64_t ldx, const void* W,
                      const void* bias, void* out, int64_t ldo, int64_t B, int64_t D, int64_t F,
                      int64_t O, int64_t G, int32_t dtype, void* stream);

/*
 * The forward of an fp32 layer:
 *   out[b, l] = sum_j xT[idx[l/G, j], b] * W[l, j]  (+ bias[l]),  fp32 accumulation,
 * with xT and W in fp16, bias (may be NULL) and out in fp32 (out 16-byte
 * aligned, ldo % 8 == 0).  Replaces the fp32 instantiation of ffi_forward_cuda
 * (group_shared_fanin_v1_fp32, shared_ffi/ffi_forward_kernels.cu:289-485,
 * dispatched at :549-557), which rounds the fp32 features and weights to fp16
 * (to nearest) as it loads them, accumulates in fp32 and adds the fp32 bias;
 * here the caller passes the fp16 copies.
 */
int haste_ffi_forward_f16_f32out(const int32_t* idx, const void* xT, int64_t ldx, const void* W,
                                 const float* bias, float* out, int64_t ldo, int64_t B, int64_t D,
                                 int64_t F, int64_t O, int64_t G, void* stream);

/*
 * Grouped FFI forward fused with the sparse BCE loss of the application's
 * training loop (src/runner.py:469-478, labels in the COO [nnz, 2] int32
 * (row, label) form of src/data.py:26-46):
 *   x[b, l]  = the forward's bf16 logit (RNE of the fp32 sum + bias);
 *   dY[b, l] = RNE(sigma(x) - y[b, l]), the gradient of the loss in x (the
 *              autograd of the reference formula through PyTorch's bf16 ops is
 *              this up to rounding);
 *   *loss    = sum over b < B, l < O of max(x, 0) - y*x + log(1 + exp(-|x|)),
 *              fp32, summed in a fixed order (deterministic).
 * y is 1 at the listed (row, label) pairs (duplicates count once; pairs
 * outside [0, B) x [0, O) are ignored).  dY has the layout of haste_ffi_forward's
 * out (columns >= O of the last group are zero); logits, if not NULL, also
 * receives x.  loss is a device pointer to one float.  The workspace
 * (haste_ffi_forward_bce_workspace_size bytes, 16-byte aligned) must be zero
 * before its first use; every call leaves it zero again.  No counterpart in
 * shared_ffi: replaces the application's logits -> _bce_loss -> autograd
 * sequence, so the logits need not make a round trip through HBM.
 */
int64_t haste_ffi_forward_bce_workspace_size(int64_t B, int64_t O, int64_t G);
int haste_ffi_forward_bce(const int32_t* idx, const void* xT, int64_t ldx, const void* W,
                          const void* bias, const int32_t* labels, int64_t nnz, void* dY,
                          int64_t ldo, void* logits, float* loss, void* workspace,
                          int64_t ws_bytes, int64_t B, int64_t D, int64_t F, int64_t O,
                          int64_t G, int32_t dtype, void* stream);

/*
 * haste_ffi_forward_bce that allocates nothing and takes no workspace: the
 * workspace is the library's own device scratch array, HASTE_FORWARD_BCE_SCRATCH_BYTES
 * (64 MiB) on every GPU the library runs on, held until the process ends.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc); no counterpart in the
 * reference.  Shapes whose haste_ffi_forward_bce_workspace_size exceeds the
 * scratch are rejected with HASTE_ERR_WORKSPACE (BASELINE configs 0-3 fit;
 * config 4's 384 MB label bitmap does not).  Results are bit-identical to
 * haste_ffi_forward_bce.  All calls on one GPU share its scratch, so calls that
 * overlap in time on one GPU (on different streams) race; calls on one stream
 * are ordered.  Each call clears the part of the scratch it needs (a fill
 * kernel, no memset node).
 */
#define HASTE_FORWARD_BCE_SCRATCH_BYTES (64ll << 20)
int haste_ffi_forward_bce_noalloc(const int32_t* idx, const void* xT, int64_t ldx, const void* W,
                                  const void* bias, const int32_t* labels, int64_t nnz, void* dY,
                                  int64_t ldo, void* logits, float* loss, int64_t B, int64_t D,
                                  int64_t F, int64_t O, int64_t G, int32_t dtype, void* stream);

/*
 * Workspace bytes needed by haste_ffi_bwd_features / haste_ffi_bwd_features_sr.
 * Returns a negative HASTE_ERR_* code for unsupported shapes.
 */
int64_t haste_ffi_bwd_features_workspace_size(int64_t B, int64_t D, int64_t F, int64_t O,
                                              int64_t G, int32_t dtype);

/*
 * How haste_ffi_bwd_features splits the work for these sizes (host-only, no
 * GPU call): cfg[0] = batch columns per workgroup, cfg[1] = W^T tiles of 16
 * positions per LDS ring round (0 for the staged build, whose waves own one
 * tile each), cfg[2] = feature ranges, cfg[3] = group slices.  The split
 * depends on the build selected by haste_ffi_bwd_features_set_build.  For
 * tuning and tests; no counterpart in the reference.
 */
int haste_ffi_bwd_features_config(int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                                  int32_t dtype, int64_t* cfg);

/*
 * Selects the main kernel of later bwd-features calls in this process
 * (host-only): 0 (the default) and 3 the staged build for G >= 32, else the
 * LDS-ring build; 1 always the LDS-ring build; 2 the direct build wherever it
 * exists (G = 32 or 64, and a group slice's transposed weights under 2 GB),
 * else the ring build.  The builds give the same
 * results up to the order of fp32 additions.  The workspace layout (plan)
 * differs between the staged build and the others, so a plan made under one
 * setting must be remade (plan_ready = 0) after a change.  Returns the
 * previous setting, or HASTE_ERR_INVALID_ARG for another value.  For tests and
 * tuning; no counterpart in the reference.
 */
int haste_ffi_bwd_features_set_build(int32_t build);

/*
 * Writes the index-dependent part of the bwd-features workspace (the "plan":
 * per group, the distinct indices laid out in tiles per feature range).  It
 * depends on idx and the sizes only, so a caller may compute it once and pass
 * plan_ready = 1 to later haste_ffi_bwd_features[_sr] calls on the same
 * workspace for as long as idx is unchanged (e.g. between two rewires).
 * No counterpart in the reference (which has no index preprocessing).
 */
int haste_ffi_bwd_features_plan(const int32_t* idx, void* workspace, int64_t workspace_bytes,
                                int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                                int32_t dtype, void* stream);

/*
 * Backward to features, deterministic (no float atomics on any global buffer):
 *   dXT[d, b] = sum_{g,j: idx[g,j] = d} sum_{l in g} W[l, j] * dY[b, l]     (fp32 [D, B])
 * plan_ready = 0 computes the plan in this call; 1 reuses the plan already in
 * the workspace (see haste_ffi_bwd_features_plan); 2 also reuses the
 * transposed weights in the workspace, valid when W has not changed since the
 * call that wrote them (a bwd-features call, or haste_ffi_bwd_weights_sgd with
 * this workspace, which writes those of the weights it updates).
 * Replaces ffi_backward_features_cuda (shared_ffi/ffi_backward_features.cu:417-633,
 * bound at shared_ffi/ffi_wrapper.cpp:7-12,29).
 */
int haste_ffi_bwd_features(const int32_t* idx, const void* W, const void* dY, int64_t lddy,
                           float* dXT, void* workspace, int64_t workspace_bytes, int64_t B,
                           int64_t D, int64_t F, int64_t O, int64_t G, int32_t dtype,
                           int32_t plan_ready, void* stream);

/*
 * Backward to features fused with the bf16 stochastic rounding of
 * shared_ffi/bindings.py:44-48: writes dX[b, d] (bf16 bits, [B, D] row-major) =
 * SR(dXT[d, b], tl.randint(seed, b*D + d)).  The reference uses seed 123.
 */
int haste_ffi_bwd_features_sr(const int32_t* idx, const void* W, const void* dY, int64_t lddy,
                              uint16_t* dX, uint64_t seed, void* workspace,
                              int64_t workspace_bytes, int64_t B, int64_t D, int64_t F, int64_t O,
                              int64_t G, int32_t dtype, int32_t plan_ready, void* stream);

/*
 * The first part of haste_ffi_bwd_features[_sr]: the per-slice fp32 partial
 * sums of dX^T, left in the workspace (same arguments and plan_ready meaning).
 * The final pass -- summing the slices into dX -- is then done by
 * haste_ffi_bwd_weights_sgd_dx, inside its own launch, so that a training step
 * runs it in the tail of the fused weight update instead of as a kernel of its
 * own.  No counterpart in the reference (its bwd-features kernel writes dX^T
 * directly, shared_ffi/ffi_backward_features.cu:417-633).
 */
int haste_ffi_bwd_features_partials(const int32_t* idx, const void* W, const void* dY,
                                    int64_t lddy, void* workspace, int64_t workspace_bytes,
                                    int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                                    int32_t dtype, int32_t plan_ready, void* stream);

/*
 * Backward to weights (+ optional bias gradient):
 *   dW[l, j] = sum_b dY[b, l] * xT[idx[l/G, j], b]    stored as dW_dtype (RNE for 16-bit)
 *   dbias[l] = sum_b dY[b, l]                           stored as dbias_dtype (NULL = skip)
 * Replaces ffi_backward_weights_cuda (shared_ffi/ffi_backward_weights.cu:486-684, bound at
 * shared_ffi/ffi_wrapper.cpp:14-19,30) and the bias gradient torch.sum(grad_output, 0)
 * (shared_ffi/bindings.py:40).
 */
int haste_ffi_bwd_weights(const int32_t* idx, const void* xT, int64_t ldx, const void* dY,
                          int64_t lddy, void* dW, int32_t dW_dtype, void* dbias,
                          int32_t dbias_dtype, int64_t B, int64_t D, int64_t F, int64_t O,
                          int64_t G, int32_t dtype, void* stream);

/*
 * haste_ffi_bwd_weights (bf16 layer) that also finishes the backward to
 * features of the same grad_output: dX [B, D] bf16 = SR(sum of the partials
 * that the last haste_ffi_bwd_features_partials call with this workspace and
 * these sizes left in it, tl.randint(dx_seed, b*D + d)), bit-identical to
 * haste_ffi_bwd_features_sr, in trailing workgroups of the same launch instead
 * of a kernel of its own.  dX must not overlap the other buffers.  Replaces, for
 * one FFI layer, the reference's backward of GroupFFIMulFunction
 * (shared_ffi/bindings.py:33-54: ffi_backward_features_cuda + its bf16
 * rounding, ffi_backward_weights_cuda, torch.sum(grad_output, 0)), as
 * haste_ffi_bwd_features_partials + this call.
 */
int haste_ffi_bwd_weights_dx(const int32_t* idx, const void* xT, int64_t ldx, const void* dY,
                             int64_t lddy, void* dW, int32_t dW_dtype, void* dbias,
                             int32_t dbias_dtype, uint16_t* dX, uint64_t dx_seed,
                             void* bwdf_workspace, int64_t bwdf_workspace_bytes, int64_t B,
                             int64_t D, int64_t F, int64_t O, int64_t G, int32_t dtype,
                             void* stream);

/*
 * Backward to weights fused with the SR-SGD step on the bf16 weights and bias:
 * computes the fp32 gradients of haste_ffi_bwd_weights and applies to W [O, F]
 * and bias [O] (in place) the update of haste_sgd_sr_step with g = those fp32
 * gradients -- element offsets l*F + j for W and l for the bias, both from 0,
 * one seed -- so the result is bit-identical to haste_ffi_bwd_weights (fp32
 * dW, dbias) followed by haste_sgd_sr_step_multi over {W, bias}.  The gradients
 * are also stored when dW / dbias are non-NULL.  bias may be NULL (no bias);
 * m_W [O, F] and m_bias [O] are fp32 momentum buffers read when use_mom.
 * bwdf_workspace (may be NULL): a haste_ffi_bwd_features workspace holding the
 * plan for the current idx; the kernel then also writes into it the transposed
 * weights of the UPDATED W, so the next haste_ffi_bwd_features[_sr] call may
 * pass plan_ready = 2.  dtype must be bf16; O*F < 2^32.  Replaces, for one FFI layer, ffi_backward_weights_cuda
 * (shared_ffi/ffi_backward_weights.cu:486-684) + torch.sum(grad_output, 0)
 * (shared_ffi/bindings.py:40) + SRSgd.step's sgd_update calls on the layer's
 * weights and bias (shared_ffi/optim_sr.py:64-112, shared_ffi/sr_triton.py:172-213).
 */
int haste_ffi_bwd_weights_sgd(const int32_t* idx, const void* xT, int64_t ldx, const void* dY,
                              int64_t lddy, uint16_t* W, uint16_t* bias, float* m_W,
                              float* m_bias, void* dW, int32_t dW_dtype, void* dbias,
                              int32_t dbias_dtype, float lr, float wd, float mu, int32_t use_mom,
                              int32_t do_sr, uint64_t seed, void* bwdf_workspace,
                              int64_t bwdf_workspace_bytes, int64_t B, int64_t D, int64_t F,
                              int64_t O, int64_t G, int32_t dtype, void* stream);

/*
 * haste_ffi_bwd_weights_sgd (no dW / dbias outputs; bwdf_workspace required)
 * that also finishes the backward to features of the same step: dX [B, D] bf16
 * = SR(sum of the partials that the last haste_ffi_bwd_features_partials call
 * with this workspace and these sizes left in it, tl.randint(dx_seed, b*D + d)),
 * bit-identical to haste_ffi_bwd_features_sr.  The bwd-features call must have
 * been made with the same W as this call reads (before its update) and an
 * unchanged idx; dX must not overlap the other buffers.  Replaces, for one
 * FFI layer, the reference's backward to features with its bf16 rounding
 * (shared_ffi/bindings.py:44-48), backward to weights and the layer's SR-SGD
 * step, as haste_ffi_bwd_features_partials + this call.
 */
int haste_ffi_bwd_weights_sgd_dx(const int32_t* idx, const void* xT, int64_t ldx, const void* dY,
                                 int64_t lddy, uint16_t* W, uint16_t* bias, float* m_W,
                                 float* m_bias, float lr, float wd, float mu, int32_t use_mom,
                                 int32_t do_sr, uint64_t seed, uint16_t* dX, uint64_t dx_seed,
                                 void* bwdf_workspace, int64_t bwdf_workspace_bytes, int64_t B,
                                 int64_t D, int64_t F, int64_t O, int64_t G, int32_t dtype,
                                 void* stream);

/*
 * haste_ffi_bwd_weights_sgd_dx with the SGD step's Philox seed in device memory:
 * the launch reads *seed_dev (a uint64) as its seed and then adds 1 to it on the
 * device (one more small kernel on the stream), the per-step seed schedule of
 * SRSgd (shared_ffi/optim_sr.py:59-62) without a host value.  A training step
 * made of calls that take no host-side state that changes per step can then be
 * captured once in a HIP graph and replayed step after step.  No counterpart in
 * the reference; results are bit-identical to haste_ffi_bwd_weights_sgd_dx with
 * seed = the value *seed_dev held.
 */
int haste_ffi_bwd_weights_sgd_dx_dev_seed(const int32_t* idx, const void* xT, int64_t ldx,
                                          const void* dY, int64_t lddy, uint16_t* W,
                                          uint16_t* bias, float* m_W, float* m_bias, float lr,
                                          float wd, float mu, int32_t use_mom, int32_t do_sr,
                                          uint64_t* seed_dev, uint16_t* dX, uint64_t dx_seed,
                                          void* bwdf_workspace, int64_t bwdf_workspace_bytes,
                                          int64_t B, int64_t D, int64_t F, int64_t O, int64_t G,
                                          int32_t dtype, void* stream);

/*
 * haste_sgd_sr_step on the weights W [O, F] (bf16) of an FFI layer (element
 * offsets l*F + j from 0; bit-identical), which also writes the transposed
 * weights of the UPDATED W into a haste_ffi_bwd_features workspace holding the
 * plan of the layer's idx for these sizes (B, D, F, O, G), so that the next
 * haste_ffi_bwd_features[_sr] call may pass plan_ready = 2 and skip gathering
 * them.  g: gradient [O, F] (bf16, f16 or f32); m: fp32 momentum [O, F], read
 * and written when use_mom.  Replaces, for an FFI weight matrix, SRSgd.step's
 * sgd_update call (shared_ffi/optim_sr.py:99-109, shared_ffi/sr_triton.py:172-213);
 * the transposed weights have no counterpart in the reference.
 */
int haste_sgd_sr_step_wt(uint16_t* W, const void* g, int32_t g_dtype, float* m, float lr,
                         float wd, float mu, int32_t use_mom, int32_t do_sr, uint64_t seed,
                         void* workspace, int64_t workspace_bytes, int64_t B, int64_t D, int64_t F,
                         int64_t O, int64_t G, int32_t dtype, void* stream);

/*
 * haste_sgd_sr_step_wt that also steps the layer's bias [O] (bf16) with its
 * gradient gb [O] (bf16, f16 or f32) and fp32 momentum m_bias (read and written
 * when use_mom), in the same launch: the same update as haste_sgd_sr_step on
 * the bias with the same seed (offsets l from 0), bit-identical.  Replaces, for
 * an FFI layer's weights and bias, SRSgd.step's sgd_update calls on both
 * (shared_ffi/optim_sr.py:99-109, shared_ffi/sr_triton.py:172-213).
 */
int haste_sgd_sr_step_wt_bias(uint16_t* W, const void* g, int32_t g_dtype, float* m,
                              uint16_t* bias, const void* gb, int32_t gb_dtype, float* m_bias,
                              float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                              uint64_t seed, void* workspace, int64_t workspace_bytes, int64_t B,
                              int64_t D, int64_t F, int64_t O, int64_t G, int32_t dtype,
                              void* stream);

/*
 * The random words of the stochastic rounding alone: draws tl.randint(seed, i)
 * for i < n, as the SR and SR-SGD kernels do, and writes the XOR of each 64
 * consecutive words: fold[t] = XOR of words 64t .. min(64t + 63, n - 1),
 * t < ceil(n / 64).  No counterpart in the reference: it times the arithmetic
 * floor of the SR-SGD step (Philox4x32-10 per weight, which bit-exact
 * tl.randint fixes), the bound beside HBM for those kernels.
 */
int haste_sr_words_fold(uint32_t* fold, int64_t n, uint64_t seed, void* stream);

/*
 * Stochastic rounding fp32 -> bf16: out[i] = SR(x[i], tl.randint(seed, offset0 + i)).
 * Replaces stochastic_rounding (shared_ffi/sr_triton.py:51-59).
 */
int haste_sr_round_bf16(const float* x, uint16_t* out, int64_t n, uint64_t seed,
                        uint64_t offset0, void* stream);

/*
 * stochastic_rounding (shared_ffi/sr_triton.py:43-59) for the other output
 * dtypes the reference dispatches on (out_dtype): HASTE_DTYPE_F8E4M3 takes
 * stochastic_rounding_to_fp8 (sr_triton.py:18-25: the low 20 bits of
 * tl.randint(seed, offset0 + i) added to the fp32 pattern, the low 20 bits
 * cleared, then converted); HASTE_DTYPE_BF16, HASTE_DTYPE_F16 and
 * HASTE_DTYPE_F8E5M2 take the bf16 rounding of haste_sr_round_bf16, stored in
 * the output dtype (as the reference's store converts it).  Conversions round to
 * nearest even; fp8 ones saturate (finite overflow and infinities become the
 * largest finite value with the sign kept, NaN becomes sign | 0x7F).  out holds
 * n elements of 2 (bf16, fp16) or 1 (fp8) bytes.
 */
int haste_sr_round(const float* x, void* out, int32_t out_dtype, int64_t n, uint64_t seed,
                   uint64_t offset0, void* stream);

/*
 * Fused SGD step on bf16 weights, in place (one pass):
 *   g' = fma(wd, w, g);  [m' = fma(mu, m, g'); m = m';]  w' = fma(-lr, m' or g', w)
 *   w  = do_sr ? SR(w', tl.randint(seed, offset0 + i)) : RNE(w')
 * g_dtype: bf16, f16 or f32.  m (fp32) may be NULL when use_mom == 0.
 * Replaces sgd_update / _sgd_m_wd_sr (shared_ffi/sr_triton.py:109-213).
 */
int haste_sgd_sr_step(uint16_t* w, const void* g, int32_t g_dtype, float* m, int64_t n,
                      float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                      uint64_t seed, uint64_t offset0, void* stream);

/*
 * haste_sgd_sr_step on fp16 weights: w is read as fp16, the update computed and
 * rounded to bf16 (SR or RNE) exactly as above, and that bf16 value stored as
 * fp16 (round to nearest even) -- what _sgd_m_wd_sr does with an fp16 w_ptr,
 * whose bf16 result the store converts (shared_ffi/sr_triton.py:111, 159-166;
 * fp16 parameters reach it through SRSgd.step, shared_ffi/optim_sr.py:86-109).
 */
int haste_sgd_sr_step_f16(uint16_t* w, const void* g, int32_t g_dtype, float* m, int64_t n,
                          float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                          uint64_t seed, uint64_t offset0, void* stream);

/*
 * haste_sgd_sr_step on fp8 weights (w_dtype HASTE_DTYPE_F8E4M3 or
 * HASTE_DTYPE_F8E5M2, n one-byte codes): _sgd_m_wd_sr (sr_triton.py:109-168)
 * with an fp8 w_ptr.  Weights load exactly; the bf16 result (SR or RNE) is
 * stored as fp8, rounded to nearest even and saturating as in haste_sr_round.
 */
int haste_sgd_sr_step_f8(uint8_t* w, int32_t w_dtype, const void* g, int32_t g_dtype, float* m,
                         int64_t n, float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                         uint64_t seed, uint64_t offset0, void* stream);

/*
 * The same step over several tensors in one launch (one kernel per 8
 * tensors): tensor i uses offsets offset0_i + j.  SRSgd.step calls
 * sgd_update once per parameter (shared_ffi/optim_sr.py:64-112, all
 * parameters of a group share the seed and start at offset 0); this entry
 * point replaces that loop.  n == 0 entries are skipped.
 */
typedef struct haste_sgd_tensor {
    uint16_t* w;
    const void* g;
    float* m;
    int64_t n;
    uint64_t offset0;
} haste_sgd_tensor;

int haste_sgd_sr_step_multi(const haste_sgd_tensor* tensors, int32_t count, int32_t g_dtype,
                            float lr, float wd, float mu, int32_t use_mom, int32_t do_sr,
                            uint64_t seed, void* stream);

/*
 * xT[d, b] = x[b, d] for a bf16/f16 matrix x [B, D] with row stride ldx;
 * xT has row stride ldt >= B, and columns B..ldt-1 of xT are set to zero.
 * Replaces features.transpose(0, 1).contiguous() (shared_ffi/bindings.py:19).
 */
int haste_transpose_features(const uint16_t* x, int64_t ldx, uint16_t* xT, int64_t ldt, int64_t B,
                             int64_t D, void* stream);

/*
 * On-device rewire of an FFI layer (prune + regrow), in place on W and idx.
 * W is bf16, fp16 or fp32 (w_dtype, as the reference's rewire works in the
 * weights' own dtype).  Replaces GroupFixedFanIn.rewire
 * (shared_ffi/rewire.py:143-239) with a deterministic contract:
 *   score[g, j] = (sequential fp32 sum over the group's rows of |W[l, j]|) / rows
 *   prune: THRESHOLD -> score < threshold; FRACTION -> the k smallest (score, j)
 *   regrow index: RANDOM -> floor(philox(seed; g*F+j, 1, 0).w0 * D / 2^32);
 *                 UNUSED -> attempts t = 0.. with counter (g*F+j, 1, t), first
 *                 candidate not present in the group (64 attempts, then the last)
 *   new weights of every row at a pruned slot: ZERO -> 0;
 *     RANDOM -> fma(u01, 2*bound, -bound), u01 = (philox(seed; l*F+j, 2, 0).w0 >> 8) * 2^-24,
 *     stored in W's dtype (RNE to bf16 / fp16)
 * scores_out [Gc, F] fp32 and n_pruned (one int32, incremented) may be NULL.
 * idx entries are indices in [0, D).  UNUSED regrow is a second launch on the
 * stream: between the two, the pruned slots of idx hold -1.
 */
int haste_rewire(void* W, int32_t w_dtype, int32_t* idx, float* scores_out, int32_t* n_pruned,
                 int64_t O, int64_t F, int64_t G, int64_t D, int32_t prune_mode, float threshold,
                 int64_t k, int32_t regrow_mode, int32_t init_mode, float bound, uint64_t seed,
                 void* stream);

/*
 * The application's rewire variant, GroupFixedFanInReal.rewire
 * (src/group_fanin_real.py:150-286).  haste_rewire_scores writes the fp32
 * scores [ceil(O/G), F]: per slot, the mean (HASTE_SCORE_MEAN, fp32 sum over the
 * group's rows in ascending order / rows) or the max (HASTE_SCORE_MAX) of |W|,
 * or, with grad ([O, F], bf16, fp16 or fp32) not NULL, of the saliency |W * grad|
 * (the product in torch's promoted dtype of W and grad, as the reference's tensor
 * product: rounded to bf16 / fp16 when both are that format, else fp32).
 * haste_rewire_ex is haste_rewire with those score modes and one more prune
 * mode, HASTE_PRUNE_GLOBAL_FRACTION: prune the slots whose key
 * (bits(score) << 32 | g*F + j) is <= *key_thr, the k-th smallest key of the
 * layer (so exactly k slots, the smallest scores, ties to the lower slot),
 * selected by the caller on the device from scores_in (the scores of
 * haste_rewire_scores with the same modes).  Regrow and init as haste_rewire.
 */
int haste_rewire_scores(const void* W, int32_t w_dtype, const void* grad, int32_t grad_dtype,
                        int32_t score_mode, float* scores, int64_t O, int64_t F, int64_t G,
                        void* stream);
int haste_rewire_ex(void* W, int32_t w_dtype, int32_t* idx, const void* grad, int32_t grad_dtype,
                    int32_t score_mode, const float* scores_in, const int64_t* key_thr,
                    float* scores_out, int32_t* n_pruned, int64_t O, int64_t F, int64_t G,
                    int64_t D, int32_t prune_mode, float threshold, int64_t k,
                    int32_t regrow_mode, int32_t init_mode, float bound, uint64_t seed,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HASTE_FFI_H */
