/*
 * moebius-hip C API: the MI355X (gfx950) conv/norm hot path of moebius-cpu.
 *
 * Conventions follow the reference's C API (include/moebius_cpu.h:11-19,
 * 48-51): status codes, a thread-local last-error string, no exceptions or
 * panics across the boundary. Below it, one entry point per `src/engine`
 * kernel a Rust `extern "C"` shim would bind in place of the CPU kernel
 * (each cites the reference function it replaces), plus the device plumbing
 * (context, memory, events) such a shim needs.
 *
 * Memory and ordering:
 *  - Tensors are device pointers to dense NHWC f32 (row-major over n, h, w, c),
 *    exactly the reference's `Tensor` layout (src/engine/tensor.rs:11-34).
 *  - Weights use the converter layouts (tools/convert_weights.py:25-28):
 *    1x1 [c_out, c_in], dense 3x3 [c_out, 3, 3, c_in], depthwise [3, 3, c].
 *    GEMM weights may be f32 or f16 (`Param`, src/engine/param.rs:14-17);
 *    f16 is widened to f32 exactly before the arithmetic.
 *  - Outputs must not alias inputs (src/engine/tensor.rs:58) unless the entry
 *    point says "in place".
 *  - Every kernel entry point is asynchronous on the context's stream (no
 *    host synchronisation); mh_synchronize / mh_memcpy_d2h order the host.
 *  - Shape checks that the reference asserts (a panic) return
 *    MH_ERR_INVALID_ARGUMENT with the reference's assertion text.
 */
#ifndef MOEBIUS_HIP_H
#define MOEBIUS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MH_ABI_VERSION 1u

/* Same values as MOEBIUS_OK .. MOEBIUS_ERR_INTERNAL (include/moebius_cpu.h:13-19). */
#define MH_OK 0
#define MH_ERR_INVALID_ARGUMENT 1
#define MH_ERR_WEIGHTS 2
#define MH_ERR_UNSUPPORTED_DEVICE 3 /* moebius_cpu.h: MOEBIUS_ERR_UNSUPPORTED_CPU */
#define MH_ERR_CANCELLED 4
#define MH_ERR_IO 5
#define MH_ERR_INTERNAL 6
#define MH_ERR_OUT_OF_MEMORY 7 /* new: device memory exhausted */

/* Param storage (src/engine/param.rs:14-17). */
#define MH_DTYPE_F32 0u
#define MH_DTYPE_F16 1u

/* Depthwise epilogues (src/engine/depthwise.rs:22-28). */
#define MH_EPILOGUE_NONE 0u
#define MH_EPILOGUE_RELU 1u
#define MH_EPILOGUE_GLU_SILU 2u

/* Arithmetic of the GEMM-shaped kernels. EXACT: f32 MFMA, f32 accumulate (the
 * reference's arithmetic). FAST: activations and weights rounded to f16, f16
 * MFMA with f32 accumulate, and the SiLU of those kernels and of the depthwise
 * convs from the hardware exp2 and reciprocal (within a few ulp of the
 * reference's). */
#define MH_PRECISION_EXACT 0u
#define MH_PRECISION_FAST 1u

/* Conditioning rows of a UNet step (src/unet/mod.rs:46-60). */
#define MH_GUIDANCE_CFG 0u       /* batch 2: items 0 = uncond, 1 = cond */
#define MH_GUIDANCE_COND_ONLY 1u /* batch 1: cond */

typedef struct MhContext MhContext;
typedef struct MhEvent MhEvent;
typedef struct MhUNet MhUNet;
typedef struct MhVae MhVae;

/* One converter tensor (tools/convert_weights.py:13-33 names and layouts) in
 * host memory: GEMM weights F32 or F16, everything else F32. */
typedef struct MhNamedTensor {
    const char *name;
    const void *data;
    uint32_t dtype; /* MH_DTYPE_* */
    uint32_t reserved;
    uint64_t numel;
} MhNamedTensor;

/* Per-block trace callback (src/unet/mod.rs:148-157): `dev` is a device
 * pointer valid during the call; the stream is idle when it is made. */
typedef void (*MhTraceFn)(void *user, const char *name, const float *dev, uint32_t n, uint32_t h, uint32_t w,
                          uint32_t c);

/* ---- library / context (moebius_cpu.h:48-56 conventions) ---- */
uint32_t mh_abi_version(void);
/* Message of the last failed call on the calling thread. Never NULL. */
const char *mh_last_error(void);
/* device: HIP ordinal. Creates one stream (default priority) and a workspace. */
int32_t mh_context_create(int32_t device, MhContext **out);
void mh_context_destroy(MhContext *ctx);
int32_t mh_context_set_precision(MhContext *ctx, uint32_t precision);
/* Tuning override of one context for A/B runs and tests, as MOEBIUS_GEMM picks
 * the CPU engine's GEMM backend (src/engine/gemm.rs:57-60); no other reference
 * counterpart. key: "gemm_plan" ("bm,bn,splits"), "gn_in_maxc", "dw_tiled",
 * "tap_heads" ("t8", "t4", "8", "4", "2", "1"), "cross_heads", "gn_blocks" (>= 64),
 * "gn_apply" (1: the GroupNorm apply pass walks the map from its end), "wino_fused" (-1:
 * Winograd convs in one kernel where that is faster, 1: wherever it fits, 0: never); value NULL or ""
 * restores the measured default. The same settings are read once from the
 * MOEBIUS_HIP_<KEY> environment variables when the context is created. */
int32_t mh_context_set_tuning(MhContext *ctx, const char *key, const char *value);
/* GEMM launches timed on the device while the tuning key "gemm_time" is 1 (no
 * counterpart in the reference): synchronises the context's stream, then writes
 * into buf, as JSON, one record per kernel configuration (tile, wave layout,
 * operand mode, grid) in order of first launch: {"config", "launches", "us" (the
 * summed time between events recorded before and after each launch, its split-K
 * reduce included), "flops" (2.M.N.K per launch, summed)}, and clears the
 * records. *needed receives the text's size with its terminator; a buffer
 * smaller than that returns MH_ERR_INVALID_ARGUMENT and keeps the records. */
int32_t mh_context_gemm_times(MhContext *ctx, char *buf, uint64_t len, uint64_t *needed);
/* The context's hipStream_t, for callers that order their own work with it. */
void *mh_context_stream(MhContext *ctx);
int32_t mh_synchronize(MhContext *ctx);
/* Name of the device's ISA (e.g. "gfx950") into buf; fails on other ISAs' kernels. */
int32_t mh_device_arch(MhContext *ctx, char *buf, uint32_t len);

/* ---- device memory (the reference's Vec<f32> buffers, now in HBM) ---- */
int32_t mh_malloc(MhContext *ctx, uint64_t bytes, void **out);
int32_t mh_free(MhContext *ctx, void *ptr);
/* Synchronous copies on the context's stream. */
int32_t mh_memcpy_h2d(MhContext *ctx, void *dst, const void *src, uint64_t bytes);
int32_t mh_memcpy_d2h(MhContext *ctx, void *dst, const void *src, uint64_t bytes);
int32_t mh_memcpy_d2d(MhContext *ctx, void *dst, const void *src, uint64_t bytes);

/* ---- timing on the context's stream ---- */
int32_t mh_event_create(MhContext *ctx, MhEvent **out);
int32_t mh_event_record(MhContext *ctx, MhEvent *ev);
/* Waits for `end`; milliseconds between the two records. */
int32_t mh_event_elapsed_ms(MhEvent *start, MhEvent *end, float *ms);
void mh_event_destroy(MhEvent *ev);

/* ---- engine kernels (src/engine) ---- */

/* src/engine/conv.rs:170-191 `init_output`, fused with the accumulate it
 * prepares: out[r, :] = (residual[r, :] + bias) + x[r, :]. bias and residual
 * may each be NULL (then that term is absent). rows x cols, row-major. */
int32_t mh_bias_residual_add(MhContext *ctx, const float *x, uint64_t rows, uint32_t cols, const float *bias,
                             const float *residual, float *out);

/* src/engine/conv.rs:38-55 `Conv1x1::forward`: out = x . W^T + bias (+ residual).
 * x [n,h,w,c_in]; weight [c_out, c_in] (dtype MH_DTYPE_*); bias [c_out] or NULL;
 * residual [n,h,w,c_out] or NULL; out [n,h,w,c_out]. */
int32_t mh_conv1x1_forward(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                           const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                           const float *residual, float *out);

/* Conv1x1::forward fused with what the reference does around it in a resnet
 * block (src/unet/blocks.rs:47-52, 98-109): the residual is transformed per item
 * and channel as GroupNorm's apply would, [SiLU](residual . scale + shift) with
 * scale/shift [n * c_out] from mh_group_norm_affine (the normalised block input
 * is never stored), and a second residual is added last, as the block's
 * add_inplace: out = ((residual' + bias) + x . W^T) + residual2. residual_scale
 * and residual_shift NULL: residual used as is; residual2 may be NULL. */
int32_t mh_conv1x1_fused(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                         const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                         const float *residual, const float *residual_scale, const float *residual_shift,
                         uint32_t residual_silu, const float *residual2, float *out);

/* No counterpart in the reference, whose GroupNorm always reads its input
 * (src/engine/norm.rs:57-105): the GroupNorm statistics a 1x1 conv's epilogue
 * writes, which this library's UNet hands to the next GroupNorm instead of a
 * statistics pass; exposed so they can be checked. out as mh_conv1x1_forward;
 * part [pixels / *rows][c_out][2]: per output tile of *rows pixels, each
 * channel's sum and sum of squares of the values stored (needs
 * ceil(pixels / 32) * c_out * 2 floats, 16-byte aligned). *rows is 0 (part not
 * written) when the chosen tiling cannot write them (split K, rows per item not
 * a multiple of the tile). */
int32_t mh_conv1x1_gn_partials(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                               const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                               const float *residual, float *out, float *part, uint32_t *rows);

/* src/engine/conv.rs:77-81 `Conv3x3::output_hw`. pad = [top, left, bottom, right]. */
int32_t mh_conv3x3_output_hw(uint32_t h, uint32_t w, uint32_t stride, const uint32_t pad[4], uint32_t upsample2x,
                             uint32_t *ho, uint32_t *wo);

/* src/engine/conv.rs:83-102 `Conv3x3::forward` / `forward_prologue`:
 * out = conv3x3(f(x)) + bias, any stride / padding, optional nearest-2x
 * upsample of the input; f is the GroupNorm affine (+SiLU) of
 * src/engine/norm.rs:33-37 when prologue_scale/shift ([n * c_in] each) are
 * given, applied to in-image values only (padding stays zero). As in the
 * reference, a prologue needs stride 1 and pad [1,1,1,1].
 * weight [c_out, 3, 3, c_in]; out [n, ho, wo, c_out]. */
int32_t mh_conv3x3_forward(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                           const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                           uint32_t stride, const uint32_t pad[4], uint32_t upsample2x, const float *prologue_scale,
                           const float *prologue_shift, uint32_t prologue_silu, float *out);

/* src/engine/winograd.rs:254-297 `transform_kernel` / `kernel_transform`:
 * U = G g G^T for every (output, input) channel pair, G = [[1,0,0],
 * [1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]], in the reference's operation order;
 * f16 weights are widened (exactly) first, as winograd.rs:260-263 does.
 * weight [c_out, 3, 3, c_in]; u [16, c_out, c_in] f32. */
int32_t mh_winograd_weight_transform(MhContext *ctx, const void *weight, uint32_t weight_dtype, uint32_t c_out,
                                     uint32_t c_in, float *u);

/* src/engine/winograd.rs:144-160, 210-251, 299-327 (`Geo::input_tile`,
 * `fill_strip`, `input_transform`): V = B^T d B for every 2x2 output tile
 * (tiles = n * ceil(H/2) * ceil(W/2), H x W the output = the (upsampled)
 * input size, ordered item, tile row, tile column), d the tile's 4x4 input
 * patch: zero outside the image, nearest-2x upsample when upsample2x, the
 * GroupNorm affine (+SiLU) prologue on in-image values when prologue_scale /
 * prologue_shift ([n * c] each) are given. x [n, h, w, c]; v [16, tiles, c];
 * c a multiple of 4. */
int32_t mh_winograd_input_transform(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                                    uint32_t upsample2x, const float *prologue_scale, const float *prologue_shift,
                                    uint32_t prologue_silu, float *v);

/* src/engine/winograd.rs:164-202, 329-352 (`Geo::output_band`,
 * `output_transform`): out = A^T m A + bias per tile, A^T = [[1,1,1,0],
 * [0,1,-1,-1]]; the pixels of partial tiles (odd H or W) are not written.
 * m [16, tiles, c_out]; bias [c_out] or NULL; out [n, H, W, c_out]. */
int32_t mh_winograd_output_transform(MhContext *ctx, const float *m, uint32_t n, uint32_t h, uint32_t w,
                                     uint32_t c_out, uint32_t upsample2x, const float *bias, float *out);

/* src/engine/winograd.rs:48-120 `conv3x3_same` (the stride-1 / pad-1 path of
 * `Conv3x3::forward` / `forward_prologue`, src/engine/conv.rs:92-102):
 * the input transform, 16 matrix-core GEMMs [tiles x c_in] . [c_in x c_out]
 * in one batched launch, and the output transform. u from
 * mh_winograd_weight_transform (the transformed kernel, built once per
 * weight as the reference does per call); c_in, c_out multiples of 4. */
int32_t mh_conv3x3_winograd(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                            const float *u, uint32_t c_out, const float *bias, uint32_t upsample2x,
                            const float *prologue_scale, const float *prologue_shift, uint32_t prologue_silu,
                            float *out);

/* src/engine/conv.rs:145-165 `Geometry::gather`: patch rows [3,3,c] of output
 * pixels first..first+count (the implicit-GEMM conv's A operand, materialised
 * for a bit-exact check). rows [count, 9*c]. */
int32_t mh_im2col_gather(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                         uint32_t stride, const uint32_t pad[4], uint32_t upsample2x, uint64_t first, uint64_t count,
                         float *rows);

/* src/engine/depthwise.rs:31-59 `depthwise3x3`: stride 1, zero pad 1.
 * weight [3,3,c], bias [c]; out [n,h,w,c] (c/2 channels for GLU_SILU). */
int32_t mh_depthwise3x3(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                        const float *weight, const float *bias, uint32_t epilogue, float *out);

/* depthwise3x3 reading GroupNorm's output without storing it
 * (src/unet/blocks.rs:89-90, 98-101: norm then DwConv2d): each in-image input
 * value becomes [SiLU](x . scale + shift) (scale/shift [n * c] from
 * mh_group_norm_affine) as it is loaded; the zero padding is not transformed. */
int32_t mh_depthwise3x3_fused(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                              const float *weight, const float *bias, uint32_t epilogue, const float *prologue_scale,
                              const float *prologue_shift, uint32_t prologue_silu, float *out);

/* src/engine/norm.rs:57-105 `GroupNorm::affine`: per item and channel
 * scale/shift ([n * c] each, device) with GN(x + add) = x.scale + shift.
 * add [n * c] or NULL. Statistics: f32 per-channel (sum, sum of squares) over
 * pixel chunks (64 pixels, doubled until at most 512 partial blocks remain),
 * folded per group in f64 in a fixed order. */
int32_t mh_group_norm_affine(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                             uint32_t groups, float eps, const float *gamma, const float *beta, const float *add,
                             float *scale, float *shift);

/* mh_group_norm_affine from the partials of mh_conv1x1_gn_partials (rows from
 * there; no counterpart in the reference, see above): the same f64 fold per
 * (item, group) and scale/shift, add folded per partial as GN(x + add). */
int32_t mh_group_norm_affine_partials(MhContext *ctx, const float *part, uint32_t rows, uint32_t n, uint32_t h,
                                      uint32_t w, uint32_t c, uint32_t groups, float eps, const float *gamma,
                                      const float *beta, const float *add, float *scale, float *shift);

/* src/engine/norm.rs:41-53 `GroupNorm::forward`: out = [SiLU](GN(x + add)). */
int32_t mh_group_norm_forward(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                              uint32_t groups, float eps, const float *gamma, const float *beta, const float *add,
                              uint32_t silu, float *out);

/* No counterpart in the reference: mh_group_norm_forward for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and result bits; its
 * statistics partials and scale/shift live in a fixed 1 MiB device array per
 * GPU (262144 floats, held until the process ends) instead of the context
 * workspace, so it calls no hipMalloc/hipFree. Shapes whose scratch exceeds the
 * array (partials plus 2 * n * c floats; e.g. n * c > 65536 on maps of a few
 * pixels) return MH_ERR_INVALID_ARGUMENT. Every call on a GPU shares that GPU's
 * array, which keeps the last call's contents. Calls from different contexts'
 * streams are ordered on the device (a call waits for an event the previous
 * call recorded, so they do not overlap); calls captured into HIP graphs are
 * not, and graphs that use it and run concurrently on one GPU race. */
int32_t mh_group_norm_forward_noalloc(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w,
                                      uint32_t c, uint32_t groups, float eps, const float *gamma, const float *beta,
                                      const float *add, uint32_t silu, float *out);

/* src/engine/norm.rs:132-148 `apply_affine` over n items: out = [SiLU](x.scale + shift). */
int32_t mh_apply_affine(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                        const float *scale, const float *shift, uint32_t silu, float *out);

/* src/engine/norm.rs:151-173 `layer_norm` over the channel axis of rows tokens. */
int32_t mh_layer_norm(MhContext *ctx, const float *x, uint64_t rows, uint32_t c, const float *gamma,
                      const float *beta, float eps, float *out);

/* layer_norm followed by Conv1x1::forward, as a transformer block runs them
 * (src/unet/transformer.rs:100-126 with src/engine/norm.rs:151-173 and
 * src/engine/conv.rs:38-55), in one GEMM: out [rows][c_out] = [SiLU](LayerNorm(x)
 * . W^T + bias) (silu 1: the inverted 1x1's SiLU), with the LayerNorm folded into
 * the product as rstd . (x . (W . diag gamma)^T - mean . rowsum) + W . beta +
 * bias, so LayerNorm(x) is never written. The folded weights are built in the
 * context's workspace on each call (the UNet builds them once at load). c_in and
 * c_out multiples of 4; x and out 16-byte aligned; FAST contexts multiply on the
 * f16 rounding of the folded weights. */
int32_t mh_conv1x1_layer_norm(MhContext *ctx, const float *x, uint64_t rows, uint32_t c_in, const float *gamma,
                              const float *beta, float eps, const void *weight, uint32_t weight_dtype, uint32_t c_out,
                              const float *bias, uint32_t silu, float *out);

/* mh_conv1x1_layer_norm with each row's mean and variance from partial sums
 * written by the producer of x (src/engine/norm.rs:151-173's statistics, summed
 * in a different order): row_partials [rows][per_row][2] = (sum, sum of
 * squares) over disjoint column ranges covering the row, as
 * mh_conv1x1_row_partials and mh_cross_lambda_row_sums write them; summed in
 * order in f64. 8-byte aligned; per_row 1..4096. */
int32_t mh_conv1x1_layer_norm_stats(MhContext *ctx, const float *x, uint64_t rows, uint32_t c_in, const float *gamma,
                                    const float *beta, float eps, const void *weight, uint32_t weight_dtype,
                                    uint32_t c_out, const float *bias, uint32_t silu, const float *row_partials,
                                    uint32_t per_row, float *out);

/* src/engine/conv.rs:38-55 `Conv1x1::forward` (bias, no residual) whose
 * epilogue also writes the LayerNorm row partials of its output for the
 * LayerNorm that reads it next (the transformers' proj_in before LayerNorm 1,
 * src/unet/transformer.rs:97-99): row_partials [rows][*per_row][2], room for
 * rows * ceil(c_out / 32) pairs, 8-byte aligned. *per_row receives the number
 * written per row (0 where the tiling cannot write them: then out alone). */
int32_t mh_conv1x1_row_partials(MhContext *ctx, const float *x, uint64_t rows, uint32_t c_in, const void *weight,
                                uint32_t weight_dtype, uint32_t c_out, const float *bias, float *out,
                                float *row_partials, uint32_t *per_row);

/* src/engine/ops.rs:11-13 `silu_inplace` (in place). */
int32_t mh_silu_inplace(MhContext *ctx, float *x, uint64_t len);
/* src/engine/ops.rs:16-19 `add_inplace`: a += b (in place on a). */
int32_t mh_add_inplace(MhContext *ctx, float *a, const float *b, uint64_t len);

/* src/engine/tensor.rs:59-73 `concat_channels_into`: out[p] = [a[p] || b[p]]. */
int32_t mh_concat_channels(MhContext *ctx, const float *a, uint32_t ca, const float *b, uint32_t cb,
                           uint64_t pixels, float *out);

/* src/imaging/blend.rs:21-24 `to_u8`: (clamp(v,0,1)*255) truncated, NaN -> 0. */
int32_t mh_to_u8(MhContext *ctx, const float *x, uint64_t len, uint8_t *out);

/* src/engine/math.rs:17-36 on device: y = exp(x) (which=0) or SiLU(x) (which=1),
 * the reference's Cephes polynomial, for bit-exact checks of the device math. */
int32_t mh_math_eval(MhContext *ctx, uint32_t which, const float *x, uint64_t len, float *y);

/* src/unet/lambda.rs:322-359 `softmax_lambda` per item: keys [nb][rows][k]
 * (read only), v [nb][rows][vd] -> lambda_t [nb][vd][k], the TRANSPOSE of the
 * reference's lambda_c [k][vd]. k, vd <= 160. */
int32_t mh_softmax_lambda(MhContext *ctx, const float *keys, const float *v, uint32_t nb, uint32_t rows, uint32_t k,
                          uint32_t vd, float *lambda_t);

/* src/unet/lambda.rs:154-185 `tap_filter` over nb items of hh x ww pixels, per
 * pixel, head and value channel: u = (yc + A[225]) then + A[dy*15+dx] * v[pixel +
 * (dy-7, dx-7)] over the in-image taps in (dy, dx) order; out = u, or residual + u
 * when residual is given (the block's following `add_inplace`). a_t is the
 * reference's A [pixel][head][226] stored tap-major, [nb*hh*ww][226][8];
 * v [nb*hh*ww][vd]; yc, residual, out [nb*hh*ww][8*vd]; out may alias yc or residual. */
int32_t mh_tap_filter(MhContext *ctx, const float *a_t, const float *v, const float *yc, const float *residual,
                      float *out, uint32_t nb, uint32_t hh, uint32_t ww, uint32_t vd);

/* mh_tap_filter that also writes, per output row, (sum, sum of squares) of the
 * values written over *per_row disjoint slices of the row (row_sums
 * [nb * hh * ww][*per_row][2], room for nb * hh * ww * vd / 4 pairs, 8-byte
 * aligned): the statistics of LayerNorm 2, which reads the block's hidden state
 * next (src/unet/transformer.rs:101-103), for mh_conv1x1_layer_norm_stats. */
int32_t mh_tap_filter_row_sums(MhContext *ctx, const float *a_t, const float *v, const float *yc,
                               const float *residual, float *out, uint32_t nb, uint32_t hh, uint32_t ww, uint32_t vd,
                               float *row_sums, uint32_t *per_row);

/* mh_tap_filter followed by the transformer block's `layer_norm` of its output
 * rows (src/unet/transformer.rs:104-108, src/engine/norm.rs:151-173): the same
 * out, and ln_out [nb*hh*ww][8*vd] = LayerNorm(out) (gamma, beta [8*vd]), written
 * by the kernel that finishes each row. ln_out must not alias out, yc or residual. */
int32_t mh_tap_filter_ln(MhContext *ctx, const float *a_t, const float *v, const float *yc, const float *residual,
                         float *out, uint32_t nb, uint32_t hh, uint32_t ww, uint32_t vd, const float *gamma,
                         const float *beta, float eps, float *ln_out);

/* src/unet/lambda.rs:131-137, the position path's `matmul` A = Q . W_aug
 * over nb items of hw pixels: q [nb*hw][8][k] (a pixel's 8 head rows of k),
 * w_aug_t [226][k] (the reference's w_aug [k][226] transposed: tap d < 225 is
 * the position conv's weight, tap 225 its bias) -> a_t [nb*hw][226][8], the
 * layout mh_tap_filter takes. With lambda_t [nb][k][k] (mh_softmax_lambda's
 * output) also the content path's `matmul` yc = Q . lambda_c per item
 * (lambda.rs:123), yc [nb*hw][8][k]; lambda_t and yc are both NULL or both
 * given, and so are w_aug_t and a_t (both NULL: yc alone, as the cross-lambda's
 * content term Q . lambda_c[branch] with lambda_t pointing at the first item's
 * branch). k must be 40, 80 or 160 (the UNet's three levels); f32 products
 * on the matrix cores, summed in f32. */
int32_t mh_lambda_position_coeffs(MhContext *ctx, const float *q, const float *w_aug_t, const float *lambda_t,
                                  uint32_t nb, uint32_t hw, uint32_t k, float *a_t, float *yc);

/* src/unet/lambda.rs:123, 131-137 and 154-185 in one pass: mh_lambda_position_coeffs
 * (A and yc) followed by mh_tap_filter (vd = k) without writing A or yc, the
 * position coefficients and the content term being formed where the filter uses
 * them. q [nb*hh*ww][8][k], w_aug_t [226][k], lambda_t [nb][k][k], v [nb*hh*ww][k],
 * residual (optional) and out [nb*hh*ww][8*k]; out may alias residual, not q or v.
 * row_sums (optional, 8-byte aligned): one (sum, sum of squares) pair per out row,
 * as mh_tap_filter_row_sums writes with one part per row. k must be 40, 80 or 160.
 * out and row_sums are bit-identical to the two calls' with one thread per output
 * (the tuning key tap_split = 1). */
int32_t mh_self_lambda_fused(MhContext *ctx, const float *q, const float *w_aug_t, const float *lambda_t,
                             const float *v, const float *residual, float *out, uint32_t nb, uint32_t hh, uint32_t ww,
                             uint32_t k, float *row_sums);

/* src/unet/lambda.rs:276-295 `position_term`: u = yc + (q . E) . V[branch], per
 * element in the reference's order; out = u, or residual + u when residual is
 * given. e [hw][10][k], v_branches [2][10][k], item i using branch br0 + i;
 * q, yc, residual, out [nb*hw][8*k]; out may alias yc or residual. */
int32_t mh_position_term(MhContext *ctx, const float *q, const float *e, const float *v_branches, uint32_t br0,
                         uint32_t nb, uint32_t hw, uint32_t k, const float *yc, const float *residual, float *out);

/* src/unet/lambda.rs:258-271, the body of `CrossLambda::forward` after to_q, in
 * one pass: u = q . lambda_c[branch] (src/unet/lambda.rs:265) + (q . E) . V[branch]
 * (the position term as mh_position_term computes it); out = u, or residual + u.
 * lambda_c [2][k][k] row-major; e, v_branches, q, residual, out as for
 * mh_position_term. out may alias residual, not q. k a multiple of 8, <= 256. */
int32_t mh_cross_lambda(MhContext *ctx, const float *q, const float *e, const float *lambda_c, const float *v_branches,
                        uint32_t br0, uint32_t nb, uint32_t hw, uint32_t k, const float *residual, float *out);

/* mh_cross_lambda that also writes, per output row, the (sum, sum of squares)
 * of the values written (row_sums [nb * hw][2], 8-byte aligned): the
 * statistics of LayerNorm 3, which reads the block's hidden state next
 * (src/unet/transformer.rs:104-107), for mh_conv1x1_layer_norm_stats (per_row 1). */
int32_t mh_cross_lambda_row_sums(MhContext *ctx, const float *q, const float *e, const float *lambda_c,
                                 const float *v_branches, uint32_t br0, uint32_t nb, uint32_t hw, uint32_t k,
                                 const float *residual, float *out, float *row_sums);

/* src/engine/gemm.rs:63-132 `matmul` for K-contiguous operands, on the device:
 * c [m][ldc] = a [m][lda] . b[n][ldb]^T (+ bias[n]) (+ residual [m][ldc]); b F32/F16.
 * row_group g > 1 (m a multiple of g, g <= 64) stores row i, column j at
 * c[(i / g) * ldc + j * g + i % g] (residual read the same way), e.g. the
 * lambda layer's per-(pixel, head) rows as [pixel][tap][head]; 0 or 1: plain. */
int32_t mh_gemm_nt(MhContext *ctx, const float *a, uint64_t lda, const void *b, uint32_t b_dtype, uint64_t ldb,
                   uint32_t m, uint32_t n, uint32_t k, const float *bias, const float *residual, float *c,
                   uint64_t ldc, uint32_t row_group);

/* ---- UNet (src/unet) ---- */

/* src/unet/mod.rs:86-140 `UNet::load` from the converter tensors (copied to
 * HBM; the table may be freed afterwards). Precomputes the cross-lambda
 * constants and the folded self-lambda filter. MH_ERR_WEIGHTS names the first
 * missing or mis-sized tensor. */
int32_t mh_unet_create(MhContext *ctx, const MhNamedTensor *tensors, uint32_t count, MhUNet **out);
void mh_unet_destroy(MhUNet *unet);

/* src/unet/mod.rs:144-146 `UNet::forward`: x [1,64,64,9] (noisy latent | mask |
 * masked latent) -> eps [b,64,64,4], b = 2 for MH_GUIDANCE_CFG, 1 for
 * COND_ONLY. Device pointers; asynchronous on the context stream. */
int32_t mh_unet_forward(MhUNet *unet, const float *x_dev, uint32_t timestep, uint32_t guidance, float *eps_dev);

/* The same with host buffers (synchronous), as the reference's Tensor API. */
int32_t mh_unet_forward_host(MhUNet *unet, const float *x_host, uint32_t timestep, uint32_t guidance,
                             float *eps_host);

/* src/unet/mod.rs:150-157 `forward_traced`: trace(name, tensor) after every block. */
int32_t mh_unet_forward_traced(MhUNet *unet, const float *x_dev, uint32_t timestep, uint32_t guidance,
                               float *eps_dev, MhTraceFn trace, void *user);

/* HBM held by the weights and by the activation pool. */
int32_t mh_unet_memory(MhUNet *unet, uint64_t *weight_bytes, uint64_t *pool_bytes);

/* ---- weights from the converter's safetensors files (src/weights.rs) ---- */

#define MH_MODEL_UNET 0u
#define MH_MODEL_VAE 1u

/* src/weights.rs:40-96 on the host, no device needed: maps `path`, parses the
 * safetensors header, requires the "format" metadata "moebius-cpu/1" (and, for the
 * VAE, "scaling_factor" 0.13025: src/vae/mod.rs:88-93), and checks that every
 * tensor the model loads is present with its converted shape, stored F16 or F32.
 * MH_ERR_IO when the file cannot be read, MH_ERR_WEIGHTS otherwise. */
int32_t mh_weights_validate(const char *path, uint32_t model);
/* UNet::load / Vae::load (src/unet/mod.rs:86-140, src/vae/mod.rs:88-95) from
 * unet.safetensors / vae.safetensors: the file is validated as above, each tensor
 * copied to HBM in its stored precision, and the mapping closed again. */
int32_t mh_unet_create_from_file(MhContext *ctx, const char *path, MhUNet **out);
int32_t mh_vae_create_from_file(MhContext *ctx, const char *path, MhVae **out);

/* ---- pixel-space steps around the model window (src/imaging), on the host ---- */

#define MH_PASTE_NONE 1u               /* src/preset.rs Paste; MOEBIUS_PASTE_* values */
#define MH_PASTE_FEATHER 2u
#define MH_PASTE_FEATHER_COMPENSATE 3u

/* src/imaging/mod.rs:31-46: rect {x, y, w, h} of the pixels >= 128; *found 0 when none. */
int32_t mh_mask_bbox(const uint8_t *mask, uint32_t width, uint32_t height, uint32_t stride, uint32_t *rect,
                     uint32_t *found);
/* src/imaging/mod.rs:48-77: out [height * width] = 0 / 255 mask dilated by a k x k kernel (cv2 anchor). */
int32_t mh_mask_dilate(const uint8_t *mask, uint32_t width, uint32_t height, uint32_t stride, uint32_t k,
                       uint8_t *out);
/* src/imaging/crop.rs:27-51: the square window {x, y, side} for a mask bbox {x, y, w, h}. */
int32_t mh_crop_plan(const uint32_t *bbox, uint32_t img_w, uint32_t img_h, int64_t *x, int64_t *y, uint32_t *side);
/* src/imaging/blend.rs:91-110: Pillow GaussianBlur(radius) of an 8-bit single-channel image. */
int32_t mh_gaussian_blur(const uint8_t *src, uint32_t width, uint32_t height, float radius, uint8_t *out);
/* src/imaging/blend.rs:155-232: pastes result (side x side RGB) over the image inside the
 * window {plan_x, plan_y, side}; mode MH_PASTE_*; changed {x, y, w, h} may be NULL.
 * The blur and blend run on up to 16 host threads (the bytes do not depend on it). */
int32_t mh_paste(uint8_t *pixels, uint32_t width, uint32_t height, uint32_t stride, uint32_t channels,
                 const uint8_t *mask, uint32_t mask_stride, const uint8_t *result, int64_t plan_x, int64_t plan_y,
                 uint32_t side, uint32_t mode, uint32_t *changed);
/* src/imaging/resize.rs:15-24 `resize_u8` on the device: Lanczos3 resize of an 8-bit
 * image [from_h][from_w][channels] (1, 3 or 4) to [to_h][to_w][channels], device
 * pointers, PIL's LANCZOS convolution in 22-bit fixed point (horizontal pass first);
 * same size is a copy. Returns after the stream has finished the resize. */
int32_t mh_resize_u8(MhContext *ctx, const uint8_t *src, uint32_t from_w, uint32_t from_h, uint32_t to_w,
                     uint32_t to_h, uint32_t channels, uint8_t *dst);
/* src/vae/mod.rs:60-78: latent window {x, y, w, h} of a 64 x 64 mask, grown by margin. */
int32_t mh_roi_window(const float *mask_lat, uint32_t margin, uint32_t *rect, uint32_t *found);

/* ---- samplers and the denoise loop (src/scheduler.rs, src/pipeline.rs) ---- */

#define MH_SPACING_LEADING 0u  /* src/scheduler.rs:24-29 */
#define MH_SPACING_TRAILING 1u
#define MH_SOLVER_DDIM 0u      /* src/preset.rs: Solver */
#define MH_SOLVER_DPMPP_2M 1u

/* src/scheduler.rs:30-76 `Ddim::new(steps, strength, spacing).timesteps()`, on the
 * host: out (room for 1000) receives the timesteps denoised, *count their number,
 * *pure_noise 1 when the loop starts from noise alone (strength >= 1). */
int32_t mh_schedule_timesteps(uint32_t steps, double strength, uint32_t spacing, uint32_t *out, uint32_t *count,
                              uint32_t *pure_noise);
/* src/scheduler.rs:159-172, on the host: the 1000 f32 cumulative alpha products. */
int32_t mh_schedule_alphas_cumprod(float *out);

/* src/scheduler.rs `Ddim` + `Dpm2M` over device arrays of len floats. */
typedef struct MhScheduler MhScheduler;
int32_t mh_scheduler_create(MhContext *ctx, uint32_t steps, double strength, uint32_t spacing, uint64_t len,
                            MhScheduler **out);
void mh_scheduler_destroy(MhScheduler *s);
/* src/scheduler.rs:80-86: out = sqrt(at) x0 + sqrt(1 - at) noise. */
int32_t mh_scheduler_add_noise(MhScheduler *s, const float *x0, const float *noise, uint32_t t, float *out);
/* src/pipeline.rs:330-336 then src/scheduler.rs:88-97: eps = eps_c ? eps_u +
 * guidance (eps_c - eps_u) : eps_u; one DDIM step of x (in place) at timestep t. */
int32_t mh_scheduler_ddim_step(MhScheduler *s, const float *eps_u, const float *eps_c, float guidance, uint32_t t,
                               float *x);
/* The same combine, then src/scheduler.rs:123-156: one DPM-Solver++(2M) step of
 * x from timesteps[i] to the next timestep (first order after create/restart). */
int32_t mh_scheduler_dpm_step(MhScheduler *s, const float *eps_u, const float *eps_c, float guidance, uint32_t i,
                              float *x);
/* src/scheduler.rs:117-120 */
int32_t mh_scheduler_dpm_restart(MhScheduler *s);

/* The sampling fields of src/preset.rs:27-50 `InpaintParams`. */
typedef struct MhDenoiseParams {
    double strength;  /* 0.99 in both presets */
    float guidance;   /* CFG scale, 2.5 */
    uint32_t steps;   /* 1..1000 (Exact 20, Fast 10) */
    uint32_t spacing; /* MH_SPACING_* */
    uint32_t solver;  /* MH_SOLVER_* */
    int32_t cfg_steps; /* < 0: CFG on every step; n: the first n steps, then cond-only (Fast: 3) */
    uint32_t reserved; /* 0 */
} MhDenoiseParams;

/* Called on the caller's thread after each finished step; nonzero cancels. */
typedef int32_t (*MhStepFn)(void *user, uint32_t done, uint32_t total);

/* src/pipeline.rs:295-345 (steps 7-8) resident on the device. Device arrays:
 * z_img, init, z_masked, latents [1,64,64,4]; mask_lat [64 * 64]. x starts as init
 * (strength >= 1; z_img may then be NULL) or add_noise(z_img, init, t0); each step
 * runs the UNet on [x | mask | z_masked] (CFG batch 2 while CFG is on), combines
 * u + g (c - u) and updates x with the solver (DPM restarts where CFG stops);
 * progress(user, done, total) after each step. latents receives the final x.
 * Returns when done; MH_ERR_CANCELLED leaves latents untouched. */
int32_t mh_unet_denoise(MhUNet *unet, const float *z_img, const float *init, const float *mask_lat,
                        const float *z_masked, const MhDenoiseParams *params, MhStepFn progress, void *user,
                        float *latents);

/* ---- VAE (src/vae) ---- */

/* src/vae/mod.rs:88-103 `Vae::load` from the converter tensors of vae.safetensors
 * (diffusers AutoencoderKL names at the file root; 3x3 [o,3,3,i], 1x1 and linear
 * [o,i]), copied to HBM once. The scaling_factor metadata check stays with the host. */
int32_t mh_vae_create(MhContext *ctx, const MhNamedTensor *tensors, uint32_t count, MhVae **out);
/* Destroy every MhVae / MhUNet before the context they were created on. */
void mh_vae_destroy(MhVae *vae);

/* src/vae/mod.rs:105-109 `Vae::encode` (encoder.rs:77-118), device buffers:
 * images [b,h,w,3] in [-1,1] (h, w multiples of 8), noise [b,h/8,w/8,4] ~N(0,1)
 * -> z [b,h/8,w/8,4] = (mean + exp(0.5 clamp(logvar, -30, 20)) noise) 0.13025.
 * trace (may be NULL) gets vae.encoder.item<b>.{conv_in, down.<i>, mid, moments}. */
int32_t mh_vae_encode(MhVae *vae, const float *images_dev, uint32_t b, uint32_t h, uint32_t w,
                      const float *noise_dev, float *z_dev, MhTraceFn trace, void *user);

/* src/vae/mod.rs:111-115 `Vae::decode` (decoder.rs:74-99), device buffers:
 * latents [1,h,w,4] (scaled) -> out [1,8h,8w,3] = (dec(latents / 0.13025) + 1) / 2,
 * unclamped. trace (may be NULL) gets vae.decoder.{conv_in, mid, up.<i>}. */
int32_t mh_vae_decode(MhVae *vae, const float *latents_dev, uint32_t h, uint32_t w, float *out_dev,
                      MhTraceFn trace, void *user);

/* The same on host buffers (synchronous), as the pipeline calls them
 * (src/pipeline.rs:259,266,286,358-366). */
int32_t mh_vae_encode_host(MhVae *vae, const float *images, uint32_t b, uint32_t h, uint32_t w, const float *noise,
                           float *z);
int32_t mh_vae_decode_host(MhVae *vae, const float *latents, uint32_t h, uint32_t w, float *out);

int32_t mh_vae_memory(MhVae *vae, uint64_t *weight_bytes, uint64_t *pool_bytes);

/* src/vae/mod.rs:275-294 `softmax_rows`, in place on device rows [nrows][n]
 * (n <= 15360, scale > 0): per row max, exp((v - max) scale) with values below
 * exp(-40) flushed to 0, summed in row order, times (f32)(1 / sum). */
int32_t mh_softmax_rows(MhContext *ctx, float *rows, uint64_t nrows, uint32_t n, float scale);

/* src/vae/encoder.rs:121-133 `sample`: moments [pixels][8] = mean(4) | logvar(4),
 * noise [pixels][4] -> z [pixels][4]. */
int32_t mh_vae_sample(MhContext *ctx, const float *moments, const float *noise, uint64_t pixels, float *z);

/* src/unet/embed.rs:21-30 `timestep_sinusoid` (host arithmetic, f32 libm). */
void mh_timestep_sinusoid(uint32_t t, float *out /* [320] */);

/* src/engine/mod.rs:104-117 `best_fit`: the pool's buffer choice among (len, cap)
 * pairs for a request of `len` elements; -1 when count is 0. Host only. */
int64_t mh_scratch_best_fit(const uint64_t *lens, const uint64_t *caps, uint64_t count, uint64_t len);

/* Lane-layout probe of the f32 matrix instruction the convs use (no
 * counterpart in the reference): d[32][32] = a[32][2] . b[2][32] through one
 * v_mfma_f32_32x32x2f32, all operands host memory. */
int32_t mh_selftest_mfma_f32(MhContext *ctx, const float *a, const float *b, float *d);

/* Device allocations (hipMalloc calls) this library has made since it was
 * loaded, over every context, engine and entry point (no counterpart in the
 * reference): a caller that wants to show that a call allocates nothing reads
 * it before and after. Host only; never fails for a non-NULL count. */
int32_t mh_device_allocations(uint64_t *count);

#ifdef __cplusplus
}
#endif

#endif /* MOEBIUS_HIP_H */
