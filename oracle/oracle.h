/*
 * CPU oracle: a C++ restatement of moebius-cpu's `src/engine` kernels and the
 * `src/unet` / `src/vae` block chains that call them.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path and
 * the CPU baseline of the benchmark. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library never links it
 * and has no CPU fallback.
 *
 * Every function states the reference file:line it follows (paths relative to
 * the moebius-cpu source tree). Arithmetic order follows the reference where it
 * is specified by the source (Winograd transforms, GroupNorm partial/fold order,
 * depthwise tap order, Cephes exp); the GEMM's internal summation order is that
 * of the third-party `gemm` / `private-gemm-x86` crates in the reference and is
 * pinned to tolerance only.
 *
 * Conventions: activations NHWC f32, contiguous. Weights in the converter
 * layouts (tools/convert_weights.py:25-28): 1x1 [c_out, c_in], dense 3x3
 * [c_out, 3, 3, c_in], depthwise [3, 3, c]. All pointers are host memory.
 * Outputs must not alias inputs (src/engine/tensor.rs:58).
 */
#ifndef MOEBIUS_ORACLE_H
#define MOEBIUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/engine/math.rs:17-36 */
float orc_exp(float x);
float orc_silu(float x);

/* src/engine/gemm.rs:63-132 semantics: c[m x n] (+)= a . b, with element
 * (i, p) of a at a[i*a_rs + p*a_cs] and (p, j) of b at b[p*b_rs + j*b_cs];
 * c dense row-major with leading dimension n. */
void orc_matmul(float *c, const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                int64_t b_cs, int64_t m, int64_t k, int64_t n, int accumulate);

/* src/engine/conv.rs:170-191; returns 1 if the GEMM must accumulate. */
int orc_init_output(float *out, int64_t rows, int64_t cols, const float *bias, const float *residual);

/* src/engine/conv.rs:38-55 */
void orc_conv1x1(const float *x, int64_t pixels, int64_t c_in, const float *weight, int64_t c_out,
                 const float *bias, const float *residual, float *out);

/* src/engine/conv.rs:77-81 */
void orc_conv3x3_output_hw(int64_t h, int64_t w, int stride, const int pad[4], int upsample2x,
                           int64_t *ho, int64_t *wo);

/* src/engine/conv.rs:92-102: stride 1 / pad 1 -> Winograd, else im2col.
 * prologue_scale/shift: [n * c_in] or NULL (src/engine/norm.rs:33-37). */
void orc_conv3x3_forward(const float *x, int64_t n, int64_t h, int64_t w, int64_t c_in, const float *weight,
                         int64_t c_out, const float *bias, int stride, const int pad[4], int upsample2x,
                         const float *prologue_scale, const float *prologue_shift, int prologue_silu, float *out);

/* src/engine/conv.rs:106-130, 145-165 */
void orc_conv3x3_im2col(const float *x, int64_t n, int64_t h, int64_t w, int64_t c_in, const float *weight,
                        int64_t c_out, const float *bias, int stride, const int pad[4], int upsample2x, float *out);

/* src/engine/conv.rs:145-165: one patch row [3,3,c] of output pixel p. */
void orc_im2col_gather_row(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, int64_t ho, int64_t wo,
                           int stride, int pad_top, int pad_left, int upsample2x, int64_t p, float *row);

/* src/engine/winograd.rs:48-120 */
void orc_winograd_conv3x3_same(const float *x, int64_t n, int64_t h, int64_t w, int64_t c_in,
                               const float *prologue_scale, const float *prologue_shift, int prologue_silu,
                               int upsample2x, const float *weight, const float *bias, int64_t c_out, float *out);

/* src/engine/winograd.rs:269-352 transforms, per channel vector of length c. */
void orc_wino_kernel_transform(const float *g, int64_t c, float *u);
void orc_wino_input_transform(const float *const d[16], int64_t c, float *v);
void orc_wino_output_transform(const float *const m[16], const float *bias, int64_t c, float *y);

/* src/engine/depthwise.rs:31-59; epilogue 0 none, 1 relu, 2 glu*silu. */
void orc_depthwise3x3(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, const float *weight,
                      const float *bias, int epilogue, float *out);

/* src/engine/norm.rs:57-105 (GroupNorm::affine); add: [n * c] or NULL. */
void orc_group_norm_affine(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, int64_t groups, float eps,
                           const float *gamma, const float *beta, const float *add, float *scale, float *shift);

/* src/engine/norm.rs:41-53 (GroupNorm::forward) */
void orc_group_norm_forward(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, int64_t groups, float eps,
                            const float *gamma, const float *beta, const float *add, int silu, float *out);

/* src/engine/norm.rs:132-148: per item (hw pixels), scale/shift [c]. */
void orc_apply_affine(const float *src, int64_t pixels, int64_t c, const float *scale, const float *shift, int silu,
                      float *dst);

/* src/engine/norm.rs:151-173 */
void orc_layer_norm(const float *x, int64_t rows, int64_t c, const float *gamma, const float *beta, float eps,
                    float *out);

/* src/engine/ops.rs:11-19 */
void orc_silu_inplace(float *x, int64_t len);
void orc_add_inplace(float *a, const float *b, int64_t len);

/* src/engine/tensor.rs:59-73 */
void orc_concat_channels(const float *a, int64_t ca, const float *b, int64_t cb, int64_t pixels, float *out);

/* src/imaging/blend.rs:21-24 */
void orc_to_u8(const float *x, int64_t len, uint8_t *out);

/* src/imaging/resize.rs:15-24: Lanczos3 (PIL LANCZOS) resize of an 8-bit image
 * [from_h][from_w][channels] to [to_h][to_w][channels]; same size is a copy. */
void orc_resize_u8(const uint8_t *src, int from_w, int from_h, int to_w, int to_h, int channels, uint8_t *dst);

/* OpenMP threads the oracle uses (0 = runtime default). */
void orc_set_threads(int threads);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif

#endif
