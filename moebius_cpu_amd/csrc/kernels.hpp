// Host-side C++ engine API over the gfx950 kernels: one function per
// moebius-cpu `src/engine` entry point (same argument meaning), used by the C
// ABI (capi.cpp) and by the UNet / VAE block chains. All calls are
// asynchronous on ctx.stream; shapes are validated here with the reference's
// assertion texts and raise mh::Error.
#pragma once

#include <cstdint>

#include "common.hpp"

namespace mh {

enum WeightType : uint32_t { kF32 = 0, kF16 = 1 };

// Epilogues the GEMM-shaped kernels can fuse after `acc + bias (+ residual)`.
enum class GemmEpilogue : int { None = 0, Silu = 1 };

// GroupNorm affine handed to a consumer (src/engine/norm.rs:33-37): per item
// and channel scale/shift, device arrays [n * c].
struct Affine {
    const float *scale = nullptr;
    const float *shift = nullptr;
    bool silu = false;
};

// ---- elementwise (elementwise.hip) ----
void bias_residual_add(Context &ctx, const float *x, int64_t rows, int cols, const float *bias,
                       const float *residual, float *out);
void silu_inplace(Context &ctx, float *x, int64_t len);
// dst [n][item] = SiLU(src [item]), n copies.
void silu_tile(Context &ctx, const float *src, int64_t item, int n, float *dst);
void add_inplace(Context &ctx, float *a, const float *b, int64_t len);
void concat_channels(Context &ctx, const float *a, int ca, const float *b, int cb, int64_t pixels, float *out);
void to_u8(Context &ctx, const float *x, int64_t len, uint8_t *out);
// f16 [len] -> f32 [len], exact.
void widen_f16(Context &ctx, const void *src, int64_t len, float *dst);
// f32 [len] -> f16 [len], nearest even, saturated at +-65504 (the f16 GEMM's operand rounding).
void round_f16(Context &ctx, const float *src, int64_t len, void *dst);
void math_eval(Context &ctx, int which, const float *x, int64_t len, float *y);
// dst [n][item] = src [item]: one item repeated over a batch.
void tile_items(Context &ctx, const float *src, int64_t item, int n, float *dst);

// ---- normalisation (norm.hip) ----
// add (optional): per item and channel, item b's row at add + b * add_ld (add_ld 0: c).
// x2 (optional): the input is [x | x2] per pixel, x holding the first c - c2
// channels (a multiple of 64) and x2 the last c2.
void group_norm_affine(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                       const float *gamma, const float *beta, const float *add, float *scale, float *shift,
                       int64_t add_ld = 0, const float *x2 = nullptr, int c2 = 0);
void apply_affine(Context &ctx, const float *x, int n, int h, int w, int c, const float *scale, const float *shift,
                  bool silu, float *out);
void group_norm_forward(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                        const float *gamma, const float *beta, const float *add, bool silu, float *out,
                        int64_t add_ld = 0);
void layer_norm(Context &ctx, const float *x, int64_t rows, int c, const float *gamma, const float *beta, float eps,
                float *out);
// group_norm_forward (no add row stride) with its scratch in a fixed per-device
// array instead of the context workspace: no device allocation. Shapes whose
// scratch exceeds group_norm_noalloc_max_floats() are rejected. Calls that
// overlap on one GPU share the array and race.
void group_norm_forward_noalloc(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                                const float *gamma, const float *beta, const float *add, bool silu, float *out);
int64_t group_norm_noalloc_max_floats();
// Takes the no-allocation scratch's device address for `device` (current), once.
void noalloc_scratch_setup(int device);
// GroupNorm statistics partials written by a producer's epilogue for the
// GroupNorm that follows it: part [pixels / rows][c][2] = per tile of `rows`
// pixels (inside one item of item_rows pixels) and channel, (sum y, sum y*y)
// over the values written. The caller sets part (room for pixels / 32 tiles)
// and item_rows; the producer sets rows (0: it wrote none).
struct GnPartials {
    float *part = nullptr;
    int item_rows = 0;
    int rows = 0;
};
// group_norm_affine from producer partials (rows > 0) of x alone; add, when
// given, is folded in here (per partial, in f64) as it would be for x + add.
void group_norm_affine_partials(Context &ctx, const float *part, int rows, int n, int hw, int c, int groups,
                                float eps, const float *gamma, const float *beta, const float *add, float *scale,
                                float *shift, int64_t add_ld = 0);
// Per-row (mean, rstd) of LayerNorm for consumers that apply it themselves: stats [rows][2].
void layer_norm_stats(Context &ctx, const float *x, int64_t rows, int c, float eps, float *stats);

// ---- resampling (resize.hip) ----
// Lanczos3 resize of an 8-bit image [from_h][from_w][channels] to [to_h][to_w][channels]
// (PIL's LANCZOS formulation: separable 22-bit fixed-point passes, horizontal first);
// same size is a copy. Device pointers; uses the workspace; synchronises the stream.
void resize_u8(Context &ctx, const uint8_t *src, int from_w, int from_h, int to_w, int to_h, int channels,
               uint8_t *dst);

// ---- depthwise (depthwise.hip) ----
// prologue (optional): GroupNorm affine [+SiLU] applied to in-image inputs as they load.
// x2 (optional): the input is [x | x2] per pixel, x holding the first c - c2
// channels (a multiple of 16) and x2 the last c2 (epilogue NONE or RELU).
void depthwise3x3(Context &ctx, const float *x, int n, int h, int w, int c, const float *weight, const float *bias,
                  int epilogue, float *out, const Affine *prologue = nullptr, const float *x2 = nullptr,
                  int c2 = 0);
// depthwise3x3 writing out16 in f16 (nearest even, saturated: the f16 GEMM's operand
// rounding), for FAST contexts whose only reader of the output is an f16 GEMM. False
// (nothing launched) where the tiled kernel does not take the shape or alignment.
bool depthwise3x3_h16(Context &ctx, const float *x, int n, int h, int w, int c, const float *weight,
                      const float *bias, int epilogue, void *out16, const Affine *prologue = nullptr,
                      const float *x2 = nullptr, int c2 = 0);

// ---- GEMM-shaped convs (gemm.hip) ----
// Per item and channel transform of a GEMM residual: res' = [SiLU](res . scale + shift),
// item = row / rows_per_item (a GroupNorm affine applied to the block input on the fly).
struct ResidualAffine {
    const float *scale = nullptr, *shift = nullptr;
    bool silu = false;
    int rows_per_item = 0;
};
// out = ([res'] + bias) + x' . W^T [SiLU] (+ residual2); gn (optional): GroupNorm partials of out.
// x_aff (optional): x' = [SiLU](x . scale + shift) per item (pixel / rows_per_item) and
// channel, applied as x loads (a GroupNorm's output without it being written); else x' = x.
// x2 (optional): the input is [x | x2] per pixel, x holding the first
// c_in - c2 channels (a multiple of 64) and x2 the last c2, read from the two
// buffers in place of their concatenation (not with x_aff).
// LayerNorm row statistics a producer writes for the LayerNorm that reads its
// output next: part [pixels][per_row] = per row, (sum y, sum y*y) over
// per_row disjoint column ranges of the values written. The caller sets part
// (room for pixels * ceil(c / 32) pairs); the producer sets per_row (0: none
// written).
struct LnRowPartials {
    float2 *part = nullptr;
    int per_row = 0;
};
void conv1x1(Context &ctx, const float *x, int64_t pixels, int c_in, const void *weight, WeightType wt, int c_out,
             const float *bias, const float *residual, float *out, GemmEpilogue epi = GemmEpilogue::None,
             const ResidualAffine *raff = nullptr, const float *residual2 = nullptr, GnPartials *gn = nullptr,
             const ResidualAffine *x_aff = nullptr, const float *x2 = nullptr, int c2 = 0,
             LnRowPartials *lnp = nullptr);
// conv1x1 for FAST contexts whose input is already f16 ([pixels][c_in] halves, e.g.
// from depthwise3x3_h16) and whose weight is f16: the products of the f16 GEMM on f32
// input it rounds itself, with the same epilogue (bias, residual and its transform,
// residual2, GroupNorm partials). out16: out holds halves, each output rounded as the
// f16 GEMM rounds an f32 operand (for an output that only another f16 GEMM reads).
void conv1x1_a16(Context &ctx, const void *x16, int64_t pixels, int c_in, const void *weight, int c_out,
                 const float *bias, const float *residual, float *out, const ResidualAffine *raff = nullptr,
                 const float *residual2 = nullptr, GnPartials *gn = nullptr, bool out16 = false);
// residual2 (optional, [n, ho, wo, c_out]) is added last: out = (bias + conv) + residual2.
void conv3x3(Context &ctx, const float *x, int n, int h, int w, int c_in, const void *weight, WeightType wt,
             int c_out, const float *bias, int stride, const int pad[4], bool upsample2x, const Affine *prologue,
             float *out, const float *residual2 = nullptr);
void conv3x3_output_hw(int h, int w, int stride, const int pad[4], bool upsample2x, int *ho, int *wo);
// One 1x1 conv over concatenated weights [sum widths][c_in] (bias [sum widths] or NULL)
// whose output columns land in nseg (<= 3) separate [pixels][widths[i]] buffers.
void conv1x1_segments(Context &ctx, const float *x, int64_t pixels, int c_in, const void *weight, WeightType wt,
                      const float *bias, int nseg, const int *widths, float *const *outs);
// LayerNorm folded into a 1x1 conv (LayerNorm 1 -> q | k | v and LayerNorm 3 ->
// MixFFN inverted, src/unet/transformer.rs:100-126): out = LayerNorm(x) . W^T + b,
// computed as rstd . (x . W'^T - mean . c1) + c2 with W' = W . diag(gamma),
// c1 = the row sums of W' as the kernel multiplies them, c2 = W . beta + b
// (ln_fold_weights); the row statistics come from the x values the GEMM loads.
// EXACT reads w32 / c1_32, FAST the f16 rounding w16 / c1_16. Output columns in
// nseg (<= 3) separate buffers of widths[i] columns (multiples of 4).
struct LnFolded {
    const float *w32 = nullptr, *c1_32 = nullptr;
    const void *w16 = nullptr;
    const float *c1_16 = nullptr;
    const float *c2 = nullptr;
    float eps = 1e-5f;
};
// stats (optional, per_row > 0): each row's statistics from its producer's
// partials instead of from the values this GEMM loads.
void conv1x1_ln(Context &ctx, const float *x, int64_t pixels, int c_in, const LnFolded &f, int nseg, const int *widths,
                float *const *outs, GemmEpilogue epi = GemmEpilogue::None, const LnRowPartials *stats = nullptr);
// Builds LnFolded's tensors on the device from W [n][k] (f32 or f16), gamma,
// beta [k] and bias [n] (or NULL): w32 [n][k] = W . gamma (f32), w16 its
// round-to-nearest f16 copy, c1_32 / c1_16 their row sums and c2 = W . beta +
// bias, summed in f64 in a fixed order.
void ln_fold_weights(Context &ctx, const void *w, WeightType wt, int n, int k, const float *gamma, const float *beta,
                     const float *bias, float *w32, void *w16, float *c1_32, float *c1_16, float *c2);
// C[z] = A[z] . B[z]^T (+ bias) (+ residual[z]) [SiLU] for z < batch, all K-contiguous:
// A [m][lda], B [n][ldb], C [m][ldc]; *_bs are per-item element offsets.
// row_group g > 1 stores row m, column n at (m / g) * ldc + n * g + m % g.
void gemm_nt(Context &ctx, const float *a, int64_t lda, int64_t a_bs, const void *b, WeightType wt, int64_t ldb,
             int64_t b_bs, int m, int n, int k, int batch, const float *bias, const float *residual, float *out,
             int64_t ldc, int64_t c_bs, GemmEpilogue epi = GemmEpilogue::None, int row_group = 0);
// gemm_nt without bias or residual for FAST contexts whose A is already f16 ([m][lda]
// halves, a_bs in halves) and whose B is f16: the products the f16 GEMM takes of f32
// operands it rounds itself.
void gemm_nt_a16(Context &ctx, const void *a, int64_t lda, int64_t a_bs, const void *b, int64_t ldb, int64_t b_bs,
                 int m, int n, int k, int batch, float *out, int64_t ldc, int64_t c_bs);
void im2col_gather(Context &ctx, const float *x, int n, int h, int w, int c, int stride, const int pad[4],
                   bool upsample2x, int64_t first, int64_t count, float *rows);

// ---- Winograd F(2x2,3x3) stride-1 / pad-1 conv (winograd.hip), src/engine/winograd.rs
// Tiles of a (upsampled) n x h x w map: n * ceil(H/2) * ceil(W/2), ordered (item, row, column).
int64_t winograd_tiles(int n, int h, int w, bool upsample2x);
// weight [c_out][3][3][c_in] (f32 or f16) -> u [16][c_out][c_in] f32 (G g G^T).
void winograd_weight_transform(Context &ctx, const void *weight, WeightType wt, int c_out, int c_in, float *u);
// x [n,h,w,c] -> v [16][tiles][c] (B^T d B), prologue applied to in-image values;
// h16: v in f16, rounded to nearest even and saturated as the f16 GEMM rounds operands.
void winograd_input_transform(Context &ctx, const float *x, int n, int h, int w, int c, bool upsample2x,
                              const Affine *prologue, void *v, bool h16 = false);
// m [16][tiles][c_out] -> out [n, H, W, c_out] = A^T m A + bias (+ residual2).
void winograd_output_transform(Context &ctx, const float *m, int n, int h, int w, int c_out, bool upsample2x,
                               const float *bias, const float *residual2, float *out);
// u [16][c_out][c_in] -> uf [16][c_in / 8][c_out][8], the fused kernel's operand order.
void winograd_fused_weights(Context &ctx, const float *u, int c_out, int c_in, float *uf);
// Direct 3x3 conv, stride 1 / pad 1, for c_out <= 8 on maps of at least 65536
// pixels (conv_small.hip), with the optional GN(+SiLU) prologue; false (nothing
// launched) where it does not apply.
bool conv3x3_small_co(Context &ctx, const float *x, int n, int h, int w, int c_in, const void *weight, WeightType wt,
                      int c_out, const float *bias, const Affine *prologue, float *out, const float *residual2);
// The whole conv in one kernel (winograd_fused.hip) for f32 u, c_in % 32 == 0,
// c_out % 64 == 0 and operands under 2 GiB; false (nothing launched) otherwise.
// uf: u in the fused order, or NULL (then made in the workspace for this call).
// gn (optional): GroupNorm partials of out, blocks of 128 pixels (gn->rows set,
// 0 where not written: odd output sizes, tiles per item not a multiple of 32).
bool conv3x3_winograd_fused(Context &ctx, const float *x, int n, int h, int w, int c_in, const float *u,
                            const float *uf, int c_out, const float *bias, bool upsample2x, const Affine *prologue,
                            float *out, const float *residual2, GnPartials *gn = nullptr);
// The whole conv: u from winograd_weight_transform (ut kF32) or an f16 copy of it;
// uf (optional) its fused-order copy for the one-kernel path; gn as above (only
// the one-kernel path writes partials).
void conv3x3_winograd(Context &ctx, const float *x, int n, int h, int w, int c_in, const void *u, WeightType ut,
                      int c_out, const float *bias, bool upsample2x, const Affine *prologue, float *out,
                      const float *residual2 = nullptr, const float *uf = nullptr, GnPartials *gn = nullptr);
void selftest_mfma_f32(Context &ctx, const float *a_host, const float *b_host, float *d_host);

// ---- lambda layers (lambda.hip), src/unet/lambda.rs
// keys [nb][rows][k], v [nb][rows][vd] -> lambda_t [nb][vd][k] (transposed lambda_c).
void softmax_lambda(Context &ctx, const float *keys, const float *v, int nb, int rows, int k, int vd,
                    float *lambda_t);
// LayerNorm of a kernel's output rows written beside them (src/engine/norm.rs:151-173):
// out [rows][c] = (y - mean) * rstd * gamma + beta.
struct LayerNormOut {
    const float *gamma = nullptr, *beta = nullptr;
    float eps = 0.f;
    float *out = nullptr;
};
// out [nb*hh*ww][8*vd] = (residual +) (yc + bias tap + 15x15 taps of v); a_t [nb*hh*ww][226][8]
// (heads innermost). out may alias yc or residual. lno (optional): also the LayerNorm
// of the out rows; or row_sums (optional): per out row, (sum, sum of
// squares) of the values written, for a consumer that folds the LayerNorm; the
// kernel may write several partials per row (tap_filter_row_parts, each over a
// slice of the value channels): row_sums [nb*hh*ww][row parts].
void tap_filter(Context &ctx, const float *a_t, const float *v, const float *yc, const float *residual, float *out,
                int nb, int hh, int ww, int vd, const LayerNormOut *lno = nullptr, float2 *row_sums = nullptr);
int tap_filter_row_parts(const Context &ctx, int hh, int ww, int vd);
// Position coefficients A = Q . W_aug (src/unet/lambda.rs:131-137) on the matrix cores:
// q [nb*hw][8][k] (pixel, head rows of k), w_aug_t [226][k] -> a_t [nb*hw][226][8], the
// tap-major layout tap_filter reads; with lambda_t [nb][k][k] (softmax_lambda's
// transposed lambda_c) also the content term yc [nb*hw][8][k] = Q . lambda_c per item
// (lambda.rs:123); w_aug_t and a_t null: yc alone. k must pass lambda_taps_ok (40, 80, 160).
bool lambda_taps_ok(int k);
void lambda_taps(Context &ctx, const float *q, const float *w_aug_t, const float *lambda_t, int nb, int hw, int k,
                 float *a_t, float *yc);
// lambda_taps then tap_filter (vd = k, no LayerNorm output) in one kernel that
// never writes a_t or yc: out [nb*hh*ww][8*k] = (residual +) (Yc + bias tap + 15x15
// taps of v), bit-identical to the two calls with one thread per output; row_sums
// (optional): one (sum, sum of squares) pair per out row. self_lambda_fused_ok:
// the Tuning::tap_fused choice for head width k.
bool self_lambda_fused_ok(const Context &ctx, int k);
void self_lambda_fused(Context &ctx, const float *q, const float *w_aug_t, const float *lambda_t, const float *v,
                       const float *residual, float *out, int nb, int hh, int ww, int k, float2 *row_sums = nullptr);
// out [nb*hw][8*k] = (residual +) (yc + (q . E) . V[branch]); e [hw][10][k]; v_branches [2][10][k].
// out may alias yc or residual.
void position_term(Context &ctx, const float *q, const float *e, const float *v_branches, int br0, int nb, int hw,
                   int k, const float *yc, const float *residual, float *out);
// out [nb*hw][8*k] = (residual +) (q . lambda_c[branch] + (q . E) . V[branch]) in one pass;
// lambda_c [2][k][k] row-major. out may alias residual, not q. row_sums
// (optional, [nb*hw]): per output row, (sum, sum of squares) of the values
// written, for the LayerNorm that reads out next (one partial per row).
void cross_lambda(Context &ctx, const float *q, const float *e, const float *lambda_c, const float *v_branches, int br0,
                  int nb, int hw, int k, const float *residual, float *out, float2 *row_sums = nullptr);

// ---- VAE (vae_kernels.hip), src/vae
// In place over rows [nrows][n] (n <= 15360): softmax(scale * row) with
// probabilities below e^-40 flushed to zero (src/vae/mod.rs:275-294).
void softmax_rows(Context &ctx, float *rows, int64_t nrows, int n, float scale);
// out [cols][rows] = in [rows][cols] with row stride ld_in.
void transpose(Context &ctx, const float *in, int64_t ld_in, int rows, int cols, float *out);
// z [pixels][4] = posterior sample from moments [pixels][8] and noise [pixels][4].
void vae_sample(Context &ctx, const float *moments, const float *noise, int64_t pixels, float *z);
// which 0: y = x / 0.13025; 1: y = (x + 1) * 0.5.
void vae_rescale(Context &ctx, const float *x, int64_t len, int which, float *y);

}  // namespace mh
