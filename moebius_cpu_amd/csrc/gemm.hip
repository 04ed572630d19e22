// GEMM-shaped convolutions on gfx950 matrix cores (f32 MFMA, f32 accumulate).
//
//   1x1 conv  (src/engine/conv.rs:38-55):  out[P x Co] = x[P x Ci] . W[Co x Ci]^T
//   3x3 conv  (src/engine/conv.rs:83-165): implicit GEMM, M = output pixels,
//             N = Co, K = 9*Ci in the weight's [ky][kx][ci] order; the A tile
//             is gathered straight from the NHWC input (zero outside the image,
//             nearest-2x upsample as a >>1 of the source index, any stride and
//             [top,left,bottom,right] padding), optionally through the
//             GroupNorm affine (+SiLU) prologue of src/engine/norm.rs:33-37.
//
// Both operands are K-contiguous (NHWC activations; [Co][.. Ci] weights), so
// one "NT" kernel serves every shape. Tiles: BM x BN x 32 per 256-thread
// workgroup, four 64-wide waves in a 2x2 arrangement, each owning
// (BM/2) x (BN/2) of the output as 32x32 blocks of v_mfma_f32_32x32x2f32.
// Each lane reads a float4 along K from LDS for A and for B and issues four
// MFMAs, one per component: instruction t pairs lane-group g = lane/32 with
// k = kk + 4g + t, so one float4 read feeds four matrix instructions and the
// pairs cover kk..kk+7. The K order of the sum therefore differs from the
// CPU engine's (the reference uses Winograd for stride-1 convs); results
// agree to f32 rounding.
//
// Small grids (MI355X has 256 CUs) split K across workgroups; the partial
// tiles are summed in a fixed order by a reduction kernel that also applies
// bias / residual / SiLU, so results are deterministic run to run.
#include "gemm_h16.hpp"

namespace mh {
using namespace gemm;
namespace {

// Byte extent of a row-major [rows][ld] operand whose rows hold `cols` used elements.
uint32_t extent(int64_t rows, int64_t ld, int64_t cols, int esz) {
    const int64_t bytes = rows > 0 ? ((rows - 1) * ld + cols) * esz : 0;
    MH_REQUIRE(bytes < (int64_t(1) << 31), "GEMM operand above 2 GiB");
    return uint32_t(bytes);
}

// Context precision selects the kernel family: EXACT runs f32 matrix
// instructions, FAST the f16 ones (activations rounded to f16 as they load).
void run_dense(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch, bool vec) {
    if (ctx.precision == Precision::Fast) launch_dense_h16(ctx, p, wt, epi, batch, vec);
    else launch_dense(ctx, p, wt, epi, batch, vec);
}

void run_conv(Context &ctx, GemmArgs &p, WeightType wt, int mode, bool pro) {
    if (ctx.precision == Precision::Fast) launch_conv_h16(ctx, p, wt, mode, pro);
    else launch_conv(ctx, p, wt, mode, pro);
}

__global__ void im2col_gather_kernel(GemmArgs p, int64_t first, int64_t count, float *__restrict__ rows) {
    const int64_t K = p.K;
    const int64_t total = count * K;
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
        const int64_t i = e / K;
        const int k = int(e - i * K);
        const ConvRow r = conv_row(p, int(first + i));
        const int tap = k / p.ci, c = k - (k / p.ci) * p.ci;
        const int64_t off = conv_src(p, r, tap / 3, tap % 3);
        rows[e] = off >= 0 ? p.a[off + c] : 0.0f;
    }
}

__global__ void mfma_probe_kernel(const float *a, const float *b, float *d) {
    const int lane = threadIdx.x;
    floatx16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
    // a: [32][2] row-major; b: [2][32] row-major.
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[(lane & 31) * 2 + (lane >> 5)], b[(lane >> 5) * 32 + (lane & 31)],
                                               acc, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        d[row * 32 + (lane & 31)] = acc[v];
    }
}

}  // namespace

void conv1x1(Context &ctx, const float *x, int64_t pixels, int c_in, const void *weight, WeightType wt, int c_out,
             const float *bias, const float *residual, float *out, GemmEpilogue epi, const ResidualAffine *raff,
             const float *residual2, GnPartials *gn, const ResidualAffine *x_aff, const float *x2, int c2,
             LnRowPartials *lnp) {
    MH_REQUIRE(c_in > 0 && c_out > 0, "Conv1x1: empty channel axis");
    MH_REQUIRE(pixels < (int64_t(1) << 31), "Conv1x1: too many pixels");
    if (x2) {
        const int c1 = c_in - c2;
        MH_REQUIRE(c2 > 0 && c1 > 0 && c1 % 64 == 0 && c2 % 4 == 0 && !x_aff && aligned16(x) && aligned16(x2),
                   "Conv1x1 over two inputs: first part a multiple of 64 channels, second of 4, 16-byte aligned, "
                   "no input affine");
    }
    if (raff) {
        MH_REQUIRE(residual && raff->scale && raff->shift && raff->rows_per_item > 0,
                   "Conv1x1: residual transform needs the residual, scale, shift and rows per item");
    }
    if (pixels == 0) return;
    GemmArgs p{};
    p.a = x;
    p.lda = c_in - (x2 ? c2 : 0);
    p.M = int(pixels);
    p.N = c_out;
    p.K = c_in;
    p.b = weight;
    p.ldb = c_in;
    p.a_bytes = extent(pixels, int(p.lda), int(p.lda), 4);
    if (x2) {
        p.a2 = x2;
        p.lda2 = c2;
        p.ka = c_in - c2;
        p.a2_bytes = extent(pixels, c2, c2, 4);
    }
    p.b_bytes = extent(c_out, c_in, c_in, wt == kF16 ? 2 : 4);
    p.bias = bias;
    p.res = residual;
    p.out = out;
    p.ldc = c_out;
    if (raff) {
        p.rsc = raff->scale;
        p.rsh = raff->shift;
        p.rsilu = raff->silu ? 1 : 0;
        p.r_rows = raff->rows_per_item;
    }
    p.res2 = residual2;
    if (gn) {
        p.gnp = gn->part;
        p.gn_item_rows = gn->item_rows;
    }
    if (lnp) {
        MH_REQUIRE(lnp->part, "Conv1x1: LayerNorm row partials need their buffer");
        p.lnp_out = lnp->part;
    }
    if (x_aff) {
        MH_REQUIRE(x_aff->scale && x_aff->shift && x_aff->rows_per_item > 0,
                   "Conv1x1: input affine needs scale, shift and rows per item");
        MH_REQUIRE(c_in % 4 == 0 && aligned16(x) && aligned16(x_aff->scale) && aligned16(x_aff->shift) &&
                       (reinterpret_cast<uintptr_t>(weight) % (wt == kF16 ? 8 : 16)) == 0,
                   "Conv1x1: input affine needs 4-channel aligned rows");
        p.psc = x_aff->scale;
        p.psh = x_aff->shift;
        p.psilu = x_aff->silu ? 1 : 0;
        p.pro_rows = x_aff->rows_per_item;
        if (ctx.precision == Precision::Fast) launch_dense_pro_h16(ctx, p, wt, epi);
        else launch_dense_pro(ctx, p, wt, epi);
    } else if (c_in % 4 == 0 && aligned16(x)) {
        run_dense(ctx, p, wt, epi, 1, true);
    } else {
        run_dense(ctx, p, wt, epi, 1, false);
    }
    if (gn) gn->rows = p.gn_rows;
    if (lnp) lnp->per_row = p.lnp_out ? p.lnp_ld : 0;
}

void conv1x1_segments(Context &ctx, const float *x, int64_t pixels, int c_in, const void *weight, WeightType wt,
                      const float *bias, int nseg, const int *widths, float *const *outs) {
    MH_REQUIRE(nseg >= 1 && nseg <= kMaxSeg, "Conv1x1 segments: 1 to 3 outputs");
    MH_REQUIRE(pixels < (int64_t(1) << 31), "Conv1x1: too many pixels");
    if (pixels == 0) return;
    GemmArgs p{};
    p.a = x;
    p.lda = c_in;
    p.M = int(pixels);
    int n = 0;
    p.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        MH_REQUIRE(widths[i] > 0 && outs[i], "Conv1x1 segments: empty segment");
        p.seg_col[i] = n;
        p.seg_out[i] = outs[i];
        n += widths[i];
    }
    p.seg_col[nseg] = n;
    p.N = n;
    p.K = c_in;
    p.b = weight;
    p.ldb = c_in;
    p.a_bytes = extent(pixels, c_in, c_in, 4);
    p.b_bytes = extent(n, c_in, c_in, wt == kF16 ? 2 : 4);
    p.bias = bias;
    p.ldc = n;
    run_dense(ctx, p, wt, GemmEpilogue::None, 1, c_in % 4 == 0 && aligned16(x));
}

void conv1x1_ln(Context &ctx, const float *x, int64_t pixels, int c_in, const LnFolded &f, int nseg, const int *widths,
                float *const *outs, GemmEpilogue epi, const LnRowPartials *stats) {
    MH_REQUIRE(nseg >= 1 && nseg <= kMaxSeg, "Conv1x1 (LayerNorm): 1 to 3 outputs");
    MH_REQUIRE(pixels < (int64_t(1) << 31), "Conv1x1: too many pixels");
    MH_REQUIRE(c_in % 4 == 0 && aligned16(x) && f.w32 && f.c1_32 && f.w16 && f.c1_16 && f.c2 && aligned16(f.c2) &&
                   aligned16(f.c1_32) && aligned16(f.c1_16),
               "Conv1x1 (LayerNorm): 4-channel aligned rows and the folded tensors");
    if (pixels == 0) return;
    GemmArgs p{};
    p.a = x;
    p.lda = c_in;
    p.M = int(pixels);
    int n = 0;
    p.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        MH_REQUIRE(widths[i] > 0 && widths[i] % 4 == 0 && outs[i] && aligned16(outs[i]),
                   "Conv1x1 (LayerNorm): segments of whole, aligned column quads");
        p.seg_col[i] = n;
        p.seg_out[i] = outs[i];
        n += widths[i];
    }
    p.seg_col[nseg] = n;
    if (nseg == 1) {  // one plain output
        p.nseg = 0;
        p.out = outs[0];
    }
    p.N = n;
    p.K = c_in;
    p.ldb = c_in;
    p.a_bytes = extent(pixels, c_in, c_in, 4);
    p.bias = f.c2;
    p.ldc = n;
    p.ln_eps = f.eps;
    if (stats && stats->per_row > 0) {
        MH_REQUIRE(stats->part, "Conv1x1 (LayerNorm): row partials without their buffer");
        p.lnp_in = stats->part;
        p.lnp_n = stats->per_row;
    }
    if (ctx.precision == Precision::Fast) {
        p.b = f.w16;
        p.ln_c1 = f.c1_16;
        p.b_bytes = extent(n, c_in, c_in, 2);
        launch_dense_ln_h16(ctx, p, kF16, epi);
    } else {
        p.b = f.w32;
        p.ln_c1 = f.c1_32;
        p.b_bytes = extent(n, c_in, c_in, 4);
        launch_dense_ln(ctx, p, kF32, epi);
    }
}

void gemm_nt(Context &ctx, const float *a, int64_t lda, int64_t a_bs, const void *b, WeightType wt, int64_t ldb,
             int64_t b_bs, int m, int n, int k, int batch, const float *bias, const float *residual, float *out,
             int64_t ldc, int64_t c_bs, GemmEpilogue epi, int row_group) {
    MH_REQUIRE(m >= 0 && n > 0 && k > 0 && batch > 0, "gemm: bad shape");
    MH_REQUIRE(row_group >= 0 && (row_group <= 1 || m % row_group == 0), "gemm: rows not divisible by the row group");
    if (m == 0) return;
    GemmArgs p{};
    p.a = a;
    p.lda = lda;
    p.M = m;
    p.N = n;
    p.K = k;
    p.b = b;
    p.ldb = ldb;
    p.a_bytes = extent(m, lda, k, 4);
    p.b_bytes = extent(n, ldb, k, wt == kF16 ? 2 : 4);
    p.bias = bias;
    p.res = residual;
    p.out = out;
    p.ldc = ldc;
    p.a_bs = a_bs;
    p.b_bs = b_bs;
    p.c_bs = c_bs;
    p.rg = row_group;
    const bool vec = k % 4 == 0 && lda % 4 == 0 && aligned16(a) && (batch == 1 || a_bs % 4 == 0);
    if (vec)
        run_dense(ctx, p, wt, epi, batch, true);
    else
        run_dense(ctx, p, wt, epi, batch, false);
}

void gemm_nt_a16(Context &ctx, const void *a, int64_t lda, int64_t a_bs, const void *b, int64_t ldb, int64_t b_bs,
                 int m, int n, int k, int batch, float *out, int64_t ldc, int64_t c_bs) {
    MH_REQUIRE(ctx.precision == Precision::Fast, "gemm (f16 A): FAST contexts only");
    MH_REQUIRE(m >= 0 && n > 0 && k > 0 && batch > 0, "gemm (f16 A): bad shape");
    MH_REQUIRE(k % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0 && a_bs % 4 == 0 && b_bs % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(a) & 7) == 0 && (reinterpret_cast<uintptr_t>(b) & 7) == 0,
               "gemm (f16 A): rows of whole, 8-byte aligned 4-element chunks");
    if (m == 0) return;
    GemmArgs p{};
    p.a = static_cast<const float *>(a);  // halves: the A16 kernels read it as such
    p.lda = lda;
    p.M = m;
    p.N = n;
    p.K = k;
    p.b = b;
    p.ldb = ldb;
    p.a_bytes = extent(m, lda, k, 2);
    p.b_bytes = extent(n, ldb, k, 2);
    p.out = out;
    p.ldc = ldc;
    p.a_bs = a_bs;
    p.b_bs = b_bs;
    p.c_bs = c_bs;
    gemm::launch_dense_h16_a16(ctx, p, batch);
}

void conv1x1_a16(Context &ctx, const void *x16, int64_t pixels, int c_in, const void *weight, int c_out,
                 const float *bias, const float *residual, float *out, const ResidualAffine *raff,
                 const float *residual2, GnPartials *gn, bool out16) {
    if (gn) gn->rows = 0;
    MH_REQUIRE(ctx.precision == Precision::Fast, "Conv1x1 (f16 input): FAST contexts only");
    MH_REQUIRE(pixels < (int64_t(1) << 31), "Conv1x1: too many pixels");
    MH_REQUIRE(c_in % 4 == 0 && (reinterpret_cast<uintptr_t>(x16) & 7) == 0 &&
                   (reinterpret_cast<uintptr_t>(weight) & 7) == 0,
               "Conv1x1 (f16 input): rows of whole, 8-byte aligned 4-channel chunks");
    if (raff)
        MH_REQUIRE(residual && raff->scale && raff->shift && raff->rows_per_item > 0,
                   "Conv1x1: residual transform needs the residual, scale, shift and rows per item");
    if (pixels == 0) return;
    GemmArgs p{};
    p.a = static_cast<const float *>(x16);  // halves: the A16 kernels read it as such
    p.lda = c_in;
    p.M = int(pixels);
    p.N = c_out;
    p.K = c_in;
    p.b = weight;
    p.ldb = c_in;
    p.a_bytes = extent(pixels, c_in, c_in, 2);
    p.b_bytes = extent(c_out, c_in, c_in, 2);
    p.bias = bias;
    p.res = residual;
    p.out = out;
    p.ldc = c_out;
    if (raff) {
        p.rsc = raff->scale;
        p.rsh = raff->shift;
        p.rsilu = raff->silu ? 1 : 0;
        p.r_rows = raff->rows_per_item;
    }
    p.res2 = residual2;
    if (gn) {
        p.gnp = gn->part;
        p.gn_item_rows = gn->item_rows;
    }
    gemm::launch_dense_h16_a16(ctx, p, 1, out16);
    if (gn) gn->rows = p.gn_rows;
}

void conv3x3_output_hw(int h, int w, int stride, const int pad[4], bool upsample2x, int *ho, int *wo) {
    const int up = upsample2x ? 2 : 1;
    const int hh = h * up + pad[0] + pad[2] - 3, ww = w * up + pad[1] + pad[3] - 3;
    MH_REQUIRE(stride > 0 && hh >= 0 && ww >= 0, "Conv3x3: input smaller than the kernel");
    *ho = hh / stride + 1;
    *wo = ww / stride + 1;
}

void conv3x3(Context &ctx, const float *x, int n, int h, int w, int c_in, const void *weight, WeightType wt,
             int c_out, const float *bias, int stride, const int pad[4], bool upsample2x, const Affine *prologue,
             float *out, const float *residual2) {
    MH_REQUIRE(c_in > 0 && c_out > 0, "Conv3x3 input channels");
    if (prologue) {
        MH_REQUIRE(stride == 1 && pad[0] == 1 && pad[1] == 1 && pad[2] == 1 && pad[3] == 1,
                   "Conv3x3 prologue needs the stride-1 / pad-1 Winograd path");
    }
    int ho, wo;
    conv3x3_output_hw(h, w, stride, pad, upsample2x, &ho, &wo);
    const int64_t m = int64_t(n) * ho * wo;
    MH_REQUIRE(m < (int64_t(1) << 31), "Conv3x3: too many output pixels");
    if (m == 0) return;
    const bool same = stride == 1 && pad[0] == 1 && pad[1] == 1 && pad[2] == 1 && pad[3] == 1 && !upsample2x;
    if (same && conv3x3_small_co(ctx, x, n, h, w, c_in, weight, wt, c_out, bias, prologue, out, residual2)) return;
    GemmArgs p{};
    p.a = x;
    p.M = int(m);
    p.N = c_out;
    p.K = 9 * c_in;
    p.cn = n;
    p.ch = h;
    p.cw = w;
    p.ci = c_in;
    p.ho = ho;
    p.wo = wo;
    p.stride = stride;
    p.pad_t = pad[0];
    p.pad_l = pad[1];
    p.up = upsample2x ? 1 : 0;
    p.b = weight;
    p.ldb = 9 * int64_t(c_in);
    p.a_bytes = extent(int64_t(n) * h * w, c_in, c_in, 4);
    p.b_bytes = extent(c_out, 9 * int64_t(c_in), 9 * int64_t(c_in), wt == kF16 ? 2 : 4);
    p.bias = bias;
    p.out = out;
    p.ldc = c_out;
    p.res2 = residual2;
    const bool pro = prologue != nullptr;
    if (pro) {
        p.psc = prologue->scale;
        p.psh = prologue->shift;
        p.psilu = prologue->silu ? 1 : 0;
    }
    const bool vec = c_in % 4 == 0 && aligned16(x);
    // Vector gathers need 16-byte rows of x and of the weight ([c_out][9 * c_in]).
    const int esz = wt == kF16 ? 2 : 4;
    const bool wvec = (reinterpret_cast<uintptr_t>(weight) % (4 * esz)) == 0;
    const int mode = vec && wvec ? (c_in % BK == 0 ? kConvAligned : kConvVec) : kConvScalar;
    run_conv(ctx, p, wt, mode, pro);
}

void im2col_gather(Context &ctx, const float *x, int n, int h, int w, int c, int stride, const int pad[4],
                   bool upsample2x, int64_t first, int64_t count, float *rows) {
    int ho, wo;
    conv3x3_output_hw(h, w, stride, pad, upsample2x, &ho, &wo);
    MH_REQUIRE(first >= 0 && count >= 0 && first + count <= int64_t(n) * ho * wo, "im2col: pixel range out of bounds");
    if (count == 0) return;
    GemmArgs p{};
    p.a = x;
    p.M = int(int64_t(n) * ho * wo);
    p.K = 9 * c;
    p.cn = n;
    p.ch = h;
    p.cw = w;
    p.ci = c;
    p.ho = ho;
    p.wo = wo;
    p.stride = stride;
    p.pad_t = pad[0];
    p.pad_l = pad[1];
    p.up = upsample2x ? 1 : 0;
    const int64_t total = count * 9 * c;
    const unsigned blocks = unsigned(std::min<int64_t>(ceil_div(total, 256), 1 << 20));
    im2col_gather_kernel<<<blocks, 256, 0, ctx.stream>>>(p, first, count, rows);
    MH_LAUNCH_CHECK();
}

void selftest_mfma_f32(Context &ctx, const float *a_host, const float *b_host, float *d_host) {
    float *dev = nullptr;
    mh::dev_malloc(&dev, (64 + 64 + 1024) * sizeof(float));
    HIP_CHECK(hipMemcpyAsync(dev, a_host, 64 * sizeof(float), hipMemcpyHostToDevice, ctx.stream));
    HIP_CHECK(hipMemcpyAsync(dev + 64, b_host, 64 * sizeof(float), hipMemcpyHostToDevice, ctx.stream));
    mfma_probe_kernel<<<1, 64, 0, ctx.stream>>>(dev, dev + 64, dev + 128);
    MH_LAUNCH_CHECK();
    HIP_CHECK(hipMemcpyAsync(d_host, dev + 128, 1024 * sizeof(float), hipMemcpyDeviceToHost, ctx.stream));
    HIP_CHECK(hipStreamSynchronize(ctx.stream));
    HIP_CHECK(hipFree(dev));
}

}  // namespace mh
