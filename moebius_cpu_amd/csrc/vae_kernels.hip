// Kernels the VAE chain needs beyond the engine's (src/vae/mod.rs,
// encoder.rs, decoder.rs): the mid attention's row softmax with its flush
// threshold, a tiled transpose for the attention's value operand, the
// posterior sample, and the latent / image rescalings.
#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

constexpr float kFlush = -40.0f;     // src/vae/mod.rs:271-273
constexpr float kScaling = 0.13025f; // src/config.rs:58
constexpr int kLatentC = 4;

// One wave per row (src/vae/mod.rs:275-294): the maximum (order-free), then
// e = exp((v - max) * scale) or 0 below the flush threshold into LDS, summed by
// one lane in row order in f32 (the reference's order), then v = e * (1 / sum).
__global__ __launch_bounds__(64) void softmax_rows_kernel(float *__restrict__ rows, int n, float scale) {
    extern __shared__ float e[];
    __shared__ float inv_s;
    float *row = rows + int64_t(blockIdx.x) * n;
    const int lane = threadIdx.x;
    float mx = -INFINITY;
    for (int j = lane; j < n; j += 64) mx = fmaxf(mx, row[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    for (int j = lane; j < n; j += 64) {
        const float a = (row[j] - mx) * scale;
        e[j] = a < kFlush ? 0.0f : ref_exp(a);
    }
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;
        for (int j = 0; j < n; ++j) sum += e[j];
        inv_s = 1.0f / sum;
    }
    __syncthreads();
    const float inv = inv_s;
    for (int j = lane; j < n; j += 64) row[j] = e[j] * inv;
}

// out [cols][rows] = in [rows][cols] (row stride ld_in), 32x32 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_kernel(const float *__restrict__ in, int64_t ld_in, int rows,
                                                        int cols, float *__restrict__ out) {
    __shared__ float tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) tile[i][tx] = in[int64_t(r) * ld_in + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) out[int64_t(c) * rows + r] = tile[tx][i];
    }
}

// src/vae/encoder.rs:121-133 per latent value: the log-variance clamped like
// Rust's f32::clamp (NaN stays NaN), then fma(exp(0.5 * logvar), noise, mean) * 0.13025.
__global__ void vae_sample_kernel(const float *__restrict__ moments, const float *__restrict__ noise, int64_t count,
                                  float *__restrict__ z) {
    const int64_t e = blockIdx.x * int64_t(256) + threadIdx.x;
    if (e >= count) return;
    const int64_t p = e / kLatentC;
    const int i = int(e - p * kLatentC);
    const float *m = moments + p * 2 * kLatentC;
    float lv = m[kLatentC + i];
    lv = lv < -30.0f ? -30.0f : (lv > 20.0f ? 20.0f : lv);
    z[e] = __builtin_fmaf(ref_exp(0.5f * lv), noise[e], m[i]) * kScaling;
}

// which 0: y = x / 0.13025 (decoder.rs:81-82); 1: y = (x + 1) * 0.5 (decoder.rs:96).
__global__ void vae_rescale_kernel(const float *__restrict__ x, int64_t len, int which, float *__restrict__ y) {
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < len; e += int64_t(gridDim.x) * 256)
        y[e] = which == 0 ? x[e] / kScaling : (x[e] + 1.0f) * 0.5f;
}

}  // namespace

void softmax_rows(Context &ctx, float *rows, int64_t nrows, int n, float scale) {
    MH_REQUIRE(n > 0 && n <= 15360, "softmax_rows: row length must be in 1..15360");
    MH_REQUIRE(nrows < (int64_t(1) << 31), "softmax_rows: too many rows");
    if (nrows == 0) return;
    softmax_rows_kernel<<<unsigned(nrows), 64, size_t(n) * sizeof(float), ctx.stream>>>(rows, n, scale);
    MH_LAUNCH_CHECK();
}

void transpose(Context &ctx, const float *in, int64_t ld_in, int rows, int cols, float *out) {
    MH_REQUIRE(ld_in >= cols, "transpose: leading dimension below the column count");
    if (rows == 0 || cols == 0) return;
    const dim3 grid(unsigned(ceil_div(cols, 32)), unsigned(ceil_div(rows, 32)));
    transpose_kernel<<<grid, 256, 0, ctx.stream>>>(in, ld_in, rows, cols, out);
    MH_LAUNCH_CHECK();
}

void vae_sample(Context &ctx, const float *moments, const float *noise, int64_t pixels, float *z) {
    const int64_t count = pixels * kLatentC;
    if (count == 0) return;
    vae_sample_kernel<<<unsigned(ceil_div(count, 256)), 256, 0, ctx.stream>>>(moments, noise, count, z);
    MH_LAUNCH_CHECK();
}

void vae_rescale(Context &ctx, const float *x, int64_t len, int which, float *y) {
    if (len == 0) return;
    const unsigned blocks = unsigned(std::min<int64_t>(ceil_div(len, 256), 65536));
    vae_rescale_kernel<<<blocks, 256, 0, ctx.stream>>>(x, len, which, y);
    MH_LAUNCH_CHECK();
}

}  // namespace mh
