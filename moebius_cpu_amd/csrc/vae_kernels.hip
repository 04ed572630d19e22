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
//
// The sum is one chain of adds over the LDS copy of e, read 32 floats at a time
// into two register blocks that alternate: the next block's reads are in flight
// while the current one is added. e is zero-padded to sum_pad(n) floats; adding
// +0 to a sum of non-negative terms leaves it unchanged, so the padding does not
// alter the result.
__host__ __device__ constexpr int sum_pad(int n) { return ((n + 63) / 64) * 64 + 32; }

__device__ __forceinline__ void add_block(float &sum, const float4 (&b)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        sum += b[u].x;
        sum += b[u].y;
        sum += b[u].z;
        sum += b[u].w;
    }
}

__device__ __forceinline__ void load_block(float4 (&b)[8], const float4 *p) {
#pragma unroll
    for (int u = 0; u < 8; ++u) b[u] = p[u];
}

__device__ __forceinline__ float sum_in_order(const float4 *e4, int n) {
    const int pairs = (n + 63) / 64;
    float4 a[8], b[8];
    float sum = 0.0f;
    load_block(a, e4);
    for (int p = 0; p < pairs; ++p) {
        load_block(b, e4 + 16 * p + 8);
        add_block(sum, a);
        load_block(a, e4 + 16 * p + 16);
        add_block(sum, b);
    }
    return sum;
}

__device__ __forceinline__ float flushed_exp(float v, float mx, float scale) {
    const float a = (v - mx) * scale;
    return a < kFlush ? 0.0f : ref_exp(a);
}

// Any row length: the row is read twice from memory, e kept in LDS.
__global__ __launch_bounds__(64) void softmax_rows_kernel(float *__restrict__ rows, int n, float scale) {
    extern __shared__ float4 e_lds[];  // sum_pad(n) floats
    float *e = reinterpret_cast<float *>(e_lds);
    __shared__ float inv_s;
    float *row = rows + int64_t(blockIdx.x) * n;
    const int lane = threadIdx.x;
    float mx = -INFINITY;
    for (int j = lane; j < n; j += 64) mx = fmaxf(mx, row[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    for (int j = lane; j < n; j += 64) e[j] = flushed_exp(row[j], mx, scale);
    for (int j = n + lane; j < sum_pad(n); j += 64) e[j] = 0.0f;
    __syncthreads();
    if (lane == 0) inv_s = 1.0f / sum_in_order(e_lds, n);
    __syncthreads();
    const float inv = inv_s;
    for (int j = lane; j < n; j += 64) row[j] = e[j] * inv;
}

// Rows of at most 64 * 4 * kRegF4 floats, a multiple of 4, 16-byte aligned: the
// row is read once, all its float4 loads in flight together, and stays in
// registers (a read per element per pass left each wave waiting on memory
// latency 128 times per row). Same arithmetic as softmax_rows_kernel.
constexpr int kRegF4 = 16;
__global__ __launch_bounds__(64) void softmax_rows_reg_kernel(float *__restrict__ rows, int n, float scale) {
    __shared__ float4 e4[sum_pad(64 * 4 * kRegF4) / 4];
    __shared__ float inv_s;
    float4 *row = reinterpret_cast<float4 *>(rows + int64_t(blockIdx.x) * n);
    const int lane = threadIdx.x, n4 = n / 4;
    float4 v[kRegF4];
#pragma unroll
    for (int i = 0; i < kRegF4; ++i) {
        const int j = i * 64 + lane;
        v[i] = j < n4 ? row[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kRegF4; ++i) mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
#pragma unroll
    for (int i = 0; i < kRegF4; ++i) {
        const int j = i * 64 + lane;
        v[i] = make_float4(flushed_exp(v[i].x, mx, scale), flushed_exp(v[i].y, mx, scale),
                           flushed_exp(v[i].z, mx, scale), flushed_exp(v[i].w, mx, scale));
        if (j < n4) e4[j] = v[i];
    }
    for (int j = n4 + lane; j < sum_pad(n) / 4; j += 64) e4[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    __syncthreads();
    if (lane == 0) inv_s = 1.0f / sum_in_order(e4, n);
    __syncthreads();
    const float inv = inv_s;
#pragma unroll
    for (int i = 0; i < kRegF4; ++i) {
        const int j = i * 64 + lane;
        if (j < n4) row[j] = make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv);
    }
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
    if (n % 4 == 0 && n <= 64 * 4 * kRegF4 && aligned16(rows))
        softmax_rows_reg_kernel<<<unsigned(nrows), 64, 0, ctx.stream>>>(rows, n, scale);
    else
        softmax_rows_kernel<<<unsigned(nrows), 64, size_t(sum_pad(n)) * sizeof(float), ctx.stream>>>(rows, n, scale);
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
