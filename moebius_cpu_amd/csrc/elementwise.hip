// Bandwidth-bound elementwise kernels: the fused bias + residual prefill
// (src/engine/conv.rs:170-191), SiLU / add in place (src/engine/ops.rs:11-19),
// channel concatenation (src/engine/tensor.rs:59-73), 8-bit quantisation
// (src/imaging/blend.rs:21-24), and device evaluation of the reference's
// exp/SiLU. float4 accesses whenever the row length allows.
#include <hip/hip_fp16.h>

#include <algorithm>

#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

inline unsigned grid_for(int64_t work, int per_block = 256) {
    return unsigned(std::min<int64_t>(std::max<int64_t>(ceil_div(work, per_block), 1), 1 << 20));
}

// out = (residual + bias) + x, row-major rows x cols; cols4 = cols / 4.
template <bool HAS_B, bool HAS_R>
__global__ __launch_bounds__(256) void bias_residual_add4_kernel(const float4 *__restrict__ x,
                                                                 const float4 *__restrict__ bias,
                                                                 const float4 *__restrict__ res, int64_t total4,
                                                                 int cols4, float4 *__restrict__ out) {
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total4; e += int64_t(gridDim.x) * 256) {
        const float4 v = x[e];
        float4 t;
        if (HAS_B && HAS_R) {
            const float4 r = res[e], b = bias[e % cols4];
            t = make_float4(r.x + b.x, r.y + b.y, r.z + b.z, r.w + b.w);
        } else if (HAS_B) {
            t = bias[e % cols4];
        } else {
            t = res[e];
        }
        out[e] = make_float4(t.x + v.x, t.y + v.y, t.z + v.z, t.w + v.w);
    }
}

__global__ void bias_residual_add_kernel(const float *__restrict__ x, const float *__restrict__ bias,
                                         const float *__restrict__ res, int64_t total, int cols,
                                         float *__restrict__ out) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
        float t;
        if (bias && res)
            t = res[e] + bias[e % cols];
        else if (bias)
            t = bias[e % cols];
        else
            t = res[e];
        out[e] = t + x[e];
    }
}

__global__ void silu_kernel(float *__restrict__ x, int64_t len) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < len; e += int64_t(gridDim.x) * blockDim.x)
        x[e] = ref_silu(x[e]);
}

// dst [n][item] = SiLU(src [item]) for every copy.
__global__ void silu_tile_kernel(const float *__restrict__ src, int64_t item, int n, float *__restrict__ dst) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < item; e += int64_t(gridDim.x) * blockDim.x) {
        const float v = ref_silu(src[e]);
        for (int i = 0; i < n; ++i) dst[int64_t(i) * item + e] = v;
    }
}

__global__ void add_kernel(float *__restrict__ a, const float *__restrict__ b, int64_t len) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < len; e += int64_t(gridDim.x) * blockDim.x)
        a[e] = a[e] + b[e];
}

__global__ void add4_kernel(float4 *__restrict__ a, const float4 *__restrict__ b, int64_t len4) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < len4; e += int64_t(gridDim.x) * blockDim.x) {
        const float4 u = a[e], v = b[e];
        a[e] = make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
    }
}

// One output element (T = float or float4) per thread: [a || b] per pixel.
template <typename T>
__global__ void concat_kernel(const T *__restrict__ a, int ca, const T *__restrict__ b, int cb, int64_t pixels,
                              T *__restrict__ out) {
    const int c = ca + cb;
    const int64_t total = pixels * c;
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
        const int64_t p = e / c;
        const int j = int(e - p * c);
        out[e] = j < ca ? a[p * ca + j] : b[p * cb + (j - ca)];
    }
}

__global__ void to_u8_kernel(const float *__restrict__ x, int64_t len, uint8_t *__restrict__ out) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < len; e += int64_t(gridDim.x) * blockDim.x) {
        const float v = x[e];
        // clamp keeps NaN (f32::clamp), then `as u8` saturates and maps NaN to 0.
        const float cl = (v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v)) * 255.0f;
        out[e] = (cl != cl) ? uint8_t(0) : uint8_t(cl);
    }
}

// dst [n][item] = src [item] for every item (float4 when item4 > 0).
__global__ void tile_items4_kernel(const float4 *__restrict__ src, int64_t item4, int n, float4 *__restrict__ dst) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < item4; e += int64_t(gridDim.x) * blockDim.x) {
        const float4 v = src[e];
        for (int i = 0; i < n; ++i) dst[int64_t(i) * item4 + e] = v;
    }
}

__global__ void tile_items_kernel(const float *__restrict__ src, int64_t item, int n, float *__restrict__ dst) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < item; e += int64_t(gridDim.x) * blockDim.x) {
        const float v = src[e];
        for (int i = 0; i < n; ++i) dst[int64_t(i) * item + e] = v;
    }
}

// f16 -> f32 (exact: every f16 value is an f32 value).
__global__ void widen_f16_kernel(const _Float16 *__restrict__ src, int64_t len, float *__restrict__ dst) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < len; e += int64_t(gridDim.x) * blockDim.x)
        dst[e] = float(src[e]);
}

// f32 -> f16, round to nearest even, finite values beyond f16's range saturated
// to +-65504 (NaN stays NaN): the rounding the f16 GEMM applies to f32 operands
// as it stages them.
__global__ void round_f16_kernel(const float *__restrict__ src, int64_t len, _Float16 *__restrict__ dst) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < len; e += int64_t(gridDim.x) * blockDim.x) {
        const float v = src[e];
        dst[e] = static_cast<_Float16>(__builtin_fabsf(v) > 65504.0f ? __builtin_copysignf(65504.0f, v) : v);
    }
}

// One workgroup per weight row n (LnFolded, kernels.hpp): W' = W . gamma and its
// f16 rounding (nearest, saturated at +-65504 as the f16 GEMM rounds f32
// operands), their row sums and W . beta + bias, each summed in f64 per thread
// (thread t takes k = t, t + 256, ...) and then over the threads in a fixed tree.
__global__ __launch_bounds__(256) void ln_fold_kernel(const void *__restrict__ w, int f16, int k,
                                                      const float *__restrict__ gamma, const float *__restrict__ beta,
                                                      const float *__restrict__ bias, float *__restrict__ w32,
                                                      _Float16 *__restrict__ w16, float *__restrict__ c1_32,
                                                      float *__restrict__ c1_16, float *__restrict__ c2) {
    const int n = blockIdx.x, tid = threadIdx.x;
    const int64_t row = int64_t(n) * k;
    double s32 = 0.0, s16 = 0.0, sb = 0.0;
    for (int i = tid; i < k; i += 256) {
        const float wv = f16 ? float(static_cast<const _Float16 *>(w)[row + i]) : static_cast<const float *>(w)[row + i];
        const float wg = wv * gamma[i];
        w32[row + i] = wg;
        const float sat = __builtin_fabsf(wg) > 65504.0f ? __builtin_copysignf(65504.0f, wg) : wg;
        const _Float16 h = static_cast<_Float16>(sat);
        w16[row + i] = h;
        s32 += double(wg);
        s16 += double(float(h));
        sb += double(wv) * double(beta[i]);
    }
    __shared__ double red[3][256];
    red[0][tid] = s32, red[1][tid] = s16, red[2][tid] = sb;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) {
            red[0][tid] += red[0][tid + o];
            red[1][tid] += red[1][tid + o];
            red[2][tid] += red[2][tid + o];
        }
        __syncthreads();
    }
    if (tid == 0) {
        c1_32[n] = float(red[0][0]);
        c1_16[n] = float(red[1][0]);
        c2[n] = float(red[2][0] + (bias ? double(bias[n]) : 0.0));
    }
}

__global__ void math_eval_kernel(int which, const float *__restrict__ x, int64_t len, float *__restrict__ y) {
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < len; e += int64_t(gridDim.x) * blockDim.x)
        y[e] = which == 0 ? ref_exp(x[e]) : ref_silu(x[e]);
}

}  // namespace

void bias_residual_add(Context &ctx, const float *x, int64_t rows, int cols, const float *bias,
                       const float *residual, float *out) {
    MH_REQUIRE(cols > 0, "bias_residual_add: empty rows");
    const int64_t total = rows * cols;
    if (total == 0) return;
    if (!bias && !residual) {
        if (out != x) HIP_CHECK(hipMemcpyAsync(out, x, total * sizeof(float), hipMemcpyDeviceToDevice, ctx.stream));
        return;
    }
    if (cols % 4 == 0 && aligned16(x) && aligned16(bias) && aligned16(residual) && aligned16(out)) {
        const int64_t total4 = total / 4;
        const auto *x4 = reinterpret_cast<const float4 *>(x);
        const auto *b4 = reinterpret_cast<const float4 *>(bias);
        const auto *r4 = reinterpret_cast<const float4 *>(residual);
        auto *o4 = reinterpret_cast<float4 *>(out);
        const unsigned g = grid_for(total4);
        if (bias && residual)
            bias_residual_add4_kernel<true, true><<<g, 256, 0, ctx.stream>>>(x4, b4, r4, total4, cols / 4, o4);
        else if (bias)
            bias_residual_add4_kernel<true, false><<<g, 256, 0, ctx.stream>>>(x4, b4, r4, total4, cols / 4, o4);
        else
            bias_residual_add4_kernel<false, true><<<g, 256, 0, ctx.stream>>>(x4, b4, r4, total4, cols / 4, o4);
    } else {
        bias_residual_add_kernel<<<grid_for(total), 256, 0, ctx.stream>>>(x, bias, residual, total, cols, out);
    }
    MH_LAUNCH_CHECK();
}

void silu_inplace(Context &ctx, float *x, int64_t len) {
    if (len == 0) return;
    silu_kernel<<<grid_for(len), 256, 0, ctx.stream>>>(x, len);
    MH_LAUNCH_CHECK();
}

void silu_tile(Context &ctx, const float *src, int64_t item, int n, float *dst) {
    if (item == 0 || n == 0) return;
    silu_tile_kernel<<<grid_for(item), 256, 0, ctx.stream>>>(src, item, n, dst);
    MH_LAUNCH_CHECK();
}

void add_inplace(Context &ctx, float *a, const float *b, int64_t len) {
    if (len == 0) return;
    if (len % 4 == 0 && (reinterpret_cast<uintptr_t>(a) % 16 == 0) && (reinterpret_cast<uintptr_t>(b) % 16 == 0)) {
        add4_kernel<<<grid_for(len / 4), 256, 0, ctx.stream>>>(reinterpret_cast<float4 *>(a),
                                                               reinterpret_cast<const float4 *>(b), len / 4);
    } else {
        add_kernel<<<grid_for(len), 256, 0, ctx.stream>>>(a, b, len);
    }
    MH_LAUNCH_CHECK();
}

void concat_channels(Context &ctx, const float *a, int ca, const float *b, int cb, int64_t pixels, float *out) {
    MH_REQUIRE(ca >= 0 && cb >= 0, "concat_channels: negative channel count");
    if (pixels == 0 || ca + cb == 0) return;
    if (ca % 4 == 0 && cb % 4 == 0 && aligned16(a) && aligned16(b) && aligned16(out)) {
        concat_kernel<float4><<<grid_for(pixels * (ca + cb) / 4), 256, 0, ctx.stream>>>(
            reinterpret_cast<const float4 *>(a), ca / 4, reinterpret_cast<const float4 *>(b), cb / 4, pixels,
            reinterpret_cast<float4 *>(out));
    } else {
        concat_kernel<float><<<grid_for(pixels * (ca + cb)), 256, 0, ctx.stream>>>(a, ca, b, cb, pixels, out);
    }
    MH_LAUNCH_CHECK();
}

void to_u8(Context &ctx, const float *x, int64_t len, uint8_t *out) {
    if (len == 0) return;
    to_u8_kernel<<<grid_for(len), 256, 0, ctx.stream>>>(x, len, out);
    MH_LAUNCH_CHECK();
}

void tile_items(Context &ctx, const float *src, int64_t item, int n, float *dst) {
    MH_REQUIRE(n >= 1 && item >= 0, "tile_items: bad item count or size");
    if (item == 0) return;
    if (item % 4 == 0 && aligned16(src) && aligned16(dst))
        tile_items4_kernel<<<grid_for(item / 4), 256, 0, ctx.stream>>>(reinterpret_cast<const float4 *>(src), item / 4,
                                                                     n, reinterpret_cast<float4 *>(dst));
    else
        tile_items_kernel<<<grid_for(item), 256, 0, ctx.stream>>>(src, item, n, dst);
    MH_LAUNCH_CHECK();
}

void widen_f16(Context &ctx, const void *src, int64_t len, float *dst) {
    if (len == 0) return;
    widen_f16_kernel<<<grid_for(len), 256, 0, ctx.stream>>>(static_cast<const _Float16 *>(src), len, dst);
    MH_LAUNCH_CHECK();
}

void round_f16(Context &ctx, const float *src, int64_t len, void *dst) {
    if (len == 0) return;
    round_f16_kernel<<<grid_for(len), 256, 0, ctx.stream>>>(src, len, static_cast<_Float16 *>(dst));
    MH_LAUNCH_CHECK();
}

void ln_fold_weights(Context &ctx, const void *w, WeightType wt, int n, int k, const float *gamma, const float *beta,
                     const float *bias, float *w32, void *w16, float *c1_32, float *c1_16, float *c2) {
    MH_REQUIRE(n > 0 && k > 0 && w && gamma && beta && w32 && w16 && c1_32 && c1_16 && c2,
               "ln_fold_weights: missing tensors");
    ln_fold_kernel<<<unsigned(n), 256, 0, ctx.stream>>>(w, wt == kF16 ? 1 : 0, k, gamma, beta, bias, w32,
                                                       static_cast<_Float16 *>(w16), c1_32, c1_16, c2);
    MH_LAUNCH_CHECK();
}

void math_eval(Context &ctx, int which, const float *x, int64_t len, float *y) {
    MH_REQUIRE(which == 0 || which == 1, "math_eval: which must be 0 (exp) or 1 (silu)");
    if (len == 0) return;
    math_eval_kernel<<<grid_for(len), 256, 0, ctx.stream>>>(which, x, len, y);
    MH_LAUNCH_CHECK();
}

}  // namespace mh
