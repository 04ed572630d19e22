// Normalisation kernels for gfx950: GroupNorm statistics + affine apply, and
// LayerNorm. Bandwidth-bound; NHWC keeps every access a coalesced run of
// channels.
//
// GroupNorm (src/engine/norm.rs:57-148). Statistics follow the reference's
// structure: per-channel f32 partial sums of y and y*y (fused) over 256-pixel
// chunks (norm.rs:20, 73-82), then an f64 fold per group over channels and
// chunks (norm.rs:83-90), then mean/var/rstd and the per-channel scale/shift in
// f64 (norm.rs:93-101). One launch does it all: each block reduces a
// [256 px x 64 ch] tile of one item into per-channel partials, and the last
// block of the item to finish (device-scope fence + counter) folds them.
#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

constexpr int kGnChunk = 256;  // pixels per statistics chunk (norm.rs:20)
constexpr int kGnTileC = 64;   // channels per block: 16 lanes x float4
constexpr int kGnRows = 16;    // pixel rows per block pass

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__global__ __launch_bounds__(256) void gn_stats_kernel(const float *__restrict__ x, const float *__restrict__ add,
                                                       int hw, int c, int nchunks, int nctiles, int groups,
                                                       float eps, const float *__restrict__ gamma,
                                                       const float *__restrict__ beta, float *__restrict__ part,
                                                       unsigned int *counters, float *__restrict__ scale,
                                                       float *__restrict__ shift) {
    const int chunk = blockIdx.x, ct = blockIdx.y, b = blockIdx.z;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int c0 = ct * kGnTileC + tx * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f), q = s;
    if (c0 < c) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        if (add) a = *reinterpret_cast<const float4 *>(add + size_t(b) * c + c0);
        const float *xb = x + size_t(b) * hw * c + c0;
        const int p1 = min(hw, (chunk + 1) * kGnChunk);
        for (int p = chunk * kGnChunk + ty; p < p1; p += kGnRows) {
            float4 v = *reinterpret_cast<const float4 *>(xb + size_t(p) * c);
            if (add) {
                v.x = v.x + a.x;
                v.y = v.y + a.y;
                v.z = v.z + a.z;
                v.w = v.w + a.w;
            }
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
            q.x = __builtin_fmaf(v.x, v.x, q.x);
            q.y = __builtin_fmaf(v.y, v.y, q.y);
            q.z = __builtin_fmaf(v.z, v.z, q.z);
            q.w = __builtin_fmaf(v.w, v.w, q.w);
        }
    }
    __shared__ float4 red[2][kGnRows][16];
    red[0][ty][tx] = s;
    red[1][ty][tx] = q;
    __syncthreads();
    if (ty == 0 && c0 < c) {
        for (int r = 1; r < kGnRows; ++r) {
            const float4 rs = red[0][r][tx], rq = red[1][r][tx];
            s.x += rs.x;
            s.y += rs.y;
            s.z += rs.z;
            s.w += rs.w;
            q.x += rq.x;
            q.y += rq.y;
            q.z += rq.z;
            q.w += rq.w;
        }
        float *dst = part + (size_t(b) * nchunks + chunk) * c * 2 + size_t(c0) * 2;
        *reinterpret_cast<float4 *>(dst) = make_float4(s.x, q.x, s.y, q.y);
        *reinterpret_cast<float4 *>(dst + 4) = make_float4(s.z, q.z, s.w, q.w);
    }
    // Completion: the last block of item b folds all partials of the item.
    __threadfence();
    __syncthreads();
    __shared__ bool last;
    if (threadIdx.x == 0) {
        const unsigned int prev = atomicAdd(&counters[b], 1u);
        last = prev == unsigned(nchunks * nctiles - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cg = c / groups;
    const int total = nchunks * cg;
    const double count = double(hw) * double(cg);
    const float *pb = part + size_t(b) * nchunks * c * 2;
    for (int g = wave; g < groups; g += 4) {
        double ds = 0.0, dq = 0.0;
        for (int i = lane; i < total; i += 64) {
            const int ch = i / cg, j = i - ch * cg;
            const float *e = pb + (size_t(ch) * c + g * cg + j) * 2;
            ds += double(e[0]);
            dq += double(e[1]);
        }
        ds = wave_sum(ds);
        dq = wave_sum(dq);
        const double mean = ds / count;
        const double var = fmax(dq / count - mean * mean, 0.0);
        const double rstd = 1.0 / sqrt(var + double(eps));
        for (int j = lane; j < cg; j += 64) {
            const int ch = g * cg + j;
            const double sc = rstd * double(gamma[ch]);
            const double pre = add ? double(add[size_t(b) * c + ch]) : 0.0;
            scale[size_t(b) * c + ch] = float(sc);
            shift[size_t(b) * c + ch] = float(double(beta[ch]) + (pre - mean) * sc);
        }
    }
    if (threadIdx.x == 0) counters[b] = 0u;
}

// out = [SiLU](x . scale + shift), per item b = blockIdx.y; each block handles a
// contiguous run of float4s of its item. c4 = c/4 quads per pixel.
template <int ITER>
__global__ __launch_bounds__(256) void affine_apply_kernel(const float4 *__restrict__ x,
                                                           const float4 *__restrict__ scale,
                                                           const float4 *__restrict__ shift, int item4, int c4,
                                                           int silu, float4 *__restrict__ out) {
    const int b = blockIdx.y;
    const int e0 = blockIdx.x * (256 * ITER) + threadIdx.x;
    if (e0 >= item4) return;
    const size_t base = size_t(b) * item4;
    int q = e0 % c4;
    const int step = (256 % c4);
    const float4 *sc = scale + size_t(b) * c4;
    const float4 *sh = shift + size_t(b) * c4;
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
        const int e = e0 + i * 256;
        if (e < item4) {
            const float4 v = x[base + e];
            const float4 a = sc[q], d = sh[q];
            float4 y;
            y.x = __builtin_fmaf(v.x, a.x, d.x);
            y.y = __builtin_fmaf(v.y, a.y, d.y);
            y.z = __builtin_fmaf(v.z, a.z, d.z);
            y.w = __builtin_fmaf(v.w, a.w, d.w);
            if (silu) {
                y.x = ref_silu(y.x);
                y.y = ref_silu(y.y);
                y.z = ref_silu(y.z);
                y.w = ref_silu(y.w);
            }
            out[base + e] = y;
        }
        q += step;
        if (q >= c4) q -= c4;
    }
}

// Channel counts that are not a multiple of 4: one element per thread.
__global__ void affine_apply_scalar_kernel(const float *__restrict__ x, const float *__restrict__ scale,
                                           const float *__restrict__ shift, int64_t item, int c, int n, int silu,
                                           float *__restrict__ out) {
    const int64_t total = item * n;
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
        const int64_t b = e / item;
        const int ch = int(e % c);
        float y = __builtin_fmaf(x[e], scale[b * c + ch], shift[b * c + ch]);
        if (silu) y = ref_silu(y);
        out[e] = y;
    }
}

// LayerNorm (src/engine/norm.rs:151-173): one wave per token, two-pass
// variance in f32 over values held in registers.
template <int MAXV>
__global__ __launch_bounds__(256) void layer_norm_kernel(const float *__restrict__ x, int64_t rows, int c,
                                                         const float *__restrict__ gamma,
                                                         const float *__restrict__ beta, float eps,
                                                         float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int c4 = c >> 2;
    const float4 *src = reinterpret_cast<const float4 *>(x + row * c);
    float4 v[MAXV];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
        const int q = lane + 64 * i;
        v[i] = q < c4 ? src[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    const float mean = s / float(c);
    float vs = 0.f;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
        const int q = lane + 64 * i;
        if (q < c4) {
            const float a = v[i].x - mean, b = v[i].y - mean, cc = v[i].z - mean, d = v[i].w - mean;
            vs += (a * a + b * b) + (cc * cc + d * d);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) vs += __shfl_xor(vs, off, 64);
    const float rstd = 1.0f / sqrtf(vs / float(c) + eps);
    float4 *dst = reinterpret_cast<float4 *>(out + row * c);
    const float4 *g4 = reinterpret_cast<const float4 *>(gamma);
    const float4 *b4 = reinterpret_cast<const float4 *>(beta);
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
        const int q = lane + 64 * i;
        if (q < c4) {
            const float4 g = g4[q], bb = b4[q];
            float4 y;
            y.x = __builtin_fmaf((v[i].x - mean) * rstd, g.x, bb.x);
            y.y = __builtin_fmaf((v[i].y - mean) * rstd, g.y, bb.y);
            y.z = __builtin_fmaf((v[i].z - mean) * rstd, g.z, bb.z);
            y.w = __builtin_fmaf((v[i].w - mean) * rstd, g.w, bb.w);
            dst[q] = y;
        }
    }
}

// Any channel count: one wave per token, values re-read from global.
__global__ __launch_bounds__(256) void layer_norm_generic_kernel(const float *__restrict__ x, int64_t rows, int c,
                                                                 const float *__restrict__ gamma,
                                                                 const float *__restrict__ beta, float eps,
                                                                 float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *src = x + row * c;
    float s = 0.f;
    for (int j = lane; j < c; j += 64) s += src[j];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    const float mean = s / float(c);
    float vs = 0.f;
    for (int j = lane; j < c; j += 64) {
        const float d = src[j] - mean;
        vs += d * d;
    }
    for (int off = 32; off > 0; off >>= 1) vs += __shfl_xor(vs, off, 64);
    const float rstd = 1.0f / sqrtf(vs / float(c) + eps);
    for (int j = lane; j < c; j += 64) out[row * c + j] = __builtin_fmaf((src[j] - mean) * rstd, gamma[j], beta[j]);
}

}  // namespace

void group_norm_affine(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                       const float *gamma, const float *beta, const float *add, float *scale, float *shift) {
    MH_REQUIRE(groups > 0 && c % groups == 0, "channels not divisible by groups");
    MH_REQUIRE(c % 4 == 0, "GroupNorm: channel count must be a multiple of 4 on the GPU path");
    MH_REQUIRE(n > 0 && h > 0 && w > 0, "GroupNorm: empty tensor");
    MH_REQUIRE(aligned16(x) && aligned16(add), "GroupNorm: x and add must be 16-byte aligned");
    const int hw = h * w;
    const int nchunks = int(ceil_div(hw, kGnChunk));
    const int nctiles = int(ceil_div(c, kGnTileC));
    float *part = static_cast<float *>(ctx.ws.get(size_t(n) * nchunks * c * 2 * sizeof(float), ctx.stream));
    unsigned int *ctr = ctx.counter_block(n);
    dim3 grid(nchunks, nctiles, n);
    gn_stats_kernel<<<grid, 256, 0, ctx.stream>>>(x, add, hw, c, nchunks, nctiles, groups, eps, gamma, beta, part,
                                                  ctr, scale, shift);
    MH_LAUNCH_CHECK();
}

void apply_affine(Context &ctx, const float *x, int n, int h, int w, int c, const float *scale, const float *shift,
                  bool silu, float *out) {
    const int64_t item = int64_t(h) * w * c;
    if (item == 0 || n == 0) return;
    if (c % 4 == 0 && aligned16(x) && aligned16(scale) && aligned16(shift) && aligned16(out)) {
        constexpr int ITER = 8;
        const int item4 = int(item / 4);
        dim3 grid(unsigned(ceil_div(item4, 256 * ITER)), n);
        affine_apply_kernel<ITER><<<grid, 256, 0, ctx.stream>>>(
            reinterpret_cast<const float4 *>(x), reinterpret_cast<const float4 *>(scale),
            reinterpret_cast<const float4 *>(shift), item4, c / 4, silu ? 1 : 0, reinterpret_cast<float4 *>(out));
    } else {
        const int64_t total = item * n;
        const int blocks = int(std::min<int64_t>(ceil_div(total, 256), 65536));
        affine_apply_scalar_kernel<<<blocks, 256, 0, ctx.stream>>>(x, scale, shift, item, c, n, silu ? 1 : 0, out);
    }
    MH_LAUNCH_CHECK();
}

void group_norm_forward(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                        const float *gamma, const float *beta, const float *add, bool silu, float *out) {
    // scale/shift live in the tail of the workspace's partial block.
    const size_t part_bytes =
        size_t(n) * ceil_div(int64_t(h) * w, kGnChunk) * c * 2 * sizeof(float);
    const size_t aff_off = (part_bytes + 255) & ~size_t(255);
    char *ws = static_cast<char *>(ctx.ws.get(aff_off + size_t(n) * c * 2 * sizeof(float), ctx.stream));
    float *scale = reinterpret_cast<float *>(ws + aff_off);
    float *shift = scale + size_t(n) * c;
    group_norm_affine(ctx, x, n, h, w, c, groups, eps, gamma, beta, add, scale, shift);
    apply_affine(ctx, x, n, h, w, c, scale, shift, silu, out);
}

void layer_norm(Context &ctx, const float *x, int64_t rows, int c, const float *gamma, const float *beta, float eps,
                float *out) {
    MH_REQUIRE(c > 0, "LayerNorm: empty channel axis");
    if (rows == 0) return;
    const unsigned blocks = unsigned(ceil_div(rows, 4));
    const int c4 = c / 4;
    const bool vec = c % 4 == 0 && aligned16(x) && aligned16(gamma) && aligned16(beta) && aligned16(out);
    if (!vec) {
        layer_norm_generic_kernel<<<blocks, 256, 0, ctx.stream>>>(x, rows, c, gamma, beta, eps, out);
    } else if (c4 <= 64) {
        layer_norm_kernel<1><<<blocks, 256, 0, ctx.stream>>>(x, rows, c, gamma, beta, eps, out);
    } else if (c4 <= 128) {
        layer_norm_kernel<2><<<blocks, 256, 0, ctx.stream>>>(x, rows, c, gamma, beta, eps, out);
    } else if (c4 <= 320) {
        layer_norm_kernel<5><<<blocks, 256, 0, ctx.stream>>>(x, rows, c, gamma, beta, eps, out);
    } else {
        layer_norm_generic_kernel<<<blocks, 256, 0, ctx.stream>>>(x, rows, c, gamma, beta, eps, out);
    }
    MH_LAUNCH_CHECK();
}

}  // namespace mh
