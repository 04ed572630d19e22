// Normalisation kernels for gfx950: GroupNorm statistics + affine apply, and
// LayerNorm. Bandwidth-bound; NHWC keeps every access a coalesced run of
// channels.
//
// GroupNorm (src/engine/norm.rs:57-148). Statistics keep the reference's
// structure: per-channel f32 partial sums of y and y*y (fused) over pixel
// chunks (norm.rs:73-82), folded per group in f64 over channels and chunks
// (norm.rs:83-90), then mean/var/rstd and the per-channel scale/shift in f64
// (norm.rs:93-101). Two launches: gn_partial_kernel reduces [64 px x 64 ch]
// tiles (thousands of blocks at the UNet/VAE sizes), gn_finalize_kernel folds
// one (item, group) per block with a fixed-order tree, so results are
// deterministic. The apply pass is a separate kernel, or is fused into the
// consumer (the depthwise and GEMM prologues) with the scale/shift produced here.
#include <cstdlib>
#include <mutex>
#include <string>

#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

constexpr int kGnTileC = 64;   // channels per block: 16 lanes x float4
constexpr int kGnRows = 16;    // pixel rows per block pass

// Pixels per statistics chunk: 64, doubled until the partials grid is at most
// max_blocks blocks (Tuning::gn_blocks, 512: at 512x512x128, 4096 blocks took
// 78 us and 512 blocks 66 us for statistics + SiLU apply), so small maps get
// many blocks and large maps few enough partials for the fold to stay short.
int gn_chunk_px(int n, int hw, int c, int max_blocks) {
    const int64_t ctiles = ceil_div(c, kGnTileC);
    int chunk = 64;
    while (chunk < hw && ceil_div(hw, chunk) * ctiles * n > max_blocks) chunk *= 2;
    return chunk;
}

// part [n][chunks][c][2] = per-channel (sum y, sum y*y) over the chunk, y = x (+ add).
// x2 (optional): x is [x | x2] per pixel, x holding channels [0, c1) (c1 a
// multiple of kGnTileC, so a block reads one of the two) and x2 the rest.
__global__ __launch_bounds__(256) void gn_partial_kernel(const float *__restrict__ x, const float *__restrict__ add,
                                                         int64_t add_ld, int hw, int c, int chunk_px, int nchunks,
                                                         float *__restrict__ part, const float *__restrict__ x2,
                                                         int c1) {
    const int chunk = blockIdx.x, ct = blockIdx.y, b = blockIdx.z;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int c0 = ct * kGnTileC + tx * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f), q = s;
    if (c0 < c) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        if (add) a = *reinterpret_cast<const float4 *>(add + size_t(b) * add_ld + c0);
        const bool sec = x2 && ct * kGnTileC >= c1;
        const int ld = x2 ? (sec ? c - c1 : c1) : c;
        const float *xb = sec ? x2 + size_t(b) * hw * ld + (c0 - c1) : x + size_t(b) * hw * ld + c0;
        const int p1 = min(hw, (chunk + 1) * chunk_px);
#pragma unroll 4
        for (int p = chunk * chunk_px + ty; p < p1; p += kGnRows) {
            float4 v = *reinterpret_cast<const float4 *>(xb + size_t(p) * ld);
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
}

// One block per (group, item): f64 fold of the group's partials, then scale/shift.
// part_rows > 0: the partials are of x alone, part_rows pixels each, and add
// is folded in per partial: sum (y + t) = S + r t, sum (y + t)^2 = Q + 2 t S + r t^2.
// Each thread keeps kFin independent sums with all their loads in flight (the
// producers' partials run to 16K values per group at 512x512x128), added in a
// fixed order, so the fold is deterministic.
constexpr int kFinThreads = 512, kFin = 8;
__global__ __launch_bounds__(kFinThreads) void gn_finalize_kernel(const float *__restrict__ part,
                                                                  const float *__restrict__ add, int64_t add_ld,
                                                                  int hw, int c, int nchunks, int groups,
                                                                  int part_rows, float eps,
                                                                  const float *__restrict__ gamma,
                                                                  const float *__restrict__ beta,
                                                                  float *__restrict__ scale,
                                                                  float *__restrict__ shift) {
    const int g = blockIdx.x, b = blockIdx.y;
    const int cg = c / groups;
    const int total = nchunks * cg;
    // This thread's first channel's parameters, loaded before the fold so their
    // latency overlaps it instead of following the reduction.
    const int j0 = int(threadIdx.x);
    float g0 = 0.f, b0 = 0.f, a0 = 0.f;
    if (j0 < cg) {
        const int ch = g * cg + j0;
        g0 = gamma[ch];
        b0 = beta[ch];
        if (add) a0 = add[size_t(b) * add_ld + ch];
    }
    const float *pb = part + size_t(b) * nchunks * c * 2 + size_t(g) * cg * 2;
    const bool fold = part_rows > 0 && add;
    const double r = double(part_rows);
    double ds[kFin], dq[kFin];
#pragma unroll
    for (int u = 0; u < kFin; ++u) ds[u] = dq[u] = 0.0;
    for (int i0 = threadIdx.x; i0 < total; i0 += kFin * kFinThreads) {
        float2 e[kFin];
#pragma unroll
        for (int u = 0; u < kFin; ++u) {
            const int i = i0 + u * kFinThreads;
            const int ch = i / cg, j = i - ch * cg;
            e[u] = i < total ? *reinterpret_cast<const float2 *>(pb + (size_t(ch) * c + j) * 2) : make_float2(0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < kFin; ++u) {
            const int i = i0 + u * kFinThreads;
            if (i >= total) break;
            if (fold) {
                const int j = i % cg;
                const double t = double(add[size_t(b) * add_ld + size_t(g) * cg + j]);
                ds[u] += double(e[u].x) + r * t;
                dq[u] += double(e[u].y) + 2.0 * t * double(e[u].x) + r * t * t;
            } else {
                ds[u] += double(e[u].x);
                dq[u] += double(e[u].y);
            }
        }
    }
#pragma unroll
    for (int u = 1; u < kFin; ++u) {
        ds[0] += ds[u];
        dq[0] += dq[u];
    }
    double s0 = ds[0], q0 = dq[0];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        s0 += __shfl_xor(s0, off, 64);
        q0 += __shfl_xor(q0, off, 64);
    }
    constexpr int kW = kFinThreads / 64;
    __shared__ double red[2][kW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        red[0][wave] = s0;
        red[1][wave] = q0;
    }
    __syncthreads();
    double sum = red[0][0], sumsq = red[1][0];
#pragma unroll
    for (int w = 1; w < kW; ++w) {
        sum += red[0][w];
        sumsq += red[1][w];
    }
    const double count = double(hw) * double(cg);
    const double mean = sum / count;
    const double var = fmax(sumsq / count - mean * mean, 0.0);
    const double rstd = 1.0 / sqrt(var + double(eps));
    for (int j = threadIdx.x; j < cg; j += kFinThreads) {
        const int ch = g * cg + j;
        const bool first = j == j0;
        const double sc = rstd * double(first ? g0 : gamma[ch]);
        const double pre = add ? double(first ? a0 : add[size_t(b) * add_ld + ch]) : 0.0;
        scale[size_t(b) * c + ch] = float(sc);
        shift[size_t(b) * c + ch] = float(double(first ? b0 : beta[ch]) + (pre - mean) * sc);
    }
}

// LayerNorm row statistics (src/engine/norm.rs:151-173) for a consumer that
// applies ((v - mean) * rstd) * gamma + beta itself: stats [rows][2] = (mean, rstd).
template <int MAXV>
__global__ __launch_bounds__(256) void ln_stats_kernel(const float *__restrict__ x, int64_t rows, int c, float eps,
                                                       float2 *__restrict__ stats) {
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
    if (lane == 0) stats[row] = make_float2(mean, 1.0f / sqrtf(vs / float(c) + eps));
}

template <int ITER>
__global__ __launch_bounds__(256) void affine_apply_kernel(const float4 *__restrict__ x,
                                                           const float4 *__restrict__ scale,
                                                           const float4 *__restrict__ shift, int item4, int c4,
                                                           int silu, int reverse, float4 *__restrict__ out) {
    // reverse (Tuning::gn_apply): blocks walk the map from its end, where the
    // statistics pass read last (measured equal at 512x512x128)
    const int b = blockIdx.y;
    const int bx = reverse ? int(gridDim.x) - 1 - int(blockIdx.x) : int(blockIdx.x);
    const int e0 = bx * (256 * ITER) + threadIdx.x;
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

namespace {

// Floats of the statistics partials group_norm_affine writes for this shape.
int64_t gn_partial_floats(const Context &ctx, int n, int hw, int c) {
    return int64_t(n) * ceil_div(hw, gn_chunk_px(n, hw, c, ctx.tune.gn_blocks)) * c * 2;
}

// group_norm_affine with its partials at `part` (gn_partial_floats of them).
void group_norm_affine_into(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                            const float *gamma, const float *beta, const float *add, float *scale, float *shift,
                            int64_t add_ld, float *part, const float *x2 = nullptr, int c2 = 0) {
    const int hw = h * w;
    const int chunk_px = gn_chunk_px(n, hw, c, ctx.tune.gn_blocks);
    const int nchunks = int(ceil_div(hw, chunk_px));
    const int nctiles = int(ceil_div(c, kGnTileC));
    gn_partial_kernel<<<dim3(nchunks, nctiles, n), 256, 0, ctx.stream>>>(x, add, add_ld, hw, c, chunk_px, nchunks,
                                                                        part, x2, c - c2);
    MH_LAUNCH_CHECK();
    gn_finalize_kernel<<<dim3(groups, n), kFinThreads, 0, ctx.stream>>>(part, add, add_ld, hw, c, nchunks, groups, 0, eps,
                                                                gamma, beta, scale, shift);
    MH_LAUNCH_CHECK();
}

void gn_check(int n, int h, int w, int c, int groups, const float *x, const float *add, int64_t add_ld) {
    MH_REQUIRE(add_ld % 4 == 0, "GroupNorm: add row stride must be a multiple of 4");
    MH_REQUIRE(groups > 0 && c % groups == 0, "channels not divisible by groups");
    MH_REQUIRE(c % 4 == 0, "GroupNorm: channel count must be a multiple of 4 on the GPU path");
    MH_REQUIRE(n > 0 && h > 0 && w > 0, "GroupNorm: empty tensor");
    MH_REQUIRE(aligned16(x) && aligned16(add), "GroupNorm: x and add must be 16-byte aligned");
}

}  // namespace

void group_norm_affine(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                       const float *gamma, const float *beta, const float *add, float *scale, float *shift,
                       int64_t add_ld, const float *x2, int c2) {
    if (add_ld <= 0) add_ld = c;
    gn_check(n, h, w, c, groups, x, add, add_ld);
    if (x2)
        MH_REQUIRE(c2 > 0 && c2 < c && (c - c2) % kGnTileC == 0 && c2 % 4 == 0 && aligned16(x2),
                   "GroupNorm over two inputs: first part a multiple of 64 channels, second of 4, 16-byte aligned");
    float *part = static_cast<float *>(
        ctx.ws.get(size_t(gn_partial_floats(ctx, n, h * w, c)) * sizeof(float), ctx.stream));
    group_norm_affine_into(ctx, x, n, h, w, c, groups, eps, gamma, beta, add, scale, shift, add_ld, part, x2,
                           x2 ? c2 : 0);
}

void group_norm_affine_partials(Context &ctx, const float *part, int rows, int n, int hw, int c, int groups,
                                float eps, const float *gamma, const float *beta, const float *add, float *scale,
                                float *shift, int64_t add_ld) {
    if (add_ld <= 0) add_ld = c;
    MH_REQUIRE(groups > 0 && c % groups == 0, "channels not divisible by groups");
    MH_REQUIRE(n > 0 && hw > 0 && rows > 0 && hw % rows == 0, "GroupNorm partials: tiles must divide the item");
    MH_REQUIRE(aligned16(part), "GroupNorm partials must be 16-byte aligned");
    gn_finalize_kernel<<<dim3(groups, n), kFinThreads, 0, ctx.stream>>>(part, add, add_ld, hw, c, hw / rows, groups, rows,
                                                                eps, gamma, beta, scale, shift);
    MH_LAUNCH_CHECK();
}

void layer_norm_stats(Context &ctx, const float *x, int64_t rows, int c, float eps, float *stats) {
    MH_REQUIRE(c % 4 == 0 && c <= 1280 && aligned16(x), "LayerNorm stats: channels must be a multiple of 4, <= 1280");
    if (rows == 0) return;
    const unsigned blocks = unsigned(ceil_div(rows, 4));
    float2 *st = reinterpret_cast<float2 *>(stats);
    const int c4 = c / 4;
    if (c4 <= 64)
        ln_stats_kernel<1><<<blocks, 256, 0, ctx.stream>>>(x, rows, c, eps, st);
    else if (c4 <= 128)
        ln_stats_kernel<2><<<blocks, 256, 0, ctx.stream>>>(x, rows, c, eps, st);
    else
        ln_stats_kernel<5><<<blocks, 256, 0, ctx.stream>>>(x, rows, c, eps, st);
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
            reinterpret_cast<const float4 *>(shift), item4, c / 4, silu ? 1 : 0, ctx.tune.gn_apply,
            reinterpret_cast<float4 *>(out));
    } else {
        const int64_t total = item * n;
        const int blocks = int(std::min<int64_t>(ceil_div(total, 256), 65536));
        affine_apply_scalar_kernel<<<blocks, 256, 0, ctx.stream>>>(x, scale, shift, item, c, n, silu ? 1 : 0, out);
    }
    MH_LAUNCH_CHECK();
}

namespace {

// Floats group_norm_forward needs beyond its input and output: the statistics
// partials, then (from the next 256-byte boundary) scale and shift [n * c] each.
struct GnForwardScratch {
    int64_t aff_off, total;
};

GnForwardScratch gn_forward_scratch(const Context &ctx, int n, int h, int w, int c) {
    GnForwardScratch s;
    s.aff_off = (gn_partial_floats(ctx, n, h * w, c) + 63) & ~int64_t(63);
    s.total = s.aff_off + 2 * int64_t(n) * c;
    return s;
}

void group_norm_forward_in(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                           const float *gamma, const float *beta, const float *add, bool silu, float *out,
                           int64_t add_ld, float *base, int64_t aff_off) {
    float *scale = base + aff_off;
    float *shift = scale + int64_t(n) * c;
    group_norm_affine_into(ctx, x, n, h, w, c, groups, eps, gamma, beta, add, scale, shift, add_ld, base);
    apply_affine(ctx, x, n, h, w, c, scale, shift, silu, out);
}

}  // namespace

void group_norm_forward(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                        const float *gamma, const float *beta, const float *add, bool silu, float *out,
                        int64_t add_ld) {
    if (add_ld <= 0) add_ld = c;
    gn_check(n, h, w, c, groups, x, add, add_ld);
    const GnForwardScratch s = gn_forward_scratch(ctx, n, h, w, c);
    float *base = static_cast<float *>(ctx.ws.get(size_t(s.total) * sizeof(float), ctx.stream));
    group_norm_forward_in(ctx, x, n, h, w, c, groups, eps, gamma, beta, add, silu, out, add_ld, base, s.aff_off);
}

// ---- GroupNorm forward without allocation ----
// Its scratch (the statistics partials, scale and shift) is this fixed device
// array, one copy per GPU, held until the process ends. Host code never passes
// `scratch` itself to a kernel (on the host the name is only a stand-in): the
// device address comes from hipGetSymbolAddress, taken once per device when a
// context is created on it (noalloc_scratch_setup) and kept in g_scratch_ptr.
// Calls from different streams (two contexts on one GPU) are ordered on the
// device: each call records g_scratch_done on its stream, and a call from
// another stream first waits for that event, so its kernels start only after
// the previous user of the array has finished with it. A stream under graph
// capture takes no part in this ordering (its graph's launches are ordered by
// whoever launches them).
constexpr int64_t kNoAllocScratchFloats = int64_t(1) << 18;  // 1 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxDevices] = {};
hipEvent_t g_scratch_done[kMaxDevices] = {};
hipStream_t g_scratch_last[kMaxDevices] = {};  // stream of the last recorded call
}  // namespace

void noalloc_scratch_setup(int device) {
    MH_REQUIRE(device >= 0 && device < kMaxDevices, "device ordinal beyond the library's device table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return;
    int cur = -1;
    HIP_CHECK(hipGetDevice(&cur));
    if (cur != device) fail(kInternal, "noalloc scratch set-up: the device is not current");
    void *ptr = nullptr;
    HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) fail(kInternal, "hipGetSymbolAddress returned no address for the GroupNorm scratch");
    hipEvent_t done = nullptr;
    HIP_CHECK(hipEventCreateWithFlags(&done, hipEventDisableTiming));
    g_scratch_ptr[device] = static_cast<float *>(ptr);
    g_scratch_done[device] = done;
}

int64_t group_norm_noalloc_max_floats() { return kNoAllocScratchFloats; }

void group_norm_forward_noalloc(Context &ctx, const float *x, int n, int h, int w, int c, int groups, float eps,
                                const float *gamma, const float *beta, const float *add, bool silu, float *out) {
    const int64_t add_ld = c;
    gn_check(n, h, w, c, groups, x, add, add_ld);
    const GnForwardScratch s = gn_forward_scratch(ctx, n, h, w, c);
    if (s.total > kNoAllocScratchFloats) {
        fail(kInvalidArgument, "GroupNorm (no allocation): this shape needs " + std::to_string(s.total) +
                                   " floats of scratch (statistics partials plus scale/shift for n * c = " +
                                   std::to_string(int64_t(n) * c) + "), more than the fixed " +
                                   std::to_string(kNoAllocScratchFloats) + " (1 MiB)");
    }
    // held across the launches, so that host threads take the array in the
    // order their waits and records were queued
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    const int dev = ctx.device;
    float *base = dev >= 0 && dev < kMaxDevices ? g_scratch_ptr[dev] : nullptr;
    if (!base) fail(kInternal, "GroupNorm (no allocation): scratch address not set up for this device");
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_CHECK(hipStreamIsCapturing(ctx.stream, &cap));
    const bool order = cap == hipStreamCaptureStatusNone;
    if (order && g_scratch_last[dev] && g_scratch_last[dev] != ctx.stream)
        HIP_CHECK(hipStreamWaitEvent(ctx.stream, g_scratch_done[dev], 0));
    group_norm_forward_in(ctx, x, n, h, w, c, groups, eps, gamma, beta, add, silu, out, add_ld, base, s.aff_off);
    if (order) {
        HIP_CHECK(hipEventRecord(g_scratch_done[dev], ctx.stream));
        g_scratch_last[dev] = ctx.stream;
    }
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
