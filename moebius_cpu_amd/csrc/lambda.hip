// Lambda-layer kernels of the UNet's MixTransformer (src/unet/lambda.rs).
//
// softmax_lambda (lambda.rs:322-359): lambda_c[kk][j] = sum_r softmax_r(K)[r][kk] * V[r][j]
//   1. column maxima of K over rows, per row chunk;
//   2. per chunk: e = exp(K - colmax) (the reference's Cephes exp), f32 column
//      sums over the chunk, and the chunk's partial e^T V in f32;
//   3. finalise: partials summed over chunks in order (f32 for lambda, f64 for
//      the sums, as the reference folds its chunk sums in f64), row kk scaled by
//      (f32)(1 / sum[kk]); written transposed ([j][kk]) so Yc = Q . lambda_c is
//      an NT GEMM.
// tap_filter (lambda.rs:154-185): per pixel, head and value channel,
//   o = Yc + A[., 225] then + A[., dy*15+dx] * V[pixel + (dy-7, dx-7)] over the
//   in-image taps in (dy, dx) order with fused multiply-adds: the reference's
//   per-element operation order. A arrives tap-major ([pixel][226][8], written
//   that way by the GEMM that makes it) so one thread's heads share each value
//   load; the block's residual add can be folded into the store.
// position_term (lambda.rs:276-295): per pixel, B[h][m] = q_h . E[n][m] with
//   the reference's 8-lane dot, then o_h += B[h][m] * V[m] for m = 0..9; the
//   block's residual add can be folded into the store.
#include <cstdlib>

#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

constexpr int kWin = 15, kTaps = 225, kPad = 7, kTapsB = 226;
constexpr int kHeads = 8, kTokens = 10;

// softmax_lambda work split: chunks of rows per item (about 16-32, so the
// finalising fold stays short) and tiles of tk key columns per block, so the
// UNet's three sizes get 300+ blocks: 64x64 x 40 -> 128 rows x 8 columns,
// 32x32 x 80 -> 64 x 16, 16x16 x 160 -> 16 x 16.
struct LambdaSplit {
    int ch, chunks, tk, ktiles;
};

LambdaSplit lambda_split(int rows, int k, int vd) {
    LambdaSplit s;
    s.ch = 128;
    while (s.ch > 8 && ceil_div(rows, s.ch) < 16) s.ch >>= 1;
    while (s.ch > 8 && int64_t(s.ch) * (16 + vd) > 12288) s.ch >>= 1;  // LDS: keys tile + values
    s.chunks = int(ceil_div(rows, s.ch));
    s.tk = k % 16 == 0 && k >= 80 ? 16 : (k % 8 == 0 ? 8 : 4);
    s.ktiles = int(ceil_div(k, s.tk));
    return s;
}

// One block per (chunk, item, key tile): chunk-local column maxima m of its tk
// key columns, e = exp(K - m) (the reference's Cephes exp), f32 column sums of
// e and the partial e^T V [tk][vd] over the chunk's rows. The chunk results
// are rescaled to the global maximum when they are folded (finalize), so no
// separate maximum pass is needed. Dynamic LDS: e [ch][tk], v [ch][vd],
// reduction scratch [256].
__global__ __launch_bounds__(256) void lambda_partial_kernel(const float *__restrict__ keys,
                                                             const float *__restrict__ v, int rows, int k, int vd,
                                                             int ch, int chunks, int tk, float *__restrict__ pmax,
                                                             float *__restrict__ psum, float *__restrict__ plam) {
    extern __shared__ float lds[];
    float *es = lds, *vs = lds + ch * tk, *red = vs + ch * vd;
    const int chunk = blockIdx.x, b = blockIdx.y, k0 = blockIdx.z * tk;
    const int r0 = chunk * ch, nr = min(ch, rows - r0);
    const int nk = min(tk, k - k0);
    const float *kb = keys + (size_t(b) * rows + r0) * k + k0;
    for (int i = threadIdx.x; i < nr * tk; i += 256) {
        const int r = i / tk, j = i - r * tk;
        es[i] = j < nk ? kb[size_t(r) * k + j] : 0.0f;
    }
    const float4 *vb4 = reinterpret_cast<const float4 *>(v + (size_t(b) * rows + r0) * vd);
    float4 *vs4 = reinterpret_cast<float4 *>(vs);
    for (int i = threadIdx.x; i < nr * (vd >> 2); i += 256) vs4[i] = vb4[i];
    __syncthreads();
    // column maxima and (after exp) column sums: column j = t % tk, rows
    // r = g, g + G, ... for row group g = t / tk; groups folded in order
    const int G = 256 / tk;
    const int j = threadIdx.x % tk, g = threadIdx.x / tk;
    float m = -INFINITY;
    if (g < G)
        for (int r = g; r < nr; r += G) m = fmaxf(m, es[r * tk + j]);
    red[threadIdx.x] = m;
    __syncthreads();
    if (threadIdx.x < tk) {
        float mm = red[threadIdx.x];
        for (int q = 1; q < G; ++q) mm = fmaxf(mm, red[q * tk + threadIdx.x]);
        red[threadIdx.x] = mm;  // read back below as the column maximum
    }
    __syncthreads();
    const float colmax = red[j];
    __syncthreads();
    for (int i = threadIdx.x; i < nr * tk; i += 256) es[i] = ref_exp(es[i] - red[i % tk]);
    // (red[0..tk) still holds the maxima: the loop above only reads it)
    float sum = 0.0f;
    __syncthreads();
    if (g < G)
        for (int r = g; r < nr; r += G) sum += es[r * tk + j];
    __syncthreads();
    red[threadIdx.x] = sum;
    __syncthreads();
    if (threadIdx.x < nk) {
        float t = red[threadIdx.x];
        for (int q = 1; q < G; ++q) t += red[q * tk + threadIdx.x];
        const size_t o = (size_t(b) * chunks + chunk) * k + k0 + threadIdx.x;
        psum[o] = t;
        pmax[o] = colmax;
    }
    // e^T V: task (kk, j quad) per thread and pass
    const int vq = vd >> 2;
    float4 *pl = reinterpret_cast<float4 *>(plam + ((size_t(b) * chunks + chunk) * k + k0) * vd);
    for (int t = threadIdx.x; t < nk * vq; t += 256) {
        const int kk = t / vq, jq = t - kk * vq;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 *vr = vs4 + jq;
#pragma unroll 4
        for (int r = 0; r < nr; ++r) {
            const float e = es[r * tk + kk];
            const float4 x = vr[r * vq];
            acc.x = __builtin_fmaf(e, x.x, acc.x);
            acc.y = __builtin_fmaf(e, x.y, acc.y);
            acc.z = __builtin_fmaf(e, x.z, acc.z);
            acc.w = __builtin_fmaf(e, x.w, acc.w);
        }
        pl[t] = acc;
    }
}

// out_t [b][vd][k] = (sum over chunks of plam[b][c][kk][j] * f_c) * (f32)(1 /
// sum over chunks of psum[b][c][kk] * f_c), f_c = exp(m_c - max over chunks of
// m_c): the chunk partials rescaled to the global column maximum. Block: kt
// key rows kk of one item. Per row one wave takes the chunks on its lanes
// (chunks <= 64): maximum and f_c, then the f64 sum of psum * f_c over a fixed
// shuffle tree; then every thread folds lambda over the chunks in order (f32).
__global__ __launch_bounds__(256) void lambda_finalize_kernel(const float *__restrict__ pmax,
                                                              const float *__restrict__ psum,
                                                              const float *__restrict__ plam, int k, int vd,
                                                              int chunks, int kt, float *__restrict__ out_t) {
    __shared__ float fs[64][64];  // [row in tile][chunk]
    __shared__ float sinv[64];
    const int b = blockIdx.y, kk0 = blockIdx.x * kt;
    const int nk = min(kt, k - kk0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = int(blockDim.x) >> 6;
    for (int r = wave; r < nk; r += waves) {
        const int kk = kk0 + r;
        const size_t o = (size_t(b) * chunks + lane) * k + kk;
        const float m = lane < chunks ? pmax[o] : -INFINITY;
        float mx = m;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        const float f = lane < chunks ? ref_exp(m - mx) : 0.0f;
        fs[r][lane] = f;
        double t = lane < chunks ? double(psum[o]) * double(f) : 0.0;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
        if (lane == 0) sinv[r] = float(1.0 / t);
    }
    __syncthreads();
    for (int t = threadIdx.x; t < nk * vd; t += blockDim.x) {
        const int r = t / vd, j = t - r * vd, kk = kk0 + r;
        const float *pl = plam + size_t(b) * chunks * size_t(k) * vd + size_t(kk) * vd + j;
        float acc = 0.0f;
#pragma unroll 8
        for (int c = 0; c < chunks; ++c) acc = __builtin_fmaf(pl[size_t(c) * k * vd], fs[r][c], acc);
        out_t[(size_t(b) * vd + j) * k + kk] = acc * sinv[r];
    }
}

// LayerNorm of the rows a kernel has just written, for kernels whose block
// holds whole pixel rows (src/engine/norm.rs:151-173: mean, then the mean of
// squared deviations, rstd = 1 / sqrt(var + eps), y = (v - mean) * rstd * g + b):
// thread t of a pixel holds HG float4 of the row; the per_px threads' sums are
// added in thread order through LDS, so the statistics are deterministic.
struct LnOut {
    const float *gamma = nullptr, *beta = nullptr;
    float eps = 0.f;
    float *out = nullptr;  // [pixels][c]
    // Instead of the LayerNorm: per pixel row, (sum, sum of squares) of the
    // values written, for a consumer that folds the LayerNorm itself.
    float2 *row_sums = nullptr;
};

// LayerNorm row partials of the rows a kernel has just written (LnOut::row_sums):
// thread r of a pixel's per_px threads sums its HG float4 in order; the
// threads' sums are added in chunks of 8 and the chunks in order through LDS
// (red: 2 * blockDim.x floats), so the partials are deterministic. Every
// thread of the block reaches both barriers.
template <int HG>
__device__ __forceinline__ void ln_pixel_sums(const LnOut &ln, const float4 (&u)[HG], bool active, float *red, int p,
                                              int per_px, int r, int64_t pix) {
    float s = 0.f, q = 0.f;
#pragma unroll
    for (int i = 0; i < HG; ++i) {
        s += u[i].x, s += u[i].y, s += u[i].z, s += u[i].w;
        q = __builtin_fmaf(u[i].x, u[i].x, q);
        q = __builtin_fmaf(u[i].y, u[i].y, q);
        q = __builtin_fmaf(u[i].z, u[i].z, q);
        q = __builtin_fmaf(u[i].w, u[i].w, q);
    }
    float2 *red2 = reinterpret_cast<float2 *>(red);
    red2[threadIdx.x] = active ? float2{s, q} : float2{0.f, 0.f};
    __syncthreads();
    const int nch = (per_px + 7) / 8;
    float2 cs{0.f, 0.f};
    if (active && r < nch) {
        const int j1 = min(per_px, 8 * r + 8);
        for (int j = 8 * r; j < j1; ++j) {
            const float2 v = red2[p * per_px + j];
            cs.x += v.x, cs.y += v.y;
        }
    }
    __syncthreads();
    if (active && r < nch) red2[p * per_px + r] = cs;
    __syncthreads();
    if (active && r == 0) {
        float2 t = red2[p * per_px];
        for (int j = 1; j < nch; ++j) {
            const float2 v = red2[p * per_px + j];
            t.x += v.x, t.y += v.y;
        }
        ln.row_sums[pix] = t;
    }
}

template <int HG>
__device__ __forceinline__ void ln_pixel_rows(const LnOut &ln, const float4 (&u)[HG], bool active, float *red, int p,
                                              int per_px, int c, int64_t pix, int hg, int jq, int k4) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < HG; ++i) s += (u[i].x + u[i].y) + (u[i].z + u[i].w);
    red[threadIdx.x] = active ? s : 0.f;
    __syncthreads();
    float tot = 0.f;
    if (active)
        for (int j = 0; j < per_px; ++j) tot += red[p * per_px + j];
    const float mean = tot / float(c);
    __syncthreads();  // every sum is read before the squares overwrite it
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < HG; ++i) {
        const float a = u[i].x - mean, b = u[i].y - mean, cc = u[i].z - mean, d = u[i].w - mean;
        q += (a * a + b * b) + (cc * cc + d * d);
    }
    red[threadIdx.x] = active ? q : 0.f;
    __syncthreads();
    if (!active) return;  // no barrier follows
    float vs = 0.f;
    for (int j = 0; j < per_px; ++j) vs += red[p * per_px + j];
    const float rstd = 1.0f / sqrtf(vs / float(c) + ln.eps);
    const float4 *g4 = reinterpret_cast<const float4 *>(ln.gamma);
    const float4 *b4 = reinterpret_cast<const float4 *>(ln.beta);
    float4 *o4 = reinterpret_cast<float4 *>(ln.out);
#pragma unroll
    for (int i = 0; i < HG; ++i) {
        const int q4 = (hg * HG + i) * k4 + jq;
        const float4 g = g4[q4], bb = b4[q4];
        float4 y;
        y.x = __builtin_fmaf((u[i].x - mean) * rstd, g.x, bb.x);
        y.y = __builtin_fmaf((u[i].y - mean) * rstd, g.y, bb.y);
        y.z = __builtin_fmaf((u[i].z - mean) * rstd, g.z, bb.z);
        y.w = __builtin_fmaf((u[i].w - mean) * rstd, g.w, bb.w);
        o4[pix * (kHeads * k4) + q4] = y;
    }
}

// HG heads' coefficients of one tap: a_t row [226][8] (heads innermost).
template <int HG>
__device__ __forceinline__ void load_heads(const float *__restrict__ p, float (&c)[HG]) {
    if constexpr (HG >= 4) {
#pragma unroll
        for (int i = 0; i < HG; i += 4) {
            const float4 t = *reinterpret_cast<const float4 *>(p + i);
            c[i] = t.x;
            c[i + 1] = t.y;
            c[i + 2] = t.z;
            c[i + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < HG; ++i) c[i] = p[i];
    }
}

// One thread per (pixel, head group of HG, 4 value channels): the value taps
// are loaded once and used for HG heads; the HG coefficients of a tap are one
// or two 16-byte loads from the tap-major a_t. Per output element the
// operations are the reference's: (yc + bias) then one fused multiply-add per
// in-image tap in (dy, dx) order; then residual + u when a residual is given.
// RS > 1: the 15 tap rows of an output are split over RS threads of one block
// (thread s of output o is threadIdx.x = s * opb + o, opb = blockDim.x / RS),
// which take consecutive row ranges; their sums are added in row order through
// LDS by the first, which then adds the residual. For maps whose pixel count
// leaves the chip under one wave per SIMD (the 32x32 and 16x16 latents), where
// one thread's 225 dependent taps expose the load latency. The sum then runs
// in three or five partial chains instead of one: f32-rounding close to the
// reference's order, no longer bit-identical to it.
template <int HG, bool LN, int RS = 1>
__global__ __launch_bounds__(256) void tap_filter_kernel(const float *__restrict__ a_t, const float *__restrict__ v,
                                                         const float *yc, const float *res, float *out, int nb,
                                                         int hh, int ww, int vd, LnOut ln) {
    constexpr int NG = kHeads / HG;
    const int v4 = vd >> 2;
    const int64_t total = int64_t(nb) * hh * ww * NG * v4;
    const int opb = int(blockDim.x) / RS;
    const int split = RS > 1 ? int(threadIdx.x) / opb : 0;
    const int lt = RS > 1 ? int(threadIdx.x) - split * opb : int(threadIdx.x);
    const int64_t t0 = int64_t(blockIdx.x) * opb + lt;
    const bool active = t0 < total && split < RS;
    // With the LayerNorm or a row split, a block is whole outputs (pixels with
    // the LayerNorm) and every thread stays for its barriers.
    if (!LN && RS == 1 && !active) return;
    const int64_t t = active ? t0 : 0;
    const int jq = int(t % v4);
    const int64_t r = t / v4;
    const int hg = int(r % NG);
    const int64_t pix = r / NG;  // b*hw + y*ww + x
    const int hw = hh * ww;
    const int b = int(pix / hw);
    const int rem = int(pix - int64_t(b) * hw);
    const int y = rem / ww, x = rem - (rem / ww) * ww;
    const float *ap = a_t + pix * (kTapsB * kHeads) + hg * HG;
    const int64_t obase = pix * (kHeads * v4) + int64_t(hg) * HG * v4 + jq;  // in float4 units
    float4 acc[HG];
    if (split == 0) {
        float bias[HG];
        load_heads<HG>(ap + kTaps * kHeads, bias);
#pragma unroll
        for (int i = 0; i < HG; ++i) {
            const float4 c = reinterpret_cast<const float4 *>(yc)[obase + i * v4];
            acc[i] = make_float4(c.x + bias[i], c.y + bias[i], c.z + bias[i], c.w + bias[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < HG; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float4 *vb = reinterpret_cast<const float4 *>(v + int64_t(b) * hw * vd) + jq;
    const int kx0 = max(kPad - x, 0), kx1 = min(kWin, ww + kPad - x);
    constexpr int RR = (kWin + RS - 1) / RS;  // tap rows per split
    const int ky0 = max(max(kPad - y, 0), split * RR), ky1 = min(min(kWin, hh + kPad - y), split * RR + RR);
    // A whole 15-tap row is loaded before any of it is used (the loads of a
    // thread overlap instead of queueing one tap at a time); columns outside the
    // image are loaded from a clamped, valid address and skipped in the sum.
    for (int ky = ky0; ky < ky1; ++ky) {
        const float4 *vr = vb + int64_t(y + ky - kPad) * ww * v4;
        const float *ar = ap + (ky * kWin) * kHeads;
        float c[kWin][HG];
        float4 s[kWin];
#pragma unroll
        for (int kx = 0; kx < kWin; ++kx) {
            const int ix = min(max(x + kx - kPad, 0), ww - 1);
            s[kx] = vr[int64_t(ix) * v4];
            load_heads<HG>(ar + kx * kHeads, c[kx]);
        }
#pragma unroll
        for (int kx = 0; kx < kWin; ++kx) {
            if (kx >= kx0 && kx < kx1) {
#pragma unroll
                for (int i = 0; i < HG; ++i) {
                    acc[i].x = __builtin_fmaf(c[kx][i], s[kx].x, acc[i].x);
                    acc[i].y = __builtin_fmaf(c[kx][i], s[kx].y, acc[i].y);
                    acc[i].z = __builtin_fmaf(c[kx][i], s[kx].z, acc[i].z);
                    acc[i].w = __builtin_fmaf(c[kx][i], s[kx].w, acc[i].w);
                }
            }
        }
    }
    extern __shared__ float red[];  // LN: [2 * blockDim.x]; RS > 1: then [RS - 1][opb][HG] float4
    if constexpr (RS > 1) {
        float4 *part = reinterpret_cast<float4 *>(red + (LN ? (2 * blockDim.x + 3) / 4 * 4 : 0));  // 16-byte aligned
        if (split > 0 && active)
#pragma unroll
            for (int i = 0; i < HG; ++i) part[((split - 1) * opb + lt) * HG + i] = acc[i];
        __syncthreads();
        if (split == 0 && active)
            for (int s2 = 1; s2 < RS; ++s2)
#pragma unroll
                for (int i = 0; i < HG; ++i) {
                    const float4 u = part[((s2 - 1) * opb + lt) * HG + i];
                    acc[i] = make_float4(acc[i].x + u.x, acc[i].y + u.y, acc[i].z + u.z, acc[i].w + u.w);
                }
    }
    const bool owner = active && split == 0;
    float4 *o4 = reinterpret_cast<float4 *>(out);
#pragma unroll
    for (int i = 0; i < HG; ++i) {
        if (res && owner) {
            const float4 h = reinterpret_cast<const float4 *>(res)[obase + i * v4];
            acc[i] = make_float4(h.x + acc[i].x, h.y + acc[i].y, h.z + acc[i].z, h.w + acc[i].w);
        }
        if (owner) o4[obase + i * v4] = acc[i];
    }
    if constexpr (LN) {
        const int tpp = NG * v4;
        if (ln.row_sums) ln_pixel_sums<HG>(ln, acc, owner, red, lt / tpp, tpp, lt % tpp, pix);
        else ln_pixel_rows<HG>(ln, acc, owner, red, lt / tpp, tpp, kHeads * vd, pix, hg, jq, v4);
    }
}

// Tap filter with LDS staging: a block takes tx consecutive pixels of one
// image row; its threads are (pixel, group of HG heads, channel quad). For each
// tap row (dy) the value row segment [x0 - 7, x0 + tx + 7) and the block's
// pixels' 15 x 8 coefficients of that row are staged into LDS with coalesced
// loads (double-buffered, one barrier per row), so the inner loop reads LDS
// only and every value and coefficient leaves HBM/L2 once per block. Per output
// element the operations are tap_filter_kernel's (the reference's order).
constexpr int kStageRegs = 4;  // float4 per thread of a staged value / coefficient row

// cq > 0: the block takes the value channel quads [cq * blockIdx.y, + cq) of its
// pixels only (LayerNorm row sums then per pixel and channel slice, LnOut
// row_sums [pixels][v4 / cq]; the full LayerNorm needs cq 0, whole rows).
template <int HG, bool LN, int JQ = 1>
__global__ __launch_bounds__(256) void tap_filter_tile_kernel(const float *__restrict__ a_t,
                                                              const float *__restrict__ v, const float *yc,
                                                              const float *res, float *out, int hh, int ww, int vd,
                                                              int tx, LnOut ln, int cq) {
    extern __shared__ float4 sh4[];
    constexpr int kRowC4 = kWin * kHeads / 4;  // float4 of coefficients per pixel and tap row: 30
    constexpr int NG = kHeads / HG;
    const int v4 = vd >> 2, cqn = cq > 0 ? cq : v4, q0 = cq > 0 ? int(blockIdx.y) * cq : 0;
    const int tpp = NG * (cqn / JQ), span = tx + kWin - 1;
    float4 *vls = sh4;                   // [2][span][cqn]
    float4 *cls = sh4 + 2 * span * cqn;  // [2][tx][30]
    const int tiles_x = (ww + tx - 1) / tx;
    const int bx = int(blockIdx.x % unsigned(tiles_x));
    const int row = int(blockIdx.x / unsigned(tiles_x));  // b * hh + y
    const int b = row / hh, y = row - b * hh;
    const int x0 = bx * tx, ntx = min(tx, ww - x0);
    const int xl = int(threadIdx.x) / tpp, r = int(threadIdx.x) - xl * tpp;
    const int hg = r / (cqn / JQ), jl = (r - hg * (cqn / JQ)) * JQ, jq = q0 + jl;  // JQ quads from jq
    const int x = x0 + xl;
    const bool active = xl < ntx;
    const int64_t pix0 = int64_t(row) * ww + x0, pix = pix0 + xl;
    const float4 *a4 = reinterpret_cast<const float4 *>(a_t);
    const int64_t o4 = pix * (kHeads * v4) + int64_t(hg) * HG * v4 + jq;  // output float4 of head hg*HG
    float4 acc[JQ * HG];  // acc[u * HG + i]: quad jq + u of head hg * HG + i
    if (active) {
        const float4 *yc4 = reinterpret_cast<const float4 *>(yc);
#pragma unroll
        for (int g = 0; g < HG / 4; ++g) {
            const float4 bias = a4[pix * (kTapsB * kHeads / 4) + (kTaps * kHeads) / 4 + hg * (HG / 4) + g];
            const float bb[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int u = 0; u < JQ; ++u) {
                    const float4 c = yc4[o4 + u + (g * 4 + i) * v4];
                    acc[u * HG + g * 4 + i] = make_float4(c.x + bb[i], c.y + bb[i], c.z + bb[i], c.w + bb[i]);
                }
        }
    }
    const int ky0 = max(kPad - y, 0), ky1 = min(kWin, hh + kPad - y);
    const int kx0 = max(kPad - x, 0), kx1 = min(kWin, ww + kPad - x);
    const float4 *vb = reinterpret_cast<const float4 *>(v) + int64_t(b) * hh * ww * v4;
    // Staging of tap row ky in two halves: load() issues the row's global loads
    // into registers (up to kStageRegs float4 per thread for the value row and
    // for the coefficient row), commit() writes them to LDS buffer buf, so the
    // loads of row ky + 1 land while row ky is computed.
    float4 sv[kStageRegs], sc[kStageRegs];
    auto load = [&](int ky) {
        const int iy = y + ky - kPad;
#pragma unroll
        for (int i = 0; i < kStageRegs; ++i) {
            const int t = int(threadIdx.x) + i * int(blockDim.x);
            const int c = t / cqn, q = t - c * cqn, ix = x0 - kPad + c;
            sv[i] = (t < span * cqn && ix >= 0 && ix < ww) ? vb[(int64_t(iy) * ww + ix) * v4 + q0 + q]
                                                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < kStageRegs; ++i) {
            const int t = int(threadIdx.x) + i * int(blockDim.x);
            const int p = t / kRowC4, w = t - p * kRowC4;
            sc[i] = t < ntx * kRowC4 ? a4[(pix0 + p) * (kTapsB * kHeads / 4) + ky * kRowC4 + w]
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    // commit() also copies directly whatever the registers do not hold (small
    // blocks whose rows exceed kStageRegs float4 per thread).
    auto commit = [&](int ky, int buf) {
        const int iy = y + ky - kPad, reg_end = kStageRegs * int(blockDim.x);
        float4 *vd4 = vls + buf * span * cqn;
#pragma unroll
        for (int i = 0; i < kStageRegs; ++i) {
            const int t = int(threadIdx.x) + i * int(blockDim.x);
            if (t < span * cqn) vd4[t] = sv[i];
        }
        for (int t = int(threadIdx.x) + reg_end; t < span * cqn; t += blockDim.x) {
            const int c = t / cqn, q = t - c * cqn, ix = x0 - kPad + c;
            vd4[t] = (ix >= 0 && ix < ww) ? vb[(int64_t(iy) * ww + ix) * v4 + q0 + q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float4 *cd4 = cls + buf * tx * kRowC4;
#pragma unroll
        for (int i = 0; i < kStageRegs; ++i) {
            const int t = int(threadIdx.x) + i * int(blockDim.x);
            if (t < ntx * kRowC4) cd4[t] = sc[i];
        }
        for (int t = int(threadIdx.x) + reg_end; t < ntx * kRowC4; t += blockDim.x) {
            const int p = t / kRowC4, w = t - p * kRowC4;
            cd4[t] = a4[(pix0 + p) * (kTapsB * kHeads / 4) + ky * kRowC4 + w];
        }
    };
    load(ky0);
    commit(ky0, 0);
    __syncthreads();
    for (int ky = ky0; ky < ky1; ++ky) {
        const int buf = (ky - ky0) & 1;
        const bool next = ky + 1 < ky1;
        if (next) load(ky + 1);
        if (active) {
            const float4 *vr = vls + buf * span * cqn + xl * cqn + jl;
            const float4 *cr = cls + buf * tx * kRowC4 + xl * kRowC4 + hg * (HG / 4);
#pragma unroll
            for (int kx = 0; kx < kWin; ++kx) {
                if (kx >= kx0 && kx < kx1) {
                    float cf[HG];
#pragma unroll
                    for (int g = 0; g < HG / 4; ++g) {
                        const float4 c4 = cr[kx * 2 + g];
                        cf[4 * g] = c4.x, cf[4 * g + 1] = c4.y, cf[4 * g + 2] = c4.z, cf[4 * g + 3] = c4.w;
                    }
#pragma unroll
                    for (int u = 0; u < JQ; ++u) {
                        const float4 s = vr[kx * cqn + u];
#pragma unroll
                        for (int i = 0; i < HG; ++i) {
                            float4 &a = acc[u * HG + i];
                            a.x = __builtin_fmaf(cf[i], s.x, a.x);
                            a.y = __builtin_fmaf(cf[i], s.y, a.y);
                            a.z = __builtin_fmaf(cf[i], s.z, a.z);
                            a.w = __builtin_fmaf(cf[i], s.w, a.w);
                        }
                    }
                }
            }
        }
        if (next) commit(ky + 1, buf ^ 1);
        __syncthreads();
    }
    if (active) {
        float4 *out4 = reinterpret_cast<float4 *>(out);
        const float4 *res4 = reinterpret_cast<const float4 *>(res);
#pragma unroll
        for (int u = 0; u < JQ; ++u)
#pragma unroll
            for (int i = 0; i < HG; ++i) {
                float4 &a = acc[u * HG + i];
                if (res) {
                    const float4 h = res4[o4 + u + i * v4];
                    a = make_float4(h.x + a.x, h.y + a.y, h.z + a.z, h.w + a.w);
                }
                out4[o4 + u + i * v4] = a;
            }
    }
    if constexpr (LN) {
        float *red = reinterpret_cast<float *>(cls + 2 * tx * kRowC4);  // [2 * blockDim.x]
        if (ln.row_sums) {
            const int nsl = v4 / cqn;
            ln_pixel_sums<JQ * HG>(ln, acc, active, red, xl, tpp, r, pix * nsl + int(blockIdx.y));
        } else if constexpr (JQ == 1) {
            ln_pixel_rows<HG>(ln, acc, active, red, xl, tpp, kHeads * vd, pix, hg, jq, v4);
        }
    }
}

// Position coefficients A = Q . W_aug (lambda.rs:131-137) written tap-major,
// a [pixel][226][8], and optionally the content term Yc = Q . lambda_c
// (lambda.rs:123), on the matrix cores. The general GEMM writes A, 7.2 KB per
// pixel, through a tile epilogue per 64x64 tile with K = 40 or 80, which
// leaves it at 1.5 TB/s. Here the 226 taps (padded to 240 = 15 row blocks of
// 16) are split in kTapParts parts of 80 (grid y), and Yc is one more part
// whose rows are the item's lambda_t [vd][k] (grid z: the item); a workgroup
// stages its part's rows in LDS once, and a wave computes the transposed
// product for two pixels (16 columns = 2 pixels x 8 heads) over the part's row
// blocks: register v of lane l is row 16 blk + 4 (l / 16) + v of column l % 16.
// The wave writes its results to its own LDS rows in the output's order, then
// stores each pixel's contiguous run with 16-byte stores. K runs in float4
// chunks of 16 (lane group g holds k = 16 f + 4 g + t for instruction t), then
// k % 16 in single instructions (k = 16 NF + 4 u + g). R16 (the FAST
// precision): every operand is rounded to f16 (nearest even, saturating at
// +-65504) as it is loaded, so the products are those of f16 operands, summed in
// f32 as the f16 GEMM does.
constexpr int kTapRows = 240;
// Rows per part (PR, the template argument): 80 (3 tap parts) where the map
// gives every SIMD several waves, 48 or 16 on the smaller maps, whose waves would
// otherwise each walk 80 rows in one MFMA chain after another.
template <int PR>
constexpr int tap_parts() { return kTapRows / PR; }
template <int PR>
constexpr int stage_ld() { return PR * kHeads + 8; }  // one pixel's staged run (+8: the two pixels on other banks)
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <bool R16>
__device__ __forceinline__ float op_round(float v) {
    if constexpr (R16) {
        const float x = __builtin_fabsf(v) > 65504.0f ? __builtin_copysignf(65504.0f, v) : v;
        return float(static_cast<_Float16>(x));
    } else {
        return v;
    }
}

template <bool R16>
__device__ __forceinline__ float4 op_round4(float4 v) {
    return make_float4(op_round<R16>(v.x), op_round<R16>(v.y), op_round<R16>(v.z), op_round<R16>(v.w));
}

template <int NF, int TAIL, bool R16, int PR>
__global__ __launch_bounds__(256) void lambda_taps_kernel(const float *__restrict__ q,
                                                          const float *__restrict__ w_aug_t,
                                                          const float *__restrict__ lam_t, int hw,
                                                          float *__restrict__ a, float *__restrict__ yc, int part0) {
    constexpr int K = 16 * NF + 4 * TAIL, K4 = K / 4;
    constexpr int WS = K + 4;  // LDS row stride: (K + 4) / 4 odd puts the 16 rows of a read on distinct banks
    constexpr int kPartRows = PR, kTapParts = tap_parts<PR>(), kStageLd = stage_ld<PR>();
    static_assert((WS / 4) % 2 == 1 && K % kPartRows % 4 == 0 && kTapRows % PR == 0 && PR % 16 == 0, "LDS layout");
    __shared__ float ws[kPartRows * WS];
    __shared__ float4 st4[4][2 * kStageLd / 4];  // per wave: two pixels' runs
    const int part = int(blockIdx.y) + part0, item = int(blockIdx.z);
    // parts past the taps: Yc, lambda_t's rows (value channels j) PR at a time
    const bool content = part >= kTapParts;
    const int r0 = (content ? part - kTapParts : part) * kPartRows;
    const int rows = min(kPartRows, (content ? K : kTapsB) - r0);  // valid rows of the part
    const float4 *src4 = reinterpret_cast<const float4 *>(content ? lam_t + int64_t(item) * K * K : w_aug_t) +
                         int64_t(r0) * K4;
    for (int i = threadIdx.x; i < kPartRows * K4; i += blockDim.x) {
        const int r = i / K4, c4 = i - r * K4;
        *reinterpret_cast<float4 *>(ws + r * WS + 4 * c4) =
            r < rows ? op_round4<R16>(src4[int64_t(r) * K4 + c4]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4, h = col & 7, pc = col >> 3;
    float *st = reinterpret_cast<float *>(st4[wave]);
    const int nblk = (rows + 15) >> 4;
    const int run = rows * kHeads;  // floats of a pixel's run in this part
    const int64_t px0 = int64_t(item) * hw;
    const int ntask = (hw + 1) >> 1, stride = int(gridDim.x) * 4;
    // Q of a task's 16 (pixel, head) rows: loaded one task ahead, so the loads
    // land while the previous task computes and stores
    floatx4 bq[NF > 0 ? NF : 1];
    float bt[TAIL > 0 ? TAIL : 1];
    auto load_q = [&](int task, floatx4(&fq)[NF > 0 ? NF : 1], float(&ft)[TAIL > 0 ? TAIL : 1]) {
        const int p = 2 * task + pc;
        const bool pv = task < ntask && p < hw;
        const float *qr = q + (pv ? ((px0 + p) * kHeads + h) * K : 0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            fq[f] = pv ? *reinterpret_cast<const floatx4 *>(qr + 16 * f + 4 * g) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) fq[f][t] = op_round<R16>(fq[f][t]);
        }
#pragma unroll
        for (int u = 0; u < TAIL; ++u) ft[u] = pv ? op_round<R16>(qr[16 * NF + 4 * u + g]) : 0.f;
    };
    int task = int(blockIdx.x) * 4 + wave;
    load_q(task, bq, bt);
    for (; task < ntask; task += stride) {
        floatx4 nq[NF > 0 ? NF : 1];
        float nt[TAIL > 0 ? TAIL : 1];
        load_q(task + stride, nq, nt);
        // the previous task's reads of st are done before it is rewritten
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int blk = 0; blk < kPartRows / 16; ++blk) {
            if (blk >= nblk) break;
            const float *wr = ws + (blk * 16 + col) * WS;
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const floatx4 aw = *reinterpret_cast<const floatx4 *>(wr + 16 * f + 4 * g);
#pragma unroll
                for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(aw[t], bq[f][t], acc, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < TAIL; ++u)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wr[16 * NF + 4 * u + g], bt[u], acc, 0, 0, 0);
            // A: [tap][head] per pixel; Yc: [head][channel] per pixel
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = blk * 16 + 4 * g + v;
                if (!content) st[pc * kStageLd + r * kHeads + h] = acc[v];
                else if (r < rows) st[pc * kStageLd + h * rows + r] = acc[v];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // A: one run of the pixel's row per part; Yc: eight runs (one per head) of
        // the part's rows values at channel r0
        const int run4 = run >> 2, seg4 = content ? rows >> 2 : run4;
        float *dst = content ? yc + r0 : a + r0 * kHeads;
        const int64_t pitch = content ? int64_t(kHeads) * K : int64_t(kTapsB) * kHeads;
        for (int i = lane; i < 2 * run4; i += 64) {
            const int p = i >= run4, j = i - p * run4;
            const int hh = j / seg4, j4 = j - hh * seg4;
            const int pp = 2 * task + p;
            if (pp < hw)
                *reinterpret_cast<float4 *>(dst + (px0 + pp) * pitch + hh * K + 4 * j4) =
                    *reinterpret_cast<const float4 *>(st + p * kStageLd + 4 * j);
        }
#pragma unroll
        for (int f = 0; f < NF; ++f) bq[f] = nq[f];
#pragma unroll
        for (int u = 0; u < TAIL; ++u) bt[u] = nt[u];
    }
}

// The self-lambda's position path in one pass (lambda.rs:123, 131-137 and
// 154-185): tap_filter_tile_kernel's row tiles, with the coefficients A and the
// content term Yc formed in the block on the matrix cores from Q, W_aug and
// lambda_t instead of read back from the [pixel][226][8] and [pixel][8][k]
// tensors lambda_taps_kernel writes (7.2 KB + 32 k bytes per pixel that would
// cross HBM twice). Wave w owns the block's pixel pairs w and w + 4 (16 MFMA
// columns = 2 pixels x 8 heads, their Q rows the B operand, held in registers
// for the whole block). First the content rows (lambda_t's, 16 at a time) and
// the bias row (W_aug row 225) go to LDS for the accumulators' start values;
// then per tap row the A operand is that row's 15 W_aug rows (one per lane row,
// read through the cache) and the products land in the LDS coefficient rows the
// tap loop reads, one tap row ahead of it. Each coefficient comes out of
// lambda_taps_kernel's instruction sequence (K in float4 chunks of 16 by lane
// group, then the tail) and each output of tap_filter_tile_kernel's tap order,
// so out and the row sums are bit-identical to those two kernels' (one thread
// per output). Blocks of 256 threads, tx <= 16 pixels (tx * 4 * k / 4 threads
// busy in the tap loop); RS: LayerNorm row sums per pixel (LnOut::row_sums).
template <int NF, int TAIL, bool R16, bool RS>
__global__ __launch_bounds__(256) void tap_fused_kernel(const float *__restrict__ q,
                                                        const float *__restrict__ w_aug_t,
                                                        const float *__restrict__ lam_t,
                                                        const float *__restrict__ v, const float *res, float *out,
                                                        int hh, int ww, int tx, LnOut ln) {
    constexpr int K = 16 * NF + 4 * TAIL, V4 = K / 4;
    constexpr int HG = 4, NG = kHeads / HG, TPP = NG * V4;  // threads per pixel
    constexpr int kRowC4 = kWin * kHeads / 4;               // float4 of one pixel's tap-row coefficients
    constexpr int NBJ = (K + 15) / 16;                      // 16-row blocks of lambda_t
    extern __shared__ float4 sh4[];
    const int span = tx + kWin - 1;
    float4 *vls = sh4;                                             // [2][span][V4]
    float *cls = reinterpret_cast<float *>(vls + 2 * span * V4);  // [2][tx][15][8]
    float *ycs = cls + 2 * tx * kRowC4 * 4;                        // [tx][8][K]
    float *bls = ycs + tx * kHeads * K;                            // [tx][8]
    float *red = bls + tx * kHeads;                                // row sums: [2 * 256]
    const int tiles_x = (ww + tx - 1) / tx;
    const int bx = int(blockIdx.x % unsigned(tiles_x));
    const int row = int(blockIdx.x / unsigned(tiles_x));  // b * hh + y
    const int b = row / hh, y = row - b * hh;
    const int x0 = bx * tx, ntx = min(tx, ww - x0);
    const int tid = int(threadIdx.x);
    const int xl = tid / TPP, r = tid - xl * TPP;
    const int hg = r / V4, jq = r - hg * V4;
    const int x = x0 + xl;
    const bool active = xl < ntx;
    const int64_t pix0 = int64_t(row) * ww + x0, pix = pix0 + xl;
    // matrix roles: lane (col, g) of wave w; column col = (pixel pc of the pair, head hc)
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, g = lane >> 4, hc = col & 7, pc = col >> 3;
    floatx4 bq[2][NF > 0 ? NF : 1];
    float bt[2][TAIL > 0 ? TAIL : 1];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int p = 2 * (wave + 4 * s) + pc;
        const bool pv = p < ntx;
        const float *qr = q + (pv ? ((pix0 + p) * kHeads + hc) * K : 0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            bq[s][f] = pv ? *reinterpret_cast<const floatx4 *>(qr + 16 * f + 4 * g) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) bq[s][f][t] = op_round<R16>(bq[s][f][t]);
        }
#pragma unroll
        for (int u = 0; u < TAIL; ++u) bt[s][u] = pv ? op_round<R16>(qr[16 * NF + 4 * u + g]) : 0.f;
    }
    // One 16-row product for each of this wave's pixel pairs: the A operand is
    // row `arow` of src (K wide) per lane row, zeros where arow is past rows;
    // load_a fetches it (ahead of use for the tap rows), products runs the
    // pairs' MFMA chains, interleaved when the wave has two.
    struct AOp {
        floatx4 w[NF > 0 ? NF : 1];
        float t[TAIL > 0 ? TAIL : 1];
    };
    auto load_a = [&](const float *src, int arow, int rows, AOp &o) {
        const bool av = arow < rows;
        const float *ar = src + (av ? int64_t(arow) * K : 0);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            o.w[f] = av ? *reinterpret_cast<const floatx4 *>(ar + 16 * f + 4 * g) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) o.w[f][t] = op_round<R16>(o.w[f][t]);
        }
#pragma unroll
        for (int u = 0; u < TAIL; ++u) o.t[u] = av ? op_round<R16>(ar[16 * NF + 4 * u + g]) : 0.f;
    };
    // The MFMA chains of this wave's two pixel pairs (step i: K chunk f = i / 4,
    // instruction t = i % 4, then the tail), so they can be spread over other
    // work; a pair past the row's pixels multiplies zeros and is not stored.
    constexpr int kSteps = 4 * NF + TAIL;
    floatx4 pacc[2];
    auto mfma_step = [&](const AOp &o, int i) {
        if (i < 4 * NF) {
            const int f = i >> 2, t = i & 3;
            pacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.w[f][t], bq[0][f][t], pacc[0], 0, 0, 0);
            pacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.w[f][t], bq[1][f][t], pacc[1], 0, 0, 0);
        } else {
            const int u = i - 4 * NF;
            pacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.t[u], bt[0][u], pacc[0], 0, 0, 0);
            pacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.t[u], bt[1][u], pacc[1], 0, 0, 0);
        }
    };
    auto products = [&](const AOp &o) {
        pacc[0] = pacc[1] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < kSteps; ++i) mfma_step(o, i);
    };
    // Content rows j and the bias row into LDS (register v of lane (col, g): row 4 g + v).
    const float *lamb = lam_t + int64_t(b) * K * K;
#pragma unroll
    for (int jb = 0; jb < NBJ; ++jb) {
        AOp o;
        load_a(lamb, 16 * jb + col, K, o);
        products(o);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int p = 2 * (wave + 4 * s) + pc;
            if (p >= ntx) continue;
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int j = 16 * jb + 4 * g + vv;
                if (j < K) ycs[(p * kHeads + hc) * K + j] = pacc[s][vv];
            }
        }
    }
    {
        AOp o;
        load_a(w_aug_t, kTaps, kTapsB, o);  // every lane row: W_aug row 225, the bias
        products(o);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int p = 2 * (wave + 4 * s) + pc;
        if (p < ntx && g == 0) bls[p * kHeads + hc] = pacc[s][0];
    }
    __syncthreads();
    float4 acc[HG];
    if (active) {
#pragma unroll
        for (int i = 0; i < HG; ++i) {
            const int hd = hg * HG + i;
            const float4 c = *reinterpret_cast<const float4 *>(ycs + (xl * kHeads + hd) * K + 4 * jq);
            const float bb = bls[xl * kHeads + hd];
            acc[i] = make_float4(c.x + bb, c.y + bb, c.z + bb, c.w + bb);
        }
    }
    const int ky0 = max(kPad - y, 0), ky1 = min(kWin, hh + kPad - y);
    const int kx0 = max(kPad - x, 0), kx1 = min(kWin, ww + kPad - x);
    const float4 *vb = reinterpret_cast<const float4 *>(v) + int64_t(b) * hh * ww * V4;
    // value rows: registers then LDS, as tap_filter_tile_kernel stages them
    float4 sv[kStageRegs];
    auto load_v = [&](int ky) {
        const int iy = y + ky - kPad;
#pragma unroll
        for (int i = 0; i < kStageRegs; ++i) {
            const int t = tid + i * 256;
            const int c = t / V4, qd = t - c * V4, ix = x0 - kPad + c;
            sv[i] = (t < span * V4 && ix >= 0 && ix < ww) ? vb[(int64_t(iy) * ww + ix) * V4 + qd]
                                                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto commit_v = [&](int ky, int buf) {
        const int iy = y + ky - kPad;
        float4 *vd4 = vls + buf * span * V4;
#pragma unroll
        for (int i = 0; i < kStageRegs; ++i) {
            const int t = tid + i * 256;
            if (t < span * V4) vd4[t] = sv[i];
        }
        for (int t = tid + kStageRegs * 256; t < span * V4; t += 256) {
            const int c = t / V4, qd = t - c * V4, ix = x0 - kPad + c;
            vd4[t] = (ix >= 0 && ix < ww) ? vb[(int64_t(iy) * ww + ix) * V4 + qd] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    // the coefficients of tap row ky (taps 15 ky + kx, lane row kx; row 15 of the
    // tile is W_aug row 15 ky + 15, computed and dropped) into LDS buffer buf
    auto put_coeffs = [&](int buf) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int p = 2 * (wave + 4 * s) + pc;
            if (p >= ntx) continue;
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int kx = 4 * g + vv;
                if (kx < kWin) cls[((buf * tx + p) * kWin + kx) * kHeads + hc] = pacc[s][vv];
            }
        }
    };
    // W_aug rows of the next tap row: loaded one row ahead; their products run
    // step by step inside the tap loop of the row before and go to LDS after it.
    AOp wn;
    load_v(ky0);
    load_a(w_aug_t, ky0 * kWin + col, kTapsB, wn);
    products(wn);
    if (ky0 + 1 < ky1) load_a(w_aug_t, (ky0 + 1) * kWin + col, kTapsB, wn);
    put_coeffs(0);
    commit_v(ky0, 0);
    __syncthreads();
    for (int ky = ky0; ky < ky1; ++ky) {
        const int buf = (ky - ky0) & 1;
        const bool next = ky + 1 < ky1;  // block-uniform
        if (next) load_v(ky + 1);
        pacc[0] = pacc[1] = floatx4{0.f, 0.f, 0.f, 0.f};
        // Tap column kx of row ky, then MFMA step kx of row ky + 1's products:
        // the matrix unit works beside the FMAs (one step per column, the
        // steps past column 15 after the loop).
        const float4 *vr = vls + buf * span * V4 + xl * V4 + jq;
        const float4 *cr = reinterpret_cast<const float4 *>(cls) + (buf * tx + xl) * kRowC4 + hg;
#pragma unroll
        for (int kx = 0; kx < kWin; ++kx) {
            if (active && kx >= kx0 && kx < kx1) {
                const float4 c4 = cr[kx * 2];
                const float cf[4] = {c4.x, c4.y, c4.z, c4.w};
                const float4 sx = vr[kx * V4];
#pragma unroll
                for (int i = 0; i < HG; ++i) {
                    acc[i].x = __builtin_fmaf(cf[i], sx.x, acc[i].x);
                    acc[i].y = __builtin_fmaf(cf[i], sx.y, acc[i].y);
                    acc[i].z = __builtin_fmaf(cf[i], sx.z, acc[i].z);
                    acc[i].w = __builtin_fmaf(cf[i], sx.w, acc[i].w);
                }
            }
            if (next && kx < kSteps) mfma_step(wn, kx);
        }
        if (next) {
#pragma unroll
            for (int i = kWin; i < kSteps; ++i) mfma_step(wn, i);
            if (ky + 2 < ky1) load_a(w_aug_t, (ky + 2) * kWin + col, kTapsB, wn);
            put_coeffs(buf ^ 1);
            commit_v(ky + 1, buf ^ 1);
        }
        __syncthreads();
    }
    if (active) {
        float4 *out4 = reinterpret_cast<float4 *>(out);
        const float4 *res4 = reinterpret_cast<const float4 *>(res);
        const int64_t o4 = pix * (kHeads * V4) + int64_t(hg) * HG * V4 + jq;
#pragma unroll
        for (int i = 0; i < HG; ++i) {
            if (res) {
                const float4 h = res4[o4 + i * V4];
                acc[i] = make_float4(h.x + acc[i].x, h.y + acc[i].y, h.z + acc[i].z, h.w + acc[i].w);
            }
            out4[o4 + i * V4] = acc[i];
        }
    }
    if constexpr (RS) ln_pixel_sums<HG>(ln, acc, active, red, xl, TPP, r, pix);
}

// 8-lane dot of src/unet/lambda.rs:297-309 (k a multiple of 8).
__device__ __forceinline__ float dot8_ref(const float *__restrict__ a, const float *__restrict__ b, int k) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < k; i += 8) {
        const float4 a0 = *reinterpret_cast<const float4 *>(a + i), a1 = *reinterpret_cast<const float4 *>(a + i + 4);
        const float4 b0 = *reinterpret_cast<const float4 *>(b + i), b1 = *reinterpret_cast<const float4 *>(b + i + 4);
        acc[0] = __builtin_fmaf(a0.x, b0.x, acc[0]);
        acc[1] = __builtin_fmaf(a0.y, b0.y, acc[1]);
        acc[2] = __builtin_fmaf(a0.z, b0.z, acc[2]);
        acc[3] = __builtin_fmaf(a0.w, b0.w, acc[3]);
        acc[4] = __builtin_fmaf(a1.x, b1.x, acc[4]);
        acc[5] = __builtin_fmaf(a1.y, b1.y, acc[5]);
        acc[6] = __builtin_fmaf(a1.z, b1.z, acc[6]);
        acc[7] = __builtin_fmaf(a1.w, b1.w, acc[7]);
    }
    float s = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) s += acc[l];
    return s + 0.0f;
}

// Block of 256 threads handles 8 pixels. q, yc, res, out: [b*hw][8*k]; e: [hw][10][k];
// vb: [2][10][k] (per branch); branch of item b = br0 + b. out may alias yc or res.
__global__ __launch_bounds__(256) void position_term_kernel(const float *__restrict__ q, const float *__restrict__ e,
                                                            const float *__restrict__ vbr, int br0, int nb, int hw,
                                                            int k, const float *yc, const float *res, float *out) {
    constexpr int P = 8;
    __shared__ float bm[P][kHeads][kTokens];
    const int64_t pix0 = int64_t(blockIdx.x) * P;
    const int64_t npix = int64_t(nb) * hw;
    const int c = kHeads * k;
    for (int i = threadIdx.x; i < P * kHeads * kTokens; i += 256) {
        const int p = i / (kHeads * kTokens), hm = i - p * (kHeads * kTokens);
        const int h = hm / kTokens, m = hm - h * kTokens;
        const int64_t pix = pix0 + p;
        float val = 0.0f;
        if (pix < npix) {
            const int n = int(pix % hw);
            val = dot8_ref(q + pix * c + h * k, e + (int64_t(n) * kTokens + m) * k, k);
        }
        bm[p][h][m] = val;
    }
    __syncthreads();
    // (pixel, head, 4 channels) per step: float4 loads and stores, each
    // component summed in the reference's order.
    const int k4 = k >> 2;
    const float4 *yc4 = reinterpret_cast<const float4 *>(yc);
    const float4 *res4 = reinterpret_cast<const float4 *>(res);
    float4 *out4 = reinterpret_cast<float4 *>(out);
    for (int i = threadIdx.x; i < P * kHeads * k4; i += 256) {
        const int p = i / (kHeads * k4), hq = i - p * (kHeads * k4);
        const int h = hq / k4, jq = hq - h * k4;
        const int64_t pix = pix0 + p;
        if (pix >= npix) continue;
        const int b = int(pix / hw);
        const float4 *vm = reinterpret_cast<const float4 *>(vbr + int64_t(br0 + b) * kTokens * k) + jq;
        const int64_t o = pix * (kHeads * k4) + hq;
        float4 acc = yc4[o];
#pragma unroll
        for (int m = 0; m < kTokens; ++m) {
            const float w = bm[p][h][m];
            const float4 x = vm[m * k4];
            acc.x = __builtin_fmaf(w, x.x, acc.x);
            acc.y = __builtin_fmaf(w, x.y, acc.y);
            acc.z = __builtin_fmaf(w, x.z, acc.z);
            acc.w = __builtin_fmaf(w, x.w, acc.w);
        }
        if (res) {
            const float4 r = res4[o];
            acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
        }
        out4[o] = acc;
    }
}

// Cross-lambda output (src/unet/lambda.rs:258-271) in one pass per pixel: Yc =
// Q . lambda_c[branch] (a fused multiply-add chain over kk), then the position
// term as position_term_kernel computes it (8-lane dots q_h . E[n][m], then
// o_h += B[h][m] * V[m] for m = 0..9 in order), then the block's residual. The
// block's pixels' q is staged in LDS transposed ([p][kk][h]) so a thread reads
// its HG heads of one kk in one or two 16-byte loads; lambda_c rows are shared
// by every thread with the same channel quad. Thread: (pixel, head group,
// channel quad); P pixels per block. lam: [2][k][k] row-major (lambda_c[kk][j]).
template <int HG>
__global__ __launch_bounds__(256) void cross_lambda_kernel(const float *__restrict__ q, const float *__restrict__ e,
                                                           const float *__restrict__ lam,
                                                           const float *__restrict__ vbr, int br0, int nb, int hw,
                                                           int k, int P, const float *res, float *out,
                                                           float2 *__restrict__ row_sums) {
    extern __shared__ float sm[];
    const int c = kHeads * k;
    float *qs = sm;                  // [P][k][8]
    float *bm = sm + size_t(P) * c;  // [P][8][10]
    const int64_t pix0 = int64_t(blockIdx.x) * P;
    const int np = int(min<int64_t>(P, int64_t(nb) * hw - pix0));
    const float4 *q4 = reinterpret_cast<const float4 *>(q + pix0 * c);
    for (int t = threadIdx.x; t < np * (c >> 2); t += blockDim.x) {
        const int r = t * 4, p = r / c, hk = r - p * c, h = hk / k, kk = hk - h * k;  // k % 4 == 0
        const float4 v = q4[t];
        float *d = qs + (size_t(p) * k + kk) * kHeads + h;
        d[0] = v.x, d[kHeads] = v.y, d[2 * kHeads] = v.z, d[3 * kHeads] = v.w;
    }
    __syncthreads();
    // B[p][h][m] = q_h . E[n][m]: one (pixel, token, group of HG heads) per
    // thread and pass; per head the reference's 8-lane dot (acc[l] takes
    // kk = l, l + 8, ...; the lanes summed in order).
    constexpr int NG = kHeads / HG;
    for (int t = threadIdx.x; t < np * kTokens * NG; t += blockDim.x) {
        const int p = t / (kTokens * NG), mg = t - p * (kTokens * NG), m = mg / NG, g = mg - m * NG;
        const int n = int((pix0 + p) % hw);
        const float4 *e4 = reinterpret_cast<const float4 *>(e + (int64_t(n) * kTokens + m) * k);
        const float *qp = qs + size_t(p) * k * kHeads + g * HG;
        float acc[HG][8];
#pragma unroll
        for (int h = 0; h < HG; ++h)
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[h][l] = 0.f;
        for (int i = 0; i < k; i += 8) {
            const float4 ea = e4[i >> 2], eb = e4[(i >> 2) + 1];
            const float ev[8] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                float qv[HG];
                if constexpr (HG >= 4) {
#pragma unroll
                    for (int h = 0; h < HG; h += 4) {
                        const float4 t4 = *reinterpret_cast<const float4 *>(qp + (i + l) * kHeads + h);
                        qv[h] = t4.x, qv[h + 1] = t4.y, qv[h + 2] = t4.z, qv[h + 3] = t4.w;
                    }
                } else {
                    const float2 t2 = *reinterpret_cast<const float2 *>(qp + (i + l) * kHeads);
                    qv[0] = t2.x, qv[1] = t2.y;
                }
#pragma unroll
                for (int h = 0; h < HG; ++h) acc[h][l] = __builtin_fmaf(qv[h], ev[l], acc[h][l]);
            }
        }
#pragma unroll
        for (int h = 0; h < HG; ++h) {
            float sum = 0.0f;
#pragma unroll
            for (int l = 0; l < 8; ++l) sum += acc[h][l];
            bm[(p * kHeads + g * HG + h) * kTokens + m] = sum + 0.0f;
        }
    }
    __syncthreads();
    const int k4 = k >> 2, per_px = NG * k4;
    const int p = threadIdx.x / per_px;
    // Threads past the block's pixels return here unless the row sums' barriers follow.
    if (p >= np && !row_sums) return;
    const int pc = min(p, np - 1);  // (a past-the-end thread computes a real pixel's values, unused)
    const int r = threadIdx.x - p * per_px, hg = r / k4, jq = r - hg * k4;
    const int64_t pix = pix0 + pc;
    const int br = br0 + int(pix / hw);
    const float4 *l4 = reinterpret_cast<const float4 *>(lam + int64_t(br) * k * k) + jq;
    const float *qp = qs + size_t(pc) * k * kHeads + hg * HG;
    float4 acc[HG];
#pragma unroll
    for (int i = 0; i < HG; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int kk = 0; kk < k; ++kk) {
        const float4 l = l4[kk * k4];
        float qv[HG];
        if constexpr (HG >= 4) {
#pragma unroll
            for (int i = 0; i < HG; i += 4) {
                const float4 t4 = *reinterpret_cast<const float4 *>(qp + kk * kHeads + i);
                qv[i] = t4.x, qv[i + 1] = t4.y, qv[i + 2] = t4.z, qv[i + 3] = t4.w;
            }
        } else {
            const float2 t2 = *reinterpret_cast<const float2 *>(qp + kk * kHeads);
            qv[0] = t2.x, qv[1] = t2.y;
        }
#pragma unroll
        for (int i = 0; i < HG; ++i) {
            acc[i].x = __builtin_fmaf(qv[i], l.x, acc[i].x);
            acc[i].y = __builtin_fmaf(qv[i], l.y, acc[i].y);
            acc[i].z = __builtin_fmaf(qv[i], l.z, acc[i].z);
            acc[i].w = __builtin_fmaf(qv[i], l.w, acc[i].w);
        }
    }
    const float4 *v4 = reinterpret_cast<const float4 *>(vbr + int64_t(br) * kTokens * k) + jq;
    const float *bp = bm + (size_t(pc) * kHeads + hg * HG) * kTokens;
#pragma unroll
    for (int m = 0; m < kTokens; ++m) {
        const float4 x = v4[m * k4];
#pragma unroll
        for (int i = 0; i < HG; ++i) {
            const float w = bp[i * kTokens + m];
            acc[i].x = __builtin_fmaf(w, x.x, acc[i].x);
            acc[i].y = __builtin_fmaf(w, x.y, acc[i].y);
            acc[i].z = __builtin_fmaf(w, x.z, acc[i].z);
            acc[i].w = __builtin_fmaf(w, x.w, acc[i].w);
        }
    }
    const float4 *res4 = reinterpret_cast<const float4 *>(res);
    float4 *out4 = reinterpret_cast<float4 *>(out);
#pragma unroll
    for (int i = 0; i < HG; ++i) {
        const int64_t o = pix * (kHeads * k4) + int64_t(hg * HG + i) * k4 + jq;
        float4 u = acc[i];
        if (res) {
            const float4 rr = res4[o];
            u = make_float4(rr.x + u.x, rr.y + u.y, rr.z + u.z, rr.w + u.w);
        }
        if (p < np) out4[o] = u;
        acc[i] = u;
    }
    if (!row_sums) return;
    // LayerNorm row partials of the written rows: this thread's (sum, sum of
    // squares) over its values in order, then per pixel the threads' in order,
    // in chunks of 8 and the chunks in order (through LDS past q and B).
    float2 *red = reinterpret_cast<float2 *>(sm + size_t(P) * (kHeads * k + kHeads * kTokens));
    float ls = 0.f, lq = 0.f;
#pragma unroll
    for (int i = 0; i < HG; ++i) {
        ls += acc[i].x, ls += acc[i].y, ls += acc[i].z, ls += acc[i].w;
        lq = __builtin_fmaf(acc[i].x, acc[i].x, lq);
        lq = __builtin_fmaf(acc[i].y, acc[i].y, lq);
        lq = __builtin_fmaf(acc[i].z, acc[i].z, lq);
        lq = __builtin_fmaf(acc[i].w, acc[i].w, lq);
    }
    red[threadIdx.x] = float2{ls, lq};
    __syncthreads();
    const int nch = (per_px + 7) / 8;
    float2 cs{0.f, 0.f};
    if (p < np && r < nch) {
        const int j1 = min(per_px, 8 * r + 8);
        for (int j = 8 * r; j < j1; ++j) {
            const float2 v = red[p * per_px + j];
            cs.x += v.x, cs.y += v.y;
        }
    }
    __syncthreads();
    if (p < np && r < nch) red[p * per_px + r] = cs;
    __syncthreads();
    if (p < np && r == 0) {
        float2 t = red[p * per_px];
        for (int j = 1; j < nch; ++j) {
            const float2 v = red[p * per_px + j];
            t.x += v.x, t.y += v.y;
        }
        row_sums[pix] = t;
    }
}

// Cross-lambda output with the content term on the matrix cores: Yc =
// Q . lambda_c[branch] as 16x16x4 f32 MFMA products, rows (pixel, head) and
// columns the value channels j; then per output, as cross_lambda_kernel, the
// position term added in the reference's order (o += B[h][m] * V[m] for m =
// 0..9 with fused multiply-adds, B the 8-lane dots q_h . E[n][m]) and the
// residual. A block takes P pixels of one item (so one branch) and stages
// their q and E rows in LDS first, every load in flight at once; phase 1 forms
// B from LDS; then each wave takes (pixel pair, 16 value channels) tasks: lane
// (i = l % 16, g = l / 16) supplies q[pixel 2rb + i / 8][head i % 8][kk] and
// lambda_c[kk][16cb + i] for kk = 16f + 4g + t (instruction t of chunk f), then
// kk = 16NF + 4u + g, its lambda_c values loaded before the first product;
// register v of lane l then holds row 4g + v, column l % 16. With lambda_c = 0
// the products sum to +0 and the output is the position term's exactly.
// row_sums (optional): LayerNorm row partials of the written rows, per lane
// over its four rows of one pixel, across the 16 column lanes by an xor
// butterfly, then per pixel over the column blocks and head halves in order.
template <int K>
__device__ __forceinline__ float dot8_lds(const float *a, const float *b) {  // dot8_ref's operations
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < K; i += 8) {
        const float4 a0 = *reinterpret_cast<const float4 *>(a + i), a1 = *reinterpret_cast<const float4 *>(a + i + 4);
        const float4 b0 = *reinterpret_cast<const float4 *>(b + i), b1 = *reinterpret_cast<const float4 *>(b + i + 4);
        acc[0] = __builtin_fmaf(a0.x, b0.x, acc[0]);
        acc[1] = __builtin_fmaf(a0.y, b0.y, acc[1]);
        acc[2] = __builtin_fmaf(a0.z, b0.z, acc[2]);
        acc[3] = __builtin_fmaf(a0.w, b0.w, acc[3]);
        acc[4] = __builtin_fmaf(a1.x, b1.x, acc[4]);
        acc[5] = __builtin_fmaf(a1.y, b1.y, acc[5]);
        acc[6] = __builtin_fmaf(a1.z, b1.z, acc[6]);
        acc[7] = __builtin_fmaf(a1.w, b1.w, acc[7]);
    }
    float s = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) s += acc[l];
    return s + 0.0f;
}

template <int NF, int TAIL, int P, int NT>
__global__ __launch_bounds__(NT) void cross_lambda_mfma_kernel(const float *__restrict__ q,
                                                                const float *__restrict__ e,
                                                                const float *__restrict__ lam,
                                                                const float *__restrict__ vbr, int br0, int hw,
                                                                const float *res, float *out,
                                                                float2 *__restrict__ row_sums) {
    constexpr int K = 16 * NF + 4 * TAIL, K4 = K / 4, NCB = (K + 15) / 16, RB = (P + 1) / 2, TASKS = RB * NCB;
    constexpr int QF4 = P * kHeads * K4, EF4 = P * kTokens * K4, VF4 = kTokens * K4, SF4 = QF4 + EF4 + VF4;
    constexpr int PER = (SF4 + NT - 1) / NT;
    static_assert(K % 8 == 0, "8-lane dots over whole chunks");
    __shared__ float4 stage[SF4];  // q [P][8][K], then E [P][10][K], then the branch's V [10][K]
    __shared__ float bm[P][kHeads][kTokens];
    __shared__ float2 part[P][NCB][2];
    const int item = int(blockIdx.y);
    const int p0 = int(blockIdx.x) * P;
    const int np = min(P, hw - p0);
    const int64_t pix0 = int64_t(item) * hw + p0;
    const int br = br0 + item;
    {
        const float4 *q4 = reinterpret_cast<const float4 *>(q) + pix0 * (kHeads * K4);
        const float4 *e4 = reinterpret_cast<const float4 *>(e) + int64_t(p0) * (kTokens * K4);
        const float4 *v4 = reinterpret_cast<const float4 *>(vbr) + int64_t(br) * VF4;
        float4 r[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int t = int(threadIdx.x) + NT * i;
            r[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < QF4) {
                if (t / (kHeads * K4) < np) r[i] = q4[t];
            } else if (t < QF4 + EF4) {
                if ((t - QF4) / (kTokens * K4) < np) r[i] = e4[t - QF4];
            } else if (t < SF4) {
                r[i] = v4[t - QF4 - EF4];
            }
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int t = int(threadIdx.x) + NT * i;
            if (t < SF4) stage[t] = r[i];
        }
    }
    __syncthreads();
    const float *qs = reinterpret_cast<const float *>(stage);
    const float *es = qs + QF4 * 4;
    const float *vs = es + EF4 * 4;
    // phase 1: B[p][h][m] = q_h . E[n][m] (the reference's 8-lane dot)
    for (int t = threadIdx.x; t < P * kHeads * kTokens; t += blockDim.x) {
        const int p = t / (kHeads * kTokens), hm = t - p * (kHeads * kTokens);
        const int h = hm / kTokens, m = hm - h * kTokens;
        bm[p][h][m] = p < np ? dot8_lds<K>(qs + (p * kHeads + h) * K, es + (p * kTokens + m) * K) : 0.f;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = int(blockDim.x) >> 6;
    const int col = lane & 15, g = lane >> 4;
    const float *lb = lam + int64_t(br) * K * K;
    for (int task = wave; task < TASKS; task += nwaves) {
        const int rb = task / NCB, cb = task - rb * NCB;
        const int pa = 2 * rb + (col >> 3), ha = col & 7;  // this lane's A row: pixel, head
        const float *qa = qs + (min(pa, P - 1) * kHeads + ha) * K;  // (rows past np read staged zeros)
        const int jb = 16 * cb + col;                              // this lane's B column
        const bool bv = jb < K;
        // epilogue: lane (col, g) holds rows 4g..4g+3 (one pixel, heads 4(g&1)..+3) of column jb;
        // its residuals load with the task's lambda_c values, before the products
        const int pd = 2 * rb + (g >> 1);
        const bool ok = pd < np && bv;
        const int64_t obase = ((pix0 + pd) * kHeads + 4 * (g & 1)) * K + jb;
        float rv[4] = {0.f, 0.f, 0.f, 0.f};
        if (ok && res)
#pragma unroll
            for (int v = 0; v < 4; ++v) rv[v] = res[obase + v * K];
        float bf[NF > 0 ? NF : 1][4], bt[TAIL > 0 ? TAIL : 1];
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int t = 0; t < 4; ++t) bf[f][t] = bv ? lb[int64_t(16 * f + 4 * g + t) * K + jb] : 0.f;
#pragma unroll
        for (int u = 0; u < TAIL; ++u) bt[u] = bv ? lb[int64_t(16 * NF + 4 * u + g) * K + jb] : 0.f;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const float4 a4 = *reinterpret_cast<const float4 *>(qa + 16 * f + 4 * g);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, bf[f][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, bf[f][1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, bf[f][2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, bf[f][3], acc, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < TAIL; ++u)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[16 * NF + 4 * u + g], bt[u], acc, 0, 0, 0);
        float ls = 0.f, lq = 0.f;
        if (ok) {
            float vv[kTokens];  // V[m][jb], read once for the four rows
#pragma unroll
            for (int m = 0; m < kTokens; ++m) vv[m] = vs[m * K + jb];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int h = 4 * (g & 1) + v;
                float o = acc[v];
#pragma unroll
                for (int m = 0; m < kTokens; ++m) o = __builtin_fmaf(bm[pd][h][m], vv[m], o);
                const int64_t idx = obase + v * K;
                const float u = res ? rv[v] + o : o;
                out[idx] = u;
                ls += u;
                lq = __builtin_fmaf(u, u, lq);
            }
        }
        if (row_sums) {
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                ls += __shfl_xor(ls, off, 64);
                lq += __shfl_xor(lq, off, 64);
            }
            if (col == 0 && pd < P) part[pd][cb][g & 1] = float2{ls, lq};
        }
    }
    if (!row_sums) return;
    __syncthreads();
    if (int(threadIdx.x) < np) {
        const int p = threadIdx.x;
        float2 t{0.f, 0.f};
        for (int cb = 0; cb < NCB; ++cb)
            for (int half = 0; half < 2; ++half) {
                const float2 v = part[p][cb][half];
                t.x += v.x, t.y += v.y;
            }
        row_sums[pix0 + p] = t;
    }
}

}  // namespace

void softmax_lambda(Context &ctx, const float *keys, const float *v, int nb, int rows, int k, int vd,
                    float *lambda_t) {
    MH_REQUIRE(k > 0 && k <= 256 && vd > 0 && vd <= 256, "softmax_lambda: widths above 256 are not supported");
    MH_REQUIRE(k % 4 == 0 && vd % 4 == 0, "softmax_lambda: widths must be multiples of 4");
    MH_REQUIRE(aligned16(keys) && aligned16(v), "softmax_lambda: keys and v must be 16-byte aligned");
    MH_REQUIRE(rows > 0 && nb > 0, "softmax_lambda: empty input");
    const LambdaSplit sp = lambda_split(rows, k, vd);
    MH_REQUIRE(sp.chunks <= 64, "softmax_lambda: at most 64 x 128 rows per item");
    const size_t pm = size_t(nb) * sp.chunks * k;
    const size_t pl = size_t(nb) * sp.chunks * size_t(k) * vd;
    float *ws = static_cast<float *>(ctx.ws.get((2 * pm + pl) * sizeof(float), ctx.stream));
    float *pmax = ws, *psum = ws + pm, *plam = ws + 2 * pm;
    const size_t lds = (size_t(sp.ch) * (sp.tk + vd) + 256) * sizeof(float);
    lambda_partial_kernel<<<dim3(sp.chunks, nb, sp.ktiles), 256, lds, ctx.stream>>>(
        keys, v, rows, k, vd, sp.ch, sp.chunks, sp.tk, pmax, psum, plam);
    MH_LAUNCH_CHECK();
    const int kt = std::max(1, std::min(64, 256 / vd));
    const unsigned threads = unsigned(std::max(64, std::min(256, int(ceil_div(kt * vd, 64)) * 64)));
    lambda_finalize_kernel<<<dim3(unsigned(ceil_div(k, kt)), unsigned(nb)), threads, 0, ctx.stream>>>(
        pmax, psum, plam, k, vd, sp.chunks, kt, lambda_t);
    MH_LAUNCH_CHECK();
}

namespace {

// Kernel choice of tap_filter (measured on MI355X at the UNet's three sizes):
// the LDS-staged row-tile kernel with 4 heads per thread and every value
// channel of its pixels while a block spans 10 or more pixels (its value rows
// are then staged at most 2.4 times over: 64x64 x 40 59.6 -> 47.2 us); else the
// per-thread kernel with 4 heads per thread (32x32 x 80: 28.4 us, 16x16 x 160:
// 18.7 us; the whole-row tile kernel 34.7 / 35.0, on slices of 4 channel quads
// 36.0 / 32.8 in the step). Tuning: tap_heads "t8" / "t4" forces the tile kernel
// with 8 / 4 heads per thread, 1, 2, 4 or 8 the per-thread kernel; tap_slice
// (quads dividing vd / 4) the tile kernel on channel slices of that width.
struct TapPlan {
    int tile_hg = 0;  // tile kernel heads per thread, 0: the per-thread kernel
    int cq = 0;       // tile kernel channel quads per block, 0: all
    int jq = 1;       // tile kernel channel quads per thread
};

TapPlan tap_plan(const Context &ctx, int hh, int ww, int vd, bool full_ln) {
    (void)hh;
    const int v4 = vd / 4;
    TapPlan p;
    const bool forced = ctx.tune.tap_tile >= 0;
    if (forced) {
        p.tile_hg = ctx.tune.tap_tile;
    } else if (std::min(256 / (2 * v4), ww) >= 10) {
        p.tile_hg = 4;
    } else if (!full_ln && ctx.tune.tap_slice > 0 && v4 % ctx.tune.tap_slice == 0) {
        p.tile_hg = 4;
    }
    if (p.tile_hg && ctx.tune.tap_slice > 0 && !full_ln && v4 % ctx.tune.tap_slice == 0) p.cq = ctx.tune.tap_slice;
    const int cqn = p.cq ? p.cq : v4;
    if (p.tile_hg && !full_ln && ctx.tune.tap_jq == 2 && cqn % 2 == 0) p.jq = 2;
    if (p.tile_hg && (kHeads / p.tile_hg) * (cqn / p.jq) > 256) p = TapPlan{};
    return p;
}

}  // namespace

int tap_filter_row_parts(const Context &ctx, int hh, int ww, int vd) {
    const TapPlan p = tap_plan(ctx, hh, ww, vd, false);
    return p.tile_hg && p.cq ? (vd / 4) / p.cq : 1;
}

void tap_filter(Context &ctx, const float *a_t, const float *v, const float *yc, const float *residual, float *out,
                int nb, int hh, int ww, int vd, const LayerNormOut *lno, float2 *row_sums) {
    MH_REQUIRE(vd % 4 == 0, "tap_filter: value width must be a multiple of 4");
    MH_REQUIRE(aligned16(a_t) && aligned16(v) && aligned16(yc) && aligned16(residual) && aligned16(out),
               "tap_filter: buffers must be 16-byte aligned");
    const int64_t pix = int64_t(nb) * hh * ww;
    if (pix == 0) return;
    LnOut ln;
    MH_REQUIRE(!(lno && row_sums), "tap_filter: the LayerNorm output or its row sums, not both");
    if (lno) {
        MH_REQUIRE(lno->gamma && lno->beta && lno->out && aligned16(lno->gamma) && aligned16(lno->beta) &&
                       aligned16(lno->out) && lno->out != out && lno->out != residual && lno->out != yc,
                   "tap_filter: LayerNorm output needs aligned gamma, beta and a separate output");
        ln.gamma = lno->gamma;
        ln.beta = lno->beta;
        ln.eps = lno->eps;
        ln.out = lno->out;
    }
    if (row_sums) {
        MH_REQUIRE((reinterpret_cast<uintptr_t>(row_sums) & 7) == 0, "tap_filter: row sums must be 8-byte aligned");
        ln.row_sums = row_sums;
    }
    const bool lnk = lno || row_sums;  // the kernels' LayerNorm variant (whole pixels per block)
    // Heads per thread: the most (value loads shared by more heads) that still
    // gives the chip about 2048 waves: 4 at 64x64 x 40 channels, 2 at 32x32 x 80,
    // 1 at 16x16 x 160 (batch 2).
    const int v4 = vd / 4;
    const TapPlan tp = tap_plan(ctx, hh, ww, vd, lno != nullptr);
    if (tp.tile_hg) {
        const int tile_hg = tp.tile_hg, cqn = tp.cq ? tp.cq : v4;
        const int tpp = (kHeads / tile_hg) * (cqn / tp.jq), tx = std::max(1, std::min(256 / tpp, ww));
        const size_t lds = (size_t(2) * (tx + kWin - 1) * cqn + size_t(2) * tx * (kWin * kHeads / 4)) * 16 +
                           (lnk ? size_t(tx) * tpp * sizeof(float2) : 0);
        const int64_t blocks = int64_t(nb) * hh * ceil_div(ww, tx);
        const dim3 grid(unsigned(blocks), unsigned(v4 / cqn));
        auto go = [&](auto kern) {
            kern<<<grid, unsigned(tx * tpp), lds, ctx.stream>>>(a_t, v, yc, residual, out, hh, ww, vd, tx, ln, tp.cq);
        };
        if (tp.jq == 2) {
            if (tile_hg == 8) lnk ? go(tap_filter_tile_kernel<8, true, 2>) : go(tap_filter_tile_kernel<8, false, 2>);
            else lnk ? go(tap_filter_tile_kernel<4, true, 2>) : go(tap_filter_tile_kernel<4, false, 2>);
        } else if (tile_hg == 8) {
            lnk ? go(tap_filter_tile_kernel<8, true>) : go(tap_filter_tile_kernel<8, false>);
        } else {
            lnk ? go(tap_filter_tile_kernel<4, true>) : go(tap_filter_tile_kernel<4, false>);
        }
        MH_LAUNCH_CHECK();
        return;
    }
    int hg = 4;
    if (ctx.tune.tap_tile >= 0) {
        const int want = ctx.tune.tap_heads;
        if (want == 1 || want == 2 || want == 4 || want == 8) hg = want;
    }
    const int tpp = (kHeads / hg) * v4;
    MH_REQUIRE(!lnk || tpp <= 256, "tap_filter: LayerNorm output needs a pixel's threads in one block");
    // Row split (tap_split tuning: 1, 3 or 5; default 0 chooses): three threads per
    // output while the map gives the chip fewer than two waves per SIMD of unsplit
    // threads and a pixel's 3 * tpp threads fit one block (measured alone with
    // LayerNorm 2: 32x32 x 80 34.1 -> 28.6 us, 16x16 x 160 22.9 -> 16.0 us; five
    // threads per output 40.6 / 22.3 us).
    int rs = ctx.tune.tap_split;
    if (rs != 1 && rs != 3 && rs != 5) {
        const int64_t waves = ceil_div(pix * tpp, 64);
        rs = (waves < 2 * 4 * int64_t(ctx.cu_count) && 3 * tpp <= 256) ? 3 : 1;
    }
    if (rs * tpp > 256) rs = 1;
    // Blocks of whole outputs: with the LayerNorm or a row split, P whole pixels
    // (P * tpp outputs) times rs threads each; else 256 outputs.
    const int opb = (lnk || rs > 1) ? (256 / (rs * tpp)) * tpp : 256;
    const unsigned threads = unsigned(opb * rs);
    const size_t lds = (lnk ? (2 * threads + 3) / 4 * 4 * sizeof(float) : 0) + size_t(rs - 1) * opb * hg * 16;
    const int64_t total = pix * tpp;
    const unsigned blocks = unsigned(ceil_div(total, opb));
    auto go = [&](auto kern) {
        kern<<<blocks, threads, lds, ctx.stream>>>(a_t, v, yc, residual, out, nb, hh, ww, vd, ln);
    };
    auto pick = [&](auto k1, auto k3, auto k5) {
        if (rs == 5) go(k5);
        else if (rs == 3) go(k3);
        else go(k1);
    };
    switch (hg) {
        case 8:
            lnk ? pick(tap_filter_kernel<8, true, 1>, tap_filter_kernel<8, true, 3>, tap_filter_kernel<8, true, 5>)
                : pick(tap_filter_kernel<8, false, 1>, tap_filter_kernel<8, false, 3>, tap_filter_kernel<8, false, 5>);
            break;
        case 4:
            lnk ? pick(tap_filter_kernel<4, true, 1>, tap_filter_kernel<4, true, 3>, tap_filter_kernel<4, true, 5>)
                : pick(tap_filter_kernel<4, false, 1>, tap_filter_kernel<4, false, 3>, tap_filter_kernel<4, false, 5>);
            break;
        case 2:
            lnk ? pick(tap_filter_kernel<2, true, 1>, tap_filter_kernel<2, true, 3>, tap_filter_kernel<2, true, 5>)
                : pick(tap_filter_kernel<2, false, 1>, tap_filter_kernel<2, false, 3>, tap_filter_kernel<2, false, 5>);
            break;
        default:
            lnk ? pick(tap_filter_kernel<1, true, 1>, tap_filter_kernel<1, true, 3>, tap_filter_kernel<1, true, 5>)
                : pick(tap_filter_kernel<1, false, 1>, tap_filter_kernel<1, false, 3>, tap_filter_kernel<1, false, 5>);
    }
    MH_LAUNCH_CHECK();
}

bool lambda_taps_ok(int k) { return k == 40 || k == 80 || k == 160; }

void lambda_taps(Context &ctx, const float *q, const float *w_aug_t, const float *lambda_t, int nb, int hw, int k,
                 float *a_t, float *yc) {
    MH_REQUIRE(lambda_taps_ok(k), "lambda position coefficients: k must be 40, 80 or 160");
    MH_REQUIRE(nb >= 0 && hw >= 0 && aligned16(q) && aligned16(w_aug_t) && aligned16(a_t) && aligned16(lambda_t) &&
                   aligned16(yc) && (lambda_t == nullptr) == (yc == nullptr) &&
                   (w_aug_t == nullptr) == (a_t == nullptr) && (w_aug_t || lambda_t),
               "lambda position coefficients: operands 16-byte aligned; w_aug_t with a_t, lambda_t with yc");
    if (nb == 0 || hw == 0) return;
    // Rows per part: 80 from 8192 pixels (the 64x64 latents' batch of two: four
    // waves per SIMD already), 48 from 2048, else 16 (or Tuning::taps_rows).
    const int64_t npix = int64_t(nb) * hw;
    int pr = npix >= 8192 ? 80 : npix >= 2048 ? 48 : 16;
    if (ctx.tune.taps_rows == 80 || ctx.tune.taps_rows == 48 || ctx.tune.taps_rows == 16) pr = ctx.tune.taps_rows;
    const int tap_parts_n = kTapRows / pr, ld = pr * kHeads + 8;
    // LDS per workgroup: its part's rows (pr of k + 4) and 4 waves' staging.
    const size_t lds = size_t(pr) * (k + 4) * sizeof(float) + size_t(4) * 2 * ld * sizeof(float);
    const int part0 = w_aug_t ? 0 : tap_parts_n;  // no w_aug_t: the content parts alone
    const int parts = (w_aug_t ? tap_parts_n : 0) + (lambda_t ? int(ceil_div(k, pr)) : 0);
    const int64_t tasks = (hw + 1) / 2;
    // Workgroups of 4 waves, at most as many as fit on the chip at once, each
    // wave looping over its item's pixel pairs.
    const int per_cu = int(std::max<size_t>(1, (160 * 1024) / lds));
    const int64_t cap = std::max<int64_t>(1, int64_t(ctx.cu_count) * per_cu / (parts * nb));
    const dim3 grid(unsigned(std::min<int64_t>(ceil_div(tasks, 4), cap)), unsigned(parts), unsigned(nb));
    // Products of the operands as given (f32 MFMA) in both precisions: in FAST
    // contexts they are faster than the products of f16-rounded operands the
    // FAST GEMMs take (tuning taps_r16 1, which this kernel can also run:
    // 20.8 against 13.9 us at 16x16), and more accurate.
    auto go = [&](auto kern) { kern<<<grid, 256, 0, ctx.stream>>>(q, w_aug_t, lambda_t, hw, a_t, yc, part0); };
    auto by_rows = [&](auto k80, auto k48, auto k16) { pr == 80 ? go(k80) : pr == 48 ? go(k48) : go(k16); };
    const bool r16 = ctx.precision == Precision::Fast && ctx.tune.taps_r16;
#define MH_TAPS(NF, TAIL, R) \
    by_rows(lambda_taps_kernel<NF, TAIL, R, 80>, lambda_taps_kernel<NF, TAIL, R, 48>, lambda_taps_kernel<NF, TAIL, R, 16>)
    if (k == 40) r16 ? MH_TAPS(2, 2, true) : MH_TAPS(2, 2, false);
    else if (k == 80) r16 ? MH_TAPS(5, 0, true) : MH_TAPS(5, 0, false);
    else r16 ? MH_TAPS(10, 0, true) : MH_TAPS(10, 0, false);
#undef MH_TAPS
    MH_LAUNCH_CHECK();
}

bool self_lambda_fused_ok(const Context &ctx, int k) {
    const int bit = k == 40 ? 1 : k == 80 ? 2 : k == 160 ? 4 : 0;
    return (ctx.tune.tap_fused & bit) != 0;
}

void self_lambda_fused(Context &ctx, const float *q, const float *w_aug_t, const float *lambda_t, const float *v,
                       const float *residual, float *out, int nb, int hh, int ww, int k, float2 *row_sums) {
    MH_REQUIRE(lambda_taps_ok(k), "self-lambda position path: k must be 40, 80 or 160");
    MH_REQUIRE(q && w_aug_t && lambda_t && v && out, "self-lambda position path: q, w_aug_t, lambda_t, v, out needed");
    MH_REQUIRE(aligned16(q) && aligned16(w_aug_t) && aligned16(lambda_t) && aligned16(v) && aligned16(residual) &&
                   aligned16(out) && (reinterpret_cast<uintptr_t>(row_sums) & 7) == 0,
               "self-lambda position path: buffers must be 16-byte aligned (row sums 8-byte)");
    MH_REQUIRE(out != q && out != v, "self-lambda position path: out must not alias q or v");
    MH_REQUIRE(nb >= 0 && hh >= 0 && ww >= 0, "self-lambda position path: negative size");
    const int64_t pix = int64_t(nb) * hh * ww;
    if (pix == 0) return;
    LnOut ln;
    ln.row_sums = row_sums;
    const int tpp = 2 * (k / 4);  // 4 heads per thread
    const int tx = std::min(std::min(256 / tpp, ww), 16);
    const int span = tx + kWin - 1;
    const size_t lds = size_t(2) * span * (k / 4) * 16 + size_t(2) * tx * kWin * kHeads * 4 +
                       size_t(tx) * kHeads * k * 4 + size_t(tx) * kHeads * 4 + (row_sums ? 2 * 256 * 4 : 0);
    const int64_t blocks = int64_t(nb) * hh * ceil_div(ww, tx);
    MH_REQUIRE(blocks < (int64_t(1) << 31), "self-lambda position path: map too large");
    auto go = [&](auto kern) {
        kern<<<unsigned(blocks), 256, lds, ctx.stream>>>(q, w_aug_t, lambda_t, v, residual, out, hh, ww, tx, ln);
    };
    const bool r16 = ctx.precision == Precision::Fast && ctx.tune.taps_r16, rs = row_sums != nullptr;
#define MH_FUSED(NF, TAIL)                                                                             \
    (r16 ? (rs ? go(tap_fused_kernel<NF, TAIL, true, true>) : go(tap_fused_kernel<NF, TAIL, true, false>)) \
         : (rs ? go(tap_fused_kernel<NF, TAIL, false, true>) : go(tap_fused_kernel<NF, TAIL, false, false>)))
    if (k == 40) MH_FUSED(2, 2);
    else if (k == 80) MH_FUSED(5, 0);
    else MH_FUSED(10, 0);
#undef MH_FUSED
    MH_LAUNCH_CHECK();
}

void position_term(Context &ctx, const float *q, const float *e, const float *v_branches, int br0, int nb, int hw,
                   int k, const float *yc, const float *residual, float *out) {
    MH_REQUIRE(k % 8 == 0, "position_term: head width must be a multiple of 8");
    MH_REQUIRE(aligned16(q) && aligned16(e) && aligned16(v_branches) && aligned16(yc) && aligned16(residual) &&
                   aligned16(out),
               "position_term: buffers must be 16-byte aligned");
    MH_REQUIRE(br0 >= 0 && br0 + nb <= 2, "position_term: branch out of range");
    const int64_t npix = int64_t(nb) * hw;
    if (npix == 0) return;
    position_term_kernel<<<unsigned(ceil_div(npix, 8)), 256, 0, ctx.stream>>>(q, e, v_branches, br0, nb, hw, k, yc,
                                                                             residual, out);
    MH_LAUNCH_CHECK();
}

void cross_lambda(Context &ctx, const float *q, const float *e, const float *lambda_c, const float *v_branches, int br0,
                  int nb, int hw, int k, const float *residual, float *out, float2 *row_sums) {
    MH_REQUIRE(k % 8 == 0 && k <= 256, "cross_lambda: head width must be a multiple of 8, at most 256");
    MH_REQUIRE((reinterpret_cast<uintptr_t>(row_sums) & 7) == 0, "cross_lambda: row sums must be 8-byte aligned");
    MH_REQUIRE(aligned16(q) && aligned16(e) && aligned16(lambda_c) && aligned16(v_branches) && aligned16(residual) &&
                   aligned16(out),
               "cross_lambda: buffers must be 16-byte aligned");
    MH_REQUIRE(br0 >= 0 && br0 + nb <= 2, "cross_lambda: branch out of range");
    MH_REQUIRE(out != q, "cross_lambda: out must not alias q");
    const int64_t npix = int64_t(nb) * hw;
    if (npix == 0) return;
    // The UNet's head widths take the matrix-core kernel (Tuning::cross_mfma 0 or
    // a forced head count: the per-thread kernel below).
    if (ctx.tune.cross_mfma && !ctx.tune.cross_heads && (k == 40 || k == 80 || k == 160)) {
        // P pixels per block: 12 (64x64 latents, 4 waves) or 10 (8 waves) tasks per block
        auto go = [&](auto kern, int P, int nt) {
            const dim3 grid(unsigned(ceil_div(hw, P)), unsigned(nb));
            kern<<<grid, nt, 0, ctx.stream>>>(q, e, lambda_c, v_branches, br0, hw, residual, out, row_sums);
        };
        if (k == 40) go(cross_lambda_mfma_kernel<2, 2, 8, 256>, 8, 256);
        else if (k == 80) go(cross_lambda_mfma_kernel<5, 0, 4, 512>, 4, 512);
        else go(cross_lambda_mfma_kernel<10, 0, 2, 512>, 2, 512);
        MH_LAUNCH_CHECK();
        return;
    }
    // Heads per thread: 4 while that still gives every CU a block, else 2
    // (measured at the UNet's sizes: 64x64 / k 40 15.6 us with 4 against 21.1
    // with 8, 32x32 / k 80 14.3 against 16.5 with 2, 16x16 / k 160 16.0 with 2
    // against 18.6 with 4); 8 only when forced.
    const int k4 = k / 4;
    int hg = 2;
    for (int cand : {4}) {
        const int P = 256 / ((kHeads / cand) * k4);
        if (P >= 1 && ceil_div(npix, P) >= ctx.cu_count) {
            hg = cand;
            break;
        }
    }
    if (ctx.tune.cross_heads) {  // A/B override: 2, 4 or 8
        const int want = ctx.tune.cross_heads;
        if ((want == 2 || want == 4 || want == 8) && 256 / ((kHeads / want) * k4) >= 1) hg = want;
    }
    const int P = std::max(1, 256 / ((kHeads / hg) * k4));
    const unsigned threads = unsigned(P * (kHeads / hg) * k4);
    const size_t lds = (size_t(P) * kHeads * k + size_t(P) * kHeads * kTokens) * sizeof(float) +
                       (row_sums ? size_t(threads) * sizeof(float2) : 0);
    const unsigned blocks = unsigned(ceil_div(npix, P));
    switch (hg) {
        case 8:
            cross_lambda_kernel<8><<<blocks, threads, lds, ctx.stream>>>(q, e, lambda_c, v_branches, br0, nb, hw, k,
                                                                          P, residual, out, row_sums);
            break;
        case 4:
            cross_lambda_kernel<4><<<blocks, threads, lds, ctx.stream>>>(q, e, lambda_c, v_branches, br0, nb, hw, k,
                                                                          P, residual, out, row_sums);
            break;
        default:
            cross_lambda_kernel<2><<<blocks, threads, lds, ctx.stream>>>(q, e, lambda_c, v_branches, br0, nb, hw, k,
                                                                          P, residual, out, row_sums);
    }
    MH_LAUNCH_CHECK();
}

}  // namespace mh
