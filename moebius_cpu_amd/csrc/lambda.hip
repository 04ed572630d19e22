// Lambda-layer kernels of the UNet's MixTransformer (src/unet/lambda.rs).
//
// softmax_lambda (lambda.rs:452-489): lambda_c[kk][j] = sum_r softmax_r(K)[r][kk] * V[r][j]
//   1. column maxima of K over rows, per 32-row chunk;
//   2. per chunk: e = exp(K - colmax) (the reference's Cephes exp), f32 column
//      sums over the chunk, and the chunk's partial e^T V in f32;
//   3. finalise: partials summed over chunks in order (f32 for lambda, f64 for
//      the sums, as the reference folds its chunk sums in f64), row kk scaled by
//      (f32)(1 / sum[kk]); written transposed ([j][kk]) so Yc = Q . lambda_c is
//      an NT GEMM.
// tap_filter (lambda.rs:288-314): per pixel, head and value channel,
//   o = Yc + A[., 225] then + A[., dy*15+dx] * V[pixel + (dy-7, dx-7)] over the
//   in-image taps in (dy, dx) order with fused multiply-adds: the reference's
//   per-element operation order.
// position_term (lambda.rs:406-425): per pixel, B[h][m] = q_h . E[n][m] with
//   the reference's 8-lane dot, then o_h += B[h][m] * V[m] for m = 0..9.
#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

constexpr int kLamChunk = 32;   // rows per softmax_lambda chunk
constexpr int kWin = 15, kTaps = 225, kPad = 7, kTapsB = 226;
constexpr int kHeads = 8, kTokens = 10;

// keys [b][rows][k]; partial max [b][chunks][k]
__global__ void lambda_colmax_kernel(const float *__restrict__ keys, int rows, int k, int chunks,
                                     float *__restrict__ pmax) {
    const int chunk = blockIdx.x, b = blockIdx.y;
    const float *kb = keys + (size_t(b) * rows + size_t(chunk) * kLamChunk) * k;
    const int r1 = min(kLamChunk, rows - chunk * kLamChunk);
    for (int j = threadIdx.x; j < k; j += blockDim.x) {
        float m = -INFINITY;
        for (int r = 0; r < r1; ++r) m = fmaxf(m, kb[size_t(r) * k + j]);
        pmax[(size_t(b) * chunks + chunk) * k + j] = m;
    }
}

// One block per (chunk, item): e = exp(K - max) into LDS, column sums, partial e^T V.
// LDS: e [32][k], v [32][vd] with k, vd <= 160.
__global__ __launch_bounds__(256) void lambda_partial_kernel(const float *__restrict__ keys,
                                                             const float *__restrict__ v, int rows, int k, int vd,
                                                             int chunks, const float *__restrict__ pmax,
                                                             float *__restrict__ psum, float *__restrict__ plam) {
    __shared__ float es[kLamChunk * 160];
    __shared__ float vs[kLamChunk * 160];
    __shared__ float mx[160];
    const int chunk = blockIdx.x, b = blockIdx.y;
    const int r0 = chunk * kLamChunk;
    const int r1 = min(kLamChunk, rows - r0);
    for (int j = threadIdx.x; j < k; j += blockDim.x) {
        float m = -INFINITY;
        for (int c = 0; c < chunks; ++c) m = fmaxf(m, pmax[(size_t(b) * chunks + c) * k + j]);
        mx[j] = m;
    }
    __syncthreads();
    const float *kb = keys + (size_t(b) * rows + r0) * k;
    const float *vb = v + (size_t(b) * rows + r0) * vd;
    for (int i = threadIdx.x; i < kLamChunk * k; i += blockDim.x) {
        const int r = i / k, j = i - r * k;
        es[i] = r < r1 ? ref_exp(kb[size_t(r) * k + j] - mx[j]) : 0.0f;
    }
    for (int i = threadIdx.x; i < kLamChunk * vd; i += blockDim.x) {
        const int r = i / vd;
        vs[i] = r < r1 ? vb[i] : 0.0f;
    }
    __syncthreads();
    float *ps = psum + (size_t(b) * chunks + chunk) * k;
    for (int j = threadIdx.x; j < k; j += blockDim.x) {
        float s = 0.0f;
        for (int r = 0; r < r1; ++r) s += es[r * k + j];
        ps[j] = s;
    }
    float *pl = plam + (size_t(b) * chunks + chunk) * size_t(k) * vd;
    for (int i = threadIdx.x; i < k * vd; i += blockDim.x) {
        const int kk = i / vd, j = i - kk * vd;
        float acc = 0.0f;
        for (int r = 0; r < r1; ++r) acc = __builtin_fmaf(es[r * k + kk], vs[r * vd + j], acc);
        pl[i] = acc;
    }
}

// out_t [b][vd][k] = (sum_c plam[b][c][kk][j]) * (f32)(1 / sum_c psum[b][c][kk]).
__global__ void lambda_finalize_kernel(const float *__restrict__ psum, const float *__restrict__ plam, int k, int vd,
                                       int chunks, int nb, float *__restrict__ out_t) {
    const int64_t total = int64_t(nb) * k * vd;
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
        const int b = int(e / (int64_t(k) * vd));
        const int i = int(e - int64_t(b) * k * vd);
        const int kk = i / vd, j = i - kk * vd;
        float acc = 0.0f;
        double s = 0.0;
        for (int c = 0; c < chunks; ++c) {
            acc += plam[(size_t(b) * chunks + c) * size_t(k) * vd + i];
            s += double(psum[(size_t(b) * chunks + c) * k + kk]);
        }
        const float inv = float(1.0 / s);
        out_t[(size_t(b) * vd + j) * k + kk] = acc * inv;
    }
}

// One thread per (pixel, head, 4 value channels). a: [b*hw][8][226]; v: [b*hw][vd];
// o: [b*hw][8*vd], holding Yc on entry.
__global__ __launch_bounds__(256) void tap_filter_kernel(const float *__restrict__ a, const float *__restrict__ v,
                                                         float *__restrict__ o, int nb, int hh, int ww, int vd) {
    const int v4 = vd >> 2;
    const int64_t total = int64_t(nb) * hh * ww * kHeads * v4;
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= total) return;
    const int jq = int(t % v4);
    const int64_t nh = t / v4;
    const int h = int(nh % kHeads);
    const int64_t pix = nh / kHeads;  // b*hw + y*ww + x
    const int hw = hh * ww;
    const int b = int(pix / hw);
    const int rem = int(pix - int64_t(b) * hw);
    const int y = rem / ww, x = rem - (rem / ww) * ww;
    const float *ap = a + (pix * kHeads + h) * kTapsB;
    float4 *op = reinterpret_cast<float4 *>(o + pix * (kHeads * vd) + h * vd) + jq;
    float4 acc = *op;
    const float bias = ap[kTaps];
    acc.x += bias;
    acc.y += bias;
    acc.z += bias;
    acc.w += bias;
    const float4 *vb = reinterpret_cast<const float4 *>(v + int64_t(b) * hw * vd);
    const int kx0 = max(kPad - x, 0), kx1 = min(kWin, ww + kPad - x);
    for (int ky = 0; ky < kWin; ++ky) {
        const int iy = y + ky - kPad;
        if (iy < 0 || iy >= hh) continue;
        const float4 *vr = vb + (int64_t(iy) * ww + x - kPad) * v4 + jq;
        const float *ar = ap + ky * kWin;
        for (int kx = kx0; kx < kx1; ++kx) {
            const float c = ar[kx];
            const float4 s = vr[int64_t(kx) * v4];
            acc.x = __builtin_fmaf(c, s.x, acc.x);
            acc.y = __builtin_fmaf(c, s.y, acc.y);
            acc.z = __builtin_fmaf(c, s.z, acc.z);
            acc.w = __builtin_fmaf(c, s.w, acc.w);
        }
    }
    *op = acc;
}

// 8-lane dot of src/unet/lambda.rs:429-439 (k a multiple of 8).
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

// Block of 256 threads handles 8 pixels. q, o: [b*hw][8*k]; e: [hw][10][k];
// vb: [2][10][k] (per branch); branch of item b = br0 + b.
__global__ __launch_bounds__(256) void position_term_kernel(const float *__restrict__ q, const float *__restrict__ e,
                                                            const float *__restrict__ vbr, int br0, int nb, int hw,
                                                            int k, float *__restrict__ o) {
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
    for (int i = threadIdx.x; i < P * c; i += 256) {
        const int p = i / c, hj = i - p * c;
        const int h = hj / k, j = hj - h * k;
        const int64_t pix = pix0 + p;
        if (pix >= npix) continue;
        const int b = int(pix / hw);
        const float *vm = vbr + int64_t(br0 + b) * kTokens * k;
        float acc = o[pix * c + hj];
#pragma unroll
        for (int m = 0; m < kTokens; ++m) acc = __builtin_fmaf(bm[p][h][m], vm[m * k + j], acc);
        o[pix * c + hj] = acc;
    }
}

}  // namespace

void softmax_lambda(Context &ctx, const float *keys, const float *v, int nb, int rows, int k, int vd,
                    float *lambda_t) {
    MH_REQUIRE(k > 0 && k <= 160 && vd > 0 && vd <= 160, "softmax_lambda: widths above 160 are not supported");
    MH_REQUIRE(rows > 0 && nb > 0, "softmax_lambda: empty input");
    const int chunks = int(ceil_div(rows, kLamChunk));
    const size_t pm = size_t(nb) * chunks * k;
    const size_t pl = size_t(nb) * chunks * size_t(k) * vd;
    float *ws = static_cast<float *>(ctx.ws.get((2 * pm + pl) * sizeof(float), ctx.stream));
    float *pmax = ws, *psum = ws + pm, *plam = ws + 2 * pm;
    lambda_colmax_kernel<<<dim3(chunks, nb), 64, 0, ctx.stream>>>(keys, rows, k, chunks, pmax);
    MH_LAUNCH_CHECK();
    lambda_partial_kernel<<<dim3(chunks, nb), 256, 0, ctx.stream>>>(keys, v, rows, k, vd, chunks, pmax, psum, plam);
    MH_LAUNCH_CHECK();
    const int64_t total = int64_t(nb) * k * vd;
    lambda_finalize_kernel<<<unsigned(ceil_div(total, 256)), 256, 0, ctx.stream>>>(psum, plam, k, vd, chunks, nb,
                                                                                   lambda_t);
    MH_LAUNCH_CHECK();
}

void tap_filter(Context &ctx, const float *a, const float *v, float *o, int nb, int hh, int ww, int vd) {
    MH_REQUIRE(vd % 4 == 0, "tap_filter: value width must be a multiple of 4");
    MH_REQUIRE(aligned16(v) && aligned16(o), "tap_filter: v and o must be 16-byte aligned");
    const int64_t total = int64_t(nb) * hh * ww * kHeads * (vd / 4);
    if (total == 0) return;
    tap_filter_kernel<<<unsigned(ceil_div(total, 256)), 256, 0, ctx.stream>>>(a, v, o, nb, hh, ww, vd);
    MH_LAUNCH_CHECK();
}

void position_term(Context &ctx, const float *q, const float *e, const float *v_branches, int br0, int nb, int hw,
                   int k, float *o) {
    MH_REQUIRE(k % 8 == 0, "position_term: head width must be a multiple of 8");
    MH_REQUIRE(aligned16(q) && aligned16(e), "position_term: q and e must be 16-byte aligned");
    MH_REQUIRE(br0 >= 0 && br0 + nb <= 2, "position_term: branch out of range");
    const int64_t npix = int64_t(nb) * hw;
    if (npix == 0) return;
    position_term_kernel<<<unsigned(ceil_div(npix, 8)), 256, 0, ctx.stream>>>(q, e, v_branches, br0, nb, hw, k, o);
    MH_LAUNCH_CHECK();
}

}  // namespace mh
