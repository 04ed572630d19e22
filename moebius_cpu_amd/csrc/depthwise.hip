// Depthwise 3x3 convolution, stride 1, zero padding 1, with the reference's
// fused epilogues (src/engine/depthwise.rs:22-185): none, ReLU, and
// GLU * SiLU (y[:c/2] * SiLU(y[c/2:]), so the 2x wide map is never written).
//
// Bandwidth-bound. Each thread owns one float4 of channels across a strip of
// TX output pixels of one row; it slides a (TX+2)-wide register window over the
// three input rows, so each input float4 is fetched from L2 by 3 threads at
// most and from HBM about once. Consecutive threads take consecutive channel
// quads of the same pixel: every wave reads contiguous runs of channels.
//
// Arithmetic matches the reference tap for tap: acc = bias, then for ky, for kx,
// acc = fma(w, x, acc) (depthwise.rs:118-141); rows outside the image are
// skipped and columns outside contribute fma(w, 0, acc) == acc. The GLU gate's
// and the GroupNorm prologue's SiLU are the reference's in EXACT contexts and
// fast_silu (hardware exp2 and reciprocal) in FAST ones.
#include <cstdlib>

#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

template <int VW>
struct Vec;
template <>
struct Vec<4> {
    using T = float4;
    static __device__ __forceinline__ T zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
    static __device__ __forceinline__ T fma(T a, T b, T c) {
        return make_float4(__builtin_fmaf(a.x, b.x, c.x), __builtin_fmaf(a.y, b.y, c.y),
                           __builtin_fmaf(a.z, b.z, c.z), __builtin_fmaf(a.w, b.w, c.w));
    }
    static __device__ __forceinline__ T relu(T a) {
        return make_float4(relu_ref(a.x), relu_ref(a.y), relu_ref(a.z), relu_ref(a.w));
    }
    template <bool FM>
    static __device__ __forceinline__ T glu(T v, T g) {
        return make_float4(v.x * silu_of<FM>(g.x), v.y * silu_of<FM>(g.y), v.z * silu_of<FM>(g.z),
                           v.w * silu_of<FM>(g.w));
    }
    template <bool FM>
    static __device__ __forceinline__ T silu(T a) {
        return make_float4(silu_of<FM>(a.x), silu_of<FM>(a.y), silu_of<FM>(a.z), silu_of<FM>(a.w));
    }
};
template <>
struct Vec<1> {
    using T = float;
    static __device__ __forceinline__ T zero() { return 0.f; }
    static __device__ __forceinline__ T fma(T a, T b, T c) { return __builtin_fmaf(a, b, c); }
    static __device__ __forceinline__ T relu(T a) { return relu_ref(a); }
    template <bool FM>
    static __device__ __forceinline__ T glu(T v, T g) { return v * silu_of<FM>(g); }
    template <bool FM>
    static __device__ __forceinline__ T silu(T a) { return silu_of<FM>(a); }
};

// Optional GroupNorm affine applied to every in-image input value as it is
// loaded, y = [SiLU](x . scale + shift) (src/engine/norm.rs:132-148); padded
// taps stay zero, as in the reference's normalise-then-convolve order.
struct DwPrologue {
    const float *scale = nullptr, *shift = nullptr;  // [n * c]
    int silu = 0;
};

// One channel group (value part or gate part) of TX pixels: returns accumulators.
template <int VW, int TX, bool PRO, bool FM>
__device__ __forceinline__ void dw_accumulate(const typename Vec<VW>::T *__restrict__ x, int h, int w, int cv,
                                              int b, int oy, int ox0, int q,
                                              const typename Vec<VW>::T *__restrict__ wt,
                                              typename Vec<VW>::T bias, const DwPrologue &pro,
                                              typename Vec<VW>::T (&acc)[TX]) {
    using V = Vec<VW>;
    using T = typename V::T;
    T psc = V::zero(), psh = V::zero();
    if (PRO) {
        psc = reinterpret_cast<const T *>(pro.scale)[size_t(b) * cv + q];
        psh = reinterpret_cast<const T *>(pro.shift)[size_t(b) * cv + q];
    }
#pragma unroll
    for (int j = 0; j < TX; ++j) acc[j] = bias;
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
        const int iy = oy + ky - 1;
        if (iy < 0 || iy >= h) continue;
        const T *row = x + (size_t(b) * h + iy) * size_t(w) * cv + q;
        T win[TX + 2];
#pragma unroll
        for (int j = 0; j < TX + 2; ++j) {
            const int ix = ox0 + j - 1;
            if (ix >= 0 && ix < w) {
                win[j] = row[size_t(ix) * cv];
                if (PRO) {
                    win[j] = V::fma(win[j], psc, psh);
                    if (pro.silu) win[j] = V::template silu<FM>(win[j]);
                }
            } else {
                win[j] = V::zero();
            }
        }
        const T w0 = wt[(ky * 3 + 0) * cv + q], w1 = wt[(ky * 3 + 1) * cv + q], w2 = wt[(ky * 3 + 2) * cv + q];
#pragma unroll
        for (int j = 0; j < TX; ++j) {
            acc[j] = V::fma(w0, win[j], acc[j]);
            acc[j] = V::fma(w1, win[j + 1], acc[j]);
            acc[j] = V::fma(w2, win[j + 2], acc[j]);
        }
    }
}

// cv = c / VW vectors per input pixel; co_v = output vectors per pixel.
template <int VW, int TX, int EPI, bool PRO, bool FM>
__global__ __launch_bounds__(256) void depthwise_kernel(const typename Vec<VW>::T *__restrict__ x, int n, int h,
                                                        int w, int cv, const typename Vec<VW>::T *__restrict__ wt,
                                                        const typename Vec<VW>::T *__restrict__ bias, DwPrologue pro,
                                                        typename Vec<VW>::T *__restrict__ out) {
    using V = Vec<VW>;
    using T = typename V::T;
    const int co_v = EPI == 2 ? cv / 2 : cv;
    const int strips = (w + TX - 1) / TX;
    const int64_t total = int64_t(n) * h * strips * co_v;
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= total) return;
    const int q = int(t % co_v);
    int64_t rest = t / co_v;
    const int strip = int(rest % strips);
    rest /= strips;
    const int oy = int(rest % h);
    const int b = int(rest / h);
    const int ox0 = strip * TX;

    T acc[TX];
    dw_accumulate<VW, TX, PRO, FM>(x, h, w, cv, b, oy, ox0, q, wt, bias[q], pro, acc);
    T *dst = out + (size_t(b) * h + oy) * size_t(w) * co_v + q;
    if (EPI == 2) {
        T gate[TX];
        dw_accumulate<VW, TX, PRO, FM>(x, h, w, cv, b, oy, ox0, q + co_v, wt, bias[q + co_v], pro, gate);
#pragma unroll
        for (int j = 0; j < TX; ++j)
            if (ox0 + j < w) dst[size_t(ox0 + j) * co_v] = V::template glu<FM>(acc[j], gate[j]);
    } else {
#pragma unroll
        for (int j = 0; j < TX; ++j)
            if (ox0 + j < w) dst[size_t(ox0 + j) * co_v] = EPI == 1 ? V::relu(acc[j]) : acc[j];
    }
}

// LDS-tiled variant for channel counts that are multiples of 4: a workgroup
// stages the (16+2) x (16+2) input pixels of a 16x16 output tile for 4 channel
// quads (and the matching gate quads for GLU) in LDS once, then each thread
// computes four adjacent output pixels of one quad from LDS. Every input value
// is read from L2/HBM about (18*18)/(16*16) = 1.27 times instead of 4.5, and the
// optional GroupNorm prologue is applied once per staged value. The tap order
// and the skipped out-of-image rows are those of depthwise_kernel. (Measured
// against 8x8 tiles of 16 quads, 8x16 / 16x8 of 8 and 4x16 of 16: the 32x32 GLU
// 19.6 -> 17.7 us, UNet step -30 us.)
constexpr int kDwTH = 16, kDwTW = 16, kDwCQ = 4;
static_assert(kDwCQ * kDwTH * (kDwTW / 4) == 256, "one thread per 4 outputs of a quad");
constexpr int kDwNP = (kDwTH + 2) * (kDwTW + 2);

// x2 (optional): the input is [x | x2] per pixel, x holding quads [0, cv1)
// (cv1 a multiple of kDwCQ, so a block reads one of the two) and x2 the rest.
// OUT16 (FAST contexts whose only reader is an f16 GEMM): the output rounded to
// f16 as that GEMM rounds its f32 operands (nearest even, saturated at
// +-65504), so the products are the same bits from half the bytes.
template <int EPI, bool PRO, bool FM, bool OUT16 = false>
__global__ __launch_bounds__(256) void depthwise_tile_kernel(const float4 *__restrict__ x, int n, int h, int w,
                                                             int cv, const float4 *__restrict__ wt,
                                                             const float4 *__restrict__ bias, DwPrologue pro,
                                                             void *__restrict__ out,
                                                             const float4 *__restrict__ x2, int cv1) {
    using V = Vec<4>;
    // GLU (EPI 2) convolves two input halves. They pass through one LDS tile in
    // turn (20.7 KB instead of 41.5 KB: LDS allows seven workgroups per CU
    // instead of three, registers five); the loads of both are issued up front.
    constexpr int PARTS = EPI == 2 ? 2 : 1;
    __shared__ float4 tile[kDwNP][kDwCQ];
    const int co_v = EPI == 2 ? cv / 2 : cv;
    const int tiles_x = (w + kDwTW - 1) / kDwTW, tiles_y = (h + kDwTH - 1) / kDwTH;
    int bid = blockIdx.x;
    const int tx = bid % tiles_x;
    bid /= tiles_x;
    const int ty = bid % tiles_y;
    const int b = bid / tiles_y;
    const int q0 = blockIdx.y * kDwCQ;
    const int oy0 = ty * kDwTH, ox0 = tx * kDwTW;
    // Staging: every load of the thread is issued before the first LDS store,
    // so a thread has all of its (up to 11) 16-byte loads in flight at once.
    constexpr int TOTAL = PARTS * kDwNP * kDwCQ;
    constexpr int PER = (TOTAL + 255) / 256;
    const bool sec = x2 && q0 >= cv1;
    const float4 *xs = sec ? x2 : x;
    const int xld = x2 ? (sec ? cv - cv1 : cv1) : cv, xq0 = sec ? q0 - cv1 : q0;
    // A thread stages one channel quad (threadIdx.x % kDwCQ, 256 being a
    // multiple of kDwCQ) for every pixel it loads: its prologue scale/shift per
    // part are loaded first, with the tile's loads, not per staged value.
    const int sq = threadIdx.x % kDwCQ;
    float4 psc[PARTS], psh[PARTS];
#pragma unroll
    for (int part = 0; part < PARTS; ++part) {
        psc[part] = psh[part] = V::zero();
        if (PRO && q0 + sq < co_v) {
            const size_t qi = size_t(b) * cv + q0 + sq + part * co_v;
            psc[part] = reinterpret_cast<const float4 *>(pro.scale)[qi];
            psh[part] = reinterpret_cast<const float4 *>(pro.shift)[qi];
        }
    }
    float4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int idx = threadIdx.x + 256 * i;
        const int part = idx / (kDwNP * kDwCQ);
        const int r = idx - part * (kDwNP * kDwCQ);
        const int pix = r / kDwCQ, qq = r - pix * kDwCQ;
        const int iy = oy0 - 1 + pix / (kDwTW + 2), ix = ox0 - 1 + pix % (kDwTW + 2);
        v[i] = V::zero();
        if (idx < TOTAL && q0 + qq < co_v && iy >= 0 && iy < h && ix >= 0 && ix < w)
            v[i] = xs[(size_t(b) * h + iy) * size_t(w) * xld + size_t(ix) * xld + xq0 + qq + part * co_v];
    }
    // The block's 9 taps and bias per quad and part, staged in LDS beside the
    // tile (their loads in flight with the tile's), so the products below read
    // them from LDS instead of waiting on L2 once per tap row.
    __shared__ float4 wts[PARTS][10][kDwCQ];
    float4 wv = V::zero();
    const int wtid = int(threadIdx.x);
    if (wtid < PARTS * 10 * kDwCQ) {
        const int wp = wtid / (10 * kDwCQ), wr = wtid - wp * (10 * kDwCQ);
        const int tap = wr / kDwCQ, wq = wr - tap * kDwCQ;
        if (q0 + wq < co_v) {
            const int qw = q0 + wq + wp * co_v;
            wv = tap < 9 ? wt[tap * cv + qw] : bias[qw];
        }
    }
    const int qq = threadIdx.x % kDwCQ, g = threadIdx.x / kDwCQ;
    const int r = g / (kDwTW / 4), c0 = (g % (kDwTW / 4)) * 4;
    const int q = q0 + qq, oy = oy0 + r;
    const bool active = q < co_v && oy < h;  // inactive threads still reach every barrier
    float4 acc[PARTS][4];
#pragma unroll
    for (int part = 0; part < PARTS; ++part) {
        if (part > 0) __syncthreads();  // the previous half's reads are done
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + 256 * i;
            if (idx >= TOTAL) break;
            const int ip = idx / (kDwNP * kDwCQ);
            if (ip != part) continue;
            const int rr = idx - ip * (kDwNP * kDwCQ);
            const int pix = rr / kDwCQ, pq = rr - pix * kDwCQ;
            if (PRO) {
                const int iy = oy0 - 1 + pix / (kDwTW + 2), ix = ox0 - 1 + pix % (kDwTW + 2);
                if (q0 + pq < co_v && iy >= 0 && iy < h && ix >= 0 && ix < w) {
                    v[i] = V::fma(v[i], psc[ip], psh[ip]);  // pq == sq: this thread's quad
                    if (pro.silu) v[i] = V::template silu<FM>(v[i]);
                }
            }
            tile[pix][pq] = v[i];
        }
        if (part == 0 && wtid < PARTS * 10 * kDwCQ) {
            const int wp = wtid / (10 * kDwCQ), wr = wtid - wp * (10 * kDwCQ);
            wts[wp][wr / kDwCQ][wr % kDwCQ] = wv;
        }
        __syncthreads();
        if (active) {
            const float4 bv = wts[part][9][qq];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[part][j] = bv;
#pragma unroll
            for (int ky = 0; ky < 3; ++ky) {
                const int iy = oy + ky - 1;
                if (iy < 0 || iy >= h) continue;
                float4 win[6];
#pragma unroll
                for (int j = 0; j < 6; ++j) win[j] = tile[(r + ky) * (kDwTW + 2) + c0 + j][qq];
                const float4 w0 = wts[part][ky * 3 + 0][qq], w1 = wts[part][ky * 3 + 1][qq],
                             w2 = wts[part][ky * 3 + 2][qq];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[part][j] = V::fma(w0, win[j], acc[part][j]);
                    acc[part][j] = V::fma(w1, win[j + 1], acc[part][j]);
                    acc[part][j] = V::fma(w2, win[j + 2], acc[part][j]);
                }
            }
        }
    }
    if (!active) return;
    const size_t o0 = (size_t(b) * h + oy) * size_t(w) * co_v + q;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ox = ox0 + c0 + j;
        if (ox >= w) break;
        float4 y;
        if (EPI == 2) y = V::template glu<FM>(acc[0][j], acc[PARTS - 1][j]);
        else if (EPI == 1) y = V::relu(acc[0][j]);
        else y = acc[0][j];
        if constexpr (OUT16) {
            typedef _Float16 half4 __attribute__((ext_vector_type(4)));
            auto r16 = [](float v) {
                return static_cast<_Float16>(__builtin_fabsf(v) > 65504.0f ? __builtin_copysignf(65504.0f, v) : v);
            };
            static_cast<half4 *>(out)[o0 + size_t(ox) * co_v] = half4{r16(y.x), r16(y.y), r16(y.z), r16(y.w)};
        } else {
            static_cast<float4 *>(out)[o0 + size_t(ox) * co_v] = y;
        }
    }
}

template <int EPI, bool PRO>
void launch_dw_tile_fm(bool fast, bool out16, dim3 grid, hipStream_t st, const float4 *x, int n, int h, int w,
                       int cv, const float4 *wt, const float4 *bias, const DwPrologue &pro, void *out,
                       const float4 *x2, int cv1) {
    if (out16)
        depthwise_tile_kernel<EPI, PRO, true, true><<<grid, 256, 0, st>>>(x, n, h, w, cv, wt, bias, pro, out, x2, cv1);
    else if (fast)
        depthwise_tile_kernel<EPI, PRO, true><<<grid, 256, 0, st>>>(x, n, h, w, cv, wt, bias, pro, out, x2, cv1);
    else
        depthwise_tile_kernel<EPI, PRO, false><<<grid, 256, 0, st>>>(x, n, h, w, cv, wt, bias, pro, out, x2, cv1);
}

template <int VW, int TX, int EPI, bool PRO, typename T>
void launch_dw_fm(bool fast, unsigned blocks, hipStream_t st, const T *x, int n, int h, int w, int cv, const T *wt,
                  const T *bias, const DwPrologue &pro, T *out) {
    if (fast) depthwise_kernel<VW, TX, EPI, PRO, true><<<blocks, 256, 0, st>>>(x, n, h, w, cv, wt, bias, pro, out);
    else depthwise_kernel<VW, TX, EPI, PRO, false><<<blocks, 256, 0, st>>>(x, n, h, w, cv, wt, bias, pro, out);
}

template <bool PRO>
void launch_dw_tile(Context &ctx, const float *x, int n, int h, int w, int c, const float *wt, const float *bias,
                    int epilogue, const DwPrologue &pro, void *out, const float *x2 = nullptr, int c2 = 0,
                    bool out16 = false) {
    const int cv = c / 4;
    const int co_v = epilogue == 2 ? cv / 2 : cv;
    const int64_t tiles = int64_t(n) * ceil_div(h, kDwTH) * ceil_div(w, kDwTW);
    MH_REQUIRE(tiles < (int64_t(1) << 31), "depthwise: map too large");
    const dim3 grid(unsigned(tiles), unsigned(ceil_div(co_v, kDwCQ)));
    const float4 *xv = reinterpret_cast<const float4 *>(x);
    const float4 *wv = reinterpret_cast<const float4 *>(wt);
    const float4 *bv = reinterpret_cast<const float4 *>(bias);
    const float4 *x2v = reinterpret_cast<const float4 *>(x2);
    const int cv1 = (c - c2) / 4;
    const bool fast = ctx.precision == Precision::Fast;
    MH_REQUIRE(!out16 || fast, "depthwise: f16 output in FAST contexts only");
    switch (epilogue) {
        // FAST contexts take fast_silu for the GLU gate and the prologue's SiLU
        case 0: launch_dw_tile_fm<0, PRO>(fast, out16, grid, ctx.stream, xv, n, h, w, cv, wv, bv, pro, out, x2v, cv1); break;
        case 1: launch_dw_tile_fm<1, PRO>(fast, out16, grid, ctx.stream, xv, n, h, w, cv, wv, bv, pro, out, x2v, cv1); break;
        default: launch_dw_tile_fm<2, PRO>(fast, out16, grid, ctx.stream, xv, n, h, w, cv, wv, bv, pro, out, x2v, cv1); break;
    }
    MH_LAUNCH_CHECK();
}

template <int VW, int TX, bool PRO>
void launch_dw(Context &ctx, const float *x, int n, int h, int w, int c, const float *wt, const float *bias,
               int epilogue, const DwPrologue &pro, float *out) {
    using T = typename Vec<VW>::T;
    const int cv = c / VW;
    const int co_v = epilogue == 2 ? cv / 2 : cv;
    const int strips = (w + TX - 1) / TX;
    const int64_t total = int64_t(n) * h * strips * co_v;
    const unsigned blocks = unsigned(ceil_div(total, 256));
    const T *xv = reinterpret_cast<const T *>(x);
    const T *wv = reinterpret_cast<const T *>(wt);
    const T *bv = reinterpret_cast<const T *>(bias);
    T *ov = reinterpret_cast<T *>(out);
    const bool fast = ctx.precision == Precision::Fast;
    switch (epilogue) {
        case 0: launch_dw_fm<VW, TX, 0, PRO>(fast, blocks, ctx.stream, xv, n, h, w, cv, wv, bv, pro, ov); break;
        case 1: launch_dw_fm<VW, TX, 1, PRO>(fast, blocks, ctx.stream, xv, n, h, w, cv, wv, bv, pro, ov); break;
        default: launch_dw_fm<VW, TX, 2, PRO>(fast, blocks, ctx.stream, xv, n, h, w, cv, wv, bv, pro, ov); break;
    }
    MH_LAUNCH_CHECK();
}

}  // namespace

bool depthwise3x3_h16(Context &ctx, const float *x, int n, int h, int w, int c, const float *weight,
                      const float *bias, int epilogue, void *out16, const Affine *prologue, const float *x2, int c2) {
    MH_REQUIRE(epilogue >= 0 && epilogue <= 2, "depthwise: unknown epilogue");
    if (ctx.precision != Precision::Fast || !ctx.tune.dw_tiled) return false;
    const int co = epilogue == 2 ? c / 2 : c;
    if (epilogue == 2 && (c % 2 || x2)) return false;
    if (x2 && (c2 <= 0 || c2 >= c || (c - c2) % (4 * kDwCQ) != 0 || c2 % 4 != 0)) return false;
    if (co % 4 || !aligned16(x) || !aligned16(x2) || !aligned16(weight) || !aligned16(bias) ||
        (reinterpret_cast<uintptr_t>(out16) & 7) || (prologue && (!aligned16(prologue->scale) ||
                                                                  !aligned16(prologue->shift))))
        return false;
    if (int64_t(n) * h * w * c == 0) return true;
    DwPrologue pro;
    if (prologue) {
        pro.scale = prologue->scale;
        pro.shift = prologue->shift;
        pro.silu = prologue->silu ? 1 : 0;
        launch_dw_tile<true>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out16, x2, c2, true);
    } else {
        launch_dw_tile<false>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out16, x2, c2, true);
    }
    return true;
}

void depthwise3x3(Context &ctx, const float *x, int n, int h, int w, int c, const float *weight, const float *bias,
                  int epilogue, float *out, const Affine *prologue, const float *x2, int c2) {
    MH_REQUIRE(epilogue >= 0 && epilogue <= 2, "depthwise: unknown epilogue");
    if (epilogue == 2) MH_REQUIRE(c % 2 == 0, "GLU needs an even channel count");
    if (int64_t(n) * h * w * c == 0) return;
    if (x2) {
        MH_REQUIRE(epilogue <= 1 && c2 > 0 && c2 < c && (c - c2) % (4 * kDwCQ) == 0 && c2 % 4 == 0,
                   "depthwise over two inputs: NONE or RELU, first part a multiple of 16 channels, second of 4");
        const bool tiled = ctx.tune.dw_tiled && aligned16(x) && aligned16(x2) && aligned16(weight) &&
                           aligned16(bias) && aligned16(out) && (!prologue || (aligned16(prologue->scale) &&
                                                                                aligned16(prologue->shift)));
        if (!tiled) {  // the other kernels read one input: concatenate first
            float *cat = static_cast<float *>(ctx.ws.get(size_t(n) * h * w * c * sizeof(float), ctx.stream));
            concat_channels(ctx, x, c - c2, x2, c2, int64_t(n) * h * w, cat);
            depthwise3x3(ctx, cat, n, h, w, c, weight, bias, epilogue, out, prologue);
            return;
        }
        DwPrologue pro;
        if (prologue) {
            MH_REQUIRE(prologue->scale && prologue->shift, "depthwise prologue needs scale and shift");
            pro.scale = prologue->scale;
            pro.shift = prologue->shift;
            pro.silu = prologue->silu ? 1 : 0;
            launch_dw_tile<true>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out, x2, c2);
        } else {
            launch_dw_tile<false>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out, x2, c2);
        }
        return;
    }
    const int co = epilogue == 2 ? c / 2 : c;
    DwPrologue pro;
    if (prologue) {
        MH_REQUIRE(prologue->scale && prologue->shift, "depthwise prologue needs scale and shift");
        pro.scale = prologue->scale;
        pro.shift = prologue->shift;
        pro.silu = prologue->silu ? 1 : 0;
    }
    const bool vec4 = co % 4 == 0 && aligned16(x) && aligned16(weight) && aligned16(bias) && aligned16(out) &&
                      aligned16(pro.scale) && aligned16(pro.shift);
    const int tiled = ctx.tune.dw_tiled;  // A/B override: 0 = register-window kernel
    if (vec4 && tiled) {
        if (prologue) launch_dw_tile<true>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
        else launch_dw_tile<false>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
    } else if (vec4) {
        if (prologue) launch_dw<4, 4, true>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
        else launch_dw<4, 4, false>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
    } else {
        if (prologue) launch_dw<1, 4, true>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
        else launch_dw<1, 4, false>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
    }
}

}  // namespace mh
