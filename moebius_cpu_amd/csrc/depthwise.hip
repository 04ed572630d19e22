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
// skipped and columns outside contribute fma(w, 0, acc) == acc.
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
    static __device__ __forceinline__ T glu(T v, T g) {
        return make_float4(v.x * ref_silu(g.x), v.y * ref_silu(g.y), v.z * ref_silu(g.z), v.w * ref_silu(g.w));
    }
    static __device__ __forceinline__ T silu(T a) {
        return make_float4(ref_silu(a.x), ref_silu(a.y), ref_silu(a.z), ref_silu(a.w));
    }
};
template <>
struct Vec<1> {
    using T = float;
    static __device__ __forceinline__ T zero() { return 0.f; }
    static __device__ __forceinline__ T fma(T a, T b, T c) { return __builtin_fmaf(a, b, c); }
    static __device__ __forceinline__ T relu(T a) { return relu_ref(a); }
    static __device__ __forceinline__ T glu(T v, T g) { return v * ref_silu(g); }
    static __device__ __forceinline__ T silu(T a) { return ref_silu(a); }
};

// Optional GroupNorm affine applied to every in-image input value as it is
// loaded, y = [SiLU](x . scale + shift) (src/engine/norm.rs:132-148); padded
// taps stay zero, as in the reference's normalise-then-convolve order.
struct DwPrologue {
    const float *scale = nullptr, *shift = nullptr;  // [n * c]
    int silu = 0;
};

// One channel group (value part or gate part) of TX pixels: returns accumulators.
template <int VW, int TX, bool PRO>
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
                    if (pro.silu) win[j] = V::silu(win[j]);
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
template <int VW, int TX, int EPI, bool PRO>
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
    dw_accumulate<VW, TX, PRO>(x, h, w, cv, b, oy, ox0, q, wt, bias[q], pro, acc);
    T *dst = out + (size_t(b) * h + oy) * size_t(w) * co_v + q;
    if (EPI == 2) {
        T gate[TX];
        dw_accumulate<VW, TX, PRO>(x, h, w, cv, b, oy, ox0, q + co_v, wt, bias[q + co_v], pro, gate);
#pragma unroll
        for (int j = 0; j < TX; ++j)
            if (ox0 + j < w) dst[size_t(ox0 + j) * co_v] = V::glu(acc[j], gate[j]);
    } else {
#pragma unroll
        for (int j = 0; j < TX; ++j)
            if (ox0 + j < w) dst[size_t(ox0 + j) * co_v] = EPI == 1 ? V::relu(acc[j]) : acc[j];
    }
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
    switch (epilogue) {
        case 0: depthwise_kernel<VW, TX, 0, PRO><<<blocks, 256, 0, ctx.stream>>>(xv, n, h, w, cv, wv, bv, pro, ov); break;
        case 1: depthwise_kernel<VW, TX, 1, PRO><<<blocks, 256, 0, ctx.stream>>>(xv, n, h, w, cv, wv, bv, pro, ov); break;
        default: depthwise_kernel<VW, TX, 2, PRO><<<blocks, 256, 0, ctx.stream>>>(xv, n, h, w, cv, wv, bv, pro, ov); break;
    }
    MH_LAUNCH_CHECK();
}

}  // namespace

void depthwise3x3(Context &ctx, const float *x, int n, int h, int w, int c, const float *weight, const float *bias,
                  int epilogue, float *out, const Affine *prologue) {
    MH_REQUIRE(epilogue >= 0 && epilogue <= 2, "depthwise: unknown epilogue");
    if (epilogue == 2) MH_REQUIRE(c % 2 == 0, "GLU needs an even channel count");
    if (int64_t(n) * h * w * c == 0) return;
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
    if (vec4) {
        if (prologue) launch_dw<4, 4, true>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
        else launch_dw<4, 4, false>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
    } else {
        if (prologue) launch_dw<1, 4, true>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
        else launch_dw<1, 4, false>(ctx, x, n, h, w, c, weight, bias, epilogue, pro, out);
    }
}

}  // namespace mh
