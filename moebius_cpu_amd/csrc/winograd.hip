// Winograd F(2x2, 3x3) stride-1 / pad-1 3x3 conv on gfx950 (the CPU engine's
// algorithm for `same` convs, src/engine/winograd.rs:48-120):
//
//   U[16][co][ci] = G g G^T        per output/input channel, once per weight
//                                  (winograd.rs:254-297)
//   V[16][tiles][ci] = B^T d B     per 2x2 output tile, d its 4x4 input patch
//                                  (zero outside the image, nearest-2x upsample
//                                  as a >>1 of the source index, optional
//                                  GroupNorm affine [+SiLU] on in-image values;
//                                  winograd.rs:144-160, 210-251, 299-327)
//   M[xi] = V[xi] . U[xi]^T         16 independent GEMMs [tiles x ci].[ci x co]
//                                  (winograd.rs:111-115): one batched launch of
//                                  the matrix-core GEMM, batch = 16 planes
//   Y = A^T m A + bias             2x2 outputs per tile, partial tiles of odd
//                                  sizes clipped (winograd.rs:164-202, 329-352)
//
// The transforms are elementwise over channels with the reference's operation
// order (f32, written out, no contraction), so U, V and Y given M are bit-equal
// to the CPU engine's; M's sums follow the GEMM kernel's order. Layout: tiles
// are ordered (item, tile row, tile column); each kernel thread handles one
// tile and four adjacent channels with 16-byte accesses, so every read and
// write of V, M and the NHWC maps is a coalesced run of channels.
#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

struct WinoGeo {
    int n, h, w, up;  // input map and upsample shift
    int hi, wi;       // (upsampled) image = output size
    int th, tw;       // tiles per column / row
    int64_t tiles;
};

WinoGeo wino_geo(int n, int h, int w, bool up) {
    WinoGeo g;
    g.n = n, g.h = h, g.w = w, g.up = up ? 1 : 0;
    g.hi = h << g.up, g.wi = w << g.up;
    g.th = (g.hi + 1) / 2, g.tw = (g.wi + 1) / 2;
    g.tiles = int64_t(n) * g.th * g.tw;
    return g;
}

// g: [3][3][c] (row ky, column kx) of one output channel -> u [16][c] (winograd.rs:269-297).
template <bool F16>
__global__ void wino_weight_kernel(const void *__restrict__ w, int co, int ci, float *__restrict__ u) {
    const int64_t total = int64_t(co) * ci;
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
        const int o = int(e / ci), i = int(e - int64_t(o) * ci);
        auto g = [&](int tap) -> float {
            const int64_t idx = (int64_t(o) * 9 + tap) * ci + i;
            if constexpr (F16) return float(static_cast<const _Float16 *>(w)[idx]);
            else return static_cast<const float *>(w)[idx];
        };
        float t[4][3];
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
            const float g0 = g(kx), g1 = g(3 + kx), g2 = g(6 + kx);
            t[0][kx] = g0;
            t[1][kx] = 0.5f * ((g0 + g1) + g2);
            t[2][kx] = 0.5f * ((g0 - g1) + g2);
            t[3][kx] = g2;
        }
        const int64_t plane = int64_t(co) * ci;
        float *dst = u + int64_t(o) * ci + i;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            dst[(a * 4) * plane] = t[a][0];
            dst[(a * 4 + 1) * plane] = 0.5f * ((t[a][0] + t[a][1]) + t[a][2]);
            dst[(a * 4 + 2) * plane] = 0.5f * ((t[a][0] - t[a][1]) + t[a][2]);
            dst[(a * 4 + 3) * plane] = t[a][2];
        }
    }
}

__device__ __forceinline__ float4 f4sub(float4 a, float4 b) { return make_float4(a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w); }
__device__ __forceinline__ float4 f4add(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

// Four V values stored as f32, or (H16, FAST contexts whose plane GEMM takes
// f16 operands) rounded to f16 as that GEMM rounds them: nearest even,
// saturated at +-65504, NaN kept.
template <bool H16>
__device__ __forceinline__ void store_v4(void *v, int64_t i, float4 q) {
    if constexpr (H16) {
        typedef _Float16 half4 __attribute__((ext_vector_type(4)));
        auto r = [](float x) { return static_cast<_Float16>(__builtin_fabsf(x) > 65504.0f ? __builtin_copysignf(65504.0f, x) : x); };
        *reinterpret_cast<half4 *>(static_cast<_Float16 *>(v) + i) = half4{r(q.x), r(q.y), r(q.z), r(q.w)};
    } else {
        *reinterpret_cast<float4 *>(static_cast<float *>(v) + i) = q;
    }
}

// V [16][tiles][ci] (winograd.rs:299-327); one thread per (tile, 4 channels).
template <bool PRO, bool H16>
__global__ __launch_bounds__(256) void wino_input_kernel(const float *__restrict__ x, WinoGeo g, int ci,
                                                         const float *__restrict__ psc, const float *__restrict__ psh,
                                                         int psilu, void *__restrict__ v) {
    const int c4 = ci >> 2;
    const int64_t e = blockIdx.x * int64_t(256) + threadIdx.x;
    if (e >= g.tiles * c4) return;
    const int64_t t = e / c4;
    const int c = int(e - t * c4) * 4;
    const int per_item = g.th * g.tw;
    const int b = int(t / per_item), rem = int(t - int64_t(b) * per_item);
    const int ty = rem / g.tw, tx = rem - (rem / g.tw) * g.tw;
    float4 d[16];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
        const int iy = 2 * ty + (kk >> 2) - 1, ix = 2 * tx + (kk & 3) - 1;
        if (iy >= 0 && iy < g.hi && ix >= 0 && ix < g.wi) {
            const int64_t off = ((int64_t(b) * g.h + (iy >> g.up)) * g.w + (ix >> g.up)) * ci + c;
            float4 q = *reinterpret_cast<const float4 *>(x + off);
            if constexpr (PRO) {
                const float4 sc = *reinterpret_cast<const float4 *>(psc + int64_t(b) * ci + c);
                const float4 sh = *reinterpret_cast<const float4 *>(psh + int64_t(b) * ci + c);
                q.x = __builtin_fmaf(q.x, sc.x, sh.x);
                q.y = __builtin_fmaf(q.y, sc.y, sh.y);
                q.z = __builtin_fmaf(q.z, sc.z, sh.z);
                q.w = __builtin_fmaf(q.w, sc.w, sh.w);
                if (psilu) {
                    q.x = ref_silu(q.x);
                    q.y = ref_silu(q.y);
                    q.z = ref_silu(q.z);
                    q.w = ref_silu(q.w);
                }
            }
            d[kk] = q;
        } else {
            d[kk] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float4 tt[16];
#pragma unroll
    for (int col = 0; col < 4; ++col) {
        const float4 d0 = d[col], d1 = d[4 + col], d2 = d[8 + col], d3 = d[12 + col];
        tt[col] = f4sub(d0, d2);
        tt[4 + col] = f4add(d1, d2);
        tt[8 + col] = f4sub(d2, d1);
        tt[12 + col] = f4sub(d1, d3);
    }
    const int64_t plane = g.tiles * ci;
    const int64_t dst = t * ci + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float4 *q = tt + r * 4;
        store_v4<H16>(v, dst + (r * 4) * plane, f4sub(q[0], q[2]));
        store_v4<H16>(v, dst + (r * 4 + 1) * plane, f4add(q[1], q[2]));
        store_v4<H16>(v, dst + (r * 4 + 2) * plane, f4sub(q[2], q[1]));
        store_v4<H16>(v, dst + (r * 4 + 3) * plane, f4sub(q[1], q[3]));
    }
}

// out = A^T m A + bias (+ res2), winograd.rs:329-352 and Geo::output_band 164-202.
__global__ __launch_bounds__(256) void wino_output_kernel(const float *__restrict__ m, WinoGeo g, int co,
                                                          const float *__restrict__ bias,
                                                          const float *__restrict__ res2, float *__restrict__ out) {
    const int c4 = co >> 2;
    const int64_t e = blockIdx.x * int64_t(256) + threadIdx.x;
    if (e >= g.tiles * c4) return;
    const int64_t t = e / c4;
    const int c = int(e - t * c4) * 4;
    const int per_item = g.th * g.tw;
    const int b = int(t / per_item), rem = int(t - int64_t(b) * per_item);
    const int ty = rem / g.tw, tx = rem - (rem / g.tw) * g.tw;
    const int64_t plane = g.tiles * co;
    const float *src = m + t * co + c;
    float4 u0[4], u1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float4 a = *reinterpret_cast<const float4 *>(src + (r * 4) * plane);
        const float4 bb = *reinterpret_cast<const float4 *>(src + (r * 4 + 1) * plane);
        const float4 cc = *reinterpret_cast<const float4 *>(src + (r * 4 + 2) * plane);
        const float4 dd = *reinterpret_cast<const float4 *>(src + (r * 4 + 3) * plane);
        u0[r] = f4add(f4add(a, bb), cc);
        u1[r] = f4sub(f4sub(bb, cc), dd);
    }
    const float4 bv = bias ? *reinterpret_cast<const float4 *>(bias + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 y[4];
    y[0] = f4add(f4add(f4add(u0[0], u0[1]), u0[2]), bv);
    y[1] = f4add(f4add(f4add(u1[0], u1[1]), u1[2]), bv);
    y[2] = f4add(f4sub(f4sub(u0[1], u0[2]), u0[3]), bv);
    y[3] = f4add(f4sub(f4sub(u1[1], u1[2]), u1[3]), bv);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int oy = 2 * ty + (kk >> 1), ox = 2 * tx + (kk & 1);
        if (oy >= g.hi || ox >= g.wi) continue;
        const int64_t o = ((int64_t(b) * g.hi + oy) * g.wi + ox) * co + c;
        float4 r = y[kk];
        if (res2) r = f4add(r, *reinterpret_cast<const float4 *>(res2 + o));
        *reinterpret_cast<float4 *>(out + o) = r;
    }
}

unsigned blocks_for(int64_t threads) { return unsigned(ceil_div(threads, 256)); }

}  // namespace

int64_t winograd_tiles(int n, int h, int w, bool upsample2x) { return wino_geo(n, h, w, upsample2x).tiles; }

void winograd_weight_transform(Context &ctx, const void *weight, WeightType wt, int c_out, int c_in, float *u) {
    MH_REQUIRE(c_in > 0 && c_out > 0, "Winograd: empty channel axis");
    const int64_t total = int64_t(c_out) * c_in;
    const unsigned blocks = unsigned(std::min<int64_t>(ceil_div(total, 256), 1 << 16));
    if (wt == kF16) wino_weight_kernel<true><<<blocks, 256, 0, ctx.stream>>>(weight, c_out, c_in, u);
    else wino_weight_kernel<false><<<blocks, 256, 0, ctx.stream>>>(weight, c_out, c_in, u);
    MH_LAUNCH_CHECK();
}

void winograd_input_transform(Context &ctx, const float *x, int n, int h, int w, int c, bool upsample2x,
                              const Affine *prologue, void *v, bool h16) {
    MH_REQUIRE(c % 4 == 0 && aligned16(x) && aligned16(v), "Winograd: channels must be a multiple of 4, 16-byte aligned");
    const WinoGeo g = wino_geo(n, h, w, upsample2x);
    if (g.tiles == 0) return;
    const unsigned blocks = blocks_for(g.tiles * (c / 4));
    auto go = [&](auto kern) {
        if (prologue)
            kern<<<blocks, 256, 0, ctx.stream>>>(x, g, c, prologue->scale, prologue->shift, prologue->silu ? 1 : 0, v);
        else
            kern<<<blocks, 256, 0, ctx.stream>>>(x, g, c, nullptr, nullptr, 0, v);
    };
    if (prologue)
        MH_REQUIRE(aligned16(prologue->scale) && aligned16(prologue->shift), "Winograd: prologue must be 16-byte aligned");
    if (h16) prologue ? go(wino_input_kernel<true, true>) : go(wino_input_kernel<false, true>);
    else prologue ? go(wino_input_kernel<true, false>) : go(wino_input_kernel<false, false>);
    MH_LAUNCH_CHECK();
}

void winograd_output_transform(Context &ctx, const float *m, int n, int h, int w, int c_out, bool upsample2x,
                               const float *bias, const float *residual2, float *out) {
    MH_REQUIRE(c_out % 4 == 0 && aligned16(m) && aligned16(out) && aligned16(bias) && aligned16(residual2),
               "Winograd: output channels must be a multiple of 4, 16-byte aligned");
    const WinoGeo g = wino_geo(n, h, w, upsample2x);
    if (g.tiles == 0) return;
    wino_output_kernel<<<blocks_for(g.tiles * (c_out / 4)), 256, 0, ctx.stream>>>(m, g, c_out, bias, residual2, out);
    MH_LAUNCH_CHECK();
}

void conv3x3_winograd(Context &ctx, const float *x, int n, int h, int w, int c_in, const void *u, WeightType ut,
                      int c_out, const float *bias, bool upsample2x, const Affine *prologue, float *out,
                      const float *residual2, const float *uf, GnPartials *gn) {
    if (gn) gn->rows = 0;
    MH_REQUIRE(c_in > 0 && c_out > 0 && c_in % 4 == 0 && c_out % 4 == 0,
               "Winograd conv: channel counts must be multiples of 4");
    const int64_t tiles = winograd_tiles(n, h, w, upsample2x);
    MH_REQUIRE(tiles < (int64_t(1) << 31) && tiles * std::max(c_in, c_out) * 4 < (int64_t(1) << 31),
               "Winograd conv: plane above 2 GiB");
    if (tiles == 0) return;
    // EXACT arithmetic on f32 kernels: the fused kernel, where it takes the shape
    if (ut == kF32 && ctx.precision == Precision::Exact &&
        conv3x3_winograd_fused(ctx, x, n, h, w, c_in, static_cast<const float *>(u), uf, c_out, bias, upsample2x,
                               prologue, out, residual2, gn))
        return;
    // V and M share one workspace block; the batched GEMM (batch > 1) never splits K,
    // so it does not touch the workspace itself. FAST contexts with an f16 U take V in
    // f16 too (tuning wino_v16): the transform rounds it as the plane GEMM would on
    // every load, so the products are the same bits, from half the bytes.
    const bool v16 = ut == kF16 && ctx.precision == Precision::Fast && ctx.tune.wino_v16;
    const size_t vbytes = (size_t(16) * tiles * c_in * (v16 ? 2 : 4) + 255) & ~size_t(255);
    const size_t mbytes = size_t(16) * tiles * c_out * sizeof(float);
    char *ws = static_cast<char *>(ctx.ws.get(vbytes + mbytes, ctx.stream));
    void *v = ws;
    float *m = reinterpret_cast<float *>(ws + vbytes);
    winograd_input_transform(ctx, x, n, h, w, c_in, upsample2x, prologue, v, v16);
    if (v16)
        gemm_nt_a16(ctx, v, c_in, tiles * c_in, u, c_in, int64_t(c_out) * c_in, int(tiles), c_out, c_in, 16, m, c_out,
                    tiles * c_out);
    else
        gemm_nt(ctx, static_cast<const float *>(v), c_in, tiles * c_in, u, ut, c_in, int64_t(c_out) * c_in, int(tiles),
                c_out, c_in, 16, nullptr, nullptr, m, c_out, tiles * c_out);
    winograd_output_transform(ctx, m, n, h, w, c_out, upsample2x, bias, residual2, out);
}

}  // namespace mh
