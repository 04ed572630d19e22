// Direct 3x3 conv (stride 1, pad 1) for a handful of output channels: the
// reference's Conv3x3 (src/engine/conv.rs:60-102) where c_out <= 8, i.e. the
// VAE decoder's image conv (128 -> 3 channels at 512x512). An implicit GEMM
// pads N = 3 to its 128-wide tile and wastes 97% of its matrix work (680 us
// at 512x512); here each thread computes every output channel of one pixel
// with vector FMAs, the input staged through LDS once per 16x16 tile.
//
// The optional GroupNorm(+SiLU) prologue is applied to in-image values as they
// are staged (padding stays 0, as the reference's prologue: winograd.rs:210-251),
// so the normalised map is never written.
#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

constexpr int kST = 16;            // output tile side (one pixel per thread)
constexpr int kSH = kST + 2;       // staged tile side
constexpr int kSP = kSH * kSH;     // staged pixels
constexpr int kSQ = 4;             // channel quads per chunk (16 channels)

// Per thread: pixel (ty0 + tid / 16, tx0 + tid % 16) of tile blockIdx.x (item,
// tile row, tile column); out = (bias + sum over chunks of channels, taps in
// (ky, kx) order, channels in order) (+ res2).
template <int CO, bool PRO, bool F16>
__global__ __launch_bounds__(256) void conv3x3_small_kernel(const float *__restrict__ x, int h, int w, int ci,
                                                            const void *__restrict__ wt, const float *__restrict__ bias,
                                                            const float *__restrict__ psc,
                                                            const float *__restrict__ psh, int psilu,
                                                            const float *__restrict__ res2, float *__restrict__ out,
                                                            int tiles_x, int tiles_y) {
    // [quad][pixel]: consecutive pixels of a quad are consecutive 16-byte
    // slots, so the compute loop's reads (one pixel per lane) are conflict free.
    __shared__ float4 xs[kSQ * kSP];
    const int tid = threadIdx.x;
    const int per_item = tiles_x * tiles_y;
    const int b = int(blockIdx.x) / per_item, rem = int(blockIdx.x) - b * per_item;
    const int ty0 = (rem / tiles_x) * kST, tx0 = (rem % tiles_x) * kST;
    const int py = tid / kST, px = tid % kST;
    const float4 *__restrict__ xv = reinterpret_cast<const float4 *>(x);
    auto weight4 = [&](int o, int tap, int c) -> float4 {
        const int64_t i = (int64_t(o) * 9 + tap) * ci + c;
        if constexpr (F16) {
            const _Float16 *p = static_cast<const _Float16 *>(wt) + i;
            return make_float4(float(p[0]), float(p[1]), float(p[2]), float(p[3]));
        } else {
            return *reinterpret_cast<const float4 *>(static_cast<const float *>(wt) + i);
        }
    };
    float acc[CO];
#pragma unroll
    for (int o = 0; o < CO; ++o) acc[o] = 0.f;
    for (int c0 = 0; c0 < ci; c0 += 4 * kSQ) {
        __syncthreads();  // the previous chunk's reads are done
        for (int e = tid; e < kSQ * kSP; e += 256) {
            const int q = e % kSQ, pix = e / kSQ;  // a pixel's quads on adjacent threads: 64-byte runs
            const int sy = ty0 - 1 + pix / kSH, sx = tx0 - 1 + pix % kSH;
            const int c = c0 + 4 * q;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sy >= 0 && sy < h && sx >= 0 && sx < w && c < ci) {
                v = xv[(((int64_t(b) * h + sy) * w + sx) * ci + c) >> 2];
                if constexpr (PRO) {
                    const float4 s = *reinterpret_cast<const float4 *>(psc + int64_t(b) * ci + c);
                    const float4 t = *reinterpret_cast<const float4 *>(psh + int64_t(b) * ci + c);
                    v.x = __builtin_fmaf(v.x, s.x, t.x);
                    v.y = __builtin_fmaf(v.y, s.y, t.y);
                    v.z = __builtin_fmaf(v.z, s.z, t.z);
                    v.w = __builtin_fmaf(v.w, s.w, t.w);
                    if (psilu) v = make_float4(ref_silu(v.x), ref_silu(v.y), ref_silu(v.z), ref_silu(v.w));
                }
            }
            xs[q * kSP + pix] = v;
        }
        __syncthreads();
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int ky = tap / 3, kx = tap - 3 * ky;
            const float4 *src = xs + (py + ky) * kSH + px + kx;
#pragma unroll
            for (int q = 0; q < kSQ; ++q) {
                const int c = c0 + 4 * q;
                if (c >= ci) break;  // uniform: ci % 4 == 0
                const float4 a = src[q * kSP];
#pragma unroll
                for (int o = 0; o < CO; ++o) {
                    const float4 wv = weight4(o, tap, c);
                    float s = acc[o];
                    s = __builtin_fmaf(a.x, wv.x, s);
                    s = __builtin_fmaf(a.y, wv.y, s);
                    s = __builtin_fmaf(a.z, wv.z, s);
                    s = __builtin_fmaf(a.w, wv.w, s);
                    acc[o] = s;
                }
            }
        }
    }
    const int y = ty0 + py, xx = tx0 + px;
    if (y >= h || xx >= w) return;
    const int64_t o0 = ((int64_t(b) * h + y) * w + xx) * CO;
#pragma unroll
    for (int o = 0; o < CO; ++o) {
        float r = bias ? bias[o] + acc[o] : acc[o];
        if (res2) r = r + res2[o0 + o];
        out[o0 + o] = r;
    }
}

template <int CO>
void launch_small(Context &ctx, const float *x, int n, int h, int w, int ci, const void *wt, WeightType wtype,
                  const float *bias, const Affine *pro, const float *res2, float *out) {
    const int tx = int(ceil_div(w, kST)), ty = int(ceil_div(h, kST));
    const unsigned grid = unsigned(int64_t(n) * tx * ty);
    const float *sc = pro ? pro->scale : nullptr, *sh = pro ? pro->shift : nullptr;
    const int silu = pro && pro->silu ? 1 : 0;
    if (wtype == kF16) {
        if (pro)
            conv3x3_small_kernel<CO, true, true><<<grid, 256, 0, ctx.stream>>>(x, h, w, ci, wt, bias, sc, sh, silu, res2, out, tx, ty);
        else
            conv3x3_small_kernel<CO, false, true><<<grid, 256, 0, ctx.stream>>>(x, h, w, ci, wt, bias, sc, sh, silu, res2, out, tx, ty);
    } else {
        if (pro)
            conv3x3_small_kernel<CO, true, false><<<grid, 256, 0, ctx.stream>>>(x, h, w, ci, wt, bias, sc, sh, silu, res2, out, tx, ty);
        else
            conv3x3_small_kernel<CO, false, false><<<grid, 256, 0, ctx.stream>>>(x, h, w, ci, wt, bias, sc, sh, silu, res2, out, tx, ty);
    }
    MH_LAUNCH_CHECK();
}

}  // namespace

bool conv3x3_small_co(Context &ctx, const float *x, int n, int h, int w, int c_in, const void *weight, WeightType wt,
                      int c_out, const float *bias, const Affine *prologue, float *out, const float *residual2) {
    // Where it is faster than the implicit GEMM (A/B on MI355X): maps of at
    // least 65536 pixels (256 tiles of 16x16, one per CU); smaller maps leave
    // most CUs idle.
    if (c_out < 1 || c_out > 8 || c_in % 4 != 0 || int64_t(n) * h * w < 65536) return false;
    if (!aligned16(x) || (wt == kF32 && !aligned16(weight)) || (wt == kF16 && (reinterpret_cast<uintptr_t>(weight) & 7)))
        return false;
    if (prologue && (!aligned16(prologue->scale) || !aligned16(prologue->shift))) return false;
    if (int64_t(n) * ceil_div(h, kST) * ceil_div(w, kST) >= (int64_t(1) << 31)) return false;
    switch (c_out) {
    case 1: launch_small<1>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    case 2: launch_small<2>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    case 3: launch_small<3>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    case 4: launch_small<4>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    case 5: launch_small<5>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    case 6: launch_small<6>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    case 7: launch_small<7>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    default: launch_small<8>(ctx, x, n, h, w, c_in, weight, wt, bias, prologue, residual2, out); break;
    }
    return true;
}

}  // namespace mh
