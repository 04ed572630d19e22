// Oracle restatement of moebius-cpu `src/engine` (conv, winograd, depthwise,
// norm, ops, math, tensor) plus `src/imaging/blend.rs::to_u8`.
// Test infrastructure only: see oracle.h.
//
// Build with -ffp-contract=off: the reference (Rust) never contracts a*b+c,
// so every fused multiply-add below is an explicit fmaf where the reference
// writes `mul_add`, and nothing else is fused.
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "oracle.h"

namespace {

// src/engine/math.rs:8-14
constexpr float LOG2_E = 1.44269504088896340736f;
constexpr float LN2_HI = 0.693359375f;
constexpr float LN2_LO = -2.12194440e-4f;
constexpr float MAX_X = 88.0f;
constexpr float MIN_X = -87.33655f;

// src/engine/conv.rs:25-26
constexpr int64_t COLS_BUDGET = int64_t(8) << 20;
constexpr int64_t MAX_BAND = 4096;
// src/engine/winograd.rs:38
constexpr int64_t V_BUDGET = int64_t(4) << 20;
// src/engine/norm.rs:20
constexpr int64_t STATS_CHUNK = 256;

inline float fmax0(float v) {
    // Rust f32::max(v, 0.0): returns 0.0 when v is NaN.
    return std::isnan(v) ? 0.0f : (v > 0.0f ? v : 0.0f);
}

}  // namespace

// src/engine/math.rs:17-30: Cephes range reduction + degree-6 polynomial.
extern "C" float orc_exp(float x) {
    x = std::min(std::max(x, MIN_X), MAX_X);
    const float n = std::round(x * LOG2_E);  // f32::round: half away from zero
    const float r = std::fma(n, -LN2_LO, std::fma(n, -LN2_HI, x));
    float p = 1.9875691e-4f;
    p = std::fma(p, r, 1.3981999e-3f);
    p = std::fma(p, r, 8.333452e-3f);
    p = std::fma(p, r, 4.1665796e-2f);
    p = std::fma(p, r, 1.6666665e-1f);
    p = std::fma(p, r, 5e-1f);
    const float poly = std::fma(p * r, r, r) + 1.0f;
    const uint32_t bits = uint32_t(int32_t(n) + 127) << 23;
    float scale;
    std::memcpy(&scale, &bits, sizeof(scale));
    return poly * scale;
}

// src/engine/math.rs:33-36
extern "C" float orc_silu(float x) { return x / (1.0f + orc_exp(-x)); }

// src/engine/conv.rs:170-191
extern "C" int orc_init_output(float *out, int64_t rows, int64_t cols, const float *bias, const float *residual) {
    if (!bias && !residual) return 0;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float *o = out + r * cols;
        if (bias && residual) {
            const float *rr = residual + r * cols;
            for (int64_t j = 0; j < cols; ++j) o[j] = rr[j] + bias[j];
        } else if (bias) {
            std::memcpy(o, bias, cols * sizeof(float));
        } else {
            std::memcpy(o, residual + r * cols, cols * sizeof(float));
        }
    }
    return 1;
}

// src/engine/conv.rs:38-55: out = x . W^T + bias (+ residual), W [c_out, c_in].
extern "C" void orc_conv1x1(const float *x, int64_t pixels, int64_t c_in, const float *weight, int64_t c_out,
                            const float *bias, const float *residual, float *out) {
    const int acc = orc_init_output(out, pixels, c_out, bias, residual);
    // MatRef::transposed(w, c_in, c_out): element (p, j) at w[j * c_in + p].
    orc_matmul(out, x, c_in, 1, weight, 1, c_in, pixels, c_in, c_out, acc);
}

// src/engine/conv.rs:77-81
extern "C" void orc_conv3x3_output_hw(int64_t h, int64_t w, int stride, const int pad[4], int upsample2x,
                                      int64_t *ho, int64_t *wo) {
    const int64_t up = upsample2x ? 2 : 1;
    *ho = (h * up + pad[0] + pad[2] - 3) / stride + 1;
    *wo = (w * up + pad[1] + pad[3] - 3) / stride + 1;
}

// src/engine/conv.rs:145-165: patch row order [ky][kx][c], zero outside the
// (optionally 2x-upsampled) image; the source pixel of upsampled (iy, ix) is
// (iy >> 1, ix >> 1). Negative coordinates wrap to huge values and fail the
// bounds test, as the reference's wrapping_sub.
extern "C" void orc_im2col_gather_row(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, int64_t ho,
                                      int64_t wo, int stride, int pad_top, int pad_left, int upsample2x, int64_t p,
                                      float *row) {
    (void)n;
    const int64_t b = p / (ho * wo), rem = p % (ho * wo);
    const int64_t oy = rem / wo, ox = rem % wo;
    const int shift = upsample2x ? 1 : 0;
    const uint64_t hi = uint64_t(h) << shift, wi = uint64_t(w) << shift;
    for (int ky = 0; ky < 3; ++ky) {
        const uint64_t iy = uint64_t(oy * stride + ky) - uint64_t(pad_top);
        for (int kx = 0; kx < 3; ++kx) {
            const uint64_t ix = uint64_t(ox * stride + kx) - uint64_t(pad_left);
            float *dst = row + (ky * 3 + kx) * c;
            if (iy < hi && ix < wi) {
                const int64_t src = ((b * h + int64_t(iy >> shift)) * w + int64_t(ix >> shift)) * c;
                std::memcpy(dst, x + src, c * sizeof(float));
            } else {
                std::memset(dst, 0, c * sizeof(float));
            }
        }
    }
}

// src/engine/conv.rs:106-130
extern "C" void orc_conv3x3_im2col(const float *x, int64_t n, int64_t h, int64_t w, int64_t c_in,
                                   const float *weight, int64_t c_out, const float *bias, int stride,
                                   const int pad[4], int upsample2x, float *out) {
    const int64_t k = 9 * c_in;
    int64_t ho, wo;
    orc_conv3x3_output_hw(h, w, stride, pad, upsample2x, &ho, &wo);
    const int64_t total = n * ho * wo;
    const int64_t band = std::min(std::clamp(COLS_BUDGET / k, int64_t(64), MAX_BAND), total);
    std::vector<float> cols(size_t(band * k));
    for (int64_t start = 0; start < total; start += band) {
        const int64_t m = std::min(band, total - start);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < m; ++i)
            orc_im2col_gather_row(x, n, h, w, c_in, ho, wo, stride, pad[0], pad[1], upsample2x, start + i,
                                  cols.data() + i * k);
        float *dst = out + start * c_out;
        const int acc = orc_init_output(dst, m, c_out, bias, nullptr);
        orc_matmul(dst, cols.data(), k, 1, weight, 1, k, m, k, c_out, acc);
    }
}

// src/engine/winograd.rs:269-297: U = G g G^T, G = [[1,0,0],[1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]].
// g: [3, 3, c] -> u: [16, c].
extern "C" void orc_wino_kernel_transform(const float *g, int64_t c, float *u) {
    for (int64_t i = 0; i < c; ++i) {
        float t[4][3];
        for (int kx = 0; kx < 3; ++kx) {
            const float g0 = g[kx * c + i], g1 = g[(3 + kx) * c + i], g2 = g[(6 + kx) * c + i];
            t[0][kx] = g0;
            t[1][kx] = 0.5f * (g0 + g1 + g2);
            t[2][kx] = 0.5f * (g0 - g1 + g2);
            t[3][kx] = g2;
        }
        for (int a = 0; a < 4; ++a) {
            u[(a * 4) * c + i] = t[a][0];
            u[(a * 4 + 1) * c + i] = 0.5f * (t[a][0] + t[a][1] + t[a][2]);
            u[(a * 4 + 2) * c + i] = 0.5f * (t[a][0] - t[a][1] + t[a][2]);
            u[(a * 4 + 3) * c + i] = t[a][2];
        }
    }
}

// src/engine/winograd.rs:299-327: V = B^T d B, d[r*4+col] = input row r, column col.
extern "C" void orc_wino_input_transform(const float *const d[16], int64_t c, float *v) {
    for (int64_t i = 0; i < c; ++i) {
        float t[16];
        for (int col = 0; col < 4; ++col) {
            const float d0 = d[col][i], d1 = d[4 + col][i], d2 = d[8 + col][i], d3 = d[12 + col][i];
            t[col] = d0 - d2;
            t[4 + col] = d1 + d2;
            t[8 + col] = d2 - d1;
            t[12 + col] = d1 - d3;
        }
        for (int r = 0; r < 4; ++r) {
            const float *q = t + r * 4;
            v[(r * 4) * c + i] = q[0] - q[2];
            v[(r * 4 + 1) * c + i] = q[1] + q[2];
            v[(r * 4 + 2) * c + i] = q[2] - q[1];
            v[(r * 4 + 3) * c + i] = q[1] - q[3];
        }
    }
}

// src/engine/winograd.rs:329-352: Y = A^T m A + bias into y [4][c], A^T = [[1,1,1,0],[0,1,-1,-1]].
extern "C" void orc_wino_output_transform(const float *const m[16], const float *bias, int64_t c, float *y) {
    for (int64_t i = 0; i < c; ++i) {
        float u0[4], u1[4];
        for (int r = 0; r < 4; ++r) {
            const float a = m[r * 4][i], b = m[r * 4 + 1][i], cc = m[r * 4 + 2][i], d = m[r * 4 + 3][i];
            u0[r] = a + b + cc;
            u1[r] = b - cc - d;
        }
        y[i] = u0[0] + u0[1] + u0[2] + bias[i];
        y[c + i] = u1[0] + u1[1] + u1[2] + bias[i];
        y[2 * c + i] = u0[1] - u0[2] - u0[3] + bias[i];
        y[3 * c + i] = u1[1] - u1[2] - u1[3] + bias[i];
    }
}

// src/engine/norm.rs:132-148: dst = [SiLU](src . scale + shift), fused multiply-add.
extern "C" void orc_apply_affine(const float *src, int64_t pixels, int64_t c, const float *scale, const float *shift,
                                 int silu, float *dst) {
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < pixels; ++p) {
        const float *s = src + p * c;
        float *d = dst + p * c;
        if (silu) {
            for (int64_t j = 0; j < c; ++j) d[j] = orc_silu(std::fma(s[j], scale[j], shift[j]));
        } else {
            for (int64_t j = 0; j < c; ++j) d[j] = std::fma(s[j], scale[j], shift[j]);
        }
    }
}

// src/engine/winograd.rs:48-120 (with Geo::input_tile 144-160, output_band
// 164-202, fill_strip 210-251). Bands of whole tile rows bound the V/M
// buffers exactly as the reference (winograd.rs:68); the transformed kernel is
// built once for all output channels (the reference splits it into blocks
// when it exceeds U_BUDGET, which changes memory, not arithmetic). The GroupNorm
// prologue is applied to every in-image value gathered (the reference
// normalises the band's rows into a strip first, the same values); padding
// stays zero.
extern "C" void orc_winograd_conv3x3_same(const float *x, int64_t n, int64_t h, int64_t w, int64_t ci,
                                          const float *psc, const float *psh, int psilu, int upsample2x,
                                          const float *weight, const float *bias, int64_t c_out, float *out) {
    const int shift = upsample2x ? 1 : 0;
    const int64_t hi = h << shift, wi = w << shift;
    const int64_t th = (hi + 1) / 2, tw = (wi + 1) / 2;
    const int64_t tiles = n * th * tw;
    int64_t band = std::max<int64_t>(std::clamp(V_BUDGET / (16 * ci), int64_t(256), int64_t(4096)) / tw, 1) * tw;
    band = std::min(band, tiles);

    std::vector<float> u(size_t(16 * c_out * ci));
    std::vector<float> bias_zero;
    if (!bias) {
        bias_zero.assign(size_t(c_out), 0.0f);
        bias = bias_zero.data();
    }
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < c_out; ++o) orc_wino_kernel_transform(weight + o * 9 * ci, ci, u.data() + o * 16 * ci);

    std::vector<float> v(size_t(16 * band * ci));
    std::vector<float> mbuf(size_t(16 * band * c_out));
    for (int64_t t0 = 0; t0 < tiles; t0 += band) {
        const int64_t mb = std::min(band, tiles - t0);
#pragma omp parallel
        {
            std::vector<float> zeros(static_cast<size_t>(ci), 0.0f), norm(psc ? static_cast<size_t>(16 * ci) : 0);
#pragma omp for schedule(static)
            for (int64_t i = 0; i < mb; ++i) {
                const int64_t t = t0 + i;
                const int64_t b = t / (th * tw), rem = t % (th * tw);
                const int64_t ty = rem / tw, tx = rem % tw;
                const float *rows[16];
                for (int kk = 0; kk < 16; ++kk) {
                    const int64_t iy = 2 * ty + kk / 4 - 1, ix = 2 * tx + kk % 4 - 1;
                    if (iy >= 0 && iy < hi && ix >= 0 && ix < wi) {
                        const float *src = x + ((b * h + (iy >> shift)) * w + (ix >> shift)) * ci;
                        if (psc) {
                            float *dst = norm.data() + kk * ci;
                            const float *sc = psc + b * ci, *sh = psh + b * ci;
                            for (int64_t j = 0; j < ci; ++j) {
                                const float y = std::fma(src[j], sc[j], sh[j]);
                                dst[j] = psilu ? orc_silu(y) : y;
                            }
                            rows[kk] = dst;
                        } else {
                            rows[kk] = src;
                        }
                    } else {
                        rows[kk] = zeros.data();
                    }
                }
                orc_wino_input_transform(rows, ci, v.data() + i * 16 * ci);
            }
        }
        // 16 GEMMs, plane xi: [mb x ci] . [ci x c_out] (winograd.rs:111-115).
        for (int xi = 0; xi < 16; ++xi) {
            orc_matmul(mbuf.data() + int64_t(xi) * mb * c_out, v.data() + xi * ci, 16 * ci, 1, u.data() + xi * ci, 1,
                       16 * ci, mb, ci, c_out, 0);
        }
#pragma omp parallel
        {
            std::vector<float> y(static_cast<size_t>(4 * c_out));
#pragma omp for schedule(static)
            for (int64_t lt = 0; lt < mb; ++lt) {
                const int64_t t = t0 + lt;
                const int64_t b = t / (th * tw), rem = t % (th * tw);
                const int64_t ty = rem / tw, tx = rem % tw;
                const float *planes[16];
                for (int xi = 0; xi < 16; ++xi) planes[xi] = mbuf.data() + (int64_t(xi) * mb + lt) * c_out;
                orc_wino_output_transform(planes, bias, c_out, y.data());
                for (int kk = 0; kk < 4; ++kk) {
                    const int64_t oy = 2 * ty + kk / 2, ox = 2 * tx + kk % 2;
                    if (oy >= hi || ox >= wi) continue;
                    std::memcpy(out + ((b * hi + oy) * wi + ox) * c_out, y.data() + kk * c_out, c_out * sizeof(float));
                }
            }
        }
    }
}

// Whole-map forms of the Winograd transforms above, in the device library's
// plane-major layout (test infrastructure: they pin mh_winograd_*_transform bit
// for bit). Tiles and their 4x4 patches follow orc_winograd_conv3x3_same.
// u [16][c_out][ci] from weight [c_out][3][3][ci].
extern "C" void orc_wino_kernel_transform_all(const float *weight, int64_t c_out, int64_t ci, float *u) {
    std::vector<float> one(size_t(16 * ci));
    for (int64_t o = 0; o < c_out; ++o) {
        orc_wino_kernel_transform(weight + o * 9 * ci, ci, one.data());
        for (int xi = 0; xi < 16; ++xi)
            std::memcpy(u + (xi * c_out + o) * ci, one.data() + xi * ci, size_t(ci) * sizeof(float));
    }
}

// v [16][tiles][ci] from x [n][h][w][ci] (GroupNorm prologue on in-image values).
extern "C" void orc_wino_input_transform_all(const float *x, int64_t n, int64_t h, int64_t w, int64_t ci,
                                             int upsample2x, const float *psc, const float *psh, int psilu,
                                             float *v) {
    const int shift = upsample2x ? 1 : 0;
    const int64_t hi = h << shift, wi = w << shift;
    const int64_t th = (hi + 1) / 2, tw = (wi + 1) / 2;
    const int64_t tiles = n * th * tw;
    std::vector<float> zeros(size_t(ci), 0.0f), norm(size_t(16 * ci)), one(size_t(16 * ci));
    for (int64_t t = 0; t < tiles; ++t) {
        const int64_t b = t / (th * tw), rem = t % (th * tw);
        const int64_t ty = rem / tw, tx = rem % tw;
        const float *rows[16];
        for (int kk = 0; kk < 16; ++kk) {
            const int64_t iy = 2 * ty + kk / 4 - 1, ix = 2 * tx + kk % 4 - 1;
            if (iy >= 0 && iy < hi && ix >= 0 && ix < wi) {
                const float *src = x + ((b * h + (iy >> shift)) * w + (ix >> shift)) * ci;
                if (psc) {
                    float *dst = norm.data() + kk * ci;
                    for (int64_t j = 0; j < ci; ++j) {
                        const float y = std::fma(src[j], psc[b * ci + j], psh[b * ci + j]);
                        dst[j] = psilu ? orc_silu(y) : y;
                    }
                    rows[kk] = dst;
                } else {
                    rows[kk] = src;
                }
            } else {
                rows[kk] = zeros.data();
            }
        }
        orc_wino_input_transform(rows, ci, one.data());
        for (int xi = 0; xi < 16; ++xi)
            std::memcpy(v + (xi * tiles + t) * ci, one.data() + xi * ci, size_t(ci) * sizeof(float));
    }
}

// out [n][H][W][c_out] from m [16][tiles][c_out]; partial-tile pixels skipped.
extern "C" void orc_wino_output_transform_all(const float *m, int64_t n, int64_t h, int64_t w, int64_t c_out,
                                              int upsample2x, const float *bias, float *out) {
    const int shift = upsample2x ? 1 : 0;
    const int64_t hi = h << shift, wi = w << shift;
    const int64_t th = (hi + 1) / 2, tw = (wi + 1) / 2;
    const int64_t tiles = n * th * tw;
    std::vector<float> y(size_t(4 * c_out)), zero(size_t(c_out), 0.0f);
    if (!bias) bias = zero.data();
    for (int64_t t = 0; t < tiles; ++t) {
        const int64_t b = t / (th * tw), rem = t % (th * tw);
        const int64_t ty = rem / tw, tx = rem % tw;
        const float *planes[16];
        for (int xi = 0; xi < 16; ++xi) planes[xi] = m + (xi * tiles + t) * c_out;
        orc_wino_output_transform(planes, bias, c_out, y.data());
        for (int kk = 0; kk < 4; ++kk) {
            const int64_t oy = 2 * ty + kk / 2, ox = 2 * tx + kk % 2;
            if (oy >= hi || ox >= wi) continue;
            std::memcpy(out + ((b * hi + oy) * wi + ox) * c_out, y.data() + kk * c_out, c_out * sizeof(float));
        }
    }
}

// src/engine/conv.rs:92-102
extern "C" void orc_conv3x3_forward(const float *x, int64_t n, int64_t h, int64_t w, int64_t c_in,
                                    const float *weight, int64_t c_out, const float *bias, int stride,
                                    const int pad[4], int upsample2x, const float *psc, const float *psh, int psilu,
                                    float *out) {
    if (stride == 1 && pad[0] == 1 && pad[1] == 1 && pad[2] == 1 && pad[3] == 1) {
        orc_winograd_conv3x3_same(x, n, h, w, c_in, psc, psh, psilu, upsample2x, weight, bias, c_out, out);
    } else {
        orc_conv3x3_im2col(x, n, h, w, c_in, weight, c_out, bias, stride, pad, upsample2x, out);
    }
}

// src/engine/depthwise.rs:31-185: y = bias + sum over taps (ky, then kx) of
// w . x with fused multiply-add, taps outside the image skipped; epilogue
// 0 none, 1 ReLU, 2 GLU: y[:c/2] * SiLU(y[c/2:]).
extern "C" void orc_depthwise3x3(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, const float *weight,
                                 const float *bias, int epilogue, float *out) {
    const int64_t c_out = epilogue == 2 ? c / 2 : c;
#pragma omp parallel
    {
        std::vector<float> acc(static_cast<size_t>(c));
#pragma omp for collapse(2) schedule(static)
        for (int64_t b = 0; b < n; ++b) {
            for (int64_t oy = 0; oy < h; ++oy) {
                for (int64_t ox = 0; ox < w; ++ox) {
                    std::memcpy(acc.data(), bias, c * sizeof(float));
                    for (int ky = 0; ky < 3; ++ky) {
                        const int64_t iy = oy + ky - 1;
                        if (iy < 0 || iy >= h) continue;
                        for (int kx = 0; kx < 3; ++kx) {
                            const int64_t ix = ox + kx - 1;
                            if (ix < 0 || ix >= w) continue;
                            const float *src = x + ((b * h + iy) * w + ix) * c;
                            const float *tap = weight + (ky * 3 + kx) * c;
                            for (int64_t j = 0; j < c; ++j) acc[j] = std::fma(tap[j], src[j], acc[j]);
                        }
                    }
                    float *dst = out + ((b * h + oy) * w + ox) * c_out;
                    if (epilogue == 0) {
                        std::memcpy(dst, acc.data(), c * sizeof(float));
                    } else if (epilogue == 1) {
                        for (int64_t j = 0; j < c; ++j) dst[j] = fmax0(acc[j]);
                    } else {
                        for (int64_t j = 0; j < c_out; ++j) dst[j] = acc[j] * orc_silu(acc[c_out + j]);
                    }
                }
            }
        }
    }
}

// src/engine/norm.rs:57-105, gn_stats 108-130. Per item: per-channel f32
// sums of y and y*y (fused) over 256-pixel chunks, each chunk folded into f64
// per group, chunks summed in f64 (in chunk order; the reference reduces them
// in a rayon tree, an f64-rounding-level difference).
extern "C" void orc_group_norm_affine(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, int64_t groups,
                                      float eps, const float *gamma, const float *beta, const float *add,
                                      float *scale, float *shift) {
    const int64_t hw = h * w, cg = c / groups;
    const double count = double(hw * cg);
    const int64_t chunks = (hw + STATS_CHUNK - 1) / STATS_CHUNK;
    std::vector<double> fold(size_t(chunks * groups * 2));
    for (int64_t b = 0; b < n; ++b) {
        const float *src = x + b * hw * c;
        const float *ab = add ? add + b * c : nullptr;
#pragma omp parallel
        {
            std::vector<float> s(static_cast<size_t>(c)), q(static_cast<size_t>(c));
#pragma omp for schedule(static)
            for (int64_t ch = 0; ch < chunks; ++ch) {
                std::fill(s.begin(), s.end(), 0.0f);
                std::fill(q.begin(), q.end(), 0.0f);
                const int64_t p1 = std::min(hw, (ch + 1) * STATS_CHUNK);
                for (int64_t p = ch * STATS_CHUNK; p < p1; ++p) {
                    const float *px = src + p * c;
                    for (int64_t j = 0; j < c; ++j) {
                        const float y = ab ? px[j] + ab[j] : px[j];
                        s[j] += y;
                        q[j] = std::fma(y, y, q[j]);
                    }
                }
                for (int64_t g = 0; g < groups; ++g) {
                    double fs = 0.0, fq = 0.0;
                    for (int64_t j = g * cg; j < (g + 1) * cg; ++j) {
                        fs += double(s[j]);
                        fq += double(q[j]);
                    }
                    fold[size_t((ch * groups + g) * 2)] = fs;
                    fold[size_t((ch * groups + g) * 2 + 1)] = fq;
                }
            }
        }
        for (int64_t g = 0; g < groups; ++g) {
            double sum = 0.0, sumsq = 0.0;
            for (int64_t ch = 0; ch < chunks; ++ch) {
                sum += fold[size_t((ch * groups + g) * 2)];
                sumsq += fold[size_t((ch * groups + g) * 2 + 1)];
            }
            const double mean = sum / count;
            const double var = std::max(sumsq / count - mean * mean, 0.0);
            const double rstd = 1.0 / std::sqrt(var + double(eps));
            for (int64_t j = g * cg; j < (g + 1) * cg; ++j) {
                const double sc = rstd * double(gamma[j]);
                const double pre = ab ? double(ab[j]) : 0.0;
                scale[b * c + j] = float(sc);
                shift[b * c + j] = float(double(beta[j]) + (pre - mean) * sc);
            }
        }
    }
}

// src/engine/norm.rs:41-53
extern "C" void orc_group_norm_forward(const float *x, int64_t n, int64_t h, int64_t w, int64_t c, int64_t groups,
                                       float eps, const float *gamma, const float *beta, const float *add, int silu,
                                       float *out) {
    std::vector<float> scale(size_t(n * c)), shift(size_t(n * c));
    orc_group_norm_affine(x, n, h, w, c, groups, eps, gamma, beta, add, scale.data(), shift.data());
    for (int64_t b = 0; b < n; ++b)
        orc_apply_affine(x + b * h * w * c, h * w, c, scale.data() + b * c, shift.data() + b * c, silu,
                         out + b * h * w * c);
}

// src/engine/norm.rs:151-173: per row, f32 sequential mean, two-pass f32
// variance, rstd = 1/sqrt(var + eps), out = fma((v - mean) * rstd, g, b).
extern "C" void orc_layer_norm(const float *x, int64_t rows, int64_t c, const float *gamma, const float *beta,
                               float eps, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float *s = x + r * c;
        float *d = out + r * c;
        float sum = 0.0f;
        for (int64_t j = 0; j < c; ++j) sum += s[j];
        const float mean = sum / float(c);
        float vs = 0.0f;
        for (int64_t j = 0; j < c; ++j) {
            const float dv = s[j] - mean;
            vs += dv * dv;
        }
        const float var = vs / float(c);
        const float rstd = 1.0f / std::sqrt(var + eps);
        for (int64_t j = 0; j < c; ++j) d[j] = std::fma((s[j] - mean) * rstd, gamma[j], beta[j]);
    }
}

// src/engine/ops.rs:11-19
extern "C" void orc_silu_inplace(float *x, int64_t len) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) x[i] = orc_silu(x[i]);
}

extern "C" void orc_add_inplace(float *a, const float *b, int64_t len) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) a[i] += b[i];
}

// src/engine/tensor.rs:59-73
extern "C" void orc_concat_channels(const float *a, int64_t ca, const float *b, int64_t cb, int64_t pixels,
                                    float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < pixels; ++p) {
        std::memcpy(out + p * (ca + cb), a + p * ca, ca * sizeof(float));
        std::memcpy(out + p * (ca + cb) + ca, b + p * cb, cb * sizeof(float));
    }
}

// src/imaging/blend.rs:21-24: (clamp(v, 0, 1) * 255) truncated; NaN -> 0.
extern "C" void orc_to_u8(const float *x, int64_t len, uint8_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < len; ++i) {
        const float v = x[i];
        if (std::isnan(v)) {
            out[i] = 0;
            continue;
        }
        const float cl = std::min(std::max(v, 0.0f), 1.0f) * 255.0f;
        out[i] = uint8_t(cl);
    }
}
