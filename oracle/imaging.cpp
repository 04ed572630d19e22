// Oracle restatement of the window resampling of src/imaging/resize.rs:15-24
// (fast_image_resize 6.1.0, Lanczos3, documented as PIL's LANCZOS convolution):
// Pillow's ImagingResample for 8-bit images, separable passes horizontal then
// vertical, weights normalised in double and rounded to 22-bit fixed point,
// each pass rounded and clamped to 8 bits. Test infrastructure only: see oracle.h.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "oracle.h"

namespace {

constexpr int PRECISION_BITS = 22;

double sinc(double x) {
    if (x == 0.0) return 1.0;
    x = x * M_PI;
    return std::sin(x) / x;
}

double lanczos(double x) {
    if (-3.0 <= x && x < 3.0) return sinc(x) * sinc(x / 3);
    return 0.0;
}

// Pillow precompute_coeffs + normalize_coeffs_8bpc over the whole axis.
int precompute(int in_size, int out_size, std::vector<int> &bounds, std::vector<int32_t> &kk) {
    double scale = double(in_size) / out_size, filterscale = scale;
    if (filterscale < 1.0) filterscale = 1.0;
    const double support = 3.0 * filterscale;
    const int ksize = int(std::ceil(support)) * 2 + 1;
    bounds.assign(size_t(out_size) * 2, 0);
    kk.assign(size_t(out_size) * ksize, 0);
    std::vector<double> k(static_cast<size_t>(ksize));
    for (int xx = 0; xx < out_size; xx++) {
        const double center = (xx + 0.5) * scale;
        double ww = 0.0;
        const double ss = 1.0 / filterscale;
        int xmin = int(center - support + 0.5);
        if (xmin < 0) xmin = 0;
        int xmax = int(center + support + 0.5);
        if (xmax > in_size) xmax = in_size;
        xmax -= xmin;
        for (int x = 0; x < xmax; x++) {
            const double w = lanczos((x + xmin - center + 0.5) * ss);
            k[size_t(x)] = w;
            ww += w;
        }
        for (int x = 0; x < xmax; x++) {
            if (ww != 0.0) k[size_t(x)] /= ww;
            const double v = k[size_t(x)];
            kk[size_t(xx) * ksize + x] = v < 0 ? int32_t(-0.5 + v * (1 << PRECISION_BITS))
                                               : int32_t(0.5 + v * (1 << PRECISION_BITS));
        }
        bounds[size_t(xx) * 2] = xmin;
        bounds[size_t(xx) * 2 + 1] = xmax;
    }
    return ksize;
}

uint8_t clip8(int32_t v) {
    const int32_t s = v >> PRECISION_BITS;
    return uint8_t(s < 0 ? 0 : (s > 255 ? 255 : s));
}

}  // namespace

extern "C" void orc_resize_u8(const uint8_t *src, int from_w, int from_h, int to_w, int to_h, int channels,
                              uint8_t *dst) {
    if (from_w == to_w && from_h == to_h) {
        std::memcpy(dst, src, size_t(from_w) * from_h * channels);
        return;
    }
    std::vector<int> bh, bv;
    std::vector<int32_t> kh, kv;
    const int ksh = precompute(from_w, to_w, bh, kh), ksv = precompute(from_h, to_h, bv, kv);
    std::vector<uint8_t> tmp(size_t(to_w) * from_h * channels);
    for (int y = 0; y < from_h; y++)
        for (int xx = 0; xx < to_w; xx++) {
            const int xmin = bh[size_t(xx) * 2], n = bh[size_t(xx) * 2 + 1];
            for (int c = 0; c < channels; c++) {
                int32_t ss = 1 << (PRECISION_BITS - 1);
                for (int x = 0; x < n; x++)
                    ss += int32_t(src[(size_t(y) * from_w + xmin + x) * channels + c]) * kh[size_t(xx) * ksh + x];
                tmp[(size_t(y) * to_w + xx) * channels + c] = clip8(ss);
            }
        }
    const size_t row = size_t(to_w) * channels;
    for (int yy = 0; yy < to_h; yy++) {
        const int ymin = bv[size_t(yy) * 2], n = bv[size_t(yy) * 2 + 1];
        for (size_t b = 0; b < row; b++) {
            int32_t ss = 1 << (PRECISION_BITS - 1);
            for (int y = 0; y < n; y++) ss += int32_t(tmp[size_t(ymin + y) * row + b]) * kv[size_t(yy) * ksv + y];
            dst[size_t(yy) * row + b] = clip8(ss);
        }
    }
}
