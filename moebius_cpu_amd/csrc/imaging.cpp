// Host restatement of src/imaging (mod.rs, crop.rs, blend.rs) and of
// src/vae/mod.rs:60-78 (roi_window). The integer and f64 arithmetic follows the
// reference operation by operation, so the results are the same bytes.
#include "imaging.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <exception>
#include <optional>
#include <thread>
#include <vector>

#include "common.hpp"

namespace mh {
namespace img {

namespace {
constexpr size_t kModelSide = 512;   // src/config.rs IMAGE_SIZE
constexpr size_t kBlurMargin = 16;   // src/imaging/blend.rs:112-114
constexpr double kCompensateFac = 1.1;
constexpr size_t kRingOff = 10;
constexpr size_t kLatent = 64;
}  // namespace

bool mask_bbox(const MaskView &m, Rect *out) {
    size_t x0 = SIZE_MAX, y0 = SIZE_MAX, x1 = 0, y1 = 0;
    for (size_t y = 0; y < m.height; ++y) {
        const uint8_t *row = m.data + y * m.stride;
        size_t first = SIZE_MAX, last = 0;
        for (size_t x = 0; x < m.width; ++x) {
            if (row[x] >= 128) {
                if (first == SIZE_MAX) first = x;
                last = x;
            }
        }
        if (first == SIZE_MAX) continue;
        x0 = std::min(x0, first);
        x1 = std::max(x1, last);
        y0 = std::min(y0, y);
        y1 = y;
    }
    if (x0 == SIZE_MAX) return false;
    *out = Rect{x0, y0, x1 - x0 + 1, y1 - y0 + 1};
    return true;
}

std::vector<uint8_t> dilate(const MaskView &m, size_t k) {
    const size_t w = m.width, h = m.height;
    std::vector<uint8_t> cur(w * h);
    for (size_t y = 0; y < h; ++y)
        for (size_t x = 0; x < w; ++x) cur[y * w + x] = m.data[y * m.stride + x] >= 128 ? 255 : 0;
    if (k <= 1 || w == 0 || h == 0) return cur;
    const size_t before = k / 2, after = k - 1 - k / 2;
    // The values are 0 / 255, so a window's max is 255 exactly when it holds a
    // set pixel: prefix counts give each window in O(1).
    std::vector<uint8_t> tmp(w * h);
    std::vector<size_t> pre(std::max(w, h) + 1);
    for (size_t y = 0; y < h; ++y) {
        pre[0] = 0;
        for (size_t x = 0; x < w; ++x) pre[x + 1] = pre[x] + (cur[y * w + x] != 0);
        for (size_t x = 0; x < w; ++x) {
            const size_t lo = x >= before ? x - before : 0, hi = std::min(x + after, w - 1);
            tmp[y * w + x] = pre[hi + 1] - pre[lo] ? 255 : 0;
        }
    }
    for (size_t x = 0; x < w; ++x) {
        pre[0] = 0;
        for (size_t y = 0; y < h; ++y) pre[y + 1] = pre[y] + (tmp[y * w + x] != 0);
        for (size_t y = 0; y < h; ++y) {
            const size_t lo = y >= before ? y - before : 0, hi = std::min(y + after, h - 1);
            cur[y * w + x] = pre[hi + 1] - pre[lo] ? 255 : 0;
        }
    }
    return cur;
}

namespace {
// src/imaging/crop.rs:55-66: centred on the mask, shifted inside the image
// when the window fits, else centred on the image.
int64_t place(size_t start, size_t len, size_t side, size_t extent) {
    if (side <= extent) {
        const int64_t centred = int64_t(2 * start + len) / 2 - int64_t(side) / 2;
        return std::clamp<int64_t>(centred, 0, int64_t(extent - side));
    }
    return -int64_t((side - extent) / 2);
}
}  // namespace

CropPlan crop_plan(const Rect &b, size_t img_w, size_t img_h) {
    const size_t lng = std::max(b.w, b.h);
    const size_t img_long = std::max(img_w, img_h);
    const size_t side = std::min(std::max(lng + 2 * (lng / 2), std::min(kModelSide, img_long)), img_long);
    CropPlan p;
    p.x = place(b.x, b.w, side, img_w);
    p.y = place(b.y, b.h, side, img_h);
    p.side = side;
    return p;
}

Rect source_rect(const CropPlan &p, size_t img_w, size_t img_h) {
    const size_t x0 = size_t(std::max<int64_t>(p.x, 0)), y0 = size_t(std::max<int64_t>(p.y, 0));
    const size_t x1 = std::min(size_t(p.x + int64_t(p.side)), img_w);
    const size_t y1 = std::min(size_t(p.y + int64_t(p.side)), img_h);
    return Rect{x0, y0, x1 - x0, y1 - y0};
}

namespace {

// Pillow _gaussian_blur_radius (Kovesi's box radius for `passes` box blurs),
// float arithmetic with double sqrt / floor as in the C code.
float gaussian_box_radius(float sigma, uint32_t passes) {
    const float sigma2 = sigma * sigma / float(passes);
    const float big_l = float(std::sqrt(12.0 * double(sigma2) + 1.0));
    const float l = float(std::floor((double(big_l) - 1.0) / 2.0));
    float a = (2.0f * l + 1.0f) * (l * (l + 1.0f) - 3.0f * sigma2);
    a /= 6.0f * (sigma2 - (l + 1.0f) * (l + 1.0f));
    return l + a;
}

// One fractional-radius box pass over a line (Pillow ImagingLineBoxBlur8):
// the window [x - r, x + r] plus the two taps just outside it weighted fw,
// edge pixels extended, 24-bit fixed point rounded to 8 bits.
void box_line(const uint8_t *src, uint8_t *dst, size_t n, size_t radius, uint32_t ww, uint32_t fw) {
    const int64_t last = int64_t(n) - 1, r = int64_t(radius);
    auto at = [&](int64_t i) -> uint32_t { return src[std::clamp<int64_t>(i, 0, last)]; };
    uint32_t acc = 0;
    for (int64_t i = -r; i <= r; ++i) acc += at(i);
    for (int64_t x = 0; x < int64_t(n); ++x) {
        const uint32_t far = at(x - r - 1) + at(x + r + 1);
        const uint32_t bulk = acc * ww + far * fw;
        dst[x] = uint8_t((bulk + (1u << 23)) >> 24);
        acc = acc + at(x + r + 1) - at(x - r);
    }
}

// Runs f(first, last) over [0, n) in up to `threads` contiguous row ranges
// (at least 16 rows each), the calling thread taking the first. Every row's
// result depends on that row alone, so the bytes do not depend on the split.
// A range whose thread cannot be started runs on the calling thread; an
// exception inside any range is rethrown here once every thread has joined.
template <class F>
void parallel_rows(size_t n, unsigned threads, F &&f) {
    const size_t t = std::max<size_t>(1, std::min<size_t>(threads, (n + 15) / 16));
    if (t == 1) {
        f(size_t(0), n);
        return;
    }
    const size_t chunk = (n + t - 1) / t;
    std::vector<std::exception_ptr> errors(t);
    auto guarded = [&f, &errors](size_t i, size_t a, size_t b) {
        try {
            f(a, b);
        } catch (...) {
            errors[i] = std::current_exception();
        }
    };
    std::vector<std::thread> pool;
    std::vector<size_t> inline_ranges;  // ranges whose thread could not be started
    pool.reserve(t);
    for (size_t i = 1; i < t; ++i) {
        const size_t a = i * chunk, b = std::min(n, a + chunk);
        if (a >= b) continue;
        try {
            pool.emplace_back(guarded, i, a, b);
        } catch (...) {
            inline_ranges.push_back(i);
        }
    }
    guarded(0, 0, std::min(n, chunk));
    for (size_t i : inline_ranges) guarded(i, i * chunk, std::min(n, i * chunk + chunk));
    for (std::thread &th : pool) th.join();
    for (const std::exception_ptr &e : errors)
        if (e) std::rethrow_exception(e);
}

void box_rows(uint8_t *buf, size_t w, size_t h, float fradius, uint32_t passes, unsigned threads) {
    const size_t radius = size_t(fradius);
    const uint32_t ww = uint32_t(float(1u << 24) / (fradius * 2.0f + 1.0f));
    const uint32_t fw = ((1u << 24) - uint32_t(radius * 2 + 1) * ww) / 2;
    parallel_rows(h, threads, [&](size_t y0, size_t y1) {
        std::vector<uint8_t> tmp(w);
        for (size_t y = y0; y < y1; ++y) {
            uint8_t *row = buf + y * w;
            for (uint32_t p = 0; p < passes; ++p) {
                box_line(row, tmp.data(), w, radius, ww, fw);
                std::copy(tmp.begin(), tmp.end(), row);
            }
        }
    });
}

std::vector<uint8_t> transpose(const std::vector<uint8_t> &src, size_t w, size_t h, unsigned threads) {
    std::vector<uint8_t> out(src.size());
    parallel_rows(w, threads, [&](size_t x0, size_t x1) {
        for (size_t x = x0; x < x1; ++x)
            for (size_t y = 0; y < h; ++y) out[x * h + y] = src[y * w + x];
    });
    return out;
}

// numpy's uint8 cast of a float64: truncation, saturating at 0 and 255, NaN -> 0.
uint8_t u8_of(double v) {
    if (!(v > 0.0)) return 0;
    if (v >= 255.0) return 255;
    return uint8_t(v);
}

}  // namespace

std::vector<uint8_t> gaussian_blur(const uint8_t *src, size_t w, size_t h, float radius, unsigned threads) {
    constexpr uint32_t kPasses = 3;
    std::vector<uint8_t> buf(src, src + w * h);
    if (radius <= 0.0f || w == 0 || h == 0) return buf;
    const float fr = gaussian_box_radius(radius, kPasses);
    box_rows(buf.data(), w, h, fr, kPasses, threads);
    std::vector<uint8_t> t = transpose(buf, w, h, threads);
    box_rows(t.data(), h, w, fr, kPasses, threads);
    return transpose(t, h, w, threads);
}

Rect paste(ImageView &img, const MaskView &mask, const uint8_t *result, const CropPlan &plan, Paste mode,
           unsigned threads) {
    const Rect src = source_rect(plan, img.width, img.height);
    if (src.w == 0 || src.h == 0) return Rect{};
    const size_t ox = size_t(int64_t(src.x) - plan.x), oy = size_t(int64_t(src.y) - plan.y);
    const size_t ch = img.channels, side = plan.side;
    auto result_px = [&](size_t x, size_t y) { return result + ((oy + y) * side + ox + x) * 3; };
    auto dst_px = [&](size_t x, size_t y) { return img.data + (src.y + y) * img.stride + (src.x + x) * ch; };
    if (mode == Paste::None) {
        for (size_t y = 0; y < src.h; ++y)
            for (size_t x = 0; x < src.w; ++x) std::copy(result_px(x, y), result_px(x, y) + 3, dst_px(x, y));
        return src;
    }
    const bool compensate = mode == Paste::FeatherCompensate;
    const uint8_t lo = compensate ? 129 : 128;  // Feather binarises at >= 128, the compensation at > 128
    const size_t rx0 = src.x >= kBlurMargin ? src.x - kBlurMargin : 0;
    const size_t ry0 = src.y >= kBlurMargin ? src.y - kBlurMargin : 0;
    const size_t rx1 = std::min(src.x + src.w + kBlurMargin, img.width);
    const size_t ry1 = std::min(src.y + src.h + kBlurMargin, img.height);
    const size_t rw = rx1 - rx0, rh = ry1 - ry0;
    std::vector<uint8_t> region(rw * rh);
    for (size_t y = ry0; y < ry1; ++y)
        for (size_t x = rx0; x < rx1; ++x) region[(y - ry0) * rw + x - rx0] = mask.data[y * mask.stride + x] >= lo ? 255 : 0;
    const std::vector<uint8_t> blurred = gaussian_blur(region.data(), rw, rh, 3.0f, threads);
    std::optional<std::array<double, 3>> shift;
    if (compensate) {
        // src/imaging/blend.rs:117-153 (ring_delta): the mask bbox grown by 10 px
        // around its centre, clipped to the source rect, minus the mask.
        auto set = [&](size_t x, size_t y) { return region[(src.y + y - ry0) * rw + src.x + x - rx0] != 0; };
        size_t r0 = SIZE_MAX, r1 = 0, c0 = SIZE_MAX, c1 = 0;
        for (size_t y = 0; y < src.h; ++y)
            for (size_t x = 0; x < src.w; ++x)
                if (set(x, y)) r0 = std::min(r0, y), r1 = std::max(r1, y), c0 = std::min(c0, x), c1 = std::max(c1, x);
        if (r0 != SIZE_MAX) {
            const size_t hh = (r1 - r0 + 1 + kRingOff) / 2, hw = (c1 - c0 + 1 + kRingOff) / 2;
            const size_t cr = (r0 + r1) / 2, cc = (c0 + c1) / 2;
            const size_t y0 = cr >= hh ? cr - hh : 0, y1 = std::min(cr + hh, src.h - 1);
            const size_t x0 = cc >= hw ? cc - hw : 0, x1 = std::min(cc + hw, src.w - 1);
            // integer sums: exact in any order, so each thread sums its own rows
            const size_t nr = y1 - y0 + 1;
            const size_t nt = std::max<size_t>(1, std::min<size_t>(threads, (nr + 15) / 16));
            std::vector<std::array<uint64_t, 7>> part(nt, std::array<uint64_t, 7>{});
            const size_t chunk = (nr + nt - 1) / nt;
            parallel_rows(nr, unsigned(nt), [&](size_t a, size_t b) {
                std::array<uint64_t, 7> &q = part[a / chunk];
                for (size_t y = y0 + a; y < y0 + b; ++y)
                    for (size_t x = x0; x <= x1; ++x) {
                        if (set(x, y)) continue;
                        ++q[6];
                        for (int c = 0; c < 3; ++c) q[size_t(c)] += dst_px(x, y)[c], q[3 + size_t(c)] += result_px(x, y)[c];
                    }
            });
            uint64_t ssrc[3] = {0, 0, 0}, sres[3] = {0, 0, 0}, n = 0;
            for (const auto &q : part) {
                for (int c = 0; c < 3; ++c) ssrc[c] += q[size_t(c)], sres[c] += q[3 + size_t(c)];
                n += q[6];
            }
            if (n > 0) {
                std::array<double, 3> d;
                for (int c = 0; c < 3; ++c)
                    d[size_t(c)] = kCompensateFac * (double(ssrc[c]) / double(n) - double(sres[c]) / double(n)) / 255.0;
                shift = d;
            }
        }
    }
    parallel_rows(src.h, threads, [&](size_t ya, size_t yb) {
        for (size_t y = ya; y < yb; ++y)
            for (size_t x = 0; x < src.w; ++x) {
                const double m = double(blurred[(src.y + y - ry0) * rw + src.x + x - rx0]) / 255.0;
                const uint8_t *r = result_px(x, y);
                uint8_t *o = dst_px(x, y);
                for (int c = 0; c < 3; ++c) {
                    double res = double(r[c]) / 255.0;
                    const double orig = double(o[c]) / 255.0;
                    if (shift) res += (*shift)[size_t(c)];
                    double out = res * m + (1.0 - m) * orig;
                    if (shift) out = std::clamp(out, 0.0, 1.0);
                    o[c] = u8_of(out * 255.0);
                }
            }
    });
    return src;
}

bool roi_window(const float *mask_lat, size_t margin, LatentRect *out) {
    size_t x0 = SIZE_MAX, y0 = SIZE_MAX, x1 = 0, y1 = 0;
    for (size_t i = 0; i < kLatent * kLatent; ++i) {
        if (!(mask_lat[i] > 0.5f)) continue;
        const size_t y = i / kLatent, x = i % kLatent;
        x0 = std::min(x0, x), y0 = std::min(y0, y), x1 = std::max(x1, x), y1 = std::max(y1, y);
    }
    if (x0 == SIZE_MAX) return false;
    x0 = x0 >= margin ? x0 - margin : 0;
    y0 = y0 >= margin ? y0 - margin : 0;
    x1 = std::min(x1 + margin, kLatent - 1);
    y1 = std::min(y1 + margin, kLatent - 1);
    *out = LatentRect{x0, y0, x1 - x0 + 1, y1 - y0 + 1};
    return true;
}

}  // namespace img
}  // namespace mh
