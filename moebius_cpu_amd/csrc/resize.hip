// Lanczos3 resampling of 8-bit images between the crop window and the 512x512
// model frame (src/imaging/resize.rs:15-24, which calls fast_image_resize 6.1
// with the convolution formulation of PIL's LANCZOS): two separable passes,
// horizontal then vertical, each an integer convolution with 22-bit fixed-point
// weights, rounded and clamped to 8 bits in between. Per output position the
// host computes the tap range and the normalised weights in double (Pillow's
// precompute_coeffs / normalize_coeffs_8bpc); the passes run on the device, one
// thread per output byte group.
#include <cmath>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace mh {

namespace {

constexpr int kPrecisionBits = 32 - 8 - 2;
constexpr double kSupport = 3.0;

double sinc(double x) {
    if (x == 0.0) return 1.0;
    x *= M_PI;
    return std::sin(x) / x;
}

double lanczos3(double x) { return (-3.0 <= x && x < 3.0) ? sinc(x) * sinc(x / 3.0) : 0.0; }

struct Coeffs {
    int ksize = 0;
    std::vector<int32_t> bounds;  // [out][2]: first input index, tap count
    std::vector<int32_t> k;       // [out][ksize]
};

// Tap ranges and fixed-point weights mapping `in` samples onto `out`.
Coeffs coeffs(int in, int out) {
    const double scale = double(in) / double(out);
    const double filterscale = scale < 1.0 ? 1.0 : scale;
    const double support = kSupport * filterscale;
    Coeffs c;
    c.ksize = int(std::ceil(support)) * 2 + 1;
    c.bounds.resize(size_t(out) * 2);
    c.k.assign(size_t(out) * size_t(c.ksize), 0);
    std::vector<double> w(size_t(c.ksize));
    for (int xx = 0; xx < out; ++xx) {
        const double center = (xx + 0.5) * scale;
        const double ss = 1.0 / filterscale;
        int xmin = int(center - support + 0.5);
        if (xmin < 0) xmin = 0;
        int xmax = int(center + support + 0.5);
        if (xmax > in) xmax = in;
        xmax -= xmin;
        double ww = 0.0;
        for (int x = 0; x < xmax; ++x) {
            w[size_t(x)] = lanczos3((x + xmin - center + 0.5) * ss);
            ww += w[size_t(x)];
        }
        for (int x = 0; x < xmax; ++x) {
            const double v = ww != 0.0 ? w[size_t(x)] / ww : w[size_t(x)];
            c.k[size_t(xx) * size_t(c.ksize) + size_t(x)] =
                v < 0 ? int32_t(-0.5 + v * (1 << kPrecisionBits)) : int32_t(0.5 + v * (1 << kPrecisionBits));
        }
        c.bounds[size_t(xx) * 2] = xmin;
        c.bounds[size_t(xx) * 2 + 1] = xmax;
    }
    return c;
}

__device__ __forceinline__ uint8_t clip8(int32_t v) {
    const int32_t s = v >> kPrecisionBits;  // arithmetic shift: floor division
    return uint8_t(s < 0 ? 0 : (s > 255 ? 255 : s));
}

// out [rows][out_w][C] from in [rows][in_w][C]: one thread per (row, output x).
template <int C>
__global__ __launch_bounds__(256) void resample_h_kernel(const uint8_t *__restrict__ in, int in_w, int rows,
                                                         const int32_t *__restrict__ bounds,
                                                         const int32_t *__restrict__ kk, int ksize, int out_w,
                                                         uint8_t *__restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(rows) * out_w) return;
    const int y = int(i / out_w), xx = int(i - int64_t(y) * out_w);
    const int xmin = bounds[2 * xx], n = bounds[2 * xx + 1];
    const int32_t *k = kk + int64_t(xx) * ksize;
    const uint8_t *src = in + (int64_t(y) * in_w + xmin) * C;
    int32_t ss[C];
#pragma unroll
    for (int c = 0; c < C; ++c) ss[c] = 1 << (kPrecisionBits - 1);
    for (int x = 0; x < n; ++x) {
        const int32_t w = k[x];
#pragma unroll
        for (int c = 0; c < C; ++c) ss[c] += int32_t(src[x * C + c]) * w;
    }
    uint8_t *dst = out + (int64_t(y) * out_w + xx) * C;
#pragma unroll
    for (int c = 0; c < C; ++c) dst[c] = clip8(ss[c]);
}

// out [out_h][w * C] from in [in_h][w * C]: one thread per output byte.
__global__ __launch_bounds__(256) void resample_v_kernel(const uint8_t *__restrict__ in, int row_bytes,
                                                         const int32_t *__restrict__ bounds,
                                                         const int32_t *__restrict__ kk, int ksize, int out_h,
                                                         uint8_t *__restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(out_h) * row_bytes) return;
    const int yy = int(i / row_bytes), b = int(i - int64_t(yy) * row_bytes);
    const int ymin = bounds[2 * yy], n = bounds[2 * yy + 1];
    const int32_t *k = kk + int64_t(yy) * ksize;
    int32_t ss = 1 << (kPrecisionBits - 1);
    for (int y = 0; y < n; ++y) ss += int32_t(in[int64_t(ymin + y) * row_bytes + b]) * k[y];
    out[i] = clip8(ss);
}

}  // namespace

void resize_u8(Context &ctx, const uint8_t *src, int from_w, int from_h, int to_w, int to_h, int channels,
               uint8_t *dst) {
    MH_REQUIRE(channels == 1 || channels == 3 || channels == 4, "resize: 1, 3 or 4 channels");
    MH_REQUIRE(from_w > 0 && from_h > 0 && to_w > 0 && to_h > 0, "resize: empty image");
    MH_REQUIRE(src != dst, "resize: output must not alias the input");
    const int64_t bytes_in = int64_t(from_w) * from_h * channels, bytes_out = int64_t(to_w) * to_h * channels;
    if (from_w == to_w && from_h == to_h) {  // same size: a copy, as in PIL
        HIP_CHECK(hipMemcpyAsync(dst, src, size_t(bytes_in), hipMemcpyDeviceToDevice, ctx.stream));
        return;
    }
    const Coeffs ch = coeffs(from_w, to_w), cv = coeffs(from_h, to_h);
    // workspace: horizontal and vertical tables, then the intermediate image
    const size_t th = (ch.bounds.size() + ch.k.size()) * 4, tv = (cv.bounds.size() + cv.k.size()) * 4;
    const size_t tmp_off = (th + tv + 255) & ~size_t(255);
    const int64_t tmp_bytes = int64_t(to_w) * from_h * channels;
    char *ws = static_cast<char *>(ctx.ws.get(tmp_off + size_t(tmp_bytes), ctx.stream));
    std::vector<int32_t> table;
    table.reserve((th + tv) / 4);
    table.insert(table.end(), ch.bounds.begin(), ch.bounds.end());
    table.insert(table.end(), ch.k.begin(), ch.k.end());
    table.insert(table.end(), cv.bounds.begin(), cv.bounds.end());
    table.insert(table.end(), cv.k.begin(), cv.k.end());
    HIP_CHECK(hipMemcpyAsync(ws, table.data(), table.size() * 4, hipMemcpyHostToDevice, ctx.stream));
    const int32_t *bh = reinterpret_cast<const int32_t *>(ws), *kh = bh + ch.bounds.size();
    const int32_t *bv = kh + ch.k.size(), *kv = bv + cv.bounds.size();
    uint8_t *tmp = reinterpret_cast<uint8_t *>(ws + tmp_off);
    const int64_t nh = int64_t(from_h) * to_w;
    const unsigned gh = unsigned(ceil_div(nh, 256));
    if (channels == 1) resample_h_kernel<1><<<gh, 256, 0, ctx.stream>>>(src, from_w, from_h, bh, kh, ch.ksize, to_w, tmp);
    else if (channels == 3) resample_h_kernel<3><<<gh, 256, 0, ctx.stream>>>(src, from_w, from_h, bh, kh, ch.ksize, to_w, tmp);
    else resample_h_kernel<4><<<gh, 256, 0, ctx.stream>>>(src, from_w, from_h, bh, kh, ch.ksize, to_w, tmp);
    MH_LAUNCH_CHECK();
    const int row_bytes = to_w * channels;
    resample_v_kernel<<<unsigned(ceil_div(bytes_out, 256)), 256, 0, ctx.stream>>>(tmp, row_bytes, bv, kv, cv.ksize,
                                                                                  to_h, dst);
    MH_LAUNCH_CHECK();
    // the tables are pageable host memory read by the queued copy: let it finish
    HIP_CHECK(hipStreamSynchronize(ctx.stream));
}

}  // namespace mh
