// Device steps of the inpainting pipeline between the resampled window and the
// VAE (src/pipeline.rs:230-244, 372-384): model-space image and masked image,
// the nearest-sampled latent mask, window crops and the ROI decode frame.
#include "common.hpp"
#include "inpaint.hpp"

namespace mh {

namespace {

constexpr int kSide = 512, kLat = 64, kDown = 8;

// One thread per model pixel: rgb = v / 255 * 2 - 1 computed in f64 and stored
// f32 (numpy's asarray(img) / 255. * 2 - 1); masked = rgb * keep with keep 0
// where the resized mask is >= 128, else 1; the latent mask samples pixel (8y, 8x).
__global__ __launch_bounds__(256) void model_inputs_kernel(const uint8_t *__restrict__ rgb8,
                                                           const uint8_t *__restrict__ bin8,
                                                           float *__restrict__ images, float *__restrict__ mask_lat) {
    const int p = int(blockIdx.x) * 256 + threadIdx.x;
    if (p >= kSide * kSide) return;
    const bool masked = bin8[p] >= 128;
    const float keep = masked ? 0.0f : 1.0f;
    float *img = images + int64_t(p) * 3;
    float *msk = images + int64_t(kSide) * kSide * 3 + int64_t(p) * 3;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float v = float(double(rgb8[p * 3 + c]) / 255.0 * 2.0 - 1.0);
        img[c] = v;
        msk[c] = v * keep;
    }
    const int y = p / kSide, x = p - y * kSide;
    if (y % kDown == 0 && x % kDown == 0) mask_lat[(y / kDown) * kLat + x / kDown] = masked ? 1.0f : 0.0f;
}

__global__ __launch_bounds__(256) void crop_kernel(const float *__restrict__ src, int w_full, int c, int x0, int y0,
                                                   int w, int h, float *__restrict__ dst) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int64_t row = int64_t(w) * c;
    if (i >= row * h) return;
    const int64_t y = i / row, r = i - y * row;
    dst[i] = src[((y0 + y) * w_full + x0) * c + r];
}

__global__ __launch_bounds__(256) void roi_frame_kernel(const float *__restrict__ rgb, const float *__restrict__ part,
                                                        int x0, int y0, int w, int h, float *__restrict__ frame) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(kSide) * kSide * 3) return;
    const int64_t p = i / 3, c = i - p * 3;
    const int y = int(p / kSide), x = int(p - int64_t(y) * kSide);
    const int wx = x0 * kDown, wy = y0 * kDown, ww = w * kDown, wh = h * kDown;
    if (x >= wx && x < wx + ww && y >= wy && y < wy + wh)
        frame[i] = part[(int64_t(y - wy) * ww + (x - wx)) * 3 + c];
    else
        frame[i] = (rgb[i] + 1.0f) * 0.5f;
}

}  // namespace

void model_inputs(Context &ctx, const uint8_t *rgb8, const uint8_t *bin8, float *images, float *mask_lat) {
    model_inputs_kernel<<<unsigned(ceil_div(kSide * kSide, 256)), 256, 0, ctx.stream>>>(rgb8, bin8, images, mask_lat);
    MH_LAUNCH_CHECK();
}

void crop_window(Context &ctx, const float *src, int w_full, int c, int x, int y, int w, int h, float *dst) {
    const int64_t n = int64_t(w) * h * c;
    if (n == 0) return;
    crop_kernel<<<unsigned(ceil_div(n, 256)), 256, 0, ctx.stream>>>(src, w_full, c, x, y, w, h, dst);
    MH_LAUNCH_CHECK();
}

void roi_frame(Context &ctx, const float *rgb, const float *part, int x, int y, int w, int h, float *frame) {
    roi_frame_kernel<<<unsigned(ceil_div(int64_t(kSide) * kSide * 3, 256)), 256, 0, ctx.stream>>>(rgb, part, x, y, w,
                                                                                                   h, frame);
    MH_LAUNCH_CHECK();
}

}  // namespace mh
