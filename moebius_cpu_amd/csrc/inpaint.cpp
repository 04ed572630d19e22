// Host orchestration of the device inpainting pipeline (src/pipeline.rs:161-392,
// src/preset.rs, src/ffi.rs resolve_params): validation, mask dilation and
// bounding box, the crop plan and the window gather on the host; resampling,
// VAE, denoise loop, decode and resampling back on the device; the paste on
// the host.
#include "inpaint.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <utility>

#include "kernels.hpp"

namespace mh {

namespace {

constexpr int kSide = 512, kLat = 64, kLatC = 4, kDown = 8;
constexpr int64_t kLatN = int64_t(kLat) * kLat * kLatC;
constexpr size_t kRoiMargin = 8;  // src/vae/mod.rs:58

// The call's device frames, carved from the engine's grow-only block in 256-byte
// aligned pieces; each ROI buffer is sized for the whole frame, so one layout
// serves every mask at a given window side.
struct Frames {
    uint8_t *win, *wbin, *rgb8, *bin8, *u8, *res;
    float *images, *mask_lat, *z, *noise, *crop, *part, *init, *lat, *dec, *lcrop, *dpart;

    Frames(Workspace &block, hipStream_t stream, size_t side) {
        const size_t model_px = size_t(kSide) * kSide, lat_b = size_t(kLatN) * sizeof(float);
        const size_t frame_b = model_px * 3 * sizeof(float);
        const std::pair<void **, size_t> parts[] = {
            {(void **)&win, side * side * 3},     {(void **)&wbin, side * side},
            {(void **)&rgb8, model_px * 3},       {(void **)&bin8, model_px},
            {(void **)&u8, model_px * 3},         {(void **)&res, side * side * 3},
            {(void **)&images, 2 * frame_b},      {(void **)&mask_lat, size_t(kLat) * kLat * sizeof(float)},
            {(void **)&z, 2 * lat_b},             {(void **)&noise, 2 * lat_b},
            {(void **)&crop, frame_b},            {(void **)&part, lat_b},
            {(void **)&init, lat_b},              {(void **)&lat, lat_b},
            {(void **)&dec, frame_b},             {(void **)&lcrop, lat_b},
            {(void **)&dpart, frame_b}};
        auto round = [](size_t b) { return (b + 255) & ~size_t(255); };
        size_t total = 0;
        for (const auto &q : parts) total += round(q.second);
        char *base = static_cast<char *>(block.get(total, stream));
        for (const auto &q : parts) {
            *q.first = base;
            base += round(q.second);
        }
    }
};

void h2d(Context &ctx, void *dst, const void *src, size_t bytes) {
    HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx.stream));
    HIP_CHECK(hipStreamSynchronize(ctx.stream));  // pageable source
}

void d2h(Context &ctx, void *dst, const void *src, size_t bytes) {
    HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx.stream));
    HIP_CHECK(hipStreamSynchronize(ctx.stream));
}

// splitmix64 -> 53-bit uniforms -> Box-Muller pairs (f64) -> f32: normal i of
// the stream uses pair i / 2 (uniforms 2k for the radius, 2k + 1 for the angle).
std::vector<float> normals(uint64_t seed, size_t n) {
    auto mix = [](uint64_t z) {
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    auto uniform = [&](uint64_t i) {  // output i of splitmix64 seeded with seed
        const uint64_t z = seed + 0x9E3779B97F4A7C15ull * (i + 1);
        return double(mix(z) >> 11) * (1.0 / 9007199254740992.0);
    };
    std::vector<float> out(n);
    for (size_t k = 0; 2 * k < n; ++k) {
        const double u0 = uniform(2 * k), u1 = uniform(2 * k + 1);
        const double r = std::sqrt(-2.0 * std::log1p(-u0)), t = 2.0 * M_PI * u1;
        out[2 * k] = float(r * std::cos(t));
        if (2 * k + 1 < n) out[2 * k + 1] = float(r * std::sin(t));
    }
    return out;
}

// A stage is reported done once its kernels have finished, as the CPU engine
// reports it after the work (so the callback's clock and cancellation points
// line up with the reference's stages).
void report(Context &ctx, ProgressFn fn, void *user, uint32_t stage, uint32_t done, uint32_t total) {
    if (!fn) return;
    if (done == total) HIP_CHECK(hipStreamSynchronize(ctx.stream));
    if (fn(user, stage, done, total) != 0) fail(kCancelled, "cancelled");
}

struct StepAdapter {
    ProgressFn fn;
    void *user;
    static int32_t call(void *self, uint32_t done, uint32_t total) {
        auto *a = static_cast<StepAdapter *>(self);
        return a->fn ? a->fn(a->user, 1, done, total) : 0;
    }
};

}  // namespace

InpaintParams preset_params(uint32_t preset) {
    InpaintParams p;  // Exact: 20 leading DDIM steps at strength 0.99, CFG 2.5, feather paste
    p.sampling.steps = 20;
    p.sampling.strength = 0.99;
    p.sampling.spacing = Spacing::Leading;
    p.sampling.solver = Solver::Ddim;
    p.sampling.guidance = 2.5f;
    p.sampling.cfg_steps = -1;
    if (preset == 1) {  // Fast: 10 trailing DPM-Solver++(2M) steps, CFG for 3, ROI encode
        p.sampling.steps = 10;
        p.sampling.spacing = Spacing::Trailing;
        p.sampling.solver = Solver::DpmPp2M;
        p.sampling.cfg_steps = 3;
        p.roi_encode = true;
    } else if (preset != 0) {
        fail(kInvalidArgument, "unknown preset " + std::to_string(preset));
    }
    return p;
}

NoiseSet sample_noise(uint64_t seed) {
    const std::vector<float> z = normals(seed, size_t(3 * kLatN + kLatC));
    NoiseSet s;
    s.vae_img.assign(z.begin(), z.begin() + kLatN);
    s.vae_masked.assign(z.begin() + kLatN, z.begin() + 2 * kLatN);
    s.init.assign(z.begin() + 2 * kLatN, z.begin() + 3 * kLatN);
    s.offset.assign(z.begin() + 3 * kLatN, z.end());
    return s;
}

img::Rect inpaint(Engine &e, img::ImageView &im, const img::MaskView &mask_in, const InpaintParams &p,
                  const NoiseSet &noise, ProgressFn progress, void *user, float *latents_out) {
    Context &ctx = e.ctx;
    MH_REQUIRE(im.width == mask_in.width && im.height == mask_in.height, "image and mask sizes differ");
    MH_REQUIRE(im.channels == 3 || im.channels == 4, "image must be RGB or RGBA");
    MH_REQUIRE(im.width > 0 && im.height > 0, "empty image");
    MH_REQUIRE(im.stride >= im.width * im.channels && mask_in.stride >= mask_in.width,
               "buffer smaller than width, height and stride imply");
    MH_REQUIRE(p.sampling.steps >= 1 && p.sampling.steps <= 1000,
               "steps must be 1..=1000, got " + std::to_string(p.sampling.steps));
    MH_REQUIRE(noise.vae_img.size() == size_t(kLatN) && noise.vae_masked.size() == size_t(kLatN) &&
                   noise.init.size() == size_t(kLatN) && noise.offset.size() == size_t(kLatC),
               "noise has the wrong shape");

    std::vector<uint8_t> dilated;
    img::MaskView mask = mask_in;
    if (p.mask_dilate > 0) {
        dilated = img::dilate(mask_in, p.mask_dilate);
        mask = img::MaskView{dilated.data(), mask_in.width, mask_in.height, mask_in.width};
    }
    img::Rect bbox;
    if (!img::mask_bbox(mask, &bbox)) return img::Rect{};
    const img::CropPlan plan = img::crop_plan(bbox, im.width, im.height);
    const size_t side = plan.side;

    // 2-3: the window (edge-replicated image, mask zero outside) -> 512x512 on the device.
    report(ctx, progress, user, 0, 0, 1);
    std::vector<uint8_t> win(side * side * 3), wbin(side * side);
    const int64_t w = int64_t(im.width), h = int64_t(im.height);
    for (size_t wy = 0; wy < side; ++wy) {
        const int64_t y = plan.y + int64_t(wy), yc = std::clamp<int64_t>(y, 0, h - 1);
        for (size_t wx = 0; wx < side; ++wx) {
            const int64_t x = plan.x + int64_t(wx), xc = std::clamp<int64_t>(x, 0, w - 1);
            const uint8_t *px = im.data + size_t(yc) * im.stride + size_t(xc) * im.channels;
            std::memcpy(&win[(wy * side + wx) * 3], px, 3);
            const bool inside = y >= 0 && y < h && x >= 0 && x < w;
            wbin[wy * side + wx] = inside && mask.data[size_t(yc) * mask.stride + size_t(xc)] >= 128 ? 255 : 0;
        }
    }
    const size_t model_px = size_t(kSide) * kSide;
    const Frames d(e.frames, ctx.stream, side);
    h2d(ctx, d.win, win.data(), win.size());
    h2d(ctx, d.wbin, wbin.data(), wbin.size());
    resize_u8(ctx, d.win, int(side), int(side), kSide, kSide, 3, d.rgb8);
    resize_u8(ctx, d.wbin, int(side), int(side), kSide, kSide, 1, d.bin8);
    model_inputs(ctx, d.rgb8, d.bin8, d.images, d.mask_lat);
    std::vector<float> mask_lat(size_t(kLat) * kLat);
    d2h(ctx, mask_lat.data(), d.mask_lat, mask_lat.size() * sizeof(float));

    // 4: VAE encode of [image, masked] (or the ROI encode of the Fast preset).
    float *z_img = d.z, *z_masked = d.z + kLatN;
    img::LatentRect r;
    const bool window = img::roi_window(mask_lat.data(), kRoiMargin, &r) && (r.w < size_t(kLat) || r.h < size_t(kLat));
    if (p.roi_encode && window) {
        h2d(ctx, d.noise, noise.vae_masked.data(), size_t(kLatN) * sizeof(float));
        e.vae->encode(d.images + model_px * 3, 1, kSide, kSide, d.noise, z_masked);
        const int cw = int(r.w) * kDown, chh = int(r.h) * kDown;
        crop_window(ctx, d.images, kSide, 3, int(r.x) * kDown, int(r.y) * kDown, cw, chh, d.crop);
        std::vector<float> crop_noise(r.w * r.h * kLatC);
        for (size_t y = 0; y < r.h; ++y)
            std::memcpy(&crop_noise[y * r.w * kLatC], &noise.vae_img[((r.y + y) * kLat + r.x) * kLatC],
                        r.w * kLatC * sizeof(float));
        h2d(ctx, d.noise, crop_noise.data(), crop_noise.size() * sizeof(float));
        e.vae->encode(d.crop, 1, chh, cw, d.noise, d.part);
        // the window's border latents see zero padding: keep only the part nearer the mask
        img::LatentRect inner;
        img::roi_window(mask_lat.data(), kRoiMargin / 2, &inner);
        HIP_CHECK(hipMemcpyAsync(z_img, z_masked, size_t(kLatN) * sizeof(float), hipMemcpyDeviceToDevice, ctx.stream));
        HIP_CHECK(hipMemcpy2DAsync(z_img + (inner.y * kLat + inner.x) * kLatC, size_t(kLat) * kLatC * sizeof(float),
                                   d.part + ((inner.y - r.y) * r.w + inner.x - r.x) * kLatC,
                                   r.w * kLatC * sizeof(float), inner.w * kLatC * sizeof(float), inner.h,
                                   hipMemcpyDeviceToDevice, ctx.stream));
        HIP_CHECK(hipStreamSynchronize(ctx.stream));
    } else {
        h2d(ctx, d.noise, noise.vae_img.data(), size_t(kLatN) * sizeof(float));
        h2d(ctx, d.noise + kLatN, noise.vae_masked.data(), size_t(kLatN) * sizeof(float));
        e.vae->encode(d.images, 2, kSide, kSide, d.noise, d.z);
    }
    // The CPU engine frees the encoder's 512x512 maps here (src/pipeline.rs:290-292);
    // with HBM to spare the VAE's pool stays resident, so a later call allocates nothing.
    report(ctx, progress, user, 0, 1, 1);

    // 6-8: init = N(0,1) + noise_offset * N(0,1)[per channel], then the denoise loop.
    std::vector<float> init(static_cast<size_t>(kLatN));
    for (int64_t i = 0; i < kLatN; ++i) init[size_t(i)] = noise.init[size_t(i)] + p.noise_offset * noise.offset[size_t(i % kLatC)];
    h2d(ctx, d.init, init.data(), init.size() * sizeof(float));
    {
        PrecisionScope scope(ctx, p.fast_precision ? Precision::Fast : Precision::Exact);
        StepAdapter a{progress, user};
        unet_denoise(ctx, *e.unet, z_img, d.init, d.mask_lat, z_masked, p.sampling, &StepAdapter::call, &a, d.lat);
    }
    if (latents_out) d2h(ctx, latents_out, d.lat, size_t(kLatN) * sizeof(float));

    // 9: decode (the whole frame, or the ROI window over the model-input image).
    report(ctx, progress, user, 2, 0, 1);
    img::LatentRect rd;
    if (p.roi_decode && img::roi_window(mask_lat.data(), kRoiMargin, &rd) &&
        (rd.w < size_t(kLat) || rd.h < size_t(kLat))) {
        crop_window(ctx, d.lat, kLat, kLatC, int(rd.x), int(rd.y), int(rd.w), int(rd.h), d.lcrop);
        e.vae->decode(d.lcrop, int(rd.h), int(rd.w), d.dpart);
        roi_frame(ctx, d.images, d.dpart, int(rd.x), int(rd.y), int(rd.w), int(rd.h), d.dec);
        HIP_CHECK(hipStreamSynchronize(ctx.stream));
    } else {
        e.vae->decode(d.lat, kLat, kLat, d.dec);
    }
    report(ctx, progress, user, 2, 1, 1);

    // 10: 8-bit truncation, resampled back to the window, pasted on the host.
    to_u8(ctx, d.dec, int64_t(model_px) * 3, d.u8);
    resize_u8(ctx, d.u8, kSide, kSide, int(side), int(side), 3, d.res);
    std::vector<uint8_t> result(side * side * 3);
    d2h(ctx, result.data(), d.res, result.size());
    return img::paste(im, mask, result.data(), plan, p.paste, e.host_threads);
}

}  // namespace mh
