// End-to-end inpainting on the device (src/pipeline.rs:161-392): the host
// reads the caller's mask and image window once and writes the paste back
// once; everything between (resampling to the 512x512 frame, the VAE encode,
// the denoise loop, the decode and the resampling back) runs on the GPU with
// its tensors resident in HBM.
#pragma once

#include <cstdint>
#include <memory>

#include "common.hpp"
#include "denoise.hpp"
#include "imaging.hpp"
#include "unet.hpp"
#include "vae.hpp"

namespace mh {

// src/preset.rs:34-82 (InpaintParams) with the sampling fields of DenoiseParams.
struct InpaintParams {
    DenoiseParams sampling;
    float noise_offset = 0.0357f;
    uint64_t seed = 0;
    bool roi_encode = false;
    bool roi_decode = false;
    img::Paste paste = img::Paste::Feather;
    uint32_t mask_dilate = 0;
    // FAST precision for the UNet's matrix work (no preset sets it); the VAE stays f32.
    bool fast_precision = false;
};
// src/preset.rs:52-82 `Preset::params`: 0 = Exact, 1 = Fast.
InpaintParams preset_params(uint32_t preset);

// Gaussian noise the pipeline consumes (src/pipeline.rs:64-100): [64*64*4] x 3
// and the per-channel offset [4], host memory, drawn in this order.
struct NoiseSet {
    std::vector<float> vae_img, vae_masked, init, offset;
};
// The library's seeded generator (splitmix64 -> 53-bit uniforms -> Box-Muller in
// f64 -> f32), one stream of 3 * 16384 + 4 normals; the reference's StdRng
// stream is not reproduced, so a seed gives other noise than the CPU engine.
NoiseSet sample_noise(uint64_t seed);

// Called on the caller's thread: stage 0 encode, 1 denoise, 2 decode; nonzero cancels.
using ProgressFn = int32_t (*)(void *user, uint32_t stage, uint32_t done, uint32_t total);

struct Engine {
    Context ctx;
    std::unique_ptr<UNet> unet;
    std::unique_ptr<Vae> vae;
    unsigned host_threads = 1;  // host threads for the paste around the device run
    // the inpaint call's device frames (window, model inputs, latents, decode),
    // grow-only: a call at a window side no larger than an earlier one allocates nothing
    Workspace frames;
    explicit Engine(int device) : ctx(device) {}
};

// src/pipeline.rs:161-213 + run(): inpaints img in place where mask >= 128,
// returns the rectangle written (empty for an empty mask). Cancellation
// (kCancelled) leaves img untouched. latents_out (host [64*64*4], optional)
// receives the final latents before decoding.
img::Rect inpaint(Engine &e, img::ImageView &img, const img::MaskView &mask, const InpaintParams &p,
                  const NoiseSet &noise, ProgressFn progress, void *user, float *latents_out);

// Device kernels of the pipeline (inpaint_kernels.hip).
// rgb8 [512*512*3], bin8 [512*512] (resized window and mask) -> images
// [2][512*512*3] = [rgb in [-1, 1], rgb * (1 - mask)] and mask_lat [64*64].
void model_inputs(Context &ctx, const uint8_t *rgb8, const uint8_t *bin8, float *images, float *mask_lat);
// Copies the w x h window at (x, y) of an NHWC map [h_full][w_full][c] (device).
void crop_window(Context &ctx, const float *src, int w_full, int c, int x, int y, int w, int h, float *dst);
// 512x512 frame (rgb + 1) / 2 with the decoded window part [8h][8w][3] placed at
// latent rect (x, y, w, h) (src/pipeline.rs:372-384).
void roi_frame(Context &ctx, const float *rgb, const float *part, int x, int y, int w, int h, float *frame);

}  // namespace mh
