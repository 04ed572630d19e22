// Pixel-space steps around the 512x512 model window (src/imaging): the mask's
// bounding box and dilation, the square crop plan, the feathered paste-back
// (with Pillow's Gaussian blur reproduced byte for byte) and the latent ROI
// window. Host code: these touch the caller's host image once, at the
// beginning (mask) and the end (paste); the resampling between the window and
// the model runs on the device (resize.hip).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

namespace mh {
namespace img {

struct Rect {
    size_t x = 0, y = 0, w = 0, h = 0;
};

struct MaskView {  // 8-bit mask; >= 128 is inpainted (src/imaging/mod.rs:16-29)
    const uint8_t *data;
    size_t width, height, stride;
};

struct ImageView {  // 8-bit RGB / RGBA, edited in place, alpha kept (src/imaging/mod.rs:79-88)
    uint8_t *data;
    size_t width, height, stride, channels;
};

// src/imaging/mod.rs:31-46: bounding box of the pixels >= 128; false when none.
bool mask_bbox(const MaskView &m, Rect *out);

// src/imaging/mod.rs:48-77: binarised (0 / 255) mask dilated with a k x k ones
// kernel anchored at k / 2 (cv2.dilate), stride = width; k <= 1 binarises only.
std::vector<uint8_t> dilate(const MaskView &m, size_t k);

// src/imaging/crop.rs:21-66: the square window around the mask.
struct CropPlan {
    int64_t x = 0, y = 0;  // negative where the window extends past the image
    size_t side = 0;
};
CropPlan crop_plan(const Rect &mask_bbox, size_t img_w, size_t img_h);
Rect source_rect(const CropPlan &p, size_t img_w, size_t img_h);

// src/imaging/blend.rs:39-110: Pillow's GaussianBlur(radius) of an 8-bit
// single-channel image (three fractional box-blur passes per axis, 24-bit
// fixed point, 8-bit rounding after every pass).
// threads: host threads for the row passes (the bytes do not depend on it).
std::vector<uint8_t> gaussian_blur(const uint8_t *src, size_t w, size_t h, float radius, unsigned threads = 1);

enum class Paste : uint32_t { None = 1, Feather = 2, FeatherCompensate = 3 };

// src/imaging/blend.rs:155-232: pastes `result` (side x side RGB, the model
// output resized back to the window) over `img` inside the plan's source rect,
// raw (None), through the mask blurred with radius 3 (Feather, f64 blend), or
// additionally shifted by 1.1 x the ring's mean-colour difference
// (FeatherCompensate). Returns the rectangle written.
Rect paste(ImageView &img, const MaskView &mask, const uint8_t *result, const CropPlan &plan, Paste mode,
           unsigned threads = 1);

// src/vae/mod.rs:60-78: bounding box of the 64 x 64 latent mask's nonzero
// entries grown by margin and clamped; false for an empty mask.
struct LatentRect {
    size_t x = 0, y = 0, w = 0, h = 0;
};
bool roi_window(const float *mask_lat, size_t margin, LatentRect *out);

}  // namespace img
}  // namespace mh
