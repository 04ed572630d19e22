// The VAE (src/vae, AutoencoderKL with SDXL-VAE weights) on the device:
// weights resident in HBM, every feature map in the pool, kernels queued on
// the context stream. Host C++ mirror of src/vae/{mod,encoder,decoder}.rs.
#pragma once

#include <memory>

#include "unet.hpp"

namespace mh {

class VaeDevice;

class Vae {
  public:
    Vae(Context &ctx, const NamedTensor *t, int count);
    ~Vae();
    // src/vae/encoder.rs:77-118: images_dev [b,h,w,3] in [-1,1] (h, w multiples of 8),
    // noise_dev [b,h/8,w/8,4] -> z_dev [b,h/8,w/8,4] (scaled posterior sample).
    void encode(const float *images_dev, int b, int h, int w, const float *noise_dev, float *z_dev,
                TraceFn trace = nullptr, void *user = nullptr);
    // src/vae/decoder.rs:74-99: latents_dev [1,h,w,4] (scaled) -> out_dev [1,8h,8w,3] = (dec + 1) / 2.
    void decode(const float *latents_dev, int h, int w, float *out_dev, TraceFn trace = nullptr,
                void *user = nullptr);
    size_t weight_bytes() const;
    size_t pool_bytes() const;
    // Frees the pool's idle buffers (Scratch::release_below(usize::MAX), src/engine/mod.rs:87-91).
    void release_scratch();

  private:
    std::unique_ptr<VaeDevice> d_;
};

}  // namespace mh
