// The denoise loop on the device (src/pipeline.rs:295-345) and the stateful
// sampler behind the C ABI's scheduler entry points (src/scheduler.rs).
#pragma once

#include <cstdint>

#include "common.hpp"
#include "scheduler.hpp"
#include "unet.hpp"

namespace mh {

// src/preset.rs:27-50 (the fields the loop reads).
struct DenoiseParams {
    uint32_t steps = 20;
    double strength = 0.99;
    Spacing spacing = Spacing::Leading;
    Solver solver = Solver::Ddim;
    float guidance = 2.5f;
    int cfg_steps = -1;  // < 0: CFG on every step; n: the first n steps, then cond-only
};

// Called on the caller's thread after each finished step; nonzero cancels.
using StepFn = int32_t (*)(void *user, uint32_t done, uint32_t total);

// src/pipeline.rs:295-345, steps 7-8. Device arrays: z_img, init, z_masked,
// latents [64 * 64 * 4] (NHWC [1,64,64,4]), mask_lat [64 * 64]. x starts as
// init (strength >= 1) or add_noise(z_img, init, t0); each step runs the UNet
// on [x | mask | z_masked] (CFG batch 2 while CFG is on), combines
// u + g (c - u), and updates x with the solver. latents receives the final x;
// on cancellation (kCancelled) it is left untouched. Synchronous: returns when
// the latents are written.
void unet_denoise(Context &ctx, UNet &unet, const float *z_img, const float *init, const float *mask_lat,
                  const float *z_masked, const DenoiseParams &prm, StepFn progress, void *user, float *latents);

// Ddim + Dpm2M over device arrays of len elements (src/scheduler.rs:30-156).
class Sampler {
  public:
    Sampler(Context &ctx, int steps, double strength, Spacing spacing, int64_t len);
    ~Sampler();
    Sampler(const Sampler &) = delete;
    Sampler &operator=(const Sampler &) = delete;
    const Schedule &schedule() const { return sched_; }
    void add_noise(const float *x0, const float *noise, int t, float *out);
    // eps_c NULL: eps_u is the (cond-only) noise prediction; else the CFG combine first.
    void ddim_step(const float *eps_u, const float *eps_c, float guidance, int t, float *x);
    void dpm_step(const float *eps_u, const float *eps_c, float guidance, int i, float *x);
    void restart() { has_prev_ = false; }

  private:
    Context &ctx_;
    Schedule sched_;
    int64_t len_;
    float *prev_ = nullptr;
    bool has_prev_ = false;
    double prev_lambda_ = 0.0;
};

}  // namespace mh
