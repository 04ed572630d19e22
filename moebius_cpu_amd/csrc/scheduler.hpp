// The samplers of the denoise loop (src/scheduler.rs): the noise schedule and
// timesteps on the host, the per-element updates on the device
// (denoise.hip). The host computes each step's scalars exactly as the
// reference does (f32 square roots for DDIM, f64 for DPM-Solver++(2M)), so the
// device update is the reference's per-element f32 arithmetic.
#pragma once

#include <cstdint>
#include <vector>

#include "common.hpp"

namespace mh {

enum class Spacing : uint32_t { Leading = 0, Trailing = 1 };
enum class Solver : uint32_t { Ddim = 0, DpmPp2M = 1 };

// src/scheduler.rs:30-76 (Ddim::new): the 1000 f32 cumulative alpha products,
// the timesteps kept by the strength slicing, and whether the loop starts
// from pure noise.
struct Schedule {
    std::vector<float> alphas_cumprod;
    int step_ratio = 0;
    std::vector<int> timesteps;
    bool pure_noise_start = false;
    Schedule(int steps, double strength, Spacing spacing);
};

// src/scheduler.rs:159-172
std::vector<float> scaled_linear_alphas_cumprod();

// Per-step scalars of one update (denoise.hip's guided_step_kernel).
struct StepCoeffs {
    // 0: DDIM; 1: DPM first order; 2: DPM second order; 3: DPM final step (x = x0)
    int mode = 0;
    float a = 0, b = 0, c = 0, d = 0, e = 0;
};
// src/scheduler.rs:88-97 at timestep t: a = sqrt(1 - at), b = sqrt(at),
// c = sqrt(a_prev), d = sqrt(1 - a_prev).
StepCoeffs ddim_coeffs(const Schedule &s, int t);
// src/scheduler.rs:123-156 at step i, with the previous step's lambda when
// has_prev: a = 1/alpha, b = sigma, c = sigma_next/sigma, d = phi (first
// order) or c0, e = c1; the new lambda in *lambda_out.
StepCoeffs dpm_coeffs(const Schedule &s, int i, bool has_prev, double prev_lambda, double *lambda_out);

// Device updates (denoise.hip), n elements, asynchronous on ctx.stream.
// eps = eps_c ? eps_u + guidance (eps_c - eps_u) : eps_u, then the solver
// update of x in place; DPM keeps its data prediction in prev (written when
// mode is 1 or 2, read when mode is 2).
void guided_step(Context &ctx, const StepCoeffs &k, const float *eps_u, const float *eps_c, float guidance, float *x,
                 float *prev, int64_t n);
// src/scheduler.rs:80-86: out = sqrt(at) x0 + sqrt(1 - at) noise.
void add_noise(Context &ctx, const Schedule &s, const float *x0, const float *noise, int t, float *out, int64_t n);
// The UNet input stack of src/pipeline.rs:320-324: per latent pixel
// [x(4) | mask(1) | z_masked(4)].
void unet_input(Context &ctx, const float *x, const float *mask_lat, const float *z_masked, float *out, int64_t pixels);

}  // namespace mh
