// The denoise loop on the device (src/pipeline.rs:295-345 with the samplers
// of src/scheduler.rs): latents, mask and masked-image latents stay in HBM
// for every step; the UNet input stack, the classifier-free-guidance combine
// and the DDIM / DPM-Solver++(2M) update are kernels, and only the step's
// scalars come from the host. The host checks progress / cancellation after
// each step while the next one is already queued.
#include <cmath>
#include <cstring>

#include "common.hpp"
#include "denoise.hpp"
#include "scheduler.hpp"

namespace mh {

namespace {
constexpr int kTrainSteps = 1000;
constexpr double kBetaStart = 0.00085, kBetaEnd = 0.012;
}  // namespace

std::vector<float> scaled_linear_alphas_cumprod() {
    // torch: linspace(sqrt b0, sqrt b1, 1000) in f32 (CPU linspace fills the two
    // halves from opposite ends), squared, cumprod(1 - beta) in f32.
    const float start = float(std::sqrt(kBetaStart)), end = float(std::sqrt(kBetaEnd));
    const int n = kTrainSteps;
    const float step = (end - start) / float(n - 1);
    std::vector<float> out(static_cast<size_t>(n));
    float acc = 1.0f;
    for (int i = 0; i < n; ++i) {
        const float s = i < n / 2 ? start + step * float(i) : end - step * float(n - 1 - i);
        acc *= 1.0f - s * s;
        out[size_t(i)] = acc;
    }
    return out;
}

Schedule::Schedule(int steps, double strength, Spacing spacing) {
    if (steps < 1 || steps > kTrainSteps) fail(kInvalidArgument, "steps must be 1..=1000, got " + std::to_string(steps));
    if (!(strength >= 0.0)) fail(kInvalidArgument, "strength must be a number >= 0");
    alphas_cumprod = scaled_linear_alphas_cumprod();
    step_ratio = kTrainSteps / steps;
    std::vector<int> all;
    if (spacing == Spacing::Leading) {
        for (int i = steps - 1; i >= 0; --i) all.push_back(i * step_ratio);
    } else {
        const double r = double(kTrainSteps) / double(steps);
        for (int i = 0; i < steps; ++i) all.push_back(int(std::round(double(kTrainSteps) - double(i) * r)) - 1);
    }
    // get_timesteps(): keep the last int(steps * strength) entries.
    const int init = std::min(steps, int(double(steps) * strength));
    timesteps.assign(all.begin() + (steps - init), all.end());
    pure_noise_start = strength >= 1.0;
}

StepCoeffs ddim_coeffs(const Schedule &s, int t) {
    const float a_t = s.alphas_cumprod[size_t(t)];
    const float a_prev = t >= s.step_ratio ? s.alphas_cumprod[size_t(t - s.step_ratio)] : 1.0f;
    StepCoeffs k;
    k.mode = 0;
    k.a = std::sqrt(1.0f - a_t);
    k.b = std::sqrt(a_t);
    k.c = std::sqrt(a_prev);
    k.d = std::sqrt(1.0f - a_prev);
    return k;
}

namespace {
void dpm_alpha_sigma(const Schedule &s, int t, double &alpha, double &sigma, double &lambda) {
    const double a = double(s.alphas_cumprod[size_t(t)]);
    alpha = std::sqrt(a);
    sigma = std::sqrt(1.0 - a);
    lambda = std::log(alpha) - std::log(sigma);
}
}  // namespace

StepCoeffs dpm_coeffs(const Schedule &s, int i, bool has_prev, double prev_lambda, double *lambda_out) {
    double alpha, sigma, lambda;
    dpm_alpha_sigma(s, s.timesteps[size_t(i)], alpha, sigma, lambda);
    StepCoeffs k;
    k.a = float(1.0 / alpha);
    k.b = float(sigma);
    *lambda_out = lambda;
    if (size_t(i + 1) >= s.timesteps.size()) {
        k.mode = 3;
        return k;
    }
    double alpha_n, sigma_n, lambda_n;
    dpm_alpha_sigma(s, s.timesteps[size_t(i + 1)], alpha_n, sigma_n, lambda_n);
    const double h = lambda_n - lambda;
    k.c = float(sigma_n / sigma);
    const double phi = alpha_n * (1.0 - std::exp(-h));  // -alpha_n (e^-h - 1)
    if (!has_prev) {
        k.mode = 1;
        k.d = float(phi);
    } else {
        const double r = (lambda - prev_lambda) / h;
        k.mode = 2;
        k.d = float(phi * (1.0 + 0.5 / r));
        k.e = float(phi * 0.5 / r);
    }
    return k;
}

namespace {

// One element per thread, the reference's f32 operation order (no contraction).
__global__ __launch_bounds__(256) void guided_step_kernel(StepCoeffs k, const float *__restrict__ eps_u,
                                                          const float *__restrict__ eps_c, float guidance,
                                                          float *__restrict__ x, float *__restrict__ prev, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    float e = eps_u[i];
    if (eps_c) {
        const float c = eps_c[i];
        e = e + guidance * (c - e);  // src/pipeline.rs:333: u + g (c - u)
    }
    const float xv = x[i];
    if (k.mode == 0) {  // src/scheduler.rs:93-96
        const float x0 = (xv - k.a * e) / k.b;
        x[i] = k.c * x0 + k.d * e;
        return;
    }
    const float x0 = (xv - k.b * e) * k.a;  // src/scheduler.rs:134
    if (k.mode == 3) {
        x[i] = x0;
    } else if (k.mode == 1) {
        x[i] = k.c * xv + k.d * x0;
        prev[i] = x0;
    } else {
        const float p = prev[i];
        x[i] = k.c * xv + k.d * x0 - k.e * p;
        prev[i] = x0;
    }
}

__global__ __launch_bounds__(256) void add_noise_kernel(const float *__restrict__ x0, const float *__restrict__ noise,
                                                        float sa, float sb, float *__restrict__ out, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) out[i] = sa * x0[i] + sb * noise[i];
}

__global__ __launch_bounds__(256) void unet_input_kernel(const float4 *__restrict__ x, const float *__restrict__ mask,
                                                         const float4 *__restrict__ zm, float *__restrict__ out,
                                                         int64_t pixels) {
    const int64_t p = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (p >= pixels) return;
    const float4 a = x[p], b = zm[p];
    float *o = out + p * 9;
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w;
    o[4] = mask[p];
    o[5] = b.x, o[6] = b.y, o[7] = b.z, o[8] = b.w;
}

unsigned blocks_for(int64_t n) { return unsigned(ceil_div(n, 256)); }

}  // namespace

void guided_step(Context &ctx, const StepCoeffs &k, const float *eps_u, const float *eps_c, float guidance, float *x,
                 float *prev, int64_t n) {
    if (n == 0) return;
    MH_REQUIRE(eps_u && x, "step: eps and sample must be given");
    MH_REQUIRE(k.mode == 0 || k.mode == 3 || prev, "DPM-Solver++(2M) step needs its history buffer");
    guided_step_kernel<<<blocks_for(n), 256, 0, ctx.stream>>>(k, eps_u, eps_c, guidance, x, prev, n);
    MH_LAUNCH_CHECK();
}

void add_noise(Context &ctx, const Schedule &s, const float *x0, const float *noise, int t, float *out, int64_t n) {
    MH_REQUIRE(t >= 0 && t < kTrainSteps, "timestep must be 0..999");
    if (n == 0) return;
    const float a = s.alphas_cumprod[size_t(t)];
    add_noise_kernel<<<blocks_for(n), 256, 0, ctx.stream>>>(x0, noise, std::sqrt(a), std::sqrt(1.0f - a), out, n);
    MH_LAUNCH_CHECK();
}

void unet_input(Context &ctx, const float *x, const float *mask_lat, const float *z_masked, float *out,
                int64_t pixels) {
    MH_REQUIRE(aligned16(x) && aligned16(z_masked), "UNet input: latents must be 16-byte aligned");
    unet_input_kernel<<<blocks_for(pixels), 256, 0, ctx.stream>>>(reinterpret_cast<const float4 *>(x), mask_lat,
                                                                  reinterpret_cast<const float4 *>(z_masked), out,
                                                                  pixels);
    MH_LAUNCH_CHECK();
}

// ---- the stateful sampler behind the C ABI (src/scheduler.rs Ddim + Dpm2M)

Sampler::Sampler(Context &ctx, int steps, double strength, Spacing spacing, int64_t len)
    : ctx_(ctx), sched_(steps, strength, spacing), len_(len) {
    MH_REQUIRE(len > 0, "sampler length must be positive");
    mh::dev_malloc(&prev_, size_t(len) * sizeof(float));
}

Sampler::~Sampler() {
    if (prev_) (void)hipFree(prev_);
}

void Sampler::ddim_step(const float *eps_u, const float *eps_c, float guidance, int t, float *x) {
    MH_REQUIRE(t >= 0 && t < kTrainSteps, "timestep must be 0..999");
    guided_step(ctx_, ddim_coeffs(sched_, t), eps_u, eps_c, guidance, x, nullptr, len_);
}

void Sampler::dpm_step(const float *eps_u, const float *eps_c, float guidance, int i, float *x) {
    MH_REQUIRE(i >= 0 && size_t(i) < sched_.timesteps.size(), "step index outside the schedule");
    double lambda = 0.0;
    const StepCoeffs k = dpm_coeffs(sched_, i, has_prev_, prev_lambda_, &lambda);
    guided_step(ctx_, k, eps_u, eps_c, guidance, x, prev_, len_);
    if (k.mode != 3) {
        has_prev_ = true;
        prev_lambda_ = lambda;
    }
}

void Sampler::add_noise(const float *x0, const float *noise, int t, float *out) {
    mh::add_noise(ctx_, sched_, x0, noise, t, out, len_);
}

// ---- the loop

namespace {

struct Events {
    hipEvent_t e[2] = {nullptr, nullptr};
    Events() {
        for (auto &v : e) HIP_CHECK(hipEventCreateWithFlags(&v, hipEventDisableTiming));
    }
    ~Events() {
        for (auto &v : e)
            if (v) (void)hipEventDestroy(v);
    }
};

}  // namespace

void unet_denoise(Context &ctx, UNet &unet, const float *z_img, const float *init, const float *mask_lat,
                  const float *z_masked, const DenoiseParams &prm, StepFn progress, void *user, float *latents) {
    constexpr int64_t kPixels = 64 * 64, kN = kPixels * 4;
    MH_REQUIRE(init && mask_lat && z_masked && latents, "denoise: init, mask, masked latents and output are required");
    MH_REQUIRE(prm.guidance == prm.guidance, "guidance must be a number");
    const Schedule sched(int(prm.steps), prm.strength, prm.spacing);
    MH_REQUIRE(sched.pure_noise_start || z_img, "denoise: strength < 1 starts from the image latents, z_img is NULL");
    const int total = int(sched.timesteps.size());
    // the reference indexes timesteps[0] here (src/pipeline.rs:305-313) and panics on an empty schedule
    MH_REQUIRE(total > 0, "steps * strength < 1: the schedule keeps no timestep to denoise");
    // x | UNet input | eps (two items) | DPM history, in the context's grow-only state block
    float *x = static_cast<float *>(ctx.state.get(size_t(kN + kPixels * 9 + 2 * kN + kN) * sizeof(float), ctx.stream));
    float *in = x + kN, *eps = in + kPixels * 9, *prev = eps + 2 * kN;
    if (sched.pure_noise_start)
        HIP_CHECK(hipMemcpyAsync(x, init, size_t(kN) * sizeof(float), hipMemcpyDeviceToDevice, ctx.stream));
    else
        add_noise(ctx, sched, z_img, init, sched.timesteps[0], x, kN);
    Events ev;
    bool has_prev = false;
    double prev_lambda = 0.0;
    auto report = [&](int done) {
        if (progress && progress(user, uint32_t(done), uint32_t(total)) != 0) {
            HIP_CHECK(hipStreamSynchronize(ctx.stream));  // let the queued step finish before returning
            fail(kCancelled, "cancelled");
        }
    };
    for (int i = 0; i < total; ++i) {
        const int t = sched.timesteps[size_t(i)];
        unet_input(ctx, x, mask_lat, z_masked, in, kPixels);
        const bool cfg = prm.cfg_steps < 0 || i < prm.cfg_steps;
        unet.forward(in, t, cfg, eps);
        if (prm.solver == Solver::Ddim) {
            guided_step(ctx, ddim_coeffs(sched, t), eps, cfg ? eps + kN : nullptr, prm.guidance, x, nullptr, kN);
        } else {
            if (prm.cfg_steps >= 0 && i == prm.cfg_steps) has_prev = false;  // restart where CFG stops
            double lambda = 0.0;
            const StepCoeffs k = dpm_coeffs(sched, i, has_prev, prev_lambda, &lambda);
            guided_step(ctx, k, eps, cfg ? eps + kN : nullptr, prm.guidance, x, prev, kN);
            has_prev = true;
            prev_lambda = lambda;
        }
        HIP_CHECK(hipEventRecord(ev.e[i & 1], ctx.stream));
        // Step i is queued; report step i - 1 once it has finished.
        if (i > 0) {
            HIP_CHECK(hipEventSynchronize(ev.e[(i - 1) & 1]));
            report(i);
        }
    }
    if (total > 0) {
        HIP_CHECK(hipEventSynchronize(ev.e[(total - 1) & 1]));
        report(total);
    }
    HIP_CHECK(hipMemcpyAsync(latents, x, size_t(kN) * sizeof(float), hipMemcpyDeviceToDevice, ctx.stream));
    HIP_CHECK(hipStreamSynchronize(ctx.stream));
}

}  // namespace mh
