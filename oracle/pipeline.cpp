// Oracle restatement of the reference's samplers and denoise loop
// (src/scheduler.rs, src/pipeline.rs:295-345). Test infrastructure only: see
// oracle.h. Arithmetic follows the reference operation by operation: the
// schedule in f32 with torch's linspace halves, DDIM in f32, DPM-Solver++(2M)
// coefficients in f64 and the per-element updates in f32.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "oracle.h"
#include "oracle_pipeline.h"
#include "oracle_unet.h"

namespace {

constexpr int TRAIN_STEPS = 1000;
constexpr double BETA_START = 0.00085, BETA_END = 0.012;

// src/scheduler.rs:159-172: linspace(sqrt b0, sqrt b1, 1000) in f32, the two
// halves filled from opposite ends, squared, then cumprod(1 - beta) in f32.
std::vector<float> alphas_cumprod() {
    const float start = float(std::sqrt(BETA_START)), end = float(std::sqrt(BETA_END));
    const int n = TRAIN_STEPS;
    const float step = (end - start) / float(n - 1);
    std::vector<float> out(n);
    float acc = 1.0f;
    for (int i = 0; i < n; ++i) {
        const float s = i < n / 2 ? start + step * float(i) : end - step * float(n - 1 - i);
        acc *= 1.0f - s * s;
        out[size_t(i)] = acc;
    }
    return out;
}

// src/scheduler.rs:30-97 (Ddim) and 115-156 (Dpm2M).
struct Sched {
    std::vector<float> ac;
    int step_ratio = 0;
    std::vector<int> timesteps;
    bool pure_noise = false;
    std::vector<float> prev_x0;  // Dpm2M history
    double prev_lambda = 0.0;
    bool has_prev = false;

    Sched(int steps, double strength, int spacing) {
        if (steps < 1 || steps > TRAIN_STEPS) throw std::runtime_error("steps must be 1..=1000");
        ac = alphas_cumprod();
        step_ratio = TRAIN_STEPS / steps;
        std::vector<int> all;
        if (spacing == 0) {
            for (int i = steps - 1; i >= 0; --i) all.push_back(i * step_ratio);
        } else {
            const double r = double(TRAIN_STEPS) / double(steps);
            for (int i = 0; i < steps; ++i) all.push_back(int(std::round(double(TRAIN_STEPS) - double(i) * r)) - 1);
        }
        int init = int(double(steps) * strength);
        if (init > steps) init = steps;
        if (init < 0) init = 0;
        timesteps.assign(all.begin() + (steps - init), all.end());
        pure_noise = strength >= 1.0;
    }

    void add_noise(const float *x0, const float *noise, int64_t n, int t, float *out) const {
        const float a = ac[size_t(t)];
        const float sa = std::sqrt(a), sb = std::sqrt(1.0f - a);
        for (int64_t i = 0; i < n; ++i) out[i] = sa * x0[i] + sb * noise[i];
    }

    void ddim_step(const float *eps, int64_t n, int t, float *x) const {
        const float a_t = ac[size_t(t)];
        const float a_prev = t >= step_ratio ? ac[size_t(t - step_ratio)] : 1.0f;
        const float sqrt_b_t = std::sqrt(1.0f - a_t), sqrt_a_t = std::sqrt(a_t);
        const float sqrt_a_prev = std::sqrt(a_prev), sqrt_b_prev = std::sqrt(1.0f - a_prev);
        for (int64_t i = 0; i < n; ++i) {
            const float x0 = (x[i] - sqrt_b_t * eps[i]) / sqrt_a_t;
            x[i] = sqrt_a_prev * x0 + sqrt_b_prev * eps[i];
        }
    }

    void coeffs(int t, double &alpha, double &sigma, double &lambda) const {
        const double a = double(ac[size_t(t)]);
        alpha = std::sqrt(a);
        sigma = std::sqrt(1.0 - a);
        lambda = std::log(alpha) - std::log(sigma);
    }

    void dpm_step(const float *eps, int64_t n, int i, float *x) {
        double alpha, sigma, lambda;
        coeffs(timesteps[size_t(i)], alpha, sigma, lambda);
        const float inv_alpha = float(1.0 / alpha), sigma_f = float(sigma);
        std::vector<float> x0(static_cast<size_t>(n));
        for (int64_t j = 0; j < n; ++j) x0[size_t(j)] = (x[j] - sigma_f * eps[j]) * inv_alpha;
        if (size_t(i + 1) >= timesteps.size()) {
            std::memcpy(x, x0.data(), size_t(n) * sizeof(float));
            return;
        }
        double alpha_n, sigma_n, lambda_n;
        coeffs(timesteps[size_t(i + 1)], alpha_n, sigma_n, lambda_n);
        const double h = lambda_n - lambda;
        const float keep = float(sigma_n / sigma);
        const double phi = alpha_n * (1.0 - std::exp(-h));
        if (!has_prev) {
            const float p = float(phi);
            for (int64_t j = 0; j < n; ++j) x[j] = keep * x[j] + p * x0[size_t(j)];
        } else {
            const double r = (lambda - prev_lambda) / h;
            const float c0 = float(phi * (1.0 + 0.5 / r)), c1 = float(phi * 0.5 / r);
            for (int64_t j = 0; j < n; ++j) x[j] = keep * x[j] + c0 * x0[size_t(j)] - c1 * prev_x0[size_t(j)];
        }
        prev_x0 = std::move(x0);
        prev_lambda = lambda;
        has_prev = true;
    }
};

}  // namespace

extern "C" void orc_alphas_cumprod(float *out) {
    const std::vector<float> a = alphas_cumprod();
    std::memcpy(out, a.data(), a.size() * sizeof(float));
}

extern "C" void *orc_sched_create(int steps, double strength, int spacing) {
    try {
        return new Sched(steps, strength, spacing);
    } catch (...) {
        return nullptr;
    }
}

extern "C" void orc_sched_destroy(void *s) { delete static_cast<Sched *>(s); }

extern "C" int orc_sched_timesteps(void *s, int *out, int *pure_noise) {
    const Sched *p = static_cast<Sched *>(s);
    for (size_t i = 0; i < p->timesteps.size(); ++i) out[i] = p->timesteps[i];
    *pure_noise = p->pure_noise ? 1 : 0;
    return int(p->timesteps.size());
}

extern "C" void orc_sched_add_noise(void *s, const float *x0, const float *noise, int64_t n, int t, float *out) {
    static_cast<Sched *>(s)->add_noise(x0, noise, n, t, out);
}

extern "C" void orc_sched_ddim_step(void *s, const float *eps, int64_t n, int t, float *x) {
    static_cast<Sched *>(s)->ddim_step(eps, n, t, x);
}

extern "C" void orc_sched_dpm_step(void *s, const float *eps, int64_t n, int i, float *x) {
    static_cast<Sched *>(s)->dpm_step(eps, n, i, x);
}

extern "C" void orc_sched_dpm_restart(void *s) {
    Sched *p = static_cast<Sched *>(s);
    p->has_prev = false;
    p->prev_x0.clear();
}

// src/pipeline.rs:295-345, steps 7-8: x from the initial noise (or
// add_noise(z_img, init, t0)), then per timestep the UNet input
// [x(4) | mask(1) | z_masked(4)], the UNet (CFG batch 2 for the first
// cfg_steps steps, every step when cfg_steps < 0; else cond-only), the
// guidance combine u + g (c - u), and the solver step (DPM-Solver++(2M)
// restarts where CFG stops). Arrays are [64 * 64 * 4] (mask [64 * 64]);
// latents receives the final x. Returns 0, or -1 on a failure (message in err).
extern "C" int orc_denoise(void *unet, const float *z_img, const float *init, const float *mask_lat,
                           const float *z_masked, int steps, double strength, int spacing, int solver, float guidance,
                           int cfg_steps, float *latents, char *err, int err_len) {
    try {
        constexpr int64_t LAT = 64 * 64, N = LAT * 4;
        Sched sched(steps, strength, spacing);
        std::vector<float> x(static_cast<size_t>(N)), input(static_cast<size_t>(LAT * 9)), eps(static_cast<size_t>(N)),
            e2(static_cast<size_t>(2 * N));
        if (sched.pure_noise) std::memcpy(x.data(), init, size_t(N) * sizeof(float));
        else sched.add_noise(z_img, init, N, sched.timesteps[0], x.data());
        for (size_t i = 0; i < sched.timesteps.size(); ++i) {
            const int t = sched.timesteps[i];
            for (int64_t p = 0; p < LAT; ++p) {
                std::memcpy(&input[size_t(p * 9)], &x[size_t(p * 4)], 4 * sizeof(float));
                input[size_t(p * 9 + 4)] = mask_lat[p];
                std::memcpy(&input[size_t(p * 9 + 5)], &z_masked[p * 4], 4 * sizeof(float));
            }
            const bool cfg = cfg_steps < 0 || int(i) < cfg_steps;
            if (orc_unet_forward(unet, input.data(), t, cfg ? 0 : 1, e2.data(), nullptr, nullptr) != 0)
                throw std::runtime_error("oracle UNet forward failed");
            if (cfg) {
                for (int64_t j = 0; j < N; ++j) {
                    const float u = e2[size_t(j)], c = e2[size_t(N + j)];
                    eps[size_t(j)] = u + guidance * (c - u);
                }
            } else {
                std::memcpy(eps.data(), e2.data(), size_t(N) * sizeof(float));
            }
            if (solver == 0) {
                sched.ddim_step(eps.data(), N, t, x.data());
            } else {
                if (cfg_steps >= 0 && int(i) == cfg_steps) orc_sched_dpm_restart(&sched);
                sched.dpm_step(eps.data(), N, int(i), x.data());
            }
        }
        std::memcpy(latents, x.data(), size_t(N) * sizeof(float));
        return 0;
    } catch (const std::exception &e) {
        if (err && err_len > 0) {
            std::strncpy(err, e.what(), size_t(err_len - 1));
            err[err_len - 1] = 0;
        }
        return -1;
    }
}
