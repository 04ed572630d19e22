/*
 * CPU oracle, samplers and denoise loop (src/scheduler.rs, src/pipeline.rs) —
 * test infrastructure only, see oracle.h.
 */
#ifndef MOEBIUS_ORACLE_PIPELINE_H
#define MOEBIUS_ORACLE_PIPELINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/scheduler.rs:159-172: the 1000 f32 cumulative alpha products. */
void orc_alphas_cumprod(float *out);
/* src/scheduler.rs:30-62 (Ddim::new); spacing 0 leading, 1 trailing. NULL on bad steps. */
void *orc_sched_create(int steps, double strength, int spacing);
void orc_sched_destroy(void *s);
/* The timesteps denoised (returns their count, out holds up to 1000) and whether
 * the loop starts from pure noise. */
int orc_sched_timesteps(void *s, int *out, int *pure_noise);
/* src/scheduler.rs:80-86 */
void orc_sched_add_noise(void *s, const float *x0, const float *noise, int64_t n, int t, float *out);
/* src/scheduler.rs:88-97 */
void orc_sched_ddim_step(void *s, const float *eps, int64_t n, int t, float *x);
/* src/scheduler.rs:123-156 (stateful) and 117-120 (restart). */
void orc_sched_dpm_step(void *s, const float *eps, int64_t n, int i, float *x);
void orc_sched_dpm_restart(void *s);
/* src/pipeline.rs:295-345, steps 7-8, over the oracle UNet. */
int orc_denoise(void *unet, const float *z_img, const float *init, const float *mask_lat, const float *z_masked,
                int steps, double strength, int spacing, int solver, float guidance, int cfg_steps, float *latents,
                char *err, int err_len);

#ifdef __cplusplus
}
#endif

#endif
