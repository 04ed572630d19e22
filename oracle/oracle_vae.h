/*
 * CPU oracle, VAE chain (src/vae) — test infrastructure only, see oracle.h.
 */
#ifndef MOEBIUS_ORACLE_VAE_H
#define MOEBIUS_ORACLE_VAE_H

#include <stdint.h>

#include "oracle_unet.h"

#ifdef __cplusplus
extern "C" {
#endif

/* src/vae/mod.rs:88-103 (Vae::load without the metadata check); NULL on error
 * with the message in err. The tensor data must outlive the returned object. */
void *orc_vae_create(const OrcNamed *tensors, int count, char *err, int err_len);
void orc_vae_destroy(void *vae);

/* src/vae/encoder.rs:77-118: images [b,h,w,3] in [-1,1] (h, w multiples of 8),
 * noise [b,h/8,w/8,4]; z [b,h/8,w/8,4] = scaled posterior sample. trace may be NULL.
 * 0 on success, else 1 with the message in err. */
int orc_vae_encode(void *vae, const float *images, int64_t b, int64_t h, int64_t w, const float *noise, float *z,
                   OrcTraceFn trace, void *user, char *err, int err_len);

/* src/vae/decoder.rs:74-99: latents [1,h,w,4] (scaled) -> out [1,8h,8w,3] =
 * (dec(latents / 0.13025) + 1) / 2, unclamped. */
int orc_vae_decode(void *vae, const float *latents, int64_t h, int64_t w, float *out, OrcTraceFn trace, void *user,
                   char *err, int err_len);

/* src/vae/mod.rs:275-294 `softmax_rows`: in place over rows [nrows][n], scale > 0,
 * probabilities below e^-40 flushed to zero. */
void orc_softmax_rows(float *rows, int64_t nrows, int64_t n, float scale);

/* src/vae/mod.rs:240-270 `MidAttention::forward` for x [n,h,w,c] with the weights
 * under `prefix` (the attentions.0 module); out [n,h,w,c]. */
int orc_vae_attention(const OrcNamed *tensors, int count, const char *prefix, const float *x, int64_t n, int64_t h,
                      int64_t w, int64_t c, float *out, char *err, int err_len);

/* src/vae/mod.rs:174-211 `Resnet::forward`, weights under `prefix` (resnets.j). */
int orc_vae_resnet(const OrcNamed *tensors, int count, const char *prefix, const float *x, int64_t n, int64_t h,
                   int64_t w, int64_t c_in, int64_t c_out, float *out, char *err, int err_len);

/* src/vae/encoder.rs:121-133 `sample`: moments [pixels][8] = mean(4) | logvar(4),
 * noise [pixels][4] -> z [pixels][4]. */
void orc_vae_sample(const float *moments, const float *noise, int64_t pixels, float *z);

#ifdef __cplusplus
}
#endif

#endif
