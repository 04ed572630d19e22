/*
 * CPU oracle, UNet chain (src/unet) — test infrastructure only, see oracle.h.
 */
#ifndef MOEBIUS_ORACLE_UNET_H
#define MOEBIUS_ORACLE_UNET_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One converter tensor (tools/convert_weights.py layouts), widened to f32. */
typedef struct OrcNamed {
    const char *name;
    const float *data;
    int64_t numel;
} OrcNamed;

/* Called after every block with the reference's golden names (src/unet/mod.rs:148-157). */
typedef void (*OrcTraceFn)(void *user, const char *name, const float *data, int64_t n, int64_t h, int64_t w,
                           int64_t c);

/* src/unet/embed.rs:21-30 */
void orc_timestep_sinusoid(int t, float *out /* [320] */);

/* src/unet/mod.rs:86-140 (UNet::load); NULL on error with the message in err. The
 * tensor data must outlive the returned object. */
void *orc_unet_create(const OrcNamed *tensors, int count, char *err, int err_len);
void orc_unet_destroy(void *unet);

/* src/unet/mod.rs:144-243: x [1,64,64,9]; guidance 0 = CFG (b=2, branches uncond,
 * cond), 1 = cond only (b=1); eps [b,64,64,4]. trace may be NULL. 0 on success. */
int orc_unet_forward(void *unet, const float *x, int timestep, int guidance, float *eps, OrcTraceFn trace,
                     void *user);

/* One block alone: kind 0 DwConv2d (blocks.rs:31-54), 1 DwResnet (blocks.rs:56-113,
 * temb [n,1280]), 2 SelfLambda (lambda.rs:73-152), 3 CrossLambda (lambda.rs:187-274),
 * 4 MixTransformer (transformer.rs:49-130); weights under `prefix`; branches [n]
 * for kinds 3/4. out [n,h,w,c_out]. 0 on success, else 1 with the message in err. */
int orc_block_forward(int kind, const OrcNamed *tensors, int count, const char *prefix, const float *x, int64_t n,
                      int64_t h, int64_t w, int64_t c_in, int64_t c_out, const float *temb, const int *branches,
                      float *out, char *err, int err_len);

/* src/unet/lambda.rs:322-359; keys [rows,k] is overwritten; lambda [k,vd]. */
void orc_softmax_lambda(float *keys, const float *v, int64_t rows, int64_t k, int64_t vd, float *lambda);
/* src/unet/lambda.rs:154-185 */
void orc_tap_filter(const float *a, const float *v, float *o, int64_t first, int64_t count, int64_t hh, int64_t ww,
                    int64_t vd);
/* src/unet/lambda.rs:279-295 over count pixels: q, o [count][8k]; e [count][10][k]; v [10][k]. */
void orc_position_term(const float *q, const float *e, const float *v, float *o, int64_t count, int64_t k);
/* src/unet/lambda.rs:297-309 */
float orc_dot8(const float *a, const float *b, int64_t k);
/* FLOPs of the UNet steps run since the last reset, as the upstream model
 * computes them (unfolded lambda), by category: out[6] = 1x1 convs, dense 3x3,
 * stride-2 3x3, depthwise, self-lambda position Conv3d, matrix products. */
void orc_unet_flops(double *out);
void orc_unet_flops_reset(void);

#ifdef __cplusplus
}
#endif

#endif
