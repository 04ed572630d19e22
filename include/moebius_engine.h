/*
 * moebius-hip inpainting engine: the reference's whole-pipeline C API
 * (include/moebius_cpu.h, src/ffi.rs) served by the MI355X library, plus the
 * extensions a parity run needs (explicit noise, the full parameter set, the
 * final latents).
 *
 * The `moebius_*` declarations below have the reference's names, types,
 * struct layouts, constants and error behaviour, so a host built against
 * include/moebius_cpu.h links this library unchanged. Differences:
 *  - `threads` of moebius_engine_create sets the host threads of the paste
 *    around the device run (blur and blend; 0 = one per core, at most 16);
 *    the models run on GPU 0 (mh_engine_create picks another device).
 *  - MOEBIUS_ERR_UNSUPPORTED_CPU (3) reports a missing or unusable GPU.
 *  - A seed gives other noise than the CPU engine's generator (the library
 *    draws its own seeded normals, mh_sample_noise); feed recorded noise
 *    through mh_inpaint_with_noise for run-to-run comparisons.
 *  - Calls on one engine are serialised (one device stream per engine); the
 *    reference allows concurrent calls on one engine.
 *
 * moebius_last_error and mh_last_error share one thread-local message.
 */
#ifndef MOEBIUS_ENGINE_H
#define MOEBIUS_ENGINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- the reference's API (include/moebius_cpu.h:11-69) ------------------- */

#define MOEBIUS_ABI_VERSION 1u

#define MOEBIUS_OK                   0
#define MOEBIUS_ERR_INVALID_ARGUMENT 1
#define MOEBIUS_ERR_WEIGHTS          2
#define MOEBIUS_ERR_UNSUPPORTED_CPU  3
#define MOEBIUS_ERR_CANCELLED        4
#define MOEBIUS_ERR_IO               5
#define MOEBIUS_ERR_INTERNAL         6

#define MOEBIUS_PRESET_EXACT 0u
#define MOEBIUS_PRESET_FAST  1u

#define MOEBIUS_PASTE_DEFAULT            0u
#define MOEBIUS_PASTE_NONE               1u
#define MOEBIUS_PASTE_FEATHER            2u
#define MOEBIUS_PASTE_FEATHER_COMPENSATE 3u

typedef struct MoebiusEngine MoebiusEngine;

/* Zero-initialised = Exact preset defaults (src/ffi.rs:43-53). */
typedef struct MoebiusParams {
    uint32_t preset;      /* MOEBIUS_PRESET_* */
    uint32_t steps;       /* 0 = preset default */
    float    guidance;    /* <= 0 = preset default */
    uint64_t seed;
    uint32_t paste;       /* MOEBIUS_PASTE_* */
    uint32_t mask_dilate; /* px, 0 = off */
} MoebiusParams;

typedef struct MoebiusRect {
    uint32_t x, y, width, height;
} MoebiusRect;

/* stage: 0 encode, 1 denoise, 2 decode. Return non-zero to cancel. Called on
 * the calling thread. */
typedef int32_t (*MoebiusProgressFn)(void *user, uint32_t stage, uint32_t done, uint32_t total);

/* src/ffi.rs:105-108. */
uint32_t moebius_abi_version(void);

/* src/ffi.rs:110-115: message of the last failed call on this thread. Never NULL. */
const char *moebius_last_error(void);

/* src/ffi.rs:117-137 (Engine::load, src/pipeline.rs:118-138): loads
 * weights_dir/unet.safetensors and weights_dir/vae.safetensors onto GPU 0. */
int32_t moebius_engine_create(const char *weights_dir, uint32_t threads, MoebiusEngine **out);

/* src/ffi.rs:165-172. NULL is ignored. */
void moebius_engine_destroy(MoebiusEngine *engine);

/* src/ffi.rs:174-225 (Engine::inpaint, src/pipeline.rs:140-213): in-place
 * inpaint of 8-bit RGB/RGBA `pixels` where `mask` >= 128. params, progress,
 * changed may be NULL. Alpha is preserved. On MOEBIUS_ERR_CANCELLED the image
 * is untouched. An empty mask returns MOEBIUS_OK with an empty rect. */
int32_t moebius_inpaint(const MoebiusEngine *engine,
                        uint8_t *pixels, uint32_t width, uint32_t height,
                        uint32_t stride, uint32_t channels,
                        const uint8_t *mask, uint32_t mask_stride,
                        const MoebiusParams *params,
                        MoebiusProgressFn progress, void *user,
                        MoebiusRect *changed);

/* ---- extensions ---------------------------------------------------------- */

/* Every field of the reference's InpaintParams (src/preset.rs:34-58) plus the
 * arithmetic of the UNet's matrix work. */
typedef struct MhInpaintParams {
    uint32_t steps;        /* 1..=1000 */
    uint32_t spacing;      /* MH_SPACING_* (moebius_hip.h) */
    uint32_t solver;       /* MH_SOLVER_* */
    int32_t  cfg_steps;    /* < 0: CFG on every step */
    double   strength;
    float    guidance;
    float    noise_offset;
    uint64_t seed;
    uint32_t roi_encode;   /* 0 / 1 */
    uint32_t roi_decode;   /* 0 / 1 */
    uint32_t paste;        /* MOEBIUS_PASTE_NONE .. FEATHER_COMPENSATE */
    uint32_t mask_dilate;  /* px */
    uint32_t precision;    /* MH_PRECISION_* for the UNet (the VAE stays f32) */
    uint32_t reserved;     /* 0 */
} MhInpaintParams;

/* Length of the noise block mh_inpaint_with_noise reads: vae_img, vae_masked,
 * init (each 64*64*4, NHWC [1,64,64,4]) and offset (4), in that order
 * (src/pipeline.rs:64-100 NoiseSet). */
#define MH_NOISE_FLOATS (3u * 64u * 64u * 4u + 4u)

/* src/ffi.rs:227-250 resolve_params: the preset's parameters
 * (src/preset.rs:60-82) with the caller's overrides; NULL = Exact defaults.
 * Both presets compute in MH_PRECISION_EXACT. Host only. */
int32_t mh_inpaint_params(const MoebiusParams *params, MhInpaintParams *out);

/* The library's seeded normals (splitmix64 -> 53-bit uniforms -> Box-Muller
 * in f64 -> f32), MH_NOISE_FLOATS values in NoiseSet order. Host only. */
int32_t mh_sample_noise(uint64_t seed, float *out);

/* moebius_engine_create on a chosen device. */
int32_t mh_engine_create(int32_t device, const char *weights_dir, MoebiusEngine **out);

/* Engine::inpaint_traced (src/pipeline.rs:160-213): moebius_inpaint with the
 * full parameter set, caller-supplied noise (host, MH_NOISE_FLOATS) and,
 * when latents_out is not NULL, the final scaled latents (host, 64*64*4)
 * before decoding. */
int32_t mh_inpaint_with_noise(const MoebiusEngine *engine,
                              uint8_t *pixels, uint32_t width, uint32_t height,
                              uint32_t stride, uint32_t channels,
                              const uint8_t *mask, uint32_t mask_stride,
                              const MhInpaintParams *params, const float *noise,
                              MoebiusProgressFn progress, void *user,
                              MoebiusRect *changed, float *latents_out);

/* Device memory the engine holds: weights, and the activation pools plus the
 * transform workspace. */
int32_t mh_engine_memory(const MoebiusEngine *engine, uint64_t *weight_bytes, uint64_t *pool_bytes);

/* Frees the activation pools and the workspace (Scratch::release_below,
 * src/engine/mod.rs:87-91). The CPU engine does this inside every call
 * (src/pipeline.rs:290-292); this engine keeps them resident between calls,
 * so that a repeated call allocates nothing, and frees them only on request.
 * The next call allocates them again. */
int32_t mh_engine_release_scratch(const MoebiusEngine *engine);

#ifdef __cplusplus
}
#endif

#endif /* MOEBIUS_ENGINE_H */
