// The whole-pipeline C ABI of include/moebius_engine.h: the reference's
// moebius_* entry points (src/ffi.rs) and the mh_ extensions for parity runs.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/moebius_engine.h"
#include "../../include/moebius_hip.h"
#include "capi_guard.hpp"
#include "inpaint.hpp"
#include "weights.hpp"

struct MoebiusEngine {
    mh::Engine e;
    std::mutex lock;  // one stream per engine: calls run one at a time
    explicit MoebiusEngine(int device) : e(device) {}
};

namespace {

using mh::capi::guard;
using mh::capi::need;

// src/ffi.rs:227-250 resolve_params.
mh::InpaintParams resolve(const MoebiusParams *p) {
    if (!p) return mh::preset_params(MOEBIUS_PRESET_EXACT);
    mh::InpaintParams out = mh::preset_params(p->preset);
    if (p->steps > 0) out.sampling.steps = p->steps;
    if (p->guidance > 0.0f) out.sampling.guidance = p->guidance;
    out.seed = p->seed;
    out.mask_dilate = p->mask_dilate;
    switch (p->paste) {
    case MOEBIUS_PASTE_DEFAULT: break;
    case MOEBIUS_PASTE_NONE: out.paste = mh::img::Paste::None; break;
    case MOEBIUS_PASTE_FEATHER: out.paste = mh::img::Paste::Feather; break;
    case MOEBIUS_PASTE_FEATHER_COMPENSATE: out.paste = mh::img::Paste::FeatherCompensate; break;
    default: mh::fail(mh::kInvalidArgument, "unknown paste mode " + std::to_string(p->paste));
    }
    return out;
}

MhInpaintParams to_c(const mh::InpaintParams &p) {
    MhInpaintParams c{};
    c.steps = p.sampling.steps;
    c.spacing = uint32_t(p.sampling.spacing);
    c.solver = uint32_t(p.sampling.solver);
    c.cfg_steps = p.sampling.cfg_steps;
    c.strength = p.sampling.strength;
    c.guidance = p.sampling.guidance;
    c.noise_offset = p.noise_offset;
    c.seed = p.seed;
    c.roi_encode = p.roi_encode;
    c.roi_decode = p.roi_decode;
    c.paste = uint32_t(p.paste);
    c.mask_dilate = p.mask_dilate;
    c.precision = p.fast_precision ? MH_PRECISION_FAST : MH_PRECISION_EXACT;
    return c;
}

mh::InpaintParams from_c(const MhInpaintParams &c) {
    MH_REQUIRE(c.spacing <= MH_SPACING_TRAILING, "unknown spacing " + std::to_string(c.spacing));
    MH_REQUIRE(c.solver <= MH_SOLVER_DPMPP_2M, "unknown solver " + std::to_string(c.solver));
    MH_REQUIRE(c.paste >= MOEBIUS_PASTE_NONE && c.paste <= MOEBIUS_PASTE_FEATHER_COMPENSATE,
               "unknown paste mode " + std::to_string(c.paste));
    MH_REQUIRE(c.precision <= MH_PRECISION_FAST, "unknown precision " + std::to_string(c.precision));
    MH_REQUIRE(c.roi_encode <= 1 && c.roi_decode <= 1 && c.reserved == 0, "flags must be 0 or 1, reserved 0");
    mh::InpaintParams p;
    p.sampling.steps = c.steps;
    p.sampling.spacing = mh::Spacing(c.spacing);
    p.sampling.solver = mh::Solver(c.solver);
    p.sampling.cfg_steps = c.cfg_steps;
    p.sampling.strength = c.strength;
    p.sampling.guidance = c.guidance;
    p.noise_offset = c.noise_offset;
    p.seed = c.seed;
    p.roi_encode = c.roi_encode != 0;
    p.roi_decode = c.roi_decode != 0;
    p.paste = mh::img::Paste(c.paste);
    p.mask_dilate = c.mask_dilate;
    p.fast_precision = c.precision == MH_PRECISION_FAST;
    return p;
}

void load_models(MoebiusEngine &m, const std::string &dir) {
    mh::Context &c = m.e.ctx;
    {
        const mh::WeightsFile f(dir + "/unet.safetensors");
        const std::vector<mh::NamedTensor> t = mh::model_tensors(f, mh::ModelKind::UNet);
        m.e.unet = std::make_unique<mh::UNet>(c, t.data(), int(t.size()));
        HIP_CHECK(hipStreamSynchronize(c.stream));  // the uploads have read the mapping
    }
    const mh::WeightsFile f(dir + "/vae.safetensors");
    const std::vector<mh::NamedTensor> t = mh::model_tensors(f, mh::ModelKind::Vae);
    m.e.vae = std::make_unique<mh::Vae>(c, t.data(), int(t.size()));
    HIP_CHECK(hipStreamSynchronize(c.stream));
}

// threads (the reference's worker count, 0 = one per core): here the host
// threads of the paste's blur and blend, at most 16.
int32_t create(int32_t device, const char *weights_dir, uint32_t threads, MoebiusEngine **out) {
    if (!weights_dir || !out) return mh::capi::set_error(MOEBIUS_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    return guard([&] {
        auto m = std::make_unique<MoebiusEngine>(device);
        const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
        m->e.host_threads = std::min(16u, threads ? unsigned(threads) : hw);
        load_models(*m, weights_dir);
        *out = m.release();
    });
}

// src/ffi.rs:196-205 argument checks, then the pipeline.
void run(const MoebiusEngine *engine, uint8_t *pixels, uint32_t width, uint32_t height, uint32_t stride,
         uint32_t channels, const uint8_t *mask, uint32_t mask_stride, const mh::InpaintParams &p,
         const mh::NoiseSet &noise, MoebiusProgressFn progress, void *user, MoebiusRect *changed,
         float *latents_out) {
    auto *m = const_cast<MoebiusEngine *>(engine);
    std::lock_guard<std::mutex> hold(m->lock);
    HIP_CHECK(hipSetDevice(m->e.ctx.device));
    mh::img::ImageView im{pixels, width, height, stride, channels};
    const mh::img::MaskView mk{mask, width, height, mask_stride};
    const mh::img::Rect r = mh::inpaint(m->e, im, mk, p, noise, progress, user, latents_out);
    if (changed) *changed = MoebiusRect{uint32_t(r.x), uint32_t(r.y), uint32_t(r.w), uint32_t(r.h)};
}

bool bad_dims(uint32_t w, uint32_t h, uint32_t stride, uint32_t c, uint32_t mask_stride) {
    return w == 0 || h == 0 || uint64_t(stride) < uint64_t(w) * c || mask_stride < w;
}

}  // namespace

extern "C" {

uint32_t moebius_abi_version(void) { return MOEBIUS_ABI_VERSION; }

const char *moebius_last_error(void) { return mh::capi::last_error.c_str(); }

int32_t moebius_engine_create(const char *weights_dir, uint32_t threads, MoebiusEngine **out) {
    return create(0, weights_dir, threads, out);
}

int32_t mh_engine_create(int32_t device, const char *weights_dir, MoebiusEngine **out) {
    return create(device, weights_dir, 0, out);
}

void moebius_engine_destroy(MoebiusEngine *engine) {
    if (!engine) return;
    (void)hipSetDevice(engine->e.ctx.device);
    delete engine;
}

int32_t moebius_inpaint(const MoebiusEngine *engine, uint8_t *pixels, uint32_t width, uint32_t height,
                        uint32_t stride, uint32_t channels, const uint8_t *mask, uint32_t mask_stride,
                        const MoebiusParams *params, MoebiusProgressFn progress, void *user, MoebiusRect *changed) {
    if (!engine || !pixels || !mask) return mh::capi::set_error(MOEBIUS_ERR_INVALID_ARGUMENT, "null argument");
    if (bad_dims(width, height, stride, channels, mask_stride))
        return mh::capi::set_error(MOEBIUS_ERR_INVALID_ARGUMENT, "bad dimensions or stride");
    return guard([&] {
        const mh::InpaintParams p = resolve(params);
        const mh::NoiseSet noise = mh::sample_noise(p.seed);
        run(engine, pixels, width, height, stride, channels, mask, mask_stride, p, noise, progress, user, changed,
            nullptr);
    });
}

int32_t mh_inpaint_with_noise(const MoebiusEngine *engine, uint8_t *pixels, uint32_t width, uint32_t height,
                              uint32_t stride, uint32_t channels, const uint8_t *mask, uint32_t mask_stride,
                              const MhInpaintParams *params, const float *noise, MoebiusProgressFn progress,
                              void *user, MoebiusRect *changed, float *latents_out) {
    if (!engine || !pixels || !mask || !params || !noise)
        return mh::capi::set_error(MOEBIUS_ERR_INVALID_ARGUMENT, "null argument");
    if (bad_dims(width, height, stride, channels, mask_stride))
        return mh::capi::set_error(MOEBIUS_ERR_INVALID_ARGUMENT, "bad dimensions or stride");
    return guard([&] {
        const mh::InpaintParams p = from_c(*params);
        constexpr size_t kLat = 64 * 64 * 4;
        mh::NoiseSet n;
        n.vae_img.assign(noise, noise + kLat);
        n.vae_masked.assign(noise + kLat, noise + 2 * kLat);
        n.init.assign(noise + 2 * kLat, noise + 3 * kLat);
        n.offset.assign(noise + 3 * kLat, noise + 3 * kLat + 4);
        run(engine, pixels, width, height, stride, channels, mask, mask_stride, p, n, progress, user, changed,
            latents_out);
    });
}

int32_t mh_inpaint_params(const MoebiusParams *params, MhInpaintParams *out) {
    return guard([&] {
        need(out, "out");
        *out = to_c(resolve(params));
    });
}

int32_t mh_sample_noise(uint64_t seed, float *out) {
    return guard([&] {
        need(out, "out");
        const mh::NoiseSet n = mh::sample_noise(seed);
        float *o = out;
        for (const std::vector<float> *v : {&n.vae_img, &n.vae_masked, &n.init, &n.offset}) {
            std::memcpy(o, v->data(), v->size() * sizeof(float));
            o += v->size();
        }
    });
}

int32_t mh_engine_memory(const MoebiusEngine *engine, uint64_t *weight_bytes, uint64_t *pool_bytes) {
    return guard([&] {
        need(engine, "engine");
        auto *m = const_cast<MoebiusEngine *>(engine);
        std::lock_guard<std::mutex> hold(m->lock);
        if (weight_bytes) *weight_bytes = m->e.unet->weight_bytes() + m->e.vae->weight_bytes();
        if (pool_bytes) *pool_bytes = m->e.unet->pool_bytes() + m->e.vae->pool_bytes() + m->e.ctx.ws.capacity() +
                                    m->e.ctx.state.capacity() + m->e.frames.capacity();
    });
}

int32_t mh_engine_release_scratch(const MoebiusEngine *engine) {
    return guard([&] {
        need(engine, "engine");
        auto *m = const_cast<MoebiusEngine *>(engine);
        std::lock_guard<std::mutex> hold(m->lock);
        HIP_CHECK(hipSetDevice(m->e.ctx.device));
        m->e.unet->release_scratch();
        m->e.vae->release_scratch();
        m->e.ctx.ws.release(m->e.ctx.stream);
        m->e.ctx.state.release(m->e.ctx.stream);
        m->e.frames.release(m->e.ctx.stream);
    });
}

}  // extern "C"
