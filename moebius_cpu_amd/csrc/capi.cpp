// The C ABI of include/moebius_hip.h. Every entry point validates its
// arguments, runs the C++ engine function and converts any mh::Error or other
// exception into a status code plus a thread-local message, mirroring the
// reference's FFI guard (src/ffi.rs:90-103) and moebius_last_error
// (include/moebius_cpu.h:50-51). Nothing throws across the boundary.
#include <algorithm>
#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/moebius_hip.h"
#include "capi_guard.hpp"
#include "common.hpp"
#include "denoise.hpp"
#include "imaging.hpp"
#include "kernels.hpp"
#include "pool.hpp"
#include "unet.hpp"
#include "vae.hpp"
#include "weights.hpp"

struct MhContext {
    mh::Context ctx;
    explicit MhContext(int dev) : ctx(dev) {}
};

struct MhUNet {
    MhContext *owner;
    std::unique_ptr<mh::UNet> net;
    float *x_dev = nullptr, *eps_dev = nullptr;
    ~MhUNet() {
        if (x_dev) (void)hipFree(x_dev);
        if (eps_dev) (void)hipFree(eps_dev);
    }
};

struct MhScheduler {
    MhContext *owner;
    std::unique_ptr<mh::Sampler> s;
};

struct MhVae {
    MhContext *owner;
    std::unique_ptr<mh::Vae> vae;
};

struct MhEvent {
    hipEvent_t ev = nullptr;
    int device = 0;
};

namespace {

using mh::capi::guard;
using mh::capi::need;

mh::Context &C(MhContext *c) {
    if (!c) mh::fail(mh::kInvalidArgument, "context is NULL");
    HIP_CHECK(hipSetDevice(c->ctx.device));
    return c->ctx;
}

mh::WeightType wtype(uint32_t dt) {
    if (dt == MH_DTYPE_F32) return mh::kF32;
    if (dt == MH_DTYPE_F16) return mh::kF16;
    mh::fail(mh::kInvalidArgument, "unknown weight dtype");
}

void pad4(const uint32_t *pad, int out[4]) {
    need(pad, "pad");
    for (int i = 0; i < 4; ++i) {
        if (pad[i] > 2) mh::fail(mh::kInvalidArgument, "Conv3x3: padding above 2 is not supported");
        out[i] = int(pad[i]);
    }
}

// Host threads of the imaging entry points (their bytes do not depend on it): one per core, at most 16.
unsigned host_threads() { return std::min(16u, std::max(1u, std::thread::hardware_concurrency())); }

int dim(uint32_t v, const char *what) {
    if (v > (1u << 30)) mh::fail(mh::kInvalidArgument, std::string(what) + " too large");
    return int(v);
}

}  // namespace

extern "C" {

uint32_t mh_abi_version(void) { return MH_ABI_VERSION; }

const char *mh_last_error(void) { return mh::capi::last_error.c_str(); }

int32_t mh_context_create(int32_t device, MhContext **out) {
    return guard([&] {
        need(out, "out");
        *out = nullptr;
        *out = new MhContext(device);
    });
}

void mh_context_destroy(MhContext *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->ctx.device);
    delete ctx;
}

int32_t mh_context_set_tuning(MhContext *ctx, const char *key, const char *value) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(key, "key");
        if (!mh::set_tuning(c.tune, key, value))
            mh::fail(mh::kInvalidArgument, std::string("unknown tuning key or bad value: ") + key + " = " +
                                               (value ? value : "(default)"));
    });
}

int32_t mh_device_allocations(uint64_t *count) {
    return guard([&] {
        need(count, "count");
        *count = mh::device_allocations();
    });
}

int32_t mh_context_set_precision(MhContext *ctx, uint32_t precision) {
    return guard([&] {
        mh::Context &c = C(ctx);
        if (precision == MH_PRECISION_EXACT) c.precision = mh::Precision::Exact;
        else if (precision == MH_PRECISION_FAST) c.precision = mh::Precision::Fast;
        else mh::fail(mh::kInvalidArgument, "unknown precision");
    });
}

void *mh_context_stream(MhContext *ctx) { return ctx ? static_cast<void *>(ctx->ctx.stream) : nullptr; }

int32_t mh_context_gemm_times(MhContext *ctx, char *buf, uint64_t len, uint64_t *needed) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(buf, "buf");
        need(needed, "needed");
        HIP_CHECK(hipStreamSynchronize(c.stream));
        struct Agg {
            std::string key;
            int64_t launches = 0;
            double us = 0.0, flops = 0.0;
        };
        std::vector<Agg> aggs;
        for (const mh::Context::GemmTime &g : c.gemm_times) {
            float ms = 0.0f;
            HIP_CHECK(hipEventElapsedTime(&ms, g.start, g.stop));
            auto it = std::find_if(aggs.begin(), aggs.end(), [&](const Agg &a) { return a.key == g.key; });
            if (it == aggs.end()) {
                aggs.push_back(Agg{g.key});
                it = aggs.end() - 1;
            }
            it->launches += 1;
            it->us += double(ms) * 1e3;
            it->flops += g.flops;
        }
        std::string out = "[";
        for (size_t i = 0; i < aggs.size(); ++i) {
            char row[320];
            std::snprintf(row, sizeof row, "%s{\"config\": \"%s\", \"launches\": %lld, \"us\": %.3f, \"flops\": %.0f}",
                          i ? ", " : "", aggs[i].key.c_str(), static_cast<long long>(aggs[i].launches), aggs[i].us,
                          aggs[i].flops);
            out += row;
        }
        out += "]";
        *needed = out.size() + 1;
        if (out.size() + 1 > len)
            mh::fail(mh::kInvalidArgument, "buffer too small for the GEMM timings: " + std::to_string(out.size() + 1) +
                                               " bytes needed");
        std::memcpy(buf, out.c_str(), out.size() + 1);
        for (const mh::Context::GemmTime &g : c.gemm_times) {
            c.spare_events.push_back(g.start);
            c.spare_events.push_back(g.stop);
        }
        c.gemm_times.clear();
    });
}

int32_t mh_synchronize(MhContext *ctx) { return guard([&] { HIP_CHECK(hipStreamSynchronize(C(ctx).stream)); }); }

int32_t mh_device_arch(MhContext *ctx, char *buf, uint32_t len) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(buf, "buf");
        if (len == 0) mh::fail(mh::kInvalidArgument, "buffer length is 0");
        std::strncpy(buf, c.arch.c_str(), len - 1);
        buf[len - 1] = '\0';
    });
}

int32_t mh_malloc(MhContext *ctx, uint64_t bytes, void **out) {
    return guard([&] {
        C(ctx);
        need(out, "out");
        *out = nullptr;
        mh::dev_malloc(out, bytes ? bytes : 1);
    });
}

int32_t mh_free(MhContext *ctx, void *ptr) {
    return guard([&] {
        mh::Context &c = C(ctx);
        if (!ptr) return;
        HIP_CHECK(hipStreamSynchronize(c.stream));
        HIP_CHECK(hipFree(ptr));
    });
}

int32_t mh_memcpy_h2d(MhContext *ctx, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        mh::Context &c = C(ctx);
        if (!bytes) return;
        need(dst, "dst");
        need(src, "src");
        HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c.stream));
        HIP_CHECK(hipStreamSynchronize(c.stream));
    });
}

int32_t mh_memcpy_d2h(MhContext *ctx, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        mh::Context &c = C(ctx);
        if (!bytes) return;
        need(dst, "dst");
        need(src, "src");
        HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c.stream));
        HIP_CHECK(hipStreamSynchronize(c.stream));
    });
}

int32_t mh_memcpy_d2d(MhContext *ctx, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        mh::Context &c = C(ctx);
        if (!bytes) return;
        need(dst, "dst");
        need(src, "src");
        HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c.stream));
    });
}

int32_t mh_event_create(MhContext *ctx, MhEvent **out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(out, "out");
        auto *e = new MhEvent;
        e->device = c.device;
        hipError_t err = hipEventCreate(&e->ev);
        if (err != hipSuccess) {
            delete e;
            HIP_CHECK(err);
        }
        *out = e;
    });
}

int32_t mh_event_record(MhContext *ctx, MhEvent *ev) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(ev, "event");
        HIP_CHECK(hipEventRecord(ev->ev, c.stream));
    });
}

int32_t mh_event_elapsed_ms(MhEvent *start, MhEvent *end, float *ms) {
    return guard([&] {
        need(start, "start");
        need(end, "end");
        need(ms, "ms");
        HIP_CHECK(hipEventSynchronize(end->ev));
        HIP_CHECK(hipEventElapsedTime(ms, start->ev, end->ev));
    });
}

void mh_event_destroy(MhEvent *ev) {
    if (!ev) return;
    (void)hipEventDestroy(ev->ev);
    delete ev;
}

int32_t mh_bias_residual_add(MhContext *ctx, const float *x, uint64_t rows, uint32_t cols, const float *bias,
                             const float *residual, float *out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(x, "x");
        need(out, "out");
        mh::bias_residual_add(c, x, int64_t(rows), dim(cols, "cols"), bias, residual, out);
    });
}

int32_t mh_conv1x1_forward(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                           const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                           const float *residual, float *out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(x, "x");
        need(weight, "weight");
        need(out, "out");
        const int64_t pixels = int64_t(n) * h * w;
        mh::conv1x1(c, x, pixels, dim(c_in, "c_in"), weight, wtype(weight_dtype), dim(c_out, "c_out"), bias,
                    residual, out);
    });
}

int32_t mh_conv1x1_gn_partials(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                               const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                               const float *residual, float *out, float *part, uint32_t *rows) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(x, "x");
        need(weight, "weight");
        need(out, "out");
        need(part, "part");
        need(rows, "rows");
        *rows = 0;
        MH_REQUIRE(int64_t(h) * w < (int64_t(1) << 31), "conv1x1 partials: map too large");
        mh::GnPartials gp;
        gp.part = part;
        gp.item_rows = int(dim(h, "h")) * int(dim(w, "w"));
        const int64_t pixels = int64_t(n) * h * w;
        mh::conv1x1(c, x, pixels, dim(c_in, "c_in"), weight, wtype(weight_dtype), dim(c_out, "c_out"), bias, residual,
                    out, mh::GemmEpilogue::None, nullptr, nullptr, &gp);
        *rows = uint32_t(gp.rows);
    });
}

int32_t mh_conv1x1_fused(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                         const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                         const float *residual, const float *residual_scale, const float *residual_shift,
                         uint32_t residual_silu, const float *residual2, float *out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(x, "x");
        need(weight, "weight");
        need(out, "out");
        if ((residual_scale == nullptr) != (residual_shift == nullptr))
            mh::fail(mh::kInvalidArgument, "residual_scale and residual_shift go together");
        const int64_t pixels = int64_t(n) * h * w;
        mh::ResidualAffine ra;
        ra.scale = residual_scale;
        ra.shift = residual_shift;
        ra.silu = residual_silu != 0;
        ra.rows_per_item = int(int64_t(h) * w);
        mh::conv1x1(c, x, pixels, dim(c_in, "c_in"), weight, wtype(weight_dtype), dim(c_out, "c_out"), bias,
                    residual, out, mh::GemmEpilogue::None, residual_scale ? &ra : nullptr, residual2);
    });
}

int32_t mh_conv3x3_output_hw(uint32_t h, uint32_t w, uint32_t stride, const uint32_t pad[4], uint32_t upsample2x,
                             uint32_t *ho, uint32_t *wo) {
    return guard([&] {
        need(ho, "ho");
        need(wo, "wo");
        int p[4];
        pad4(pad, p);
        int oh, ow;
        mh::conv3x3_output_hw(dim(h, "h"), dim(w, "w"), dim(stride, "stride"), p, upsample2x != 0, &oh, &ow);
        *ho = uint32_t(oh);
        *wo = uint32_t(ow);
    });
}

int32_t mh_conv3x3_forward(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                           const void *weight, uint32_t weight_dtype, uint32_t c_out, const float *bias,
                           uint32_t stride, const uint32_t pad[4], uint32_t upsample2x, const float *prologue_scale,
                           const float *prologue_shift, uint32_t prologue_silu, float *out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(x, "x");
        need(weight, "weight");
        need(out, "out");
        int p[4];
        pad4(pad, p);
        if ((prologue_scale == nullptr) != (prologue_shift == nullptr))
            mh::fail(mh::kInvalidArgument, "prologue needs both scale and shift");
        mh::Affine aff;
        aff.scale = prologue_scale;
        aff.shift = prologue_shift;
        aff.silu = prologue_silu != 0;
        mh::conv3x3(c, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c_in, "c_in"), weight, wtype(weight_dtype),
                    dim(c_out, "c_out"), bias, dim(stride, "stride"), p, upsample2x != 0,
                    prologue_scale ? &aff : nullptr, out);
    });
}

int32_t mh_winograd_weight_transform(MhContext *ctx, const void *weight, uint32_t weight_dtype, uint32_t c_out,
                                     uint32_t c_in, float *u) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(weight, "weight");
        need(u, "u");
        mh::winograd_weight_transform(c, weight, wtype(weight_dtype), dim(c_out, "c_out"), dim(c_in, "c_in"), u);
    });
}

int32_t mh_winograd_input_transform(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                                    uint32_t upsample2x, const float *prologue_scale, const float *prologue_shift,
                                    uint32_t prologue_silu, float *v) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(v, "v");
        if ((prologue_scale == nullptr) != (prologue_shift == nullptr))
            mh::fail(mh::kInvalidArgument, "prologue needs both scale and shift");
        mh::Affine aff;
        aff.scale = prologue_scale;
        aff.shift = prologue_shift;
        aff.silu = prologue_silu != 0;
        mh::winograd_input_transform(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"), upsample2x != 0,
                                     prologue_scale ? &aff : nullptr, v);
    });
}

int32_t mh_winograd_output_transform(MhContext *ctx, const float *m, uint32_t n, uint32_t h, uint32_t w,
                                     uint32_t c_out, uint32_t upsample2x, const float *bias, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(m, "m");
        need(out, "out");
        mh::winograd_output_transform(cc, m, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c_out, "c_out"),
                                      upsample2x != 0, bias, nullptr, out);
    });
}

int32_t mh_conv3x3_winograd(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c_in,
                            const float *u, uint32_t c_out, const float *bias, uint32_t upsample2x,
                            const float *prologue_scale, const float *prologue_shift, uint32_t prologue_silu,
                            float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(u, "u");
        need(out, "out");
        if ((prologue_scale == nullptr) != (prologue_shift == nullptr))
            mh::fail(mh::kInvalidArgument, "prologue needs both scale and shift");
        mh::Affine aff;
        aff.scale = prologue_scale;
        aff.shift = prologue_shift;
        aff.silu = prologue_silu != 0;
        mh::conv3x3_winograd(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c_in, "c_in"), u, mh::kF32,
                             dim(c_out, "c_out"), bias, upsample2x != 0, prologue_scale ? &aff : nullptr, out);
    });
}

int32_t mh_im2col_gather(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                         uint32_t stride, const uint32_t pad[4], uint32_t upsample2x, uint64_t first, uint64_t count,
                         float *rows) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(rows, "rows");
        int p[4];
        pad4(pad, p);
        mh::im2col_gather(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"), dim(stride, "stride"), p,
                          upsample2x != 0, int64_t(first), int64_t(count), rows);
    });
}

int32_t mh_depthwise3x3(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                        const float *weight, const float *bias, uint32_t epilogue, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(weight, "weight");
        need(bias, "bias");
        need(out, "out");
        if (epilogue > MH_EPILOGUE_GLU_SILU) mh::fail(mh::kInvalidArgument, "unknown depthwise epilogue");
        mh::depthwise3x3(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"), weight, bias, int(epilogue), out);
    });
}

int32_t mh_depthwise3x3_fused(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                              const float *weight, const float *bias, uint32_t epilogue, const float *prologue_scale,
                              const float *prologue_shift, uint32_t prologue_silu, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(weight, "weight");
        need(bias, "bias");
        need(out, "out");
        need(prologue_scale, "prologue_scale");
        need(prologue_shift, "prologue_shift");
        if (epilogue > MH_EPILOGUE_GLU_SILU) mh::fail(mh::kInvalidArgument, "unknown depthwise epilogue");
        mh::Affine aff;
        aff.scale = prologue_scale;
        aff.shift = prologue_shift;
        aff.silu = prologue_silu != 0;
        mh::depthwise3x3(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"), weight, bias, int(epilogue), out,
                         &aff);
    });
}

int32_t mh_group_norm_affine(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                             uint32_t groups, float eps, const float *gamma, const float *beta, const float *add,
                             float *scale, float *shift) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(gamma, "gamma");
        need(beta, "beta");
        need(scale, "scale");
        need(shift, "shift");
        mh::group_norm_affine(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"), dim(groups, "groups"), eps,
                              gamma, beta, add, scale, shift);
    });
}

int32_t mh_group_norm_affine_partials(MhContext *ctx, const float *part, uint32_t rows, uint32_t n, uint32_t h,
                                      uint32_t w, uint32_t c, uint32_t groups, float eps, const float *gamma,
                                      const float *beta, const float *add, float *scale, float *shift) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(part, "part");
        need(gamma, "gamma");
        need(beta, "beta");
        need(scale, "scale");
        need(shift, "shift");
        MH_REQUIRE(int64_t(h) * w < (int64_t(1) << 31), "GroupNorm partials: map too large");
        mh::group_norm_affine_partials(cc, part, int(dim(rows, "rows")), dim(n, "n"),
                                       int(dim(h, "h")) * int(dim(w, "w")), dim(c, "c"), dim(groups, "groups"), eps,
                                       gamma, beta, add, scale, shift);
    });
}

int32_t mh_group_norm_forward(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                              uint32_t groups, float eps, const float *gamma, const float *beta, const float *add,
                              uint32_t silu, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(gamma, "gamma");
        need(beta, "beta");
        need(out, "out");
        mh::group_norm_forward(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"), dim(groups, "groups"), eps,
                               gamma, beta, add, silu != 0, out);
    });
}

int32_t mh_group_norm_forward_noalloc(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w,
                                      uint32_t c, uint32_t groups, float eps, const float *gamma, const float *beta,
                                      const float *add, uint32_t silu, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(gamma, "gamma");
        need(beta, "beta");
        need(out, "out");
        mh::group_norm_forward_noalloc(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"),
                                       dim(groups, "groups"), eps, gamma, beta, add, silu != 0, out);
    });
}

int32_t mh_apply_affine(MhContext *ctx, const float *x, uint32_t n, uint32_t h, uint32_t w, uint32_t c,
                        const float *scale, const float *shift, uint32_t silu, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(scale, "scale");
        need(shift, "shift");
        need(out, "out");
        mh::apply_affine(cc, x, dim(n, "n"), dim(h, "h"), dim(w, "w"), dim(c, "c"), scale, shift, silu != 0, out);
    });
}

int32_t mh_layer_norm(MhContext *ctx, const float *x, uint64_t rows, uint32_t c, const float *gamma,
                      const float *beta, float eps, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(gamma, "gamma");
        need(beta, "beta");
        need(out, "out");
        mh::layer_norm(cc, x, int64_t(rows), dim(c, "c"), gamma, beta, eps, out);
    });
}

static void conv1x1_layer_norm_entry(MhContext *ctx, const float *x, uint64_t rows, uint32_t c_in, const float *gamma,
                                     const float *beta, float eps, const void *weight, uint32_t weight_dtype,
                                     uint32_t c_out, const float *bias, uint32_t silu, float *out,
                                     const mh::LnRowPartials *stats) {
    mh::Context &cc = C(ctx);
    need(x, "x");
    need(gamma, "gamma");
    need(beta, "beta");
    need(weight, "weight");
    need(out, "out");
    const int ci = dim(c_in, "c_in"), co = dim(c_out, "c_out");
    MH_REQUIRE(ci % 4 == 0 && co % 4 == 0, "Conv1x1 (LayerNorm): c_in and c_out must be multiples of 4");
    MH_REQUIRE(rows < (uint64_t(1) << 31), "Conv1x1 (LayerNorm): too many rows");
    auto al = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t nk = size_t(co) * ci;
    const size_t o16 = al(nk * 4), oc1 = o16 + al(nk * 2), oc16 = oc1 + al(size_t(co) * 4),
                 oc2 = oc16 + al(size_t(co) * 4), total = oc2 + al(size_t(co) * 4);
    char *ws = static_cast<char *>(cc.ws.get(total, cc.stream));
    float *w32 = reinterpret_cast<float *>(ws);
    float *c1_32 = reinterpret_cast<float *>(ws + oc1), *c1_16 = reinterpret_cast<float *>(ws + oc16);
    float *c2 = reinterpret_cast<float *>(ws + oc2);
    mh::ln_fold_weights(cc, weight, wtype(weight_dtype), co, ci, gamma, beta, bias, w32, ws + o16, c1_32, c1_16, c2);
    mh::LnFolded f;
    f.w32 = w32, f.c1_32 = c1_32, f.w16 = ws + o16, f.c1_16 = c1_16, f.c2 = c2, f.eps = eps;
    const int width = co;
    float *const outs[1] = {out};
    mh::conv1x1_ln(cc, x, int64_t(rows), ci, f, 1, &width, outs, silu ? mh::GemmEpilogue::Silu : mh::GemmEpilogue::None,
                   stats);
}

int32_t mh_conv1x1_layer_norm(MhContext *ctx, const float *x, uint64_t rows, uint32_t c_in, const float *gamma,
                              const float *beta, float eps, const void *weight, uint32_t weight_dtype, uint32_t c_out,
                              const float *bias, uint32_t silu, float *out) {
    return guard([&] {
        conv1x1_layer_norm_entry(ctx, x, rows, c_in, gamma, beta, eps, weight, weight_dtype, c_out, bias, silu, out,
                                 nullptr);
    });
}

int32_t mh_conv1x1_layer_norm_stats(MhContext *ctx, const float *x, uint64_t rows, uint32_t c_in, const float *gamma,
                                    const float *beta, float eps, const void *weight, uint32_t weight_dtype,
                                    uint32_t c_out, const float *bias, uint32_t silu, const float *row_partials,
                                    uint32_t per_row, float *out) {
    return guard([&] {
        need(row_partials, "row_partials");
        MH_REQUIRE(per_row > 0 && per_row <= 4096, "Conv1x1 (LayerNorm): 1 to 4096 row partials per row");
        MH_REQUIRE((reinterpret_cast<uintptr_t>(row_partials) & 7) == 0, "row partials must be 8-byte aligned");
        mh::LnRowPartials st;
        st.part = reinterpret_cast<float2 *>(const_cast<float *>(row_partials));
        st.per_row = int(per_row);
        conv1x1_layer_norm_entry(ctx, x, rows, c_in, gamma, beta, eps, weight, weight_dtype, c_out, bias, silu, out,
                                 &st);
    });
}

int32_t mh_conv1x1_row_partials(MhContext *ctx, const float *x, uint64_t rows, uint32_t c_in, const void *weight,
                                uint32_t weight_dtype, uint32_t c_out, const float *bias, float *out,
                                float *row_partials, uint32_t *per_row) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(weight, "weight");
        need(out, "out");
        need(row_partials, "row_partials");
        need(per_row, "per_row");
        MH_REQUIRE((reinterpret_cast<uintptr_t>(row_partials) & 7) == 0, "row partials must be 8-byte aligned");
        MH_REQUIRE(rows < (uint64_t(1) << 31), "Conv1x1: too many rows");
        mh::LnRowPartials st;
        st.part = reinterpret_cast<float2 *>(row_partials);
        mh::conv1x1(cc, x, int64_t(rows), dim(c_in, "c_in"), weight, wtype(weight_dtype), dim(c_out, "c_out"), bias,
                    nullptr, out, mh::GemmEpilogue::None, nullptr, nullptr, nullptr, nullptr, nullptr, 0, &st);
        *per_row = uint32_t(st.per_row);
    });
}

int32_t mh_silu_inplace(MhContext *ctx, float *x, uint64_t len) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        mh::silu_inplace(cc, x, int64_t(len));
    });
}

int32_t mh_add_inplace(MhContext *ctx, float *a, const float *b, uint64_t len) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(a, "a");
        need(b, "b");
        mh::add_inplace(cc, a, b, int64_t(len));
    });
}

int32_t mh_concat_channels(MhContext *ctx, const float *a, uint32_t ca, const float *b, uint32_t cb,
                           uint64_t pixels, float *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(a, "a");
        need(b, "b");
        need(out, "out");
        mh::concat_channels(cc, a, dim(ca, "ca"), b, dim(cb, "cb"), int64_t(pixels), out);
    });
}

int32_t mh_to_u8(MhContext *ctx, const float *x, uint64_t len, uint8_t *out) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(out, "out");
        mh::to_u8(cc, x, int64_t(len), out);
    });
}

int32_t mh_math_eval(MhContext *ctx, uint32_t which, const float *x, uint64_t len, float *y) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(x, "x");
        need(y, "y");
        mh::math_eval(cc, int(which), x, int64_t(len), y);
    });
}

int32_t mh_softmax_lambda(MhContext *ctx, const float *keys, const float *v, uint32_t nb, uint32_t rows, uint32_t k,
                          uint32_t vd, float *lambda_t) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(keys, "keys");
        need(v, "v");
        need(lambda_t, "lambda_t");
        mh::softmax_lambda(c, keys, v, dim(nb, "nb"), dim(rows, "rows"), dim(k, "k"), dim(vd, "vd"), lambda_t);
    });
}

int32_t mh_tap_filter(MhContext *ctx, const float *a_t, const float *v, const float *yc, const float *residual,
                      float *out, uint32_t nb, uint32_t hh, uint32_t ww, uint32_t vd) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(a_t, "a_t");
        need(v, "v");
        need(yc, "yc");
        need(out, "out");
        mh::tap_filter(c, a_t, v, yc, residual, out, dim(nb, "nb"), dim(hh, "hh"), dim(ww, "ww"), dim(vd, "vd"));
    });
}

int32_t mh_tap_filter_row_sums(MhContext *ctx, const float *a_t, const float *v, const float *yc,
                               const float *residual, float *out, uint32_t nb, uint32_t hh, uint32_t ww, uint32_t vd,
                               float *row_sums, uint32_t *per_row) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(a_t, "a_t");
        need(v, "v");
        need(yc, "yc");
        need(out, "out");
        need(row_sums, "row_sums");
        need(per_row, "per_row");
        MH_REQUIRE(vd % 4 == 0, "tap_filter: value width must be a multiple of 4");
        *per_row = uint32_t(mh::tap_filter_row_parts(c, dim(hh, "hh"), dim(ww, "ww"), dim(vd, "vd")));
        mh::tap_filter(c, a_t, v, yc, residual, out, dim(nb, "nb"), dim(hh, "hh"), dim(ww, "ww"), dim(vd, "vd"),
                       nullptr, reinterpret_cast<float2 *>(row_sums));
    });
}

int32_t mh_tap_filter_ln(MhContext *ctx, const float *a_t, const float *v, const float *yc, const float *residual,
                         float *out, uint32_t nb, uint32_t hh, uint32_t ww, uint32_t vd, const float *gamma,
                         const float *beta, float eps, float *ln_out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(a_t, "a_t");
        need(v, "v");
        need(yc, "yc");
        need(out, "out");
        need(gamma, "gamma");
        need(beta, "beta");
        need(ln_out, "ln_out");
        mh::LayerNormOut lno;
        lno.gamma = gamma;
        lno.beta = beta;
        lno.eps = eps;
        lno.out = ln_out;
        mh::tap_filter(c, a_t, v, yc, residual, out, dim(nb, "nb"), dim(hh, "hh"), dim(ww, "ww"), dim(vd, "vd"), &lno);
    });
}

int32_t mh_lambda_position_coeffs(MhContext *ctx, const float *q, const float *w_aug_t, const float *lambda_t,
                                  uint32_t nb, uint32_t hw, uint32_t k, float *a_t, float *yc) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(q, "q");
        if (!mh::lambda_taps_ok(int(k))) mh::fail(mh::kInvalidArgument, "lambda position coefficients: k must be 40, 80 or 160");
        if ((lambda_t == nullptr) != (yc == nullptr) || (w_aug_t == nullptr) != (a_t == nullptr) ||
            (!w_aug_t && !lambda_t))
            mh::fail(mh::kInvalidArgument,
                     "lambda position coefficients: w_aug_t with a_t, lambda_t with yc, at least one pair");
        mh::lambda_taps(c, q, w_aug_t, lambda_t, dim(nb, "nb"), dim(hw, "hw"), int(k), a_t, yc);
    });
}

int32_t mh_self_lambda_fused(MhContext *ctx, const float *q, const float *w_aug_t, const float *lambda_t,
                             const float *v, const float *residual, float *out, uint32_t nb, uint32_t hh, uint32_t ww,
                             uint32_t k, float *row_sums) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(q, "q");
        need(w_aug_t, "w_aug_t");
        need(lambda_t, "lambda_t");
        need(v, "v");
        need(out, "out");
        if (!mh::lambda_taps_ok(int(k))) mh::fail(mh::kInvalidArgument, "self-lambda position path: k must be 40, 80 or 160");
        mh::self_lambda_fused(c, q, w_aug_t, lambda_t, v, residual, out, dim(nb, "nb"), dim(hh, "hh"), dim(ww, "ww"),
                              int(k), reinterpret_cast<float2 *>(row_sums));
    });
}

int32_t mh_position_term(MhContext *ctx, const float *q, const float *e, const float *v_branches, uint32_t br0,
                         uint32_t nb, uint32_t hw, uint32_t k, const float *yc, const float *residual, float *out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(q, "q");
        need(e, "e");
        need(v_branches, "v_branches");
        need(yc, "yc");
        need(out, "out");
        mh::position_term(c, q, e, v_branches, dim(br0, "br0"), dim(nb, "nb"), dim(hw, "hw"), dim(k, "k"), yc,
                          residual, out);
    });
}

int32_t mh_cross_lambda(MhContext *ctx, const float *q, const float *e, const float *lambda_c, const float *v_branches,
                        uint32_t br0, uint32_t nb, uint32_t hw, uint32_t k, const float *residual, float *out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(q, "q");
        need(e, "e");
        need(lambda_c, "lambda_c");
        need(v_branches, "v_branches");
        need(out, "out");
        mh::cross_lambda(c, q, e, lambda_c, v_branches, dim(br0, "br0"), dim(nb, "nb"), dim(hw, "hw"), dim(k, "k"),
                         residual, out);
    });
}

int32_t mh_cross_lambda_row_sums(MhContext *ctx, const float *q, const float *e, const float *lambda_c,
                                 const float *v_branches, uint32_t br0, uint32_t nb, uint32_t hw, uint32_t k,
                                 const float *residual, float *out, float *row_sums) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(q, "q");
        need(e, "e");
        need(lambda_c, "lambda_c");
        need(v_branches, "v_branches");
        need(out, "out");
        need(row_sums, "row_sums");
        mh::cross_lambda(c, q, e, lambda_c, v_branches, dim(br0, "br0"), dim(nb, "nb"), dim(hw, "hw"), dim(k, "k"),
                         residual, out, reinterpret_cast<float2 *>(row_sums));
    });
}

int32_t mh_gemm_nt(MhContext *ctx, const float *a, uint64_t lda, const void *b, uint32_t b_dtype, uint64_t ldb,
                   uint32_t m, uint32_t n, uint32_t k, const float *bias, const float *residual, float *c,
                   uint64_t ldc, uint32_t row_group) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(a, "a");
        need(b, "b");
        need(c, "c");
        const uint64_t row_len = uint64_t(n) * (row_group > 1 ? row_group : 1);
        if (lda < k || ldb < k || ldc < row_len) mh::fail(mh::kInvalidArgument, "gemm: leading dimension too small");
        if (row_group > 64) mh::fail(mh::kInvalidArgument, "gemm: row group above 64");
        mh::gemm_nt(cc, a, int64_t(lda), 0, b, wtype(b_dtype), int64_t(ldb), 0, dim(m, "m"), dim(n, "n"),
                    dim(k, "k"), 1, bias, residual, c, int64_t(ldc), 0, mh::GemmEpilogue::None, int(row_group));
    });
}

int32_t mh_unet_create(MhContext *ctx, const MhNamedTensor *tensors, uint32_t count, MhUNet **out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(out, "out");
        *out = nullptr;
        need(tensors, "tensors");
        std::vector<mh::NamedTensor> t(count);
        for (uint32_t i = 0; i < count; ++i) {
            t[i].name = tensors[i].name;
            t[i].data = tensors[i].data;
            t[i].dtype = tensors[i].dtype;
            t[i].numel = tensors[i].numel;
        }
        auto u = std::make_unique<MhUNet>();
        u->owner = ctx;
        u->net = std::make_unique<mh::UNet>(c, t.data(), int(count));
        *out = u.release();
    });
}

void mh_unet_destroy(MhUNet *unet) {
    if (!unet) return;
    (void)hipSetDevice(unet->owner->ctx.device);
    delete unet;
}

static mh::Context &unet_ctx(MhUNet *u) {
    if (!u) mh::fail(mh::kInvalidArgument, "unet is NULL");
    return C(u->owner);
}

static bool guidance_cfg(uint32_t g) {
    if (g == MH_GUIDANCE_CFG) return true;
    if (g == MH_GUIDANCE_COND_ONLY) return false;
    mh::fail(mh::kInvalidArgument, "unknown guidance");
}

int32_t mh_unet_forward(MhUNet *unet, const float *x_dev, uint32_t timestep, uint32_t guidance, float *eps_dev) {
    return guard([&] {
        unet_ctx(unet);
        need(x_dev, "x");
        need(eps_dev, "eps");
        unet->net->forward(x_dev, int(timestep), guidance_cfg(guidance), eps_dev);
    });
}

int32_t mh_unet_forward_host(MhUNet *unet, const float *x_host, uint32_t timestep, uint32_t guidance,
                             float *eps_host) {
    return guard([&] {
        mh::Context &c = unet_ctx(unet);
        need(x_host, "x");
        need(eps_host, "eps");
        const bool cfg = guidance_cfg(guidance);
        if (!unet->x_dev) mh::dev_malloc(&unet->x_dev, 64 * 64 * 9 * sizeof(float));
        if (!unet->eps_dev) mh::dev_malloc(&unet->eps_dev, 2 * 64 * 64 * 4 * sizeof(float));
        HIP_CHECK(hipMemcpyAsync(unet->x_dev, x_host, 64 * 64 * 9 * sizeof(float), hipMemcpyHostToDevice, c.stream));
        unet->net->forward(unet->x_dev, int(timestep), cfg, unet->eps_dev);
        HIP_CHECK(hipMemcpyAsync(eps_host, unet->eps_dev, size_t(cfg ? 2 : 1) * 64 * 64 * 4 * sizeof(float),
                                 hipMemcpyDeviceToHost, c.stream));
        HIP_CHECK(hipStreamSynchronize(c.stream));
    });
}

namespace {
struct TraceCtx {
    MhTraceFn fn;
    void *user;
    hipStream_t stream;
};
void trace_bridge(void *user, const char *name, const float *dev, int n, int h, int w, int c) {
    auto *t = static_cast<TraceCtx *>(user);
    HIP_CHECK(hipStreamSynchronize(t->stream));
    t->fn(t->user, name, dev, uint32_t(n), uint32_t(h), uint32_t(w), uint32_t(c));
}
}  // namespace

int32_t mh_unet_forward_traced(MhUNet *unet, const float *x_dev, uint32_t timestep, uint32_t guidance,
                               float *eps_dev, MhTraceFn trace, void *user) {
    return guard([&] {
        mh::Context &c = unet_ctx(unet);
        need(x_dev, "x");
        need(eps_dev, "eps");
        TraceCtx tc{trace, user, c.stream};
        unet->net->forward(x_dev, int(timestep), guidance_cfg(guidance), eps_dev, trace ? trace_bridge : nullptr,
                           &tc);
    });
}

int32_t mh_unet_memory(MhUNet *unet, uint64_t *weight_bytes, uint64_t *pool_bytes) {
    return guard([&] {
        unet_ctx(unet);
        if (weight_bytes) *weight_bytes = unet->net->weight_bytes();
        if (pool_bytes) *pool_bytes = unet->net->pool_bytes();
    });
}

int32_t mh_vae_create(MhContext *ctx, const MhNamedTensor *tensors, uint32_t count, MhVae **out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(out, "out");
        *out = nullptr;
        need(tensors, "tensors");
        std::vector<mh::NamedTensor> t(count);
        for (uint32_t i = 0; i < count; ++i) {
            t[i].name = tensors[i].name;
            t[i].data = tensors[i].data;
            t[i].dtype = tensors[i].dtype;
            t[i].numel = tensors[i].numel;
        }
        auto v = std::make_unique<MhVae>();
        v->owner = ctx;
        v->vae = std::make_unique<mh::Vae>(c, t.data(), int(count));
        *out = v.release();
    });
}

void mh_vae_destroy(MhVae *vae) {
    if (!vae) return;
    (void)hipSetDevice(vae->owner->ctx.device);
    delete vae;
}

static mh::Context &vae_ctx(MhVae *v) {
    if (!v) mh::fail(mh::kInvalidArgument, "vae is NULL");
    return C(v->owner);
}

int32_t mh_vae_encode(MhVae *vae, const float *images_dev, uint32_t b, uint32_t h, uint32_t w,
                      const float *noise_dev, float *z_dev, MhTraceFn trace, void *user) {
    return guard([&] {
        mh::Context &c = vae_ctx(vae);
        need(images_dev, "images");
        need(noise_dev, "noise");
        need(z_dev, "z");
        TraceCtx tc{trace, user, c.stream};
        vae->vae->encode(images_dev, dim(b, "b"), dim(h, "h"), dim(w, "w"), noise_dev, z_dev,
                         trace ? trace_bridge : nullptr, &tc);
    });
}

int32_t mh_vae_decode(MhVae *vae, const float *latents_dev, uint32_t h, uint32_t w, float *out_dev,
                      MhTraceFn trace, void *user) {
    return guard([&] {
        mh::Context &c = vae_ctx(vae);
        need(latents_dev, "latents");
        need(out_dev, "out");
        TraceCtx tc{trace, user, c.stream};
        vae->vae->decode(latents_dev, dim(h, "h"), dim(w, "w"), out_dev, trace ? trace_bridge : nullptr, &tc);
    });
}

int32_t mh_vae_encode_host(MhVae *vae, const float *images, uint32_t b, uint32_t h, uint32_t w, const float *noise,
                           float *z) {
    return guard([&] {
        mh::Context &c = vae_ctx(vae);
        need(images, "images");
        need(noise, "noise");
        need(z, "z");
        const size_t ib = size_t(b) * h * w * 3 * sizeof(float);
        const size_t zb = size_t(b) * (h / 8) * (w / 8) * 4 * sizeof(float);
        float *d = nullptr;
        mh::dev_malloc(&d, ib + 2 * zb);
        struct Free {
            float *p;
            ~Free() { (void)hipFree(p); }
        } f{d};
        float *dn = d + ib / sizeof(float), *dz = dn + zb / sizeof(float);
        HIP_CHECK(hipMemcpyAsync(d, images, ib, hipMemcpyHostToDevice, c.stream));
        HIP_CHECK(hipMemcpyAsync(dn, noise, zb, hipMemcpyHostToDevice, c.stream));
        vae->vae->encode(d, dim(b, "b"), dim(h, "h"), dim(w, "w"), dn, dz);
        HIP_CHECK(hipMemcpyAsync(z, dz, zb, hipMemcpyDeviceToHost, c.stream));
        HIP_CHECK(hipStreamSynchronize(c.stream));
    });
}

int32_t mh_vae_decode_host(MhVae *vae, const float *latents, uint32_t h, uint32_t w, float *out) {
    return guard([&] {
        mh::Context &c = vae_ctx(vae);
        need(latents, "latents");
        need(out, "out");
        const size_t lb = size_t(h) * w * 4 * sizeof(float);
        const size_t ob = size_t(h) * w * 64 * 3 * sizeof(float);
        float *d = nullptr;
        mh::dev_malloc(&d, lb + ob);
        struct Free {
            float *p;
            ~Free() { (void)hipFree(p); }
        } f{d};
        float *dout = d + lb / sizeof(float);
        HIP_CHECK(hipMemcpyAsync(d, latents, lb, hipMemcpyHostToDevice, c.stream));
        vae->vae->decode(d, dim(h, "h"), dim(w, "w"), dout);
        HIP_CHECK(hipMemcpyAsync(out, dout, ob, hipMemcpyDeviceToHost, c.stream));
        HIP_CHECK(hipStreamSynchronize(c.stream));
    });
}

int32_t mh_vae_memory(MhVae *vae, uint64_t *weight_bytes, uint64_t *pool_bytes) {
    return guard([&] {
        vae_ctx(vae);
        if (weight_bytes) *weight_bytes = vae->vae->weight_bytes();
        if (pool_bytes) *pool_bytes = vae->vae->pool_bytes();
    });
}

int32_t mh_softmax_rows(MhContext *ctx, float *rows, uint64_t nrows, uint32_t n, float scale) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(rows, "rows");
        if (!(scale > 0.0f)) mh::fail(mh::kInvalidArgument, "softmax_rows: scale must be positive");
        mh::softmax_rows(c, rows, int64_t(nrows), dim(n, "n"), scale);
    });
}

int32_t mh_vae_sample(MhContext *ctx, const float *moments, const float *noise, uint64_t pixels, float *z) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(moments, "moments");
        need(noise, "noise");
        need(z, "z");
        mh::vae_sample(c, moments, noise, int64_t(pixels), z);
    });
}

void mh_timestep_sinusoid(uint32_t t, float *out) {
    if (out) mh::timestep_sinusoid(int(t), out);
}

int64_t mh_scratch_best_fit(const uint64_t *lens, const uint64_t *caps, uint64_t count, uint64_t len) {
    if (count == 0 || !lens || !caps) return -1;
    return mh::best_fit(lens, caps, int64_t(count), len);
}

int32_t mh_selftest_mfma_f32(MhContext *ctx, const float *a, const float *b, float *d) {
    return guard([&] {
        mh::Context &cc = C(ctx);
        need(a, "a");
        need(b, "b");
        need(d, "d");
        mh::selftest_mfma_f32(cc, a, b, d);
    });
}

}  // extern "C"

// ---- samplers and the denoise loop

static mh::Spacing spacing_of(uint32_t v) {
    if (v == MH_SPACING_LEADING) return mh::Spacing::Leading;
    if (v == MH_SPACING_TRAILING) return mh::Spacing::Trailing;
    mh::fail(mh::kInvalidArgument, "unknown spacing");
}

int32_t mh_schedule_timesteps(uint32_t steps, double strength, uint32_t spacing, uint32_t *out, uint32_t *count,
                              uint32_t *pure_noise) {
    return guard([&] {
        need(out, "out");
        need(count, "count");
        const mh::Schedule s(int(std::min<uint32_t>(steps, 1u << 30)), strength, spacing_of(spacing));
        for (size_t i = 0; i < s.timesteps.size(); ++i) out[i] = uint32_t(s.timesteps[i]);
        *count = uint32_t(s.timesteps.size());
        if (pure_noise) *pure_noise = s.pure_noise_start ? 1u : 0u;
    });
}

int32_t mh_schedule_alphas_cumprod(float *out) {
    return guard([&] {
        need(out, "out");
        const std::vector<float> a = mh::scaled_linear_alphas_cumprod();
        std::memcpy(out, a.data(), a.size() * sizeof(float));
    });
}

int32_t mh_scheduler_create(MhContext *ctx, uint32_t steps, double strength, uint32_t spacing, uint64_t len,
                            MhScheduler **out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(out, "out");
        *out = nullptr;
        auto s = std::make_unique<MhScheduler>();
        s->owner = ctx;
        s->s = std::make_unique<mh::Sampler>(c, int(std::min<uint32_t>(steps, 1u << 30)), strength,
                                             spacing_of(spacing), int64_t(len));
        *out = s.release();
    });
}

void mh_scheduler_destroy(MhScheduler *s) {
    if (!s) return;
    (void)hipSetDevice(s->owner->ctx.device);
    delete s;
}

static mh::Sampler &sampler(MhScheduler *s) {
    if (!s) mh::fail(mh::kInvalidArgument, "scheduler is NULL");
    C(s->owner);
    return *s->s;
}

int32_t mh_scheduler_add_noise(MhScheduler *s, const float *x0, const float *noise, uint32_t t, float *out) {
    return guard([&] {
        mh::Sampler &p = sampler(s);
        need(x0, "x0");
        need(noise, "noise");
        need(out, "out");
        p.add_noise(x0, noise, int(std::min<uint32_t>(t, 1u << 30)), out);
    });
}

int32_t mh_scheduler_ddim_step(MhScheduler *s, const float *eps_u, const float *eps_c, float guidance, uint32_t t,
                               float *x) {
    return guard([&] {
        mh::Sampler &p = sampler(s);
        need(eps_u, "eps");
        need(x, "x");
        p.ddim_step(eps_u, eps_c, guidance, int(std::min<uint32_t>(t, 1u << 30)), x);
    });
}

int32_t mh_scheduler_dpm_step(MhScheduler *s, const float *eps_u, const float *eps_c, float guidance, uint32_t i,
                              float *x) {
    return guard([&] {
        mh::Sampler &p = sampler(s);
        need(eps_u, "eps");
        need(x, "x");
        p.dpm_step(eps_u, eps_c, guidance, int(std::min<uint32_t>(i, 1u << 30)), x);
    });
}

int32_t mh_scheduler_dpm_restart(MhScheduler *s) {
    return guard([&] { sampler(s).restart(); });
}

int32_t mh_unet_denoise(MhUNet *unet, const float *z_img, const float *init, const float *mask_lat,
                        const float *z_masked, const MhDenoiseParams *params, MhStepFn progress, void *user,
                        float *latents) {
    return guard([&] {
        mh::Context &c = unet_ctx(unet);
        need(params, "params");
        need(init, "init");
        need(mask_lat, "mask_lat");
        need(z_masked, "z_masked");
        need(latents, "latents");
        mh::DenoiseParams p;
        p.steps = params->steps;
        p.strength = params->strength;
        p.spacing = spacing_of(params->spacing);
        if (params->solver == MH_SOLVER_DDIM) p.solver = mh::Solver::Ddim;
        else if (params->solver == MH_SOLVER_DPMPP_2M) p.solver = mh::Solver::DpmPp2M;
        else mh::fail(mh::kInvalidArgument, "unknown solver");
        p.guidance = params->guidance;
        p.cfg_steps = params->cfg_steps;
        mh::unet_denoise(c, *unet->net, z_img, init, mask_lat, z_masked, p, progress, user, latents);
    });
}

// ---- weights from files

static mh::ModelKind model_of(uint32_t m) {
    if (m == MH_MODEL_UNET) return mh::ModelKind::UNet;
    if (m == MH_MODEL_VAE) return mh::ModelKind::Vae;
    mh::fail(mh::kInvalidArgument, "unknown model");
}

int32_t mh_weights_validate(const char *path, uint32_t model) {
    return guard([&] {
        need(path, "path");
        const mh::ModelKind kind = model_of(model);
        const mh::WeightsFile f(path);
        (void)mh::model_tensors(f, kind);
    });
}

int32_t mh_unet_create_from_file(MhContext *ctx, const char *path, MhUNet **out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(out, "out");
        *out = nullptr;
        need(path, "path");
        const mh::WeightsFile f(path);
        const std::vector<mh::NamedTensor> t = mh::model_tensors(f, mh::ModelKind::UNet);
        auto u = std::make_unique<MhUNet>();
        u->owner = ctx;
        u->net = std::make_unique<mh::UNet>(c, t.data(), int(t.size()));
        HIP_CHECK(hipStreamSynchronize(c.stream));  // the uploads have read the mapping
        *out = u.release();
    });
}

int32_t mh_vae_create_from_file(MhContext *ctx, const char *path, MhVae **out) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(out, "out");
        *out = nullptr;
        need(path, "path");
        const mh::WeightsFile f(path);
        const std::vector<mh::NamedTensor> t = mh::model_tensors(f, mh::ModelKind::Vae);
        auto v = std::make_unique<MhVae>();
        v->owner = ctx;
        v->vae = std::make_unique<mh::Vae>(c, t.data(), int(t.size()));
        HIP_CHECK(hipStreamSynchronize(c.stream));
        *out = v.release();
    });
}

// ---- imaging (host)

int32_t mh_mask_bbox(const uint8_t *mask, uint32_t width, uint32_t height, uint32_t stride, uint32_t *rect,
                     uint32_t *found) {
    return guard([&] {
        need(mask, "mask");
        need(rect, "rect");
        MH_REQUIRE(stride >= width, "mask stride below its width");
        mh::img::Rect r;
        const bool f = mh::img::mask_bbox({mask, width, height, stride}, &r);
        rect[0] = uint32_t(r.x), rect[1] = uint32_t(r.y), rect[2] = uint32_t(r.w), rect[3] = uint32_t(r.h);
        if (found) *found = f ? 1u : 0u;
    });
}

int32_t mh_mask_dilate(const uint8_t *mask, uint32_t width, uint32_t height, uint32_t stride, uint32_t k,
                       uint8_t *out) {
    return guard([&] {
        need(mask, "mask");
        need(out, "out");
        MH_REQUIRE(stride >= width, "mask stride below its width");
        const std::vector<uint8_t> d = mh::img::dilate({mask, width, height, stride}, k);
        std::memcpy(out, d.data(), d.size());
    });
}

int32_t mh_crop_plan(const uint32_t *bbox, uint32_t img_w, uint32_t img_h, int64_t *x, int64_t *y, uint32_t *side) {
    return guard([&] {
        need(bbox, "bbox");
        need(x, "x");
        need(y, "y");
        need(side, "side");
        MH_REQUIRE(bbox[2] > 0 && bbox[3] > 0 && uint64_t(bbox[0]) + bbox[2] <= img_w &&
                       uint64_t(bbox[1]) + bbox[3] <= img_h,
                   "mask bbox outside the image");
        const mh::img::CropPlan p = mh::img::crop_plan({bbox[0], bbox[1], bbox[2], bbox[3]}, img_w, img_h);
        *x = p.x, *y = p.y, *side = uint32_t(p.side);
    });
}

int32_t mh_gaussian_blur(const uint8_t *src, uint32_t width, uint32_t height, float radius, uint8_t *out) {
    return guard([&] {
        need(src, "src");
        need(out, "out");
        const std::vector<uint8_t> b = mh::img::gaussian_blur(src, width, height, radius, host_threads());
        std::memcpy(out, b.data(), b.size());
    });
}

static mh::img::Paste paste_of(uint32_t m) {
    if (m == MH_PASTE_NONE) return mh::img::Paste::None;
    if (m == MH_PASTE_FEATHER) return mh::img::Paste::Feather;
    if (m == MH_PASTE_FEATHER_COMPENSATE) return mh::img::Paste::FeatherCompensate;
    mh::fail(mh::kInvalidArgument, "unknown paste mode " + std::to_string(m));
}

int32_t mh_paste(uint8_t *pixels, uint32_t width, uint32_t height, uint32_t stride, uint32_t channels,
                 const uint8_t *mask, uint32_t mask_stride, const uint8_t *result, int64_t plan_x, int64_t plan_y,
                 uint32_t side, uint32_t mode, uint32_t *changed) {
    return guard([&] {
        need(pixels, "pixels");
        need(mask, "mask");
        need(result, "result");
        MH_REQUIRE(channels == 3 || channels == 4, "image must be RGB or RGBA");
        MH_REQUIRE(stride >= uint64_t(width) * channels && mask_stride >= width, "bad dimensions or stride");
        mh::img::ImageView im{pixels, width, height, stride, channels};
        mh::img::CropPlan p;
        p.x = plan_x, p.y = plan_y, p.side = side;
        MH_REQUIRE(side > 0 && plan_x < int64_t(width) && plan_y < int64_t(height) && plan_x + int64_t(side) > 0 &&
                       plan_y + int64_t(side) > 0,
                   "paste window does not overlap the image");
        const mh::img::Rect r = mh::img::paste(im, {mask, width, height, mask_stride}, result, p, paste_of(mode),
                                               host_threads());
        if (changed) changed[0] = uint32_t(r.x), changed[1] = uint32_t(r.y), changed[2] = uint32_t(r.w),
                     changed[3] = uint32_t(r.h);
    });
}

int32_t mh_roi_window(const float *mask_lat, uint32_t margin, uint32_t *rect, uint32_t *found) {
    return guard([&] {
        need(mask_lat, "mask_lat");
        need(rect, "rect");
        mh::img::LatentRect r;
        const bool f = mh::img::roi_window(mask_lat, margin, &r);
        rect[0] = uint32_t(r.x), rect[1] = uint32_t(r.y), rect[2] = uint32_t(r.w), rect[3] = uint32_t(r.h);
        if (found) *found = f ? 1u : 0u;
    });
}

int32_t mh_resize_u8(MhContext *ctx, const uint8_t *src, uint32_t from_w, uint32_t from_h, uint32_t to_w,
                     uint32_t to_h, uint32_t channels, uint8_t *dst) {
    return guard([&] {
        mh::Context &c = C(ctx);
        need(src, "src");
        need(dst, "dst");
        MH_REQUIRE(from_w <= 65536 && from_h <= 65536 && to_w <= 65536 && to_h <= 65536, "resize: image too large");
        mh::resize_u8(c, src, int(from_w), int(from_h), int(to_w), int(to_h), int(channels), dst);
    });
}
