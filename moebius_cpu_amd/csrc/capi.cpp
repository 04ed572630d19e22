// The C ABI of include/moebius_hip.h. Every entry point validates its
// arguments, runs the C++ engine function and converts any mh::Error or other
// exception into a status code plus a thread-local message, mirroring the
// reference's FFI guard (src/ffi.rs:90-103) and moebius_last_error
// (include/moebius_cpu.h:50-51). Nothing throws across the boundary.
#include <cstring>
#include <exception>
#include <new>
#include <string>

#include "../../include/moebius_hip.h"
#include "common.hpp"
#include "kernels.hpp"

struct MhContext {
    mh::Context ctx;
    explicit MhContext(int dev) : ctx(dev) {}
};

struct MhEvent {
    hipEvent_t ev = nullptr;
    int device = 0;
};

namespace {

thread_local std::string g_last_error = "no error";

int32_t set_error(int32_t code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

template <typename F>
int32_t guard(F &&f) {
    try {
        f();
        return mh::kOk;
    } catch (const mh::Error &e) {
        return set_error(e.code, e.what());
    } catch (const std::bad_alloc &) {
        return set_error(mh::kOutOfMemory, "host allocation failed");
    } catch (const std::exception &e) {
        return set_error(mh::kInternal, std::string("internal error: ") + e.what());
    } catch (...) {
        return set_error(mh::kInternal, "internal error: unknown exception");
    }
}

mh::Context &C(MhContext *c) {
    if (!c) mh::fail(mh::kInvalidArgument, "context is NULL");
    HIP_CHECK(hipSetDevice(c->ctx.device));
    return c->ctx;
}

void need(const void *p, const char *what) {
    if (!p) mh::fail(mh::kInvalidArgument, std::string(what) + " is NULL");
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

int dim(uint32_t v, const char *what) {
    if (v > (1u << 30)) mh::fail(mh::kInvalidArgument, std::string(what) + " too large");
    return int(v);
}

}  // namespace

extern "C" {

uint32_t mh_abi_version(void) { return MH_ABI_VERSION; }

const char *mh_last_error(void) { return g_last_error.c_str(); }

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

int32_t mh_context_set_precision(MhContext *ctx, uint32_t precision) {
    return guard([&] {
        mh::Context &c = C(ctx);
        if (precision == MH_PRECISION_EXACT) c.precision = mh::Precision::Exact;
        else if (precision == MH_PRECISION_FAST) c.precision = mh::Precision::Fast;
        else mh::fail(mh::kInvalidArgument, "unknown precision");
    });
}

void *mh_context_stream(MhContext *ctx) { return ctx ? static_cast<void *>(ctx->ctx.stream) : nullptr; }

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
        HIP_CHECK(hipMalloc(out, bytes ? bytes : 1));
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
