// Device VAE: src/vae/{mod,encoder,decoder}.rs over the gfx950 kernels.
//
// Every GroupNorm + SiLU in front of a 3x3 conv is written out once (the
// reference fuses it into the conv's gather to save CPU memory traffic; here
// the gather would re-evaluate SiLU per tap and tile); the resnet's identity
// add is the conv epilogue's second residual. The mid attention keeps its
// whole 4096 x 4096 score matrix per item in HBM: q.k^T on the matrix cores,
// the row softmax with the reference's flush threshold, then P.v. The encoder
// runs its batch together (the reference runs items one after the other;
// every statistic is per item).
#include "vae.hpp"

#include <cmath>
#include <string>
#include <vector>

namespace mh {

namespace {

// src/config.rs:50-58
constexpr int VCH[4] = {128, 256, 512, 512};
constexpr int GROUPS = 32;
constexpr float VAE_EPS = 1e-6f;
constexpr int LATENT_C = 4;
constexpr int IMAGE_C = 3;
constexpr int LAYERS = 2;  // src/vae/encoder.rs:23

struct Env {
    Context &ctx;
    Pool &pool;
};

// Attaches the GroupNorm partials a producer wrote to its output, or returns the buffer.
void attach(Env &e, DT &out, const GnPartials &gp) {
    if (!gp.part) return;
    if (gp.rows > 0) {
        out.gn = gp.part;
        out.gn_rows = gp.rows;
    } else {
        e.pool.recycle(gp.part);
    }
}

struct GNv {  // GroupNorm, eps 1e-6 (src/engine/norm.rs:22-105)
    int c = 0;
    const float *g = nullptr, *b = nullptr;
    void load(const WeightStore &W, const std::string &p, int c_) {
        c = c_;
        g = W.get(p + ".weight", c, false).f();
        b = W.get(p + ".bias", c, false).f();
    }
    // The statistics come from the producer's partials where it wrote them
    // (the one-kernel Winograd conv, the 1x1 GEMMs), else from a pass over x.
    DT fwd(Env &e, const DT &x, bool silu = false) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, x.c);
        if (x.gn) {
            float *ss = affine(e, x);
            apply_affine(e.ctx, x.p, x.n, x.h, x.w, x.c, ss, ss + int64_t(x.n) * x.c, silu, out.p);
            e.pool.recycle(ss);
        } else {
            group_norm_forward(e.ctx, x.p, x.n, x.h, x.w, x.c, GROUPS, VAE_EPS, g, b, nullptr, silu, out.p);
        }
        return out;
    }
    // Statistics only: [scale | shift], each [n * c], for a consumer that applies them.
    float *affine(Env &e, const DT &x) const {
        float *ss = e.pool.floats(int64_t(2) * x.n * x.c);
        if (x.gn)
            group_norm_affine_partials(e.ctx, x.gn, x.gn_rows, x.n, x.h * x.w, x.c, GROUPS, VAE_EPS, g, b, nullptr, ss,
                                       ss + int64_t(x.n) * x.c);
        else
            group_norm_affine(e.ctx, x.p, x.n, x.h, x.w, x.c, GROUPS, VAE_EPS, g, b, nullptr, ss,
                              ss + int64_t(x.n) * x.c);
        return ss;
    }
};

// Conv3x3 (src/engine/conv.rs:60-102). Stride-1 / pad-1 convs run as
// Winograd F(2x2,3x3) like the reference's (conv.rs:92-98), with the kernel
// transformed at load (1.2-2.4x faster than the implicit GEMM at the VAE's
// 128-512-channel shapes, f32); the others (stride-2 downsample, 3-channel
// image and latent convs) are implicit GEMMs.
struct Conv3v {
    int ci = 0, co = 0, stride = 1;
    int pad[4] = {1, 1, 1, 1};
    bool up = false;
    DParam w;
    const float *u = nullptr;
    const float *uf = nullptr;  // u in the one-kernel path's order (channel counts it takes)
    const float *b = nullptr;
    void load(const WeightStore &W, const std::string &p, int ci_, int co_, int stride_ = 1,
              const int *pad_ = nullptr, bool up_ = false) {
        ci = ci_, co = co_, stride = stride_, up = up_;
        if (pad_)
            for (int i = 0; i < 4; ++i) pad[i] = pad_[i];
        w = W.get(p + ".weight", int64_t(co) * 9 * ci, true);
        b = W.get(p + ".bias", co, false).f();
        const bool same = stride == 1 && pad[0] == 1 && pad[1] == 1 && pad[2] == 1 && pad[3] == 1;
        if (same && ci % 4 == 0 && co % 4 == 0) u = W.winograd_kernel(w, co, ci);
        if (u && ci % 32 == 0 && co % 64 == 0) uf = W.winograd_kernel_fused(u, co, ci);
    }
    // res2 (optional) added last: out = (bias + conv) + res2.
    DT fwd(Env &e, const DT &x, const float *res2 = nullptr, float *out_p = nullptr) const {
        int ho, wo;
        conv3x3_output_hw(x.h, x.w, stride, pad, up, &ho, &wo);
        DT out = out_p ? DT{out_p, x.n, ho, wo, co} : e.pool.tensor(x.n, ho, wo, co);
        if (u) {
            // GroupNorm partials for the next GroupNorm, where the one-kernel path runs
            GnPartials gp;
            if (uf && !out_p) {
                gp.part = e.pool.floats(ceil_div(winograd_tiles(x.n, x.h, x.w, up), 32) * co * 2);
                gp.item_rows = ho * wo;
            }
            conv3x3_winograd(e.ctx, x.p, x.n, x.h, x.w, x.c, u, kF32, co, b, up, nullptr, out.p, res2, uf,
                             gp.part ? &gp : nullptr);
            attach(e, out, gp);
        } else {
            conv3x3(e.ctx, x.p, x.n, x.h, x.w, x.c, w.p, w.wt, co, b, stride, pad, up, nullptr, out.p, res2);
        }
        return out;
    }
    // conv(SiLU(GN(x))): the normalised map is written once and read by the conv.
    // (Applying GN + SiLU inside the conv's gather, as the reference's
    // forward_prologue does, re-evaluates SiLU for every tap and column tile:
    // on the matrix cores that costs more than one extra pass over the map.)
    // The exception is the image conv (c_out <= 8, no Winograd kernel): its
    // direct kernel stages each input value once per tile, so it applies
    // GN + SiLU itself and the normalised map is never written.
    DT fwd_gn(Env &e, const GNv &gn, const DT &x, const float *res2 = nullptr, float *out_p = nullptr) const {
        const bool same = stride == 1 && pad[0] == 1 && pad[1] == 1 && pad[2] == 1 && pad[3] == 1 && !up;
        if (co <= 8 && !u && same) {
            float *ss = gn.affine(e, x);
            const Affine a{ss, ss + int64_t(x.n) * x.c, true};
            DT out = out_p ? DT{out_p, x.n, x.h, x.w, co} : e.pool.tensor(x.n, x.h, x.w, co);
            conv3x3(e.ctx, x.p, x.n, x.h, x.w, x.c, w.p, w.wt, co, b, stride, pad, up, &a, out.p, res2);
            e.pool.recycle(ss);
            return out;
        }
        DT a = gn.fwd(e, x, true);
        DT out = fwd(e, a, res2, out_p);
        e.pool.recycle(a);
        return out;
    }
};

struct Lin {  // Conv1x1 (src/engine/conv.rs:28-55)
    int ci = 0, co = 0;
    DParam w;
    const float *b = nullptr;
    void load(const WeightStore &W, const std::string &p, int ci_, int co_) {
        ci = ci_, co = co_;
        w = W.get(p + ".weight", int64_t(ci) * co, true);
        b = W.get(p + ".bias", co, false).f();
    }
    DT fwd(Env &e, const DT &x, const float *res = nullptr) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, co);
        GnPartials gp;  // for a following GroupNorm (channel counts that have one)
        if (co % GROUPS == 0) {
            gp.part = e.pool.floats(ceil_div(x.px(), 32) * co * 2);
            gp.item_rows = x.h * x.w;
        }
        conv1x1(e.ctx, x.p, x.px(), ci, w.p, w.wt, co, b, res, out.p, GemmEpilogue::None, nullptr, nullptr,
                gp.part ? &gp : nullptr);
        attach(e, out, gp);
        return out;
    }
};

// src/vae/mod.rs:174-211
struct Resnet {
    int ci = 0, co = 0;
    GNv n1, n2;
    Conv3v c1, c2;
    bool has_sc = false;
    Lin sc;
    void load(const WeightStore &W, const std::string &p, int ci_, int co_) {
        ci = ci_, co = co_;
        n1.load(W, p + ".norm1", ci);
        c1.load(W, p + ".conv1", ci, co);
        n2.load(W, p + ".norm2", co);
        c2.load(W, p + ".conv2", co, co);
        has_sc = ci != co;
        if (has_sc) sc.load(W, p + ".conv_shortcut", ci, co);
    }
    DT fwd(Env &e, const DT &x) const {
        DT h = c1.fwd_gn(e, n1, x);
        DT out;
        if (has_sc) {
            // h2 = conv2(...), then shortcut(x) with residual h2 (mod.rs:205-207)
            DT h2 = c2.fwd_gn(e, n2, h);
            out = sc.fwd(e, x, h2.p);
            e.pool.recycle(h2);
        } else {
            out = c2.fwd_gn(e, n2, h, x.p);  // conv2 + x (mod.rs:209)
        }
        e.pool.recycle(h);
        return out;
    }
};

// src/vae/mod.rs:215-270. q, k and v come out of one GEMM over the
// concatenated weights ([3c][c], row blocks q | k | v).
struct MidAttention {
    int c = 0;
    GNv norm;
    void *wqkv = nullptr;
    WeightType wt = kF32;
    float *bqkv = nullptr;
    Lin out;
    void load(Context &ctx, const WeightStore &W, const std::string &p, int c_) {
        c = c_;
        norm.load(W, p + ".group_norm", c);
        const char *names[3] = {".to_q", ".to_k", ".to_v"};
        DParam ws[3];
        const float *bs[3];
        for (int i = 0; i < 3; ++i) {
            ws[i] = W.get(p + names[i] + ".weight", int64_t(c) * c, true);
            bs[i] = W.get(p + names[i] + ".bias", c, false).f();
        }
        const WeightGroup grp = concat_weights(ctx, ws, 3);
        wqkv = grp.p;
        wt = grp.wt;
        mh::dev_malloc(&bqkv, 3 * size_t(c) * sizeof(float));
        for (int i = 0; i < 3; ++i)
            HIP_CHECK(hipMemcpyAsync(bqkv + i * c, bs[i], size_t(c) * sizeof(float), hipMemcpyDeviceToDevice,
                                     ctx.stream));
        out.load(W, p + ".to_out.0", c, c);
    }
    void release() {
        if (wqkv) (void)hipFree(wqkv);
        if (bqkv) (void)hipFree(bqkv);
        wqkv = nullptr;
        bqkv = nullptr;
    }
    DT fwd(Env &e, const DT &x) const {
        const int hw = x.h * x.w;
        DT t = norm.fwd(e, x);
        float *qkv = e.pool.floats(x.px() * 3 * c);
        conv1x1(e.ctx, t.p, x.px(), c, wqkv, wt, 3 * c, bqkv, nullptr, qkv);
        const float scale = 1.0f / std::sqrt(float(c));
        float *scores = e.pool.floats(int64_t(hw) * hw);
        float *vt = e.pool.floats(int64_t(c) * hw);
        DT &att = t;  // the normalised input is dead: its buffer takes the attention output
        for (int b = 0; b < x.n; ++b) {
            const float *q = qkv + int64_t(b) * hw * 3 * c;
            // scores = q . k^T, softmax per row, then P . v (v transposed to K-contiguous)
            gemm_nt(e.ctx, q, 3 * c, 0, q + c, kF32, 3 * c, 0, hw, hw, c, 1, nullptr, nullptr, scores, hw, 0);
            softmax_rows(e.ctx, scores, hw, hw, scale);
            transpose(e.ctx, q + 2 * c, 3 * c, hw, c, vt);
            gemm_nt(e.ctx, scores, hw, 0, vt, kF32, hw, 0, hw, c, hw, 1, nullptr, nullptr,
                    att.p + int64_t(b) * hw * c, c, 0);
        }
        e.pool.recycle(vt);
        e.pool.recycle(scores);
        e.pool.recycle(qkv);
        DT o = out.fwd(e, att, x.p);  // to_out(att) + x
        e.pool.recycle(t);
        return o;
    }
};

// src/vae/mod.rs:297-312
struct MidBlock {
    Resnet r0, r1;
    MidAttention attn;
    void load(Context &ctx, const WeightStore &W, const std::string &p, int c) {
        r0.load(W, p + ".resnets.0", c, c);
        attn.load(ctx, W, p + ".attentions.0", c);
        r1.load(W, p + ".resnets.1", c, c);
    }
    DT fwd(Env &e, const DT &x) const {
        DT a = r0.fwd(e, x);
        DT b = attn.fwd(e, a);
        e.pool.recycle(a);
        DT c = r1.fwd(e, b);
        e.pool.recycle(b);
        return c;
    }
};

}  // namespace

class VaeDevice {
  public:
    // The VAE's 3x3 convs read f32 Winograd kernels built at load, so its f16-stored
    // weights are not widened: the GEMMs that read them directly are a small share.
    VaeDevice(Context &ctx, const NamedTensor *t, int count) : ctx_(ctx), pool_(ctx), W_(ctx, t, count, false) {
        const std::string e = "encoder";
        int c_prev = VCH[0];
        for (int i = 0; i < 4; ++i) {
            const int c = VCH[i];
            const std::string b = e + ".down_blocks." + std::to_string(i);
            e_res_.emplace_back();
            for (int j = 0; j < LAYERS; ++j) {
                e_res_.back().emplace_back();
                e_res_.back().back().load(W_, b + ".resnets." + std::to_string(j), j == 0 ? c_prev : c, c);
            }
            if (i + 1 < 4) {
                // Downsample2D(padding=0) = pad (0, 1, 0, 1) then stride 2 (encoder.rs:7-8, 57)
                const int pad[4] = {0, 0, 1, 1};
                e_down_.emplace_back();
                e_down_.back().load(W_, b + ".downsamplers.0.conv", c, c, 2, pad);
            }
            c_prev = c;
        }
        e_in_.load(W_, e + ".conv_in", IMAGE_C, VCH[0]);
        e_mid_.load(ctx_, W_, e + ".mid_block", VCH[3]);
        e_norm_.load(W_, e + ".conv_norm_out", VCH[3]);
        e_out_.load(W_, e + ".conv_out", VCH[3], 2 * LATENT_C);
        quant_.load(W_, "quant_conv", 2 * LATENT_C, 2 * LATENT_C);

        const std::string d = "decoder";
        c_prev = VCH[3];
        for (int i = 0; i < 4; ++i) {
            const int c = VCH[3 - i];
            const std::string b = d + ".up_blocks." + std::to_string(i);
            d_res_.emplace_back();
            for (int j = 0; j <= LAYERS; ++j) {
                d_res_.back().emplace_back();
                d_res_.back().back().load(W_, b + ".resnets." + std::to_string(j), j == 0 ? c_prev : c, c);
            }
            if (i + 1 < 4) {
                d_up_.emplace_back();
                d_up_.back().load(W_, b + ".upsamplers.0.conv", c, c, 1, nullptr, true);
            }
            c_prev = c;
        }
        post_quant_.load(W_, "post_quant_conv", LATENT_C, LATENT_C);
        d_in_.load(W_, d + ".conv_in", LATENT_C, VCH[3]);
        d_mid_.load(ctx_, W_, d + ".mid_block", VCH[3]);
        d_norm_.load(W_, d + ".conv_norm_out", VCH[0]);
        d_out_.load(W_, d + ".conv_out", VCH[0], IMAGE_C);
        HIP_CHECK(hipStreamSynchronize(ctx_.stream));
    }

    ~VaeDevice() {
        (void)hipStreamSynchronize(ctx_.stream);
        e_mid_.attn.release();
        d_mid_.attn.release();
    }

    // src/vae/encoder.rs:77-118
    void encode(const float *images, int nb, int h, int w, const float *noise, float *z, TraceFn trace, void *user) {
        // f32 arithmetic whatever the context's precision: the SDXL VAE's
        // activations overflow f16 (src/vae/mod.rs:2-3).
        PrecisionScope exact(ctx_, Precision::Exact);
        if (nb <= 0 || h <= 0 || w <= 0 || h % 8 || w % 8) fail(kInvalidArgument, "image size must be a multiple of 8");
        Env e{ctx_, pool_};
        auto tr = [&](const std::string &name, const DT &t) {
            if (!trace) return;
            const int64_t item = int64_t(t.h) * t.w * t.c;
            for (int b = 0; b < t.n; ++b)
                trace(user, ("vae.encoder.item" + std::to_string(b) + name).c_str(), t.p + b * item, 1, t.h, t.w,
                      t.c);
        };
        const DT x{const_cast<float *>(images), nb, h, w, IMAGE_C};
        DT cur = e_in_.fwd(e, x);
        tr(".conv_in", cur);
        for (int i = 0; i < 4; ++i) {
            for (const Resnet &r : e_res_[size_t(i)]) {
                DT t = r.fwd(e, cur);
                pool_.recycle(cur);
                cur = t;
            }
            if (i + 1 < 4) {
                DT t = e_down_[size_t(i)].fwd(e, cur);
                pool_.recycle(cur);
                cur = t;
            }
            tr(".down." + std::to_string(i), cur);
        }
        DT m = e_mid_.fwd(e, cur);
        pool_.recycle(cur);
        tr(".mid", m);
        DT o = e_out_.fwd_gn(e, e_norm_, m);
        pool_.recycle(m);
        DT moments = quant_.fwd(e, o);
        pool_.recycle(o);
        tr(".moments", moments);
        vae_sample(ctx_, moments.p, noise, moments.px(), z);
        pool_.recycle(moments);
    }

    // src/vae/decoder.rs:74-99
    void decode(const float *latents, int h, int w, float *out, TraceFn trace, void *user) {
        // f32 arithmetic whatever the context's precision: the SDXL VAE's
        // activations overflow f16 (src/vae/mod.rs:2-3).
        PrecisionScope exact(ctx_, Precision::Exact);
        if (h <= 0 || w <= 0) fail(kInvalidArgument, "empty latent");
        Env e{ctx_, pool_};
        auto tr = [&](const char *name, const DT &t) {
            if (trace) trace(user, name, t.p, t.n, t.h, t.w, t.c);
        };
        DT z = pool_.tensor(1, h, w, LATENT_C);
        vae_rescale(ctx_, latents, z.numel(), 0, z.p);
        DT pq = post_quant_.fwd(e, z);
        pool_.recycle(z);
        DT cur = d_in_.fwd(e, pq);
        pool_.recycle(pq);
        tr("vae.decoder.conv_in", cur);
        DT m = d_mid_.fwd(e, cur);
        pool_.recycle(cur);
        cur = m;
        tr("vae.decoder.mid", cur);
        for (int i = 0; i < 4; ++i) {
            for (const Resnet &r : d_res_[size_t(i)]) {
                DT t = r.fwd(e, cur);
                pool_.recycle(cur);
                cur = t;
            }
            if (i + 1 < 4) {
                DT t = d_up_[size_t(i)].fwd(e, cur);
                pool_.recycle(cur);
                cur = t;
            }
            tr(("vae.decoder.up." + std::to_string(i)).c_str(), cur);
        }
        DT o = d_out_.fwd_gn(e, d_norm_, cur, nullptr, out);
        pool_.recycle(cur);
        vae_rescale(ctx_, o.p, o.numel(), 1, out);
    }

    size_t weight_bytes() const { return W_.bytes(); }
    size_t pool_bytes() const { return pool_.bytes_held(); }
    void release_scratch() { pool_.release_below(INT64_MAX); }

  private:
    Context &ctx_;
    Pool pool_;
    WeightStore W_;
    Conv3v e_in_, e_out_, d_in_, d_out_;
    std::vector<std::vector<Resnet>> e_res_, d_res_;
    std::vector<Conv3v> e_down_, d_up_;
    MidBlock e_mid_, d_mid_;
    GNv e_norm_, d_norm_;
    Lin quant_, post_quant_;
};

Vae::Vae(Context &ctx, const NamedTensor *t, int count) : d_(new VaeDevice(ctx, t, count)) {}
Vae::~Vae() = default;
void Vae::encode(const float *images_dev, int b, int h, int w, const float *noise_dev, float *z_dev, TraceFn trace,
                 void *user) {
    d_->encode(images_dev, b, h, w, noise_dev, z_dev, trace, user);
}
void Vae::decode(const float *latents_dev, int h, int w, float *out_dev, TraceFn trace, void *user) {
    d_->decode(latents_dev, h, w, out_dev, trace, user);
}
size_t Vae::weight_bytes() const { return d_->weight_bytes(); }
size_t Vae::pool_bytes() const { return d_->pool_bytes(); }
void Vae::release_scratch() { d_->release_scratch(); }

}  // namespace mh
