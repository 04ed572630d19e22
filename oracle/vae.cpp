// Oracle restatement of the moebius-cpu VAE (src/vae/{mod,encoder,decoder}.rs,
// src/config.rs) over the oracle engine. Test infrastructure only: see oracle.h.
//
// Weights are the converter's tensors (diffusers AutoencoderKL names at the
// file root; 3x3 [o, 3, 3, i], 1x1 and attention linears [o, i]), handed in as
// named f32 arrays the caller keeps alive.
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "model.hpp"
#include "oracle.h"
#include "oracle_vae.h"

namespace {

using namespace orc_model;

// src/config.rs:50-58
constexpr int VCH[4] = {128, 256, 512, 512};
constexpr float VAE_EPS = 1e-6f;
constexpr float SCALING = 0.13025f;
constexpr int LATENT_C = 4;
constexpr int IMAGE_C = 3;
// src/vae/encoder.rs:23-26, decoder.rs:24
constexpr int LAYERS = 2;
constexpr float LOGVAR_LO = -30.0f, LOGVAR_HI = 20.0f;
// src/vae/mod.rs:223-225, 271-273
constexpr int64_t BAND = 512;
constexpr float FLUSH = -40.0f;

struct Conv3 {  // Conv3x3 (src/engine/conv.rs:60-102)
    int ci = 0, co = 0, stride = 1, up = 0;
    int pad[4] = {1, 1, 1, 1};
    const float *w = nullptr, *b = nullptr;
    void load(const Weights &W, const std::string &p, int ci_, int co_, int stride_ = 1, const int *pad_ = nullptr,
              bool up_ = false) {
        ci = ci_, co = co_, stride = stride_, up = up_ ? 1 : 0;
        if (pad_) std::memcpy(pad, pad_, sizeof(pad));
        w = W.get(p + ".weight", int64_t(co) * 9 * ci);
        b = W.get(p + ".bias", co);
    }
    // out = conv(x'), x' = SiLU(x . scale + shift) when a prologue is given.
    void fwd(const T4 &x, T4 &out, const Vec *sc = nullptr, const Vec *sh = nullptr) const {
        int64_t ho, wo;
        orc_conv3x3_output_hw(x.h, x.w, stride, pad, up, &ho, &wo);
        out.set(x.n, ho, wo, co);
        orc_conv3x3_forward(x.p(), x.n, x.h, x.w, x.c, w, co, b, stride, pad, up, sc ? sc->data() : nullptr,
                            sh ? sh->data() : nullptr, sc ? 1 : 0, out.p());
    }
};

// src/vae/mod.rs:174-211
struct Resnet {
    int ci = 0, co = 0;
    GN n1, n2;
    Conv3 c1, c2;
    bool has_sc = false;
    Lin sc;
    void load(const Weights &W, const std::string &p, int ci_, int co_) {
        ci = ci_, co = co_;
        n1.load(W, p + ".norm1", ci, VAE_EPS);
        c1.load(W, p + ".conv1", ci, co);
        n2.load(W, p + ".norm2", co, VAE_EPS);
        c2.load(W, p + ".conv2", co, co);
        has_sc = ci != co;
        if (has_sc) sc.load(W, p + ".conv_shortcut", ci, co, true);
    }
    void fwd(const T4 &x, T4 &out) const {
        Vec s, t;
        n1.affine(x, s, t);
        T4 h;
        c1.fwd(x, h, &s, &t);
        n2.affine(h, s, t);
        c2.fwd(h, out, &s, &t);
        if (has_sc) {
            T4 r;
            sc.fwd(x, r, &out);  // shortcut(x) with residual = out
            out = std::move(r);
        } else {
            orc_add_inplace(out.p(), x.p(), int64_t(out.d.size()));
        }
    }
};

// src/vae/mod.rs:215-270
struct MidAttention {
    int c = 0;
    GN norm;
    Lin q, k, v, o;
    void load(const Weights &W, const std::string &p, int c_) {
        c = c_;
        norm.load(W, p + ".group_norm", c, VAE_EPS);
        q.load(W, p + ".to_q", c, c, true);
        k.load(W, p + ".to_k", c, c, true);
        v.load(W, p + ".to_v", c, c, true);
        o.load(W, p + ".to_out.0", c, c, true);
    }
    void fwd(const T4 &x, T4 &out) const {
        T4 t, qt, kt, vt;
        norm.fwd(x, nullptr, false, t);
        q.fwd(t, qt);
        k.fwd(t, kt);
        v.fwd(t, vt);
        const int64_t hw = x.h * x.w;
        const float scale = 1.0f / std::sqrt(float(c));
        Vec scores(size_t(std::min(BAND, hw) * hw));
        T4 &att = t;  // the normalised input is dead: its buffer takes the attention output
        for (int64_t b = 0; b < x.n; ++b) {
            const float *qi = qt.p() + b * hw * c, *ki = kt.p() + b * hw * c, *vi = vt.p() + b * hw * c;
            for (int64_t start = 0; start < hw; start += BAND) {
                const int64_t rows = std::min(BAND, hw - start);
                // scores = q_band . k^T, then softmax per row, then band . v
                orc_matmul(scores.data(), qi + start * c, c, 1, ki, 1, c, rows, c, hw, 0);
                orc_softmax_rows(scores.data(), rows, hw, scale);
                orc_matmul(att.p() + (b * hw + start) * c, scores.data(), hw, 1, vi, c, 1, rows, hw, c, 0);
            }
        }
        o.fwd(att, out, &x);
    }
};

// src/vae/mod.rs:297-312
struct MidBlock {
    Resnet r0, r1;
    MidAttention attn;
    void load(const Weights &W, const std::string &p, int c) {
        r0.load(W, p + ".resnets.0", c, c);
        attn.load(W, p + ".attentions.0", c);
        r1.load(W, p + ".resnets.1", c, c);
    }
    void fwd(T4 &cur) const {
        T4 t;
        r0.fwd(cur, t);
        attn.fwd(t, cur);
        r1.fwd(cur, t);
        cur = std::move(t);
    }
};

void trace_out(OrcTraceFn trace, void *user, const std::string &name, const T4 &t) {
    if (trace) trace(user, name.c_str(), t.p(), t.n, t.h, t.w, t.c);
}

struct Vae {
    // encoder (src/vae/encoder.rs:35-73)
    Conv3 e_in;
    std::vector<std::vector<Resnet>> e_res;
    std::vector<Conv3> e_down;
    MidBlock e_mid;
    GN e_norm;
    Conv3 e_out;
    Lin quant;
    // decoder (src/vae/decoder.rs:32-70)
    Lin post_quant;
    Conv3 d_in;
    MidBlock d_mid;
    std::vector<std::vector<Resnet>> d_res;
    std::vector<Conv3> d_up;
    GN d_norm;
    Conv3 d_out;

    void load(const Weights &W) {
        const std::string e = "encoder";
        int c_prev = VCH[0];
        for (int i = 0; i < 4; ++i) {
            const int c = VCH[i];
            const std::string b = e + ".down_blocks." + std::to_string(i);
            e_res.emplace_back();
            for (int j = 0; j < LAYERS; ++j) {
                e_res.back().emplace_back();
                e_res.back().back().load(W, b + ".resnets." + std::to_string(j), j == 0 ? c_prev : c, c);
            }
            if (i + 1 < 4) {
                // Downsample2D(padding=0): pad (0, 1, 0, 1) then stride 2 (encoder.rs:7-8)
                const int pad[4] = {0, 0, 1, 1};
                e_down.emplace_back();
                e_down.back().load(W, b + ".downsamplers.0.conv", c, c, 2, pad);
            }
            c_prev = c;
        }
        e_in.load(W, e + ".conv_in", IMAGE_C, VCH[0]);
        e_mid.load(W, e + ".mid_block", VCH[3]);
        e_norm.load(W, e + ".conv_norm_out", VCH[3], VAE_EPS);
        e_out.load(W, e + ".conv_out", VCH[3], 2 * LATENT_C);
        quant.load(W, "quant_conv", 2 * LATENT_C, 2 * LATENT_C, true);

        const std::string d = "decoder";
        c_prev = VCH[3];
        for (int i = 0; i < 4; ++i) {
            const int c = VCH[3 - i];
            const std::string b = d + ".up_blocks." + std::to_string(i);
            d_res.emplace_back();
            for (int j = 0; j <= LAYERS; ++j) {
                d_res.back().emplace_back();
                d_res.back().back().load(W, b + ".resnets." + std::to_string(j), j == 0 ? c_prev : c, c);
            }
            if (i + 1 < 4) {
                d_up.emplace_back();
                d_up.back().load(W, b + ".upsamplers.0.conv", c, c, 1, nullptr, true);
            }
            c_prev = c;
        }
        post_quant.load(W, "post_quant_conv", LATENT_C, LATENT_C, true);
        d_in.load(W, d + ".conv_in", LATENT_C, VCH[3]);
        d_mid.load(W, d + ".mid_block", VCH[3]);
        d_norm.load(W, d + ".conv_norm_out", VCH[0], VAE_EPS);
        d_out.load(W, d + ".conv_out", VCH[0], IMAGE_C);
    }

    // src/vae/encoder.rs:77-118, items one after the other.
    void encode(const float *images, int64_t nb, int64_t h, int64_t w, const float *noise, float *z, OrcTraceFn trace,
                void *user) const {
        if (h % 8 || w % 8 || h <= 0 || w <= 0) throw std::runtime_error("image size must be a multiple of 8");
        const int64_t zl = (h / 8) * (w / 8) * LATENT_C;
        for (int64_t b = 0; b < nb; ++b) {
            const std::string pre = "vae.encoder.item" + std::to_string(b);
            T4 x, cur, t;
            x.set(1, h, w, IMAGE_C);
            std::memcpy(x.p(), images + b * h * w * IMAGE_C, x.d.size() * sizeof(float));
            e_in.fwd(x, cur);
            trace_out(trace, user, pre + ".conv_in", cur);
            for (int i = 0; i < 4; ++i) {
                for (const Resnet &r : e_res[size_t(i)]) {
                    r.fwd(cur, t);
                    std::swap(cur, t);
                }
                if (i + 1 < 4) {
                    e_down[size_t(i)].fwd(cur, t);
                    std::swap(cur, t);
                }
                trace_out(trace, user, pre + ".down." + std::to_string(i), cur);
            }
            e_mid.fwd(cur);
            trace_out(trace, user, pre + ".mid", cur);
            Vec s, sh;
            e_norm.affine(cur, s, sh);
            e_out.fwd(cur, t, &s, &sh);
            T4 moments;
            quant.fwd(t, moments);
            trace_out(trace, user, pre + ".moments", moments);
            orc_vae_sample(moments.p(), noise + b * zl, moments.px(), z + b * zl);
        }
    }

    // src/vae/decoder.rs:74-99
    void decode(const float *latents, int64_t h, int64_t w, float *out, OrcTraceFn trace, void *user) const {
        T4 zt, cur, t;
        zt.set(1, h, w, LATENT_C);
        for (size_t i = 0; i < zt.d.size(); ++i) zt.d[i] = latents[i] / SCALING;
        post_quant.fwd(zt, t);
        d_in.fwd(t, cur);
        trace_out(trace, user, "vae.decoder.conv_in", cur);
        d_mid.fwd(cur);
        trace_out(trace, user, "vae.decoder.mid", cur);
        for (int i = 0; i < 4; ++i) {
            for (const Resnet &r : d_res[size_t(i)]) {
                r.fwd(cur, t);
                std::swap(cur, t);
            }
            if (i + 1 < 4) {
                d_up[size_t(i)].fwd(cur, t);
                std::swap(cur, t);
            }
            trace_out(trace, user, "vae.decoder.up." + std::to_string(i), cur);
        }
        Vec s, sh;
        d_norm.affine(cur, s, sh);
        d_out.fwd(cur, t, &s, &sh);
        for (size_t i = 0; i < t.d.size(); ++i) out[i] = (t.d[i] + 1.0f) * 0.5f;
    }
};

Weights table(const OrcNamed *tensors, int count) {
    Weights W;
    for (int i = 0; i < count; ++i) W.m[tensors[i].name] = {tensors[i].data, tensors[i].numel};
    return W;
}

void set_err(char *err, int err_len, const char *what) {
    if (err && err_len > 0) {
        std::strncpy(err, what, size_t(err_len - 1));
        err[err_len - 1] = 0;
    }
}

}  // namespace

// src/vae/mod.rs:275-294: max, then v = exp((v - max) * scale) or 0 below the
// flush threshold, summed in row order in f32, then scaled by (f32)(1 / sum).
extern "C" void orc_softmax_rows(float *rows, int64_t nrows, int64_t n, float scale) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nrows; ++r) {
        float *row = rows + r * n;
        float mx = -INFINITY;
        for (int64_t j = 0; j < n; ++j) mx = std::fmax(mx, row[j]);
        float sum = 0.0f;
        for (int64_t j = 0; j < n; ++j) {
            const float a = (row[j] - mx) * scale;
            row[j] = a < FLUSH ? 0.0f : orc_exp(a);
            sum += row[j];
        }
        const float inv = 1.0f / sum;
        for (int64_t j = 0; j < n; ++j) row[j] *= inv;
    }
}

// src/vae/encoder.rs:121-133: z = fma(exp(0.5 * clamp(logvar)), noise, mean) * 0.13025
extern "C" void orc_vae_sample(const float *moments, const float *noise, int64_t pixels, float *z) {
    for (int64_t p = 0; p < pixels; ++p) {
        const float *m = moments + p * 2 * LATENT_C;
        for (int i = 0; i < LATENT_C; ++i) {
            // Rust's f32::clamp: NaN stays NaN
            float lv = m[LATENT_C + i];
            lv = lv < LOGVAR_LO ? LOGVAR_LO : (lv > LOGVAR_HI ? LOGVAR_HI : lv);
            z[p * LATENT_C + i] = std::fma(orc_exp(0.5f * lv), noise[p * LATENT_C + i], m[i]) * SCALING;
        }
    }
}

extern "C" void *orc_vae_create(const OrcNamed *tensors, int count, char *err, int err_len) {
    try {
        auto v = std::make_unique<Vae>();
        v->load(table(tensors, count));
        return v.release();
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return nullptr;
    }
}

extern "C" void orc_vae_destroy(void *vae) { delete static_cast<Vae *>(vae); }

extern "C" int orc_vae_encode(void *vae, const float *images, int64_t b, int64_t h, int64_t w, const float *noise,
                              float *z, OrcTraceFn trace, void *user, char *err, int err_len) {
    try {
        static_cast<Vae *>(vae)->encode(images, b, h, w, noise, z, trace, user);
        return 0;
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return 1;
    }
}

extern "C" int orc_vae_decode(void *vae, const float *latents, int64_t h, int64_t w, float *out, OrcTraceFn trace,
                              void *user, char *err, int err_len) {
    try {
        static_cast<Vae *>(vae)->decode(latents, h, w, out, trace, user);
        return 0;
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return 1;
    }
}

extern "C" int orc_vae_attention(const OrcNamed *tensors, int count, const char *prefix, const float *x, int64_t n,
                                 int64_t h, int64_t w, int64_t c, float *out, char *err, int err_len) {
    try {
        const Weights W = table(tensors, count);
        MidAttention a;
        a.load(W, prefix, int(c));
        T4 xt, o;
        xt.set(n, h, w, c);
        std::memcpy(xt.p(), x, xt.d.size() * sizeof(float));
        a.fwd(xt, o);
        std::memcpy(out, o.p(), o.d.size() * sizeof(float));
        return 0;
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return 1;
    }
}

extern "C" int orc_vae_resnet(const OrcNamed *tensors, int count, const char *prefix, const float *x, int64_t n,
                              int64_t h, int64_t w, int64_t c_in, int64_t c_out, float *out, char *err, int err_len) {
    try {
        const Weights W = table(tensors, count);
        Resnet r;
        r.load(W, prefix, int(c_in), int(c_out));
        T4 xt, o;
        xt.set(n, h, w, c_in);
        std::memcpy(xt.p(), x, xt.d.size() * sizeof(float));
        r.fwd(xt, o);
        std::memcpy(out, o.p(), o.d.size() * sizeof(float));
        return 0;
    } catch (const std::exception &e) {
        set_err(err, err_len, e.what());
        return 1;
    }
}
