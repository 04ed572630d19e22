// Oracle restatement of the moebius-cpu UNet (src/unet/{mod,blocks,
// transformer,lambda,embed,load}.rs, src/config.rs) over the oracle engine.
// Test infrastructure only: see oracle.h.
//
// Weights are the converter's `moebius-cpu/1` tensors (names and layouts of
// src/unet/load.rs and tools/convert_weights.py:13-33), handed in as a table of
// named f32 arrays the caller keeps alive (f16-stored GEMM weights arrive
// widened, which is exact: src/engine/param.rs:45-59).
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "model.hpp"
#include "oracle.h"
#include "oracle_unet.h"

namespace {

using namespace orc_model;

// src/config.rs
constexpr int CH[3] = {320, 640, 1280};
constexpr int LAYERS = 2;
constexpr int HEADS = 8;
constexpr int TIME_PROJ = 320;
constexpr int TIME_EMBED = 1280;
constexpr int TOKENS = 10;
constexpr int EHS = 3072;
constexpr int XDIM = 768;
constexpr float RESNET_EPS = 1e-5f;
constexpr float TGN_EPS = 1e-6f;
constexpr float LN_EPS = 1e-5f;
// src/unet/lambda.rs:56-71
constexpr int WIN = 15, TAPS = WIN * WIN, PAD = WIN / 2, TAPS_B = TAPS + 1;
constexpr int SOFTMAX_CHUNK = 256;

// FLOPs of the step as the upstream model executes it, tallied per layer from
// the shapes each call runs at, in the categories of the reference's
// meta-device count (tools/count_flops.py: conv kinds by kernel, everything
// else FlopCounterMode counts as matrix products): 1x1 convs, dense 3x3,
// stride-2 3x3, depthwise, the self-lambda's position Conv3d, and the matrix
// products (linears, lambda einsums). Multiply-add = 2. The oracle runs the
// folded lambda (lambda.rs:7-24); its layers tally the unfolded products they
// stand for (pos_conv over [b, k, v, N] x 225 taps, Yp = Q.lambda_p), which is
// what the 632 GFLOP of docs/PLAN.md:56 counts.
enum FlopKind { kF1x1 = 0, kFDense3, kFStride2, kFDepthwise, kFPosConv, kFMatmul, kFKinds };
double g_flops[kFKinds] = {};
void tally(FlopKind k, double f) { g_flops[k] += f; }

struct LNp {  // LayerNormParams (src/unet/transformer.rs:33-47)
    const float *g = nullptr, *b = nullptr;
    int c = 0;
    void load(const Weights &W, const std::string &p, int c_) {
        c = c_;
        g = W.get(p + ".weight", c);
        b = W.get(p + ".bias", c);
    }
    void fwd(const T4 &x, T4 &out) const {
        out.set(x.n, x.h, x.w, x.c);
        orc_layer_norm(x.p(), x.px(), c, g, b, LN_EPS, out.p());
    }
};

// src/unet/blocks.rs:31-54
struct DwConv2d {
    int ci = 0, co = 0;
    const float *dw = nullptr, *dwb = nullptr;
    Lin pw;
    void load(const Weights &W, const std::string &p, int ci_, int co_) {
        ci = ci_, co = co_;
        dw = W.get(p + ".conv_dw.weight", int64_t(9) * ci);
        dwb = W.get(p + ".conv_dw.bias", ci);
        pw.load(W, p + ".conv_pw", ci, co, true);
    }
    void fwd(const T4 &x, T4 &out) const {
        T4 mid;
        mid.set(x.n, x.h, x.w, x.c);
        orc_depthwise3x3(x.p(), x.n, x.h, x.w, x.c, dw, dwb, 1, mid.p());
        pw.fwd(mid, out, ci == co ? &x : nullptr);
        tally(kFDepthwise, 18.0 * double(x.px()) * ci);
        tally(kF1x1, 2.0 * double(x.px()) * ci * co);
    }
};

// src/unet/blocks.rs:56-113
struct DwResnet {
    int ci = 0, co = 0;
    GN norm1, norm2;
    DwConv2d conv1, conv2;
    Lin temb_proj, shortcut;
    bool has_shortcut = false;
    void load(const Weights &W, const std::string &p, int ci_, int co_) {
        ci = ci_, co = co_;
        norm1.load(W, p + ".norm1", ci, RESNET_EPS);
        conv1.load(W, p + ".conv1", ci, co);
        temb_proj.load(W, p + ".time_emb_proj", TIME_EMBED, co, true);
        norm2.load(W, p + ".norm2", co, RESNET_EPS);
        conv2.load(W, p + ".conv2", co, co);
        has_shortcut = ci != co;
        if (has_shortcut) shortcut.load(W, p + ".conv_shortcut", ci, co, true);
    }
    // temb: [n, 1280] raw embedding.
    void fwd(const T4 &x, const Vec &temb, T4 &out) const {
        T4 a, b;
        norm1.fwd(x, nullptr, true, a);
        conv1.fwd(a, b);
        Vec t = temb;
        orc_silu_inplace(t.data(), int64_t(t.size()));
        Vec tp(size_t(x.n * co));
        temb_proj.fwd(t.data(), x.n, tp.data());
        tally(kFMatmul, 2.0 * double(x.n) * TIME_EMBED * co);
        norm2.fwd(b, tp.data(), true, a);
        conv2.fwd(a, out);
        if (has_shortcut) {
            shortcut.fwd(x, b);
            tally(kF1x1, 2.0 * double(x.px()) * ci * co);
            orc_add_inplace(out.p(), b.p(), int64_t(out.d.size()));
        } else {
            orc_add_inplace(out.p(), x.p(), int64_t(out.d.size()));
        }
    }
};

// src/unet/lambda.rs:322-359
Vec softmax_lambda(float *keys, const float *v, int64_t rows, int64_t k, int64_t vd) {
    const int64_t chunks = (rows + SOFTMAX_CHUNK - 1) / SOFTMAX_CHUNK;
    Vec mx(size_t(k), -INFINITY);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < k; ++j) mx[j] = std::max(mx[j], keys[r * k + j]);
    std::vector<double> sum(size_t(k), 0.0);
    for (int64_t ch = 0; ch < chunks; ++ch) {
        Vec s(size_t(k), 0.0f);
        for (int64_t r = ch * SOFTMAX_CHUNK; r < std::min(rows, (ch + 1) * SOFTMAX_CHUNK); ++r) {
            for (int64_t j = 0; j < k; ++j) {
                float &e = keys[r * k + j];
                e = orc_exp(e - mx[j]);
                s[j] += e;
            }
        }
        for (int64_t j = 0; j < k; ++j) sum[j] += double(s[j]);
    }
    Vec lambda(size_t(k * vd), 0.0f);
    // keys^T: element (kk, r) at keys[r * k + kk].
    orc_matmul(lambda.data(), keys, 1, k, v, vd, 1, k, rows, vd, 0);
    for (int64_t j = 0; j < k; ++j) {
        const float inv = float(1.0 / sum[j]);
        for (int64_t i = 0; i < vd; ++i) lambda[j * vd + i] *= inv;
    }
    return lambda;
}

// src/unet/lambda.rs:154-185: adds the 15x15 position filter of V to o.
void tap_filter(const float *a, const float *v, float *o, int64_t first, int64_t count, int64_t hh, int64_t ww,
                int64_t vd) {
    const int64_t c = HEADS * vd;
    for (int64_t i = 0; i < count; ++i) {
        const int64_t y = (first + i) / ww, x = (first + i) % ww;
        const float *ai = a + i * HEADS * TAPS_B;
        float *oi = o + i * c;
        for (int h = 0; h < HEADS; ++h) {
            const float bias = ai[h * TAPS_B + TAPS];
            for (int64_t j = 0; j < vd; ++j) oi[h * vd + j] += bias;
        }
        const int64_t kx0 = std::max<int64_t>(PAD - x, 0);
        const int64_t kx1 = std::min<int64_t>(WIN, ww + PAD - x);
        for (int ky = 0; ky < WIN; ++ky) {
            const int64_t iy = y + ky - PAD;
            if (iy < 0 || iy >= hh) continue;
            for (int64_t kx = kx0; kx < kx1; ++kx) {
                const float *vr = v + (iy * ww + x + kx - PAD) * vd;
                const int64_t d = ky * WIN + kx;
                for (int h = 0; h < HEADS; ++h) {
                    const float coef = ai[h * TAPS_B + d];
                    float *oh = oi + h * vd;
                    for (int64_t j = 0; j < vd; ++j) oh[j] = std::fma(coef, vr[j], oh[j]);
                }
            }
        }
    }
}

// src/unet/lambda.rs:73-152
struct SelfLambda {
    int c = 0, k = 0;
    Lin to_q, to_k, to_v;
    Vec w_aug;  // [k, 226]
    void load(const Weights &W, const std::string &p, int c_) {
        c = c_, k = c / HEADS;
        const float *w = W.get(p + ".pos_conv.weight", int64_t(k) * TAPS);
        const float *b = W.get(p + ".pos_conv.bias", k);
        w_aug.assign(size_t(k * TAPS_B), 0.0f);
        for (int kk = 0; kk < k; ++kk) {
            std::memcpy(w_aug.data() + kk * TAPS_B, w + kk * TAPS, TAPS * sizeof(float));
            w_aug[size_t(kk * TAPS_B + TAPS)] = b[kk];
        }
        to_q.load(W, p + ".to_q", c, c, true);
        to_k.load(W, p + ".to_k", c, k, false);
        to_v.load(W, p + ".to_v", c, k, true);
    }
    void fwd(const T4 &x, T4 &out) const {
        const int64_t hh = x.h, ww = x.w, hw = hh * ww;
        T4 q, kt, vt;
        to_q.fwd(x, q);
        to_k.fwd(x, kt);
        to_v.fwd(x, vt);
        {
            const double bn = double(x.n) * hw, kv = double(k) * k;
            tally(kF1x1, 2.0 * double(x.px()) * c * (c + 2 * k));
            tally(kFPosConv, 2.0 * bn * kv * TAPS);                   // lambda_p = Conv3d(V), 15x15
            tally(kFMatmul, 2.0 * bn * kv * (1 + 2 * HEADS));         // lambda_c, Yc, Yp
        }
        out.set(x.n, hh, ww, c);
        const int64_t band_rows = 16;
        Vec a(size_t(std::min<int64_t>(band_rows, hh) * ww * HEADS * TAPS_B));
        for (int64_t b = 0; b < x.n; ++b) {
            const float *qi = q.p() + b * hw * c;
            const float *vi = vt.p() + b * hw * k;
            float *oi = out.p() + b * hw * c;
            Vec lc = softmax_lambda(kt.p() + b * hw * k, vi, hw, k, k);
            orc_matmul(oi, qi, k, 1, lc.data(), k, 1, hw * HEADS, k, k, 0);
            for (int64_t y0 = 0; y0 < hh; y0 += band_rows) {
                const int64_t rows = std::min(band_rows, hh - y0), px = rows * ww;
                orc_matmul(a.data(), qi + y0 * ww * c, k, 1, w_aug.data(), TAPS_B, 1, px * HEADS, k, TAPS_B, 0);
                tap_filter(a.data(), vi, oi + y0 * ww * c, y0 * ww, px, hh, ww, k);
            }
        }
    }
};

// src/unet/lambda.rs:297-309: 8 fused-multiply-add lanes, then lanes summed in order.
float dot8(const float *a, const float *b, int64_t k) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int64_t full = k / 8 * 8;
    float tail = 0.0f;
    for (int64_t i = full; i < k; ++i) tail += a[i] * b[i];
    for (int64_t i = 0; i < full; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = std::fma(a[i + l], b[i + l], acc[l]);
    float s = 0.0f;
    for (int l = 0; l < 8; ++l) s += acc[l];
    return s + tail;
}

// src/unet/lambda.rs:187-274
struct CrossLambda {
    int c = 0, k = 0;
    int64_t n = 0;
    Lin to_q;
    const float *e = nullptr;  // [n, 10, k]
    Vec lambda_c[2], v[2];     // [k, k], [10, k]
    void load(const Weights &W, const std::string &p, int c_, const Vec ehs[2]) {
        c = c_, k = c / HEADS;
        const int64_t side = 64 * 320 / c;
        n = side * side;
        const float *wk = W.get(p + ".to_k.weight", int64_t(k) * XDIM);
        const float *wv = W.get(p + ".to_v.weight", int64_t(k) * XDIM);
        const float *bv = W.get(p + ".to_v.bias", k);
        for (int br = 0; br < 2; ++br) {
            Vec keys(size_t(TOKENS * k)), vv(size_t(TOKENS * k));
            orc_matmul(keys.data(), ehs[br].data(), XDIM, 1, wk, 1, XDIM, TOKENS, XDIM, k, 0);
            orc_matmul(vv.data(), ehs[br].data(), XDIM, 1, wv, 1, XDIM, TOKENS, XDIM, k, 0);
            for (int t = 0; t < TOKENS; ++t)
                for (int j = 0; j < k; ++j) vv[size_t(t * k + j)] += bv[j];
            lambda_c[br] = softmax_lambda(keys.data(), vv.data(), TOKENS, k, k);
            v[br] = vv;
        }
        to_q.load(W, p + ".to_q", c, c, true);
        e = W.get(p + ".rel_pos_emb", n * TOKENS * k);
    }
    void fwd(const T4 &x, const std::vector<int> &branches, T4 &out) const {
        const int64_t hw = x.h * x.w;
        if (hw != n) throw std::runtime_error("CrossLambda input size does not match the position table");
        T4 q;
        to_q.fwd(x, q);
        {
            const double bn = double(x.n) * hw, kv = double(k) * k;
            tally(kF1x1, 2.0 * double(x.px()) * c * c);
            // per step upstream: to_k / to_v of the text states, lambda_c = K.V^T,
            // Yc, lambda_p = E.V over the m = 10 tokens, Yp
            tally(kFMatmul, 2.0 * 2.0 * double(x.n) * TOKENS * XDIM * k + 2.0 * double(x.n) * kv * TOKENS +
                                2.0 * bn * kv * HEADS * 2 + 2.0 * bn * TOKENS * kv);
        }
        out.set(x.n, x.h, x.w, c);
        for (int64_t b = 0; b < x.n; ++b) {
            const int br = branches[size_t(b)];
            const float *qi = q.p() + b * hw * c;
            float *oi = out.p() + b * hw * c;
            orc_matmul(oi, qi, k, 1, lambda_c[br].data(), k, 1, hw * HEADS, k, k, 0);
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < hw; ++i) {
                const float *ei = e + i * TOKENS * k;
                for (int h = 0; h < HEADS; ++h) {
                    const float *qh = qi + i * c + h * k;
                    float *oh = oi + i * c + h * k;
                    for (int m = 0; m < TOKENS; ++m) {
                        const float bb = dot8(qh, ei + m * k, k);
                        const float *vm = v[br].data() + m * k;
                        for (int j = 0; j < k; ++j) oh[j] = std::fma(bb, vm[j], oh[j]);
                    }
                }
            }
        }
    }
};

// src/unet/transformer.rs:49-130
struct MixTransformer {
    int c = 0, hidden = 0;
    GN norm;
    Lin proj_in, proj_out, inverted, point;
    LNp ln1, ln2, ln3;
    SelfLambda attn1;
    CrossLambda attn2;
    const float *dw = nullptr, *dwb = nullptr;
    void load(const Weights &W, const std::string &p, int c_, const Vec ehs[2]) {
        c = c_;
        hidden = int(float(c) * 2.5f);
        const std::string b = p + ".transformer_blocks.0";
        const std::string ff = b + ".ff";
        dw = W.get(ff + ".depth_conv.conv.weight", int64_t(9) * 2 * hidden);
        dwb = W.get(ff + ".depth_conv.conv.bias", 2 * hidden);
        norm.load(W, p + ".norm", c, TGN_EPS);
        proj_in.load(W, p + ".proj_in", c, c, true);
        ln1.load(W, b + ".norm1", c);
        attn1.load(W, b + ".attn1", c);
        ln2.load(W, b + ".norm2", c);
        attn2.load(W, b + ".attn2", c, ehs);
        ln3.load(W, b + ".norm3", c);
        inverted.load(W, ff + ".inverted_conv.conv", c, 2 * hidden, true);
        point.load(W, ff + ".point_conv.conv", hidden, c, false);
        proj_out.load(W, p + ".proj_out", c, c, true);
    }
    void fwd(const T4 &x, const std::vector<int> &branches, T4 &out) const {
        T4 t, u, h;
        tally(kF1x1, 2.0 * double(x.px()) * (2.0 * c * c + 3.0 * c * hidden));  // proj_in/out, inverted, point
        tally(kFDepthwise, 18.0 * double(x.px()) * 2 * hidden);
        norm.fwd(x, nullptr, false, t);
        proj_in.fwd(t, h);
        ln1.fwd(h, t);
        attn1.fwd(t, u);
        orc_add_inplace(h.p(), u.p(), int64_t(h.d.size()));
        ln2.fwd(h, t);
        attn2.fwd(t, branches, u);
        orc_add_inplace(h.p(), u.p(), int64_t(h.d.size()));
        ln3.fwd(h, t);
        // ffn (transformer.rs:121-129)
        T4 a, bb;
        inverted.fwd(t, a);
        orc_silu_inplace(a.p(), int64_t(a.d.size()));
        bb.set(a.n, a.h, a.w, hidden);
        orc_depthwise3x3(a.p(), a.n, a.h, a.w, a.c, dw, dwb, 2, bb.p());
        point.fwd(bb, u, &h);
        proj_out.fwd(u, out, &x);
    }
};

struct Conv3 {  // Downsample / Upsample (src/unet/blocks.rs:116-145)
    int c = 0, stride = 1, up = 0;
    const float *w = nullptr, *b = nullptr;
    void load(const Weights &W, const std::string &p, int c_, int stride_, int up_) {
        c = c_, stride = stride_, up = up_;
        w = W.get(p + ".conv.weight", int64_t(9) * c * c);
        b = W.get(p + ".conv.bias", c);
    }
    void fwd(const T4 &x, T4 &out) const {
        const int pad[4] = {1, 1, 1, 1};
        int64_t ho, wo;
        orc_conv3x3_output_hw(x.h, x.w, stride, pad, up, &ho, &wo);
        out.set(x.n, ho, wo, c);
        orc_conv3x3_forward(x.p(), x.n, x.h, x.w, x.c, w, c, b, stride, pad, up, nullptr, nullptr, 0, out.p());
        tally(stride > 1 ? kFStride2 : kFDense3, 2.0 * double(out.px()) * 9 * x.c * c);
    }
};

struct UNet {
    Lin lin1, lin2;
    DwConv2d conv_in, conv_out;
    GN norm_out;
    struct Block {
        std::vector<DwResnet> res;
        std::vector<MixTransformer> attn;
        bool has_sample = false;
        Conv3 sample;
    };
    std::vector<Block> down, up;

    void load(const Weights &W) {
        // embed::conditioning (src/unet/embed.rs:72-83): [uncond = rows 10..20, cond = rows 0..10]
        const float *table = W.get("embedding_layer.weight", int64_t(20) * EHS);
        Lin proj;
        proj.load(W, "diff_model.encoder_hid_proj", EHS, XDIM, true);
        Vec ehs[2];
        for (int br = 0; br < 2; ++br) {
            ehs[br].resize(size_t(TOKENS * XDIM));
            const int first = br == 0 ? TOKENS : 0;
            proj.fwd(table + int64_t(first) * EHS, TOKENS, ehs[br].data());
        }
        const std::string d = "diff_model";
        int c_prev = CH[0];
        for (int i = 0; i < 3; ++i) {
            Block blk;
            const std::string l = d + ".down_blocks." + std::to_string(i);
            for (int j = 0; j < LAYERS; ++j) {
                DwResnet r;
                r.load(W, l + ".resnets." + std::to_string(j), j == 0 ? c_prev : CH[i], CH[i]);
                blk.res.push_back(std::move(r));
                MixTransformer t;
                t.load(W, l + ".attentions." + std::to_string(j), CH[i], ehs);
                blk.attn.push_back(std::move(t));
            }
            if (i + 1 < 3) {
                blk.has_sample = true;
                blk.sample.load(W, l + ".downsamplers.0", CH[i], 2, 0);
            }
            down.push_back(std::move(blk));
            c_prev = CH[i];
        }
        std::vector<int> skips = {CH[0]};
        for (int i = 0; i < 3; ++i) {
            skips.push_back(CH[i]);
            skips.push_back(CH[i]);
            if (i + 1 < 3) skips.push_back(CH[i]);
        }
        int h_c = CH[2];
        for (int i = 0; i < 3; ++i) {
            const int c = CH[2 - i];
            Block blk;
            const std::string l = d + ".up_blocks." + std::to_string(i);
            for (int j = 0; j <= LAYERS; ++j) {
                const int skip_c = skips.back();
                skips.pop_back();
                DwResnet r;
                r.load(W, l + ".resnets." + std::to_string(j), h_c + skip_c, c);
                blk.res.push_back(std::move(r));
                MixTransformer t;
                t.load(W, l + ".attentions." + std::to_string(j), c, ehs);
                blk.attn.push_back(std::move(t));
                h_c = c;
            }
            if (i + 1 < 3) {
                blk.has_sample = true;
                blk.sample.load(W, l + ".upsamplers.0", c, 1, 1);
            }
            up.push_back(std::move(blk));
        }
        lin1.load(W, d + ".time_embedding.linear_1", TIME_PROJ, TIME_EMBED, true);
        lin2.load(W, d + ".time_embedding.linear_2", TIME_EMBED, TIME_EMBED, true);
        conv_in.load(W, d + ".conv_in", 9, CH[0]);
        norm_out.load(W, d + ".conv_norm_out", CH[0], RESNET_EPS);
        conv_out.load(W, d + ".conv_out", CH[0], 4);
    }

    // src/unet/mod.rs:150-243
    void forward(const float *x, int timestep, int guidance, float *eps, OrcTraceFn trace, void *user) const {
        std::vector<int> branches = guidance == 0 ? std::vector<int>{0, 1} : std::vector<int>{1};
        const int64_t b = int64_t(branches.size());
        auto tr = [&](const std::string &name, const T4 &t) {
            if (trace) trace(user, name.c_str(), t.p(), t.n, t.h, t.w, t.c);
        };
        // time embedding (src/unet/embed.rs:21-66)
        float sinus[TIME_PROJ];
        orc_timestep_sinusoid(timestep, sinus);
        Vec a1(TIME_EMBED), a2(TIME_EMBED);
        lin1.fwd(sinus, 1, a1.data());
        orc_silu_inplace(a1.data(), TIME_EMBED);
        lin2.fwd(a1.data(), 1, a2.data());
        // upstream runs the time embedding on the batch and projects the text
        // states every step (the oracle does the latter once, at load)
        tally(kFMatmul, 2.0 * double(b) * (TIME_PROJ * TIME_EMBED + TIME_EMBED * TIME_EMBED) +
                            2.0 * double(b) * TOKENS * EHS * XDIM);
        T4 temb;
        temb.set(b, 1, 1, TIME_EMBED);
        for (int64_t i = 0; i < b; ++i) std::memcpy(temb.p() + i * TIME_EMBED, a2.data(), TIME_EMBED * sizeof(float));
        tr("unet.temb", temb);

        T4 input;
        input.set(b, 64, 64, 9);
        for (int64_t i = 0; i < b; ++i) std::memcpy(input.p() + i * 64 * 64 * 9, x, 64 * 64 * 9 * sizeof(float));
        std::vector<T4> skips(1);
        conv_in.fwd(input, skips[0]);
        tr("unet.conv_in", skips[0]);
        for (size_t i = 0; i < down.size(); ++i) {
            for (size_t j = 0; j < down[i].res.size(); ++j) {
                T4 a, h;
                down[i].res[j].fwd(skips.back(), temb.d, a);
                tr("unet.down." + std::to_string(i) + ".res." + std::to_string(j), a);
                down[i].attn[j].fwd(a, branches, h);
                tr("unet.down." + std::to_string(i) + ".attn." + std::to_string(j), h);
                skips.push_back(std::move(h));
            }
            if (down[i].has_sample) {
                T4 h;
                down[i].sample.fwd(skips.back(), h);
                skips.push_back(std::move(h));
            }
            tr("unet.down." + std::to_string(i) + ".out", skips.back());
        }
        T4 h = skips.back();
        for (size_t i = 0; i < up.size(); ++i) {
            for (size_t j = 0; j < up[i].res.size(); ++j) {
                T4 skip = std::move(skips.back());
                skips.pop_back();
                T4 cat;
                cat.set(h.n, h.h, h.w, h.c + skip.c);
                orc_concat_channels(h.p(), h.c, skip.p(), skip.c, h.px(), cat.p());
                T4 a;
                up[i].res[j].fwd(cat, temb.d, a);
                tr("unet.up." + std::to_string(i) + ".res." + std::to_string(j), a);
                up[i].attn[j].fwd(a, branches, h);
                tr("unet.up." + std::to_string(i) + ".attn." + std::to_string(j), h);
            }
            if (up[i].has_sample) {
                T4 a;
                up[i].sample.fwd(h, a);
                h = std::move(a);
            }
            tr("unet.up." + std::to_string(i) + ".out", h);
        }
        T4 a, out;
        norm_out.fwd(h, nullptr, true, a);
        conv_out.fwd(a, out);
        tr("unet.out", out);
        std::memcpy(eps, out.p(), out.d.size() * sizeof(float));
    }
};

}  // namespace

// The FLOP tally since the last reset: out[6] = 1x1, dense 3x3, stride-2 3x3,
// depthwise, position Conv3d, matrix products.
extern "C" void orc_unet_flops(double *out) {
    for (int i = 0; i < kFKinds; ++i) out[i] = g_flops[i];
}

extern "C" void orc_unet_flops_reset(void) {
    for (int i = 0; i < kFKinds; ++i) g_flops[i] = 0.0;
}

// src/unet/embed.rs:21-30: [cos | sin] of t * exp(-ln(10000) * i / 160), f32 with libm.
extern "C" void orc_timestep_sinusoid(int t, float *out) {
    const int half = TIME_PROJ / 2;
    const float log_period = -float(std::log(10000.0));
    for (int i = 0; i < half; ++i) {
        const float freq = std::exp(log_period * float(i) / float(half));
        const float arg = float(t) * freq;
        out[i] = std::cos(arg);
        out[half + i] = std::sin(arg);
    }
}

extern "C" void *orc_unet_create(const OrcNamed *tensors, int count, char *err, int err_len) {
    try {
        Weights W;
        for (int i = 0; i < count; ++i) W.m[tensors[i].name] = {tensors[i].data, tensors[i].numel};
        auto u = std::make_unique<UNet>();
        u->load(W);
        return u.release();
    } catch (const std::exception &e) {
        if (err && err_len > 0) {
            std::strncpy(err, e.what(), size_t(err_len - 1));
            err[err_len - 1] = 0;
        }
        return nullptr;
    }
}

extern "C" void orc_unet_destroy(void *unet) { delete static_cast<UNet *>(unet); }

extern "C" int orc_unet_forward(void *unet, const float *x, int timestep, int guidance, float *eps, OrcTraceFn trace,
                                void *user) {
    try {
        static_cast<UNet *>(unet)->forward(x, timestep, guidance, eps, trace, user);
        return 0;
    } catch (const std::exception &) {
        return 1;
    }
}

// One block of the UNet on its own: kind 0 DwConv2d, 1 DwResnet (temb [n,1280]),
// 2 SelfLambda, 3 CrossLambda, 4 MixTransformer; tensors under `prefix`. Kinds 3
// and 4 also read embedding_layer.weight and diff_model.encoder_hid_proj.*.
// branches: per item, 0 = uncond, 1 = cond. Returns 0, or 1 with err set.
extern "C" int orc_block_forward(int kind, const OrcNamed *tensors, int count, const char *prefix, const float *x,
                                 int64_t n, int64_t h, int64_t w, int64_t c_in, int64_t c_out, const float *temb,
                                 const int *branches, float *out, char *err, int err_len) {
    try {
        Weights W;
        for (int i = 0; i < count; ++i) W.m[tensors[i].name] = {tensors[i].data, tensors[i].numel};
        T4 xt;
        xt.set(n, h, w, c_in);
        std::memcpy(xt.p(), x, xt.d.size() * sizeof(float));
        T4 y;
        std::vector<int> br(branches ? branches : nullptr, branches ? branches + n : nullptr);
        auto ehs = [&](Vec e[2]) {
            const float *table = W.get("embedding_layer.weight", int64_t(20) * EHS);
            Lin proj;
            proj.load(W, "diff_model.encoder_hid_proj", EHS, XDIM, true);
            for (int b = 0; b < 2; ++b) {
                e[b].resize(size_t(TOKENS * XDIM));
                proj.fwd(table + int64_t(b == 0 ? TOKENS : 0) * EHS, TOKENS, e[b].data());
            }
        };
        switch (kind) {
            case 0: {
                DwConv2d m;
                m.load(W, prefix, int(c_in), int(c_out));
                m.fwd(xt, y);
                break;
            }
            case 1: {
                DwResnet m;
                m.load(W, prefix, int(c_in), int(c_out));
                Vec t(temb, temb + n * TIME_EMBED);
                m.fwd(xt, t, y);
                break;
            }
            case 2: {
                SelfLambda m;
                m.load(W, prefix, int(c_in));
                m.fwd(xt, y);
                break;
            }
            case 3: {
                Vec e[2];
                ehs(e);
                CrossLambda m;
                m.load(W, prefix, int(c_in), e);
                m.fwd(xt, br, y);
                break;
            }
            case 4: {
                Vec e[2];
                ehs(e);
                MixTransformer m;
                m.load(W, prefix, int(c_in), e);
                m.fwd(xt, br, y);
                break;
            }
            default:
                throw std::runtime_error("unknown block kind");
        }
        std::memcpy(out, y.p(), y.d.size() * sizeof(float));
        return 0;
    } catch (const std::exception &e) {
        if (err && err_len > 0) {
            std::strncpy(err, e.what(), size_t(err_len - 1));
            err[err_len - 1] = 0;
        }
        return 1;
    }
}

extern "C" void orc_softmax_lambda(float *keys, const float *v, int64_t rows, int64_t k, int64_t vd, float *lambda) {
    Vec l = softmax_lambda(keys, v, rows, k, vd);
    std::memcpy(lambda, l.data(), l.size() * sizeof(float));
}

extern "C" void orc_tap_filter(const float *a, const float *v, float *o, int64_t first, int64_t count, int64_t hh,
                               int64_t ww, int64_t vd) {
    tap_filter(a, v, o, first, count, hh, ww, vd);
}

extern "C" float orc_dot8(const float *a, const float *b, int64_t k) { return dot8(a, b, k); }

// src/unet/lambda.rs:279-295 over `count` pixels: q, o [count][8k]; e [count][10][k]; v [10][k].
extern "C" void orc_position_term(const float *q, const float *e, const float *v, float *o, int64_t count, int64_t k) {
    const int64_t c = HEADS * k;
    for (int64_t i = 0; i < count; ++i) {
        for (int h = 0; h < HEADS; ++h) {
            const float *qh = q + i * c + h * k;
            float *oh = o + i * c + h * k;
            for (int m = 0; m < TOKENS; ++m) {
                const float bb = dot8(qh, e + (i * TOKENS + m) * k, k);
                for (int64_t j = 0; j < k; ++j) oh[j] = std::fma(bb, v[m * k + j], oh[j]);
            }
        }
    }
}
