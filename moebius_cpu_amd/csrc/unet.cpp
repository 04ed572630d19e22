// Device UNet: src/unet/{mod,blocks,transformer,lambda,embed,load}.rs over the
// gfx950 kernels. The whole denoise step stays in HBM: inputs tiled to the CFG
// batch on the device, the skip stack held in pooled buffers, and only eps
// leaves the device.
#include <cstdlib>
#include "unet.hpp"

#include <cmath>
#include <cstring>

namespace mh {

namespace {

constexpr int CH[3] = {320, 640, 1280};
constexpr int LAYERS = 2;
constexpr int HEADS = 8;
constexpr int GROUPS = 32;
constexpr int TIME_PROJ = 320;
constexpr int TIME_EMBED = 1280;
constexpr int TOKENS = 10;
constexpr int EHS = 3072;
constexpr int XDIM = 768;
constexpr int TAPS = 225, TAPS_B = 226;
constexpr float RESNET_EPS = 1e-5f;
constexpr float TGN_EPS = 1e-6f;
constexpr float LN_EPS = 1e-5f;

uint16_t f32_to_f16_bits(float f) {
    _Float16 h = static_cast<_Float16>(f);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return static_cast<float>(h);
}

}  // namespace

void timestep_sinusoid(int t, float *out) {
    const int half = TIME_PROJ / 2;
    const float log_period = -float(std::log(10000.0));
    for (int i = 0; i < half; ++i) {
        const float freq = std::exp(log_period * float(i) / float(half));
        const float arg = float(t) * freq;
        out[i] = std::cos(arg);
        out[half + i] = std::sin(arg);
    }
}

// ---------------------------------------------------------------- weights
WeightStore::WeightStore(Context &ctx, const NamedTensor *t, int count, bool widen) : ctx_(ctx) {
    std::vector<size_t> off(static_cast<size_t>(count));
    size_t total = 0;
    for (int i = 0; i < count; ++i) {
        if (!t[i].name || !t[i].data) fail(kInvalidArgument, "weight table entry with NULL name or data");
        if (t[i].dtype != kF32 && t[i].dtype != kF16) fail(kInvalidArgument, std::string("bad dtype for ") + t[i].name);
        off[size_t(i)] = total;
        total += (t[i].numel * (t[i].dtype == kF16 ? 2 : 4) + 255) & ~size_t(255);
    }
    mh::dev_malloc(&block_, total ? total : 256);
    bytes_ = total;
    for (int i = 0; i < count; ++i) {
        char *dst = static_cast<char *>(block_) + off[size_t(i)];
        const size_t nb = t[i].numel * (t[i].dtype == kF16 ? 2 : 4);
        HIP_CHECK(hipMemcpyAsync(dst, t[i].data, nb, hipMemcpyHostToDevice, ctx.stream));
        Entry e;
        e.d.p = dst;
        e.d.wt = t[i].dtype == kF16 ? kF16 : kF32;
        e.d.numel = int64_t(t[i].numel);
        e.host = t[i].data;
        e.host_dtype = t[i].dtype;
        if (!m_.emplace(t[i].name, e).second) fail(kInvalidArgument, std::string("duplicate tensor ") + t[i].name);
    }
    // f32 widenings of the f16-stored (GEMM) weights, for EXACT arithmetic
    size_t wide = 0;
    for (auto &kv : m_)
        if (widen && kv.second.d.wt == kF16) wide += (size_t(kv.second.d.numel) * 4 + 255) & ~size_t(255);
    if (wide) {
        void *blk = nullptr;
        mh::dev_malloc(&blk, wide);
        derived_.push_back(blk);
        derived_bytes_ += wide;
        char *dst = static_cast<char *>(blk);
        for (auto &kv : m_) {
            DParam &d = kv.second.d;
            if (d.wt != kF16) continue;
            widen_f16(ctx, d.p, d.numel, reinterpret_cast<float *>(dst));
            d.p32 = reinterpret_cast<const float *>(dst);
            dst += (size_t(d.numel) * 4 + 255) & ~size_t(255);
        }
    }
    HIP_CHECK(hipStreamSynchronize(ctx.stream));
}

WeightStore::~WeightStore() {
    if (block_) (void)hipFree(block_);
    for (void *d : derived_) (void)hipFree(d);
}

const float *WeightStore::winograd_kernel(const DParam &w, int co, int ci) const {
    if (w.numel != int64_t(co) * 9 * ci) fail(kWeights, "Winograd kernel: 3x3 weight has the wrong size");
    const size_t bytes = size_t(16) * co * ci * sizeof(float);
    void *u = nullptr;
    mh::dev_malloc(&u, bytes);
    derived_.push_back(u);
    derived_bytes_ += bytes;
    winograd_weight_transform(ctx_, w.p, w.wt, co, ci, static_cast<float *>(u));
    return static_cast<const float *>(u);
}

const void *WeightStore::winograd_kernel_f16(const float *u, int co, int ci) const {
    const size_t len = size_t(16) * co * ci;
    void *u16 = nullptr;
    mh::dev_malloc(&u16, len * 2);
    derived_.push_back(u16);
    derived_bytes_ += len * 2;
    round_f16(ctx_, u, int64_t(len), u16);
    return u16;
}

const float *WeightStore::winograd_kernel_fused(const float *u, int co, int ci) const {
    const size_t bytes = size_t(16) * co * ci * sizeof(float);
    void *uf = nullptr;
    mh::dev_malloc(&uf, bytes);
    derived_.push_back(uf);
    derived_bytes_ += bytes;
    winograd_fused_weights(ctx_, u, co, ci, static_cast<float *>(uf));
    return static_cast<const float *>(uf);
}

DParam WeightStore::get(const std::string &name, int64_t numel, bool gemm) const {
    auto it = m_.find(name);
    if (it == m_.end()) fail(kWeights, "missing tensor " + name);
    const DParam &d = it->second.d;
    if (d.numel != numel)
        fail(kWeights, "tensor " + name + " has " + std::to_string(d.numel) + " values, expected " +
                           std::to_string(numel));
    if (!gemm && d.wt != kF32) fail(kWeights, "tensor " + name + " must be stored f32");
    return d;
}

const float *WeightStore::host_f32(const std::string &name, int64_t numel, std::vector<float> &scratch) const {
    auto it = m_.find(name);
    if (it == m_.end()) fail(kWeights, "missing tensor " + name);
    if (it->second.d.numel != numel) fail(kWeights, "tensor " + name + " has the wrong size");
    if (it->second.host_dtype == kF32) return static_cast<const float *>(it->second.host);
    scratch.resize(size_t(numel));
    const uint16_t *h = static_cast<const uint16_t *>(it->second.host);
    for (int64_t i = 0; i < numel; ++i) scratch[size_t(i)] = f16_bits_to_f32(h[i]);
    return scratch.data();
}

WeightGroup concat_weights(Context &ctx, const DParam *members, int count) {
    WeightGroup g;
    bool all_f16 = true;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        all_f16 = all_f16 && members[i].wt == kF16;
        total += members[i].numel;
    }
    g.wt = all_f16 ? kF16 : kF32;
    const size_t esz = all_f16 ? 2 : 4;
    mh::dev_malloc(&g.p, size_t(total) * esz);
    char *dst = static_cast<char *>(g.p);
    for (int i = 0; i < count; ++i) {
        const DParam &m = members[i];
        if (m.wt == g.wt)
            HIP_CHECK(hipMemcpyAsync(dst, m.p, size_t(m.numel) * esz, hipMemcpyDeviceToDevice, ctx.stream));
        else  // an f16 member of an f32 group
            widen_f16(ctx, m.p, m.numel, reinterpret_cast<float *>(dst));
        dst += size_t(m.numel) * esz;
    }
    return g;
}

// ---------------------------------------------------------------- layers
namespace {

struct Env {
    Context &ctx;
    Pool &pool;
};

// GroupNorm partials request for a producer writing a [x.n, x.h, x.w, c] tensor.
GnPartials gn_request(Env &e, const DT &x, int c) {
    GnPartials gp;
    gp.part = e.pool.floats(ceil_div(x.px(), 32) * c * 2);
    gp.item_rows = x.h * x.w;
    return gp;
}

// Attaches the partials the producer wrote to its output, or returns the buffer.
void gn_attach(Env &e, DT &out, const GnPartials &gp) {
    if (gp.rows > 0) {
        out.gn = gp.part;
        out.gn_rows = gp.rows;
    } else {
        e.pool.recycle(gp.part);
    }
}

// t repeated to a batch of n items (t holds one); t is recycled.
DT widen(Env &e, DT &t, int n) {
    DT w = e.pool.tensor(n, t.h, t.w, t.c);
    tile_items(e.ctx, t.p, int64_t(t.h) * t.w * t.c, n, w.p);
    e.pool.recycle(t);
    return w;
}

struct Lin {  // Conv1x1 (src/engine/conv.rs:28-55)
    int ci = 0, co = 0;
    DParam w;
    const float *b = nullptr;
    void load(const WeightStore &W, const std::string &p, int ci_, int co_, bool bias) {
        ci = ci_, co = co_;
        w = W.get(p + ".weight", int64_t(ci) * co, true);
        b = bias ? W.get(p + ".bias", co, false).f() : nullptr;
    }
    void fwd(Env &e, const float *x, int64_t px, float *out, const float *res = nullptr,
             GemmEpilogue epi = GemmEpilogue::None) const {
        const DParam wd = w.at(e.ctx);
        conv1x1(e.ctx, x, px, ci, wd.p, wd.wt, co, b, res, out, epi);
    }
    DT fwd(Env &e, const DT &x, const DT *res = nullptr, GemmEpilogue epi = GemmEpilogue::None) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, co);
        fwd(e, x.p, x.px(), out.p, res ? res->p : nullptr, epi);
        return out;
    }
    // The same, writing LayerNorm row partials of the output (lnp) for the
    // LayerNorm that reads it next.
    DT fwd_lnp(Env &e, const DT &x, LnRowPartials *lnp) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, co);
        const DParam wd = w.at(e.ctx);
        conv1x1(e.ctx, x.p, x.px(), ci, wd.p, wd.wt, co, b, nullptr, out.p, GemmEpilogue::None, nullptr, nullptr,
                nullptr, nullptr, nullptr, 0, lnp);
        return out;
    }
    // The same of [xa | xb] per pixel, read from the two tensors.
    DT fwd2(Env &e, const DT &xa, const DT &xb) const {
        DT out = e.pool.tensor(xa.n, xa.h, xa.w, co);
        const DParam wd = w.at(e.ctx);
        conv1x1(e.ctx, xa.p, xa.px(), ci, wd.p, wd.wt, co, b, nullptr, out.p, GemmEpilogue::None, nullptr, nullptr,
                nullptr, nullptr, xb.p, xb.c);
        return out;
    }
    // The same of GroupNorm(x) given its affine (ss = [scale | shift] per item
    // and channel, no SiLU), applied as x loads: the normalised tensor is not
    // written, and every value is the one the apply pass would write.
    DT fwd_gn_in(Env &e, const DT &x, const float *ss, LnRowPartials *lnp = nullptr) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, co);
        ResidualAffine xa;
        xa.scale = ss;
        xa.shift = ss + int64_t(x.n) * x.c;
        xa.silu = false;
        xa.rows_per_item = x.h * x.w;
        const DParam wd = w.at(e.ctx);
        conv1x1(e.ctx, x.p, x.px(), ci, wd.p, wd.wt, co, b, nullptr, out.p, GemmEpilogue::None, nullptr, nullptr,
                nullptr, &xa, nullptr, 0, lnp);
        return out;
    }
    // The same, with the GroupNorm partials of the output attached for the
    // GroupNorm that reads it next.
    DT fwd_gnp(Env &e, const DT &x, const DT *res = nullptr) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, co);
        GnPartials gp = gn_request(e, x, co);
        const DParam wd = w.at(e.ctx);
        conv1x1(e.ctx, x.p, x.px(), ci, wd.p, wd.wt, co, b, res ? res->p : nullptr, out.p, GemmEpilogue::None, nullptr,
                nullptr, &gp);
        gn_attach(e, out, gp);
        return out;
    }
};

struct GN {
    int c = 0;
    float eps = 0;
    const float *g = nullptr, *b = nullptr;
    void load(const WeightStore &W, const std::string &p, int c_, float eps_) {
        c = c_, eps = eps_;
        g = W.get(p + ".weight", c, false).f();
        b = W.get(p + ".bias", c, false).f();
    }
    DT fwd(Env &e, const DT &x, const float *add, bool silu, int64_t add_ld = 0) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, x.c);
        if (x.gn) {
            float *ss = affine(e, x, add, add_ld);
            apply_affine(e.ctx, x.p, x.n, x.h, x.w, x.c, ss, ss + int64_t(x.n) * x.c, silu, out.p);
            e.pool.recycle(ss);
        } else {
            group_norm_forward(e.ctx, x.p, x.n, x.h, x.w, x.c, GROUPS, eps, g, b, add, silu, out.p, add_ld);
        }
        return out;
    }
    // The same of [xa | xb] per pixel (the up path's concatenation, not written).
    float *affine2(Env &e, const DT &xa, const DT &xb) const {
        const int cc = xa.c + xb.c;
        float *ss = e.pool.floats(int64_t(2) * xa.n * cc);
        group_norm_affine(e.ctx, xa.p, xa.n, xa.h, xa.w, cc, GROUPS, eps, g, b, nullptr, ss, ss + int64_t(xa.n) * cc,
                          0, xb.p, xb.c);
        return ss;
    }
    // Statistics only: [scale | shift], each [n * c], for a consumer that
    // applies them; from the producer's partials when x carries them.
    float *affine(Env &e, const DT &x, const float *add, int64_t add_ld = 0) const {
        float *ss = e.pool.floats(int64_t(2) * x.n * x.c);
        if (x.gn)
            group_norm_affine_partials(e.ctx, x.gn, x.gn_rows, x.n, x.h * x.w, x.c, GROUPS, eps, g, b, add, ss,
                                       ss + int64_t(x.n) * x.c, add_ld);
        else
            group_norm_affine(e.ctx, x.p, x.n, x.h, x.w, x.c, GROUPS, eps, g, b, add, ss, ss + int64_t(x.n) * x.c,
                              add_ld);
        return ss;
    }
};

struct LNp {
    int c = 0;
    const float *g = nullptr, *b = nullptr;
    void load(const WeightStore &W, const std::string &p, int c_) {
        c = c_;
        g = W.get(p + ".weight", c, false).f();
        b = W.get(p + ".bias", c, false).f();
    }
    DT fwd(Env &e, const DT &x) const {
        DT out = e.pool.tensor(x.n, x.h, x.w, x.c);
        layer_norm(e.ctx, x.p, x.px(), c, g, b, LN_EPS, out.p);
        return out;
    }
};

// src/unet/blocks.rs:31-54: pw1x1(relu(dw3x3(x) + b1)) + b2 (+ x when c_in == c_out)
// FAST contexts: a depthwise conv whose output only the next 1x1 reads writes it
// in f16 (depthwise3x3_h16) for that 1x1 to read as f16 (conv1x1_a16): the
// products the f16 GEMM would take of the f32 output, from half the bytes. Needs
// the 1x1's weight in f16 (tuning dw_out16 0: f32 output).
bool dw_h16(const Env &e, const DParam &pw) { return e.ctx.tune.dw_out16 && pw.wt == kF16; }

struct DwConv2d {
    int ci = 0, co = 0;
    const float *dw = nullptr, *dwb = nullptr;
    Lin pw;
    void load(const WeightStore &W, const std::string &p, int ci_, int co_) {
        ci = ci_, co = co_;
        dw = W.get(p + ".conv_dw.weight", int64_t(9) * ci, false).f();
        dwb = W.get(p + ".conv_dw.bias", ci, false).f();
        pw.load(W, p + ".conv_pw", ci, co, true);
    }
    // res2: added last (the resnet's shortcut). out: caller's buffer or a new tensor.
    DT fwd(Env &e, const DT &x, const float *res2 = nullptr, float *out_p = nullptr) const {
        DT mid = e.pool.tensor(x.n, x.h, x.w, x.c);
        const DParam wd = pw.w.at(e.ctx);
        const bool h16 = dw_h16(e, wd) && depthwise3x3_h16(e.ctx, x.p, x.n, x.h, x.w, x.c, dw, dwb, 1, mid.p);
        if (!h16) depthwise3x3(e.ctx, x.p, x.n, x.h, x.w, x.c, dw, dwb, 1, mid.p);
        DT out = out_p ? DT{out_p, x.n, x.h, x.w, co} : e.pool.tensor(x.n, x.h, x.w, co);
        if (h16)
            conv1x1_a16(e.ctx, mid.p, mid.px(), ci, wd.p, co, pw.b, ci == co ? x.p : nullptr, out.p, nullptr, res2);
        else
            conv1x1(e.ctx, mid.p, mid.px(), ci, wd.p, wd.wt, co, pw.b, ci == co ? x.p : nullptr, out.p,
                    GemmEpilogue::None, nullptr, res2);
        e.pool.recycle(mid);
        return out;
    }
    // The same of a = SiLU(x . scale + shift) (a GroupNorm affine, ss = [scale |
    // shift] per item and channel) without writing a: the depthwise conv applies
    // the affine as it stages its input, and the identity residual (c_in ==
    // c_out) is a transformed in the pointwise conv's epilogue. Every value is
    // computed as the separate apply pass would (fma, then SiLU), so the result
    // is bit-identical to fwd(apply(x)). gn_out: attach the output's GroupNorm
    // partials (for the GroupNorm that reads it next).
    // fwd_gn of [xa | xb] per pixel (c_in = xa.c + xb.c != c_out), read from
    // the two tensors: the depthwise conv stages from both.
    DT fwd_gn2(Env &e, const DT &xa, const DT &xb, const float *ss, bool gn_out) const {
        const int cc = xa.c + xb.c;
        if (cc != ci || ci == co) fail(kInternal, "DwConv2d over two inputs: channel mismatch");
        Affine aff;
        aff.scale = ss;
        aff.shift = ss + int64_t(xa.n) * cc;
        aff.silu = true;
        DT mid = e.pool.tensor(xa.n, xa.h, xa.w, cc);
        const DParam wd = pw.w.at(e.ctx);
        const bool h16 = dw_h16(e, wd) &&
                         depthwise3x3_h16(e.ctx, xa.p, xa.n, xa.h, xa.w, cc, dw, dwb, 1, mid.p, &aff, xb.p, xb.c);
        if (!h16) depthwise3x3(e.ctx, xa.p, xa.n, xa.h, xa.w, cc, dw, dwb, 1, mid.p, &aff, xb.p, xb.c);
        DT out = e.pool.tensor(xa.n, xa.h, xa.w, co);
        GnPartials gp;
        if (gn_out) gp = gn_request(e, xa, co);
        if (h16)
            conv1x1_a16(e.ctx, mid.p, mid.px(), ci, wd.p, co, pw.b, nullptr, out.p, nullptr, nullptr,
                        gn_out ? &gp : nullptr);
        else
            conv1x1(e.ctx, mid.p, mid.px(), ci, wd.p, wd.wt, co, pw.b, nullptr, out.p, GemmEpilogue::None, nullptr,
                    nullptr, gn_out ? &gp : nullptr);
        if (gn_out) gn_attach(e, out, gp);
        e.pool.recycle(mid);
        return out;
    }
    DT fwd_gn(Env &e, const DT &x, const float *ss, const float *res2 = nullptr, float *out_p = nullptr,
              bool gn_out = false) const {
        Affine aff;
        aff.scale = ss;
        aff.shift = ss + int64_t(x.n) * x.c;
        aff.silu = true;
        DT mid = e.pool.tensor(x.n, x.h, x.w, x.c);
        const DParam wd = pw.w.at(e.ctx);
        const bool h16 = dw_h16(e, wd) && depthwise3x3_h16(e.ctx, x.p, x.n, x.h, x.w, x.c, dw, dwb, 1, mid.p, &aff);
        if (!h16) depthwise3x3(e.ctx, x.p, x.n, x.h, x.w, x.c, dw, dwb, 1, mid.p, &aff);
        DT out = out_p ? DT{out_p, x.n, x.h, x.w, co} : e.pool.tensor(x.n, x.h, x.w, co);
        ResidualAffine ra;
        ra.scale = aff.scale;
        ra.shift = aff.shift;
        ra.silu = true;
        ra.rows_per_item = x.h * x.w;
        GnPartials gp;
        if (gn_out) gp = gn_request(e, x, co);
        if (h16)
            conv1x1_a16(e.ctx, mid.p, mid.px(), ci, wd.p, co, pw.b, ci == co ? x.p : nullptr, out.p,
                        ci == co ? &ra : nullptr, res2, gn_out ? &gp : nullptr);
        else
            conv1x1(e.ctx, mid.p, mid.px(), ci, wd.p, wd.wt, co, pw.b, ci == co ? x.p : nullptr, out.p,
                    GemmEpilogue::None, ci == co ? &ra : nullptr, res2, gn_out ? &gp : nullptr);
        if (gn_out) gn_attach(e, out, gp);
        e.pool.recycle(mid);
        return out;
    }
};

// src/unet/blocks.rs:56-113
struct DwResnet {
    int ci = 0, co = 0;
    GN norm1, norm2;
    DwConv2d conv1, conv2;
    Lin temb_proj, shortcut;
    bool has_shortcut = false;
    int temb_off = 0;  // this block's columns in the step's batched time projection
    void load(const WeightStore &W, const std::string &p, int ci_, int co_) {
        ci = ci_, co = co_;
        norm1.load(W, p + ".norm1", ci, RESNET_EPS);
        conv1.load(W, p + ".conv1", ci, co);
        temb_proj.load(W, p + ".time_emb_proj", TIME_EMBED, co, true);
        norm2.load(W, p + ".norm2", co, RESNET_EPS);
        conv2.load(W, p + ".conv2", co, co);
        has_shortcut = ci != co;
        if (has_shortcut) shortcut.load(W, p + ".conv_shortcut", ci, co, true);
    }
    // temb_silu: [n, 1280] = SiLU(temb), shared by every resnet of the step.
    // tp: this block's time projection, item i's row at tp + i * tp_ld (all the
    // step's projections come out of one GEMM, UNetDevice::forward), folded into
    // norm2's shift. Neither GroupNorm output is written: each DwConv2d applies
    // GN + SiLU as its depthwise conv stages the input in LDS (about 1.6
    // evaluations per value), and its identity residual in the pointwise
    // epilogue. The shortcut (or x) is added in conv2's pointwise epilogue.
    DT fwd(Env &e, const DT &x, const float *tp, int64_t tp_ld) const {
        float *ss1 = norm1.affine(e, x, nullptr);
        DT b = conv1.fwd_gn(e, x, ss1, nullptr, nullptr, true);
        e.pool.recycle(ss1);
        float *ss2 = norm2.affine(e, b, tp, tp_ld);
        DT s;
        if (has_shortcut) s = shortcut.fwd(e, x);
        DT out = conv2.fwd_gn(e, b, ss2, has_shortcut ? s.p : x.p, nullptr, true);
        if (has_shortcut) e.pool.recycle(s);
        e.pool.recycle(ss2);
        e.pool.recycle(b);
        return out;
    }
    // fwd of [xa | xb] per pixel (the up path's skip concatenation,
    // src/unet/mod.rs:208-213) without writing it: norm1's statistics, conv1's
    // depthwise staging and the shortcut read both tensors. Needs a shortcut
    // (c_in != c_out) and xa.c a multiple of 64.
    bool takes_two(const DT &xa, const DT &xb) const {
        return has_shortcut && xa.c + xb.c == ci && xa.c % 64 == 0 && xb.c % 4 == 0 && xa.n == xb.n &&
               xa.h == xb.h && xa.w == xb.w;
    }
    DT fwd2(Env &e, const DT &xa, const DT &xb, const float *tp, int64_t tp_ld) const {
        float *ss1 = norm1.affine2(e, xa, xb);
        DT b = conv1.fwd_gn2(e, xa, xb, ss1, true);
        e.pool.recycle(ss1);
        float *ss2 = norm2.affine(e, b, tp, tp_ld);
        DT s = shortcut.fwd2(e, xa, xb);
        DT out = conv2.fwd_gn(e, b, ss2, s.p, nullptr, true);
        e.pool.recycle(s);
        e.pool.recycle(ss2);
        e.pool.recycle(b);
        return out;
    }
};

// A LayerNorm folded into the 1x1 conv that reads it (LnFolded): owns the
// folded weights W . diag(gamma) (f32 and the f16 rounding), their row sums
// and W . beta + b, built once at load.
struct LnFold {
    float *w32 = nullptr, *c1_32 = nullptr, *c1_16 = nullptr, *c2 = nullptr;
    void *w16 = nullptr;
    void build(Context &ctx, const void *w, WeightType wt, int n, int k, const float *gamma, const float *beta,
               const float *bias) {
        mh::dev_malloc(&w32, size_t(n) * k * sizeof(float));
        mh::dev_malloc(&w16, size_t(n) * k * 2);
        mh::dev_malloc(&c1_32, size_t(n) * sizeof(float));
        mh::dev_malloc(&c1_16, size_t(n) * sizeof(float));
        mh::dev_malloc(&c2, size_t(n) * sizeof(float));
        ln_fold_weights(ctx, w, wt, n, k, gamma, beta, bias, w32, w16, c1_32, c1_16, c2);
    }
    LnFolded view(float eps) const {
        LnFolded f;
        f.w32 = w32, f.c1_32 = c1_32, f.w16 = w16, f.c1_16 = c1_16, f.c2 = c2, f.eps = eps;
        return f;
    }
    void release() {
        for (void *q : {static_cast<void *>(w32), w16, static_cast<void *>(c1_32), static_cast<void *>(c1_16),
                        static_cast<void *>(c2)})
            if (q) (void)hipFree(q);
        w32 = c1_32 = c1_16 = c2 = nullptr;
        w16 = nullptr;
    }
};

// src/unet/lambda.rs:73-152
struct SelfLambda {
    int c = 0, k = 0;
    Lin to_q, to_k, to_v;
    float *w_aug_t = nullptr;  // [226][k]: column d of the folded filter per row
    void *wqkv = nullptr;      // [c + 2k][c]: to_q | to_k | to_v
    float *wqkv32 = nullptr;   // its f32 widening when stored f16 (EXACT reads it)
    float *bqkv = nullptr;
    WeightType wt = kF32;
    void load(Env &e, const WeightStore &W, const std::string &p, int c_) {
        c = c_, k = c / HEADS;
        std::vector<float> s1, s2;
        const float *w = W.host_f32(p + ".pos_conv.weight", int64_t(k) * TAPS, s1);
        const float *b = W.host_f32(p + ".pos_conv.bias", k, s2);
        std::vector<float> t(size_t(TAPS_B) * k);
        for (int kk = 0; kk < k; ++kk) {
            for (int d = 0; d < TAPS; ++d) t[size_t(d) * k + kk] = w[kk * TAPS + d];
            t[size_t(TAPS) * k + kk] = b[kk];
        }
        mh::dev_malloc(&w_aug_t, t.size() * sizeof(float));
        HIP_CHECK(hipMemcpy(w_aug_t, t.data(), t.size() * sizeof(float), hipMemcpyHostToDevice));
        to_q.load(W, p + ".to_q", c, c, true);
        to_k.load(W, p + ".to_k", c, k, false);
        to_v.load(W, p + ".to_v", c, k, true);
        // q | k | v weights [c + 2k][c] and bias (k has none: zeros), for one GEMM.
        const DParam members[3] = {to_q.w, to_k.w, to_v.w};
        const WeightGroup grp = concat_weights(e.ctx, members, 3);
        wqkv = grp.p;
        wt = grp.wt;
        mh::dev_malloc(&bqkv, size_t(c + 2 * k) * sizeof(float));
        if (wt == kF16) {
            mh::dev_malloc(&wqkv32, size_t(c + 2 * k) * c * sizeof(float));
            widen_f16(e.ctx, wqkv, int64_t(c + 2 * k) * c, wqkv32);
        }
        std::vector<float> zeros(size_t(k), 0.0f);
        HIP_CHECK(hipMemcpyAsync(bqkv, to_q.b, size_t(c) * sizeof(float), hipMemcpyDeviceToDevice, e.ctx.stream));
        HIP_CHECK(hipMemcpy(bqkv + c, zeros.data(), size_t(k) * sizeof(float), hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpyAsync(bqkv + c + k, to_v.b, size_t(k) * sizeof(float), hipMemcpyDeviceToDevice,
                                 e.ctx.stream));
        HIP_CHECK(hipStreamSynchronize(e.ctx.stream));
    }
    void release() {
        if (w_aug_t) (void)hipFree(w_aug_t);
        if (wqkv) (void)hipFree(wqkv);
        if (wqkv32) (void)hipFree(wqkv32);
        if (bqkv) (void)hipFree(bqkv);
        w_aug_t = nullptr;
        wqkv = nullptr;
        wqkv32 = nullptr;
        bqkv = nullptr;
    }
    // h [x.px()][c] += SelfLambda(x): the block's residual add is folded into the tap filter.
    // ln: x is the block's hidden state and LayerNorm 1 is folded into the q | k | v GEMM.
    // row_sums (optional, instead of lno): LayerNorm row partials of the new h, one per pixel.
    void fwd_add(Env &e, const DT &x, float *h, const LayerNormOut *lno = nullptr,
                 const LnFolded *ln = nullptr, const LnRowPartials *ln_stats = nullptr,
                 float2 *row_sums = nullptr) const {
        const int hw = x.h * x.w;
        DT q = e.pool.tensor(x.n, x.h, x.w, c);
        DT kt = e.pool.tensor(x.n, x.h, x.w, k);
        DT vt = e.pool.tensor(x.n, x.h, x.w, k);
        {
            const int widths[3] = {c, k, k};
            float *const outs[3] = {q.p, kt.p, vt.p};
            const bool w32 = wqkv32 && e.ctx.precision == Precision::Exact;
            if (ln)
                conv1x1_ln(e.ctx, x.p, x.px(), c, *ln, 3, widths, outs, GemmEpilogue::None, ln_stats);
            else
                conv1x1_segments(e.ctx, x.p, x.px(), c, w32 ? wqkv32 : wqkv, w32 ? kF32 : wt, bqkv, 3, widths,
                                 outs);
        }
        float *lam_t = e.pool.floats(int64_t(x.n) * k * k);
        softmax_lambda(e.ctx, kt.p, vt.p, x.n, hw, k, k, lam_t);
        e.pool.recycle(kt);
        if (!lno && self_lambda_fused_ok(e.ctx, k)) {
            // A and Yc formed inside the tap filter's row tiles, never written
            self_lambda_fused(e.ctx, q.p, w_aug_t, lam_t, vt.p, h, h, x.n, x.h, x.w, k, row_sums);
            e.pool.recycle(lam_t);
            e.pool.recycle(q);
            e.pool.recycle(vt);
            return;
        }
        DT yc = e.pool.tensor(x.n, x.h, x.w, c);
        // A = Q . W_aug over every pixel and head of the batch, stored [pixel][tap][head],
        // and Yc = Q . lambda_c per item (Q viewed as [(hw*8) x k]), both by one dedicated
        // kernel (64x64 x 40, batch 2: 25.4 us for both against 34.5 + 12 us for the two
        // GEMMs; whole EXACT step 7.60 -> 7.50 ms; in FAST on f16-rounded operands, as the
        // FAST GEMMs take them), or (the lambda_taps tuning off) two general GEMMs.
        float *a = e.pool.floats(x.px() * HEADS * TAPS_B);
        if (e.ctx.tune.lambda_taps && lambda_taps_ok(k)) {
            lambda_taps(e.ctx, q.p, w_aug_t, lam_t, x.n, hw, k, a, yc.p);
        } else {
            gemm_nt(e.ctx, q.p, k, int64_t(hw) * c, lam_t, kF32, k, int64_t(k) * k, hw * HEADS, k, k, x.n, nullptr,
                    nullptr, yc.p, k, int64_t(hw) * c);
            gemm_nt(e.ctx, q.p, k, 0, w_aug_t, kF32, k, 0, int(x.px() * HEADS), TAPS_B, k, 1, nullptr, nullptr, a,
                    int64_t(TAPS_B) * HEADS, 0, GemmEpilogue::None, HEADS);
        }
        e.pool.recycle(lam_t);
        tap_filter(e.ctx, a, vt.p, yc.p, h, h, x.n, x.h, x.w, k, lno, row_sums);
        e.pool.recycle(a);
        e.pool.recycle(yc);
        e.pool.recycle(q);
        e.pool.recycle(vt);
    }
};

// src/unet/lambda.rs:187-274
struct CrossLambda {
    int c = 0, k = 0, n = 0;
    Lin to_q;
    const float *e = nullptr;       // rel_pos_emb [n][10][k]
    float *lambda_c = nullptr;      // [2][k][k] lambda_c per branch (row-major)
    float *v = nullptr;             // [2][10][k]
    void load(Env &env, const WeightStore &W, const std::string &p, int c_, const float *ehs_dev /*[2][10][768]*/) {
        c = c_, k = c / HEADS;
        const int side = 64 * 320 / c;
        n = side * side;
        const DParam wk = W.get(p + ".to_k.weight", int64_t(k) * XDIM, true);
        const DParam wv = W.get(p + ".to_v.weight", int64_t(k) * XDIM, true);
        const float *bv = W.get(p + ".to_v.bias", k, false).f();
        mh::dev_malloc(&lambda_c, size_t(2) * k * k * sizeof(float));
        mh::dev_malloc(&v, size_t(2) * TOKENS * k * sizeof(float));
        float *keys = env.pool.floats(int64_t(2) * TOKENS * k);
        for (int br = 0; br < 2; ++br) {
            const float *x = ehs_dev + int64_t(br) * TOKENS * XDIM;
            gemm_nt(env.ctx, x, XDIM, 0, wk.p, wk.wt, XDIM, 0, TOKENS, k, XDIM, 1, nullptr, nullptr,
                    keys + int64_t(br) * TOKENS * k, k, 0);
            // v = ehs . Wv^T, then + bias (src/unet/lambda.rs:225-235)
            gemm_nt(env.ctx, x, XDIM, 0, wv.p, wv.wt, XDIM, 0, TOKENS, k, XDIM, 1, nullptr, nullptr,
                    v + int64_t(br) * TOKENS * k, k, 0);
            bias_residual_add(env.ctx, v + int64_t(br) * TOKENS * k, TOKENS, k, bv, nullptr,
                              v + int64_t(br) * TOKENS * k);
        }
        float *lambda_t = env.pool.floats(int64_t(2) * k * k);
        softmax_lambda(env.ctx, keys, v, 2, TOKENS, k, k, lambda_t);
        for (int br = 0; br < 2; ++br)
            transpose(env.ctx, lambda_t + int64_t(br) * k * k, k, k, k, lambda_c + int64_t(br) * k * k);
        env.pool.recycle(lambda_t);
        env.pool.recycle(keys);
        to_q.load(W, p + ".to_q", c, c, true);
        e = W.get(p + ".rel_pos_emb", int64_t(n) * TOKENS * k, false).f();
    }
    void release() {
        if (lambda_c) (void)hipFree(lambda_c);
        if (v) (void)hipFree(v);
        lambda_c = v = nullptr;
    }
    // h [x.px()][c] += CrossLambda(x): Yc = Q . lambda_c, the position term and
    // the residual add in one kernel after the q projection.
    // The same with LayerNorm 2 of hs folded into to_q (f: to_q on W . diag(gamma),
    // st: hs's row statistics); hs is h itself, read before the kernel updates it.
    void fwd_add_ln(Env &env, const DT &hs, int br0, float *h, const LnFolded &f, const LnRowPartials &st,
                    float2 *row_sums) const {
        const int hw = hs.h * hs.w;
        if (hw != n) fail(kInvalidArgument, "CrossLambda input size does not match the position table");
        DT q = env.pool.tensor(hs.n, hs.h, hs.w, c);
        float *const outs[1] = {q.p};
        conv1x1_ln(env.ctx, hs.p, hs.px(), c, f, 1, &c, outs, GemmEpilogue::None, &st);
        cross_lambda(env.ctx, q.p, e, lambda_c, v, br0, hs.n, hw, k, h, h, row_sums);
        env.pool.recycle(q);
    }
    // row_sums (optional): LayerNorm row partials of the new h, one per pixel.
    void fwd_add(Env &env, const DT &x, int br0, float *h, float2 *row_sums = nullptr) const {
        const int hw = x.h * x.w;
        if (hw != n) fail(kInvalidArgument, "CrossLambda input size does not match the position table");
        DT q = to_q.fwd(env, x);
        cross_lambda(env.ctx, q.p, e, lambda_c, v, br0, x.n, hw, k, h, h, row_sums);
        env.pool.recycle(q);
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
    LnFold ln1q, ln2q, ln3f;  // LayerNorms 1, 2, 3 folded into q | k | v, the cross to_q, the inverted 1x1
    const float *dw = nullptr, *dwb = nullptr;
    void load(Env &env, const WeightStore &W, const std::string &p, int c_, const float *ehs_dev) {
        c = c_;
        hidden = int(float(c) * 2.5f);
        const std::string b = p + ".transformer_blocks.0";
        const std::string ff = b + ".ff";
        dw = W.get(ff + ".depth_conv.conv.weight", int64_t(9) * 2 * hidden, false).f();
        dwb = W.get(ff + ".depth_conv.conv.bias", 2 * hidden, false).f();
        norm.load(W, p + ".norm", c, TGN_EPS);
        proj_in.load(W, p + ".proj_in", c, c, true);
        ln1.load(W, b + ".norm1", c);
        attn1.load(env, W, b + ".attn1", c);
        ln2.load(W, b + ".norm2", c);
        attn2.load(env, W, b + ".attn2", c, ehs_dev);
        ln3.load(W, b + ".norm3", c);
        inverted.load(W, ff + ".inverted_conv.conv", c, 2 * hidden, true);
        point.load(W, ff + ".point_conv.conv", hidden, c, false);
        proj_out.load(W, p + ".proj_out", c, c, true);
        ln1q.build(env.ctx, attn1.wqkv, attn1.wt, c + 2 * attn1.k, c, ln1.g, ln1.b, attn1.bqkv);
        ln2q.build(env.ctx, attn2.to_q.w.p, attn2.to_q.w.wt, c, c, ln2.g, ln2.b, attn2.to_q.b);
        ln3f.build(env.ctx, inverted.w.p, inverted.w.wt, 2 * hidden, c, ln3.g, ln3.b, inverted.b);
        HIP_CHECK(hipStreamSynchronize(env.ctx.stream));
    }
    void release() {
        attn1.release();
        attn2.release();
        ln1q.release();
        ln2q.release();
        ln3f.release();
    }
    DT fwd(Env &e, const DT &x, int br0) const { return fwd(e, x, x, br0); }
    // xs: the input for everything before the cross-lambda, xr: the same at the
    // full batch, the residual of proj_out. With CFG both branches see the same
    // values until the first cross-lambda, so the first block runs that part
    // on one item (xs.n == 1) and repeats h and LayerNorm 2's output to the batch
    // just before the cross-lambda; the results equal a batch-2 run's.
    DT fwd(Env &e, const DT &xs, const DT &xr, int br0) const {
        const DT &x = xs;
        // The GroupNorm affine goes into proj_in's operand loads up to 640 channels
        // (EXACT) / 320 (FAST): the loads cost per K tile, and at 1280 channels
        // (and 640 in FAST) they cost more than the separate apply pass (whole
        // steps: EXACT 7.764 ms unfused, 7.728 to 640, 7.773 to 1280; FAST 5.744,
        // 5.731 to 320, 5.778 to 640).
        // LayerNorms 1 and 3 (ln_fold 2, the default): folded into the GEMMs that
        // read them (q | k | v and the inverted 1x1, on W . diag(gamma)), with each
        // row's statistics from partial sums the producers of h write beside it
        // (proj_in's epilogue per column tile, the cross-lambda kernel per row):
        // no LayerNorm launch, no normalised tensor, no second read of h.
        const int fold = e.ctx.tune.ln_fold;
        LnRowPartials st1, st3;
        if (fold == 2) st1.part = reinterpret_cast<float2 *>(e.pool.floats(x.px() * 2 * ceil_div(c, 32)));
        DT h;
        const int max_c = e.ctx.tune.gn_in_maxc >= 0 ? e.ctx.tune.gn_in_maxc
                                                      : (e.ctx.precision == Precision::Fast ? 320 : 640);
        if (x.c <= max_c) {
            float *ss = norm.affine(e, x, nullptr);
            h = proj_in.fwd_gn_in(e, x, ss, fold == 2 ? &st1 : nullptr);
            e.pool.recycle(ss);
        } else {
            DT t = norm.fwd(e, x, nullptr, false);
            h = fold == 2 ? proj_in.fwd_lnp(e, t, &st1) : proj_in.fwd(e, t);
            e.pool.recycle(t);
        }
        // ln_fold 2 folds LayerNorm 2 into the cross-lambda's to_q the same way, from
        // row sums the tap filter writes as it finishes h. ln_fold 1: LayerNorms 1
        // and 3 folded with the row statistics summed by the GEMMs from the values
        // they load; 0: LayerNorm passes of their own. With 1 and 0 LayerNorm 2 is
        // written beside h by the tap filter (a separate pass costs a launch and a
        // re-read of h: whole step -29 us EXACT, -36 us FAST).
        const LnFolded lnq = ln1q.view(LN_EPS), lnf = ln3f.view(LN_EPS);
        if (fold == 2) {
            LnRowPartials st2;  // LayerNorm 2's row sums, per_row slices of the channels each
            st2.per_row = self_lambda_fused_ok(e.ctx, attn1.k) ? 1 : tap_filter_row_parts(e.ctx, h.h, h.w, attn1.k);
            st2.part = reinterpret_cast<float2 *>(e.pool.floats(h.px() * 2 * st2.per_row));
            if (st1.per_row > 0) {
                attn1.fwd_add(e, h, h.p, nullptr, &lnq, &st1, st2.part);
            } else {
                DT t = ln1.fwd(e, h);
                attn1.fwd_add(e, t, h.p, nullptr, nullptr, nullptr, st2.part);
                e.pool.recycle(t);
            }
            e.pool.recycle(reinterpret_cast<float *>(st1.part));
            if (xs.n != xr.n) {  // h and its row sums repeated to the batch
                h = widen(e, h, xr.n);
                float *w2 = e.pool.floats(h.px() * 2 * st2.per_row);
                tile_items(e.ctx, reinterpret_cast<const float *>(st2.part), int64_t(xs.px()) * 2 * st2.per_row, xr.n,
                           w2);
                e.pool.recycle(reinterpret_cast<float *>(st2.part));
                st2.part = reinterpret_cast<float2 *>(w2);
            }
            st3.part = reinterpret_cast<float2 *>(e.pool.floats(h.px() * 2));
            st3.per_row = 1;
            attn2.fwd_add_ln(e, h, br0, h.p, ln2q.view(LN_EPS), st2, st3.part);
            e.pool.recycle(reinterpret_cast<float *>(st2.part));
        } else {
            DT t2 = e.pool.tensor(h.n, h.h, h.w, h.c);
            LayerNormOut lno2;
            lno2.gamma = ln2.g;
            lno2.beta = ln2.b;
            lno2.eps = LN_EPS;
            lno2.out = t2.p;
            if (fold == 1) {
                attn1.fwd_add(e, h, h.p, &lno2, &lnq);
            } else {
                DT t = ln1.fwd(e, h);
                attn1.fwd_add(e, t, h.p, &lno2);
                e.pool.recycle(t);
            }
            if (xs.n != xr.n) {
                h = widen(e, h, xr.n);
                t2 = widen(e, t2, xr.n);
            }
            attn2.fwd_add(e, t2, br0, h.p);
            e.pool.recycle(t2);
        }
        // MixFFN (transformer.rs:121-129): SiLU(inverted(LN3 h)) -> GLU depthwise -> point + h
        DT a;
        if (fold) {
            a = e.pool.tensor(h.n, h.h, h.w, 2 * hidden);
            const int width = 2 * hidden;
            float *const outs[1] = {a.p};
            conv1x1_ln(e.ctx, h.p, h.px(), c, lnf, 1, &width, outs, GemmEpilogue::Silu, fold == 2 ? &st3 : nullptr);
            if (st3.part) e.pool.recycle(reinterpret_cast<float *>(st3.part));
        } else {
            DT t = ln3.fwd(e, h);
            a = inverted.fwd(e, t, nullptr, GemmEpilogue::Silu);
            e.pool.recycle(t);
        }
        DT g = e.pool.tensor(a.n, a.h, a.w, hidden);
        const DParam pwd = point.w.at(e.ctx);
        const bool h16 = dw_h16(e, pwd) && depthwise3x3_h16(e.ctx, a.p, a.n, a.h, a.w, a.c, dw, dwb, 2, g.p);
        if (!h16) depthwise3x3(e.ctx, a.p, a.n, a.h, a.w, a.c, dw, dwb, 2, g.p);
        e.pool.recycle(a);
        DT u;
        // u, read only by proj_out: f16 as well when proj_out's weight is
        const DParam powd = proj_out.w.at(e.ctx);
        const bool u16 = h16 && powd.wt == kF16;
        if (h16) {
            u = e.pool.tensor(g.n, g.h, g.w, point.co);
            conv1x1_a16(e.ctx, g.p, g.px(), point.ci, pwd.p, point.co, point.b, h.p, u.p, nullptr, nullptr, nullptr,
                        u16);
        } else {
            u = point.fwd(e, g, &h);
        }
        e.pool.recycle(g);
        e.pool.recycle(h);
        DT out;
        if (u16) {
            out = e.pool.tensor(u.n, u.h, u.w, proj_out.co);
            GnPartials gp = gn_request(e, u, proj_out.co);
            conv1x1_a16(e.ctx, u.p, u.px(), proj_out.ci, powd.p, proj_out.co, proj_out.b, xr.p, out.p, nullptr,
                        nullptr, &gp);
            gn_attach(e, out, gp);
        } else {
            out = proj_out.fwd_gnp(e, u, &xr);
        }
        e.pool.recycle(u);
        return out;
    }
};

// Downsample / Upsample (src/unet/blocks.rs:116-145). The upsample convs
// (stride 1, pad 1) run as Winograd F(2x2,3x3), the reference's algorithm for
// them (src/engine/conv.rs:92-98), with the kernel transformed at load: on the
// matrix cores it takes 2.1-2.3x less time than the implicit GEMM at these
// shapes (640 and 1280 channels), in f32 and f16 alike. The stride-2
// downsample convs are implicit GEMMs (the reference's im2col path).
struct Conv3 {
    int c = 0, stride = 1;
    bool up = false;
    DParam w;
    const float *u = nullptr;
    const void *u16 = nullptr;  // u rounded to f16, for FAST contexts (the same products, half the bytes)
    const float *b = nullptr;
    void load(const WeightStore &W, const std::string &p, int c_, int stride_, bool up_) {
        c = c_, stride = stride_, up = up_;
        w = W.get(p + ".conv.weight", int64_t(9) * c * c, true);
        b = W.get(p + ".conv.bias", c, false).f();
        if (stride == 1 && c % 4 == 0) {
            u = W.winograd_kernel(w, c, c);
            u16 = W.winograd_kernel_f16(u, c, c);
        }
    }
    DT fwd(Env &e, const DT &x) const {
        const int pad[4] = {1, 1, 1, 1};
        int ho, wo;
        conv3x3_output_hw(x.h, x.w, stride, pad, up, &ho, &wo);
        DT out = e.pool.tensor(x.n, ho, wo, c);
        if (u && e.ctx.precision == Precision::Fast && e.ctx.tune.wino_u16)
            conv3x3_winograd(e.ctx, x.p, x.n, x.h, x.w, x.c, u16, kF16, c, b, up, nullptr, out.p);
        else if (u)
            conv3x3_winograd(e.ctx, x.p, x.n, x.h, x.w, x.c, u, kF32, c, b, up, nullptr, out.p);
        else
            conv3x3(e.ctx, x.p, x.n, x.h, x.w, x.c, w.at(e.ctx).p, w.at(e.ctx).wt, c, b, stride, pad, up, nullptr,
                    out.p);
        return out;
    }
};

}  // namespace

// ---------------------------------------------------------------- model
class UNetDevice {
  public:
    UNetDevice(Context &ctx, const NamedTensor *t, int count) : ctx_(ctx), pool_(ctx), W_(ctx, t, count, true) {
        Env env{ctx_, pool_};
        // embed::conditioning (src/unet/embed.rs:72-83): [uncond = rows 10..20, cond = rows 0..10]
        const DParam table = W_.get("embedding_layer.weight", int64_t(20) * EHS, false);
        Lin proj;
        proj.load(W_, "diff_model.encoder_hid_proj", EHS, XDIM, true);
        float *ehs = pool_.floats(int64_t(2) * TOKENS * XDIM);
        proj.fwd(env, table.f() + int64_t(TOKENS) * EHS, TOKENS, ehs);
        proj.fwd(env, table.f(), TOKENS, ehs + TOKENS * XDIM);

        const std::string d = "diff_model";
        int c_prev = CH[0];
        for (int i = 0; i < 3; ++i) {
            Block blk;
            const std::string l = d + ".down_blocks." + std::to_string(i);
            for (int j = 0; j < LAYERS; ++j) {
                blk.res.emplace_back();
                blk.res.back().load(W_, l + ".resnets." + std::to_string(j), j == 0 ? c_prev : CH[i], CH[i]);
                blk.attn.emplace_back();
                blk.attn.back().load(env, W_, l + ".attentions." + std::to_string(j), CH[i], ehs);
            }
            if (i + 1 < 3) {
                blk.has_sample = true;
                blk.sample.load(W_, l + ".downsamplers.0", CH[i], 2, false);
            }
            down_.push_back(std::move(blk));
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
                blk.res.emplace_back();
                blk.res.back().load(W_, l + ".resnets." + std::to_string(j), h_c + skip_c, c);
                blk.attn.emplace_back();
                blk.attn.back().load(env, W_, l + ".attentions." + std::to_string(j), c, ehs);
                h_c = c;
            }
            if (i + 1 < 3) {
                blk.has_sample = true;
                blk.sample.load(W_, l + ".upsamplers.0", c, 1, true);
            }
            up_.push_back(std::move(blk));
        }
        // Every resnet's time_emb_proj in one [sum c_out][1280] matrix (and bias),
        // so a step projects the time embedding for all of them in one GEMM.
        {
            std::vector<DwResnet *> rs;
            for (auto *v : {&down_, &up_})
                for (auto &blk : *v)
                    for (auto &r : blk.res) rs.push_back(&r);
            temb_total_ = 0;
            std::vector<DParam> members;
            for (DwResnet *r : rs) {
                r->temb_off = temb_total_;
                temb_total_ += r->co;
                members.push_back(r->temb_proj.w);
            }
            const WeightGroup grp = concat_weights(ctx_, members.data(), int(members.size()));
            temb_w_ = grp.p;
            temb_wt_ = grp.wt;
            mh::dev_malloc(&temb_b_, size_t(temb_total_) * sizeof(float));
            for (DwResnet *r : rs)
                HIP_CHECK(hipMemcpyAsync(temb_b_ + r->temb_off, r->temb_proj.b, size_t(r->co) * sizeof(float),
                                         hipMemcpyDeviceToDevice, ctx_.stream));
            if (temb_wt_ == kF16) {
                mh::dev_malloc(&temb_w32_, size_t(temb_total_) * TIME_EMBED * sizeof(float));
                widen_f16(ctx_, temb_w_, int64_t(temb_total_) * TIME_EMBED, temb_w32_);
            }
        }
        lin1_.load(W_, d + ".time_embedding.linear_1", TIME_PROJ, TIME_EMBED, true);
        lin2_.load(W_, d + ".time_embedding.linear_2", TIME_EMBED, TIME_EMBED, true);
        conv_in_.load(W_, d + ".conv_in", 9, CH[0]);
        norm_out_.load(W_, d + ".conv_norm_out", CH[0], RESNET_EPS);
        conv_out_.load(W_, d + ".conv_out", CH[0], 4);
        HIP_CHECK(hipStreamSynchronize(ctx_.stream));
        pool_.recycle(ehs);
        // Sinusoids of every timestep the schedulers use (0..999), computed on the
        // host once, so a step reads its row from HBM with no host copy or sync.
        std::vector<float> sinus(size_t(kSinusSteps + 1) * TIME_PROJ);
        for (int t = 0; t < kSinusSteps; ++t) timestep_sinusoid(t, sinus.data() + size_t(t) * TIME_PROJ);
        mh::dev_malloc(&sinus_dev_, sinus.size() * sizeof(float));
        HIP_CHECK(hipMemcpy(sinus_dev_, sinus.data(), size_t(kSinusSteps) * TIME_PROJ * sizeof(float),
                            hipMemcpyHostToDevice));
    }

    ~UNetDevice() {
        (void)hipStreamSynchronize(ctx_.stream);
        for (auto *v : {&down_, &up_})
            for (auto &b : *v)
                for (auto &a : b.attn) a.release();
        if (sinus_dev_) (void)hipFree(sinus_dev_);
        if (temb_w_) (void)hipFree(temb_w_);
        if (temb_w32_) (void)hipFree(temb_w32_);
        if (temb_b_) (void)hipFree(temb_b_);
    }

    // src/unet/mod.rs:150-243
    void forward(const float *x_dev, int timestep, bool cfg, float *eps_dev, TraceFn trace, void *user) {
        Env e{ctx_, pool_};
        const int b = cfg ? 2 : 1;
        const int br0 = cfg ? 0 : 1;  // branch of item 0: uncond with CFG, cond otherwise
        auto tr = [&](const std::string &name, const DT &t) {
            if (trace) trace(user, name.c_str(), t.p, t.n, t.h, t.w, t.c);
        };
        // time embedding (src/unet/embed.rs:48-66), computed once and tiled to the batch
        const bool in_table = timestep >= 0 && timestep < kSinusSteps;
        const float *sinus = sinus_dev_ + int64_t(in_table ? timestep : kSinusSteps) * TIME_PROJ;
        if (!in_table) {  // outside the table: the spare last row
            float host[TIME_PROJ];
            timestep_sinusoid(timestep, host);
            HIP_CHECK(hipMemcpyAsync(sinus_dev_ + int64_t(kSinusSteps) * TIME_PROJ, host, sizeof(host),
                                     hipMemcpyHostToDevice, ctx_.stream));
            HIP_CHECK(hipStreamSynchronize(ctx_.stream));  // the host array goes out of scope
        }
        float *a1 = pool_.floats(TIME_EMBED);
        lin1_.fwd(e, sinus, 1, a1);
        silu_inplace(ctx_, a1, TIME_EMBED);
        DT temb = pool_.tensor(b, 1, 1, TIME_EMBED);
        lin2_.fwd(e, a1, 1, temb.p);
        pool_.recycle(a1);
        if (trace) {  // the traced tensor holds every item's row
            for (int i = 1; i < b; ++i)
                HIP_CHECK(hipMemcpyAsync(temb.p + int64_t(i) * TIME_EMBED, temb.p, TIME_EMBED * sizeof(float),
                                         hipMemcpyDeviceToDevice, ctx_.stream));
            tr("unet.temb", temb);
        }
        // SiLU(temb) written once per item in one launch
        float *temb_silu = pool_.floats(int64_t(b) * TIME_EMBED);
        silu_tile(ctx_, temb.p, TIME_EMBED, b, temb_silu);
        // all resnets' time projections: tp [b][temb_total_]
        float *tp = pool_.floats(int64_t(b) * temb_total_);
        const bool t32 = temb_w32_ && ctx_.precision == Precision::Exact;
        conv1x1(ctx_, temb_silu, b, TIME_EMBED, t32 ? temb_w32_ : temb_w_, t32 ? kF32 : temb_wt_, temb_total_, temb_b_,
                nullptr, tp);

        // Both CFG branches take the same input, time embedding and weights until
        // the first cross-lambda (the only place the text conditioning enters):
        // conv_in, the first resnet and the first transformer's self-lambda run
        // once, on one item, and are repeated to the batch where needed (the
        // conv_in skip, the resnet's output as the transformer's residual, and h
        // before the cross-lambda). Every kernel computes each item on its own,
        // so this equals the batch-2 run.
        const int bs = cfg ? 1 : b;
        DT input = pool_.tensor(bs, 64, 64, 9);
        HIP_CHECK(hipMemcpyAsync(input.p, x_dev, 64 * 64 * 9 * sizeof(float), hipMemcpyDeviceToDevice, ctx_.stream));
        std::vector<DT> skips;
        DT c0 = conv_in_.fwd(e, input);
        pool_.recycle(input);
        DT c0b;
        if (bs != b) {
            c0b = pool_.tensor(b, c0.h, c0.w, c0.c);
            tile_items(ctx_, c0.p, int64_t(c0.h) * c0.w * c0.c, b, c0b.p);
        } else {
            c0b = c0;
        }
        skips.push_back(c0b);
        tr("unet.conv_in", skips.back());
        for (size_t i = 0; i < down_.size(); ++i) {
            for (size_t j = 0; j < down_[i].res.size(); ++j) {
                const DwResnet &r = down_[i].res[j];
                const bool shared = bs != b && i == 0 && j == 0;
                DT a = r.fwd(e, shared ? c0 : skips.back(), tp + r.temb_off, temb_total_);
                if (shared) pool_.recycle(c0);
                DT ab = a;
                if (shared) {
                    ab = pool_.tensor(b, a.h, a.w, a.c);
                    tile_items(ctx_, a.p, int64_t(a.h) * a.w * a.c, b, ab.p);
                }
                tr("unet.down." + std::to_string(i) + ".res." + std::to_string(j), ab);
                DT h = down_[i].attn[j].fwd(e, a, ab, br0);
                if (shared) pool_.recycle(ab);
                pool_.recycle(a);
                tr("unet.down." + std::to_string(i) + ".attn." + std::to_string(j), h);
                skips.push_back(h);
            }
            if (down_[i].has_sample) skips.push_back(down_[i].sample.fwd(e, skips.back()));
            tr("unet.down." + std::to_string(i) + ".out", skips.back());
        }
        // The last down output is both the hidden state and the first skip: h
        // starts as that same buffer (read twice by the first concat, returned once).
        DT h = skips.back();
        for (size_t i = 0; i < up_.size(); ++i) {
            for (size_t j = 0; j < up_[i].res.size(); ++j) {
                DT skip = skips.back();
                skips.pop_back();
                const DwResnet &r = up_[i].res[j];
                DT a;
                if (!ctx_.tune.up_concat && r.takes_two(h, skip)) {  // [h | skip] read in place
                    a = r.fwd2(e, h, skip, tp + r.temb_off, temb_total_);
                } else {
                    DT cat = pool_.tensor(h.n, h.h, h.w, h.c + skip.c);
                    concat_channels(ctx_, h.p, h.c, skip.p, skip.c, h.px(), cat.p);
                    a = r.fwd(e, cat, tp + r.temb_off, temb_total_);
                    pool_.recycle(cat);
                }
                pool_.recycle(skip);
                if (h.p != skip.p) pool_.recycle(h);
                tr("unet.up." + std::to_string(i) + ".res." + std::to_string(j), a);
                h = up_[i].attn[j].fwd(e, a, br0);
                pool_.recycle(a);
                tr("unet.up." + std::to_string(i) + ".attn." + std::to_string(j), h);
            }
            if (up_[i].has_sample) {
                DT a = up_[i].sample.fwd(e, h);
                pool_.recycle(h);
                h = a;
            }
            tr("unet.up." + std::to_string(i) + ".out", h);
        }
        if (!skips.empty()) fail(kInternal, "skip stack not consumed");
        // norm_out + SiLU applied inside conv_out, which writes the caller's eps buffer.
        float *ss = norm_out_.affine(e, h, nullptr);
        conv_out_.fwd_gn(e, h, ss, nullptr, eps_dev);
        pool_.recycle(ss);
        pool_.recycle(h);
        pool_.recycle(temb);
        pool_.recycle(temb_silu);
        pool_.recycle(tp);
        if (trace) {
            DT o{eps_dev, b, 64, 64, 4};
            tr("unet.out", o);
        }
    }

    size_t weight_bytes() const { return W_.bytes(); }
    size_t pool_bytes() const { return pool_.bytes_held(); }
    void release_scratch() { pool_.release_below(INT64_MAX); }

  private:
    struct Block {
        std::vector<DwResnet> res;
        std::vector<MixTransformer> attn;
        bool has_sample = false;
        Conv3 sample;
    };
    Context &ctx_;
    Pool pool_;
    WeightStore W_;
    std::vector<Block> down_, up_;
    Lin lin1_, lin2_;
    DwConv2d conv_in_, conv_out_;
    GN norm_out_;
    static constexpr int kSinusSteps = 1000;
    float *sinus_dev_ = nullptr;  // [kSinusSteps + 1][TIME_PROJ]
    void *temb_w_ = nullptr;  // [temb_total_][1280]: every resnet's time_emb_proj.weight
    float *temb_w32_ = nullptr;  // its f32 widening when stored f16 (EXACT reads it)
    float *temb_b_ = nullptr;
    WeightType temb_wt_ = kF32;
    int temb_total_ = 0;
};

UNet::UNet(Context &ctx, const NamedTensor *t, int count) : d_(new UNetDevice(ctx, t, count)) {}
UNet::~UNet() = default;
void UNet::forward(const float *x_dev, int timestep, bool cfg, float *eps_dev, TraceFn trace, void *user) {
    d_->forward(x_dev, timestep, cfg, eps_dev, trace, user);
}
size_t UNet::weight_bytes() const { return d_->weight_bytes(); }
size_t UNet::pool_bytes() const { return d_->pool_bytes(); }
void UNet::release_scratch() { d_->release_scratch(); }

}  // namespace mh
