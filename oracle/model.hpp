// Shared pieces of the oracle's model restatements (unet.cpp, vae.cpp): an
// NHWC f32 tensor, the named-weight table and the engine layers both models
// use. Test infrastructure only: see oracle.h.
#pragma once
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "oracle.h"

namespace orc_model {

constexpr int GROUPS = 32;  // src/config.rs: every GroupNorm has 32 groups

using Vec = std::vector<float>;

struct T4 {
    Vec d;
    int64_t n = 0, h = 0, w = 0, c = 0;
    void set(int64_t n_, int64_t h_, int64_t w_, int64_t c_) {
        n = n_, h = h_, w = w_, c = c_;
        d.resize(size_t(n * h * w * c));
    }
    int64_t px() const { return n * h * w; }
    float *p() { return d.data(); }
    const float *p() const { return d.data(); }
};

struct Weights {
    std::map<std::string, std::pair<const float *, int64_t>> m;
    const float *get(const std::string &name, int64_t numel) const {
        auto it = m.find(name);
        if (it == m.end()) throw std::runtime_error("missing tensor " + name);
        if (it->second.second != numel)
            throw std::runtime_error("tensor " + name + " has " + std::to_string(it->second.second) +
                                     " values, expected " + std::to_string(numel));
        return it->second.first;
    }
    bool has(const std::string &name) const { return m.count(name) != 0; }
};

struct Lin {  // Conv1x1 (src/engine/conv.rs:28-55)
    int ci = 0, co = 0;
    const float *w = nullptr, *b = nullptr;
    void load(const Weights &W, const std::string &p, int ci_, int co_, bool bias) {
        ci = ci_, co = co_;
        w = W.get(p + ".weight", int64_t(ci) * co);
        b = bias ? W.get(p + ".bias", co) : nullptr;
    }
    void fwd(const float *x, int64_t px, float *out, const float *res = nullptr) const {
        orc_conv1x1(x, px, ci, w, co, b, res, out);
    }
    void fwd(const T4 &x, T4 &out, const T4 *res = nullptr) const {
        out.set(x.n, x.h, x.w, co);
        fwd(x.p(), x.px(), out.p(), res ? res->p() : nullptr);
    }
};

struct GN {  // GroupNorm (src/engine/norm.rs:22-105)
    int c = 0;
    float eps = 0;
    const float *g = nullptr, *b = nullptr;
    void load(const Weights &W, const std::string &p, int c_, float eps_) {
        c = c_, eps = eps_;
        g = W.get(p + ".weight", c);
        b = W.get(p + ".bias", c);
    }
    void fwd(const T4 &x, const float *add, bool silu, T4 &out) const {
        out.set(x.n, x.h, x.w, x.c);
        orc_group_norm_forward(x.p(), x.n, x.h, x.w, x.c, GROUPS, eps, g, b, add, silu ? 1 : 0, out.p());
    }
    // The statistics pass only (norm.rs:57-105): per item and channel scale, shift.
    void affine(const T4 &x, Vec &scale, Vec &shift) const {
        scale.resize(size_t(x.n * x.c));
        shift.resize(size_t(x.n * x.c));
        orc_group_norm_affine(x.p(), x.n, x.h, x.w, x.c, GROUPS, eps, g, b, nullptr, scale.data(), shift.data());
    }
};


}  // namespace orc_model
