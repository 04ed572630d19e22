// The Moebius UNet on the device (src/unet): weights resident in HBM, every
// activation of a denoise step in the pool, kernels queued on the context
// stream. Host C++ mirror of src/unet/{mod,blocks,transformer,lambda,embed}.rs.
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"
#include "pool.hpp"

namespace mh {

// One converter tensor handed in by the host (tools/convert_weights.py layouts).
struct NamedTensor {
    const char *name;
    const void *data;  // host memory
    uint32_t dtype;    // kF32 / kF16
    uint64_t numel;
};

// Device copy of a tensor in its stored precision (src/engine/param.rs:14-17).
// An f16-stored GEMM weight also has its f32 widening (p32), which EXACT
// arithmetic reads: the same products the f16-weight kernels form after
// widening each value as they load it, without the conversion in the loop
// and with the f32 kernels' tilings.
struct DParam {
    const void *p = nullptr;
    WeightType wt = kF32;
    int64_t numel = 0;
    const float *p32 = nullptr;
    const float *f() const { return static_cast<const float *>(p); }
    // The copy the context's precision reads.
    DParam at(const Context &ctx) const {
        if (p32 && ctx.precision == Precision::Exact) return DParam{p32, kF32, numel, nullptr};
        return *this;
    }
};

// Uploads tensors into one HBM block; GEMM weights keep their dtype, every
// other tensor is stored f32.
class WeightStore {
  public:
    // widen_f16: also keep the f32 widening of every f16-stored tensor (DParam::p32),
    // for a model whose EXACT arithmetic reads its GEMM weights through DParam::at.
    WeightStore(Context &ctx, const NamedTensor *t, int count, bool widen_f16);
    ~WeightStore();
    WeightStore(const WeightStore &) = delete;
    WeightStore &operator=(const WeightStore &) = delete;
    // Shape-checked lookup (by element count); gemm: may be f16.
    DParam get(const std::string &name, int64_t numel, bool gemm) const;
    const float *host_f32(const std::string &name, int64_t numel, std::vector<float> &scratch) const;
    // Winograd kernel U = G g G^T [16][co][ci] (f32) of a 3x3 conv weight
    // [co][3][3][ci], built on the device once and owned by the store.
    const float *winograd_kernel(const DParam &w, int co, int ci) const;
    // u (from winograd_kernel) in the one-kernel Winograd path's order.
    const float *winograd_kernel_fused(const float *u, int co, int ci) const;
    // u rounded to f16 as the FAST plane GEMM rounds it on every load, for FAST contexts.
    const void *winograd_kernel_f16(const float *u, int co, int ci) const;
    size_t bytes() const { return bytes_ + derived_bytes_; }

  private:
    struct Entry {
        DParam d;
        const void *host;
        uint32_t host_dtype;
    };
    Context &ctx_;
    std::map<std::string, Entry> m_;
    void *block_ = nullptr;
    size_t bytes_ = 0;
    mutable std::vector<void *> derived_;
    mutable size_t derived_bytes_ = 0;
};

// Several GEMM weights [rows_i][cols] stacked into one [sum rows_i][cols]
// matrix, so one GEMM writes all their outputs (self-lambda q | k | v, every
// resnet's time projection, the VAE attention's q | k | v). Stored f16 when every
// member is f16; otherwise f32, with the f16 members widened exactly: the
// converter keeps a GEMM weight f32 when its f16 copy would overflow
// (tools/convert_weights.py:27-30), and the reference reads each tensor in its
// own stored precision (src/engine/param.rs:14-59). The caller frees `p`.
struct WeightGroup {
    void *p = nullptr;
    WeightType wt = kF32;
};
WeightGroup concat_weights(Context &ctx, const DParam *members, int count);

using TraceFn = void (*)(void *user, const char *name, const float *dev, int n, int h, int w, int c);

class UNetDevice;

class UNet {
  public:
    UNet(Context &ctx, const NamedTensor *t, int count);
    ~UNet();
    // x_dev [1,64,64,9] -> eps_dev [b,64,64,4]; b = 2 with CFG (branches uncond, cond), else 1.
    void forward(const float *x_dev, int timestep, bool cfg, float *eps_dev, TraceFn trace = nullptr,
                 void *user = nullptr);
    size_t weight_bytes() const;
    size_t pool_bytes() const;
    // Frees the pool's idle buffers (Scratch::release_below(usize::MAX), src/engine/mod.rs:87-91).
    void release_scratch();

  private:
    std::unique_ptr<UNetDevice> d_;
};

// src/unet/embed.rs:21-30 (host, libm), shared with the C ABI tests.
void timestep_sinusoid(int t, float *out /* [320] */);

}  // namespace mh
