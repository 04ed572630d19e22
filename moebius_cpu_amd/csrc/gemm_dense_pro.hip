// Instantiations of the f32 GEMM kernel for dense A operands read through the
// GroupNorm prologue: a 1x1 conv of GroupNorm(x) that reads x, so the
// normalised tensor is never written (the transformers' proj_in).
#include "gemm_kernel.hpp"

namespace mh {
namespace gemm {

void launch_dense_pro(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi) {
    if (wt == kF16) launch_tiles<kDense, true, true, true>(ctx, p, epi, 1);
    else launch_tiles<kDense, true, false, true>(ctx, p, epi, 1);
}

}  // namespace gemm
}  // namespace mh
