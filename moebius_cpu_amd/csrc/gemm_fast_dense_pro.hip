// Instantiations of the fast-precision GEMM kernel for dense A operands read
// through the GroupNorm prologue (see gemm_dense_pro.hip).
#include "gemm_h16.hpp"

namespace mh {
namespace gemm {

void launch_dense_pro_h16(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi) {
    if (wt == kF16) launch_tiles_h16<kDense, true, true, true>(ctx, p, epi, 1);
    else launch_tiles_h16<kDense, true, false, true>(ctx, p, epi, 1);
}

}  // namespace gemm
}  // namespace mh
