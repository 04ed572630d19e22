// Instantiations of the GEMM kernel for dense, K-contiguous A operands (1x1
// convs, linear layers, the lambda layers' batched products).
#include "gemm_kernel.hpp"

namespace mh {
namespace gemm {

void launch_dense(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch, bool vec) {
    if (vec)
        launch_b<kDense, false>(ctx, p, wt, epi, batch);
    else
        launch_b<kDenseScalar, false>(ctx, p, wt, epi, batch);
}

}  // namespace gemm
}  // namespace mh
