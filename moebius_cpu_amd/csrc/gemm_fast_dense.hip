// Instantiations of the fast-precision (f16 matrix core) GEMM kernel for dense,
// K-contiguous A operands (1x1 convs, linear layers, batched products).
#include "gemm_h16.hpp"

namespace mh {
namespace gemm {

void launch_dense_h16(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch, bool vec) {
    if (vec)
        launch_b_h16<kDense, false>(ctx, p, wt, epi, batch);
    else
        launch_b_h16<kDenseScalar, false>(ctx, p, wt, epi, batch);
}

}  // namespace gemm
}  // namespace mh
