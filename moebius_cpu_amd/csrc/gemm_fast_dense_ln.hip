// Instantiations of the fast-precision GEMM kernel for dense A operands
// entering through a folded LayerNorm (see gemm_dense_ln.hip).
#include "gemm_h16.hpp"

namespace mh {
namespace gemm {

void launch_dense_ln_h16(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi) {
    if (p.lnp_in) {  // row statistics from the producer's partials (f16 folded weights here)
        MH_REQUIRE(wt == kF16, "folded LayerNorm from partials: f16 folded weights in FAST precision");
        launch_tiles_h16<kDense, kProLnPart, true, true>(ctx, p, epi, 1);
    } else if (wt == kF16) {
        launch_tiles_h16<kDense, kProLn, true, true>(ctx, p, epi, 1);
    } else {
        launch_tiles_h16<kDense, kProLn, false, true>(ctx, p, epi, 1);
    }
}

}  // namespace gemm
}  // namespace mh
