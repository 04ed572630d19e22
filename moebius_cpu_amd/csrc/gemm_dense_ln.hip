// Instantiations of the f32 GEMM kernel for dense A operands entering through a
// folded LayerNorm (kProLn, or kProLnPart with the row statistics from the
// producer's partials): the transformers' q | k | v projection of
// LayerNorm 1 and MixFFN inverted 1x1 of LayerNorm 3, which read the block's
// hidden state itself, so the normalised tensor is never written.
#include "gemm_kernel.hpp"

namespace mh {
namespace gemm {

void launch_dense_ln(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi) {
    if (p.lnp_in) {  // row statistics from the producer's partials (the folded weights are f32 here)
        MH_REQUIRE(wt == kF32, "folded LayerNorm from partials: f32 folded weights");
        launch_tiles<kDense, kProLnPart, false, true>(ctx, p, epi, 1);
    } else if (wt == kF16) {
        launch_tiles<kDense, kProLn, true, true>(ctx, p, epi, 1);
    } else {
        launch_tiles<kDense, kProLn, false, true>(ctx, p, epi, 1);
    }
}

}  // namespace gemm
}  // namespace mh
