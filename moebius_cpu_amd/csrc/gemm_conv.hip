// Instantiations of the GEMM kernel for the 3x3 conv's gathered A operand,
// with and without the GroupNorm prologue.
#include "gemm_kernel.hpp"

namespace mh {
namespace gemm {

void launch_conv(Context &ctx, GemmArgs &p, WeightType wt, int mode, bool pro) {
    switch (mode) {
        case kConvAligned:
            if (pro) launch_b<kConvAligned, true>(ctx, p, wt, GemmEpilogue::None);
            else launch_b<kConvAligned, false>(ctx, p, wt, GemmEpilogue::None);
            break;
        case kConvVec:
            if (pro) launch_b<kConvVec, true>(ctx, p, wt, GemmEpilogue::None);
            else launch_b<kConvVec, false>(ctx, p, wt, GemmEpilogue::None);
            break;
        default:
            if (pro) launch_b<kConvScalar, true>(ctx, p, wt, GemmEpilogue::None);
            else launch_b<kConvScalar, false>(ctx, p, wt, GemmEpilogue::None);
    }
}

}  // namespace gemm
}  // namespace mh
