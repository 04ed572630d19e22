// Instantiations of the fast-precision (f16 matrix core) GEMM kernel for the
// 3x3 conv's gathered A operand, with and without the GroupNorm prologue.
#include "gemm_h16.hpp"

namespace mh {
namespace gemm {

void launch_conv_h16(Context &ctx, GemmArgs &p, WeightType wt, int mode, bool pro) {
    // One tap per 64-wide K tile needs Ci % 64 == 0; otherwise the gather finds
    // the tap per 4-element chunk.
    if (mode == kConvAligned && p.ci % BKH != 0) mode = kConvVec;
    switch (mode) {
        case kConvAligned:
            if (pro) launch_b_h16<kConvAligned, true>(ctx, p, wt, GemmEpilogue::None);
            else launch_b_h16<kConvAligned, false>(ctx, p, wt, GemmEpilogue::None);
            break;
        case kConvVec:
            if (pro) launch_b_h16<kConvVec, true>(ctx, p, wt, GemmEpilogue::None);
            else launch_b_h16<kConvVec, false>(ctx, p, wt, GemmEpilogue::None);
            break;
        default:
            if (pro) launch_b_h16<kConvScalar, true>(ctx, p, wt, GemmEpilogue::None);
            else launch_b_h16<kConvScalar, false>(ctx, p, wt, GemmEpilogue::None);
    }
}

}  // namespace gemm
}  // namespace mh
