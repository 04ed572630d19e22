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

void launch_dense_h16_a16(Context &ctx, GemmArgs &p, int batch, bool out16) {
    Plan pl = plan_h16(p.M, p.N, p.K, int(ceil_div(ctx.cu_count, batch)), true);
    if (batch > 1) pl.splits = 1;
    if (pl.splits == 1) pl.k_split = p.K;
    auto go = [&](auto o16) {
        constexpr bool O = decltype(o16)::value;
        if (pl.bm == 32) launch_a16_cfg<32, 32, O>(ctx, p, pl, batch);
        else if (pl.bm == 128) launch_a16_cfg<128, 128, O>(ctx, p, pl, batch);
        else launch_a16_cfg<64, 64, O>(ctx, p, pl, batch);
    };
    if (out16) go(std::true_type{});
    else go(std::false_type{});
}

}  // namespace gemm
}  // namespace mh
