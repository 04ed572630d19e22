// Fast-precision GEMM kernel (f16 matrix cores, f32 accumulate) shared by
// gemm_fast_dense.hip and gemm_fast_conv.hip. Same operands, conv gathers,
// epilogues and split-K reduction as the f32 kernel of gemm_kernel.hpp; what
// changes is the arithmetic:
//   - the A operand (f32 activations, or the gathered conv input after the
//     optional GroupNorm prologue) is rounded to f16 (round to nearest even,
//     saturated at +-65504 so an outlier does not become inf) as it is staged
//     in LDS;
//   - f16 weights enter as stored; f32 weights are rounded like A;
//   - products run on v_mfma_f32_32x32x16_f16 (tiles of 64 or more in both
//     dimensions) or v_mfma_f32_16x16x32_f16 (32-wide tiles), summed in f32;
//   - every SiLU (the inverted 1x1's epilogue, the GroupNorm prologue and the
//     residual transform) is fast_silu, from the hardware exp2 and reciprocal:
//     the reference's exp polynomial and IEEE division took 12.6 of 51.6 us in
//     the 8192x1600x320 inverted 1x1.
// Each lane reads eight consecutive K of one A row and of one B column from
// LDS with one 16-byte read per instruction; A and B use the same lane-to-K
// assignment, so the sum covers every K exactly once whatever order the
// matrix unit takes the eight values in.
#pragma once

#include "gemm_kernel.hpp"

namespace mh {
namespace gemm {

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

// Launchers of the fast kernels (gemm_fast_dense.hip, gemm_fast_conv.hip).
void launch_dense_h16(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch, bool vec);
// Dense A stored in f16 (GemmArgs::a holds halves; a_bs, lda in halves), f16
// vector weights, no prologue, no SiLU epilogue; out16: the output in f16 too
// (GemmArgs::out holds halves, rounded as the f16 GEMM rounds f32 operands).
void launch_dense_h16_a16(Context &ctx, GemmArgs &p, int batch, bool out16 = false);
void launch_dense_pro_h16(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi);
void launch_dense_ln_h16(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi);
void launch_conv_h16(Context &ctx, GemmArgs &p, WeightType wt, int mode, bool pro);

namespace {

constexpr int BKH = 64;          // K per LDS stage
constexpr int LDS_H = BKH + 8;   // padded LDS row stride (halves): 144 bytes (+16 and +24: 0.7% and 2.8% slower steps)
constexpr int KCH = BKH / 4;     // 4-element chunks per tile row

template <int M>
struct MfH {
    static constexpr int kAccRegs = M * M / 64;
    static constexpr int kKStep = M == 32 ? 16 : 32;  // K per instruction
    typedef std::conditional_t<M == 32, floatx16, floatx4> Acc;
    static __device__ __forceinline__ Acc mfma(halfx8 a, halfx8 b, const Acc &c) {
        if constexpr (M == 32) return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
        else return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// f32 -> f16, round to nearest even; finite values beyond f16's range saturate
// to +-65504, NaN stays NaN.
__device__ __forceinline__ halfx4 to_h4(floatx4 v) {
    halfx4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float x = __builtin_fabsf(v[e]) > 65504.0f ? __builtin_copysignf(65504.0f, v[e]) : v[e];
        h[e] = static_cast<_Float16>(x);
    }
    return h;
}

// Four consecutive K of A row m, starting at k (k0: first K of the tile, whose
// tap the aligned conv gather shares across the tile).
template <int MODE, int PRO>
__device__ __forceinline__ floatx4 load_a_h(const GemmArgs &p, __amdgpu_buffer_rsrc_t ar, const ConvRow &r, int m,
                                            int k, int k_end, int tky, int tkx, int tci, int k0, int64_t lda = -1) {
    if constexpr (MODE == kDense) {
        const bool ok = m < p.M && k < k_end;
        const floatx4 v = buf_load4(ar, ok ? int((int64_t(m) * (lda < 0 ? p.lda : lda) + k) * 4) : kOob);
        if constexpr (PRO == kProAffine) return dense_prologue<true>(p, r.b, k, ok, v);
        return v;
    } else if constexpr (MODE == kConvAligned || MODE == kConvVec) {
        int ky, kx, c;
        if constexpr (MODE == kConvAligned) {
            ky = tky;
            kx = tkx;
            c = tci + (k - k0);
        } else {
            const int tap = k / p.ci;
            c = k - tap * p.ci;
            ky = tap / 3;
            kx = tap - ky * 3;
        }
        const int64_t src = conv_src(p, r, ky, kx);
        const bool ok = k < k_end && src >= 0;
        floatx4 v = buf_load4(ar, ok ? int((src + c) * 4) : kOob);
        if constexpr (PRO == kProAffine) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = ok ? prologue1<true>(p, r.b, c + e, v[e]) : 0.0f;
        }
        return v;
    } else {  // scalar modes
        return k < k_end ? load_a<MODE, PRO, true>(p, r, m, k, tky, tkx, tci) : zero4();
    }
}

// B chunk as stored: f16 weights with vector rows come as raw halves.
template <bool F16, bool BVEC>
struct BChunk {
    typedef std::conditional_t<F16 && BVEC, halfx4, floatx4> T;
};

template <bool F16, bool BVEC>
__device__ __forceinline__ typename BChunk<F16, BVEC>::T load_b_h(const GemmArgs &p, __amdgpu_buffer_rsrc_t br,
                                                                   int n, int k, int k_end) {
    if constexpr (F16 && BVEC) {
        const bool ok = n < p.N && k < k_end;
        const auto raw =
            __builtin_amdgcn_raw_buffer_load_b64(br, ok ? int((int64_t(n) * p.ldb + k) * 2) : kOob, 0, 0);
        return __builtin_bit_cast(halfx4, raw);
    } else if constexpr (BVEC) {
        return load_b_buf<false>(p, br, n, k, k_end);
    } else {
        return k < k_end ? load_b<F16, false>(p, n, k) : zero4();
    }
}

__device__ __forceinline__ halfx4 as_h4(halfx4 v) { return v; }
__device__ __forceinline__ halfx4 as_h4(floatx4 v) { return to_h4(v); }

// Four consecutive K of an f16 A row (A16: dense operands already rounded by
// their producer, e.g. the Winograd input transform of FAST contexts).
__device__ __forceinline__ halfx4 load_a_f16(const GemmArgs &p, __amdgpu_buffer_rsrc_t ar, int m, int k, int k_end) {
    const bool ok = m < p.M && k < k_end;
    const auto raw = __builtin_amdgcn_raw_buffer_load_b64(ar, ok ? int((int64_t(m) * p.lda + k) * 2) : kOob, 0, 0);
    return __builtin_bit_cast(halfx4, raw);
}

template <int BM, int BN, int MODE, int PRO, bool F16, bool BVEC, int EPI, bool SPLIT, bool A16 = false,
          bool OUT16 = false>
__global__ __launch_bounds__(256) void gemm_h16_kernel(GemmArgs p) {
    static_assert(!A16 || (MODE == kDense && PRO == kProNone), "f16 A operands: dense, no prologue");
    constexpr int MF = mf_for<BM, BN>();
    using MI = MfH<MF>;
    constexpr int FM = BM / 2 / MF, FN = BN / 2 / MF;
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    const TileIdx ti = tile_index(tiles_m, tiles_n);
    if (ti.y) {
        const int64_t bz = ti.y;
        p.a = reinterpret_cast<const float *>(reinterpret_cast<const char *>(p.a) + bz * p.a_bs * (A16 ? 2 : 4));
        p.b = static_cast<const char *>(p.b) + bz * p.b_bs * (F16 ? 2 : 4);
        p.out += bz * p.c_bs;
        if (p.res) p.res += bz * p.c_bs;
    }
    constexpr int A_LD = BM * KCH / 256, B_LD = BN * KCH / 256;
    constexpr int SMEM_H = 2 * (BM + BN) * LDS_H;  // halves
    static_assert(BM * (BN + 8) * 2 <= SMEM_H && SMEM_H >= 2 * 2048,
                  "C tile and GroupNorm sums must fit in the staging space");
    __shared__ __align__(16) _Float16 smem[SMEM_H];
    _Float16(*As)[BM * LDS_H] = reinterpret_cast<_Float16(*)[BM * LDS_H]>(smem);
    _Float16(*Bs)[BN * LDS_H] = reinterpret_cast<_Float16(*)[BN * LDS_H]>(smem + 2 * BM * LDS_H);

    const int m0 = ti.tm * BM, n0 = ti.tn * BN;
    const int k_begin = SPLIT ? ti.z * p.k_split : 0;
    const int k_end = SPLIT ? min(p.K, k_begin + p.k_split) : p.K;
    const int ktiles = (k_end - k_begin + BKH - 1) / BKH;

    const int tid = threadIdx.x;
    const int lrow = tid >> 4, lc = tid & 15;  // load slot: row within a 16-row pass, 4-element chunk

    ConvRow crow[A_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        if (MODE >= kConvAligned) crow[i] = conv_row(p, m0 + lrow + 16 * i);
        else if (PRO == kProAffine) crow[i] = ConvRow{min(m0 + lrow + 16 * i, p.M - 1) / p.pro_rows, 0, 0, true};
        else crow[i] = ConvRow{0, 0, 0, true};
    }

    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.a, p.a_bytes);
    const __amdgpu_buffer_rsrc_t a2_rsrc = make_rsrc(p.a2 ? p.a2 : p.a, p.a2 ? p.a2_bytes : p.a_bytes);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(p.b, p.b_bytes);
    using BT = typename BChunk<F16, BVEC>::T;
    using AT = std::conditional_t<A16, halfx4, floatx4>;
    AT ra0[A_LD], ra1[A_LD];
    BT rb0[B_LD], rb1[B_LD];
    double ln_s1[A_LD], ln_s2[A_LD];  // kProLn: row sums of the f32 values as loaded (before rounding)
#pragma unroll
    for (int i = 0; i < A_LD; ++i) ln_s1[i] = ln_s2[i] = 0.0;
    auto fetch = [&](int kt, AT (&ra)[A_LD], BT (&rb)[B_LD]) {
        const int k0 = k_begin + kt * BKH;
        int tky = 0, tkx = 0, tci = 0;
        if (MODE == kConvAligned) {
            const int tap = k0 / p.ci;
            tci = k0 - tap * p.ci;
            tky = tap / 3;
            tkx = tap - tky * 3;
        }
        const int k = k0 + lc * 4;
        // a tile past ka reads the second operand (whole tiles: ka % BKH == 0)
        const bool sec = MODE == kDense && p.a2 && k0 >= p.ka;
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            if constexpr (A16)
                ra[i] = load_a_f16(p, a_rsrc, m0 + lrow + 16 * i, k, k_end);
            else
                ra[i] = sec ? load_a_h<MODE, PRO>(p, a2_rsrc, crow[i], m0 + lrow + 16 * i, k - p.ka, k_end - p.ka, tky,
                                                  tkx, tci, k0 - p.ka, p.lda2)
                            : load_a_h<MODE, PRO>(p, a_rsrc, crow[i], m0 + lrow + 16 * i, k, k_end, tky, tkx, tci, k0);
        }
        if constexpr (PRO == kProLn && !A16) {
#pragma unroll
            for (int i = 0; i < A_LD; ++i) {
                const double a0 = ra[i][0], a1 = ra[i][1], a2 = ra[i][2], a3 = ra[i][3];
                ln_s1[i] += (a0 + a1) + (a2 + a3);
                ln_s2[i] += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
            }
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) rb[i] = load_b_h<F16, BVEC>(p, b_rsrc, n0 + lrow + 16 * i, k, k_end);
    };
    auto stash = [&](int buf, const AT (&ra)[A_LD], const BT (&rb)[B_LD]) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i)
            *reinterpret_cast<halfx4 *>(As[buf] + (lrow + 16 * i) * LDS_H + lc * 4) = as_h4(ra[i]);
#pragma unroll
        for (int i = 0; i < B_LD; ++i)
            *reinterpret_cast<halfx4 *>(Bs[buf] + (lrow + 16 * i) * LDS_H + lc * 4) = as_h4(rb[i]);
    };

    typename MI::Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < MI::kAccRegs; ++v) acc[i][j][v] = 0.f;

    // Lane l reads eight consecutive K at row l % MF, K offset 8 * (l / MF).
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int a_off = (wm * (BM / 2) + (lane % MF)) * LDS_H + (lane / MF) * 8;
    const int b_off = (wn * (BN / 2) + (lane % MF)) * LDS_H + (lane / MF) * 8;
    auto compute = [&](int buf) {
        const _Float16 *as_w = As[buf] + a_off;
        const _Float16 *bs_w = Bs[buf] + b_off;
#pragma unroll
        for (int kk = 0; kk < BKH; kk += MI::kKStep) {
            halfx8 a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = *reinterpret_cast<const halfx8 *>(as_w + i * MF * LDS_H + kk);
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = *reinterpret_cast<const halfx8 *>(bs_w + j * MF * LDS_H + kk);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = MI::mfma(a[i], b[j], acc[i][j]);
        }
    };

    // The same two-register-stage / two-LDS-stage pipeline as gemm_f32_kernel.
    fetch(0, ra0, rb0);
    fetch(1, ra1, rb1);
    stash(0, ra0, rb0);
    fetch(2, ra0, rb0);
    __syncthreads();
    int kt = 0;
    for (; kt + 3 < ktiles; kt += 2) {
        compute(0);
        stash(1, ra1, rb1);
        fetch(kt + 3, ra1, rb1);
        __syncthreads();
        compute(1);
        stash(0, ra0, rb0);
        fetch(kt + 4, ra0, rb0);
        __syncthreads();
    }
    compute(0);
    if (kt + 1 < ktiles) {
        stash(1, ra1, rb1);
        __syncthreads();
        compute(1);
        if (kt + 2 < ktiles) {
            stash(0, ra0, rb0);
            __syncthreads();
            compute(0);
        }
    }
    __shared__ float ln_st[PRO >= kProLn ? 2 * BM : 1];
    if constexpr (PRO == kProLn) ln_row_stats<A_LD, 16, KCH, BM>(p, ln_s1, ln_s2, lrow, lc, ln_st);
    if constexpr (PRO == kProLnPart) ln_stats_from_parts<BM, 256>(p, m0, ln_st);
    __syncthreads();
    write_tile<BM, BN, 2, 2, 1, MF, EPI, SPLIT, true, OUT16>(p, reinterpret_cast<float *>(smem), acc, m0, n0, ti.z,
                                                PRO >= kProLn ? ln_st : nullptr);
}

// Tile shape and K split of the fast kernel, from sweeps of every (tile,
// split) on MI355X over the UNet's GEMM shapes. Its products run at 16x the
// f32 rate, so these GEMMs are bound by operand traffic and per-workgroup
// latency:
//  - implicit-GEMM convs: 64x64 tiles, K split up to 4 ways while each split
//    keeps 10 or more K tiles (every UNet 3x3 conv: 15-30% faster than unsplit);
//  - a few rows (the time-embedding linears): 32x32;
//  - long K (25+ tiles) on small grids: 64x64 with K split up to 4 ways;
//  - batched products of 512+ rows on 32 CUs or fewer per item (the 16-plane
//    Winograd GEMMs of the upsample convs, 16 x 512x1280x1280 and 16 x
//    2048x640x640): 128x128, half the operand traffic of 64x64 (140 and 129 ->
//    125 us per launch, FAST step 5.042 -> 5.021 ms);
//  - otherwise 64x64, or 32x32 when 64x64 leaves a quarter of the CUs idle.
// (The wide MixFFN inverted 1x1s, 2048x3200x640 and 512x6400x1280, had 128x128
// tiles from those sweeps; timed in the UNet step, each with every tiling in
// turn, 64x64 is faster: the FAST step 13 and 25 us shorter.)
inline Plan plan_h16(int M, int N, int K, int cus, bool dense) {
    const int ktiles = int(ceil_div(K, BKH));
    const int64_t t64 = ceil_div(M, 64) * ceil_div(N, 64);
    auto plan = [&](int bm, int want) {
        want = std::max(1, std::min(want, ktiles));
        const int per = int(ceil_div(ktiles, want));
        const int splits = int(ceil_div(ktiles, per));
        return Plan{bm, bm, splits, splits > 1 ? per * BKH : K};
    };
    if (!dense) return plan(64, t64 >= 2 * int64_t(cus) ? 1 : std::min(4, ktiles / 10));
    if (M <= 32) return plan(32, 1);
    if (cus <= 32 && M >= 512 && N >= 512 && K >= 512) return plan(128, 1);  // batched planes
    if (ktiles >= 25 && t64 < 2 * int64_t(cus)) return plan(64, int(std::min<int64_t>(4, ceil_div(2 * cus, t64))));
    if (4 * t64 < 3 * int64_t(cus)) return plan(32, 1);
    return plan(64, 1);
}

template <int BM, int BN, int MODE, int PRO, bool F16, bool BVEC>
void launch_cfg_h16(Context &ctx, GemmArgs &p, const Plan &pl, GemmEpilogue epi, int batch) {
    const unsigned tiles = unsigned(ceil_div(p.M, BM) * ceil_div(p.N, BN));
    log_gemm(ctx, "f16", p, BM, BN, pl.splits, MODE, PRO, F16, epi, batch);
    const GemmTimer timer(ctx, "f16", p, BM, BN, 2, 2, 1, pl.splits, MODE, batch);
    if (pl.splits > 1) {
        const size_t bytes = size_t(pl.splits) * p.M * p.N * sizeof(float);
        p.partial = static_cast<float *>(ctx.ws.get(bytes, ctx.stream));
        p.k_split = pl.k_split;
        p.vec_out = (p.N & 3) == 0 && (reinterpret_cast<uintptr_t>(p.partial) & 15) == 0;
        gn_partials_plan(p, BM, BN, pl.splits, batch);
        ln_partials_plan(p, BN, pl.splits, batch);
        dim3 grid(tiles, 1, pl.splits);
        gemm_h16_kernel<BM, BN, MODE, PRO, F16, BVEC, 0, true><<<grid, 256, 0, ctx.stream>>>(p);
        MH_LAUNCH_CHECK();
        const int64_t total = int64_t(p.M) * p.N;
        if (reduce_vec_ok(p)) {
            const unsigned rb = unsigned(std::min<int64_t>(ceil_div(total / 4, 256), 8192));
            if (epi == GemmEpilogue::Silu)
                splitk_reduce_kernel<1, true, true><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
            else
                splitk_reduce_kernel<0, true, true><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
        } else {
            const unsigned rb = unsigned(std::min<int64_t>(ceil_div(total, 256), 8192));
            if (epi == GemmEpilogue::Silu)
                splitk_reduce_kernel<1, false, true><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
            else
                splitk_reduce_kernel<0, false, true><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
        }
    } else {
        p.k_split = p.K;
        p.vec_out = out_vec_ok(p, BM);
        gn_partials_plan(p, BM, BN, 1, batch);
        ln_partials_plan(p, BN, 1, batch);
        const dim3 grid(tiles, unsigned(batch));
        if constexpr (MODE <= kDenseScalar) {
            if (epi == GemmEpilogue::Silu) {
                gemm_h16_kernel<BM, BN, MODE, PRO, F16, BVEC, 1, false><<<grid, 256, 0, ctx.stream>>>(p);
                MH_LAUNCH_CHECK();
                return;
            }
        } else {
            MH_REQUIRE(epi == GemmEpilogue::None, "conv GEMM: SiLU epilogue not available");
        }
        gemm_h16_kernel<BM, BN, MODE, PRO, F16, BVEC, 0, false><<<grid, 256, 0, ctx.stream>>>(p);
    }
    MH_LAUNCH_CHECK();
}

template <int MODE, int PRO, bool F16, bool BVEC>
void launch_tiles_h16(Context &ctx, GemmArgs &p, GemmEpilogue epi, int batch) {
    Plan pl = plan_h16(p.M, p.N, p.K, int(ceil_div(ctx.cu_count, batch)), MODE <= kDenseScalar);
    // The context's gemm_plan tuning forces the tiling, as for the f32 kernel.
    ShapePlan fp;
    if (forced_plan(ctx.tune, p.M, p.N, p.K, fp)) {
        const int bm = fp.bm, bn = fp.bn, sp = fp.splits;
        if (bm == bn && (bm == 32 || bm == 64 || bm == 128)) {
            const int ktiles = int(ceil_div(p.K, BKH));
            const int per = int(ceil_div(ktiles, sp));
            pl = Plan{bm, bn, int(ceil_div(ktiles, per)), per * BKH};
        }
    }
    if (batch > 1 || PRO >= kProLn) pl.splits = 1;  // the folded LayerNorm needs whole rows of K
    if (pl.splits == 1) pl.k_split = p.K;
    if constexpr (MODE <= kDenseScalar) {
        if (pl.bm == 32) {
            launch_cfg_h16<32, 32, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
            return;
        }
    }
    if (pl.bm == 128)
        launch_cfg_h16<128, 128, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
    else
        launch_cfg_h16<64, 64, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
}

// f16 A operands (launch_dense_h16_a16): the planner's tiling and K split, as
// launch_cfg_h16 runs them for f32 A.
template <int BM, int BN, bool OUT16>
void launch_a16_cfg(Context &ctx, GemmArgs &p, const Plan &pl, int batch) {
    const unsigned tiles = unsigned(ceil_div(p.M, BM) * ceil_div(p.N, BN));
    log_gemm(ctx, "f16a", p, BM, BN, pl.splits, kDense, kProNone, true, GemmEpilogue::None, batch);
    const GemmTimer timer(ctx, "f16a", p, BM, BN, 2, 2, 1, pl.splits, kDense, batch);
    if (pl.splits > 1) {
        p.partial = static_cast<float *>(ctx.ws.get(size_t(pl.splits) * p.M * p.N * sizeof(float), ctx.stream));
        p.k_split = pl.k_split;
        p.vec_out = (p.N & 3) == 0 && (reinterpret_cast<uintptr_t>(p.partial) & 15) == 0;
        gn_partials_plan(p, BM, BN, pl.splits, batch);
        ln_partials_plan(p, BN, pl.splits, batch);
        MH_REQUIRE(!OUT16 || (p.vec_out == 1 && reduce_vec_ok(p)), "f16 GEMM output: four columns at a time");
        gemm_h16_kernel<BM, BN, kDense, kProNone, true, true, 0, true, true>
            <<<dim3(tiles, 1, pl.splits), 256, 0, ctx.stream>>>(p);
        MH_LAUNCH_CHECK();
        const int64_t total = int64_t(p.M) * p.N;
        if (reduce_vec_ok(p))
            splitk_reduce_kernel<0, true, true, OUT16>
                <<<unsigned(std::min<int64_t>(ceil_div(total / 4, 256), 8192)), 256, 0, ctx.stream>>>(p, pl.splits);
        else if constexpr (!OUT16)
            splitk_reduce_kernel<0, false, true>
                <<<unsigned(std::min<int64_t>(ceil_div(total, 256), 8192)), 256, 0, ctx.stream>>>(p, pl.splits);
        MH_LAUNCH_CHECK();
        return;
    }
    p.k_split = p.K;
    p.vec_out = out_vec_ok(p, BM);
    MH_REQUIRE(!OUT16 || p.vec_out == 1, "f16 GEMM output: four columns at a time");
    gn_partials_plan(p, BM, BN, 1, batch);
    ln_partials_plan(p, BN, 1, batch);
    const dim3 grid(tiles, unsigned(batch));
    gemm_h16_kernel<BM, BN, kDense, kProNone, true, true, 0, false, true, OUT16><<<grid, 256, 0, ctx.stream>>>(p);
    MH_LAUNCH_CHECK();
}

template <int MODE, int PRO>
void launch_b_h16(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch = 1) {
    const int esz = wt == kF16 ? 2 : 4;
    const bool bvec = p.K % 4 == 0 && p.ldb % 4 == 0 && (reinterpret_cast<uintptr_t>(p.b) % (4 * esz)) == 0 &&
                      (batch == 1 || p.b_bs % 4 == 0);
    if constexpr (MODE == kConvAligned || MODE == kConvVec) {
        MH_REQUIRE(bvec, "conv GEMM: weight rows must be 4-element aligned for the vector gather");
        if (wt == kF16) launch_tiles_h16<MODE, PRO, true, true>(ctx, p, epi, batch);
        else launch_tiles_h16<MODE, PRO, false, true>(ctx, p, epi, batch);
    } else if constexpr (MODE == kConvScalar) {
        if (wt == kF16) launch_tiles_h16<MODE, PRO, true, false>(ctx, p, epi, batch);
        else launch_tiles_h16<MODE, PRO, false, false>(ctx, p, epi, batch);
    } else {
        if (wt == kF16) {
            if (bvec) launch_tiles_h16<MODE, PRO, true, true>(ctx, p, epi, batch);
            else launch_tiles_h16<MODE, PRO, true, false>(ctx, p, epi, batch);
        } else {
            if (bvec) launch_tiles_h16<MODE, PRO, false, true>(ctx, p, epi, batch);
            else launch_tiles_h16<MODE, PRO, false, false>(ctx, p, epi, batch);
        }
    }
}

}  // namespace
}  // namespace gemm
}  // namespace mh
