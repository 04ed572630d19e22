// GEMM-shaped convolutions on gfx950 matrix cores (f32 MFMA, f32 accumulate).
//
//   1x1 conv  (src/engine/conv.rs:38-55):  out[P x Co] = x[P x Ci] . W[Co x Ci]^T
//   3x3 conv  (src/engine/conv.rs:83-165): implicit GEMM, M = output pixels,
//             N = Co, K = 9*Ci in the weight's [ky][kx][ci] order; the A tile
//             is gathered straight from the NHWC input (zero outside the image,
//             nearest-2x upsample as a >>1 of the source index, any stride and
//             [top,left,bottom,right] padding), optionally through the
//             GroupNorm affine (+SiLU) prologue of src/engine/norm.rs:33-37.
//
// Both operands are K-contiguous (NHWC activations; [Co][.. Ci] weights), so
// one "NT" kernel serves every shape. Tiles: BM x BN x 32 per 256-thread
// workgroup, four 64-wide waves in a 2x2 arrangement, each owning
// (BM/2) x (BN/2) of the output as 32x32 blocks of v_mfma_f32_32x32x2f32.
// Each lane reads a float4 along K from LDS for A and for B and issues four
// MFMAs, one per component: instruction t pairs lane-group g = lane/32 with
// k = kk + 4g + t, so one float4 read feeds four matrix instructions and the
// pairs cover kk..kk+7. The K order of the sum therefore differs from the
// CPU engine's (the reference uses Winograd for stride-1 convs); results
// agree to f32 rounding.
//
// Small grids (MI355X has 256 CUs) split K across workgroups; the partial
// tiles are summed in a fixed order by a reduction kernel that also applies
// bias / residual / SiLU, so results are deterministic run to run.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstring>

#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 32;          // K per LDS stage
constexpr int LDS_S = BK + 4;   // padded LDS row stride (floats): conflict-free b128 reads
constexpr int K4 = BK / 4;      // float4 per tile row

enum AMode : int {
    kDense = 0,      // A[m][k] row-major with leading dimension lda, K % 4 == 0
    kDenseScalar,    // same, any K
    kConvAligned,    // conv gather, Ci % BK == 0: one tap per K tile
    kConvVec,        // conv gather, Ci % 4 == 0: one tap per float4
    kConvScalar,     // conv gather, any Ci
};

struct GemmArgs {
    const float *a;
    int64_t lda;
    int M, N, K;
    // conv geometry
    int cn, ch, cw, ci, ho, wo, stride, pad_t, pad_l, up;
    const float *psc, *psh;
    int psilu;
    // B operand: [N][ldb]
    const void *b;
    int64_t ldb;
    // epilogue
    const float *bias, *res;
    float *out;
    int64_t ldc;
    // split K
    int k_split;      // K per split (multiple of BK)
    float *partial;   // [splits][M][N] when splitting
    // batch (grid y): element offsets of item z's A, B and output/residual
    int64_t a_bs, b_bs, c_bs;
};

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// Per-row conv geometry, fixed over the K loop.
struct ConvRow {
    int b, iy0, ix0;
    bool valid;
};

__device__ __forceinline__ ConvRow conv_row(const GemmArgs &p, int m) {
    ConvRow r;
    r.valid = m < p.M;
    const int mm = r.valid ? m : 0;
    const int hw = p.ho * p.wo;
    r.b = mm / hw;
    const int rem = mm - r.b * hw;
    const int oy = rem / p.wo, ox = rem - (rem / p.wo) * p.wo;
    r.iy0 = oy * p.stride - p.pad_t;
    r.ix0 = ox * p.stride - p.pad_l;
    return r;
}

// Source element offset of (row, tap) or -1 outside the (upsampled) image.
__device__ __forceinline__ int64_t conv_src(const GemmArgs &p, const ConvRow &r, int ky, int kx) {
    const int iy = r.iy0 + ky, ix = r.ix0 + kx;
    const int hi = p.ch << p.up, wi = p.cw << p.up;
    if (!r.valid || iy < 0 || ix < 0 || iy >= hi || ix >= wi) return -1;
    return ((int64_t(r.b) * p.ch + (iy >> p.up)) * p.cw + (ix >> p.up)) * p.ci;
}

__device__ __forceinline__ float prologue1(const GemmArgs &p, int b, int c, float v) {
    const float y = __builtin_fmaf(v, p.psc[int64_t(b) * p.ci + c], p.psh[int64_t(b) * p.ci + c]);
    return p.psilu ? ref_silu(y) : y;
}

template <int MODE, bool PRO>
__device__ __forceinline__ floatx4 load_a(const GemmArgs &p, const ConvRow &r, int m, int k, int tap_ky,
                                          int tap_kx, int tap_ci0) {
    if (MODE == kDense) {
        if (m >= p.M || k >= p.K) return zero4();
        return *reinterpret_cast<const floatx4 *>(p.a + int64_t(m) * p.lda + k);
    } else if (MODE == kDenseScalar) {
        floatx4 v = zero4();
        if (m < p.M) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (k + e < p.K) v[e] = p.a[int64_t(m) * p.lda + k + e];
        }
        return v;
    } else if (MODE == kConvAligned || MODE == kConvVec) {
        if (k >= p.K) return zero4();
        int ky, kx, c;
        if (MODE == kConvAligned) {
            ky = tap_ky;
            kx = tap_kx;
            c = tap_ci0 + (k & (BK - 1));
        } else {
            const int tap = k / p.ci;
            c = k - tap * p.ci;
            ky = tap / 3;
            kx = tap - ky * 3;
        }
        const int64_t off = conv_src(p, r, ky, kx);
        if (off < 0) return zero4();
        floatx4 v = *reinterpret_cast<const floatx4 *>(p.a + off + c);
        if (PRO) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = prologue1(p, r.b, c + e, v[e]);
        }
        return v;
    } else {  // kConvScalar
        floatx4 v = zero4();
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int kk = k + e;
            if (kk >= p.K) break;
            const int tap = kk / p.ci;
            const int c = kk - tap * p.ci;
            const int ky = tap / 3, kx = tap - ky * 3;
            const int64_t off = conv_src(p, r, ky, kx);
            if (off >= 0) {
                float x = p.a[off + c];
                if (PRO) x = prologue1(p, r.b, c, x);
                v[e] = x;
            }
        }
        return v;
    }
}

template <bool F16, bool BVEC>
__device__ __forceinline__ floatx4 load_b(const GemmArgs &p, int n, int k) {
    floatx4 v = zero4();
    if (n >= p.N) return v;
    if (BVEC) {
        if (k >= p.K) return v;
        if (F16) {
            const halfx4 h = *reinterpret_cast<const halfx4 *>(static_cast<const _Float16 *>(p.b) + int64_t(n) * p.ldb + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = float(h[e]);
        } else {
            v = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(p.b) + int64_t(n) * p.ldb + k);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (k + e < p.K) {
                if (F16)
                    v[e] = float(static_cast<const _Float16 *>(p.b)[int64_t(n) * p.ldb + k + e]);
                else
                    v[e] = static_cast<const float *>(p.b)[int64_t(n) * p.ldb + k + e];
            }
        }
    }
    return v;
}

template <int BM, int BN, int MODE, bool PRO, bool F16, bool BVEC, int EPI, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs p) {
    constexpr int FM = BM / 64, FN = BN / 64;        // 32x32 blocks per wave
    if (blockIdx.y) {
        const int64_t bz = blockIdx.y;
        p.a += bz * p.a_bs;
        p.b = static_cast<const char *>(p.b) + bz * p.b_bs * (F16 ? 2 : 4);
        p.out += bz * p.c_bs;
        if (p.res) p.res += bz * p.c_bs;
    }
    constexpr int A_LD = BM * K4 / 256, B_LD = BN * K4 / 256;
    __shared__ float As[BM * LDS_S];
    __shared__ float Bs[BN * LDS_S];

    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    // Grouped tile order: 8 tile-rows share their B panels while they run.
    int tm, tn;
    {
        constexpr int GROUP = 8;
        const int pid = blockIdx.x;
        const int in_group = GROUP * tiles_n;
        const int gid = pid / in_group;
        const int first = gid * GROUP;
        const int gsize = min(tiles_m - first, GROUP);
        const int r = pid - gid * in_group;
        tm = first + r % gsize;
        tn = r / gsize;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int k_begin = SPLIT ? blockIdx.z * p.k_split : 0;
    const int k_end = SPLIT ? min(p.K, k_begin + p.k_split) : p.K;
    const int ktiles = (k_end - k_begin + BK - 1) / BK;

    const int tid = threadIdx.x;
    const int lrow = tid >> 3, lc4 = tid & 7;  // load slot: row within 32-row pass, float4 column

    ConvRow crow[A_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        if (MODE >= kConvAligned) crow[i] = conv_row(p, m0 + lrow + 32 * i);
        else crow[i] = ConvRow{0, 0, 0, true};
    }

    floatx4 ra[A_LD], rb[B_LD];
    auto fetch = [&](int kt) {
        const int k0 = k_begin + kt * BK;
        int tky = 0, tkx = 0, tci = 0;
        if (MODE == kConvAligned) {
            const int tap = k0 / p.ci;
            tci = k0 - tap * p.ci;
            tky = tap / 3;
            tkx = tap - tky * 3;
        }
        const int k = k0 + lc4 * 4;
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            ra[i] = (k < k_end) ? load_a<MODE, PRO>(p, crow[i], m0 + lrow + 32 * i, k, tky, tkx, tci) : zero4();
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) rb[i] = (k < k_end) ? load_b<F16, BVEC>(p, n0 + lrow + 32 * i, k) : zero4();
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) *reinterpret_cast<floatx4 *>(As + (lrow + 32 * i) * LDS_S + lc4 * 4) = ra[i];
#pragma unroll
        for (int i = 0; i < B_LD; ++i) *reinterpret_cast<floatx4 *>(Bs + (lrow + 32 * i) * LDS_S + lc4 * 4) = rb[i];
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const float *as_w = As + (wm * (BM / 2) + (lane & 31)) * LDS_S + (lane >> 5) * 4;
    const float *bs_w = Bs + (wn * (BN / 2) + (lane & 31)) * LDS_S + (lane >> 5) * 4;

    if (ktiles > 0) {
        fetch(0);
        stash();
    }
    __syncthreads();
    for (int kt = 0; kt < ktiles; ++kt) {
        if (kt + 1 < ktiles) fetch(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 8) {
            floatx4 a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = *reinterpret_cast<const floatx4 *>(as_w + i * 32 * LDS_S + kk);
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = *reinterpret_cast<const floatx4 *>(bs_w + j * 32 * LDS_S + kk);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][t], b[j][t], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
        if (kt + 1 < ktiles) {
            stash();
            __syncthreads();
        }
    }

    // Epilogue. Block (i, j), register v, lane l: row 8*(v/4) + 4*(l/32) + v%4, column l%32.
    const int row_base = m0 + wm * (BM / 2) + 4 * (lane >> 5);
    const int col_base = n0 + wn * (BN / 2) + (lane & 31);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int col = col_base + j * 32;
        if (col >= p.N) continue;
        const float bcol = (!SPLIT && p.bias) ? p.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = row_base + i * 32 + 8 * (v >> 2) + (v & 3);
                if (row >= p.M) continue;
                const float r = acc[i][j][v];
                if (SPLIT) {
                    p.partial[(int64_t(blockIdx.z) * p.M + row) * p.N + col] = r;
                } else {
                    float y;
                    if (p.res) {
                        const float t = p.bias ? p.res[int64_t(row) * p.ldc + col] + bcol
                                               : p.res[int64_t(row) * p.ldc + col];
                        y = t + r;
                    } else {
                        y = p.bias ? bcol + r : r;
                    }
                    if (EPI == 1) y = ref_silu(y);
                    p.out[int64_t(row) * p.ldc + col] = y;
                }
            }
        }
    }
}

// Sums split-K partials in split order, then (residual + bias) + sum [SiLU].
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ partial, int splits, int M,
                                                            int N, const float *__restrict__ bias,
                                                            const float *__restrict__ res, int64_t ldc,
                                                            float *__restrict__ out) {
    const int64_t total = int64_t(M) * N;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        float s = partial[e];
        for (int z = 1; z < splits; ++z) s += partial[int64_t(z) * total + e];
        const int64_t row = e / N;
        const int col = int(e - row * N);
        float y;
        if (res) {
            const float t = bias ? res[row * ldc + col] + bias[col] : res[row * ldc + col];
            y = t + s;
        } else {
            y = bias ? bias[col] + s : s;
        }
        if (EPI == 1) y = ref_silu(y);
        out[row * ldc + col] = y;
    }
}

struct Plan {
    int bm, bn, splits, k_split;
};

Plan plan_for(int M, int N, int K, int cus) {
    auto tiles = [&](int bm, int bn) { return int64_t(ceil_div(M, bm)) * ceil_div(N, bn); };
    Plan pl{64, 64, 1, K};
    if (tiles(128, 128) >= cus) {
        pl.bm = 128;
        pl.bn = 128;
    } else if (tiles(128, 64) >= cus) {
        pl.bm = 128;
        pl.bn = 64;
    }
    const int64_t t = tiles(pl.bm, pl.bn);
    const int ktiles = int(ceil_div(K, BK));
    if (t < cus && ktiles >= 16) {
        // Split K so the grid covers the chip about twice, keeping >= 8 K tiles per split.
        int want = int(std::min<int64_t>(ceil_div(2 * int64_t(cus), t), ktiles / 8));
        want = std::max(want, 1);
        const int per = int(ceil_div(ktiles, want));
        pl.k_split = per * BK;
        pl.splits = int(ceil_div(ktiles, per));
    }
    return pl;
}

template <int BM, int BN, int MODE, bool PRO, bool F16, bool BVEC>
void launch_cfg(Context &ctx, GemmArgs &p, const Plan &pl, GemmEpilogue epi, int batch) {
    const unsigned tiles = unsigned(ceil_div(p.M, BM) * ceil_div(p.N, BN));
    if (pl.splits > 1) {
        const size_t bytes = size_t(pl.splits) * p.M * p.N * sizeof(float);
        p.partial = static_cast<float *>(ctx.ws.get(bytes, ctx.stream));
        p.k_split = pl.k_split;
        dim3 grid(tiles, 1, pl.splits);
        gemm_f32_kernel<BM, BN, MODE, PRO, F16, BVEC, 0, true><<<grid, 256, 0, ctx.stream>>>(p);
        MH_LAUNCH_CHECK();
        const int64_t total = int64_t(p.M) * p.N;
        const unsigned rb = unsigned(std::min<int64_t>(ceil_div(total, 256), 8192));
        if (epi == GemmEpilogue::Silu)
            splitk_reduce_kernel<1><<<rb, 256, 0, ctx.stream>>>(p.partial, pl.splits, p.M, p.N, p.bias, p.res, p.ldc,
                                                                p.out);
        else
            splitk_reduce_kernel<0><<<rb, 256, 0, ctx.stream>>>(p.partial, pl.splits, p.M, p.N, p.bias, p.res, p.ldc,
                                                                p.out);
    } else {
        p.k_split = p.K;
        const dim3 grid(tiles, unsigned(batch));
        if (epi == GemmEpilogue::Silu)
            gemm_f32_kernel<BM, BN, MODE, PRO, F16, BVEC, 1, false><<<grid, 256, 0, ctx.stream>>>(p);
        else
            gemm_f32_kernel<BM, BN, MODE, PRO, F16, BVEC, 0, false><<<grid, 256, 0, ctx.stream>>>(p);
    }
    MH_LAUNCH_CHECK();
}

template <int MODE, bool PRO, bool F16, bool BVEC>
void launch_tiles(Context &ctx, GemmArgs &p, GemmEpilogue epi, int batch) {
    Plan pl = plan_for(p.M, p.N, p.K, int(ceil_div(ctx.cu_count, batch)));
    if (batch > 1) pl.splits = 1;
    if (pl.bm == 128 && pl.bn == 128)
        launch_cfg<128, 128, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
    else if (pl.bm == 128)
        launch_cfg<128, 64, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
    else
        launch_cfg<64, 64, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
}

template <int MODE, bool PRO>
void launch_b(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch = 1) {
    const int esz = wt == kF16 ? 2 : 4;
    const bool bvec = p.K % 4 == 0 && p.ldb % 4 == 0 && (reinterpret_cast<uintptr_t>(p.b) % (4 * esz)) == 0 &&
                      (batch == 1 || p.b_bs % 4 == 0);
    if (wt == kF16) {
        if (bvec) launch_tiles<MODE, PRO, true, true>(ctx, p, epi, batch);
        else launch_tiles<MODE, PRO, true, false>(ctx, p, epi, batch);
    } else {
        if (bvec) launch_tiles<MODE, PRO, false, true>(ctx, p, epi, batch);
        else launch_tiles<MODE, PRO, false, false>(ctx, p, epi, batch);
    }
}

__global__ void im2col_gather_kernel(GemmArgs p, int64_t first, int64_t count, float *__restrict__ rows) {
    const int64_t K = p.K;
    const int64_t total = count * K;
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
        const int64_t i = e / K;
        const int k = int(e - i * K);
        const ConvRow r = conv_row(p, int(first + i));
        const int tap = k / p.ci, c = k - (k / p.ci) * p.ci;
        const int64_t off = conv_src(p, r, tap / 3, tap % 3);
        rows[e] = off >= 0 ? p.a[off + c] : 0.0f;
    }
}

__global__ void mfma_probe_kernel(const float *a, const float *b, float *d) {
    const int lane = threadIdx.x;
    floatx16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
    // a: [32][2] row-major; b: [2][32] row-major.
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[(lane & 31) * 2 + (lane >> 5)], b[(lane >> 5) * 32 + (lane & 31)],
                                               acc, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        d[row * 32 + (lane & 31)] = acc[v];
    }
}

}  // namespace

void conv1x1(Context &ctx, const float *x, int64_t pixels, int c_in, const void *weight, WeightType wt, int c_out,
             const float *bias, const float *residual, float *out, GemmEpilogue epi) {
    MH_REQUIRE(c_in > 0 && c_out > 0, "Conv1x1: empty channel axis");
    MH_REQUIRE(pixels < (int64_t(1) << 31), "Conv1x1: too many pixels");
    if (pixels == 0) return;
    GemmArgs p{};
    p.a = x;
    p.lda = c_in;
    p.M = int(pixels);
    p.N = c_out;
    p.K = c_in;
    p.b = weight;
    p.ldb = c_in;
    p.bias = bias;
    p.res = residual;
    p.out = out;
    p.ldc = c_out;
    if (c_in % 4 == 0 && aligned16(x))
        launch_b<kDense, false>(ctx, p, wt, epi);
    else
        launch_b<kDenseScalar, false>(ctx, p, wt, epi);
}

void gemm_nt(Context &ctx, const float *a, int64_t lda, int64_t a_bs, const void *b, WeightType wt, int64_t ldb,
             int64_t b_bs, int m, int n, int k, int batch, const float *bias, const float *residual, float *out,
             int64_t ldc, int64_t c_bs, GemmEpilogue epi) {
    MH_REQUIRE(m >= 0 && n > 0 && k > 0 && batch > 0, "gemm: bad shape");
    if (m == 0) return;
    GemmArgs p{};
    p.a = a;
    p.lda = lda;
    p.M = m;
    p.N = n;
    p.K = k;
    p.b = b;
    p.ldb = ldb;
    p.bias = bias;
    p.res = residual;
    p.out = out;
    p.ldc = ldc;
    p.a_bs = a_bs;
    p.b_bs = b_bs;
    p.c_bs = c_bs;
    const bool vec = k % 4 == 0 && lda % 4 == 0 && aligned16(a) && (batch == 1 || a_bs % 4 == 0);
    if (vec)
        launch_b<kDense, false>(ctx, p, wt, epi, batch);
    else
        launch_b<kDenseScalar, false>(ctx, p, wt, epi, batch);
}

void conv3x3_output_hw(int h, int w, int stride, const int pad[4], bool upsample2x, int *ho, int *wo) {
    const int up = upsample2x ? 2 : 1;
    const int hh = h * up + pad[0] + pad[2] - 3, ww = w * up + pad[1] + pad[3] - 3;
    MH_REQUIRE(stride > 0 && hh >= 0 && ww >= 0, "Conv3x3: input smaller than the kernel");
    *ho = hh / stride + 1;
    *wo = ww / stride + 1;
}

void conv3x3(Context &ctx, const float *x, int n, int h, int w, int c_in, const void *weight, WeightType wt,
             int c_out, const float *bias, int stride, const int pad[4], bool upsample2x, const Affine *prologue,
             float *out) {
    MH_REQUIRE(c_in > 0 && c_out > 0, "Conv3x3 input channels");
    if (prologue) {
        MH_REQUIRE(stride == 1 && pad[0] == 1 && pad[1] == 1 && pad[2] == 1 && pad[3] == 1,
                   "Conv3x3 prologue needs the stride-1 / pad-1 Winograd path");
    }
    int ho, wo;
    conv3x3_output_hw(h, w, stride, pad, upsample2x, &ho, &wo);
    const int64_t m = int64_t(n) * ho * wo;
    MH_REQUIRE(m < (int64_t(1) << 31), "Conv3x3: too many output pixels");
    if (m == 0) return;
    GemmArgs p{};
    p.a = x;
    p.M = int(m);
    p.N = c_out;
    p.K = 9 * c_in;
    p.cn = n;
    p.ch = h;
    p.cw = w;
    p.ci = c_in;
    p.ho = ho;
    p.wo = wo;
    p.stride = stride;
    p.pad_t = pad[0];
    p.pad_l = pad[1];
    p.up = upsample2x ? 1 : 0;
    p.b = weight;
    p.ldb = 9 * int64_t(c_in);
    p.bias = bias;
    p.out = out;
    p.ldc = c_out;
    const bool pro = prologue != nullptr;
    if (pro) {
        p.psc = prologue->scale;
        p.psh = prologue->shift;
        p.psilu = prologue->silu ? 1 : 0;
    }
    const bool vec = c_in % 4 == 0 && aligned16(x);
    if (vec && c_in % BK == 0) {
        if (pro) launch_b<kConvAligned, true>(ctx, p, wt, GemmEpilogue::None);
        else launch_b<kConvAligned, false>(ctx, p, wt, GemmEpilogue::None);
    } else if (vec) {
        if (pro) launch_b<kConvVec, true>(ctx, p, wt, GemmEpilogue::None);
        else launch_b<kConvVec, false>(ctx, p, wt, GemmEpilogue::None);
    } else {
        if (pro) launch_b<kConvScalar, true>(ctx, p, wt, GemmEpilogue::None);
        else launch_b<kConvScalar, false>(ctx, p, wt, GemmEpilogue::None);
    }
}

void im2col_gather(Context &ctx, const float *x, int n, int h, int w, int c, int stride, const int pad[4],
                   bool upsample2x, int64_t first, int64_t count, float *rows) {
    int ho, wo;
    conv3x3_output_hw(h, w, stride, pad, upsample2x, &ho, &wo);
    MH_REQUIRE(first >= 0 && count >= 0 && first + count <= int64_t(n) * ho * wo, "im2col: pixel range out of bounds");
    if (count == 0) return;
    GemmArgs p{};
    p.a = x;
    p.M = int(int64_t(n) * ho * wo);
    p.K = 9 * c;
    p.cn = n;
    p.ch = h;
    p.cw = w;
    p.ci = c;
    p.ho = ho;
    p.wo = wo;
    p.stride = stride;
    p.pad_t = pad[0];
    p.pad_l = pad[1];
    p.up = upsample2x ? 1 : 0;
    const int64_t total = count * 9 * c;
    const unsigned blocks = unsigned(std::min<int64_t>(ceil_div(total, 256), 1 << 20));
    im2col_gather_kernel<<<blocks, 256, 0, ctx.stream>>>(p, first, count, rows);
    MH_LAUNCH_CHECK();
}

void selftest_mfma_f32(Context &ctx, const float *a_host, const float *b_host, float *d_host) {
    float *dev = nullptr;
    HIP_CHECK(hipMalloc(&dev, (64 + 64 + 1024) * sizeof(float)));
    HIP_CHECK(hipMemcpyAsync(dev, a_host, 64 * sizeof(float), hipMemcpyHostToDevice, ctx.stream));
    HIP_CHECK(hipMemcpyAsync(dev + 64, b_host, 64 * sizeof(float), hipMemcpyHostToDevice, ctx.stream));
    mfma_probe_kernel<<<1, 64, 0, ctx.stream>>>(dev, dev + 64, dev + 128);
    MH_LAUNCH_CHECK();
    HIP_CHECK(hipMemcpyAsync(d_host, dev + 128, 1024 * sizeof(float), hipMemcpyDeviceToHost, ctx.stream));
    HIP_CHECK(hipStreamSynchronize(ctx.stream));
    HIP_CHECK(hipFree(dev));
}

}  // namespace mh
