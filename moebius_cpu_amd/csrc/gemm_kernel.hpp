// Implicit-GEMM kernel template shared by the GEMM translation units (one
// file per family of A-operand modes, so they compile in parallel). Everything
// here has internal linkage: each file launches only its own instantiations.
#pragma once
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace gemm {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 32;          // K per LDS stage
constexpr int K4 = BK / 4;      // float4 per tile row
constexpr int kMaxSeg = 3;      // column segments of a segmented output

// Matrix instruction: v_mfma_f32_32x32x2f32 (MF = 32) when each wave's half
// of the tile is a multiple of 32 in both dimensions, else v_mfma_f32_16x16x4f32
// (MF = 16: the 32-row or 32-column tiles of the small GEMMs). Output lane
// layouts: 16x16: register v of lane l is row 4 * (l / 16) + v, column l % 16;
// 32x32: row 8 * (v / 4) + 4 * (l / 32) + v % 4, column l % 32.
template <int BM, int BN>
constexpr int mf_for() { return ((BM / 2) % 32 == 0 && (BN / 2) % 32 == 0) ? 32 : 16; }

template <int M>
struct Mf {
    static constexpr int kAccRegs = M * M / 64;
    static constexpr int kKStep = M == 32 ? 8 : 16;  // K covered by one float4 read per lane
    typedef std::conditional_t<M == 32, floatx16, floatx4> Acc;
    static __device__ __forceinline__ Acc mfma(float a, float b, const Acc &c) {
        if constexpr (M == 32) return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
        else return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ int acc_row(int v, int lane) {
        if constexpr (M == 32) return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        else return 4 * (lane >> 4) + v;
    }
};

// A-operand prologue kinds (the PRO template argument): none; the GroupNorm
// affine [SiLU](x . scale + shift) per (item, channel) as values load; or the
// LayerNorm of each row folded into the product (kProLn, dense operands: the
// workgroup sums its rows' values in f64 as they load, and the epilogue forms
// rstd . (acc - mean . ln_c1) with B = W . diag(gamma), bias = W . beta + b);
// or the same fold with each row's statistics from partial sums its producer
// wrote (kProLnPart: GemmArgs::lnp_in), the A values loading as they are.
constexpr int kProNone = 0, kProAffine = 1, kProLn = 2, kProLnPart = 3;

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
    // row grouping of the output (0 or 1: plain): row m, column n is stored at
    // (m / rg) * ldc + n * rg + m % rg, e.g. [pixel][tap][head] from (pixel, head) rows
    int rg;
    // residual transform: res' = [SiLU](res . rsc + rsh), per item (rows / r_rows) and column
    const float *rsc, *rsh;
    int rsilu, r_rows;
    // second residual, added last: y = y + res2
    const float *res2;
    // column segments (0: one output): see out_ptr
    int nseg;
    int seg_col[kMaxSeg + 1];
    float *seg_out[kMaxSeg];
    // byte extents of one item's A (or conv input) and of B, for the buffer
    // loads' range check (< 2^31): an access at or past the extent reads zero
    uint32_t a_bytes, b_bytes;
    // set by the launcher: 1: the output (or split partials) may be written four
    // adjacent columns at a time with 16-byte accesses (see out_vec_ok); 2: grouped
    // rows written four rows at a time (see out_vec_ok); 0: one element at a time
    int vec_out;
    // GroupNorm statistics of the output (optional): row tile t writes, per
    // column, (sum y, sum y*y) over its BM rows of the values stored to
    // gnp [t][N][2]; gn_item_rows = rows per batch item (tiles must not straddle
    // items). The launcher clears gnp where it cannot honour it and reports the
    // rows per partial in gn_rows (0: none written).
    float *gnp;
    int gn_item_rows, gn_rows;
    // dense operands with the prologue (psc/psh [items][K]): rows per item
    int pro_rows;
    // dense operands only: the A row is [a row (ka columns) | a2 row], a2
    // [M][lda2] holding columns ka.. (ka a multiple of 64, so each K tile reads
    // one of the two); a2_bytes its extent. a2 null: one operand.
    const float *a2;
    int64_t lda2;
    int ka;
    uint32_t a2_bytes;
    // kProLn: per output column, the sum over K of the folded weights (the
    // mean's coefficient), and the LayerNorm epsilon; the row width is K
    const float *ln_c1;
    float ln_eps;
    // Row statistics of the output for a LayerNorm that reads it next
    // (optional): lnp_out [M][lnp_ld] = per row and column tile, (sum y, sum
    // y*y) over the tile's stored values. The launcher sets lnp_ld (tiles
    // across N), or clears lnp_out where the tiling cannot honour it.
    float2 *lnp_out;
    int lnp_ld;
    // kProLnPart: the same partials of the A rows, lnp_n per row (summed in
    // order in f64 for each row's mean and variance over K columns).
    const float2 *lnp_in;
    int lnp_n;
};

// (residual [transformed] + bias) + acc [SiLU] (+ res2): the reference's
// Conv1x1 epilogue (src/engine/conv.rs:38-55) followed by the block's add_inplace.
// FM: the FAST precision kernel's SiLU (fast_silu) instead of the reference's.
template <int EPI, bool FM = false>
__device__ __forceinline__ float epilogue_value(const GemmArgs &p, int row, int col, int64_t o, float acc, float bcol) {
    float y;
    if (p.res) {
        float rv = p.res[o];
        if (p.rsc) {
            const int64_t i = int64_t(row / p.r_rows) * p.N + col;
            rv = __builtin_fmaf(rv, p.rsc[i], p.rsh[i]);
            if (p.rsilu) rv = silu_of<FM>(rv);
        }
        const float t = p.bias ? rv + bcol : rv;
        y = t + acc;
    } else {
        y = p.bias ? bcol + acc : acc;
    }
    if (EPI == 1) y = silu_of<FM>(y);
    if (p.res2) y = y + p.res2[o];
    return y;
}

// Launchers, one per A-operand family (gemm_dense.hip, gemm_conv.hip).
void launch_dense(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch, bool vec);
// Dense operands with the GroupNorm prologue (K-contiguous vector rows, no batch).
void launch_dense_pro(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi);
// Dense operands whose rows enter through a folded LayerNorm (kProLn; no batch).
void launch_dense_ln(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi);
void launch_conv(Context &ctx, GemmArgs &p, WeightType wt, int mode, bool pro);

namespace {


__device__ __forceinline__ int64_t out_index(const GemmArgs &p, int row, int col) {
    if (p.rg > 1) return int64_t(row / p.rg) * p.ldc + int64_t(col) * p.rg + row % p.rg;
    return int64_t(row) * p.ldc + col;
}

// Column-segmented output: columns [seg_col[s], seg_col[s+1]) go to their own
// row-major buffer seg_out[s] (leading dimension = segment width), so one GEMM
// over concatenated weights fills several separate tensors.
__device__ __forceinline__ float *out_ptr(const GemmArgs &p, int row, int col, int64_t &o) {
    if (p.nseg == 0) {
        o = out_index(p, row, col);
        return p.out;
    }
    // constant indices only: a runtime index into the by-value arguments would
    // move them to scratch memory
    float *dst = p.seg_out[0];
    int c0 = 0, c1 = p.seg_col[1];
    if (p.nseg > 1 && col >= p.seg_col[1]) {
        dst = p.seg_out[1];
        c0 = p.seg_col[1];
        c1 = p.seg_col[2];
    }
    if (p.nseg > 2 && col >= p.seg_col[2]) {
        dst = p.seg_out[2];
        c0 = p.seg_col[2];
        c1 = p.seg_col[3];
    }
    o = int64_t(row) * (c1 - c0) + (col - c0);
    return dst;
}

// epilogue_value for four adjacent columns col..col+3 of one row, with 16-byte
// loads and one 16-byte store (the caller has checked out_vec_ok); returns the
// values stored.
// OUT16: the output is f16 (GemmArgs::out holds halves), each value rounded to
// nearest even and saturated as the f16 GEMM rounds its f32 operands; the f32
// values are returned (for the partial sums).
template <int EPI, bool FM = false, bool OUT16 = false>
__device__ __forceinline__ float4 store4(const GemmArgs &p, int row, int col, float4 s) {
    int64_t o;
    float *dst = out_ptr(p, row, col, o);
    float y[4] = {s.x, s.y, s.z, s.w};
    const float4 bv = p.bias ? *reinterpret_cast<const float4 *>(p.bias + col) : float4{0.f, 0.f, 0.f, 0.f};
    const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
    if (p.res) {
        const float4 r4 = *reinterpret_cast<const float4 *>(p.res + o);
        float rv[4] = {r4.x, r4.y, r4.z, r4.w};
        if (p.rsc) {
            const int64_t i = int64_t(row / p.r_rows) * p.N + col;
            const float4 sc = *reinterpret_cast<const float4 *>(p.rsc + i);
            const float4 sh = *reinterpret_cast<const float4 *>(p.rsh + i);
            rv[0] = __builtin_fmaf(rv[0], sc.x, sh.x);
            rv[1] = __builtin_fmaf(rv[1], sc.y, sh.y);
            rv[2] = __builtin_fmaf(rv[2], sc.z, sh.z);
            rv[3] = __builtin_fmaf(rv[3], sc.w, sh.w);
            if (p.rsilu)
#pragma unroll
                for (int j = 0; j < 4; ++j) rv[j] = silu_of<FM>(rv[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = (p.bias ? rv[j] + bb[j] : rv[j]) + y[j];
    } else if (p.bias) {
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = bb[j] + y[j];
    }
    if (EPI == 1)
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = silu_of<FM>(y[j]);
    if (p.res2) {
        const float4 r2 = *reinterpret_cast<const float4 *>(p.res2 + o);
        y[0] = y[0] + r2.x, y[1] = y[1] + r2.y, y[2] = y[2] + r2.z, y[3] = y[3] + r2.w;
    }
    const float4 r{y[0], y[1], y[2], y[3]};
    if constexpr (OUT16) {
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        auto r16 = [](float v) {
            return static_cast<_Float16>(__builtin_fabsf(v) > 65504.0f ? __builtin_copysignf(65504.0f, v) : v);
        };
        *reinterpret_cast<half4_t *>(reinterpret_cast<_Float16 *>(dst) + o) = half4_t{r16(r.x), r16(r.y), r16(r.z),
                                                                                     r16(r.w)};
    } else {
        *reinterpret_cast<float4 *>(dst + o) = r;
    }
    return r;
}

// How the output can be written 16 bytes at a time (GemmArgs::vec_out): 1 when N,
// the leading dimensions, batch strides and segment bounds are multiples of 4
// with no row grouping; 2 for grouped rows with rg % 4 == 0, BM % rg == 0,
// M % rg == 0, ldc and the batch stride multiples of 4, one output; buffers
// 16-byte aligned; else 0.
inline int out_vec_ok(const GemmArgs &p, int bm) {
    auto al = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    if (p.rg > 1) {
        const bool ok = p.rg % 4 == 0 && bm % p.rg == 0 && p.M % p.rg == 0 && (p.ldc & 3) == 0 &&
                        (p.c_bs & 3) == 0 && p.nseg == 0 && al(p.out) && al(p.res) && al(p.res2);
        return ok ? 2 : 0;
    }
    if ((p.N & 3) || (p.c_bs & 3)) return false;
    if (!al(p.bias) || !al(p.res) || !al(p.res2) || !al(p.rsc) || !al(p.rsh)) return false;
    if (p.nseg == 0) return ((p.ldc & 3) == 0 && al(p.out)) ? 1 : 0;
    for (int s = 0; s < p.nseg; ++s)
        if ((p.seg_col[s] & 3) || (p.seg_col[s + 1] & 3) || !al(p.seg_out[s])) return 0;
    return 1;
}

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

template <bool FM = false>
__device__ __forceinline__ float prologue1(const GemmArgs &p, int b, int c, float v) {
    const float y = __builtin_fmaf(v, p.psc[int64_t(b) * p.ci + c], p.psh[int64_t(b) * p.ci + c]);
    return p.psilu ? silu_of<FM>(y) : y;
}

template <int MODE, int PRO, bool FM = false>
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
        if (PRO == kProAffine) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = prologue1<FM>(p, r.b, c + e, v[e]);
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
                if (PRO == kProAffine) x = prologue1<FM>(p, r.b, c, x);
                v[e] = x;
            }
        }
        return v;
    }
}

// Buffer loads: a lane whose element is outside the operand (rows past M or
// N, K past the split's end, conv padding) gets an offset past the resource's
// extent, which the hardware answers with zeros. The loads are therefore
// unconditional (no branch per load), and the compiler can wait for one K
// tile's loads while the next tile's are still in flight.
constexpr int kOob = int(0x80000000u);

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), short(0), int(bytes), 0x00020000);
}

__device__ __forceinline__ floatx4 buf_load4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Prologue of a dense A operand: the consumer-side GroupNorm affine
// [SiLU](x . scale + shift) of row item b (r.b = row / pro_rows), channels
// k..k+3 (psc/psh [items][K], K % 4 == 0, 16-byte aligned), computed as the
// separate apply pass does; zero where the load was out of range.
template <bool FM = false>
__device__ __forceinline__ floatx4 dense_prologue(const GemmArgs &p, int b, int k, bool ok, floatx4 v) {
    const int64_t i = int64_t(b) * p.K + (ok ? k : 0);
    const float4 sc = *reinterpret_cast<const float4 *>(p.psc + i);
    const float4 sh = *reinterpret_cast<const float4 *>(p.psh + i);
    const float s4[4] = {sc.x, sc.y, sc.z, sc.w}, h4[4] = {sh.x, sh.y, sh.z, sh.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float y = __builtin_fmaf(v[e], s4[e], h4[e]);
        if (p.psilu) y = silu_of<FM>(y);
        v[e] = ok ? y : 0.0f;
    }
    return v;
}

template <int MODE, int PRO>
__device__ __forceinline__ floatx4 load_a_buf(const GemmArgs &p, __amdgpu_buffer_rsrc_t ar, const ConvRow &r, int m,
                                              int k, int k_end, int tap_ky, int tap_kx, int tap_ci0,
                                              int64_t lda = -1) {
    if constexpr (MODE == kDense) {
        const bool ok = m < p.M && k < k_end;
        const floatx4 v = buf_load4(ar, ok ? int((int64_t(m) * (lda < 0 ? p.lda : lda) + k) * 4) : kOob);
        if constexpr (PRO == kProAffine) return dense_prologue(p, r.b, k, ok, v);
        return v;
    } else {
        int ky, kx, c;
        if constexpr (MODE == kConvAligned) {
            ky = tap_ky;
            kx = tap_kx;
            c = tap_ci0 + (k & (BK - 1));
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
            for (int e = 0; e < 4; ++e) v[e] = ok ? prologue1(p, r.b, c + e, v[e]) : 0.0f;
        }
        return v;
    }
}

template <bool F16>
__device__ __forceinline__ floatx4 load_b_buf(const GemmArgs &p, __amdgpu_buffer_rsrc_t br, int n, int k, int k_end) {
    const bool ok = n < p.N && k < k_end;
    const int64_t e = int64_t(n) * p.ldb + k;
    if constexpr (F16) {
        const auto raw = __builtin_amdgcn_raw_buffer_load_b64(br, ok ? int(e * 2) : kOob, 0, 0);
        const halfx4 h = __builtin_bit_cast(halfx4, raw);
        floatx4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = float(h[i]);
        return v;
    } else {
        return buf_load4(br, ok ? int(e * 4) : kOob);
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

// Tile order, shared by the f32 and f16 kernels: groups of 8 tile rows share
// their B panels while they run; MI355X dispatches workgroups round-robin over
// its 8 XCDs, so the 8 rows of a group land on different XCDs and each row
// panel of A stays within one XCD's L2. (Measured against remapping each XCD
// to one contiguous row-major range of tiles, batch items and K splits: that
// is 4-20% faster on some GEMMs alone but 0.4% slower over a UNet step, and
// column-major ranges are slower still; the grouped order stays.)
struct TileIdx {
    int tm, tn, y, z;
};

__device__ __forceinline__ TileIdx tile_index(int tiles_m, int tiles_n) {
    constexpr int GROUP = 8;
    const int pid = blockIdx.x;
    const int in_group = GROUP * tiles_n;
    const int gid = pid / in_group;
    const int first = gid * GROUP;
    const int gsize = min(tiles_m - first, GROUP);
    const int rr = pid - gid * in_group;
    TileIdx r;
    r.tm = first + rr % gsize;
    r.tn = rr / gsize;
    r.y = blockIdx.y;
    r.z = blockIdx.z;
    return r;
}

// GroupNorm partials of one output tile (GemmArgs::gnp): thread t holds the
// sums over its rows of column quad t % (BN / 4). The lanes of a wave that
// share a quad are added with an xor butterfly (every lane ends with the same
// bits), then the four waves' sums in wave order through LDS, so the partials
// are deterministic.
template <int BM, int BN>
__device__ __forceinline__ void gn_tile_partials(const GemmArgs &p, float *smem, float4 s, float4 q, int m0, int n0) {
    constexpr int C4 = BN / 4;
    static_assert(C4 <= 64 && 64 % C4 == 0, "whole column quads per wave");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int off = C4; off < 64; off <<= 1) {
        s.x += __shfl_xor(s.x, off, 64), s.y += __shfl_xor(s.y, off, 64);
        s.z += __shfl_xor(s.z, off, 64), s.w += __shfl_xor(s.w, off, 64);
        q.x += __shfl_xor(q.x, off, 64), q.y += __shfl_xor(q.y, off, 64);
        q.z += __shfl_xor(q.z, off, 64), q.w += __shfl_xor(q.w, off, 64);
    }
    float4 *red = reinterpret_cast<float4 *>(smem);
    __syncthreads();  // every thread is done with the C tile
    if (lane < C4) {
        red[wave * C4 + lane] = s;
        red[4 * C4 + wave * C4 + lane] = q;
    }
    __syncthreads();
    if (tid < C4) {
        const int col = n0 + tid * 4;
        if (col < p.N) {
            float4 ts = red[tid], tq = red[4 * C4 + tid];
#pragma unroll
            for (int r = 1; r < 4; ++r) {
                const float4 a = red[r * C4 + tid], b = red[4 * C4 + r * C4 + tid];
                ts.x += a.x, ts.y += a.y, ts.z += a.z, ts.w += a.w;
                tq.x += b.x, tq.y += b.y, tq.z += b.z, tq.w += b.w;
            }
            float *dst = p.gnp + (int64_t(m0 / BM) * p.N + col) * 2;
            *reinterpret_cast<float4 *>(dst) = float4{ts.x, tq.x, ts.y, tq.y};
            *reinterpret_cast<float4 *>(dst + 4) = float4{ts.z, tq.z, ts.w, tq.w};
        }
    }
}

// Mean and 1 / sqrt(var + eps) of the A rows a workgroup loaded (kProLn):
// slot i of this thread covers row lrow + RPP * i, its KL lanes (adjacent, one
// wave) hold the row's partial sums; biased variance, as LayerNorm's.
template <int A_LD, int RPP, int KL, int BM>
__device__ __forceinline__ void ln_row_stats(const GemmArgs &p, const double (&s1)[A_LD], const double (&s2)[A_LD],
                                             int lrow, int lc, float *st) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        double a = s1[i], b = s2[i];
#pragma unroll
        for (int o = 1; o < KL; o <<= 1) {
            a += __shfl_xor(a, o, 64);
            b += __shfl_xor(b, o, 64);
        }
        const int r = lrow + RPP * i;
        if (lc == 0 && r < BM) {
            const double mean = a / double(p.K);
            const double var = fmax(b / double(p.K) - mean * mean, 0.0);
            st[2 * r] = float(mean);
            st[2 * r + 1] = float(1.0 / sqrt(var + double(p.ln_eps)));
        }
    }
}

// The folded LayerNorm's correction of four adjacent columns of tile row rr:
// rstd . (acc - mean . c1[col]).
__device__ __forceinline__ float4 ln_correct(const GemmArgs &p, const float *st, int rr, int col, float4 v) {
    const float mean = st[2 * rr], rs = st[2 * rr + 1];
    const float4 c = *reinterpret_cast<const float4 *>(p.ln_c1 + col);
    v.x = rs * __builtin_fmaf(-mean, c.x, v.x);
    v.y = rs * __builtin_fmaf(-mean, c.y, v.y);
    v.z = rs * __builtin_fmaf(-mean, c.z, v.z);
    v.w = rs * __builtin_fmaf(-mean, c.w, v.w);
    return v;
}

// GroupNorm partials of one output tile from the stored values, for wave
// layouts other than the 2x2 one (any number of column quads): the store pass
// has written y over the C tile (row stride CS); thread t sums column quad
// t % C4 over rows g, g + G, ... (g = t / C4, G = NT / C4 row groups), then
// the G group sums are added in group order through LDS past the C tile.
template <int BM, int BN, int NT, int CS>
__device__ __forceinline__ void gn_tile_partials_lds(const GemmArgs &p, float *smem, int m0, int n0) {
    constexpr int C4 = BN / 4;
    constexpr int G = NT / C4;
    static_assert(G >= 1, "a thread per column quad");
    float4 *red = reinterpret_cast<float4 *>(smem + BM * CS);  // [2][G][C4]
    const int tid = threadIdx.x;
    if (tid < G * C4) {
        const int q = tid % C4, g = tid / C4;
        float4 s{0.f, 0.f, 0.f, 0.f}, sq = s;
        for (int r = g; r < BM && m0 + r < p.M; r += G) {  // rows past M were not stored
            const float4 y = *reinterpret_cast<const float4 *>(smem + r * CS + q * 4);
            s.x += y.x, s.y += y.y, s.z += y.z, s.w += y.w;
            sq.x = __builtin_fmaf(y.x, y.x, sq.x);
            sq.y = __builtin_fmaf(y.y, y.y, sq.y);
            sq.z = __builtin_fmaf(y.z, y.z, sq.z);
            sq.w = __builtin_fmaf(y.w, y.w, sq.w);
        }
        red[g * C4 + q] = s;
        red[(G + g) * C4 + q] = sq;
    }
    __syncthreads();
    if (tid < C4) {
        const int col = n0 + tid * 4;
        if (col < p.N) {
            float4 ts = red[tid], tq = red[G * C4 + tid];
            for (int g = 1; g < G; ++g) {
                const float4 a = red[g * C4 + tid], b = red[(G + g) * C4 + tid];
                ts.x += a.x, ts.y += a.y, ts.z += a.z, ts.w += a.w;
                tq.x += b.x, tq.y += b.y, tq.z += b.z, tq.w += b.w;
            }
            float *dst = p.gnp + (int64_t(m0 / BM) * p.N + col) * 2;
            *reinterpret_cast<float4 *>(dst) = float4{ts.x, tq.x, ts.y, tq.y};
            *reinterpret_cast<float4 *>(dst + 4) = float4{ts.z, tq.z, ts.w, tq.w};
        }
    }
}

// LayerNorm row partials of one output tile (GemmArgs::lnp_out) from the
// stored values in the C tile (row stride CS): 8 adjacent lanes per row, lane
// s summing column quads s, s + 8, ... in order, then an xor butterfly over
// the 8 lanes; rows past M and columns past N were not stored and are skipped.
template <int BM, int BN, int NT, int CS>
__device__ __forceinline__ void ln_tile_partials(const GemmArgs &p, const float *smem, int m0, int n0) {
    constexpr int C4 = BN / 4, RPASS = NT / 8;
    static_assert(NT % 64 == 0, "whole waves");
    const int tid = threadIdx.x, s = tid & 7;
    const int q_end = min(C4, (p.N - n0 + 3) / 4);
    for (int r = tid >> 3; r < BM; r += RPASS) {  // every lane of a row group runs the same passes
        float sum = 0.f, sq = 0.f;
        for (int q = s; q < q_end; q += 8) {
            const float4 y = *reinterpret_cast<const float4 *>(smem + r * CS + q * 4);
            sum += y.x, sum += y.y, sum += y.z, sum += y.w;
            sq = __builtin_fmaf(y.x, y.x, sq);
            sq = __builtin_fmaf(y.y, y.y, sq);
            sq = __builtin_fmaf(y.z, y.z, sq);
            sq = __builtin_fmaf(y.w, y.w, sq);
        }
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) {
            sum += __shfl_xor(sum, off, 64);
            sq += __shfl_xor(sq, off, 64);
        }
        if (s == 0 && m0 + r < p.M) p.lnp_out[int64_t(m0 + r) * p.lnp_ld + n0 / BN] = float2{sum, sq};
    }
}

// kProLnPart: each tile row's mean and 1 / sqrt(var + eps) from its producer's
// partials, summed in order in f64 (biased variance, as LayerNorm's).
template <int BM, int NT>
__device__ __forceinline__ void ln_stats_from_parts(const GemmArgs &p, int m0, float *st) {
    for (int r = threadIdx.x; r < BM; r += NT) {
        const int row = min(m0 + r, p.M - 1);
        const float2 *src = p.lnp_in + int64_t(row) * p.lnp_n;
        double a = 0.0, b = 0.0;
        for (int j = 0; j < p.lnp_n; ++j) {
            const float2 v = src[j];
            a += double(v.x);
            b += double(v.y);
        }
        const double mean = a / double(p.K);
        const double var = fmax(b / double(p.K) - mean * mean, 0.0);
        st[2 * r] = float(mean);
        st[2 * r + 1] = float(1.0 / sqrt(var + double(p.ln_eps)));
    }
}

// Wave layout of a workgroup: WM x WN waves over the output tile, each owning
// a (BM / WM) x (BN / WN) block of it, times WK wave groups that split every
// LDS stage's K between them (their sums are added in group order in the
// epilogue). 2x2x1 is the original layout of the square tiles.
template <int BM, int BN, int WM, int WN, int WK>
struct Waves {
    static constexpr int kWaves = WM * WN * WK;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int TM = BM / WM, TN = BN / WN;
    static constexpr int MF = (TM % 32 == 0 && TN % 32 == 0) ? 32 : 16;
    static constexpr int FM = TM / MF, FN = TN / MF;
    static constexpr int CS = BN + (MF == 16 ? 4 : 8);  // C tile row stride (floats)
    // The 2x2 layout's epilogue, where each thread keeps one column quad over its
    // rows for the GroupNorm sums (256 threads, 256 % (BN / 4) == 0); every
    // other layout sums them from LDS.
    static constexpr bool kFixedQuads = WM == 2 && WN == 2 && WK == 1 && 256 % (BN / 4) == 0 &&
                                        (BM * (BN / 4)) % 256 == 0;
    static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tiles of whole 16x16 blocks");
    static __device__ __forceinline__ void index(int wave, int &wm, int &wn, int &wk) {
        wk = wave / (WM * WN);
        const int r = wave - wk * (WM * WN);
        wm = r / WN;
        wn = r - wm * WN;
    }
};

// Epilogue through LDS, shared by the f32 and f16 kernels (smem holds at least
// WK * BM * CS floats, plus 2048 floats or, outside the 2x2 layout, BM * CS +
// 8 * NT for the GroupNorm sums, and is free): block (i, j), register v, lane l
// of wave (wm, wn, wk) holds row acc_row(v, l), column l % MF of its group's
// partial sum; the K groups' tiles are added in LDS, then each thread finishes
// four adjacent columns of a row at a time (16-byte loads and stores), or one
// element at a time where that is not possible.
template <int BM, int BN, int WM, int WN, int WK, int MF, int EPI, bool SPLIT, bool FSILU = false,
          bool OUT16 = false, typename Acc, int FM, int FN>
__device__ __forceinline__ void write_tile(const GemmArgs &p, float *smem, const Acc (&acc)[FM][FN], int m0, int n0,
                                           int z, const float *ln_st = nullptr) {
    using MI = Mf<MF>;
    using L = Waves<BM, BN, WM, WN, WK>;
    constexpr int NT = L::kThreads;
    // C tile row stride: the lane groups of one register's store sit 4 rows
    // apart (16x16 blocks: 16 columns per group) or 4 rows apart in two halves
    // (32x32: 32 columns); BN + 4 (resp. + 8) puts those groups on disjoint banks.
    constexpr int CS = L::CS;
    static_assert(MF == L::MF && FM == L::FM && FN == L::FN, "accumulators of the wave layout");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int wm, wn, wk;
    L::index(wave, wm, wn, wk);
    {
        float *slab = smem + wk * (BM * CS);
        const int r0 = wm * L::TM, c0 = wn * L::TN + (lane % MF);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int v = 0; v < MI::kAccRegs; ++v)
                    slab[(r0 + i * MF + MI::acc_row(v, lane)) * CS + c0 + j * MF] = acc[i][j][v];
    }
    __syncthreads();
    if constexpr (WK > 1) {  // K groups' partial tiles summed in group order into the first
        constexpr int C4 = BN / 4;
        for (int e = tid; e < BM * C4; e += NT) {
            const int rr = e / C4, cc = (e - rr * C4) * 4;
            float4 t = *reinterpret_cast<const float4 *>(smem + rr * CS + cc);
#pragma unroll
            for (int w = 1; w < WK; ++w) {
                const float4 u = *reinterpret_cast<const float4 *>(smem + w * BM * CS + rr * CS + cc);
                t.x += u.x, t.y += u.y, t.z += u.z, t.w += u.w;
            }
            *reinterpret_cast<float4 *>(smem + rr * CS + cc) = t;
        }
        __syncthreads();
    }
    if (p.vec_out == 1) {
        constexpr int C4 = BN / 4;  // float4 per tile row
        if constexpr (L::kFixedQuads) {
            static_assert(BM * C4 % 256 == 0, "whole passes over the C tile");
            // GroupNorm sums: a thread keeps one column quad over all its rows.
            constexpr bool kGn = !SPLIT && 256 % C4 == 0;
            float4 gs{0.f, 0.f, 0.f, 0.f}, gq = gs;
#pragma unroll
            for (int it = 0; it < BM * C4 / 256; ++it) {
                const int e = tid + it * 256, rr = e / C4, cc = (e - rr * C4) * 4;
                const int row = m0 + rr, col = n0 + cc;
                if (row >= p.M || col >= p.N) continue;  // N % 4 == 0: the whole float4 is inside
                float4 v = *reinterpret_cast<const float4 *>(smem + rr * CS + cc);
                if (ln_st) v = ln_correct(p, ln_st, rr, col, v);
                if (SPLIT) {
                    *reinterpret_cast<float4 *>(p.partial + (int64_t(z) * p.M + row) * p.N + col) = v;
                } else {
                    const float4 y = store4<EPI, FSILU, OUT16>(p, row, col, v);
                    if (kGn && p.gnp) {
                        gs.x += y.x, gs.y += y.y, gs.z += y.z, gs.w += y.w;
                        gq.x = __builtin_fmaf(y.x, y.x, gq.x);
                        gq.y = __builtin_fmaf(y.y, y.y, gq.y);
                        gq.z = __builtin_fmaf(y.z, y.z, gq.z);
                        gq.w = __builtin_fmaf(y.w, y.w, gq.w);
                    }
                    if (p.lnp_out) *reinterpret_cast<float4 *>(smem + rr * CS + cc) = y;  // for the row sums
                }
            }
            if (!SPLIT && p.lnp_out) {  // before the GroupNorm sums reuse the C tile's memory
                __syncthreads();
                ln_tile_partials<BM, BN, NT, CS>(p, smem, m0, n0);
            }
            if constexpr (kGn) {
                if (p.gnp) gn_tile_partials<BM, BN>(p, smem, gs, gq, m0, n0);
            }
        } else {
            const bool gn = !SPLIT && p.gnp, lnr = !SPLIT && p.lnp_out;
            for (int e = tid; e < BM * C4; e += NT) {
                const int rr = e / C4, cc = (e - rr * C4) * 4;
                const int row = m0 + rr, col = n0 + cc;
                if (row >= p.M || col >= p.N) continue;
                float *c = smem + rr * CS + cc;
                float4 v = *reinterpret_cast<const float4 *>(c);
                if (ln_st) v = ln_correct(p, ln_st, rr, col, v);
                if (SPLIT) {
                    *reinterpret_cast<float4 *>(p.partial + (int64_t(z) * p.M + row) * p.N + col) = v;
                } else {
                    const float4 y = store4<EPI, FSILU, OUT16>(p, row, col, v);
                    if (gn || lnr) *reinterpret_cast<float4 *>(c) = y;  // the stored values, for the sums
                }
            }
            if (gn || lnr) __syncthreads();
            if (lnr) ln_tile_partials<BM, BN, NT, CS>(p, smem, m0, n0);  // reads the C tile only
            if (gn) gn_tile_partials_lds<BM, BN, NT, CS>(p, smem, m0, n0);
        }
    } else if (OUT16) {
        // f16 outputs are written four columns at a time only (the launcher checks vec_out)
    } else if (p.vec_out == 2) {
        // Grouped rows (out index (row / rg) * ldc + col * rg + row % rg, rg % 4 == 0,
        // BM % rg == 0): rows 4j..4j+3 of a group at one column are four adjacent
        // floats, written as one 16-byte store; consecutive threads take the group's
        // row quads, then columns, so a wave writes contiguous runs.
        const int rq = p.rg >> 2;
        for (int e = tid; e < BM * BN / 4; e += NT) {
            const int hq = e % rq, rest = e / rq, cc = rest % BN, rr = (rest / BN) * p.rg + hq * 4;
            const int row = m0 + rr, col = n0 + cc;
            if (row >= p.M || col >= p.N) continue;  // M % rg == 0: the whole quad is inside
            const int64_t o = out_index(p, row, col);
            const float bcol = p.bias ? p.bias[col] : 0.f;
            float y[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] = epilogue_value<EPI, FSILU>(p, row + j, col, o + j, smem[(rr + j) * CS + cc], bcol);
            *reinterpret_cast<float4 *>(p.out + o) = float4{y[0], y[1], y[2], y[3]};
        }
    } else {
        // One element per thread and pass; consecutive threads take consecutive
        // rows when rows are grouped (their outputs are adjacent), else columns.
        const bool by_row = p.rg > 1;
        for (int e = tid; e < BM * BN; e += NT) {
            const int rr = by_row ? e % BM : e / BN, cc = by_row ? e / BM : e % BN;
            const int row = m0 + rr, col = n0 + cc;
            if (row >= p.M || col >= p.N) continue;
            const float r = smem[rr * CS + cc];
            if (SPLIT) {
                p.partial[(int64_t(z) * p.M + row) * p.N + col] = r;
            } else {
                int64_t o;
                float *dst = out_ptr(p, row, col, o);
                dst[o] = epilogue_value<EPI, FSILU>(p, row, col, o, r, p.bias ? p.bias[col] : 0.f);
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, int WK, int MODE, int PRO, bool F16, bool BVEC, int EPI, bool SPLIT,
          bool PIPE = false, int BKT = BK>
__global__ __launch_bounds__(64 * WM * WN * WK) void gemm_f32_kernel(GemmArgs p) {
    using L = Waves<BM, BN, WM, WN, WK>;
    constexpr int NT = L::kThreads;
    constexpr int MF = L::MF;
    using MI = Mf<MF>;
    constexpr int FM = L::FM, FN = L::FN;  // MF x MF blocks per wave
    // K per LDS stage: BK, or 16 for dense operands in the wide layouts (half
    // the staging registers and LDS, so big wave tiles keep several waves per SIMD)
    static_assert(BKT == BK || (BKT == 16 && MODE == kDense), "16-deep stages for dense operands only");
    constexpr int K4T = BKT / 4;           // float4 per tile row
    constexpr int KW = BKT / WK;           // K of each LDS stage per wave group
    static_assert(KW % MI::kKStep == 0, "whole float4 steps per wave group");
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    const TileIdx ti = tile_index(tiles_m, tiles_n);
    if (ti.y) {
        const int64_t bz = ti.y;
        p.a += bz * p.a_bs;
        p.b = static_cast<const char *>(p.b) + bz * p.b_bs * (F16 ? 2 : 4);
        p.out += bz * p.c_bs;
        if (p.res) p.res += bz * p.c_bs;
    }
    // Load slots: NT / K4 rows per pass, one float4 column each; the last pass of
    // a tile whose rows are not a multiple of that is partial.
    constexpr int RPP = NT / K4T;
    constexpr int A_LD = (BM + RPP - 1) / RPP, B_LD = (BN + RPP - 1) / RPP;
    // Two LDS stages: tile kt+1 is written while tile kt is read, one barrier
    // per K tile. The epilogue reuses the space for the C tile (row stride CS:
    // the two row halves of a 32x32 block's store fall on different banks).
    constexpr int CS = L::CS;
    // LDS row stride: BK + 4 for the 32x32 instruction; the 16x16 instruction's
    // lane layout (rows l % 16, K offsets 4 * (l / 16)) took 10% of its LDS
    // cycles in bank conflicts at that stride, and BK + 8 is 0.5% faster over a
    // UNet step (BK + 12 and + 20 cost a workgroup of occupancy and are slower).
    // (16-deep stages: BKT + 4, whose 80-byte rows put the 16 rows one read
    // instruction touches on distinct bank quads.)
    constexpr int LDS_S = BKT == 16 ? BKT + 4 : (MF == 16 ? BK + 8 : BK + 4);
    // The pipelined loop stores every load slot (rows past the tile land in
    // padding rows, read by no wave), so its loop body has no branch.
    constexpr int BMP = PIPE ? A_LD * RPP : BM, BNP = PIPE ? B_LD * RPP : BN;
    constexpr int STAGES = 2 * (BMP + BNP) * LDS_S;
    constexpr int EPI_F = L::kFixedQuads ? WK * BM * CS : (WK * BM * CS > BM * CS + 8 * NT ? WK * BM * CS
                                                                                        : BM * CS + 8 * NT);
    // The epilogue reuses the staging space: C tile (and GroupNorm sums past it).
    constexpr int SMEM = STAGES > EPI_F ? (STAGES > 2048 ? STAGES : 2048) : (EPI_F > 2048 ? EPI_F : 2048);
    static_assert(WK * BM * CS <= SMEM && SMEM >= 2048, "C tile and GroupNorm sums must fit in the staging space");
    static_assert(L::kFixedQuads || BM * CS + 8 * NT <= SMEM, "GroupNorm sums past the C tile");
    __shared__ float smem[SMEM];
    float(*As)[BMP * LDS_S] = reinterpret_cast<float(*)[BMP * LDS_S]>(smem);
    float(*Bs)[BNP * LDS_S] = reinterpret_cast<float(*)[BNP * LDS_S]>(smem + 2 * BMP * LDS_S);

    const int m0 = ti.tm * BM, n0 = ti.tn * BN;
    const int k_begin = SPLIT ? ti.z * p.k_split : 0;
    const int k_end = SPLIT ? min(p.K, k_begin + p.k_split) : p.K;
    const int ktiles = (k_end - k_begin + BKT - 1) / BKT;

    const int tid = threadIdx.x;
    const int lrow = tid / K4T, lc4 = tid % K4T;  // load slot: row within a pass, float4 column
    // Slot i holds tile row lrow + RPP * i when that is inside the tile; a slot
    // past it loads from row M / column N (out of range: zeros) and is not stored.
    auto a_in = [&](int i) { return BM % RPP == 0 || i + 1 < A_LD || lrow + RPP * i < BM; };
    auto b_in = [&](int i) { return BN % RPP == 0 || i + 1 < B_LD || lrow + RPP * i < BN; };

    ConvRow crow[A_LD];
    int arow[A_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        arow[i] = a_in(i) ? m0 + lrow + RPP * i : p.M;
        if (MODE >= kConvAligned) crow[i] = conv_row(p, arow[i]);
        else if (PRO == kProAffine) crow[i] = ConvRow{min(arow[i], p.M - 1) / p.pro_rows, 0, 0, true};
        else crow[i] = ConvRow{0, 0, 0, true};
    }

    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.a, p.a_bytes);
    const __amdgpu_buffer_rsrc_t a2_rsrc = make_rsrc(p.a2 ? p.a2 : p.a, p.a2 ? p.a2_bytes : p.a_bytes);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(p.b, p.b_bytes);
    // Two register stages (tiles kt+1 and kt+2 in flight while LDS stage kt&1
    // is consumed), two LDS stages: a load has two compute phases to land.
    floatx4 ra0[A_LD], rb0[B_LD], ra1[A_LD], rb1[B_LD];
    double ln_s1[A_LD], ln_s2[A_LD];  // kProLn: this thread's share of each slot row's sum and sum of squares
#pragma unroll
    for (int i = 0; i < A_LD; ++i) ln_s1[i] = ln_s2[i] = 0.0;
    auto fetch = [&](int kt, floatx4 (&ra)[A_LD], floatx4 (&rb)[B_LD]) {
        const int k0 = k_begin + kt * BKT;
        int tky = 0, tkx = 0, tci = 0;
        if (MODE == kConvAligned) {
            const int tap = k0 / p.ci;
            tci = k0 - tap * p.ci;
            tky = tap / 3;
            tkx = tap - tky * 3;
        }
        const int k = k0 + lc4 * 4;
        // a tile past ka reads the second operand (whole tiles: ka % BKT == 0)
        const bool sec = MODE == kDense && p.a2 && k0 >= p.ka;
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            if constexpr (MODE == kDense)
                ra[i] = sec ? load_a_buf<MODE, PRO>(p, a2_rsrc, crow[i], arow[i], k - p.ka, k_end - p.ka, tky, tkx, tci,
                                                    p.lda2)
                            : load_a_buf<MODE, PRO>(p, a_rsrc, crow[i], arow[i], k, k_end, tky, tkx, tci);
            else if constexpr (MODE == kConvAligned || MODE == kConvVec)
                ra[i] = load_a_buf<MODE, PRO>(p, a_rsrc, crow[i], arow[i], k, k_end, tky, tkx, tci);
            else
                ra[i] = (k < k_end) ? load_a<MODE, PRO>(p, crow[i], arow[i], k, tky, tkx, tci) : zero4();
        }
        if constexpr (PRO == kProLn) {  // row sums of the values as loaded (zeros outside the operand)
#pragma unroll
            for (int i = 0; i < A_LD; ++i) {
                const double a0 = ra[i][0], a1 = ra[i][1], a2 = ra[i][2], a3 = ra[i][3];
                ln_s1[i] += (a0 + a1) + (a2 + a3);
                ln_s2[i] += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
            }
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            const int n = b_in(i) ? n0 + lrow + RPP * i : p.N;
            if constexpr (BVEC)
                rb[i] = load_b_buf<F16>(p, b_rsrc, n, k, k_end);
            else
                rb[i] = (k < k_end) ? load_b<F16, BVEC>(p, n, k) : zero4();
        }
    };
    auto stash = [&](int buf, const floatx4 (&ra)[A_LD], const floatx4 (&rb)[B_LD]) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i)
            if (PIPE || a_in(i)) *reinterpret_cast<floatx4 *>(As[buf] + (lrow + RPP * i) * LDS_S + lc4 * 4) = ra[i];
#pragma unroll
        for (int i = 0; i < B_LD; ++i)
            if (PIPE || b_in(i)) *reinterpret_cast<floatx4 *>(Bs[buf] + (lrow + RPP * i) * LDS_S + lc4 * 4) = rb[i];
    };

    typename MI::Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < MI::kAccRegs; ++v) acc[i][j][v] = 0.f;

    // Lane l reads a float4 along K at row l % MF, K offset 4 * (l / MF): the
    // four lane groups (two for 32x32) each cover 4 consecutive K. Wave group
    // wk takes K columns [wk * KW, (wk + 1) * KW) of every stage.
    const int lane = tid & 63, wave = tid >> 6;
    int wm, wn, wk;
    L::index(wave, wm, wn, wk);
    const int a_off = (wm * L::TM + (lane % MF)) * LDS_S + (lane / MF) * 4 + wk * KW;
    const int b_off = (wn * L::TN + (lane % MF)) * LDS_S + (lane / MF) * 4 + wk * KW;
    auto compute = [&](int buf) {
        const float *as_w = As[buf] + a_off;
        const float *bs_w = Bs[buf] + b_off;
#pragma unroll
        for (int kk = 0; kk < KW; kk += MI::kKStep) {
            floatx4 a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = *reinterpret_cast<const floatx4 *>(as_w + i * MF * LDS_S + kk);
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = *reinterpret_cast<const floatx4 *>(bs_w + j * MF * LDS_S + kk);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] = MI::mfma(a[i][t], b[j][t], acc[i][j]);
        }
    };

    if constexpr (PIPE) {
        // One wave per SIMD (the wide layouts): the products of tile t run from
        // fragments already in registers, after the barrier that publishes tile
        // t+1 and after issuing that tile's fragment reads, its successor's LDS
        // store and the next global loads, so the matrix unit covers the barrier,
        // the LDS latency and the load issue. Two LDS stages, two register stages
        // (a global load has a whole iteration to land) and two fragment sets.
        // An LDS stage is rewritten only after a barrier that every wave passed
        // with its fragments of that stage's previous tile in registers.
        constexpr int KS = KW / MI::kKStep;  // float4 steps per stage and wave
        floatx4 fa0[KS][FM], fb0[KS][FN], fa1[KS][FM], fb1[KS][FN];
        auto read_frag = [&](int buf, floatx4 (&fa)[KS][FM], floatx4 (&fb)[KS][FN]) {
            const float *as_w = As[buf] + a_off;
            const float *bs_w = Bs[buf] + b_off;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    fa[s][i] = *reinterpret_cast<const floatx4 *>(as_w + i * MF * LDS_S + s * MI::kKStep);
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    fb[s][j] = *reinterpret_cast<const floatx4 *>(bs_w + j * MF * LDS_S + s * MI::kKStep);
            }
        };
        auto products = [&](const floatx4 (&fa)[KS][FM], const floatx4 (&fb)[KS][FN]) {
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int j = 0; j < FN; ++j) acc[i][j] = MI::mfma(fa[s][i][t], fb[s][j][t], acc[i][j]);
        };
        // Tiles past the end are fetched as zeros and never multiplied.
        fetch(0, ra0, rb0);
        fetch(1, ra1, rb1);
        stash(0, ra0, rb0);
        fetch(2, ra0, rb0);
        __syncthreads();
        read_frag(0, fa0, fb0);
        int t = 0;
        for (; t + 2 <= ktiles; t += 2) {
            stash(1, ra1, rb1);  // tile t+1
            fetch(t + 3, ra1, rb1);
            __syncthreads();
            read_frag(1, fa1, fb1);
            products(fa0, fb0);  // tile t
            stash(0, ra0, rb0);  // tile t+2
            fetch(t + 4, ra0, rb0);
            __syncthreads();
            read_frag(0, fa0, fb0);
            products(fa1, fb1);  // tile t+1
        }
        if (t < ktiles) products(fa0, fb0);  // an odd count: the last tile
    } else {
        // Even half: LDS 0 holds tile kt, registers 1 hold kt+1, registers 0 kt+2.
        // Odd half: LDS 1 holds kt+1, registers 0 hold kt+2, registers 1 kt+3.
        // Tiles past the end are fetched as zeros (out-of-range offsets) and never
        // computed; the loop body has no per-tile conditions, so the compiler waits
        // only for the older register stage before each LDS store.
        fetch(0, ra0, rb0);
        fetch(1, ra1, rb1);
        stash(0, ra0, rb0);
        fetch(2, ra0, rb0);
        __syncthreads();
        int kt = 0;
        for (; kt + 3 < ktiles; kt += 2) {  // four or more tiles left: one pair, no exits inside
            compute(0);
            stash(1, ra1, rb1);
            fetch(kt + 3, ra1, rb1);
            __syncthreads();
            compute(1);
            stash(0, ra0, rb0);
            fetch(kt + 4, ra0, rb0);
            __syncthreads();
        }
        // one to three tiles left: kt in LDS 0, kt+1 in registers 1, kt+2 in registers 0
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
    }

    // kProLn: each row's mean and 1 / sqrt(var + eps) from the sums of its K4T
    // load lanes (adjacent lanes of one wave), in f64, for the epilogue.
    __shared__ float ln_st[PRO >= kProLn ? 2 * BM : 1];
    if constexpr (PRO == kProLn)
        ln_row_stats<A_LD, RPP, K4T, BM>(p, ln_s1, ln_s2, lrow, lc4, ln_st);
    if constexpr (PRO == kProLnPart) ln_stats_from_parts<BM, NT>(p, m0, ln_st);
    __syncthreads();
    write_tile<BM, BN, WM, WN, WK, MF, EPI, SPLIT>(p, smem, acc, m0, n0, ti.z, PRO >= kProLn ? ln_st : nullptr);
}

// Sums split-K partials in split order, then (residual + bias) + sum [SiLU].
// VEC: four adjacent columns per thread (N, the output's leading dimensions and
// segment bounds multiples of 4, M * N < 2^31, 16-byte aligned buffers; checked
// by the launcher), so every load and store is 16 bytes wide.
template <int EPI, bool VEC, bool FSILU = false, bool OUT16 = false>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs p, int splits) {
    static_assert(!OUT16 || VEC, "f16 outputs: four columns at a time");
    const int64_t total = int64_t(p.M) * p.N;
    if constexpr (VEC) {
        const uint32_t n4 = uint32_t(p.N) >> 2;
        const uint32_t total4 = uint32_t(total >> 2);
        const float4 *pp = reinterpret_cast<const float4 *>(p.partial);
        for (uint32_t e = blockIdx.x * 256u + threadIdx.x; e < total4; e += gridDim.x * 256u) {
            float4 s = pp[e];
            for (int z = 1; z < splits; ++z) {
                const float4 t = pp[uint64_t(z) * total4 + e];
                s.x += t.x, s.y += t.y, s.z += t.z, s.w += t.w;
            }
            const int row = int(e / n4);
            store4<EPI, FSILU, OUT16>(p, row, int(e - uint32_t(row) * n4) << 2, s);
        }
    } else {
        for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
            float s = p.partial[e];
            for (int z = 1; z < splits; ++z) s += p.partial[int64_t(z) * total + e];
            const int row = int(e / p.N);
            const int col = int(e - int64_t(row) * p.N);
            int64_t o;
            float *dst = out_ptr(p, row, col, o);
            dst[o] = epilogue_value<EPI, FSILU>(p, row, col, o, s, p.bias ? p.bias[col] : 0.0f);
        }
    }
}

// Whether the split-K reduction may use 16-byte accesses (see splitk_reduce_kernel).
inline bool reduce_vec_ok(const GemmArgs &p) {
    return out_vec_ok(p, 1) == 1 && (reinterpret_cast<uintptr_t>(p.partial) & 15) == 0 &&
           int64_t(p.M) * p.N < (int64_t(1) << 31);
}

struct Plan {
    int bm, bn, splits, k_split;
    int wm = 2, wn = 2, wk = 1;  // wave layout (Waves)
    int pipe = 0;                // 1: the pipelined main loop (gemm_f32_kernel PIPE)
    int bk = BK;                 // K per LDS stage (gemm_f32_kernel BKT)
};

// Keeps the GroupNorm partials request (GemmArgs::gnp) when a BM x BN tiling
// without K split can honour it: one output, plain rows, 16-byte stores, tiles
// inside one item, and in the 2x2 wave layout a fixed column quad per epilogue
// thread (square: 256 % (BN / 4) == 0); other layouts sum from LDS, any width.
inline void gn_partials_plan(GemmArgs &p, int bm, int bn, int splits, int batch, bool square = true) {
    p.gn_rows = 0;
    if (!p.gnp) return;
    const bool ok = splits == 1 && batch == 1 && p.vec_out == 1 && p.nseg == 0 && p.rg <= 1 &&
                    (!square || 256 % (bn / 4) == 0) &&
                    p.gn_item_rows > 0 && p.gn_item_rows % bm == 0 && p.M % p.gn_item_rows == 0 &&
                    (reinterpret_cast<uintptr_t>(p.gnp) & 15) == 0;
    if (ok) p.gn_rows = bm;
    else p.gnp = nullptr;
}

// Keeps the LayerNorm row partials request (GemmArgs::lnp_out) when the tiling
// stores plain rows of 16-byte column quads in one pass (no K split, no
// batch, no segments or grouped rows), and sets the partials per row.
inline void ln_partials_plan(GemmArgs &p, int bn, int splits, int batch) {
    if (!p.lnp_out) return;
    const bool ok = splits == 1 && batch == 1 && p.vec_out == 1 && p.nseg == 0 && p.rg <= 1 &&
                    (reinterpret_cast<uintptr_t>(p.lnp_out) & 7) == 0;
    if (ok) p.lnp_ld = int(ceil_div(p.N, bn));
    else p.lnp_out = nullptr;
}

// Tile shape and K split, from sweeps of every (tile, split) on MI355X over
// the UNet's GEMM shapes (M 2..65536, N 4..6400, K 9..11520) and the VAE's
// convs (M up to 262144, K 1152..4608):
//  - Many 128x128 tiles (two per CU or more) and K >= 1024: 128x128, no split
//    (71-80% of f32 MFMA peak on the VAE's 3x3 convs, against 60-77% at 64x64).
//  - Long K (>= 4096, the upsample / downsample convs): 128x128 tiles, K split
//    in 3; 75-77% of f32 MFMA peak, against 67% unsplit.
//  - Dense operands (1x1 convs, linears): 64x64 tiles when there are four per
//    CU or more; 64x64 with K split in 3 for long K (>= 1536) on grids of
//    fewer than four 32x32 tiles per CU; otherwise 32x32 tiles (16x16 MFMA),
//    K split in up to 3 only under two tiles per CU with K >= 1024. Against
//    64x64 tiles with up to 6 splits this takes 10-30% off the UNet's
//    16x16- and 32x32-latent GEMMs (2048x640x640: 28.4 -> 19.7 us). With eight
//    32x32 tiles per CU or more, N % 64 == 0 and K < 1024, 32x64 tiles (half
//    the workgroups, two 16x16 blocks per wave): 8192x320x320 21.9 -> 20.6 us
//    (at K = 1280, 512x6400 with the SiLU epilogue, 32x64 is 5% slower).
//  - Implicit-GEMM convs otherwise: 64x64 tiles, K split while the grid is under
//    three times the CU count and each split keeps at least 8 K tiles.
inline Plan plan_for(int M, int N, int K, int cus, bool dense) {
    const int ktiles = int(ceil_div(K, BK));
    auto split = [&](int64_t tiles, int64_t target, int max_splits) {
        int want = 1;
        if (tiles < target) want = int(std::min<int64_t>(ceil_div(target, tiles), std::max(1, ktiles / 8)));
        want = std::max(1, std::min(want, max_splits));
        const int per = int(ceil_div(ktiles, want));
        return std::make_pair(int(ceil_div(ktiles, per)), per * BK);
    };
    const int64_t t128 = ceil_div(M, 128) * ceil_div(N, 128);
    if (K >= 1024 && t128 >= 2 * int64_t(cus)) return Plan{128, 128, 1, K};  // VAE-sized convs: 71-80%
    if (K >= 4096 && M >= 1024) {
        const auto s = split(t128, 3 * int64_t(cus), 3);
        return Plan{128, 128, s.first, s.second};
    }
    const int64_t t64 = ceil_div(M, 64) * ceil_div(N, 64);
    if (dense) {
        const int64_t t32 = ceil_div(M, 32) * ceil_div(N, 32);
        if (t64 >= 4 * int64_t(cus)) return Plan{64, 64, 1, K};
        if (K >= 1536 && t32 < 4 * int64_t(cus)) {
            const auto s = split(t64, 3 * t64, 3);
            return Plan{64, 64, s.first, s.first > 1 ? s.second : K};
        }
        if (K >= 1024 && t32 < 2 * int64_t(cus)) {
            const auto s = split(t32, 2 * int64_t(cus), 3);
            return Plan{32, 32, s.first, s.first > 1 ? s.second : K};
        }
        if (t32 >= 8 * int64_t(cus) && N % 64 == 0 && K < 1024) return Plan{32, 64, 1, K};
        return Plan{32, 32, 1, K};
    }
    const auto s = split(t64, 3 * int64_t(cus), 6);
    return Plan{64, 64, s.first, s.first > 1 ? s.second : K};
}

// Wide-layout plan for a dense GEMM with vector f32 weights, or bm = 0 to keep
// plan_for's. Timed inside the UNet step (kernel trace of a whole step, each
// GEMM in its place: cold weights, its producer's output just written back),
// which is not what a GEMM repeated on its own operands measures: of the
// layouts that beat the square tilings alone, these two also win in the step:
//  - the MixFFN's inverted 1x1 at 32x32 latents (N >= 3200, M >= 2048):
//    64x80 tiles of four 16x80 waves, pipelined loop (2048x3200x640: 79.8
//    against 84.2 us per launch);
//  - batched products of M <= 512 rows (the 16-plane Winograd GEMM of the
//    16x16 -> 32x32 upsample conv, 16 x 512x1280x1280): 64x80 tiles (224.5
//    against 248.9 us).
// Elsewhere the square tilings stay: in the step the wide layouts lost 5-60 us
// per shape (the 512-row GEMMs at K >= 1920 against the K-split tilings, the
// 8192x320 and 2048x640 GEMMs at K >= 640, the 512x6400 inverted 1x1).
inline Plan plan_wide(int M, int N, int K, int cus, int batch) {
    auto wide = [&](int bm, int bn, int wm, int wn, int wk, int pipe) {
        Plan p{bm, bn, 1, K, wm, wn, wk, pipe, BK};
        return p;
    };
    if (N % 80) return Plan{0, 0, 1, K};
    const int64_t t64 = ceil_div(M, 64) * ceil_div(N, 80);
    if (batch == 1 && N >= 3200 && M >= 2048 && t64 >= 2 * int64_t(cus)) return wide(64, 80, 4, 1, 1, 1);
    if (batch > 1 && M <= 512 && K >= 640 && t64 >= 2 * int64_t(cus)) return wide(64, 80, 4, 1, 1, 0);
    return Plan{0, 0, 1, K};
}

// The launch census (Tuning::gemm_log): one line per GEMM launch with its shape,
// tiling and epilogue, in launch order, to match against a kernel trace.
inline void log_gemm(const Context &ctx, const char *family, const GemmArgs &p, int bm, int bn, int splits, int mode,
                     int pro, bool f16, GemmEpilogue epi, int batch, int wm = 2, int wn = 2, int wk = 1) {
    if (!ctx.tune.gemm_log) return;
    std::fprintf(stderr,
                 "[gemm] %s M=%d N=%d K=%d batch=%d tile=%dx%d waves=%dx%dx%d splits=%d mode=%d pro=%d f16w=%d "
                 "silu=%d bias=%d res=%d rsc=%d res2=%d gnp=%d nseg=%d rg=%d a2=%d\n",
                 family, p.M, p.N, p.K, batch, bm, bn, wm, wn, wk, splits, mode, int(pro), int(f16),
                 int(epi == GemmEpilogue::Silu),
                 int(p.bias != nullptr), int(p.res != nullptr), int(p.rsc != nullptr), int(p.res2 != nullptr),
                 int(p.gnp != nullptr), p.nseg, p.rg, int(p.a2 != nullptr));
}

// Device timing of one GEMM launch (its split-K reduce included) while
// tune.gemm_time is set: an event before the launch here, one after it when the
// timer leaves scope, keyed by the kernel configuration and its grid.
struct GemmTimer {
    Context &ctx;
    bool on;
    GemmTimer(Context &c, const char *family, const GemmArgs &p, int bm, int bn, int wm, int wn, int wk, int splits,
              int mode, int batch)
        : ctx(c), on(c.tune.gemm_time != 0) {
        if (!on) return;
        const int64_t tiles = ceil_div(p.M, bm) * ceil_div(p.N, bn);
        char key[160];
        std::snprintf(key, sizeof key, "%s %dx%d waves %dx%dx%d mode %d grid %lldx%dx%d", family, bm, bn, wm, wn, wk,
                      mode, static_cast<long long>(tiles), splits > 1 ? 1 : batch, splits);
        Context::GemmTime g{key, 2.0 * double(p.M) * p.N * p.K * batch, c.take_event(), c.take_event()};
        HIP_CHECK(hipEventRecord(g.start, c.stream));
        c.gemm_times.push_back(std::move(g));
    }
    ~GemmTimer() {
        if (on) (void)hipEventRecord(ctx.gemm_times.back().stop, ctx.stream);
    }
    GemmTimer(const GemmTimer &) = delete;
    GemmTimer &operator=(const GemmTimer &) = delete;
};

template <int BM, int BN, int WM, int WN, int WK, int MODE, int PRO, bool F16, bool BVEC, bool PIPE = false,
          int BKT = BK>
void launch_cfg(Context &ctx, GemmArgs &p, const Plan &pl, GemmEpilogue epi, int batch) {
    constexpr int NT = Waves<BM, BN, WM, WN, WK>::kThreads;
    constexpr bool kSquare = Waves<BM, BN, WM, WN, WK>::kFixedQuads;
    const unsigned tiles = unsigned(ceil_div(p.M, BM) * ceil_div(p.N, BN));
    log_gemm(ctx, PIPE ? "f32p" : "f32", p, BM, BN, pl.splits, MODE, PRO, F16, epi, batch, WM, WN, WK);
    const GemmTimer timer(ctx, PIPE ? "f32p" : "f32", p, BM, BN, WM, WN, WK, pl.splits, MODE, batch);
    if (pl.splits > 1) {
        const size_t bytes = size_t(pl.splits) * p.M * p.N * sizeof(float);
        p.partial = static_cast<float *>(ctx.ws.get(bytes, ctx.stream));
        p.k_split = pl.k_split;
        p.vec_out = (p.N & 3) == 0 && (reinterpret_cast<uintptr_t>(p.partial) & 15) == 0;
        gn_partials_plan(p, BM, BN, pl.splits, batch, kSquare);
        ln_partials_plan(p, BN, pl.splits, batch);
        dim3 grid(tiles, 1, pl.splits);
        gemm_f32_kernel<BM, BN, WM, WN, WK, MODE, PRO, F16, BVEC, 0, true, PIPE, BKT><<<grid, NT, 0, ctx.stream>>>(p);
        MH_LAUNCH_CHECK();
        const int64_t total = int64_t(p.M) * p.N;
        if (reduce_vec_ok(p)) {
            const unsigned rb = unsigned(std::min<int64_t>(ceil_div(total / 4, 256), 8192));
            if (epi == GemmEpilogue::Silu)
                splitk_reduce_kernel<1, true><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
            else
                splitk_reduce_kernel<0, true><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
        } else {
            const unsigned rb = unsigned(std::min<int64_t>(ceil_div(total, 256), 8192));
            if (epi == GemmEpilogue::Silu)
                splitk_reduce_kernel<1, false><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
            else
                splitk_reduce_kernel<0, false><<<rb, 256, 0, ctx.stream>>>(p, pl.splits);
        }
    } else {
        p.k_split = p.K;
        p.vec_out = out_vec_ok(p, BM);
        gn_partials_plan(p, BM, BN, 1, batch, kSquare);
        ln_partials_plan(p, BN, 1, batch);
        const dim3 grid(tiles, unsigned(batch));
        // The SiLU epilogue is only instantiated for dense operands (the convs never use it).
        if constexpr (MODE <= kDenseScalar) {
            if (epi == GemmEpilogue::Silu) {
                gemm_f32_kernel<BM, BN, WM, WN, WK, MODE, PRO, F16, BVEC, 1, false, PIPE, BKT><<<grid, NT, 0, ctx.stream>>>(p);
                MH_LAUNCH_CHECK();
                return;
            }
        } else {
            MH_REQUIRE(epi == GemmEpilogue::None, "conv GEMM: SiLU epilogue not available");
        }
        gemm_f32_kernel<BM, BN, WM, WN, WK, MODE, PRO, F16, BVEC, 0, false, PIPE, BKT><<<grid, NT, 0, ctx.stream>>>(p);
    }
    MH_LAUNCH_CHECK();
}

// Wide wave layouts for dense operands with vector f32 weight rows: large
// per-wave tiles (16 or 32 rows x 80 columns, 48 x 48, 80 x 32) and grids of
// about one workgroup per CU, where the 2x2 layout of the square tiles needs
// many small workgroups (a 32x32 tile moves 8 KB per 64 KFLOP of products; a
// 128x80 tile 26 KB per 655 KFLOP). Entries: bm, bn, wm, wn, wk.
constexpr int kWide[][7] = {
    // bm, bn, wm, wn, wk, pipelined loop, K per stage: the planner's two
    // (64x80 of four 16x80 waves, plain and pipelined), and one of each other
    // code path (partial load passes, K split over wave groups, 16-deep stages)
    // for the gemm_plan tuning and the tests
    {64, 80, 4, 1, 1, 1, 32},
    {64, 80, 4, 1, 1, 0, 32},
    {128, 80, 4, 1, 1, 1, 32},  // waves 32x80
    {64, 160, 2, 2, 1, 1, 32},  // waves 32x80
    {32, 80, 2, 1, 2, 1, 32},   // waves 16x80, K split over two wave groups
    {32, 80, 2, 1, 2, 0, 32},
    {160, 64, 2, 2, 1, 1, 32},  // waves 80x32
    {160, 64, 2, 2, 1, 1, 16},  // 16-deep stages
    {64, 80, 4, 1, 1, 0, 16},
    {128, 128, 2, 2, 1, 1, 16},
};
constexpr int kWideCount = int(sizeof(kWide) / sizeof(kWide[0]));

inline int wide_index(const Plan &pl) {
    for (int i = 0; i < kWideCount; ++i)
        if (kWide[i][0] == pl.bm && kWide[i][1] == pl.bn && kWide[i][2] == pl.wm && kWide[i][3] == pl.wn &&
            kWide[i][4] == pl.wk && kWide[i][5] == pl.pipe && kWide[i][6] == pl.bk)
            return i;
    return -1;
}

template <int I, int MODE, int PRO, bool F16, bool BVEC>
void launch_wide(Context &ctx, GemmArgs &p, const Plan &pl, GemmEpilogue epi, int batch, int idx) {
    if constexpr (I < kWideCount) {
        if (idx == I) {
            launch_cfg<kWide[I][0], kWide[I][1], kWide[I][2], kWide[I][3], kWide[I][4], MODE, PRO, F16, BVEC,
                       kWide[I][5] != 0, kWide[I][6]>(ctx, p, pl, epi, batch);
            return;
        }
        launch_wide<I + 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch, idx);
    }
}

// The tiling the context's tuning forces on a GEMM of this shape: its
// gemm_shape_plan entry, else gemm_plan; false when neither applies.
inline bool forced_plan(const Tuning &t, int M, int N, int K, ShapePlan &f) {
    for (int i = 0; i < t.n_shape_plans; ++i) {
        const ShapePlan &s = t.shape_plans[i];
        if (s.m == M && s.n == N && s.k == K) {
            f = s;
            return true;
        }
    }
    if (t.gemm_splits <= 0) return false;
    f.bm = t.gemm_bm, f.bn = t.gemm_bn, f.splits = t.gemm_splits;
    f.wm = t.gemm_wm, f.wn = t.gemm_wn, f.wk = t.gemm_wk, f.pipe = t.gemm_pipe, f.bk = t.gemm_bk;
    return true;
}

template <int MODE, int PRO, bool F16, bool BVEC>
void launch_tiles(Context &ctx, GemmArgs &p, GemmEpilogue epi, int batch) {
    Plan pl = plan_for(p.M, p.N, p.K, int(ceil_div(ctx.cu_count, batch)), MODE <= kDenseScalar);
    constexpr bool kWideOk = MODE == kDense && BVEC && !F16;
    if constexpr (kWideOk) {
        const Plan w = ctx.tune.gemm_wide ? plan_wide(p.M, p.N, p.K, int(ceil_div(ctx.cu_count, batch)), batch)
                                          : Plan{0, 0, 1, p.K};
        if (w.bm) pl = w;
    }
    // The context's gemm_plan tuning ("bm,bn,splits[,wm,wn,wk]") forces the tiling
    // (tuning and A/B runs), as MOEBIUS_GEMM selects the CPU engine's GEMM backend
    // (src/engine/gemm.rs:57-60).
    ShapePlan fp;
    if (forced_plan(ctx.tune, p.M, p.N, p.K, fp)) {
        const int bm = fp.bm, bn = fp.bn, sp = fp.splits;
        Plan f{bm, bn, 1, p.K, fp.wm, fp.wn, fp.wk, fp.pipe, fp.bk};
        const bool square = (bm == 32 || bm == 64 || bm == 128) && (bn == 32 || bn == 64 || bn == 128) &&
                            (bm == 32) == (bn == 32) && f.wm == 2 && f.wn == 2 && f.wk == 1 && !f.pipe &&
                            f.bk == BK;
        const bool wide = ((bm == 32 && bn == 64) || (bm == 64 && bn == 32)) && f.wm == 2 && f.wn == 2 && f.wk == 1 &&
                          !f.pipe && f.bk == BK;
        if (square || (wide && MODE == kDense && BVEC) || (kWideOk && wide_index(f) >= 0)) {
            const int ktiles = int(ceil_div(p.K, BK));
            const int per = int(ceil_div(ktiles, sp));
            f.splits = int(ceil_div(ktiles, per));
            f.k_split = per * BK;
            pl = f;
        }
    }
    if (batch > 1 || PRO >= kProLn) pl.splits = 1;  // the folded LayerNorm needs whole rows of K
    if (pl.splits == 1) pl.k_split = p.K;
    if constexpr (kWideOk) {
        const int wi = wide_index(pl);
        if (wi >= 0) {
            launch_wide<0, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch, wi);
            return;
        }
    }
    if constexpr (MODE == kDense && BVEC) {  // 32x64 / 64x32 tiles: vector dense operands only
        if (pl.bm == 32 && pl.bn == 64) {
            launch_cfg<32, 64, 2, 2, 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
            return;
        }
        if (pl.bm == 64 && pl.bn == 32) {
            launch_cfg<64, 32, 2, 2, 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
            return;
        }
    }
    if constexpr (MODE <= kDenseScalar) {  // small tiles for the small dense GEMMs only
        if (pl.bm == 32) {
            launch_cfg<32, 32, 2, 2, 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
            return;
        }
    }
    if (pl.bm == 128 && pl.bn == 128)
        launch_cfg<128, 128, 2, 2, 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
    else if (pl.bm == 128)
        launch_cfg<128, 64, 2, 2, 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
    else if (pl.bn == 128)
        launch_cfg<64, 128, 2, 2, 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
    else
        launch_cfg<64, 64, 2, 2, 1, MODE, PRO, F16, BVEC>(ctx, p, pl, epi, batch);
}

template <int MODE, int PRO>
void launch_b(Context &ctx, GemmArgs &p, WeightType wt, GemmEpilogue epi, int batch = 1) {
    const int esz = wt == kF16 ? 2 : 4;
    const bool bvec = p.K % 4 == 0 && p.ldb % 4 == 0 && (reinterpret_cast<uintptr_t>(p.b) % (4 * esz)) == 0 &&
                      (batch == 1 || p.b_bs % 4 == 0);
    // Vector conv gathers come with vector weight rows (9 * c_in, c_in % 4 == 0);
    // the scalar gather takes any weight layout. Only those pairs are built.
    if constexpr (MODE == kConvAligned || MODE == kConvVec) {
        MH_REQUIRE(bvec, "conv GEMM: weight rows must be 4-element aligned for the vector gather");
        if (wt == kF16) launch_tiles<MODE, PRO, true, true>(ctx, p, epi, batch);
        else launch_tiles<MODE, PRO, false, true>(ctx, p, epi, batch);
    } else if constexpr (MODE == kConvScalar) {
        if (wt == kF16) launch_tiles<MODE, PRO, true, false>(ctx, p, epi, batch);
        else launch_tiles<MODE, PRO, false, false>(ctx, p, epi, batch);
    } else {
        if (wt == kF16) {
            if (bvec) launch_tiles<MODE, PRO, true, true>(ctx, p, epi, batch);
            else launch_tiles<MODE, PRO, true, false>(ctx, p, epi, batch);
        } else {
            if (bvec) launch_tiles<MODE, PRO, false, true>(ctx, p, epi, batch);
            else launch_tiles<MODE, PRO, false, false>(ctx, p, epi, batch);
        }
    }
}

}  // namespace
}  // namespace gemm
}  // namespace mh
