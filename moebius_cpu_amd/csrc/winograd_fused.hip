// Winograd F(2x2, 3x3) conv in one kernel (src/engine/winograd.rs:48-120):
// the input transform, the 16 plane products and the output transform of a
// block of 32 tiles x 64 output channels stay on chip, so V and M (16 planes
// of tiles x channels each) never reach HBM. The separate path writes and
// reads both: about 4.2 GB per 512x512x128 conv of the VAE decoder.
//
// Workgroup: 512 threads, one per CU (LDS: two V stages of 72 KB), walking
// a share of the (channel block, tile block) items. Per chunk of 32 input
// channels every thread transforms one tile's 4x4 patch for two channels (the
// reference's operation order, as wino_input_kernel) into the V stage
// [plane][tile][channel]; the 16 channel pairs of a tile sit on adjacent
// lanes, so a patch load reads 128-byte runs. Wave w (of 8, two per SIMD)
// multiplies planes 2w and 2w + 1 on v_mfma_f32_32x32x2f32 (tiles x 64
// channels, two 32x32 blocks per plane), reading V from LDS and U from global
// memory (L2 resident) in the fused order [16][ci / 8][co][8]: the 32
// channels of one block at one K sub-step are 1 KB of consecutive bytes, so
// each U load of a wave reads whole cache lines (from [16][co][ci] a load
// touches 32 lines for 32 bytes each). The next chunk's patch loads are in
// flight during the current chunk's last three quarters of products. At the
// end the 16 planes go through LDS and each thread applies the output
// transform (winograd.rs:329-352, as wino_output_kernel) to one tile and four
// channels, adding bias and the optional residual.
//
// At 512x512x128 -> 128 (A/B on MI355X): 730 us for transforms + batched
// GEMM; this kernel with U in [16][co][ci] order and a tile's channels on
// lanes 32 apart, 495 us (with its MFMAs removed it still took 490 us: the
// operand loads bound it); with the layouts above 372 us; one workgroup per
// CU with the next item's loads issued early, 361 us; every thread a
// producer, 358 us (256x256x256: 347 -> 334, upsampled 128x128x512:
// 1327 -> 1286). The products alone run at 91% of the f32 MFMA peak.
#include <algorithm>

#include "common.hpp"
#include "dmath.hpp"
#include "kernels.hpp"

namespace mh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

constexpr int kFT = 32;        // tiles per workgroup
constexpr int kFC = 64;        // output channels per workgroup
constexpr int kFK = 32;        // input channels per chunk
constexpr int kVS = kFK + 4;   // V row stride in LDS (floats)
constexpr int kMS = kFC + 4;   // M row stride in LDS (floats)
constexpr int kVStage = 16 * kFT * kVS;
constexpr int kLds = 2 * kVStage;  // 36864 floats = 144 KB
static_assert(16 * kFT * kMS <= kLds, "the M exchange fits in the V stages");
constexpr int kRed = 16 * kFT * kMS;  // GroupNorm reduction scratch, past the M exchange
static_assert(kRed + 2 * 8 * 64 <= kLds && kRed >= kVStage, "reduction scratch fits, in V stage 1");
constexpr int kOob = int(0x80000000u);

struct FGeo {
    int h, w, hi, wi, th, tw;
    int64_t tiles;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), short(0), int(bytes), 0x00020000);
}

__device__ __forceinline__ floatx4 ld4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ floatx2 ld2(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(floatx2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

__device__ __forceinline__ floatx4 sub4(floatx4 a, floatx4 b) { return floatx4{a[0] - b[0], a[1] - b[1], a[2] - b[2], a[3] - b[3]}; }
__device__ __forceinline__ floatx4 add4(floatx4 a, floatx4 b) { return floatx4{a[0] + b[0], a[1] + b[1], a[2] + b[2], a[3] + b[3]}; }

constexpr int kFThreads = 512;  // 8 waves, two per SIMD
constexpr int kFPlanes = 16 / (kFThreads / 64);  // planes per wave

template <int UP, bool PRO>
__global__ __launch_bounds__(kFThreads, 2) void wino_fused_kernel(const float *__restrict__ x, uint32_t x_bytes, FGeo g,
                                                            int ci, const float *__restrict__ u, uint32_t u_bytes,
                                                            int co, const float *__restrict__ psc,
                                                            const float *__restrict__ psh, int psilu,
                                                            const float *__restrict__ bias,
                                                            const float *__restrict__ res2, float *__restrict__ out,
                                                            float *__restrict__ gnp, int nco_blocks, int nwork) {
    __shared__ float lds[kLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Work items (channel block, tile block), channel block outer. Workgroup i
    // runs on XCD i % 8 (round-robin dispatch); each XCD takes one contiguous
    // eighth of the items, so it works through few channel blocks and their U
    // panels stay in its L2, and its workgroups take every (grid / 8)-th item
    // of that range. The grid holds one workgroup per CU, and a workgroup
    // issues its next item's first patch and U loads before the current
    // item's last products and output transform, which hide their latency.
    const int ntb = nwork / nco_blocks;
    const int per_xcd = (nwork + 7) / 8;
    const int slots = int(gridDim.x) / 8;
    const int item_end = min(nwork, (int(blockIdx.x) % 8 + 1) * per_xcd);
    int item = (int(blockIdx.x) % 8) * per_xcd + int(blockIdx.x) / 8;
    if (item >= item_end) return;
    const __amdgpu_buffer_rsrc_t xr = rsrc(x, x_bytes), ur = rsrc(u, u_bytes);
    const int per_item = g.th * g.tw;
    const int n_items = int(g.tiles / per_item);

    // Producer role (every thread, so the transform's work is spread over
    // both waves of each SIMD): tile vt of the block, channel pair vq of the
    // chunk; the 16 pairs of a tile sit on 16 adjacent lanes (128-byte runs).
    const int vq = tid & (kFK / 2 - 1), vt = (tid >> 4) & (kFT - 1);
    // Consumer role: wave w, planes kFPlanes w .. + kFPlanes - 1, two 32x32 blocks of 64 channels.
    // Lane l reads a float4 along K of row l % 32 at K offset 4 (l / 32); MFMA t
    // takes its component t, so both operands pair k = 8 s + 4 (l / 32) + t.
    const int row = lane & 31, kq = 4 * (lane >> 5);
    // Per item: the block's first tile and channel; the producer's patch
    // origin (byte offset of source pixel (sy - 1, sx - 1), channel 4 vq; the
    // patch's rows and columns sit at -1, 0, 1, 2 from (sy, sx), or -1, 0, 0, 1
    // when upsampling) with one bit per pixel inside the image, and its batch
    // item; the consumer's U offsets in [16][ci / 8][co][8] (plane
    // kFPlanes w + p, channel co0 + 32 j + row, K offset kq within the
    // sub-step's 8; sub-step k8 adds k8 * co * 8 floats).
    int64_t t0 = 0;
    int co0 = 0, vb = 0, porg = 0;
    unsigned valid = 0;
    int uoff[kFPlanes][2];
    const int prow = g.w * ci * 4, pcol = ci * 4;  // bytes per source row, per pixel
    constexpr int kStep[4] = {0, 1, 2 - UP, 3 - UP};  // patch row / column k -> source offset + 1
    auto setup = [&](int it) {
        t0 = int64_t(it % ntb) * kFT;
        co0 = (it / ntb) * kFC;
        const int64_t tv = t0 + vt;
        const int b = int(tv / per_item), rem = int(tv - int64_t(b) * per_item);
        const int ty = rem / g.tw, tx = rem - ty * g.tw;
        vb = min(b, n_items - 1);  // a tile past the end reads nothing, but keeps its prologue loads in range
        const int sy = (2 * ty) >> UP, sx = (2 * tx) >> UP;
        porg = tv < g.tiles ? (((b * g.h + sy - 1) * g.w + sx - 1) * ci + 2 * vq) * 4 : 0;
        valid = 0;
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            const int iy = 2 * ty + (kk >> 2) - 1, ix = 2 * tx + (kk & 3) - 1;
            const bool in = tv < g.tiles && iy >= 0 && iy < g.hi && ix >= 0 && ix < g.wi;
            valid |= in ? (1u << kk) : 0u;
        }
#pragma unroll
        for (int p = 0; p < kFPlanes; ++p)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                uoff[p][j] = ((((kFPlanes * wave + p) * (ci / 8)) * co + co0 + 32 * j + row) * 8 + kq) * 4;
    };
    floatx2 d[16];
    auto produce = [&](int kc) {
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            const int off = porg + kStep[kk >> 2] * prow + kStep[kk & 3] * pcol + kc * kFK * 4;
            d[kk] = ld2(xr, (valid >> kk) & 1u ? off : kOob);
        }
    };
    auto transform_store = [&](int kc, int stage) {
        if constexpr (PRO) {
            const int c = kc * kFK + 2 * vq;
            const floatx2 sc = *reinterpret_cast<const floatx2 *>(psc + int64_t(vb) * ci + c);
            const floatx2 sh = *reinterpret_cast<const floatx2 *>(psh + int64_t(vb) * ci + c);
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                if (valid & (1u << kk)) {
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        float y = __builtin_fmaf(d[kk][e], sc[e], sh[e]);
                        if (psilu) y = ref_silu(y);
                        d[kk][e] = y;
                    }
                }
            }
        }
        floatx2 tt[16];
#pragma unroll
        for (int col = 0; col < 4; ++col) {
            const floatx2 d0 = d[col], d1 = d[4 + col], d2 = d[8 + col], d3 = d[12 + col];
            tt[col] = d0 - d2;
            tt[4 + col] = d1 + d2;
            tt[8 + col] = d2 - d1;
            tt[12 + col] = d1 - d3;
        }
        float *vs = lds + stage * kVStage + vt * kVS + 2 * vq;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const floatx2 *q = tt + r * 4;
            *reinterpret_cast<floatx2 *>(vs + (r * 4) * kFT * kVS) = q[0] - q[2];
            *reinterpret_cast<floatx2 *>(vs + (r * 4 + 1) * kFT * kVS) = q[1] + q[2];
            *reinterpret_cast<floatx2 *>(vs + (r * 4 + 2) * kFT * kVS) = q[2] - q[1];
            *reinterpret_cast<floatx2 *>(vs + (r * 4 + 3) * kFT * kVS) = q[1] - q[3];
        }
    };

    floatx16 acc[kFPlanes][2];
    // Loads are waited for in issue order, so the order is chosen to never
    // wait on more than the next operands: U for sub-step 1 is issued with
    // sub-step 0, U for sub-steps 2 and 3 with sub-step 1 and after them the
    // next chunk's patch (it lands during the last three sub-steps' products;
    // the transform waits for it), and U for the next chunk's first sub-step
    // after the last products, to land during the transform.
    static_assert(kFK / 8 == 4, "four K sub-steps per chunk");
    floatx4 b0[kFPlanes][2], b1[kFPlanes][2], b2[kFPlanes][2], b3[kFPlanes][2];
    auto load_b = [&](floatx4 (&dst)[kFPlanes][2], int kc, int s) {
#pragma unroll
        for (int p = 0; p < kFPlanes; ++p)
#pragma unroll
            for (int j = 0; j < 2; ++j) dst[p][j] = ld4(ur, uoff[p][j] + (kc * (kFK / 8) + s) * co * 32);
    };
    auto mfma_step = [&](const float *vs, int s, const floatx4 (&b)[kFPlanes][2]) {
        floatx4 a[kFPlanes];
#pragma unroll
        for (int p = 0; p < kFPlanes; ++p)
            a[p] = *reinterpret_cast<const floatx4 *>(vs + (kFPlanes * wave + p) * kFT * kVS + 8 * s);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int p = 0; p < kFPlanes; ++p)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[p][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[p][t], b[p][j][t], acc[p][j], 0, 0, 0);
    };
    const int nk = ci / kFK;
    setup(item);
    produce(0);
    load_b(b0, 0, 0);
    for (;;) {
        transform_store(0, 0);
#pragma unroll
        for (int p = 0; p < kFPlanes; ++p)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[p][j][v] = 0.f;
        __syncthreads();
        const int next = item + slots;
        const bool has_next = next < item_end;
        const int64_t et0 = t0;
        const int eco0 = co0;
        for (int kc = 0; kc < nk; ++kc) {
            const bool more = kc + 1 < nk;
            const float *vs = lds + (kc & 1) * kVStage + row * kVS + kq;
            load_b(b1, kc, 1);
            mfma_step(vs, 0, b0);
            load_b(b2, kc, 2);
            load_b(b3, kc, 3);
            if (more) {
                produce(kc + 1);
            } else if (has_next) {  // this item's U loads are all issued: switch to the next
                setup(next);
                produce(0);
            }
            mfma_step(vs, 1, b1);
            mfma_step(vs, 2, b2);
            mfma_step(vs, 3, b3);
            if (more) {
                load_b(b0, kc + 1, 0);
                transform_store(kc + 1, (kc + 1) & 1);
            } else if (has_next) {
                load_b(b0, 0, 0);
            }
            __syncthreads();
        }

    // M [16][tile][channel] through LDS: register v of lane l holds row
    // 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32 of its block.
#pragma unroll
    for (int p = 0; p < kFPlanes; ++p)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int tr = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                lds[((kFPlanes * wave + p) * kFT + tr) * kMS + 32 * j + row] = acc[p][j][v];
            }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < (kFT * kFC / 4) / kFThreads; ++r) {
        const int item = tid + kFThreads * r;
        const int tl = item / (kFC / 4), q = item - tl * (kFC / 4);
        const int64_t t = et0 + tl;
        if (t >= g.tiles) continue;
        const int b = int(t / per_item), rem = int(t - int64_t(b) * per_item);
        const int ty = rem / g.tw, tx = rem - ty * g.tw;
        const float *src = lds + tl * kMS + 4 * q;
        floatx4 u0[4], u1[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(src + (rr * 4) * kFT * kMS);
            const floatx4 bb = *reinterpret_cast<const floatx4 *>(src + (rr * 4 + 1) * kFT * kMS);
            const floatx4 cc = *reinterpret_cast<const floatx4 *>(src + (rr * 4 + 2) * kFT * kMS);
            const floatx4 dd = *reinterpret_cast<const floatx4 *>(src + (rr * 4 + 3) * kFT * kMS);
            u0[rr] = add4(add4(a, bb), cc);
            u1[rr] = sub4(sub4(bb, cc), dd);
        }
        const int c = eco0 + 4 * q;
        const floatx4 bv = bias ? *reinterpret_cast<const floatx4 *>(bias + c) : floatx4{0.f, 0.f, 0.f, 0.f};
        floatx4 gs{0.f, 0.f, 0.f, 0.f}, gq = gs;  // GroupNorm sums of the values stored
        floatx4 y[4];
        y[0] = add4(add4(add4(u0[0], u0[1]), u0[2]), bv);
        y[1] = add4(add4(add4(u1[0], u1[1]), u1[2]), bv);
        y[2] = add4(sub4(sub4(u0[1], u0[2]), u0[3]), bv);
        y[3] = add4(sub4(sub4(u1[1], u1[2]), u1[3]), bv);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int oy = 2 * ty + (kk >> 1), ox = 2 * tx + (kk & 1);
            if (oy >= g.hi || ox >= g.wi) continue;
            const int64_t o = ((int64_t(b) * g.hi + oy) * g.wi + ox) * co + c;
            floatx4 rv = y[kk];
            if (res2) rv = add4(rv, *reinterpret_cast<const floatx4 *>(res2 + o));
            *reinterpret_cast<floatx4 *>(out + o) = rv;
            if (gnp) {
                gs = add4(gs, rv);
#pragma unroll
                for (int e = 0; e < 4; ++e) gq[e] = __builtin_fmaf(rv[e], rv[e], gq[e]);
            }
        }
        if (gnp) {
            // GroupNorm partials of this block (per channel: sum and sum of
            // squares over its 128 pixels), for the next GroupNorm's fold in
            // place of a statistics pass: the four threads of a wave that hold
            // channel quad q (tiles 4w .. 4w + 3) by xor butterfly, then the
            // eight waves in order through LDS past the M exchange (V stage 1,
            // not written again before the next item's second chunk).
#pragma unroll
            for (int off = 16; off < 64; off <<= 1)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    gs[e] += __shfl_xor(gs[e], off, 64);
                    gq[e] += __shfl_xor(gq[e], off, 64);
                }
            floatx4 *red = reinterpret_cast<floatx4 *>(lds + kRed);
            if (lane < kFC / 4) {
                red[wave * (kFC / 4) + lane] = gs;
                red[(kFThreads / 64 + wave) * (kFC / 4) + lane] = gq;
            }
            __syncthreads();
            if (tid < kFC / 4) {
                floatx4 ts = red[tid], tq = red[(kFThreads / 64) * (kFC / 4) + tid];
#pragma unroll
                for (int w8 = 1; w8 < kFThreads / 64; ++w8) {
                    ts = add4(ts, red[w8 * (kFC / 4) + tid]);
                    tq = add4(tq, red[(kFThreads / 64 + w8) * (kFC / 4) + tid]);
                }
                float *dst = gnp + ((et0 / kFT) * co + eco0 + 4 * tid) * 2;
                *reinterpret_cast<floatx4 *>(dst) = floatx4{ts[0], tq[0], ts[1], tq[1]};
                *reinterpret_cast<floatx4 *>(dst + 4) = floatx4{ts[2], tq[2], ts[3], tq[3]};
            }
        }
    }
        if (!has_next) break;
        __syncthreads();  // the output transform's reads of M are done before V stage 0 is written
        item = next;
    }
}

// u [16][co][ci] -> uf [16][ci / 8][co][8], one float4 per thread.
__global__ void wino_u_fused_kernel(const float *__restrict__ u, int co, int ci, float *__restrict__ uf) {
    const int64_t total4 = int64_t(16) * co * ci / 4;
    for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total4; e += int64_t(gridDim.x) * blockDim.x) {
        const int64_t f = e * 4, plane_sz = int64_t(co) * ci;
        const int64_t plane = f / plane_sz, rem = f - plane * plane_sz;
        const int k8 = int(rem / (int64_t(co) * 8));
        const int r2 = int(rem - int64_t(k8) * co * 8), c = r2 >> 3, kk = r2 & 7;
        *reinterpret_cast<floatx4 *>(uf + f) =
            *reinterpret_cast<const floatx4 *>(u + (plane * co + c) * ci + k8 * 8 + kk);
    }
}

template <int UP, bool PRO>
void launch_fused(Context &ctx, int nwork, const float *x, uint32_t xb, const FGeo &g, int ci, const float *u,
                  uint32_t ub, int co, const Affine *pro, const float *bias, const float *res2, float *out,
                  float *gnp) {
    // one workgroup per CU (its LDS holds one), a multiple of 8 (see the work
    // order in the kernel), no more than the items of one XCD's share need
    const int64_t per_xcd = ceil_div(nwork, 8);
    const unsigned grid = unsigned(8 * std::max<int64_t>(1, std::min<int64_t>(ctx.cu_count / 8, per_xcd)));
    wino_fused_kernel<UP, PRO><<<grid, kFThreads, 0, ctx.stream>>>(x, xb, g, ci, u, ub, co, pro ? pro->scale : nullptr,
                                                             pro ? pro->shift : nullptr, pro && pro->silu ? 1 : 0,
                                                             bias, res2, out, gnp, co / kFC, nwork);
}

}  // namespace

void winograd_fused_weights(Context &ctx, const float *u, int c_out, int c_in, float *uf) {
    MH_REQUIRE(c_in % 8 == 0 && aligned16(u) && aligned16(uf), "Winograd fused weights: c_in % 8, 16-byte aligned");
    const int64_t total4 = int64_t(16) * c_out * c_in / 4;
    if (total4 == 0) return;
    const unsigned blocks = unsigned(std::min<int64_t>(ceil_div(total4, 256), 65536));
    wino_u_fused_kernel<<<blocks, 256, 0, ctx.stream>>>(u, c_out, c_in, uf);
    MH_LAUNCH_CHECK();
}

bool conv3x3_winograd_fused(Context &ctx, const float *x, int n, int h, int w, int c_in, const float *u,
                            const float *uf, int c_out, const float *bias, bool upsample2x, const Affine *prologue,
                            float *out, const float *residual2, GnPartials *gn) {
    if (gn) gn->rows = 0;
    if (ctx.tune.wino_fused == 0 || c_in % kFK || c_out % kFC) return false;
    // Where it is faster (A/B per conv on MI355X, three kernels -> this one):
    // 512x512x128 746 -> 419 us, 256x256x256 552 -> 401, the same upsampled
    // 1824 -> 1352, 128x128x512 437 -> 402, the same upsampled 1471 -> 1335;
    // slower on small maps, where the batched plane GEMM fills the chip at 83%
    // of f32 MFMA peak and the V / M traffic is small: 64x64x512 100 -> 117 us,
    // the UNet's 2x64x64x320 92 -> 124, 2x32x32x640 upsampled 281 -> 348. So:
    // at least 4096 tiles, up to the measured 512 channels.
    if (ctx.tune.wino_fused < 0 && (c_in > 512 || c_out > 512)) return false;
    if (!aligned16(x) || !aligned16(u) || !aligned16(out) || !aligned16(bias) || !aligned16(residual2)) return false;
    if (prologue && (!aligned16(prologue->scale) || !aligned16(prologue->shift))) return false;
    const int64_t x_bytes = int64_t(n) * h * w * c_in * 4, u_bytes = int64_t(16) * c_out * c_in * 4;
    if (x_bytes >= (int64_t(1) << 31) || u_bytes >= (int64_t(1) << 31)) return false;
    FGeo g;
    const int up = upsample2x ? 1 : 0;
    g.h = h, g.w = w, g.hi = h << up, g.wi = w << up;
    g.th = (g.hi + 1) / 2, g.tw = (g.wi + 1) / 2;
    g.tiles = int64_t(n) * g.th * g.tw;
    if (ctx.tune.wino_fused < 0 && g.tiles < 4096) return false;
    if (g.tiles == 0) return true;
    const int64_t blocks = ceil_div(g.tiles, kFT) * (c_out / kFC);
    if (blocks >= (int64_t(1) << 30)) return false;
    const int nwork = int(blocks);
    const uint32_t xb = uint32_t(x_bytes), ub = uint32_t(u_bytes);
    if (!uf) {  // no precomputed fused-order copy: make one in the workspace
        float *tmp = static_cast<float *>(ctx.ws.get(size_t(u_bytes), ctx.stream));
        winograd_fused_weights(ctx, u, c_out, c_in, tmp);
        uf = tmp;
    } else if (!aligned16(uf)) {
        return false;
    }
    u = uf;
    // GroupNorm partials: blocks of 32 whole tiles (128 pixels) within one item
    float *gnp = nullptr;
    if (gn && gn->part && aligned16(gn->part) && g.hi % 2 == 0 && g.wi % 2 == 0 &&
        int64_t(g.th) * g.tw % kFT == 0 && gn->item_rows == g.hi * g.wi) {
        gnp = gn->part;
        gn->rows = 4 * kFT;
    }
    if (up) {
        if (prologue) launch_fused<1, true>(ctx, nwork, x, xb, g, c_in, u, ub, c_out, prologue, bias, residual2, out, gnp);
        else launch_fused<1, false>(ctx, nwork, x, xb, g, c_in, u, ub, c_out, prologue, bias, residual2, out, gnp);
    } else {
        if (prologue) launch_fused<0, true>(ctx, nwork, x, xb, g, c_in, u, ub, c_out, prologue, bias, residual2, out, gnp);
        else launch_fused<0, false>(ctx, nwork, x, xb, g, c_in, u, ub, c_out, prologue, bias, residual2, out, gnp);
    }
    MH_LAUNCH_CHECK();
    return true;
}

}  // namespace mh
