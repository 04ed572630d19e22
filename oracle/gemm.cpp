// Oracle GEMM: the semantics of moebius-cpu `engine::gemm::matmul`
// (src/engine/gemm.rs:63-132): c[m x n] = a . b, or c += a . b, with arbitrary
// operand strides (src/engine/gemm.rs:24-53 `MatRef`).
//
// The reference delegates the arithmetic to the `gemm` 0.19.0 and
// `private-gemm-x86` 0.1.22 crates (un-vendored, not in /root/reference); their
// internal summation order is not restated. This is a plain packed GEMM
// (Goto/BLIS blocking, 6x16 AVX2 FMA micro-kernel, OpenMP over blocks): every
// c element is one FMA chain over k in increasing order, seeded with c itself
// when accumulating. Pinned to tolerance by the reference's own gemm tests
// (src/engine/gemm.rs:139-187) restated in tests/.
#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "oracle.h"

namespace {

constexpr int MR = 6;
constexpr int NR = 16;
constexpr int64_t KC = 256;
constexpr int64_t MC = 120;  // multiple of MR
constexpr int64_t NCOLS = 64;  // columns per parallel task (multiple of NR)

struct AlignedBuf {
    float *p = nullptr;
    size_t cap = 0;
    ~AlignedBuf() { std::free(p); }
    float *get(size_t n) {
        if (n > cap) {
            std::free(p);
            cap = (n + 15) & ~size_t(15);
            p = static_cast<float *>(std::aligned_alloc(64, cap * sizeof(float)));
        }
        return p;
    }
};

// A block rows [i0, i0+mc) x k [p0, p0+kc) into MR-row panels: [panel][p][MR].
void pack_a(const float *a, int64_t rs, int64_t cs, int64_t i0, int64_t mc, int64_t p0, int64_t kc, float *dst) {
    for (int64_t ip = 0; ip < mc; ip += MR) {
        const int64_t rows = std::min<int64_t>(MR, mc - ip);
        float *d = dst + ip * kc;
        for (int64_t p = 0; p < kc; ++p) {
            const float *src = a + (i0 + ip) * rs + (p0 + p) * cs;
            for (int r = 0; r < MR; ++r) d[p * MR + r] = r < rows ? src[r * rs] : 0.0f;
        }
    }
}

// B block k [p0, p0+kc) x cols [j0, j0+nc) into NR-column panels: [panel][p][NR].
void pack_b(const float *b, int64_t rs, int64_t cs, int64_t p0, int64_t kc, int64_t j0, int64_t nc, float *dst) {
    for (int64_t jp = 0; jp < nc; jp += NR) {
        const int64_t cols = std::min<int64_t>(NR, nc - jp);
        float *d = dst + jp * kc;
        for (int64_t p = 0; p < kc; ++p) {
            const float *src = b + (p0 + p) * rs + (j0 + jp) * cs;
            if (cs == 1 && cols == NR) {
                std::memcpy(d + p * NR, src, NR * sizeof(float));
            } else {
                for (int j = 0; j < NR; ++j) d[p * NR + j] = j < cols ? src[j * cs] : 0.0f;
            }
        }
    }
}

// c[6 x 16] (ldc) (+)= Ap . Bp over kc; rows/cols < MR/NR go through a buffer.
void micro_kernel(int64_t kc, const float *ap, const float *bp, float *c, int64_t ldc, bool load_c, int rows,
                  int cols) {
    alignas(32) float tmp[MR * NR];
    float *dst = c;
    int64_t ld = ldc;
    const bool full = rows == MR && cols == NR;
    if (!full) {
        dst = tmp;
        ld = NR;
        for (int r = 0; r < MR; ++r)
            for (int j = 0; j < NR; ++j) tmp[r * NR + j] = (load_c && r < rows && j < cols) ? c[r * ldc + j] : 0.0f;
    }
    __m256 acc[MR][2];
    for (int r = 0; r < MR; ++r) {
        if (load_c || !full) {
            acc[r][0] = _mm256_loadu_ps(dst + r * ld);
            acc[r][1] = _mm256_loadu_ps(dst + r * ld + 8);
        } else {
            acc[r][0] = _mm256_setzero_ps();
            acc[r][1] = _mm256_setzero_ps();
        }
    }
    for (int64_t p = 0; p < kc; ++p) {
        const __m256 b0 = _mm256_load_ps(bp + p * NR);
        const __m256 b1 = _mm256_load_ps(bp + p * NR + 8);
        for (int r = 0; r < MR; ++r) {
            const __m256 av = _mm256_broadcast_ss(ap + p * MR + r);
            acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
            acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
        }
    }
    for (int r = 0; r < MR; ++r) {
        _mm256_storeu_ps(dst + r * ld, acc[r][0]);
        _mm256_storeu_ps(dst + r * ld + 8, acc[r][1]);
    }
    if (!full) {
        for (int r = 0; r < rows; ++r)
            for (int j = 0; j < cols; ++j) c[r * ldc + j] = tmp[r * NR + j];
    }
}

}  // namespace

extern "C" void orc_matmul(float *c, const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                           int64_t b_cs, int64_t m, int64_t k, int64_t n, int accumulate) {
    if (m <= 0 || n <= 0) return;
    if (k <= 0) {
        if (!accumulate)
            for (int64_t i = 0; i < m * n; ++i) c[i] = 0.0f;
        return;
    }
    const int64_t nb_panels = (n + NR - 1) / NR;
    static thread_local AlignedBuf bbuf;
    float *bp = bbuf.get(size_t(nb_panels) * NR * KC);
    for (int64_t p0 = 0; p0 < k; p0 += KC) {
        const int64_t kc = std::min<int64_t>(KC, k - p0);
        const bool load_c = accumulate || p0 > 0;
#pragma omp parallel for schedule(static)
        for (int64_t jp = 0; jp < nb_panels; ++jp) {
            const int64_t j0 = jp * NR;
            pack_b(b, b_rs, b_cs, p0, kc, j0, std::min<int64_t>(NR, n - j0), bp + jp * NR * kc);
        }
        const int64_t mblocks = (m + MC - 1) / MC;
        const int64_t nblocks = (n + NCOLS - 1) / NCOLS;
#pragma omp parallel
        {
            static thread_local AlignedBuf abuf;
            float *ap = abuf.get(size_t(MC) * KC);
#pragma omp for collapse(2) schedule(dynamic)
            for (int64_t ib = 0; ib < mblocks; ++ib) {
                for (int64_t jb = 0; jb < nblocks; ++jb) {
                    const int64_t i0 = ib * MC, mc = std::min<int64_t>(MC, m - i0);
                    pack_a(a, a_rs, a_cs, i0, mc, p0, kc, ap);
                    const int64_t j_end = std::min<int64_t>(n, (jb + 1) * NCOLS);
                    for (int64_t j0 = jb * NCOLS; j0 < j_end; j0 += NR) {
                        const int cols = int(std::min<int64_t>(NR, n - j0));
                        const float *bpanel = bp + (j0 / NR) * NR * kc;
                        for (int64_t ir = 0; ir < mc; ir += MR) {
                            const int rows = int(std::min<int64_t>(MR, mc - ir));
                            micro_kernel(kc, ap + ir * kc, bpanel, c + (i0 + ir) * n + j0, n, load_c, rows, cols);
                        }
                    }
                }
            }
        }
    }
}

extern "C" void orc_set_threads(int threads) {
    if (threads > 0) omp_set_num_threads(threads);
}

extern "C" int orc_get_threads(void) { return omp_get_max_threads(); }
