/*
 * CPU baseline: the reference's pooled CPU kernels, restated with AVX2+FMA and OpenMP.
 *
 * TEST/BENCH INFRASTRUCTURE ONLY (see oracle.h): bench.py times this beside the GPU path.
 *
 * - GEMM: matmul_reuse (src/kernel.rs:1383-1477) with the production knobs (96-row activation
 *   tile, 4-row groups, two dequantized weight rows per pass, r_block 1024;
 *   kernel.rs:1328-1369). The inner step is dot_f32_avx2_x4x2 (kernel.rs:1162-1202): two weight
 *   rows against four activation rows, one 8-lane FMA accumulator per output, hsum, scalar tail.
 * - Split-axis policy of QMat::matmul (src/qmat.rs:185-272): X <= 6 MiB splits activation rows,
 *   larger X splits weight (output) rows.
 * - GEMV: QMat::matvec's row split (qmat.rs:97-124); each row dequantizes block by block and
 *   folds the block into an 8-lane FMA accumulator (the reference's fused AVX2 dots,
 *   kernel.rs:488-954, follow the same per-block dequant + FMA structure).
 * - Pool: OpenMP's persistent team stands in for src/pool.rs:145-163.
 * Rows whose length n is not a multiple of the block size are stored as whole blocks (the padded
 * row rule of the GPU library and of orc_qmat_*); only the first n dequantized elements of a row
 * enter a dot. n must be a multiple of 32.
 */
#include <immintrin.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#include "oracle.h"

#include "blocks.h"   /* this file's own copy of the block dequantizers */

static inline float hsum256(__m256 acc) {                     /* kernel.rs:367-372, 1017-1020 */
    __m128 v = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    __m128 t = _mm_add_ps(v, _mm_movehl_ps(v, v));
    t = _mm_add_ss(t, _mm_shuffle_ps(t, t, 0x55));
    return _mm_cvtss_f32(t);
}

static float dot_f32_avx2(const float *a, const float *b, size_t n) {  /* kernel.rs:1002-1025 */
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
    float s = hsum256(acc);
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

/* kernel.rs:1162-1202 */
static void dot_x4x2(const float *a0, const float *a1, const float *const b[4], size_t n,
                     float o0[4], float o1[4]) {
    __m256 c0[4], c1[4];
    for (int k = 0; k < 4; ++k) { c0[k] = _mm256_setzero_ps(); c1[k] = _mm256_setzero_ps(); }
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 v0 = _mm256_loadu_ps(a0 + i), v1 = _mm256_loadu_ps(a1 + i);
        for (int k = 0; k < 4; ++k) {
            __m256 bv = _mm256_loadu_ps(b[k] + i);
            c0[k] = _mm256_fmadd_ps(v0, bv, c0[k]);
            c1[k] = _mm256_fmadd_ps(v1, bv, c1[k]);
        }
    }
    for (int k = 0; k < 4; ++k) {
        o0[k] = hsum256(c0[k]);
        o1[k] = hsum256(c1[k]);
        for (size_t j = i; j < n; ++j) { o0[k] += a0[j] * b[k][j]; o1[k] += a1[j] * b[k][j]; }
    }
}

/* matmul_reuse with tile 96, group 4, w_rows 2, r_block 1024 (kernel.rs:1383-1477).
 * W is m rows of ceil(n/qk) blocks, X rows x n, out rows x m with row stride ldo. */
static void matmul_reuse_avx2(const uint8_t *w, size_t m, size_t n, const float *x, size_t rows,
                              float *out, size_t ldo, size_t qk, size_t bb,
                              void (*dq)(const uint8_t *, float *), float *rb0b, float *rb1b) {
    const size_t tile = 96, r_block = 1024;
    size_t blocks = (n + qk - 1) / qk, row_bytes = blocks * bb;
    for (size_t rb0 = 0; rb0 < m; rb0 += r_block) {
        size_t rb1 = rb0 + r_block < m ? rb0 + r_block : m;
        for (size_t r0 = 0; r0 < rows; r0 += tile) {
            size_t r1 = r0 + tile < rows ? r0 + tile : rows;
            size_t r = rb0;
            while (r < rb1) {
                if (r + 1 < rb1) {
                    for (size_t b = 0; b < blocks; ++b) {
                        dq(w + r * row_bytes + b * bb, rb0b + b * qk);
                        dq(w + (r + 1) * row_bytes + b * bb, rb1b + b * qk);
                    }
                    size_t row = r0;
                    for (; row + 4 <= r1; row += 4) {
                        const float *bs[4] = {x + row * n, x + (row + 1) * n, x + (row + 2) * n, x + (row + 3) * n};
                        float g0[4], g1[4];
                        dot_x4x2(rb0b, rb1b, bs, n, g0, g1);
                        for (int k = 0; k < 4; ++k) { out[(row + k) * ldo + r] = g0[k]; out[(row + k) * ldo + r + 1] = g1[k]; }
                    }
                    for (; row < r1; ++row) {
                        out[row * ldo + r] = dot_f32_avx2(rb0b, x + row * n, n);
                        out[row * ldo + r + 1] = dot_f32_avx2(rb1b, x + row * n, n);
                    }
                    r += 2;
                } else {
                    for (size_t b = 0; b < blocks; ++b) dq(w + r * row_bytes + b * bb, rb0b + b * qk);
                    for (size_t row = r0; row < r1; ++row) out[row * ldo + r] = dot_f32_avx2(rb0b, x + row * n, n);
                    r += 1;
                }
            }
        }
    }
}

static int nthreads(int threads) {
    if (threads > 0) return threads;
    return omp_get_max_threads();
}

/* qmat.rs:169-272 */
int orc_cpu_matmul(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, size_t rows,
                   float *out, int threads) {
    size_t qk, bb;
    void (*dq)(const uint8_t *, float *);
    if (quant_geom_raw(t, &qk, &bb, &dq)) return ORC_ERR_TYPE;
    if (n % 32) return ORC_ERR_SIZE;
    int th = nthreads(threads);
    size_t blocks = (n + qk - 1) / qk, row_bytes = blocks * bb;
    int split_w = rows * n * 4 > 6u * 1024 * 1024;             /* MATMUL_X_L3_BUDGET, qmat.rs:18 */
    size_t span = split_w ? m : rows;
    size_t chunk = (span + (size_t)th - 1) / (size_t)th;
    size_t jobs = (span + chunk - 1) / chunk;
#pragma omp parallel for num_threads(th) schedule(static, 1)
    for (size_t j = 0; j < jobs; ++j) {
        const size_t nb = blocks * qk;
        float *bufs = (float *)aligned_alloc(64, ((2 * nb * sizeof(float)) + 63) / 64 * 64);
        size_t lo = j * chunk, cnt = chunk < span - lo ? chunk : span - lo;
        if (split_w)   /* qmat.rs:256-262: weight-row slice, whole X, strided stitch */
            matmul_reuse_avx2(w + lo * row_bytes, cnt, n, x, rows, out + lo, m, qk, bb, dq, bufs, bufs + nb);
        else           /* qmat.rs:206-217: activation-row slice */
            matmul_reuse_avx2(w, m, n, x + lo * n, cnt, out + lo * m, m, qk, bb, dq, bufs, bufs + nb);
        free(bufs);
    }
    return ORC_OK;
}

/* qmat.rs:80-127 with a per-block dequant + 8-lane FMA fused dot */
int orc_cpu_matvec(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, float *out,
                   int threads) {
    size_t qk, bb;
    void (*dq)(const uint8_t *, float *);
    if (quant_geom_raw(t, &qk, &bb, &dq)) return ORC_ERR_TYPE;
    if (n % 32) return ORC_ERR_SIZE;
    int th = nthreads(threads);
    size_t blocks = (n + qk - 1) / qk, row_bytes = blocks * bb;
#pragma omp parallel for num_threads(th) schedule(static)
    for (size_t r = 0; r < m; ++r) {
        float buf[256] __attribute__((aligned(32)));
        __m256 acc = _mm256_setzero_ps();
        const uint8_t *row = w + r * row_bytes;
        for (size_t b = 0; b < blocks; ++b) {
            dq(row + b * bb, buf);
            const float *xb = x + b * qk;
            const size_t len = n - b * qk < qk ? n - b * qk : qk;
            for (size_t i = 0; i < len; i += 8)
                acc = _mm256_fmadd_ps(_mm256_load_ps(buf + i), _mm256_loadu_ps(xb + i), acc);
        }
        out[r] = hsum256(acc);
    }
    return ORC_OK;
}
