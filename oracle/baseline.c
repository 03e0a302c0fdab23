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
 * - GEMV: QMat::matvec (qmat.rs:80-127): serial below PAR_MAC_MIN = 2^18 MACs, else rows split in
 *   ceil(m / threads) chunks; each row runs quant_row_dot (kernel.rs:1998-2008), i.e. the
 *   per-type AVX2 fused dots: dot_q4_0_avx2 (kernel.rs:653-682), dot_q8_0_avx2 (488-514),
 *   dot_q5_0_avx2 (848-885), dot_q4_k_avx2 (693-736), dot_q6_k_avx2 (746-837), and the scalar
 *   dot_q5_k (297-308; the reference has no SIMD Q5_K dot). Each restates the reference's lane
 *   structure: widen 8 quants to i32, convert, scale, FMA (or mul + add) into one or two 8-lane
 *   accumulators, fold 256 -> 128 bits, hsum_ps_sse2 (kernel.rs:367-372). Rows padded to whole
 *   blocks (n % QK != 0) take a generic dequant + FMA dot over the first n elements.
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

static inline float fold_hsum(__m256 acc) {                   /* kernel.rs:510-513 */
    return hsum256(acc);
}

/* kernel.rs:653-682: split-half nibbles, lo -> b[0..16], hi -> b[16..32], two accumulators */
static float dot_q4_0_avx2(const uint8_t *a, size_t nb, const float *b) {
    const __m256i mask = _mm256_set1_epi32(0x0F), eight = _mm256_set1_epi32(8);
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    for (size_t k = 0; k < nb; ++k) {
        const uint8_t *blk = a + k * 18;
        const __m256 dv = _mm256_set1_ps(f16_to_f32_bits(rd16(blk)));
        const uint8_t *qs = blk + 2;
        const float *bo = b + k * 32;
        for (int jj = 0; jj < 16; jj += 8) {
            const __m256i v = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qs + jj)));
            const __m256i lo = _mm256_sub_epi32(_mm256_and_si256(v, mask), eight);
            const __m256i hi = _mm256_sub_epi32(_mm256_srli_epi32(v, 4), eight);
            acc0 = _mm256_fmadd_ps(_mm256_mul_ps(dv, _mm256_cvtepi32_ps(lo)), _mm256_loadu_ps(bo + jj), acc0);
            acc1 = _mm256_fmadd_ps(_mm256_mul_ps(dv, _mm256_cvtepi32_ps(hi)), _mm256_loadu_ps(bo + 16 + jj), acc1);
        }
    }
    return fold_hsum(_mm256_add_ps(acc0, acc1));
}

/* kernel.rs:488-514: i8 quants widened eight at a time into two accumulators */
static float dot_q8_0_avx2(const uint8_t *a, size_t nb, const float *b) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    for (size_t k = 0; k < nb; ++k) {
        const uint8_t *blk = a + k * 34;
        const __m256 dv = _mm256_set1_ps(f16_to_f32_bits(rd16(blk)));
        const uint8_t *qs = blk + 2;
        const float *bo = b + k * 32;
        for (int jj = 0; jj < 32; jj += 16) {
            const __m256 v0 = _mm256_mul_ps(dv, _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(qs + jj)))));
            acc0 = _mm256_fmadd_ps(v0, _mm256_loadu_ps(bo + jj), acc0);
            const __m256 v1 = _mm256_mul_ps(dv, _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(qs + jj + 8)))));
            acc1 = _mm256_fmadd_ps(v1, _mm256_loadu_ps(bo + jj + 8), acc1);
        }
    }
    return fold_hsum(_mm256_add_ps(acc0, acc1));
}

/* kernel.rs:848-885: nibbles plus the fifth bit gathered per lane with a variable shift */
static float dot_q5_0_avx2(const uint8_t *a, size_t nb, const float *b) {
    const __m256i mask = _mm256_set1_epi32(0x0F), sixteen = _mm256_set1_epi32(16), ones = _mm256_set1_epi32(1);
    const __m256i shifts = _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7);
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    for (size_t k = 0; k < nb; ++k) {
        const uint8_t *blk = a + k * 22;
        const __m256 dv = _mm256_set1_ps(f16_to_f32_bits(rd16(blk)));
        const uint32_t qh = rd32(blk + 2);
        const uint8_t *qs = blk + 6;
        const float *bo = b + k * 32;
        for (int jj = 0; jj < 16; jj += 8) {
            const __m256i v = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qs + jj)));
            const __m256i b0 = _mm256_set1_epi32((int)((qh >> jj) & 0xFF));
            const __m256i b1 = _mm256_set1_epi32((int)((qh >> (jj + 16)) & 0xFF));
            const __m256i bit0 = _mm256_slli_epi32(_mm256_and_si256(_mm256_srlv_epi32(b0, shifts), ones), 4);
            const __m256i bit1 = _mm256_slli_epi32(_mm256_and_si256(_mm256_srlv_epi32(b1, shifts), ones), 4);
            const __m256i lo = _mm256_sub_epi32(_mm256_or_si256(_mm256_and_si256(v, mask), bit0), sixteen);
            const __m256i hi = _mm256_sub_epi32(_mm256_or_si256(_mm256_srli_epi32(v, 4), bit1), sixteen);
            acc0 = _mm256_fmadd_ps(_mm256_mul_ps(dv, _mm256_cvtepi32_ps(lo)), _mm256_loadu_ps(bo + jj), acc0);
            acc1 = _mm256_fmadd_ps(_mm256_mul_ps(dv, _mm256_cvtepi32_ps(hi)), _mm256_loadu_ps(bo + 16 + jj), acc1);
        }
    }
    return fold_hsum(_mm256_add_ps(acc0, acc1));
}

/* kernel.rs:693-736: per 64-element group (d*sc, min*m) of the low / high nibbles; mul + add */
static float dot_q4_k_avx2(const uint8_t *a, size_t nb, const float *b) {
    const __m256i mask = _mm256_set1_epi32(0x0F);
    __m256 acc = _mm256_setzero_ps();
    for (size_t k = 0; k < nb; ++k) {
        const uint8_t *blk = a + k * 144;
        const float d = f16_to_f32_bits(rd16(blk)), mn = f16_to_f32_bits(rd16(blk + 2));
        const uint8_t *qs = blk + 16;
        const float *bo = b + k * 256;
        for (int grp = 0; grp < 4; ++grp) {
            uint8_t sc0, m0, sc1, m1;
            scale_min_k4(2 * grp, blk + 4, &sc0, &m0);
            scale_min_k4(2 * grp + 1, blk + 4, &sc1, &m1);
            const __m256 d1 = _mm256_set1_ps(d * (float)sc0), dm1 = _mm256_set1_ps(mn * (float)m0);
            const __m256 d2 = _mm256_set1_ps(d * (float)sc1), dm2 = _mm256_set1_ps(mn * (float)m1);
            for (int jj = 0; jj < 32; jj += 8) {
                const __m256i v = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qs + grp * 32 + jj)));
                const __m256 lo = _mm256_sub_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_and_si256(v, mask)), d1), dm1);
                const __m256 hi = _mm256_sub_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_srli_epi32(v, 4)), d2), dm2);
                acc = _mm256_add_ps(acc, _mm256_mul_ps(lo, _mm256_loadu_ps(bo + grp * 64 + jj)));
                acc = _mm256_add_ps(acc, _mm256_mul_ps(hi, _mm256_loadu_ps(bo + grp * 64 + 32 + jj)));
            }
        }
    }
    return fold_hsum(acc);
}

/* kernel.rs:746-837: per half-block, 8 lanes of each of the four 32-element quarters, the
 * 6-bit quant (ql nibble | 2 qh bits << 4) - 32 times d * int8 sub-scale; mul + add */
static float dot_q6_k_avx2(const uint8_t *a, size_t nb, const float *b) {
    const __m256i mask = _mm256_set1_epi32(0x0F), m2 = _mm256_set1_epi32(0x03), bias = _mm256_set1_epi32(32);
    __m256 acc = _mm256_setzero_ps();
    for (size_t k = 0; k < nb; ++k) {
        const uint8_t *blk = a + k * 210;
        const float d = f16_to_f32_bits(rd16(blk + 208));
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float *bo = b + k * 256;
        for (int half = 0; half < 2; ++half) {
            const uint8_t *qlh = ql + half * 64, *qhh = qh + half * 32;
            const int8_t *sch = sc + half * 8;
            const float *ob = bo + half * 128;
            for (int l = 0; l < 32; l += 8) {
                const int is = l / 16;
                const __m256i la = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qlh + l)));
                const __m256i lb = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qlh + l + 32)));
                const __m256i h = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qhh + l)));
                const __m256i q1 = _mm256_sub_epi32(_mm256_or_si256(_mm256_and_si256(la, mask),
                    _mm256_slli_epi32(_mm256_and_si256(h, m2), 4)), bias);
                const __m256i q2 = _mm256_sub_epi32(_mm256_or_si256(_mm256_and_si256(lb, mask),
                    _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 2), m2), 4)), bias);
                const __m256i q3 = _mm256_sub_epi32(_mm256_or_si256(_mm256_srli_epi32(la, 4),
                    _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 4), m2), 4)), bias);
                const __m256i q4 = _mm256_sub_epi32(_mm256_or_si256(_mm256_srli_epi32(lb, 4),
                    _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 6), m2), 4)), bias);
                const __m256 s0 = _mm256_set1_ps(d * (float)sch[is]), s2 = _mm256_set1_ps(d * (float)sch[is + 2]);
                const __m256 s4 = _mm256_set1_ps(d * (float)sch[is + 4]), s6 = _mm256_set1_ps(d * (float)sch[is + 6]);
                acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(q1), s0), _mm256_loadu_ps(ob + l)));
                acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(q2), s2), _mm256_loadu_ps(ob + l + 32)));
                acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(q3), s4), _mm256_loadu_ps(ob + l + 64)));
                acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(q4), s6), _mm256_loadu_ps(ob + l + 96)));
            }
        }
    }
    return fold_hsum(acc);
}

/* kernel.rs:297-308: dequantize each super-block, then a sequential f32 sum */
static float dot_q5_k_scalar(const uint8_t *a, size_t nb, const float *b) {
    float s = 0.0f, buf[256];
    for (size_t k = 0; k < nb; ++k) {
        dq_q5_k(a + k * 176, buf);
        float part = 0.0f;
        for (int i = 0; i < 256; ++i) part += buf[i] * b[k * 256 + i];
        s += part;
    }
    return s;
}

/* quant_row_dot (kernel.rs:1998-2008) for a row of nb whole blocks */
static float row_dot(uint32_t t, const uint8_t *row, size_t nb, const float *x) {
    switch (t) {
        case 2: return dot_q4_0_avx2(row, nb, x);
        case 6: return dot_q5_0_avx2(row, nb, x);
        case 8: return dot_q8_0_avx2(row, nb, x);
        case 12: return dot_q4_k_avx2(row, nb, x);
        case 13: return dot_q5_k_scalar(row, nb, x);
        default: return dot_q6_k_avx2(row, nb, x);
    }
}

/* qmat.rs:80-127 */
int orc_cpu_matvec(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, float *out,
                   int threads) {
    size_t qk, bb;
    void (*dq)(const uint8_t *, float *);
    if (quant_geom_raw(t, &qk, &bb, &dq)) return ORC_ERR_TYPE;
    if (n % 32) return ORC_ERR_SIZE;
    int th = nthreads(threads);
    size_t blocks = (n + qk - 1) / qk, row_bytes = blocks * bb;
    if (m * n < ((size_t)1 << 18) || m < 2) th = 1;                 /* workers_for, qmat.rs:21-26 */
    if (th > (int)m) th = (int)m;
    if (n % qk == 0) {
        const size_t chunk = (m + (size_t)th - 1) / (size_t)th;       /* qmat.rs:106-121 */
        const size_t jobs = (m + chunk - 1) / chunk;
#pragma omp parallel for num_threads(th) schedule(static, 1)
        for (size_t j = 0; j < jobs; ++j) {
            const size_t end = (j + 1) * chunk < m ? (j + 1) * chunk : m;
            for (size_t r = j * chunk; r < end; ++r) out[r] = row_dot(t, w + r * row_bytes, blocks, x);
        }
        return ORC_OK;
    }
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
