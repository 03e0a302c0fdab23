/*
 * CPU oracle: plain-C restatement of platinoff/rusty-engine's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Compiled with -ffp-contract=off: every f32
 * statement rounds exactly where the Rust statement it restates rounds. Rust's float
 * `Iterator::sum` folds from -0.0, so the sequential sums below start from -0.0f too.
 */
#include "oracle.h"
#include "blocks.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[256];

const char *orc_last_error(void) { return g_err; }

static int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
#include <stdarg.h>
static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}


/* ---- src/quant.rs:25-45 ------------------------------------------------------------ */
float orc_f16_to_f32(uint16_t h) { return f16_to_f32_bits(h); }

/* ---- src/quant.rs:48-72 (truncating narrow, saturating to Inf) ---------------------- */
uint16_t orc_f32_to_f16(float x) {
    uint32_t b = f32_bits(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    int exp = (int)((b >> 23) & 0xFF);
    uint32_t frac = b & 0x7FFFFF;
    if (exp == 0xFF) {
        if (frac == 0) return sign | 0x7C00;
        return (uint16_t)(sign | 0x7E00 | (frac >> 13));
    }
    int new_exp = exp - 127 + 15;
    if (new_exp >= 0x1F) return sign | 0x7C00;
    if (new_exp <= 0) {
        if (new_exp < -10) return sign;
        uint32_t mant = (frac | 0x800000) >> (1 - new_exp + 13);
        return (uint16_t)(sign | mant);
    }
    return (uint16_t)(sign | ((uint32_t)new_exp << 10) | (frac >> 13));
}

/* ---- src/quant.rs:75-101 ---------------------------------------------------------- */
int orc_block_info(uint32_t t, size_t *elements, size_t *bytes) {
    size_t e, b;
    switch (t) {
    case 0: e = 1; b = 4; break;
    case 1: case 30: e = 1; b = 2; break;
    case 2: e = 32; b = 18; break;
    case 6: e = 32; b = 22; break;
    case 8: e = 32; b = 34; break;
    case 12: e = 256; b = 144; break;
    case 13: e = 256; b = 176; break;
    case 14: e = 256; b = 210; break;
    default: return fail(ORC_ERR_TYPE, "unknown ggml type %u", t);
    }
    if (elements) *elements = e;
    if (bytes) *bytes = b;
    return ORC_OK;
}

int orc_bytes_for_numel(uint32_t t, size_t numel, size_t *bytes) {
    size_t e, b;
    int rc = orc_block_info(t, &e, &b);
    if (rc) return rc;
    if (e == 1) { *bytes = numel * b; return ORC_OK; }
    if (numel % e != 0) return fail(ORC_ERR_SIZE, "numel %zu not a whole number of blocks", numel);
    *bytes = numel / e * b;
    return ORC_OK;
}

/* ---- src/quant.rs:250-258 --------------------------------------------------------- */
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) { scale_min_k4(j, q, sc, m); }

static int quant_geom(uint32_t t, size_t *qk, size_t *bb, dq_fn *dq) {
    if (quant_geom_raw(t, qk, bb, dq)) return fail(ORC_ERR_TYPE, "no fused kernel for ggml type %u", t);
    return ORC_OK;
}

int orc_internal_geom(uint32_t t, size_t *qk, size_t *bb, dq_fn *dq) { return quant_geom(t, qk, bb, dq); }

int orc_cpu_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* ---- src/quant.rs:363-453 ---------------------------------------------------------- */
int orc_dequant(uint32_t t, const uint8_t *data, size_t len, float *out, size_t *n_out) {
    switch (t) {
    case 0:
        if (len % 4) return fail(ORC_ERR_SIZE, "F32 data len %zu not a multiple of 4", len);
        *n_out = len / 4;
        if (out) for (size_t i = 0; i < len / 4; ++i) out[i] = bits_f32(rd32(data + 4 * i));
        return ORC_OK;
    case 1:
        if (len % 2) return fail(ORC_ERR_SIZE, "F16 data len %zu not a multiple of 2", len);
        *n_out = len / 2;
        if (out) for (size_t i = 0; i < len / 2; ++i) out[i] = orc_f16_to_f32(rd16(data + 2 * i));
        return ORC_OK;
    case 30:
        if (len % 2) return fail(ORC_ERR_SIZE, "BF16 data len %zu not a multiple of 2", len);
        *n_out = len / 2;
        if (out) for (size_t i = 0; i < len / 2; ++i) out[i] = bits_f32((uint32_t)rd16(data + 2 * i) << 16);
        return ORC_OK;
    default: break;
    }
    static const char *names[15] = {0, 0, "Q4_0", 0, 0, 0, "Q5_0", 0, "Q8_0", 0, 0, 0,
                                    "Q4_K", "Q5_K", "Q6_K"};
    size_t qk, bb;
    dq_fn dq;
    if (t > 14 || !names[t] || quant_geom(t, &qk, &bb, &dq))
        return fail(ORC_ERR_TYPE, "no scalar dequant for ggml type %u", t);
    if (len % bb) return fail(ORC_ERR_SIZE, "%s data len %zu not a multiple of %zu", names[t], len, bb);
    *n_out = len / bb * qk;
    if (out) for (size_t i = 0; i < len / bb; ++i) dq(data + i * bb, out + i * qk);
    return ORC_OK;
}

/* ---- src/quant.rs:162-229 ----------------------------------------------------------- */
int orc_quantize_q8_0(const float *src, size_t n, uint8_t *out) {
    if (n % 32) return fail(ORC_ERR_SIZE, "q8_0 quantize: len %zu not multiple of 32", n);
    for (size_t b = 0; b < n / 32; ++b) {
        const float *blk = src + 32 * b;
        uint8_t *o = out + 34 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) { float ax = fabsf(blk[j]); if (ax > amax) amax = ax; }
        float d = amax / 127.0f;
        float id = d == 0.0f ? 0.0f : 1.0f / d;
        uint16_t h = orc_f32_to_f16(d);
        o[0] = (uint8_t)(h & 0xFF); o[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; ++j) {
            float q = d == 0.0f ? 0.0f : fminf(fmaxf(roundf(blk[j] * id), -127.0f), 127.0f);
            o[2 + j] = (uint8_t)(int8_t)q;
        }
    }
    return ORC_OK;
}

int orc_quantize_q4_0(const float *src, size_t n, uint8_t *out) {
    if (n % 32) return fail(ORC_ERR_SIZE, "q4_0 quantize: len %zu not multiple of 32", n);
    for (size_t b = 0; b < n / 32; ++b) {
        const float *blk = src + 32 * b;
        uint8_t *o = out + 18 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) { float ax = fabsf(blk[j]); if (ax > amax) amax = ax; }
        float d = amax / 7.0f;
        float id = d == 0.0f ? 0.0f : 1.0f / d;
        uint16_t h = orc_f32_to_f16(d);
        o[0] = (uint8_t)(h & 0xFF); o[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 16; ++j) {
            int q0 = d == 0.0f ? 8 : (int)fminf(fmaxf(roundf(blk[j] * id), -8.0f), 7.0f) + 8;
            int q1 = d == 0.0f ? 8 : (int)fminf(fmaxf(roundf(blk[j + 16] * id), -8.0f), 7.0f) + 8;
            o[2 + j] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
        }
    }
    return ORC_OK;
}

/* ---- src/kernel.rs:70-166: int8 activations and the integer Q8_0 dot -------------- */
/* Q8Activation::from_f32 (kernel.rs:88-105): per 32-value block d = max|x| / 127 (the f32::max
 * fold from 0, so NaN inputs never win), inv = 1/d or 0 when d == 0, q = x*inv rounded half away
 * from zero and clamped to [-127, 127]; a NaN product becomes 0 (Rust's saturating `as i8`). */
int orc_quantize_q8_act(const float *x, size_t n, float *scales, int8_t *qs) {
    if (n % 32) return fail(ORC_ERR_SIZE, "Q8Activation::from_f32: length %zu not a multiple of 32", n);
    for (size_t b = 0; b < n / 32; ++b) {
        const float *blk = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(blk[j]));
        const float d = amax / 127.0f;
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        for (int j = 0; j < 32; ++j) {
            float r = roundf(blk[j] * inv);
            if (isnan(r)) r = 0.0f;
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            qs[32 * b + j] = (int8_t)r;
        }
        scales[b] = d;
    }
    return ORC_OK;
}

/* dot_q8_0_i8 (kernel.rs:123-142): per block the exact i32 sum of w_i * q_i, then
 * s += (isum as f32) * dw * dx evaluated left to right, blocks in order from s = 0. */
float orc_dot_q8_0_i8(const uint8_t *a, size_t nb, const float *scales, const int8_t *qs) {
    float s = 0.0f;
    for (size_t k = 0; k < nb; ++k) {
        const uint8_t *blk = a + 34 * k;
        const float dw = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        int32_t isum = 0;
        for (int j = 0; j < 32; ++j) isum += (int32_t)(int8_t)blk[2 + j] * (int32_t)qs[32 * k + j];
        float t = (float)isum * dw;
        t = t * scales[k];
        s = s + t;
    }
    return s;
}

/* matvec_q8_0_i8 / matmul_q8_0_i8 (kernel.rs:145-166): row by row; activation row r holds
 * scales[r*nb ..] and qs[r*n ..]; out is rows x m. */
int orc_matmul_q8_0_i8(const uint8_t *w, size_t m, size_t n, const float *scales, const int8_t *qs,
                       size_t rows, float *out) {
    if (n % 32) return fail(ORC_ERR_SIZE, "matvec_q8_0_i8: n = %zu not a multiple of 32", n);
    const size_t nb = n / 32, row_bytes = nb * 34;
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < m; ++i)
            out[r * m + i] = orc_dot_q8_0_i8(w + i * row_bytes, nb, scales + r * nb, qs + r * n);
    return ORC_OK;
}

/* ---- scalar fused dots: kernel.rs:17-46, 171-191, 283-322 ------------------------- */
static float seq_sum_products(const float *a, const float *b, size_t n) {
    float s = -0.0f;
    for (size_t i = 0; i < n; ++i) s = s + a[i] * b[i];
    return s;
}

float orc_dot_seq(const float *a, const float *b, size_t n) { return seq_sum_products(a, b, n); }

float orc_dot(uint32_t t, const uint8_t *row, size_t nb, const float *x) {
    float s = 0.0f;
    switch (t) {
    case 2: /* kernel.rs:17-31 */
        for (size_t k = 0; k < nb; ++k) {
            const uint8_t *blk = row + 18 * k;
            const float *lo = x + 32 * k, *hi = lo + 16;
            float d = orc_f16_to_f32(rd16(blk));
            for (int j = 0; j < 16; ++j) {
                uint8_t q = blk[2 + j];
                s += d * (float)((int)(q & 0x0F) - 8) * lo[j];
                s += d * (float)((int)(q >> 4) - 8) * hi[j];
            }
        }
        return s;
    case 8: /* kernel.rs:34-46 */
        for (size_t k = 0; k < nb; ++k) {
            const uint8_t *blk = row + 34 * k;
            float d = orc_f16_to_f32(rd16(blk));
            for (int j = 0; j < 32; ++j) s += (float)(int8_t)blk[2 + j] * d * x[32 * k + j];
        }
        return s;
    case 6: /* kernel.rs:171-191 */
        for (size_t k = 0; k < nb; ++k) {
            const uint8_t *blk = row + 22 * k;
            const float *lo = x + 32 * k, *hi = lo + 16;
            float d = orc_f16_to_f32(rd16(blk));
            uint32_t qh = rd32(blk + 2);
            const uint8_t *qs = blk + 6;
            for (int j = 0; j < 16; ++j) {
                int bit0 = (int)(((qh >> j) & 1) << 4);
                int bit1 = (int)(((qh >> (j + 16)) & 1) << 4);
                int x0 = ((int)(qs[j] & 0x0F) | bit0) - 16;
                int x1 = ((int)(qs[j] >> 4) | bit1) - 16;
                s += (float)x0 * d * lo[j];
                s += (float)x1 * d * hi[j];
            }
        }
        return s;
    case 12: case 13: case 14: { /* kernel.rs:283-322 */
        size_t qk, bb;
        dq_fn dq;
        quant_geom(t, &qk, &bb, &dq);
        float buf[256];
        for (size_t k = 0; k < nb; ++k) {
            dq(row + bb * k, buf);
            s += seq_sum_products(buf, x + 256 * k, 256);
        }
        return s;
    }
    default:
        fail(ORC_ERR_TYPE, "quant_row_dot: no fused kernel for ggml type %u", t);
        return NAN;
    }
}

int orc_matvec(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, float *out) {
    size_t qk, bb;
    dq_fn dq;
    int rc = quant_geom(t, &qk, &bb, &dq);
    if (rc) return rc;
    if (n % qk) return fail(ORC_ERR_SIZE, "matvec: n %zu must be a multiple of %zu", n, qk);
    size_t rb = n / qk * bb;
    for (size_t r = 0; r < m; ++r) out[r] = orc_dot(t, w + r * rb, n / qk, x);
    return ORC_OK;
}

/* ---- AVX2 f32 dot order, restated scalar: kernel.rs:1002-1025 + 367-372 ------------ */
float orc_dot_f32(const float *a, const float *b, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
    float v0 = acc[0] + acc[4], v1 = acc[1] + acc[5], v2 = acc[2] + acc[6], v3 = acc[3] + acc[7];
    float s = (v0 + v2) + (v1 + v3);
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

/* ---- matmul_reuse: kernel.rs:1383-1590 ---------------------------------------------
 * The x4/x8/x4x2 dot variants keep dot_f32's per-output order (kernel.rs:1040-1050), so
 * every (row, r) output is dot_f32(dequant_row(r), x_row) whatever the knobs; the loop nest
 * below keeps the reference's walk so the knob-invariance tests exercise it. */
static void dequant_row(const uint8_t *raw, float *out, size_t blocks, size_t bb, size_t qk, dq_fn dq) {
    for (size_t b = 0; b < blocks; ++b) dq(raw + b * bb, out + b * qk);
}

static void dot_tile_rows(const float *a, const float *x, size_t n, size_t m, size_t r,
                          size_t r0, size_t r1, size_t group, float *out) {
    size_t row = r0;
    if (group == 8)
        for (; row + 8 <= r1; row += 8)
            for (size_t k = 0; k < 8; ++k) out[(row + k) * m + r] = orc_dot_f32(a, x + (row + k) * n, n);
    if (group >= 4)
        for (; row + 4 <= r1; row += 4)
            for (size_t k = 0; k < 4; ++k) out[(row + k) * m + r] = orc_dot_f32(a, x + (row + k) * n, n);
    for (; row < r1; ++row) out[row * m + r] = orc_dot_f32(a, x + row * n, n);
}

static void dot_tile_rows_pair(const float *a0, const float *a1, const float *x, size_t n,
                               size_t m, size_t r, size_t r0, size_t r1, float *out) {
    size_t row = r0;
    for (; row + 4 <= r1; row += 4)
        for (size_t k = 0; k < 4; ++k) {
            out[(row + k) * m + r] = orc_dot_f32(a0, x + (row + k) * n, n);
            out[(row + k) * m + r + 1] = orc_dot_f32(a1, x + (row + k) * n, n);
        }
    for (; row < r1; ++row) {
        out[row * m + r] = orc_dot_f32(a0, x + row * n, n);
        out[row * m + r + 1] = orc_dot_f32(a1, x + row * n, n);
    }
}

int orc_matmul_reuse(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x,
                     size_t rows, size_t tile, size_t group, size_t w_rows, size_t r_block,
                     float *out) {
    size_t qk, bb;
    dq_fn dq;
    int rc = quant_geom(t, &qk, &bb, &dq);
    if (rc) return rc;
    if (n % qk) return fail(ORC_ERR_SIZE, "matmul: n %zu must be a multiple of %zu", n, qk);
    if (tile < 1) tile = 1;
    if (group < 1) group = 1;
    if (group > 8) group = 8;
    if (w_rows < 1) w_rows = 1;
    if (w_rows > 4) w_rows = 4;
    if (r_block < 1) r_block = 1;
    size_t blocks = n / qk, row_bytes = blocks * bb;
    float *buf = (float *)malloc(4 * n * sizeof(float) + 16);
    if (!buf) return fail(ORC_ERR_ARG, "out of memory");
    float *rb1b = buf, *rb2b = buf + n, *rb3b = buf + 2 * n, *rb4b = buf + 3 * n;
    memset(out, 0, rows * m * sizeof(float));
    for (size_t rb0 = 0; rb0 < m;) {
        size_t rb1 = rb0 + r_block < m ? rb0 + r_block : m;
        for (size_t r0 = 0; r0 < rows;) {
            size_t r1 = r0 + tile < rows ? r0 + tile : rows;
            size_t r = rb0;
            while (r < rb1) {
                if (w_rows >= 4 && group == 4 && r + 3 < rb1) {
                    dequant_row(w + r * row_bytes, rb1b, blocks, bb, qk, dq);
                    dequant_row(w + (r + 1) * row_bytes, rb2b, blocks, bb, qk, dq);
                    dequant_row(w + (r + 2) * row_bytes, rb3b, blocks, bb, qk, dq);
                    dequant_row(w + (r + 3) * row_bytes, rb4b, blocks, bb, qk, dq);
                    dot_tile_rows_pair(rb1b, rb2b, x, n, m, r, r0, r1, out);
                    dot_tile_rows_pair(rb3b, rb4b, x, n, m, r + 2, r0, r1, out);
                    r += 4;
                } else if (w_rows >= 2 && group == 4 && r + 1 < rb1) {
                    dequant_row(w + r * row_bytes, rb1b, blocks, bb, qk, dq);
                    dequant_row(w + (r + 1) * row_bytes, rb2b, blocks, bb, qk, dq);
                    dot_tile_rows_pair(rb1b, rb2b, x, n, m, r, r0, r1, out);
                    r += 2;
                } else {
                    dequant_row(w + r * row_bytes, rb1b, blocks, bb, qk, dq);
                    dot_tile_rows(rb1b, x, n, m, r, r0, r1, group, out);
                    r += 1;
                }
            }
            r0 = r1;
        }
        rb0 = rb1;
    }
    free(buf);
    return ORC_OK;
}

/* kernel.rs:1328-1369 constants, 1640-1947 entries, 2012-2029 dispatch */
int orc_matmul(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, size_t rows,
               float *out) {
    return orc_matmul_reuse(t, w, m, n, x, rows, 96, 4, 2, 1024, out);
}

/* kernel.rs:1596-1637 */
int orc_matmul_blocks(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x,
                      size_t rows, size_t tile, float *out) {
    size_t qk, bb;
    dq_fn dq;
    int rc = quant_geom(t, &qk, &bb, &dq);
    if (rc) return rc;
    if (n % qk) return fail(ORC_ERR_SIZE, "matmul: n %zu must be a multiple of %zu", n, qk);
    if (tile < 1) tile = 1;
    size_t blocks = n / qk, row_bytes = blocks * bb;
    float buf[256];
    float *acc = (float *)malloc((tile < rows ? tile : rows) * sizeof(float) + 4);
    if (!acc) return fail(ORC_ERR_ARG, "out of memory");
    memset(out, 0, rows * m * sizeof(float));
    for (size_t r = 0; r < m; ++r) {
        const uint8_t *wr = w + r * row_bytes;
        for (size_t r0 = 0; r0 < rows;) {
            size_t r1 = r0 + tile < rows ? r0 + tile : rows;
            for (size_t i = 0; i < r1 - r0; ++i) acc[i] = 0.0f;
            for (size_t b = 0; b < blocks; ++b) {
                dq(wr + b * bb, buf);
                for (size_t i = 0; i < r1 - r0; ++i)
                    acc[i] += orc_dot_f32(buf, x + (r0 + i) * n + b * qk, qk);
            }
            for (size_t i = 0; i < r1 - r0; ++i) out[(r0 + i) * m + r] = acc[i];
            r0 = r1;
        }
    }
    free(acc);
    return ORC_OK;
}

/* QMat::F32 and QMat::Quant over F16/BF16 carry no fused kernel: the whole matrix widens
 * through quant::dequant (quant.rs:365-397) and each output is moe::matvec's sequential
 * sum of products (moe.rs:271-277, qmat.rs:132, 146-151, 277-283). One element per block. */
static void dq_f32(const uint8_t *b, float *o) { *o = bits_f32(rd32(b)); }
static void dq_f16(const uint8_t *b, float *o) { *o = orc_f16_to_f32(rd16(b)); }
static void dq_bf16(const uint8_t *b, float *o) { *o = bits_f32((uint32_t)rd16(b) << 16); }

static int dense_geom(uint32_t t, size_t *qk, size_t *bb, dq_fn *dq) {
    switch (t) {
    case 0: *qk = 1; *bb = 4; *dq = dq_f32; return 1;
    case 1: *qk = 1; *bb = 2; *dq = dq_f16; return 1;
    case 30: *qk = 1; *bb = 2; *dq = dq_bf16; return 1;
    default: return 0;
    }
}

/* ---- QMat-level semantics with padded rows ---------------------------------------- */
int orc_qmat_row_bytes(uint32_t t, size_t n, size_t *row_bytes) {
    size_t qk = 0, bb = 0;
    dq_fn dq;
    int rc = dense_geom(t, &qk, &bb, &dq) ? ORC_OK : quant_geom(t, &qk, &bb, &dq);
    if (rc) return rc;
    *row_bytes = (n + qk - 1) / qk * bb;
    return ORC_OK;
}

static int qmat_check(uint32_t t, size_t nbytes, size_t m, size_t n, size_t *qk, size_t *bb,
                      dq_fn *dq, size_t *rb) {
    int rc = dense_geom(t, qk, bb, dq) ? ORC_OK : quant_geom(t, qk, bb, dq);
    if (rc) return rc;
    if (n == 0) return fail(ORC_ERR_SIZE, "QMat: n must be > 0");
    *rb = (n + *qk - 1) / *qk * *bb;
    if (nbytes != m * *rb)
        return fail(ORC_ERR_SIZE, "QMat: %zu bytes for %zu x %zu type %u (want %zu)", nbytes, m, n, t, m * *rb);
    return ORC_OK;
}

int orc_qmat_matvec(uint32_t t, const uint8_t *w, size_t nbytes, size_t m, size_t n,
                    const float *x, float *out) {
    size_t qk, bb, rb;
    dq_fn dq;
    int rc = qmat_check(t, nbytes, m, n, &qk, &bb, &dq, &rb);
    if (rc) return rc;
    if (qk > 1 && n % qk == 0) return orc_matvec(t, w, m, n, x, out);
    size_t nb = rb / bb;
    float *row = (float *)malloc(nb * qk * sizeof(float));
    if (!row) return fail(ORC_ERR_ARG, "out of memory");
    for (size_t r = 0; r < m; ++r) {
        dequant_row(w + r * rb, row, nb, bb, qk, dq);
        out[r] = seq_sum_products(row, x, n);
    }
    free(row);
    return ORC_OK;
}

int orc_qmat_matmul(uint32_t t, const uint8_t *w, size_t nbytes, size_t m, size_t n,
                    const float *x, size_t rows, float *out) {
    size_t qk, bb, rb;
    dq_fn dq;
    int rc = qmat_check(t, nbytes, m, n, &qk, &bb, &dq, &rb);
    if (rc) return rc;
    if (qk > 1 && n % qk == 0) return orc_matmul(t, w, m, n, x, rows, out);
    for (size_t i = 0; i < rows; ++i) {
        rc = orc_qmat_matvec(t, w, nbytes, m, n, x + i * n, out + i * m);
        if (rc) return rc;
    }
    return ORC_OK;
}

int orc_qmat_absdot(uint32_t t, const uint8_t *w, size_t nbytes, size_t m, size_t n,
                    const float *x, size_t rows, double *out) {
    size_t qk, bb, rb;
    dq_fn dq;
    int rc = qmat_check(t, nbytes, m, n, &qk, &bb, &dq, &rb);
    if (rc) return rc;
    size_t nb = rb / bb;
    float *row = (float *)malloc(nb * qk * sizeof(float));
    if (!row) return fail(ORC_ERR_ARG, "out of memory");
    for (size_t r = 0; r < m; ++r) {
        dequant_row(w + r * rb, row, nb, bb, qk, dq);
        for (size_t i = 0; i < rows; ++i) {
            double s = 0.0;
            const float *xi = x + i * n;
            for (size_t k = 0; k < n; ++k) s += fabs((double)row[k] * (double)xi[k]);
            out[i * m + r] = s;
        }
    }
    free(row);
    return ORC_OK;
}

/* ---- src/moe.rs --------------------------------------------------------------------- */
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }   /* moe.rs:44-46 */
float orc_silu(float x) { return x * orc_sigmoid(x); }           /* moe.rs:49-51 */

void orc_softmax_in_place(float *x, size_t n) {                 /* moe.rs:61-72 */
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = fmaxf(max, x[i]);      /* f32::max ignores NaN */
    for (size_t i = 0; i < n; ++i) x[i] = expf(x[i] - max);
    float sum = -0.0f;
    for (size_t i = 0; i < n; ++i) sum = sum + x[i];
    if (sum != 0.0f)
        for (size_t i = 0; i < n; ++i) x[i] /= sum;
}

/* Stable descending sort of indices by score; NaN comparisons count as equal, like
 * `partial_cmp(..).unwrap_or(Equal)` under Rust's stable `sort_by` (moe.rs:80-84). */
static void stable_sort_desc(const float *s, uint32_t *idx, size_t n) {
    uint32_t *tmp = (uint32_t *)malloc(n * sizeof(uint32_t));
    if (!tmp) return;
    for (size_t w = 1; w < n; w *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * w) {
            size_t mid = lo + w < n ? lo + w : n, hi = lo + 2 * w < n ? lo + 2 * w : n;
            size_t i = lo, j = mid, k = lo;
            while (i < mid && j < hi) {
                /* take right only if it is strictly greater (keeps stability) */
                if (s[idx[j]] > s[idx[i]]) tmp[k++] = idx[j++];
                else tmp[k++] = idx[i++];
            }
            while (i < mid) tmp[k++] = idx[i++];
            while (j < hi) tmp[k++] = idx[j++];
        }
        memcpy(idx, tmp, n * sizeof(uint32_t));
    }
    free(tmp);
}

size_t orc_top_k(const float *scores, size_t n, size_t k, uint32_t *ids, float *weights) {
    if (n == 0) return 0;
    if (k > n) k = n;
    uint32_t *idx = (uint32_t *)malloc(n * sizeof(uint32_t));
    if (!idx) return 0;
    for (size_t i = 0; i < n; ++i) idx[i] = (uint32_t)i;
    stable_sort_desc(scores, idx, n);
    for (size_t i = 0; i < k; ++i) { ids[i] = idx[i]; weights[i] = scores[idx[i]]; }
    orc_softmax_in_place(weights, k);
    free(idx);
    return k;
}

size_t orc_top_k_sigmoid(const float *scores, size_t n, size_t k, uint32_t *ids, float *weights) {
    if (n == 0) return 0;
    if (k > n) k = n;
    float *sig = (float *)malloc(n * sizeof(float));
    uint32_t *idx = (uint32_t *)malloc(n * sizeof(uint32_t));
    if (!sig || !idx) { free(sig); free(idx); return 0; }
    for (size_t i = 0; i < n; ++i) { sig[i] = orc_sigmoid(scores[i]); idx[i] = (uint32_t)i; }
    stable_sort_desc(sig, idx, n);
    float wsum = -0.0f;
    for (size_t i = 0; i < k; ++i) wsum = wsum + sig[idx[i]];
    for (size_t i = 0; i < k; ++i) {
        ids[i] = idx[i];
        weights[i] = wsum == 0.0f ? 0.0f : sig[idx[i]] / wsum;
    }
    free(sig);
    free(idx);
    return k;
}

/* moe.rs:132-268, both group routers: `top2` selects the group score (0: the group's sum,
 * route_group; 1: its top two, route_noaux_tc). Every step in the reference's order: scores in
 * index order, group sums accumulated in index order from 0.0, groups and candidates ranked by
 * the stable descending sort, the weight sum accumulated in rank order. */
static size_t route_groups(const float *logits, size_t n, const float *bias, size_t bias_len, size_t n_groups,
                           size_t top_k, size_t top_k_group, int top2, uint32_t *ids, float *weights) {
    if (n == 0) return 0;
    float *ex = (float *)malloc(n * sizeof(float));
    uint32_t *cand = (uint32_t *)malloc(n * sizeof(uint32_t));
    size_t ng = n_groups < 1 ? 1 : n_groups;
    if (ng > n) ng = n;
    float *gscore = (float *)malloc(ng * sizeof(float));
    float *t1 = (float *)malloc(ng * sizeof(float));
    float *t2 = (float *)malloc(ng * sizeof(float));
    uint32_t *gorder = (uint32_t *)malloc(ng * sizeof(uint32_t));
    unsigned char *allowed = (unsigned char *)malloc(ng);
    size_t k = 0;
    if (!ex || !cand || !gscore || !t1 || !t2 || !gorder || !allowed) goto out;
    for (size_t i = 0; i < n; ++i) ex[i] = orc_sigmoid(logits[i] + (bias && i < bias_len ? bias[i] : 0.0f));
    for (size_t g = 0; g < ng; ++g) { gscore[g] = 0.0f; t1[g] = -FLT_MAX; t2[g] = -FLT_MAX; }
    for (size_t i = 0; i < n; ++i) {
        const size_t g = i * ng / n;
        if (!top2) {
            gscore[g] += ex[i];                       /* moe.rs:157-160 */
        } else if (ex[i] >= t1[g]) {                  /* moe.rs:222-231 */
            t2[g] = t1[g];
            t1[g] = ex[i];
        } else if (ex[i] > t2[g]) {
            t2[g] = ex[i];
        }
    }
    if (top2)
        for (size_t g = 0; g < ng; ++g) gscore[g] = t1[g] + (t2[g] == -FLT_MAX ? 0.0f : t2[g]);   /* moe.rs:232-234 */
    if (top_k_group == 0) {                           /* None: every group */
        memset(allowed, 1, ng);
    } else {                                          /* moe.rs:165-179, 238-252 */
        for (size_t g = 0; g < ng; ++g) gorder[g] = (uint32_t)g;
        stable_sort_desc(gscore, gorder, ng);
        memset(allowed, 0, ng);
        const size_t take = top_k_group < ng ? top_k_group : ng;
        for (size_t j = 0; j < take; ++j) allowed[gorder[j]] = 1;
    }
    size_t nc = 0;                                    /* moe.rs:182-193, 255-267 */
    for (size_t i = 0; i < n; ++i)
        if (allowed[i * ng / n]) cand[nc++] = (uint32_t)i;
    stable_sort_desc(ex, cand, nc);
    k = top_k < nc ? top_k : nc;
    float wsum = 0.0f;
    for (size_t j = 0; j < k; ++j) wsum += ex[cand[j]];
    for (size_t j = 0; j < k; ++j) {
        ids[j] = cand[j];
        weights[j] = wsum == 0.0f ? 0.0f : ex[cand[j]] / wsum;
    }
out:
    free(ex); free(cand); free(gscore); free(t1); free(t2); free(gorder); free(allowed);
    return k;
}

size_t orc_route_group(const float *logits, size_t n, const float *bias, size_t bias_len, size_t n_groups,
                       size_t top_k, size_t top_k_group, uint32_t *ids, float *weights) {
    return route_groups(logits, n, bias, bias_len, n_groups, top_k, top_k_group, 0, ids, weights);
}

size_t orc_route_noaux_tc(const float *logits, size_t n, const float *bias, size_t bias_len, size_t n_groups,
                          size_t top_k, size_t top_k_group, uint32_t *ids, float *weights) {
    return route_groups(logits, n, bias, bias_len, n_groups, top_k, top_k_group, 1, ids, weights);
}

/* moe.rs:271-277 on a dequantized (padded-row) matrix */
static void matvec_deq(const float *wd, size_t m, size_t n, size_t row_stride, const float *x, float *out) {
    for (size_t r = 0; r < m; ++r) out[r] = seq_sum_products(wd + r * row_stride, x, n);
}

static float *dequant_matrix(uint32_t t, const uint8_t *w, size_t m, size_t n, size_t *stride) {
    size_t qk, bb;
    dq_fn dq;
    if (quant_geom(t, &qk, &bb, &dq)) return NULL;
    size_t nb = (n + qk - 1) / qk;
    float *out = (float *)malloc(m * nb * qk * sizeof(float));
    if (!out) return NULL;
    for (size_t r = 0; r < m; ++r) dequant_row(w + r * nb * bb, out + r * nb * qk, nb, bb, qk, dq);
    *stride = nb * qk;
    return out;
}

int orc_moe_ffn(uint32_t gate_t, const uint8_t *gate, size_t gate_stride,
                uint32_t up_t, const uint8_t *up, size_t up_stride,
                uint32_t down_t, const uint8_t *down, size_t down_stride,
                size_t n_experts, size_t hidden, size_t inter,
                const float *x, size_t tokens, size_t k, const uint32_t *ids,
                const float *weights, float *out) {
    size_t pairs = tokens * k;
    for (size_t p = 0; p < pairs; ++p)
        if (ids[p] >= n_experts) return fail(ORC_ERR_ARG, "expert id %u out of range", ids[p]);
    /* per-pair expert outputs, computed expert by expert so each expert is dequantized once */
    float *eo = (float *)malloc(pairs * hidden * sizeof(float));
    float *g = (float *)malloc(inter * sizeof(float));
    float *u = (float *)malloc(inter * sizeof(float));
    if (!eo || !g || !u) { free(eo); free(g); free(u); return fail(ORC_ERR_ARG, "out of memory"); }
    for (size_t e = 0; e < n_experts; ++e) {
        int used = 0;
        for (size_t p = 0; p < pairs && !used; ++p) used = ids[p] == e;
        if (!used) continue;
        size_t sg, su, sd;
        float *wg = dequant_matrix(gate_t, gate + e * gate_stride, inter, hidden, &sg);
        float *wu = dequant_matrix(up_t, up + e * up_stride, inter, hidden, &su);
        float *wd = dequant_matrix(down_t, down + e * down_stride, hidden, inter, &sd);
        if (!wg || !wu || !wd) {
            free(wg); free(wu); free(wd); free(eo); free(g); free(u);
            return fail(ORC_ERR_TYPE, "moe: bad expert type or out of memory");
        }
        for (size_t p = 0; p < pairs; ++p) {
            if (ids[p] != e) continue;
            const float *xt = x + (p / k) * hidden;
            matvec_deq(wg, inter, hidden, sg, xt, g);           /* moe.rs:296 */
            matvec_deq(wu, inter, hidden, su, xt, u);           /* moe.rs:297 */
            for (size_t i = 0; i < inter; ++i) g[i] = orc_silu(g[i]) * u[i]; /* moe.rs:280-283 */
            matvec_deq(wd, hidden, inter, sd, g, eo + p * hidden);           /* moe.rs:299 */
        }
        free(wg); free(wu); free(wd);
    }
    /* moe.rs:376-383: out += w * eo in routing order */
    for (size_t t = 0; t < tokens; ++t) {
        float *o = out + t * hidden;
        for (size_t i = 0; i < hidden; ++i) o[i] = 0.0f;
        for (size_t j = 0; j < k; ++j) {
            float wt = weights[t * k + j];
            const float *v = eo + (t * k + j) * hidden;
            for (size_t i = 0; i < hidden; ++i) o[i] += wt * v[i];
        }
    }
    free(eo); free(g); free(u);
    return ORC_OK;
}
