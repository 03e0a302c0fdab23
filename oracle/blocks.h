/*
 * Block dequantizers and geometry shared by the oracle and the CPU baseline.
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Included by oracle.c and baseline.c, each of
 * which compiles its own static copy.
 */
#ifndef RE_ORACLE_BLOCKS_H
#define RE_ORACLE_BLOCKS_H
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* src/quant.rs:25-45 */
static inline float f16_to_f32_bits(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t frac = h & 0x3FF;
    uint32_t bits;
    if (exp == 0 && frac == 0) {
        bits = sign;
    } else if (exp == 0) {
        uint32_t e = 113, f = frac;
        while ((f & 0x400) == 0) { f <<= 1; e -= 1; }
        bits = sign | (e << 23) | ((f & 0x3FF) << 13);
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (frac << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (frac << 13);
    }
    return bits_f32(bits);
}

/* src/quant.rs:250-258 */
static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ---- block dequantizers: kernel.rs:965-993 (32-blocks), 206-279 (K-quants) ----------
 * These equal quant.rs:106-357 value for value (every product is exact, the K-quant
 * subtraction rounds once in both). */
static void dq_q4_0(const uint8_t *b, float *out) {          /* kernel.rs:965-972 */
    float d = f16_to_f32_bits(rd16(b));
    const uint8_t *qs = b + 2;
    for (int j = 0; j < 16; ++j) {
        out[j] = d * (float)((int)(qs[j] & 0x0F) - 8);
        out[16 + j] = d * (float)((int)(qs[j] >> 4) - 8);
    }
}

static void dq_q5_0(const uint8_t *b, float *out) {          /* kernel.rs:975-985 */
    float d = f16_to_f32_bits(rd16(b));
    uint32_t qh = rd32(b + 2);
    const uint8_t *qs = b + 6;
    for (int j = 0; j < 16; ++j) {
        int bit0 = (int)(((qh >> j) & 1) << 4);
        int bit1 = (int)(((qh >> (j + 16)) & 1) << 4);
        out[j] = d * (float)(((int)(qs[j] & 0x0F) | bit0) - 16);
        out[16 + j] = d * (float)(((int)(qs[j] >> 4) | bit1) - 16);
    }
}

static void dq_q8_0(const uint8_t *b, float *out) {          /* kernel.rs:988-993 */
    float d = f16_to_f32_bits(rd16(b));
    for (int j = 0; j < 32; ++j) out[j] = (float)(int8_t)b[2 + j] * d;
}

static void dq_q4_k(const uint8_t *b, float *out) {          /* kernel.rs:206-225 */
    float d = f16_to_f32_bits(rd16(b));
    float min = f16_to_f32_bits(rd16(b + 2));
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int g = 0; g < 4; ++g) {
        uint8_t sc0, m0, sc1, m1;
        scale_min_k4(g * 2, scales, &sc0, &m0);
        scale_min_k4(g * 2 + 1, scales, &sc1, &m1);
        float d1 = d * (float)sc0, dm1 = min * (float)m0;
        float d2 = d * (float)sc1, dm2 = min * (float)m1;
        for (int l = 0; l < 32; ++l) {
            uint8_t q = qs[g * 32 + l];
            out[g * 64 + l] = d1 * (float)(q & 0xF) - dm1;
            out[g * 64 + 32 + l] = d2 * (float)(q >> 4) - dm2;
        }
    }
}

static void dq_q5_k(const uint8_t *b, float *out) {          /* kernel.rs:229-252 */
    float d = f16_to_f32_bits(rd16(b));
    float min = f16_to_f32_bits(rd16(b + 2));
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    for (int g = 0; g < 4; ++g) {
        uint8_t sc0, m0, sc1, m1;
        scale_min_k4(g * 2, scales, &sc0, &m0);
        scale_min_k4(g * 2 + 1, scales, &sc1, &m1);
        float d1 = d * (float)sc0, dm1 = min * (float)m0;
        float d2 = d * (float)sc1, dm2 = min * (float)m1;
        uint8_t u1 = (uint8_t)(1u << (2 * g)), u2 = (uint8_t)(2u << (2 * g));
        for (int l = 0; l < 32; ++l) {
            int lo = (int)(qs[g * 32 + l] & 0xF) + ((qh[l] & u1) ? 16 : 0);
            int hi = (int)(qs[g * 32 + l] >> 4) + ((qh[l] & u2) ? 16 : 0);
            out[g * 64 + l] = d1 * (float)lo - dm1;
            out[g * 64 + 32 + l] = d2 * (float)hi - dm2;
        }
    }
}

static void dq_q6_k(const uint8_t *b, float *out) {          /* kernel.rs:256-279 */
    float d = f16_to_f32_bits(rd16(b + 208));
    const uint8_t *ql = b, *qh = b + 128, *sc = b + 192;
    for (int half = 0; half < 2; ++half) {
        int qb = half * 64, hb = half * 32, sb = half * 8;
        float *o = out + half * 128;
        for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            int q1 = ((int)(ql[qb + l] & 0xF) | ((int)(qh[hb + l] & 3) << 4)) - 32;
            int q2 = ((int)(ql[qb + l + 32] & 0xF) | ((int)((qh[hb + l] >> 2) & 3) << 4)) - 32;
            int q3 = ((int)(ql[qb + l] >> 4) | ((int)((qh[hb + l] >> 4) & 3) << 4)) - 32;
            int q4 = ((int)(ql[qb + l + 32] >> 4) | ((int)((qh[hb + l] >> 6) & 3) << 4)) - 32;
            o[l] = d * (float)(int8_t)sc[sb + is] * (float)q1;
            o[l + 32] = d * (float)(int8_t)sc[sb + is + 2] * (float)q2;
            o[l + 64] = d * (float)(int8_t)sc[sb + is + 4] * (float)q3;
            o[l + 96] = d * (float)(int8_t)sc[sb + is + 6] * (float)q4;
        }
    }
}

typedef void (*dq_fn)(const uint8_t *, float *);

/* type -> (elements per block, bytes per block, dequantizer); kernel.rs:1891-1898, 1983-1993 */
static inline int quant_geom_raw(uint32_t t, size_t *qk, size_t *bb, dq_fn *dq) {
    switch (t) {
    case 2: *qk = 32; *bb = 18; *dq = dq_q4_0; return 0;
    case 6: *qk = 32; *bb = 22; *dq = dq_q5_0; return 0;
    case 8: *qk = 32; *bb = 34; *dq = dq_q8_0; return 0;
    case 12: *qk = 256; *bb = 144; *dq = dq_q4_k; return 0;
    case 13: *qk = 256; *bb = 176; *dq = dq_q5_k; return 0;
    case 14: *qk = 256; *bb = 210; *dq = dq_q6_k; return 0;
    default: return 1;
    }
}
#endif
