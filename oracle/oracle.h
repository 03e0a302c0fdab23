/*
 * CPU oracle for the fused GGUF dequant-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C, the arithmetic of
 * platinoff/rusty-engine for the quantized matmul path so the HIP product can be checked
 * against it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it;
 * the product library (librehip.so) never links, calls or falls back to it.
 *
 * Every function names the reference file:line it follows. Floating-point statements keep
 * the reference's association order; the library is compiled with -ffp-contract=off so no
 * multiply-add is fused unless the reference itself fuses it (the AVX2 f32 dot, restated
 * with fmaf()).
 */
#ifndef RE_ORACLE_H
#define RE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type codes accepted by the path (src/quant.rs:75-88). */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q5_0 = 6, ORC_Q8_0 = 8,
    ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_BF16 = 30
};

/* Return codes. */
enum { ORC_OK = 0, ORC_ERR_TYPE = 1, ORC_ERR_SIZE = 2, ORC_ERR_ARG = 3 };

const char *orc_last_error(void);

/* ---- src/quant.rs ---------------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h);                        /* quant.rs:25-45 */
uint16_t orc_f32_to_f16(float x);                        /* quant.rs:48-72 */
int orc_block_info(uint32_t t, size_t *elements, size_t *bytes);   /* quant.rs:75-88 */
int orc_bytes_for_numel(uint32_t t, size_t numel, size_t *bytes);  /* quant.rs:92-101 */
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m); /* 250-258 */

/* quant.rs:363-453: length-checked dispatch. On success writes *n_out values to out
 * (out may be NULL to query the length). Error codes and messages mirror the reference. */
int orc_dequant(uint32_t t, const uint8_t *data, size_t len, float *out, size_t *n_out);

/* quant.rs:162-229 quantizers (used only to build fixtures). */
int orc_quantize_q8_0(const float *src, size_t n, uint8_t *out);
int orc_quantize_q4_0(const float *src, size_t n, uint8_t *out);

/* ---- src/kernel.rs:70-166: int8 activations (Q8Activation) and the integer Q8_0 dot ---- */
/* Q8Activation::from_f32: scales[n/32] (f32), qs[n] (i8); n a multiple of 32 */
int orc_quantize_q8_act(const float *x, size_t n, float *scales, int8_t *qs);
/* dot_q8_0_i8 over nb whole Q8_0 blocks */
float orc_dot_q8_0_i8(const uint8_t *a, size_t nb, const float *scales, const int8_t *qs);
/* matvec/matmul_q8_0_i8: W m x n Q8_0, activation rows (scales rows x n/32, qs rows x n) */
int orc_matmul_q8_0_i8(const uint8_t *w, size_t m, size_t n, const float *scales, const int8_t *qs,
                       size_t rows, float *out);

/* ---- src/kernel.rs scalar fused dots and GEMV -------------------------------------- */
/* dot over `nb` whole blocks of type t against x[nb*QK] (kernel.rs:17-46, 171-191, 283-322) */
float orc_dot(uint32_t t, const uint8_t *row, size_t nb, const float *x);
/* serial matvec, whole-block rows (kernel.rs:49-68, 194-202, 324-360) */
int orc_matvec(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, float *out);

/* AVX2 f32 dot accumulation order (kernel.rs:1002-1025 + hsum_ps_sse2 367-372), scalar */
float orc_dot_f32(const float *a, const float *b, size_t n);
/* plain sequential f32 dot (infer.rs:66-69, moe.rs:271-277) */
float orc_dot_seq(const float *a, const float *b, size_t n);

/* matmul_reuse (kernel.rs:1383-1590) with explicit knobs; tile/group/w_rows/r_block as in
 * the reference (group clamped to 1..8, w_rows to 1..4). Out is rows x m row-major. */
int orc_matmul_reuse(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x,
                     size_t rows, size_t tile, size_t group, size_t w_rows, size_t r_block,
                     float *out);
/* production constants (kernel.rs:1328-1369, 1640-1947, 2012-2029) */
int orc_matmul(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x, size_t rows,
               float *out);
/* per-block accumulator (kernel.rs:1596-1637) */
int orc_matmul_blocks(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x,
                      size_t rows, size_t tile, float *out);

/* ---- QMat semantics (src/qmat.rs) with the padded-row extension ---------------------
 * Rows hold ceil(n/QK) whole blocks. For n % QK == 0 this is the reference layout; for
 * n % QK != 0 (K-quants at n = 896) element indices >= n are padding and are ignored.
 * matvec: per-row dequant + sequential f32 dot over the first n elements
 * (qmat.rs:145-151 fallback semantics). matmul: row-wise matvec (qmat.rs:357-367). */
int orc_qmat_row_bytes(uint32_t t, size_t n, size_t *row_bytes);
int orc_qmat_matvec(uint32_t t, const uint8_t *w, size_t nbytes, size_t m, size_t n,
                    const float *x, float *out);
int orc_qmat_matmul(uint32_t t, const uint8_t *w, size_t nbytes, size_t m, size_t n,
                    const float *x, size_t rows, float *out);
/* sum_k |w_rk * x_k| per output (the tolerance scale), f64 accumulate */
int orc_qmat_absdot(uint32_t t, const uint8_t *w, size_t nbytes, size_t m, size_t n,
                    const float *x, size_t rows, double *out);

/* ---- src/moe.rs --------------------------------------------------------------------- */
float orc_sigmoid(float x);                                  /* moe.rs:44-46 */
float orc_silu(float x);                                     /* moe.rs:49-51 */
void orc_softmax_in_place(float *x, size_t n);               /* moe.rs:61-72 */
/* moe.rs:75-93: ids/weights must hold min(k, n) entries; returns the count */
size_t orc_top_k(const float *scores, size_t n, size_t k, uint32_t *ids, float *weights);
/* moe.rs:97-117 */
size_t orc_top_k_sigmoid(const float *scores, size_t n, size_t k, uint32_t *ids,
                         float *weights);

/* Bias-corrected group routing (moe.rs:126-268): scores sigmoid(logit + bias[i]) (bias entries
 * past bias_len count as 0), experts split into n_groups contiguous groups (group_of(i) =
 * i * ng / n, ng = clamp(n_groups, 1, n)); the top_k_group best groups are eligible
 * (top_k_group 0: every group, the reference's None); the top_k best eligible experts are
 * renormalised over their scores. orc_route_group scores a group by the sum of its scores
 * (route_group, moe.rs:132-194), orc_route_noaux_tc by the sum of its top two (route_noaux_tc,
 * moe.rs:196-268). ids/weights hold min(top_k, n) entries; returns the count written (fewer
 * when the eligible groups hold fewer experts). */
size_t orc_route_group(const float *logits, size_t n, const float *bias, size_t bias_len, size_t n_groups,
                       size_t top_k, size_t top_k_group, uint32_t *ids, float *weights);
size_t orc_route_noaux_tc(const float *logits, size_t n, const float *bias, size_t bias_len, size_t n_groups,
                          size_t top_k, size_t top_k_group, uint32_t *ids, float *weights);

/* Quantized expert FFN layer for a batch of tokens (moe.rs:288-300 + 360-388 applied to
 * dequantized experts): for token t, out[t] = sum over its k routed experts, in routing
 * order, of weight * down(silu(gate x) * up x). gate/up are inter x hidden, down is
 * hidden x inter; expert e's bytes start at gate + e*gate_stride (etc). */
int orc_moe_ffn(uint32_t gate_t, const uint8_t *gate, size_t gate_stride,
                uint32_t up_t, const uint8_t *up, size_t up_stride,
                uint32_t down_t, const uint8_t *down, size_t down_stride,
                size_t n_experts, size_t hidden, size_t inter,
                const float *x, size_t tokens, size_t k, const uint32_t *ids,
                const float *weights, float *out);

/* ---- CPU baseline (reference-restated pooled kernels, AVX2+FMA) ---------------------- */
/* Pooled QMat::matmul (qmat.rs:169-272) over matmul_reuse with AVX2 dot_f32_x4x2, and
 * pooled QMat::matvec (qmat.rs:80-127). threads = 0 -> online CPU count. */
int orc_cpu_matmul(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x,
                   size_t rows, float *out, int threads);
int orc_cpu_matvec(uint32_t t, const uint8_t *w, size_t m, size_t n, const float *x,
                   float *out, int threads);
int orc_cpu_has_avx2(void);

#ifdef __cplusplus
}
#endif
#endif
