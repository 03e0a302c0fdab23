/*
 * librehip: MI355X (gfx950) fused GGUF dequant-matmul behind a C ABI.
 *
 * Drop-in for the quantized projection path of platinoff/rusty-engine:
 *   QMat::matvec  src/qmat.rs:80     -> re_qmat_matvec
 *   QMat::matmul  src/qmat.rs:169    -> re_qmat_matmul
 *   QMat::from_bytes / from_model    -> re_qmat_create   (src/qmat.rs:52-59, 312-330)
 *   quant::dequant src/quant.rs:363  -> re_dequant        (bit-exact, quant and float types)
 *   moe expert FFN + combine          -> re_moe_forward    (src/moe.rs:288-300, 360-388)
 *
 * Conventions (from the reference):
 *   - W is m x n row-major; each row is a run of GGUF blocks (kernel.rs:51, 329). GGUF dims
 *     are [n, m] (qmat.rs:310-311).
 *   - X is rows x n row-major f32; Y is rows x m row-major f32, Y[row*m + r] (kernel.rs:1508).
 *   - ggml types: 2 Q4_0, 6 Q5_0, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K (quant.rs:75-88).
 *   - n must be a multiple of 32. When n is not a multiple of the type's block size (the
 *     K-quants at n = 896), each row holds ceil(n/256) whole super-blocks and the elements
 *     past n are ignored.
 *
 * Every entry point returns 0 on success or an RE_ERR_* code; re_last_error() gives the
 * message of the calling thread's last failure. Nothing panics or throws across the ABI.
 * Host-pointer entry points are synchronous and thread-safe (calls on one matrix serialize).
 * Device-pointer entry points (*_dev) enqueue on the caller's HIP stream and return at once;
 * calls on the same matrix object must not overlap in time (they share its split scratch).
 */
#ifndef REHIP_H
#define REHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RE_OK 0
#define RE_ERR_TYPE 1      /* unknown / unsupported ggml type (kernel.rs:2006, 2027 panic) */
#define RE_ERR_SIZE 2      /* byte count or shape mismatch (quant.rs:402-447) */
#define RE_ERR_ARG 3       /* null pointer or invalid argument */
#define RE_ERR_HIP 4       /* HIP runtime failure */
#define RE_ERR_NODEV 5     /* no usable gfx950 device */

#define RE_MODE_BF16 0     /* GEMM: bf16 MFMA, f32 accumulate (|err| <= 1e-2 rel-to-norm) */
#define RE_MODE_F32 1      /* GEMM: f32-accurate mode (|err| <= 2^-10 sum|w*x|): GEMMs run bf16 MFMAs on
                              split operands (hi*hi + hi*lo + lo*hi; two MFMAs for BF16 weights, whose
                              low part is zero); REHIP_GEMM_SP=0 keeps f32 MFMAs above 64 rows */

typedef struct re_qmat re_qmat;
typedef struct re_moe re_moe;

/* Library state. re_init selects the current HIP device; it is called implicitly. */
int re_init(void);
const char *re_last_error(void);
const char *re_version(void);

/* ---- layout (host only; no GPU needed) ------------------------------------------------ */
/* Bytes of one padded GGUF row: ceil(n/QK) * block_bytes (kernel.rs:1983-1993, padded). */
int re_row_bytes(uint32_t ggml_type, size_t n, size_t *out);
/* Size of the GPU-resident tiled layout of an m x n matrix. */
int re_tiled_bytes(uint32_t ggml_type, size_t m, size_t n, size_t *out);
/* Repack GGUF rows into the tiled layout on the host (out holds re_tiled_bytes bytes). */
int re_repack(uint32_t ggml_type, const uint8_t *bytes, size_t nbytes, size_t m, size_t n,
              uint8_t *out, size_t out_len);

/* ---- QMat (src/qmat.rs:30-42) ---------------------------------------------------------- */
/* Upload and repack once. nbytes must equal m * re_row_bytes(type, n). F32 (0), F16 (1) and
 * BF16 (30) bytes are QMat::F32 / the no-fused-kernel arms (qmat.rs:45-49, 128-151): kept
 * row-major, nbytes = m * n * element size; they do not stack. Below 16 activation rows their
 * products are f32 in every mode; from 16 rows (n a multiple of 8) an MFMA GEMM, with bf16
 * operands in bf16 mode and f32 ones in f32 mode. re_qmat_matvec_ex_dev's RMS-norm runs as its own
 * launch into a buffer the matrix owns, and re_ffn_create pairs two dense matrices of one type. */
int re_qmat_create(uint32_t ggml_type, const uint8_t *bytes, size_t nbytes, size_t m, size_t n,
                   re_qmat **out);
/* A stack of `count` same-type, same-shape matrices (nbytes = count * m * row bytes, one after
 * the other, as ExpertWeights holds experts, moe.rs:349-353); every other entry point works on
 * matrix 0, re_qmat_matvec_stacked_dev on any range of them in one launch. */
int re_qmat_create_stacked(uint32_t ggml_type, const uint8_t *bytes, size_t nbytes, size_t m, size_t n,
                           size_t count, re_qmat **out);
size_t re_qmat_count(const re_qmat *q);
void re_qmat_destroy(re_qmat *q);
size_t re_qmat_rows(const re_qmat *q);   /* m (qmat.rs:62-66) */
size_t re_qmat_cols(const re_qmat *q);   /* n (qmat.rs:69-73) */
uint32_t re_qmat_type(const re_qmat *q);

/* y[m] = W x[n] (qmat.rs:80). Host pointers, synchronous. f32 accumulation. */
int re_qmat_matvec(re_qmat *q, const float *x, float *y);
/* Y[rows x m] = X[rows x n] W^T (qmat.rs:169). Host pointers, synchronous. rows == 1 runs
 * the GEMV; otherwise the MFMA GEMM in the given mode. */
int re_qmat_matmul(re_qmat *q, const float *x, size_t rows, float *y, int mode);

/* Device-pointer variants; `stream` is a hipStream_t (NULL = default stream). */
int re_qmat_matvec_dev(re_qmat *q, const float *d_x, float *d_y, void *stream);
int re_qmat_matmul_dev(re_qmat *q, const float *d_x, size_t rows, float *d_y, int mode,
                       void *stream);
/* re_qmat_matmul_dev that allocates nothing, for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). It has no
 * counterpart in the reference. The GEMM's K-split partial tiles go to a static device scratch of
 * 32 MiB per GPU instead of a buffer the matrix grows on first use; the same plan, kernels and
 * results as re_qmat_matmul_dev. A plan whose partials exceed the scratch fails with RE_ERR_SIZE
 * (the planned splits of every shape fit: the planner caps partial tiles at 32 MiB). The scratch
 * is shared by every call on a GPU. Outside stream capture, a call on a different stream than the
 * previous call on that GPU first waits for the previous call's launches (an event set up once per
 * device), so calls from several streams or threads stay ordered. Inside stream capture no
 * ordering is added: replays of captured graphs that use the scratch must not overlap in time. */
int re_qmat_matmul_noalloc_dev(re_qmat *q, const float *d_x, size_t rows, float *d_y, int mode, void *stream);
/* Dequantize the resident weights to d_out[m x n] f32, bit-exact with quant::dequant. */
int re_qmat_dequant_dev(re_qmat *q, float *d_out, void *stream);

/* Flat-stream dequant on the GPU (quant::dequant, src/quant.rs:363-453) for the six quant
 * types and F32/F16/BF16: out receives nbytes / block_bytes * QK floats (nbytes / element size
 * for the float types). Same length errors as the reference. */
int re_dequant(uint32_t ggml_type, const uint8_t *bytes, size_t nbytes, float *out, size_t out_len);

/* ---- MoE expert FFN (src/moe.rs:288-300, 360-388) ------------------------------------- */
/* Experts stored like a GGUF expert tensor: gate/up are n_experts x inter x hidden, down is
 * n_experts x hidden x inter, each expert's rows as GGUF blocks. */
int re_moe_create(uint32_t gate_type, const uint8_t *gate, size_t gate_bytes,
                  uint32_t up_type, const uint8_t *up, size_t up_bytes,
                  uint32_t down_type, const uint8_t *down, size_t down_bytes,
                  size_t n_experts, size_t hidden, size_t inter, re_moe **out);
void re_moe_destroy(re_moe *e);
/* out[t] = sum_j weights[t*k+j] * down_e(silu(gate_e x_t) * up_e x_t), e = ids[t*k+j], summed
 * in routing order j = 0..k-1 (moe.rs:376-383). Routing comes from the host router
 * (moe.rs:75-125). Host pointers, synchronous. */
int re_moe_forward(re_moe *e, const float *x, size_t tokens, size_t top_k, const uint32_t *ids,
                   const float *weights, float *out, int mode);
/* Device x/out; ids and weights stay on the host (they shape the grouped launch). */
int re_moe_forward_dev(re_moe *e, const float *d_x, size_t tokens, size_t top_k,
                       const uint32_t *ids, const float *weights, float *d_out, int mode,
                       void *stream);
/* Shared expert (moe_layer_forward's `shared`, moe.rs:380-385 and 424-429; combine, moe.rs:339-343):
 * a dense SwiGLU FFN (gate and up inter x hidden, down hidden x inter, each of any type QMat takes)
 * run on every token and added after the routed sum, out[t] = sum_j w_j expert_j(x_t) +
 * down(silu(gate x_t) * up x_t). Once set, every forward call of e adds it (re_moe_forward, _dev,
 * _routed_dev, re_moe_layer_dev). All three pointers NULL removes it. It takes e's lock (held
 * by re_moe_forward) and waits for the device to drain before freeing the previous shared
 * matrices, so forwards queued before the call finish with them; device-pointer forwards that
 * another thread enqueues while it runs are not ordered with it. */
int re_moe_set_shared(re_moe *e, uint32_t gate_type, const uint8_t *gate, size_t gate_bytes,
                      uint32_t up_type, const uint8_t *up, size_t up_bytes,
                      uint32_t down_type, const uint8_t *down, size_t down_bytes, size_t inter);

/* ---- MoE layer with the routing on the device (moe.rs:75-125, 360-388): no host round trip --
 * re_moe_router_logits_dev: logits[t][e] = router_w[e] . x[t] (router_w f32, n_experts x hidden;
 *   the matvec of moe.rs:367).
 * re_moe_route_dev: top_k experts per token (ties to the lower expert index, as the reference's
 *   stable descending sort) and their weights: RE_GATE_SOFTMAX = softmax over the chosen logits
 *   (top_k, moe.rs:75-93), RE_GATE_SIGMOID = per-expert sigmoid renormalised over the chosen
 *   (top_k_sigmoid, moe.rs:98-118). n_experts <= 1024. NaN logits rank as -inf.
 * re_moe_forward_routed_dev: re_moe_forward_dev with device ids/weights (tokens x top_k); the
 *   grouping by expert and the task lists are built by a kernel; tokens * top_k <= 8192. An id
 *   outside [0, n_experts) contributes nothing.
 * re_moe_layer_dev: the three in one stream (scratch for logits/ids/weights is kept by e).
 * re_moe_route_group_dev: the bias-corrected group routers (moe.rs:126-268): scores
 *   sigmoid(logit + bias[e]) (bias entries past bias_len count as 0; d_bias may be NULL with
 *   bias_len 0), experts in n_groups contiguous groups (expert e in group e * ng / n_experts,
 *   ng = n_groups clamped to 1 ..= n_experts), only the top_k_group best groups eligible
 *   (0 = every group), the top_k best eligible experts renormalised over their scores.
 *   RE_GATE_GROUP scores a group by its summed scores (route_group, moe.rs:132-194),
 *   RE_GATE_NOAUX_TC by its two best (route_noaux_tc, moe.rs:196-268, DeepSeek-V3 / Qwen3).
 *   Ties go to the lower group / expert index. When the eligible groups hold fewer than top_k
 *   experts, the remaining slots get id -1 and weight 0 (they contribute nothing downstream).
 * re_moe_layer_group_dev: router logits, group routing and the FFN in one stream. */
#define RE_GATE_SOFTMAX 0
#define RE_GATE_SIGMOID 1
#define RE_GATE_GROUP 2
#define RE_GATE_NOAUX_TC 3
int re_moe_router_logits_dev(const float *d_x, const float *d_router_w, size_t tokens, size_t hidden,
                             size_t n_experts, float *d_logits, void *stream);
int re_moe_route_dev(const float *d_logits, size_t tokens, size_t n_experts, size_t top_k, int gate,
                     int *d_ids, float *d_weights, void *stream);
int re_moe_forward_routed_dev(re_moe *e, const float *d_x, size_t tokens, size_t top_k, const int *d_ids,
                              const float *d_weights, float *d_out, int mode, void *stream);
int re_moe_layer_dev(re_moe *e, const float *d_x, size_t tokens, const float *d_router_w, size_t top_k,
                     int gate, float *d_out, int mode, void *stream);
int re_moe_route_group_dev(const float *d_logits, size_t tokens, size_t n_experts, size_t top_k, int gate,
                           const float *d_bias, size_t bias_len, size_t n_groups, size_t top_k_group,
                           int *d_ids, float *d_weights, void *stream);
int re_moe_layer_group_dev(re_moe *e, const float *d_x, size_t tokens, const float *d_router_w, size_t top_k,
                           int gate, const float *d_bias, size_t bias_len, size_t n_groups,
                           size_t top_k_group, float *d_out, int mode, void *stream);

/* ---- device-resident transformer steps (src/forward.rs, src/infer.rs, src/runner.rs) ------
 * Device pointers, enqueued on `stream`. Positions come from a device int (*d_pos) so that a
 * captured graph serves every decode step; re_pos_add_dev advances it on the stream. */
typedef struct re_ffn re_ffn;

/* y = W norm(x) + add, with the pieces of the transformer block around a projection folded in:
 *   d_norm_w  NULL, or x is RMS-normalised first, x * (1/sqrt(mean(x^2) + eps)) * norm_w
 *             (the attention/FFN/output norms, infer.rs:72-82, forward.rs:432, 479, runner.rs:275);
 *   d_add     NULL, or added to the result (may equal y): the residual adds (forward.rs:472-485);
 *   d_best    NULL, or RE_ARGMAX_SLOTS uint64 slots that keep the maximum of key(y[r], r) over
 *             the rows, the key ordering by value and then by index, so the low 32 bits of the
 *             largest slot end as the greedy token (infer.rs:217-223: the last index among equal
 *             maxima). The slots must start at 0 (re_decode_advance_dev clears them).
 * x and norm_w are 16-byte aligned. */
/* y_b = W_b x_b for the matrices b = first .. first + count - 1 of a stack, in one launch:
 * x_b = d_x + (b - first) * x_stride (x_stride 0: one shared x), y_b = d_y + (b - first) *
 * y_stride. Each result is the GEMV of re_qmat_matvec_dev (qmat.rs:80) up to summation order:
 * the launch shape is planned for the whole stack. */
int re_qmat_matvec_stacked_dev(re_qmat *q, size_t first, size_t count, const float *d_x, size_t x_stride,
                               float *d_y, size_t y_stride, void *stream);
/* Launch shape the GEMV of re_qmat_matvec_dev (count = 1) or of a re_qmat_matvec_stacked_dev call
 * over `count` matrices would use, for tests and profiles (no counterpart in the reference, whose
 * GEMV has one shape): kernel RE_GEMV_TILE (one 64-row tile per workgroup), RE_GEMV_ROWS (row
 * groups of 4/8/16 rows), RE_GEMV_SPLIT (rows split over workgroups + a reduce) or RE_GEMV_DENSE
 * (F32/F16/BF16 weights); waves per workgroup; half = 1 when super-blocks stream half blocks. */
#define RE_GEMV_SPLIT 0
#define RE_GEMV_ROWS 1
#define RE_GEMV_TILE 2
#define RE_GEMV_DENSE 3
int re_qmat_gemv_plan(const re_qmat *q, size_t count, int *kernel, int *rows_per_group, int *waves, int *half);
int re_qmat_matvec_ex_dev(re_qmat *q, const float *d_x, const float *d_norm_w, float eps, const float *d_add,
                          float *d_y, unsigned long long *d_best, void *stream);
/* out[r] = x[r] * (1 / sqrt(mean(x[r]^2) + eps)) * w for rows x d (infer.rs:72-82). */
int re_rmsnorm_dev(const float *d_x, const float *d_w, size_t rows, size_t d, float eps, float *d_out,
                   void *stream);
/* NeoX rotate-half of rows x heads x head_dim in place, row r at position *d_pos + pos_offset + r
 * (infer.rs:90-139, angle = pos * theta^(-2i/head_dim)). */
int re_rope_dev(float *d_x, size_t rows, size_t heads, size_t head_dim, float theta, const int *d_pos,
                int pos_offset, void *stream);
/* Append rows x kv_dim of K and V at cache rows *d_pos + r (the rotated-key cache of
 * forward.rs:347-363). The caches hold max_seq rows; rows that would land at or past max_seq
 * are not stored (the caller keeps *d_pos + rows <= max_seq). */
int re_kv_append_dev(const float *d_k, const float *d_v, size_t rows, size_t kv_dim, float *d_kcache,
                     float *d_vcache, size_t max_seq, const int *d_pos, void *stream);
/* Causal GQA attention of rows x n_heads x head_dim queries at positions *d_pos + r over cache
 * rows 0..position (forward.rs:232-277, 437-470); max_seq <= 32768 cache rows, positions are
 * clamped to them. Output rows x n_heads x head_dim. Rows >= 8 with head_dim 64 run as f32 MFMA
 * flash attention; fewer rows use d_work (re_attention_work_bytes bytes; NULL = one workgroup
 * per head and row, slower for long caches) to split the cache over workgroups. Buffers are
 * 16-byte aligned. */
size_t re_attention_work_bytes(size_t rows, size_t n_heads, size_t head_dim, size_t max_seq);
int re_attention_dev(const float *d_q, const float *d_kcache, const float *d_vcache, size_t rows,
                     size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t max_seq,
                     const int *d_pos, float *d_work, size_t work_bytes, float *d_ctx, void *stream);
/* NeoX RoPE table (infer.rs:90-139): d_table[(p * head_dim/2 + i) * 2 + {0, 1}] = cos, sin of pair
 * i's angle at position p, for p < rows (rows * head_dim floats), computed exactly as the rotation
 * kernels compute them, so a rotation read from the table has the same bits. head_dim even. */
int re_rope_table_dev(float theta, size_t head_dim, size_t rows, float *d_table, void *stream);
/* One decode row's attention with the q/k/v epilogue folded in (forward.rs:347-363, 437-470):
 * d_q / d_k / d_v are the raw projection outputs of the row (no bias, not rotated); q and k get
 * their biases and NeoX RoPE at *d_pos, v its bias, k and v are appended at cache row *d_pos
 * (not stored at or past max_seq), and attention over rows 0..*d_pos is written to d_ctx
 * (n_heads x head_dim). Same results as re_qkv_rope_append_dev followed by re_attention_dev with
 * rows = 1, in two kernels instead of three. d_rope: NULL, or re_rope_table_dev's table for theta
 * and head_dim with max_seq rows; with it (head_dim % 8 == 0 and q, k, v, biases and table 16-byte
 * aligned) the rotation reads its cosines and sines instead of computing them (same results,
 * shorter critical path). d_work: re_attention_work_bytes(1, ...) bytes. */
int re_attention_decode_dev(const float *d_q, const float *d_k, const float *d_v, const float *d_bq,
                            const float *d_bk, const float *d_bv, size_t n_heads, size_t n_kv_heads,
                            size_t head_dim, float theta, const float *d_rope, const int *d_pos, float *d_kcache,
                            float *d_vcache, size_t max_seq, float *d_work, size_t work_bytes, float *d_ctx,
                            void *stream);
/* The q/k/v projections' epilogue (forward.rs:347-363, 437-449): q = q + bq and k = k + bk
 * rotated (NeoX, as re_rope_dev) at position *d_pos + r, v = v + bv; rotated q written to
 * d_qout (rows x n_heads x head_dim), k and v appended at cache rows *d_pos + r (rows past
 * max_seq are not stored). The three inputs are row-strided (ldq/ldk/ldv floats), so they may
 * be slices of one fused q|k|v projection. Biases may be NULL. */
int re_qkv_rope_append_dev(const float *d_q, size_t ldq, const float *d_k, size_t ldk, const float *d_v,
                           size_t ldv, const float *d_bq, const float *d_bk, const float *d_bv, size_t rows,
                           size_t n_heads, size_t n_kv_heads, size_t head_dim, float theta, const int *d_pos,
                           float *d_qout, float *d_kcache, float *d_vcache, size_t max_seq, void *stream);
/* End of a greedy step (runner.rs:262-282): *d_tok = the token in the largest of the
 * RE_ARGMAX_SLOTS slots at d_best (low 32 bits), *d_pos += delta, d_hist[*d_pos] = *d_tok when
 * d_hist is given and *d_pos < hist_len, and the slots cleared for the next step. */
#define RE_ARGMAX_SLOTS 8
int re_decode_advance_dev(unsigned long long *d_best, int *d_tok, int *d_pos, int delta, int *d_hist,
                          size_t hist_len, void *stream);
/* out[i] = a[i] + b[i % nb] (residual add for nb == n, per-column bias for nb | n). */
int re_add_dev(const float *d_a, const float *d_b, size_t n, size_t nb, float *d_out, void *stream);
/* h = silu(g) * u elementwise (moe.rs:44-51, 280-283). */
int re_swiglu_dev(const float *d_g, const float *d_u, float *d_h, size_t n, void *stream);
/* *d_idx = index of the largest of n values; the last one among equal maxima (infer.rs:217-223). */
int re_argmax_dev(const float *d_x, size_t n, int *d_idx, void *stream);
/* out[r] = table[tok[r]] for rows tokens of an n_vocab x d f32 table (runner.rs:105-122); a token
 * outside [0, n_vocab) gives a zero row (the host checks prompt ids before upload). */
int re_embed_dev(const float *d_table, size_t n_vocab, size_t d, const int *d_tok, size_t rows, float *d_out,
                 void *stream);
/* *d_pos += delta on the stream. */
int re_pos_add_dev(int *d_pos, int delta, void *stream);
/* A gate/up pair (same type and shape, inter x hidden) read side by side for one activation row:
 * h = silu(gate x) * (up x) in one launch (the SwiGLU FFN input, forward.rs:100-105). Dense
 * (F32/F16/BF16) pairs run the norm, the two products and SwiGLU as four launches through a buffer
 * the pair owns. The pair keeps references to the two matrices, which must outlive it. */
int re_ffn_create(re_qmat *gate, re_qmat *up, re_ffn **out);
void re_ffn_destroy(re_ffn *f);
/* d_norm_w: NULL, or x is RMS-normalised first (the FFN norm, forward.rs:479). */
int re_ffn_forward_dev(re_ffn *f, const float *d_x, const float *d_norm_w, float eps, float *d_h, void *stream);

/* ---- int8 activations (src/kernel.rs:70-166) ------------------------------------------
 * re_quantize_q8_act[_dev]: Q8Activation::from_f32 (kernel.rs:88-105) of `rows` activation rows
 * of n values (n a multiple of 32): scales rows x n/32 f32 (d = max|x|/127 per block) and qs
 * rows x n i8 (round half away from zero of x/d, clamped to [-127, 127]), each row laid out like
 * one Q8Activation. The _dev form needs x and qs 16-byte aligned. Bit-identical to the reference.
 * re_qmat_matmul_i8[_dev]: matvec_q8_0_i8 / matmul_q8_0_i8 (kernel.rs:145-166) of a Q8_0 QMat
 * against such rows: y (rows x m) = per block the exact i32 dot of weight and activation i8,
 * folded as s += ((f32)isum * dw) * dx in block order; bit-identical to dot_q8_0_i8
 * (kernel.rs:123-142). RE_ERR_TYPE for a matrix that is not Q8_0. */
int re_quantize_q8_act(const float *x, size_t rows, size_t n, float *scales, int8_t *qs);
int re_quantize_q8_act_dev(const float *d_x, size_t rows, size_t n, float *d_scales, int8_t *d_qs, void *stream);
int re_qmat_matmul_i8(re_qmat *q, const float *scales, const int8_t *qs, size_t rows, float *y);
int re_qmat_matmul_i8_dev(re_qmat *q, const float *d_scales, const int8_t *d_qs, size_t rows, float *d_y,
                          void *stream);

/* ---- GGUF model files (src/gguf.rs:17-392, src/loader.rs:17-130) ----
 * re_gguf_open maps the file read-only and parses its header: magic "GGUF", version 2 (u32
 * counts) or 3 (u64 counts), metadata of every value kind (nested arrays included), up to 8 dims
 * per tensor, data start = header end rounded up to general.alignment (U32 or U64; default 32).
 * Parse failures return RE_ERR_ARG with "gguf parse error at <offset>: <message>" (gguf.rs:60-70).
 * Strings and tensor data returned below point into the mapping and live until re_gguf_close. */
typedef struct re_gguf re_gguf;
int re_gguf_open(const char *path, re_gguf **out);               /* MmapModel::open (loader.rs:30-50) */
void re_gguf_close(re_gguf *g);
uint32_t re_gguf_version(const re_gguf *g);
size_t re_gguf_kv_count(const re_gguf *g);
size_t re_gguf_tensor_count(const re_gguf *g);
uint64_t re_gguf_alignment(const re_gguf *g);                  /* GgufFile::alignment (gguf.rs:143-150) */
size_t re_gguf_data_offset(const re_gguf *g);                  /* header end, before alignment */
size_t re_gguf_data_start(const re_gguf *g);                   /* aligned_start (loader.rs:17-21) */
/* i-th metadata key (NUL-terminated copy) and its value kind (0 U8 .. 12 F64, gguf.rs:274-312). */
int re_gguf_kv(const re_gguf *g, size_t i, const char **key, uint32_t *kind);
/* First value under `key` (gguf.rs:139-141): integers and Bool widened to int64, F32/F64 to
 * double, strings as (pointer, length) without a NUL, arrays as element kind and count. */
int re_gguf_get_int(const re_gguf *g, const char *key, int64_t *v);
int re_gguf_get_float(const re_gguf *g, const char *key, double *v);
int re_gguf_get_str(const re_gguf *g, const char *key, const char **s, size_t *len);
int re_gguf_get_array(const re_gguf *g, const char *key, uint32_t *elem_kind, uint64_t *count);
/* Tensor i: name, ggml type, dims (dims[0..7], zero past n_dims) and byte offset past data start. */
int re_gguf_tensor_info(const re_gguf *g, size_t i, const char **name, uint32_t *type, uint32_t *n_dims,
                        uint64_t *dims, uint64_t *offset);
int re_gguf_find_tensor(const re_gguf *g, const char *name, size_t *index);
/* MmapModel::tensor_bytes (loader.rs:95-101): [data_start + offset, + nbytes) of the mapping,
 * nbytes from the type and element count (quant.rs:75-101); RE_ERR_TYPE for an unsized type or
 * a count that is not whole blocks, RE_ERR_SIZE when the range leaves the file. */
int re_gguf_tensor_data(const re_gguf *g, size_t i, const uint8_t **data, size_t *nbytes);
/* QMat::from_model (qmat.rs:310-330): W[m x n] from the tensor with dims [n, m] (or [n, m, count]:
 * a stacked QMat of count matrices). The mapped bytes are copied to the device unchanged and
 * repacked there. Errors: "QMat: tensor '<name>' missing" / "... bytes out of bounds". */
int re_qmat_from_gguf(const re_gguf *g, const char *name, size_t m, size_t n, re_qmat **out);
/* One MoE layer's stacked experts (model.rs:372-389): gate and up tensors with dims
 * [hidden, inter, n_experts], down with [inter, hidden, n_experts]. */
int re_moe_from_gguf(const re_gguf *g, const char *gate, const char *up, const char *down, size_t n_experts,
                     size_t hidden, size_t inter, re_moe **out);

#ifdef __cplusplus
}
#endif
#endif /* REHIP_H */
