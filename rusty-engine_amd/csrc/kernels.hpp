// Kernel argument blocks and host-side launchers shared by the C ABI (api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace rehip {

struct GemvArgs {
  const uint8_t* W;      // tiled slabs of one matrix
  const float* x;        // K floats
  float* y;              // m floats
  float* partial;        // splits * m_pad floats (splits > 1), reduced by a second kernel
  int m, m_pad, K, KB, tiles;
  int kb_per_split, splits;     // split launch (rows_per_group == 0)
  int rows_per_group;           // row-group launch: 64, 16, 8 or 4 rows per workgroup; 0 = split launch
  int groups;                   // row-group launch: tiles * 64 / rows_per_group
  const float* add;             // nullptr, or y[r] = (W x)[r] + add[r] (add may equal y)
  const float* norm_w;          // nullptr, or x is RMS-normalised first: x * (1/sqrt(mean(x^2)+eps)) * norm_w
  float norm_eps;
  unsigned long long* best;     // nullptr, or kArgmaxSlots slots max-folded with argmax_key(y[r], r)
  // row-group launch over a stack of same-shape matrices: matrix b at W + b * w_stride reads
  // x + b * x_stride and writes y + b * y_stride (batch <= 1: one matrix)
  int batch;
  size_t w_stride;
  int x_stride, y_stride;
};

constexpr int kArgmaxSlots = 8;

// Fold one argmax_key per lane of a wave into best[kArgmaxSlots]: the wave's maximum goes to
// slot blockIdx.x % kArgmaxSlots (the workgroup's XCD under the 1-D grid mapping), and only when
// it beats the slot's current value (a relaxed read first: slots only grow, so a stale read can
// only let a needless atomic through). Spreading and filtering keep thousands of workgroups from
// serialising on one address.
__device__ __forceinline__ void wave_argmax_fold(unsigned long long key, unsigned long long* best) {
  unsigned hi = (unsigned)(key >> 32), lo = (unsigned)key;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned ohi = __shfl_xor(hi, off, 64), olo = __shfl_xor(lo, off, 64);
    if (ohi > hi || (ohi == hi && olo > lo)) { hi = ohi; lo = olo; }
  }
  const unsigned long long k = ((unsigned long long)hi << 32) | lo;
  unsigned long long* slot = best + (blockIdx.x % kArgmaxSlots);
  if ((threadIdx.x & 63) == 0 && k > __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
    atomicMax(slot, k);
}


// Order-preserving key of (value, index): the largest value wins and, among equal values, the
// largest index (the last maximum, as Iterator::max_by). -0 counts as +0; 0 is below every key.
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
  unsigned b = __float_as_uint(v == 0.0f ? 0.0f : v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned)i;
}

// LDS one workgroup may use on gfx950 (160 KiB per CU)
constexpr size_t kMaxLdsBytes = 160u * 1024u;

// longest row (elements) a GEMV workgroup stages in LDS: x, its per-16 sums and the wave
// partials stay under 64 KiB of dynamic LDS
constexpr int kGemvRowsMaxK = 12288;

// Effective shape of a GEMV launch. The tile kernel (64 rows per workgroup) runs 2, 4 or 8
// waves; super-block types stream half blocks once each wave has two or more blocks. The
// row-group kernels run 4, 8 or 16 waves.
inline int gemv_tile_waves(int waves) { return waves >= 8 ? 8 : waves <= 2 ? 2 : 4; }
inline bool gemv_tile_half(int qk, int kb, int tile_waves) { return qk == 256 && kb >= 2 * tile_waves; }
inline int gemv_rows_waves(int waves) { return waves == 16 ? 16 : waves == 8 ? 8 : 4; }

// waves per workgroup: 4, 8 or 16
hipError_t launch_gemv(uint32_t type, const GemvArgs& a, int waves, hipStream_t s);
hipError_t launch_dequant(uint32_t type, const uint8_t* W, float* out, int m, int n, int KB, int tiles,
                          hipStream_t s);
// Dense F32 / F16 / BF16 weights (dense.hip): row-major as stored, m x n elements
bool dense_type(uint32_t type);                  // ggml types 0, 1, 30
size_t dense_elem_bytes(uint32_t type);
// Y (rows x m) = X (rows x n) W^T (+ add[r] per output row when given). From kDenseMmaMinRows
// rows (n % 8 == 0, 16-byte aligned x) an MFMA GEMM: mode 1 (f32) f32 MFMA, else bf16 operands.
// best (one row only): the greedy argmax of y folded into the kArgmaxSlots slots. The MFMA GEMM may
// split K over `splits` slices (partial: splits x rows x m floats, no add), added in slice order.
constexpr int kDenseMmaMinRows = 16;
bool dense_mma_rows(int n, int rows, const float* x);     // the MFMA GEMM takes this call
int dense_mma_splits(int m, int n, int rows);             // its planned K slices
hipError_t launch_dense_gemm(uint32_t type, const void* W, const float* x, float* y, int m, int n, int rows,
                             const float* add, int mode, unsigned long long* best, float* partial, int splits,
                             hipStream_t s);
hipError_t launch_dense_to_f32(uint32_t type, const void* src, float* dst, size_t count, hipStream_t s);
// Int8 activations (i8.hip): Q8Activation::from_f32 of rows x n f32 (n % 32 == 0, x 16-byte
// aligned) into scales (rows x n/32) and qs (rows x n, 16-byte aligned); and the Q8_0 x i8 GEMM
// over tiled Q8_0 weights, y rows x m.
hipError_t launch_quantize_q8_act(const float* x, int rows, int n, float* scales, int8_t* qs, hipStream_t s);
hipError_t launch_q8_i8_gemm(const uint8_t* W, int tiles, const float* xs, const int8_t* xq, float* y, int m, int n,
                             int rows, hipStream_t s);
// GGUF row-major blocks -> tiled slabs (repack.hip): `mats` matrices of m rows x kb blocks,
// mat_src bytes apart at src (device) and dst_stride bytes apart at dst, `tiles` tiles each
hipError_t launch_repack(uint32_t type, const uint8_t* src, uint8_t* dst, int m, int kb, int tiles, int mats,
                         size_t mat_src, size_t dst_stride, hipStream_t s);

// GEMM: K steps of 128 elements.
constexpr int kGemmBK = 128;
constexpr int kMoeTile = 64;   // tile of the grouped (MoE) launches (64 x 64, four waves)

enum class GemmTile { k64x64, k128x128, k128x256, k256x128, k128x192 };

// Work item of a grouped launch (MoE): one tile of one expert.
struct GemmTask {
  int expert;     // weight matrix index (byte offset expert * w_stride)
  int mtile;      // weight-row tile
  int r0;         // first gathered row of the tile
  int rn;         // valid rows in the tile (<= tile)
};

struct GemmArgs {
  const uint8_t* W;        // tiled slabs (expert 0)
  uint32_t w_bytes;        // bytes readable from W (all experts); < 2 GiB
  size_t w_stride;         // bytes between experts
  const void* X;           // activations, row-major, K floats per row (K bf16 when x_bf16)
  uint32_t x_bytes;        // bytes readable from X; < 2 GiB
  int x_bf16;              // grouped bf16-mode launch: X already rounded to bf16
  const uint8_t* W2;       // grouped bf16 launch with bf16 X: up weights beside W (gate), same geometry;
                           // the tile writes silu(gate) * up as bf16 (ldy elements per row)
  float* Y;                // output, row stride ldy
  int m, K, KB, tiles;     // weight geometry (per expert)
  int N;                   // activation rows (dense launch)
  int ldy;
  int splits;              // dense: K steps divided over this many workgroups (>= 1)
  int steps_per_split;
  float* partial;          // splits > 1: splits * N * ldy floats, summed by a second kernel
  const GemmTask* tasks;   // grouped launch: one task per workgroup (nullptr = dense grid)
  const int* xrow;         // grouped: X row of gathered row p (nullptr = p itself)
  const int* ntasks;       // grouped: nullptr, or the task count on the device (larger grids exit early)
  // split bf16 operands (register-decoded expert GEMMs in f32 mode): X holds the bf16 rounding of
  // each activation (hi) and, x_lo bytes further, the bf16 rounding of what hi leaves (lo); a
  // gate/up pair writes h's hi to Y and its lo y_lo elements further
  uint32_t x_lo;
  size_t y_lo;
};

struct GemmPlan {
  GemmTile tile = GemmTile::k64x64;
  int kgroups = 1;         // K-groups per workgroup (1 or 2): waves that share a tile, split K
  int splits = 1;          // K split over workgroups (partials + reduce kernel)
  int steps_per_split = 1;
};

// tile, K-groups and K split of a dense m x n-row launch over K (mode 0 bf16, 1 f32)
// launch mode of the tiled GEMM beside RE_MODE_BF16 / RE_MODE_F32: f32 mode computed with bf16
// MFMAs on split operands (each operand's bf16 rounding and the bf16 rounding of its remainder;
// products hi*hi + hi*lo + lo*hi, each within 2^-16 relative)
constexpr int kGemmModeSplit = 2;
GemmPlan plan_gemm(int m, int n, int K, int mode);
// K-groups for `workgroups` tiles of `tile` over `steps` K steps
int gemm_kgroups(GemmTile tile, int mode, long workgroups, int steps);
hipError_t launch_gemm(uint32_t type, int mode, const GemmArgs& a, int ntasks, GemmTile tile, int kgroups,
                       hipStream_t s);
// Few-row dense GEMM (skinny.hip): Y[N x m] = X[N x K] W^T for N <= 64 rows of f32 X, a 64-row
// weight tile and a K slice of blocks_per_split whole blocks per workgroup; splits > 1 writes
// partial[split][N][ldy] for the split-K reduce (launch with launch_gemm_reduce).
struct SkinnyArgs {
  const uint8_t* W;        // tiled slabs
  uint32_t w_bytes;
  const float* X;          // N x K f32 rows
  uint32_t x_bytes;
  float* Y;                // splits == 1: N x ldy
  float* partial;          // splits > 1: splits x N x ldy
  int N, m, K, KB, tiles, ldy;
  int blocks_per_split, splits;
};
struct SkinnyPlan {
  int blocks_per_split = 1;
  int splits = 1;
};
constexpr int kSkinnyMaxK = 512;          // staged k per slice (LDS)
SkinnyPlan plan_skinny(int m, int K, int qk);
size_t skinny_lds_bytes(int staged_k, bool split_operands);
// split_operands: f32 mode (split bf16 operands, three MFMAs per product)
hipError_t launch_gemm_skinny(uint32_t type, const SkinnyArgs& a, bool split_operands, hipStream_t s);
// y = sum over splits, in split order, of partial[split] (n floats each), streaming stores
hipError_t launch_gemm_reduce(const float* partial, float* y, size_t n, int splits, hipStream_t s);

// xb[i] = bf16(x[i]), round to nearest even; n a multiple of 8, both buffers 16-byte aligned
hipError_t launch_x_to_bf16(const float* x, void* xb, size_t n, hipStream_t s);
// split form: xb[i] = hi = bf16(x[i]) and xb[n + i] = lo = bf16(x[i] - hi), both rounded to nearest
// even, so hi + lo holds x to 2^-16 relative
hipError_t launch_x_to_bf16_split(const float* x, void* xb, size_t n, hipStream_t s);

// Grouped expert GEMV (few gathered rows per expert): one task per workgroup
struct MoeGemvTask {
  int expert;   // expert index
  int row0;     // first weight row (multiple of kMoeGemvRows, inside one 64-row tile)
  int p0;       // first gathered row
  int np;       // gathered rows of the task (1..kMoeGemvBatch)
};
struct MoeGemvArgs {
  const uint8_t* W0;          // tiled slabs of expert 0 (gate, or down)
  const uint8_t* W1;          // up (dual launch) or nullptr
  size_t w_stride;            // bytes between experts
  const float* X;             // activation rows, K floats each
  const int* xrow;            // X row of gathered row p (nullptr = p itself)
  float* Y;                   // output row of gathered row p: Y + p * ldy
  const MoeGemvTask* tasks;   // nullptr: workgroup b takes rows b * rows_per_task.. of expert 0, activation row 0
  int m, K, KB, ldy;          // weight rows and row length (per expert)
  int max_rows;               // largest np over the tasks
  const float* norm_w;        // nullptr, or each X row is RMS-normalised first (as GemvArgs)
  float norm_eps;
  const int* ntasks;          // nullptr, or the task count on the device (larger grids exit early)
  int rows_per_task;          // kMoeGemvRows, or kFfnGemvRows (single-row dual launches only)
  // one activation row routed to k experts (tasks == nullptr, ids or id_inline): workgroup b takes
  // rows (b % id_tiles) * rows_per_task.. of expert ids[b / id_tiles] (id_v when id_inline) and
  // writes output row b / id_tiles; an id outside [0, n_experts) leaves its row unwritten (the
  // down + combine launch skips it)
  const int* ids;
  int id_tiles, n_experts, id_inline;
  int id_v[8];
};
// Down projection and combine of one token routed to k <= kMoeOneTokenMaxK experts, one launch:
// out[r] = sum over j (in order, skipping ids outside [0, n_experts)) of w[j] * (Wd[ids[j]] row r . h[j])
constexpr int kMoeOneTokenMaxK = 8;
static_assert(sizeof(MoeGemvArgs::id_v) / sizeof(int) == kMoeOneTokenMaxK, "inline ids of a one-token call");
struct MoeDownCombineArgs {
  const uint8_t* W;           // tiled slabs of the down stack (expert 0)
  size_t w_stride;            // bytes between experts
  const float* H;             // k rows of K floats (SwiGLU outputs)
  const int* ids;             // device ids and weights, or nullptr: id_v / w_v (host calls)
  const float* wts;
  float* out;                 // m floats
  int m, K, KB, k, n_experts;
  int id_v[kMoeOneTokenMaxK];
  float w_v[kMoeOneTokenMaxK];
};
hipError_t launch_moe_down_combine(uint32_t type, const MoeDownCombineArgs& a, hipStream_t s);
size_t moe_down_combine_lds(uint32_t type, int KB, int k);
// weight rows per expert task: with 16, staging the task's activation rows costs as many bytes
// as its weights; 64 leaves too few tasks
constexpr int kMoeGemvRows = 32;
// weight rows per down-projection GEMV task: 64 (its rows are short, K = inter), or
// REHIP_MOE_DROWS = 32 / 64
int moe_gemv_rows_down();
// weight rows per task of the one-row gate/up pair (re_ffn): more, smaller tasks suit decode
constexpr int kFfnGemvRows = 16;
constexpr int kMoeGemvWaves = 4;
constexpr int kMoeGemvBatch = 4;   // gathered rows per task
// dual: gate and up (W0, W1) with SwiGLU output; else one matrix
hipError_t launch_moe_gemv(uint32_t type, bool dual, const MoeGemvArgs& a, int ntasks, hipStream_t s);
// Grouped expert GEMM with register-decoded weights, bf16 mode (moe_qmma.hip): GemmTasks of up to
// max_rows <= 64 gathered rows, X bf16 rows (gathered through xrow when given). pair:
//   kQmmaOneTile   64-row weight tile mtile of W, Y receives f32;
//   kQmmaGateUp    the tile of W (gate) and W2 (up) of one geometry, Y receives h = silu(gate) * up
//                  as bf16;
//   kQmmaTwoTiles  128 rows (tiles 2 mtile, 2 mtile + 1) of W, Y receives f32.
// Uses W, W2, w_bytes, w_stride, X, x_bytes, xrow, Y, m, K, KB, ldy, tasks, ntasks of GemmArgs.
// split (f32 mode): every product is hi(x) hi(w) + hi(x) lo(w) + lo(x) hi(w), three bf16 MFMAs
// accumulated in f32 (each operand split as launch_x_to_bf16_split does; x_lo / y_lo locate
// the lo halves, and a gate/up pair writes h as hi and lo).
constexpr int kQmmaOneTile = 0, kQmmaGateUp = 1, kQmmaTwoTiles = 2;
hipError_t launch_moe_qmma(uint32_t type, int pair, int max_rows, const GemmArgs& a, int ntasks, hipStream_t s,
                           bool split = false);

// Dense transformer steps on device buffers (layer.hip)
hipError_t launch_rmsnorm(const float* x, const float* w, int rows, int d, float eps, float* out, hipStream_t s);
hipError_t launch_rope(float* x, int rows, int heads, int hd, float base, const int* pos, int off, hipStream_t s);
hipError_t launch_kv_append(const float* k, const float* v, int rows, int kv_dim, float* kc, float* vc,
                            int max_seq, const int* pos, hipStream_t s);
// work: nullptr, or attention_work_floats(...) floats for the key-split path of few rows
size_t attention_work_floats(int rows, int heads, int hd, int max_seq);
// One decode row: the q|k|v epilogue (bias, RoPE at *pos, k/v appended at row *pos) folded into
// the key-split attention; q/k/v are the raw projection outputs of the row
hipError_t launch_rope_table(float base, int hd, int rows, float* tab, hipStream_t s);
hipError_t launch_attention_decode(const float* q, const float* k, const float* v, const float* bq, const float* bk,
                                   const float* bv, int heads, int kv_heads, int hd, float base, const float* rope,
                                   const int* pos, float* kc, float* vc, int max_seq, float* work, float* ctx,
                                   hipStream_t s);
hipError_t launch_attention(const float* q, const float* kc, const float* vc, int rows, int heads, int kv_heads,
                            int hd, int max_seq, const int* pos, float* work, float* ctx, hipStream_t s);
// q/k/v projections (+ bias) -> rotated q (rows x heads*hd), rotated k and v appended at cache rows *pos + r
hipError_t launch_qkv_rope_append(const float* qs, int ldq, const float* ks, int ldk, const float* vs, int ldv,
                                  const float* bq, const float* bk, const float* bv, int rows, int heads,
                                  int kv_heads, int hd, float base, const int* pos, float* qout, float* kc,
                                  float* vc, int max_seq, hipStream_t s);
// *tok = index of *best; *pos += delta; hist[*pos] = *tok (hist may be null); *best = 0
hipError_t launch_decode_advance(unsigned long long* best, int* tok, int* pos, int delta, int* hist, int hist_len,
                                 hipStream_t s);
hipError_t launch_add(const float* a, const float* b, size_t n, size_t nb, float* out, hipStream_t s);
hipError_t launch_argmax(const float* x, int n, int* idx, hipStream_t s);
hipError_t launch_embed(const float* table, int n_vocab, int d, const int* tok, int rows, float* out, hipStream_t s);
hipError_t launch_pos_add(int* pos, int delta, hipStream_t s);

// MoE helpers
// Device-side routing (moe.rs:75-125): top-k experts per token, gate 0 = softmax over the chosen
// logits, 1 = per-expert sigmoid renormalised over the chosen
hipError_t launch_moe_route(const float* logits, int tokens, int n_experts, int k, int gate, int* ids,
                            float* weights, hipStream_t s);
// route_group (top2 = 0) / route_noaux_tc (top2 = 1) of moe.rs:126-268; top_k_group 0 = every group
hipError_t launch_moe_route_group(const float* logits, int tokens, int n_experts, int k, int top2, const float* bias,
                                  int bias_len, int n_groups, int top_k_group, int* ids, float* weights,
                                  hipStream_t s);
// logits[t][e] = router_w[e] . x[t] (f32)
hipError_t launch_moe_router_logits(const float* x, const float* router_w, int tokens, int hidden, int n_experts,
                                    float* logits, hipStream_t s);
// Device-side grouping of tokens * k (token, slot) pairs by expert (pair order kept inside an
// expert) and the task lists of the grouped launches. meta layout (ints): xrow[P] | pos[P] |
// ntasks[2] | pad | tasks_gu[max_gu] | tasks_d[max_d]; chunk = rows per task (kMoeGemvBatch or 1
// for the GEMV tasks, kMoeTile for GEMM tasks); rows_gu / rows_d = weight rows per task
// (kMoeGemvRows or kMoeTile); gemv selects MoeGemvTask or GemmTask records.
constexpr int kMoeMaxDevicePairs = 8192;
struct MoePlanShape {
  int pairs, k, n_experts, chunk, gemv;
  int tiles_gu, tiles_d;        // weight-row tasks per chunk (ceil(inter/rows), ceil(hidden/rows))
  int rows_gu, rows_d;          // weight rows per GEMV task (gate/up, down); GEMM tasks name a tile
  int max_gu, max_d;            // capacity of the task lists
};
size_t moe_meta_bytes(const MoePlanShape& sh);
// x / xb / n: also round the n floats of x to bf16 into xb (n % 8 == 0), or xb = nullptr;
// split: xb also receives the lo halves at xb + n (as launch_x_to_bf16_split)
hipError_t launch_moe_plan(const int* ids, const MoePlanShape& sh, void* meta, const float* x, void* xb, size_t n,
                           hipStream_t s, bool split = false);
hipError_t launch_swiglu(const float* g, const float* u, float* h, size_t n, hipStream_t s);
hipError_t launch_swiglu_bf16(const float* g, const float* u, void* h, size_t n, hipStream_t s);
hipError_t launch_combine(const float* yp, const int* pos, const float* w, float* out, int tokens,
                          int k, int hidden, hipStream_t s);

}  // namespace rehip
