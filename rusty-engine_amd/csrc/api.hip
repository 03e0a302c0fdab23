// C ABI of librehip (include/rehip.h): weight upload and repack, GEMV/GEMM dispatch, the
// bit-exact dequant and the grouped MoE expert FFN.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/rehip.h"
#include "common.hpp"
#include "kernels.hpp"

using namespace rehip;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

#define HIP_TRY(expr)                                                                      \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess) return fail(RE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

}  // namespace

namespace rehip {
// error reporting for the other translation units of the library (gguf.cpp)
int report_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}
}  // namespace rehip

namespace {

const char* type_name(uint32_t t) {
  switch (t) {
    case T_Q4_0: return "Q4_0";
    case T_Q5_0: return "Q5_0";
    case T_Q8_0: return "Q8_0";
    case T_Q4_K: return "Q4_K";
    case T_Q5_K: return "Q5_K";
    case T_Q6_K: return "Q6_K";
    case 0: return "F32";
    case 1: return "F16";
    case 30: return "BF16";
    default: return "?";
  }
}

int scratch_for_current_device(float** out, int* dev_out = nullptr);

std::once_flag g_init_once;
int g_init_rc = RE_OK;
char g_init_msg[512] = "";

int do_init() {
  std::call_once(g_init_once, [] {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
      g_init_rc = RE_ERR_NODEV;
      snprintf(g_init_msg, sizeof g_init_msg, "no HIP device (%s)", hipGetErrorString(e));
      return;
    }
    hipDeviceProp_t prop;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      g_init_rc = RE_ERR_NODEV;
      snprintf(g_init_msg, sizeof g_init_msg, "cannot query HIP device");
      return;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
      g_init_rc = RE_ERR_NODEV;
      snprintf(g_init_msg, sizeof g_init_msg, "device %d is %s, librehip is built for gfx950", dev,
               prop.gcnArchName);
      return;
    }
    float* p = nullptr;                  // the initial device's static scratch address
    if (scratch_for_current_device(&p) != RE_OK) {
      g_init_rc = RE_ERR_HIP;
      snprintf(g_init_msg, sizeof g_init_msg, "static scratch: %s", g_err);
    }
  });
  if (g_init_rc != RE_OK) return fail(g_init_rc, "%s", g_init_msg);
  return RE_OK;
}

// Geometry checks shared by every entry point taking GGUF rows.
int check_matrix(uint32_t type, size_t nbytes, size_t m, size_t n, MatGeom* g) {
  const TypeInfo* ti = type_info(type);
  if (!ti) return fail(RE_ERR_TYPE, "no fused kernel for ggml type %u", type);
  if (m == 0 || n == 0) return fail(RE_ERR_SIZE, "empty matrix %zu x %zu", m, n);
  if (n % 32 != 0) return fail(RE_ERR_SIZE, "n = %zu must be a multiple of 32", n);
  if (m > (1u << 30) || n > (1u << 24)) return fail(RE_ERR_SIZE, "matrix %zu x %zu too large", m, n);
  make_geom(type, m, n, g);
  const size_t want = m * g->kb * (size_t)g->bb;
  if (nbytes != want)
    return fail(RE_ERR_SIZE, "%s weight %zu x %zu needs %zu bytes, got %zu", type_name(type), m, n, want,
                nbytes);
  return RE_OK;
}

// Scratch of the no-allocation GEMM entry point: the K-split partial tiles live in this array
// (one copy per GPU, held until the process ends). Host code never passes `scratch` itself to a
// kernel: that name is a host-side stand-in; g_scratch_dev[dev] holds the device address that
// hipGetSymbolAddress returns for the device, taken once per device with that device current.
constexpr size_t kScratchBytes = 32u << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

struct Staging {
  void* p = nullptr;
  size_t cap = 0;
  int ensure(size_t bytes) {
    if (bytes <= cap) return RE_OK;
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    HIP_TRY(hipMalloc(&p, bytes));
    cap = bytes;
    return RE_OK;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
  }
};

// pinned host buffer (grown on demand) and the device's address of it
struct Pinned {
  void* h = nullptr;
  void* d = nullptr;
  size_t cap = 0;
  int ensure(size_t bytes) {
    if (bytes <= cap) return RE_OK;
    release();
    HIP_TRY(hipHostMalloc(&h, bytes, hipHostMallocDefault));
    HIP_TRY(hipHostGetDevicePointer(&d, h, 0));
    cap = bytes;
    return RE_OK;
  }
  void release() {
    if (h) (void)hipHostFree(h);
    h = d = nullptr;
    cap = 0;
  }
};

}  // namespace

struct re_qmat {
  MatGeom g{};                            // dense types: only type, m and n are set
  bool dense = false;                     // F32 / F16 / BF16 weights, row-major as stored (no tiles)
  uint8_t* d_w = nullptr;                 // count matrices, w_stride bytes apart
  size_t count = 1, w_stride = 0;
  float* d_partial = nullptr;
  float* d_norm = nullptr;                // dense weights: the RMS-normed x of matvec_ex (n floats)
  int splits = 1, kb_per_split = 1, waves = 4;
  int rows_per_group = 0, groups = 0;   // row-group GEMV launch (0 = split launch)
  std::mutex mu;
  hipStream_t stream = nullptr;
  Staging sx, sy, spart;
  Pinned hx, hy;                          // host-pointer calls: x staged for the copy, y written in place
};

struct re_moe {
  size_t n_experts = 0, hidden = 0, inter = 0;
  MatGeom gg{}, gu{}, gd{};
  uint8_t *d_gate = nullptr, *d_up = nullptr, *d_down = nullptr;
  std::mutex mu;
  hipStream_t stream = nullptr;
  Staging sx, sout, sg, su, sh, syp, smeta;
  Pinned hx, hout;                        // host-buffer calls: pinned staging of x and out
  Staging sxb;                            // bf16 copy of the activation rows (grouped GEMM path)
  Staging dmeta, droute;                  // device-routed path: plan + task lists; logits, ids, weights
  // pinned host staging of the per-call routing metadata, reused once its last upload is done
  void* hmeta = nullptr;
  size_t hmeta_cap = 0;
  hipEvent_t meta_ev = nullptr;
  bool meta_pending = false;
  // shared expert: a dense SwiGLU FFN of every token, added after the routed sum
  re_qmat *sh_gate = nullptr, *sh_up = nullptr, *sh_down = nullptr;
  size_t sh_inter = 0;
  Staging ssg, ssu, ssh, ssy;
};

namespace {

// integer tuning knob from the environment (dflt when unset or empty)
size_t env_size(const char* name, size_t dflt) {
  const char* v = std::getenv(name);
  return (v && *v) ? (size_t)std::strtoull(v, nullptr, 10) : dflt;
}

bool aligned16(const void* p);

}  // namespace

// weight rows per gate/up task of a one-token call (gate and up of one type): 16, twice the
// workgroups of 32 for the few experts one token hits (REHIP_MOE_GUROWS1 = 16 / 32)
static int moe_gemv_rows_gu1() {
  const size_t r = env_size("REHIP_MOE_GUROWS1", 0);
  return r == 16 || r == 32 ? (int)r : kFfnGemvRows;
}

int rehip::moe_gemv_rows_down() {
  const size_t r = env_size("REHIP_MOE_DROWS", 0);
  return r == 32 || r == 64 ? (int)r : 64;   // down (K = inter, short rows): 64 measured faster
}

namespace {

// bf16 mode of the grouped MoE GEMMs: the activation rows are rounded to bf16 once and SwiGLU
// writes h as bf16 -- the rounding each GEMM tile would apply while staging them -- so the
// tiles stage half the bytes and convert nothing (identical results). REHIP_MOE_XB=0 turns it off.
bool moe_bf16_acts(const re_moe* e, const float* d_x, int mode) {
  return mode == RE_MODE_BF16 && e->hidden % 8 == 0 && e->inter % 8 == 0 && aligned16(d_x) &&
         env_size("REHIP_MOE_XB", 1) != 0;
}

// bf16 mode with one gate/up type: the grouped expert GEMMs with register-decoded weights
// (moe_qmma.hip) serve every batch of more than one token; a one-token call keeps the expert GEMV
// (its few tasks want the GEMV's four waves per weight tile). REHIP_MOE_QMMA=0 turns it off.
bool moe_qmma_path(const re_moe* e, const float* d_x, size_t tokens, int mode) {
  return moe_bf16_acts(e, d_x, mode) && e->gg.type == e->gu.type && tokens > 1 &&
         env_size("REHIP_MOE_QMMA", 1) != 0;
}

// f32 mode with one gate/up type and more rows than the expert GEMV serves: the same register-
// decoded grouped GEMMs with split bf16 operands (three MFMAs per product, each operand held to
// 2^-16 relative, far inside the f32 bar of 2^-10 * sum|w x|): at 512 tokens on the
// Qwen3-30B-A3B shape they replace the LDS-staged f32 MFMA GEMMs. REHIP_MOE_SPLIT=0 turns it off.
bool moe_split_path(const re_moe* e, const float* d_x, size_t tokens, int mode, bool few) {
  return mode == RE_MODE_F32 && !few && tokens > 1 && e->gg.type == e->gu.type && e->hidden % 8 == 0 &&
         e->inter % 8 == 0 && aligned16(d_x) && env_size("REHIP_MOE_SPLIT", 1) != 0;
}

// Gathered rows per grouped-GEMM task: 32 (one token tile) while the experts get few rows each,
// else 64; REHIP_MOE_CHUNK = 32 / 64 overrides for the register-decoded GEMMs.
int moe_qmma_chunk(bool qmma, bool few) {
  if (!qmma) return kMoeTile;
  const size_t v = env_size("REHIP_MOE_CHUNK", 0);
  if (v == 32 || v == 64) return (int)v;
  return few ? 32 : kMoeTile;
}

// The grouped expert GEMV stages each task's activation rows (kMoeGemvBatch rows of K floats
// plus their per-16 sums) and the wave partials in LDS; when a projection's rows are too long for
// that, the grouped GEMM tasks (fixed LDS per tile) serve every batch size.
bool moe_gemv_fits(const re_moe* e) {
  auto lds = [](size_t kp) {
    return (kMoeGemvBatch * kp * 17 / 16 + (size_t)kMoeGemvWaves * 2 * kMoeGemvBatch * 64 +
            (size_t)kMoeGemvWaves * kMoeGemvBatch) * sizeof(float);
  };
  return lds(e->gg.kb * e->gg.qk) <= kMaxLdsBytes && lds(e->gu.kb * e->gu.qk) <= kMaxLdsBytes &&
         lds(e->gd.kb * e->gd.qk) <= kMaxLdsBytes;
}

// GEMV launch shape. Work units are 32-quant chunks (KB * chunks-per-block per row).
// Rows up to kGemvRowsMaxK long use the row-group kernel: the rows per workgroup are the largest
// of 64/16/8/4 that still give >= 512 workgroups (two per CU), and the waves per workgroup are
// the fewest of 4/8/16 that leave each lane-group slot one unit (up to 16 waves; 4 units for
// 64-row groups), so a slot's loads are all in flight at once and a latency-bound launch spends
// little time in any one wave (Q6_K down projection of the Qwen2.5-0.5B decode step: 16 waves
// instead of 8, 787 -> 780 us per token). Longer rows split the row over workgroups (partials
// + a reduce kernel). Measured on MI355X over the Qwen2.5-0.5B projections in all six types.
// Row-group shape for `tiles` 64-row tiles (of one matrix, or of a whole stack in one launch)
// whose rows have `units` 32-quant chunks.
void rows_shape(size_t tiles, size_t units, size_t nch, int* rows_per_group, int* waves) {
  int r = 64;
  for (int c : {64, 16, 8, 4}) {
    r = c;
    if (tiles * 64 / (size_t)c >= 512) break;
  }
  if (const size_t e = env_size("REHIP_GEMV_ROWS", 0); e == 64 || e == 16 || e == 8 || e == 4) r = (int)e;
  const size_t per_slot = r == 64 ? 4 : 1;
  const size_t slots = (units + per_slot - 1) / per_slot;
  const size_t per_wave = 64 / (size_t)r;
  const size_t w = (slots + per_wave - 1) / per_wave;
  *waves = w <= 4 ? 4 : w <= 8 ? 8 : 16;
  if (r == 64) {
    // tile kernel: waves take the tile's steps (a super-block, or four 32-blocks) in turn; two
    // waves for up to 4 steps, four for up to 12, else eight (measured on the batched Qwen2.5
    // projections: Q6_K 896x4864, 19 steps, 72.0 -> 74.7 % of HBM with eight)
    const size_t steps = nch == 8 ? units / 8 : (units + 3) / 4;
    *waves = steps <= 4 ? 2 : steps <= 12 ? 4 : 8;
  }
  if (const size_t e = env_size("REHIP_GEMV_WAVES", 0); e == 2 || e == 4 || e == 8 || e == 16) *waves = (int)e;
  *rows_per_group = r;
}

void plan_gemv(re_qmat* q) {
  const size_t kb = q->g.kb;
  const size_t nch = q->g.qk == 256 ? 8 : 1;
  const size_t units = kb * nch;
  q->rows_per_group = 0;
  q->groups = 0;
  if (q->g.n <= (size_t)kGemvRowsMaxK) {
    int r = 64;
    rows_shape(q->g.tiles, units, nch, &r, &q->waves);
    q->rows_per_group = r;
    q->groups = (int)(q->g.tiles * 64 / (size_t)r);
    q->splits = 1;
    q->kb_per_split = (int)kb;
    return;
  }
  const size_t cycles = units * 112;              // per-CU VALU cycles for one tile (4 SIMDs)
  size_t want = cycles > 6000 ? (cycles + 2399) / 2400 : 1;
  // a split stages its slice of x in LDS
  const size_t max_per = std::max<size_t>(1, (size_t)kGemvRowsMaxK / (size_t)q->g.qk);
  want = std::max<size_t>({(size_t)1, std::min(want, kb), (kb + max_per - 1) / max_per});
  want = std::min(want, std::max<size_t>(1, env_size("REHIP_GEMV_MAX_SPLITS", want)));
  const size_t per = (kb + want - 1) / want;
  q->kb_per_split = (int)per;
  q->splits = (int)((kb + per - 1) / per);
  const size_t per_wg = per * nch;
  q->waves = per_wg <= 16 ? 4 : per_wg <= 32 ? 8 : 16;
  if (const size_t w = env_size("REHIP_GEMV_WAVES", 0); w == 4 || w == 8 || w == 16) q->waves = (int)w;
}

// Uploads `count` matrices stored as GGUF row-major blocks (back to back in host memory, e.g. a
// mapped file) into the tiled layout at d_dst (dst_stride bytes apart). The bytes move as they
// are, in chunks of up to 32 MiB (whole matrices, or whole 64-row tiles of one large matrix),
// into one of two device staging buffers on a copy stream (the runtime's pageable-copy path: it
// measured at twice the rate of a host memcpy into pinned staging followed by a DMA); the repack
// kernel permutes each chunk on a second stream while the next chunk is copied into the other
// buffer. The staging buffers (2 x 32 MiB of device memory) and the two streams are made on a
// device's first upload and kept until the process ends; uploads serialize on them.
constexpr size_t kUploadChunk = 32u << 20;
constexpr int kMaxDevices = 64;

struct Uploader {
  hipStream_t cs = nullptr, ks = nullptr;            // copies, repack kernels
  hipEvent_t copied[2] = {nullptr, nullptr}, done[2] = {nullptr, nullptr};
  void* d[2] = {nullptr, nullptr};
  bool ready = false;
  int setup() {
    if (ready) return RE_OK;
    if (!cs) HIP_TRY(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
    if (!ks) HIP_TRY(hipStreamCreateWithFlags(&ks, hipStreamNonBlocking));
    for (int b = 0; b < 2; ++b) {
      if (!copied[b]) HIP_TRY(hipEventCreateWithFlags(&copied[b], hipEventDisableTiming));
      if (!done[b]) HIP_TRY(hipEventCreateWithFlags(&done[b], hipEventDisableTiming));
      if (!d[b]) HIP_TRY(hipMalloc(&d[b], kUploadChunk));
    }
    ready = true;
    return RE_OK;
  }
};
std::mutex g_up_mu;
Uploader g_up[kMaxDevices];

int upload_tiled(const MatGeom& g, const uint8_t* src, size_t count, uint8_t* d_dst, size_t dst_stride) {
  const size_t row_bytes = g.kb * (size_t)g.bb;
  const size_t mat_src = g.m * row_bytes;
  const size_t tile_src = row_bytes * kTileRows;
  if (tile_src > kUploadChunk)
    return fail(RE_ERR_SIZE, "64-row tile of %zu bytes exceeds the upload staging (%zu)", tile_src, kUploadChunk);
  // whole matrices per chunk when they fit, else whole tiles of one matrix
  const size_t mats_per_chunk = mat_src <= kUploadChunk ? std::min(count, kUploadChunk / mat_src) : 1;
  const size_t tiles_per_chunk = mat_src <= kUploadChunk ? g.tiles : kUploadChunk / tile_src;
  if (mats_per_chunk * g.tiles * g.kb > (size_t)INT32_MAX) return fail(RE_ERR_SIZE, "repack grid too large");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(RE_ERR_ARG, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_up_mu);
  Uploader& u = g_up[dev];
  int rc = u.setup();
  if (rc) return rc;
  auto drain = [&](hipError_t e) {
    (void)hipStreamSynchronize(u.cs);
    (void)hipStreamSynchronize(u.ks);
    return fail(RE_ERR_HIP, "upload: %s", hipGetErrorString(e));
  };
  size_t it = 0;
  for (size_t i0 = 0; i0 < count; i0 += mats_per_chunk) {
    const size_t nm = std::min(mats_per_chunk, count - i0);
    for (size_t t0 = 0; t0 < g.tiles; t0 += tiles_per_chunk, ++it) {
      const size_t nt = std::min(tiles_per_chunk, g.tiles - t0);
      const size_t row0 = t0 * kTileRows;
      const size_t rows = std::min(g.m - row0, nt * kTileRows);
      const size_t bytes = nm > 1 ? nm * mat_src : rows * row_bytes;
      const int b = (int)(it & 1);
      hipError_t e = hipSuccess;
      if (it >= 2) e = hipEventSynchronize(u.done[b]);   // the repack of chunk it - 2 has left d[b]
      if (e == hipSuccess)
        e = hipMemcpyAsync(u.d[b], src + i0 * mat_src + row0 * row_bytes, bytes, hipMemcpyHostToDevice, u.cs);
      if (e == hipSuccess) e = hipEventRecord(u.copied[b], u.cs);
      if (e == hipSuccess) e = hipStreamWaitEvent(u.ks, u.copied[b], 0);
      if (e == hipSuccess)
        e = launch_repack(g.type, (const uint8_t*)u.d[b], d_dst + i0 * dst_stride + t0 * g.kb * g.slab_bytes,
                          nm > 1 ? (int)g.m : (int)rows, (int)g.kb, (int)nt, (int)nm, mat_src, dst_stride, u.ks);
      if (e == hipSuccess) e = hipEventRecord(u.done[b], u.ks);
      if (e != hipSuccess) return drain(e);
    }
  }
  hipError_t e = hipStreamSynchronize(u.ks);
  if (e != hipSuccess) return drain(e);
  return RE_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int gemv_enqueue(re_qmat* q, const float* d_x, float* d_y, hipStream_t s, const float* d_add = nullptr,
                 const float* d_norm = nullptr, float eps = 0.0f, unsigned long long* d_best = nullptr) {
  if (!aligned16(d_x) || !aligned16(d_norm)) return fail(RE_ERR_ARG, "x and norm weights must be 16-byte aligned");
  GemvArgs a{};
  a.add = d_add;
  a.norm_w = d_norm;
  a.norm_eps = eps;
  a.best = d_best;
  a.W = q->d_w;
  a.x = d_x;
  a.y = d_y;
  a.partial = q->d_partial;
  a.m = (int)q->g.m;
  a.m_pad = (int)(q->g.tiles * kTileRows);
  a.K = (int)q->g.n;
  a.KB = (int)q->g.kb;
  a.tiles = (int)q->g.tiles;
  a.kb_per_split = q->kb_per_split;
  a.splits = q->splits;
  a.rows_per_group = q->rows_per_group;
  a.groups = q->groups;
  HIP_TRY(launch_gemv(q->g.type, a, q->waves, s));
  return RE_OK;
}

// fixed_partial: nullptr (the matrix's own partial buffer, grown on first use), or a caller-owned
// buffer of fixed_cap bytes for the split partials (the no-allocation entry point)
int gemm_enqueue(re_qmat* q, const float* d_x, size_t rows, float* d_y, int mode, hipStream_t s,
                 float* fixed_partial = nullptr, size_t fixed_cap = 0) {
  const size_t xbytes = rows * q->g.n * sizeof(float);
  if (xbytes >= (1ull << 31) || q->g.bytes >= (1ull << 31))
    return fail(RE_ERR_SIZE, "GEMM operands must stay below 2 GiB (X %zu B, W %zu B)", xbytes, q->g.bytes);
  // few rows: the few-row GEMM (weights decoded in registers, one workgroup per 64-row tile and
  // K slice, K slices for ~256 workgroups). It is faster than the tiled GEMM for 2..32 rows in bf16
  // mode (one 32-row token tile) and for 2..64 rows in f32 mode, where the tiled GEMM stages f32
  // tiles. REHIP_SKINNY=0 keeps the tiled GEMM for A/B runs.
  const size_t skinny_max = mode == RE_MODE_F32 ? 64 : 32;
  if (rows >= 2 && rows <= skinny_max && aligned16(d_x) && env_size("REHIP_SKINNY", 1) != 0 &&
      !env_size("REHIP_GEMM_TILE", 0)) {
    const SkinnyPlan sp = plan_skinny((int)q->g.m, (int)q->g.n, (int)q->g.qk);
    SkinnyArgs a{};
    a.W = q->d_w;
    a.w_bytes = (uint32_t)q->g.bytes;
    a.X = d_x;
    a.x_bytes = (uint32_t)xbytes;
    a.Y = d_y;
    a.N = (int)rows;
    a.m = (int)q->g.m;
    a.K = (int)q->g.n;
    a.KB = (int)q->g.kb;
    a.tiles = (int)q->g.tiles;
    a.ldy = (int)q->g.m;
    a.blocks_per_split = sp.blocks_per_split;
    a.splits = sp.splits;
    const size_t part_bytes = (size_t)a.splits * rows * q->g.m * sizeof(float);
    if (a.splits > 1) {
      if (fixed_partial) {
        if (part_bytes > fixed_cap)
          return fail(RE_ERR_SIZE, "GEMM %zu x %zu x %zu with %d K slices needs %zu bytes of split scratch; the "
                      "static scratch holds %zu", rows, q->g.m, q->g.n, a.splits, part_bytes, fixed_cap);
        a.partial = fixed_partial;
      } else if (part_bytes > q->spart.cap) {
        // grown on first use; under stream capture nothing may be allocated, so an un-warmed shape
        // runs as one K slice (same result up to summation order)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIP_TRY(hipStreamIsCapturing(s, &cs));
        if (cs != hipStreamCaptureStatusNone) {
          a.blocks_per_split = (int)q->g.kb;
          a.splits = 1;
        } else {
          int rc = q->spart.ensure(part_bytes);
          if (rc) return rc;
        }
      }
      if (!fixed_partial && a.splits > 1) a.partial = (float*)q->spart.p;
    }
    if (a.splits == 1 && (size_t)a.blocks_per_split * q->g.qk > (size_t)kSkinnyMaxK) {
      // one slice of more than the staging holds: the tiled GEMM below
    } else {
      HIP_TRY(launch_gemm_skinny(q->g.type, a, mode == RE_MODE_F32, s));
      if (a.splits > 1) HIP_TRY(launch_gemm_reduce(a.partial, d_y, rows * q->g.m, a.splits, s));
      return RE_OK;
    }
  }
  // f32 mode on bf16 MFMAs with split operands (REHIP_GEMM_SP=0: the f32 MFMA tiles)
  const int kmode = mode == RE_MODE_F32 && env_size("REHIP_GEMM_SP", 1) != 0 ? kGemmModeSplit : mode;
  GemmPlan pl = plan_gemm((int)q->g.m, (int)rows, (int)q->g.n, kmode);
  // tuning knobs: REHIP_GEMM_TILE (1 64x64, 2 128x128, 3 128x256, 4 256x128, 5 128x192), REHIP_GEMM_KG,
  // REHIP_GEMM_SPLITS; a combination the library does not build fails at launch
  if (const size_t t = env_size("REHIP_GEMM_TILE", 0); t >= 1 && t <= 5) {
    pl.tile = (GemmTile)(t - 1);
    pl.kgroups = (int)env_size("REHIP_GEMM_KG", 1);
    const int steps = (int)((q->g.n + kGemmBK - 1) / kGemmBK);
    const int sp = std::max(1, std::min(steps, (int)env_size("REHIP_GEMM_SPLITS", 1)));
    pl.steps_per_split = (steps + sp - 1) / sp;
    pl.splits = (steps + pl.steps_per_split - 1) / pl.steps_per_split;
  }
  const size_t part_bytes = (size_t)pl.splits * rows * q->g.m * sizeof(float);
  if (fixed_partial && pl.splits > 1 && part_bytes > fixed_cap)
    return fail(RE_ERR_SIZE, "GEMM %zu x %zu x %zu with %d K splits needs %zu bytes of split scratch; the static "
                "scratch holds %zu", rows, q->g.m, q->g.n, pl.splits, part_bytes, fixed_cap);
  if (!fixed_partial && pl.splits > 1 && part_bytes > q->spart.cap) {
    // the partial-sum buffer grows on first use; under stream capture nothing may be allocated,
    // so an un-warmed shape runs unsplit (same result up to summation order)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(s, &cs));
    if (cs != hipStreamCaptureStatusNone) {
      pl.splits = 1;
      pl.steps_per_split = (int)((q->g.n + kGemmBK - 1) / kGemmBK);
    }
  }
  GemmArgs a{};
  a.W = q->d_w;
  a.w_bytes = (uint32_t)q->g.bytes;
  a.w_stride = 0;
  a.X = d_x;
  a.x_bytes = (uint32_t)xbytes;
  a.Y = d_y;
  a.m = (int)q->g.m;
  a.K = (int)q->g.n;
  a.KB = (int)q->g.kb;
  a.tiles = (int)q->g.tiles;
  a.N = (int)rows;
  a.ldy = (int)q->g.m;
  a.splits = pl.splits;
  a.steps_per_split = pl.steps_per_split;
  a.tasks = nullptr;
  a.xrow = nullptr;
  if (pl.splits > 1) {
    if (fixed_partial) {
      a.partial = fixed_partial;
    } else {
      int rc = q->spart.ensure(part_bytes);
      if (rc) return rc;
      a.partial = (float*)q->spart.p;
    }
  }
  HIP_TRY(launch_gemm(q->g.type, kmode, a, 0, pl.tile, pl.kgroups, s));
  return RE_OK;
}

}  // namespace

extern "C" {

int re_init(void) {
  int rc = do_init();
  if (rc) return rc;
  float* p = nullptr;                    // the current device's static scratch address, taken once
  return scratch_for_current_device(&p);
}

const char* re_last_error(void) { return g_err; }

const char* re_version(void) { return "librehip 0.1 (gfx950)"; }

int re_row_bytes(uint32_t ggml_type, size_t n, size_t* out) {
  const TypeInfo* ti = type_info(ggml_type);
  if (!ti) return fail(RE_ERR_TYPE, "no fused kernel for ggml type %u", ggml_type);
  if (!out) return fail(RE_ERR_ARG, "null out");
  *out = (n + ti->qk - 1) / ti->qk * ti->bb;
  return RE_OK;
}

int re_tiled_bytes(uint32_t ggml_type, size_t m, size_t n, size_t* out) {
  MatGeom g;
  if (!type_info(ggml_type)) return fail(RE_ERR_TYPE, "no fused kernel for ggml type %u", ggml_type);
  if (!out || !make_geom(ggml_type, m, n, &g)) return fail(RE_ERR_ARG, "bad shape or null out");
  *out = g.bytes;
  return RE_OK;
}

int re_repack(uint32_t ggml_type, const uint8_t* bytes, size_t nbytes, size_t m, size_t n, uint8_t* out,
              size_t out_len) {
  MatGeom g;
  int rc = check_matrix(ggml_type, nbytes, m, n, &g);
  if (rc) return rc;
  if (!bytes || !out) return fail(RE_ERR_ARG, "null pointer");
  if (out_len != g.bytes) return fail(RE_ERR_SIZE, "tiled layout needs %zu bytes, got %zu", g.bytes, out_len);
  repack_host(g, bytes, out);
  return RE_OK;
}

// QMat::F32 and the float arms of the fallback (qmat.rs:128-151): the row-major elements as stored
int create_dense(uint32_t ggml_type, const uint8_t* bytes, size_t nbytes, size_t m, size_t n, re_qmat** out) {
  if (m == 0 || n == 0) return fail(RE_ERR_SIZE, "empty matrix %zu x %zu", m, n);
  if (m > (1u << 30) || n > (1u << 30)) return fail(RE_ERR_SIZE, "matrix %zu x %zu too large", m, n);
  const size_t want = m * n * dense_elem_bytes(ggml_type);
  if (nbytes != want)
    return fail(RE_ERR_SIZE, "%s weight %zu x %zu needs %zu bytes, got %zu", type_name(ggml_type), m, n, want, nbytes);
  int rc = do_init();
  if (rc) return rc;
  re_qmat* q = new (std::nothrow) re_qmat();
  if (!q) return fail(RE_ERR_ARG, "out of memory");
  q->dense = true;
  q->g.type = ggml_type;
  q->g.m = m;
  q->g.n = n;
  q->count = 1;
  if (hipMalloc(&q->d_w, nbytes) != hipSuccess || hipMalloc(&q->d_norm, n * sizeof(float)) != hipSuccess) {
    re_qmat_destroy(q);
    return fail(RE_ERR_HIP, "hipMalloc(%zu) failed", nbytes);
  }
  if (hipMemcpy(q->d_w, bytes, nbytes, hipMemcpyHostToDevice) != hipSuccess ||
      hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking) != hipSuccess) {
    re_qmat_destroy(q);
    return fail(RE_ERR_HIP, "dense weight upload failed");
  }
  *out = q;
  return RE_OK;
}

int re_qmat_create_stacked(uint32_t ggml_type, const uint8_t* bytes, size_t nbytes, size_t m, size_t n,
                           size_t count, re_qmat** out) {
  if (!out || !bytes) return fail(RE_ERR_ARG, "null pointer");
  *out = nullptr;
  if (dense_type(ggml_type)) {
    if (count != 1) return fail(RE_ERR_TYPE, "%s weights are not stacked", type_name(ggml_type));
    return create_dense(ggml_type, bytes, nbytes, m, n, out);
  }
  if (count == 0 || count > (1u << 20) || nbytes % count)
    return fail(RE_ERR_SIZE, "%zu bytes do not hold %zu equal matrices", nbytes, count);
  MatGeom g;
  int rc = check_matrix(ggml_type, nbytes / count, m, n, &g);
  if (rc) return rc;
  if ((rc = do_init())) return rc;
  re_qmat* q = new (std::nothrow) re_qmat();
  if (!q) return fail(RE_ERR_ARG, "out of memory");
  q->g = g;
  q->count = count;
  q->w_stride = (g.bytes + 255) / 256 * 256;
  plan_gemv(q);
  auto cleanup = [&](int code) {
    re_qmat_destroy(q);
    return code;
  };
  const size_t total = q->w_stride * count;
  if (hipMalloc(&q->d_w, total) != hipSuccess) return cleanup(fail(RE_ERR_HIP, "hipMalloc(%zu) failed", total));
  if ((rc = upload_tiled(g, bytes, count, q->d_w, q->w_stride))) return cleanup(rc);
  const size_t m_pad = g.tiles * kTileRows;
  if (q->splits > 1) {
    if (hipMalloc(&q->d_partial, (size_t)q->splits * m_pad * sizeof(float)) != hipSuccess)
      return cleanup(fail(RE_ERR_HIP, "hipMalloc of split scratch failed"));
  }
  if (hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking) != hipSuccess)
    return cleanup(fail(RE_ERR_HIP, "hipStreamCreate failed"));
  *out = q;
  return RE_OK;
}

int re_qmat_create(uint32_t ggml_type, const uint8_t* bytes, size_t nbytes, size_t m, size_t n,
                   re_qmat** out) {
  return re_qmat_create_stacked(ggml_type, bytes, nbytes, m, n, 1, out);
}

void re_qmat_destroy(re_qmat* q) {
  if (!q) return;
  if (q->stream) (void)hipStreamSynchronize(q->stream);
  if (q->d_w) (void)hipFree(q->d_w);
  if (q->d_partial) (void)hipFree(q->d_partial);
  if (q->d_norm) (void)hipFree(q->d_norm);
  q->sx.release();
  q->sy.release();
  q->spart.release();
  q->hx.release();
  q->hy.release();
  if (q->stream) (void)hipStreamDestroy(q->stream);
  delete q;
}

size_t re_qmat_rows(const re_qmat* q) { return q ? q->g.m : 0; }
size_t re_qmat_cols(const re_qmat* q) { return q ? q->g.n : 0; }
uint32_t re_qmat_type(const re_qmat* q) { return q ? q->g.type : 0; }

int re_qmat_matvec_dev(re_qmat* q, const float* d_x, float* d_y, void* stream) {
  if (!q || !d_x || !d_y) return fail(RE_ERR_ARG, "null pointer");
  if (q->dense) {
    HIP_TRY(launch_dense_gemm(q->g.type, q->d_w, d_x, d_y, (int)q->g.m, (int)q->g.n, 1, nullptr, RE_MODE_F32,
                              nullptr, nullptr, 1, (hipStream_t)stream));
    return RE_OK;
  }
  return gemv_enqueue(q, d_x, d_y, (hipStream_t)stream);
}

size_t re_qmat_count(const re_qmat* q) { return q ? q->count : 0; }

int re_qmat_matvec_stacked_dev(re_qmat* q, size_t first, size_t count, const float* d_x, size_t x_stride,
                               float* d_y, size_t y_stride, void* stream) {
  if (!q || !d_x || !d_y) return fail(RE_ERR_ARG, "null pointer");
  if (count == 0) return RE_OK;
  if (q->dense) return fail(RE_ERR_TYPE, "%s weights are not stacked", type_name(q->g.type));
  if (first >= q->count || count > q->count - first)
    return fail(RE_ERR_SIZE, "matrices %zu..%zu of a stack of %zu", first, first + count - 1, q->count);
  if (x_stride % 4 || x_stride > (1u << 30) || y_stride > (1u << 30) || (x_stride && x_stride < q->g.n) ||
      y_stride < q->g.m)
    return fail(RE_ERR_SIZE, "stacked strides x %zu (0 or >= %zu, multiple of 4), y %zu (>= %zu)", x_stride, q->g.n,
                y_stride, q->g.m);
  if (!aligned16(d_x)) return fail(RE_ERR_ARG, "x must be 16-byte aligned");
  const hipStream_t s = (hipStream_t)stream;
  if (!q->rows_per_group) {                // split launches: one matrix at a time
    for (size_t b = 0; b < count; ++b) {
      GemvArgs a{};
      a.W = q->d_w + (first + b) * q->w_stride;
      a.x = d_x + b * x_stride;
      a.y = d_y + b * y_stride;
      a.partial = q->d_partial;
      a.m = (int)q->g.m;
      a.m_pad = (int)(q->g.tiles * kTileRows);
      a.K = (int)q->g.n;
      a.KB = (int)q->g.kb;
      a.tiles = (int)q->g.tiles;
      a.kb_per_split = q->kb_per_split;
      a.splits = q->splits;
      HIP_TRY(launch_gemv(q->g.type, a, q->waves, s));
    }
    return RE_OK;
  }
  // the launch shape is planned for the whole stack (many matrices: bigger row groups)
  int rpg = 64, waves = 4;
  rows_shape(q->g.tiles * count, q->g.kb * (q->g.qk == 256 ? 8 : 1), q->g.qk == 256 ? 8 : 1, &rpg, &waves);
  const size_t groups = q->g.tiles * 64 / (size_t)rpg;
  if (groups * count > (size_t)INT32_MAX) return fail(RE_ERR_SIZE, "stack too large for one launch");
  GemvArgs a{};
  a.W = q->d_w + first * q->w_stride;
  a.x = d_x;
  a.y = d_y;
  a.m = (int)q->g.m;
  a.m_pad = (int)(q->g.tiles * kTileRows);
  a.K = (int)q->g.n;
  a.KB = (int)q->g.kb;
  a.tiles = (int)q->g.tiles;
  a.kb_per_split = q->kb_per_split;
  a.splits = 1;
  a.rows_per_group = rpg;
  a.groups = (int)groups;
  a.batch = (int)count;
  a.w_stride = q->w_stride;
  a.x_stride = (int)x_stride;
  a.y_stride = (int)y_stride;
  HIP_TRY(launch_gemv(q->g.type, a, waves, s));
  return RE_OK;
}

int re_qmat_gemv_plan(const re_qmat* q, size_t count, int* kernel, int* rows_per_group, int* waves, int* half) {
  if (!q || !kernel || !rows_per_group || !waves || !half) return fail(RE_ERR_ARG, "null pointer");
  if (count == 0 || count > q->count) return fail(RE_ERR_SIZE, "%zu matrices of a stack of %zu", count, q->count);
  *half = 0;
  if (q->dense) {
    *kernel = RE_GEMV_DENSE;
    *rows_per_group = 1;
    *waves = 1;
    return RE_OK;
  }
  if (!q->rows_per_group) {
    *kernel = RE_GEMV_SPLIT;
    *rows_per_group = 64;
    *waves = gemv_rows_waves(q->waves);
    return RE_OK;
  }
  int r = q->rows_per_group, w = q->waves;
  if (count > 1) rows_shape(q->g.tiles * count, q->g.kb * (q->g.qk == 256 ? 8 : 1), q->g.qk == 256 ? 8 : 1, &r, &w);
  *rows_per_group = r;
  if (r == 64) {
    *kernel = RE_GEMV_TILE;
    *waves = gemv_tile_waves(w);
    *half = gemv_tile_half(q->g.qk, (int)q->g.kb, *waves) ? 1 : 0;
  } else {
    *kernel = RE_GEMV_ROWS;
    *waves = gemv_rows_waves(w);
  }
  return RE_OK;
}

int re_qmat_matvec_ex_dev(re_qmat* q, const float* d_x, const float* d_norm_w, float eps, const float* d_add,
                          float* d_y, unsigned long long* d_best, void* stream) {
  if (!q || !d_x || !d_y) return fail(RE_ERR_ARG, "null pointer");
  if (d_norm_w && !(eps >= 0.0f)) return fail(RE_ERR_ARG, "norm eps must be >= 0");
  if (q->dense) {                        // RMS-norm into the matrix's own buffer, then the plain product
    const hipStream_t s = (hipStream_t)stream;
    const float* xin = d_x;
    if (d_norm_w) {
      HIP_TRY(launch_rmsnorm(d_x, d_norm_w, 1, (int)q->g.n, eps, q->d_norm, s));
      xin = q->d_norm;
    }
    HIP_TRY(launch_dense_gemm(q->g.type, q->d_w, xin, d_y, (int)q->g.m, (int)q->g.n, 1, d_add, RE_MODE_F32, d_best,
                              nullptr, 1, s));
    return RE_OK;
  }
  return gemv_enqueue(q, d_x, d_y, (hipStream_t)stream, d_add, d_norm_w, eps, d_best);
}

int re_qmat_matmul_dev(re_qmat* q, const float* d_x, size_t rows, float* d_y, int mode, void* stream) {
  if (!q || (rows && (!d_x || !d_y))) return fail(RE_ERR_ARG, "null pointer");
  if (mode != RE_MODE_BF16 && mode != RE_MODE_F32) return fail(RE_ERR_ARG, "unknown mode %d", mode);
  if (rows == 0) return RE_OK;
  if (rows > (1u << 24)) return fail(RE_ERR_SIZE, "rows = %zu too large", rows);
  if (q->dense) {                        // below 16 rows f32 products in either mode (the reference's
    // f32 matvec); from 16 rows the MFMA GEMM, bf16 operands in bf16 mode and split operands on
    // bf16 MFMAs in f32 mode (REHIP_GEMM_SP=0: f32 MFMAs)
    if (rows > 65535u * 4u) return fail(RE_ERR_SIZE, "rows = %zu too large for dense weights", rows);
    const hipStream_t s = (hipStream_t)stream;
    int splits = 1;
    if (dense_mma_rows((int)q->g.n, (int)rows, d_x)) {
      // few output tiles: K slices into the matrix's partial buffer, grown on first use (under
      // stream capture an unwarmed shape runs as one slice: the same result up to summation order)
      splits = dense_mma_splits((int)q->g.m, (int)q->g.n, (int)rows);
      const size_t need = (size_t)splits * rows * q->g.m * sizeof(float);
      if (splits > 1 && need > q->spart.cap) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIP_TRY(hipStreamIsCapturing(s, &cs));
        if (cs != hipStreamCaptureStatusNone || need > (32u << 20)) splits = 1;
        else if (int rc = q->spart.ensure(need)) return rc;
      }
    }
    const int kmode = mode == RE_MODE_F32 && env_size("REHIP_GEMM_SP", 1) != 0 ? kGemmModeSplit : mode;
    HIP_TRY(launch_dense_gemm(q->g.type, q->d_w, d_x, d_y, (int)q->g.m, (int)q->g.n, (int)rows, nullptr, kmode,
                              nullptr, splits > 1 ? (float*)q->spart.p : nullptr, splits, s));
    return RE_OK;
  }
  if (rows == 1) return gemv_enqueue(q, d_x, d_y, (hipStream_t)stream);
  return gemm_enqueue(q, d_x, rows, d_y, mode, (hipStream_t)stream);
}

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_dev[kScratchDevices] = {};
// per device: an event recorded after the last no-allocation call's launches, and that call's
// stream (a call on another stream waits on the event first)
hipEvent_t g_scratch_ev[kScratchDevices] = {};
hipStream_t g_scratch_last[kScratchDevices] = {};
bool g_scratch_used[kScratchDevices] = {};

// the calling thread's current device's copy of `scratch` and its ordering event, both set up
// once per device (re_init, or the first call on the device)
int scratch_for_current_device(float** out, int* dev_out) {
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kScratchDevices) return fail(RE_ERR_ARG, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(RE_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    HIP_TRY(hipEventCreateWithFlags(&g_scratch_ev[dev], hipEventDisableTiming));
    g_scratch_dev[dev] = (float*)p;
  }
  *out = g_scratch_dev[dev];
  if (dev_out) *dev_out = dev;
  return RE_OK;
}
}  // namespace

int re_qmat_matmul_noalloc_dev(re_qmat* q, const float* d_x, size_t rows, float* d_y, int mode, void* stream) {
  if (!q || (rows && (!d_x || !d_y))) return fail(RE_ERR_ARG, "null pointer");
  if (mode != RE_MODE_BF16 && mode != RE_MODE_F32) return fail(RE_ERR_ARG, "unknown mode %d", mode);
  if (rows == 0) return RE_OK;
  if (rows == 1 || q->dense) return re_qmat_matmul_dev(q, d_x, rows, d_y, mode, stream);   // no scratch
  if (rows > (1u << 24)) return fail(RE_ERR_SIZE, "rows = %zu too large", rows);
  float* part = nullptr;
  int dev = 0;
  int rc = scratch_for_current_device(&part, &dev);
  if (rc) return rc;
  const hipStream_t s = (hipStream_t)stream;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(s, &cs));
  // under capture the caller orders the replays of graphs that share the scratch
  if (cs != hipStreamCaptureStatusNone) return gemm_enqueue(q, d_x, rows, d_y, mode, s, part, kScratchBytes);
  // outside capture, calls on different streams of one GPU are ordered through the device's event
  // (the lock also orders calls from different threads); calls on one stream are ordered by it
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_used[dev] && g_scratch_last[dev] != s) HIP_TRY(hipStreamWaitEvent(s, g_scratch_ev[dev], 0));
  if ((rc = gemm_enqueue(q, d_x, rows, d_y, mode, s, part, kScratchBytes))) return rc;
  HIP_TRY(hipEventRecord(g_scratch_ev[dev], s));
  g_scratch_last[dev] = s;
  g_scratch_used[dev] = true;
  return RE_OK;
}

int re_qmat_matvec(re_qmat* q, const float* x, float* y) {
  if (!q || !x || !y) return fail(RE_ERR_ARG, "null pointer");
  return re_qmat_matmul(q, x, 1, y, RE_MODE_F32);
}

int re_qmat_matmul(re_qmat* q, const float* x, size_t rows, float* y, int mode) {
  if (!q || (rows && (!x || !y))) return fail(RE_ERR_ARG, "null pointer");
  if (mode != RE_MODE_BF16 && mode != RE_MODE_F32) return fail(RE_ERR_ARG, "unknown mode %d", mode);
  if (rows == 0) return RE_OK;
  std::lock_guard<std::mutex> lk(q->mu);
  const size_t xb = rows * q->g.n * sizeof(float), yb = rows * q->g.m * sizeof(float);
  int rc;
  // x goes through pinned staging (a DMA copy, no pageable bounce); the kernels write y straight
  // into pinned host memory, read back after the stream synchronizes. REHIP_HOST_IO = 0: pageable
  // copies both ways, 1: pinned copies both ways.
  const size_t io = env_size("REHIP_HOST_IO", 2);
  if ((rc = q->sx.ensure(xb))) return rc;
  if (io == 0) {
    if ((rc = q->sy.ensure(yb))) return rc;
    HIP_TRY(hipMemcpyAsync(q->sx.p, x, xb, hipMemcpyHostToDevice, q->stream));
    if ((rc = re_qmat_matmul_dev(q, (const float*)q->sx.p, rows, (float*)q->sy.p, mode, q->stream))) return rc;
    HIP_TRY(hipMemcpyAsync(y, q->sy.p, yb, hipMemcpyDeviceToHost, q->stream));
    HIP_TRY(hipStreamSynchronize(q->stream));
    return RE_OK;
  }
  if ((rc = q->hx.ensure(xb)) || (rc = q->hy.ensure(yb))) return rc;
  if (io == 1 && (rc = q->sy.ensure(yb))) return rc;
  std::memcpy(q->hx.h, x, xb);
  HIP_TRY(hipMemcpyAsync(q->sx.p, q->hx.h, xb, hipMemcpyHostToDevice, q->stream));
  float* dy = io == 1 ? (float*)q->sy.p : (float*)q->hy.d;
  if ((rc = re_qmat_matmul_dev(q, (const float*)q->sx.p, rows, dy, mode, q->stream))) return rc;
  if (io == 1) HIP_TRY(hipMemcpyAsync(q->hy.h, q->sy.p, yb, hipMemcpyDeviceToHost, q->stream));
  HIP_TRY(hipStreamSynchronize(q->stream));
  std::memcpy(y, q->hy.h, yb);
  return RE_OK;
}

// ---- int8 activations (kernel.rs:70-166) -------------------------------------------------
int re_quantize_q8_act_dev(const float* d_x, size_t rows, size_t n, float* d_scales, int8_t* d_qs, void* stream) {
  if (rows == 0) return RE_OK;
  if (!d_x || !d_scales || !d_qs) return fail(RE_ERR_ARG, "null pointer");
  if (n == 0 || n % 32) return fail(RE_ERR_SIZE, "Q8Activation::from_f32: length %zu not a multiple of 32", n);
  if (rows > (1u << 24) || n > (1u << 24) || rows * (n / 32) > (size_t)INT32_MAX * 256)
    return fail(RE_ERR_SIZE, "activation %zu x %zu too large", rows, n);
  if (!aligned16(d_x) || !aligned16(d_qs)) return fail(RE_ERR_ARG, "x and qs must be 16-byte aligned");
  HIP_TRY(launch_quantize_q8_act(d_x, (int)rows, (int)n, d_scales, d_qs, (hipStream_t)stream));
  return RE_OK;
}

int re_quantize_q8_act(const float* x, size_t rows, size_t n, float* scales, int8_t* qs) {
  if (rows == 0) return RE_OK;
  if (!x || !scales || !qs) return fail(RE_ERR_ARG, "null pointer");
  if (n == 0 || n % 32) return fail(RE_ERR_SIZE, "Q8Activation::from_f32: length %zu not a multiple of 32", n);
  int rc = do_init();
  if (rc) return rc;
  const size_t xb = rows * n * sizeof(float), sb = rows * (n / 32) * sizeof(float), qb = rows * n;
  void* d = nullptr;
  HIP_TRY(hipMalloc(&d, xb + sb + qb + 512));
  uint8_t* base = (uint8_t*)d;
  float* dx = (float*)base;
  float* ds = (float*)(base + (xb + 255) / 256 * 256);
  int8_t* dq = (int8_t*)(base + (xb + 255) / 256 * 256 + (sb + 255) / 256 * 256);
  hipError_t e = hipMemcpy(dx, x, xb, hipMemcpyHostToDevice);
  if (e == hipSuccess) rc = re_quantize_q8_act_dev(dx, rows, n, ds, dq, nullptr);
  if (e == hipSuccess && !rc) e = hipMemcpy(scales, ds, sb, hipMemcpyDeviceToHost);
  if (e == hipSuccess && !rc) e = hipMemcpy(qs, dq, qb, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(RE_ERR_HIP, "quantize copy: %s", hipGetErrorString(e));
  return rc;
}

int re_qmat_matmul_i8_dev(re_qmat* q, const float* d_scales, const int8_t* d_qs, size_t rows, float* d_y,
                          void* stream) {
  if (!q) return fail(RE_ERR_ARG, "null pointer");
  if (q->g.type != T_Q8_0)
    return fail(RE_ERR_TYPE, "the int8 activation path needs Q8_0 weights, this matrix is %s", type_name(q->g.type));
  if (q->count != 1) return fail(RE_ERR_ARG, "stacked matrix: use one matrix per call");
  if (rows == 0) return RE_OK;
  if (!d_scales || !d_qs || !d_y) return fail(RE_ERR_ARG, "null pointer");
  if (rows > 65535u * 32u) return fail(RE_ERR_SIZE, "%zu activation rows (at most %u)", rows, 65535u * 32u);
  if (!aligned16(d_qs)) return fail(RE_ERR_ARG, "qs must be 16-byte aligned");
  HIP_TRY(launch_q8_i8_gemm(q->d_w, (int)q->g.tiles, d_scales, d_qs, d_y, (int)q->g.m, (int)q->g.n, (int)rows,
                            (hipStream_t)stream));
  return RE_OK;
}

int re_qmat_matmul_i8(re_qmat* q, const float* scales, const int8_t* qs, size_t rows, float* y) {
  if (!q || (rows && (!scales || !qs || !y))) return fail(RE_ERR_ARG, "null pointer");
  if (q->g.type != T_Q8_0)
    return fail(RE_ERR_TYPE, "the int8 activation path needs Q8_0 weights, this matrix is %s", type_name(q->g.type));
  if (rows == 0) return RE_OK;
  std::lock_guard<std::mutex> lk(q->mu);
  const size_t qb = rows * q->g.n, sb = rows * (q->g.n / 32) * sizeof(float), yb = rows * q->g.m * sizeof(float);
  const size_t qoff = (sb + 255) / 256 * 256;
  int rc;
  if ((rc = q->sx.ensure(qoff + qb)) || (rc = q->sy.ensure(yb))) return rc;
  uint8_t* base = (uint8_t*)q->sx.p;
  HIP_TRY(hipMemcpyAsync(base, scales, sb, hipMemcpyHostToDevice, q->stream));
  HIP_TRY(hipMemcpyAsync(base + qoff, qs, qb, hipMemcpyHostToDevice, q->stream));
  if ((rc = re_qmat_matmul_i8_dev(q, (const float*)base, (const int8_t*)(base + qoff), rows, (float*)q->sy.p,
                                  q->stream)))
    return rc;
  HIP_TRY(hipMemcpyAsync(y, q->sy.p, yb, hipMemcpyDeviceToHost, q->stream));
  HIP_TRY(hipStreamSynchronize(q->stream));
  return RE_OK;
}

int re_qmat_dequant_dev(re_qmat* q, float* d_out, void* stream) {
  if (!q || !d_out) return fail(RE_ERR_ARG, "null pointer");
  if (q->dense) {
    HIP_TRY(launch_dense_to_f32(q->g.type, q->d_w, d_out, q->g.m * q->g.n, (hipStream_t)stream));
    return RE_OK;
  }
  HIP_TRY(launch_dequant(q->g.type, q->d_w, d_out, (int)q->g.m, (int)q->g.n, (int)q->g.kb, (int)q->g.tiles,
                         (hipStream_t)stream));
  return RE_OK;
}

int re_dequant(uint32_t ggml_type, const uint8_t* bytes, size_t nbytes, float* out, size_t out_len) {
  if (dense_type(ggml_type)) {            // F32 / F16 / BF16 widen element by element (quant.rs:365-392)
    const size_t es = dense_elem_bytes(ggml_type);
    if (nbytes % es)
      return fail(RE_ERR_SIZE, "%s data len %zu not a multiple of %zu", type_name(ggml_type), nbytes, es);
    const size_t count = nbytes / es;
    if (out_len != count) return fail(RE_ERR_SIZE, "out needs %zu floats, got %zu", count, out_len);
    if (count == 0) return RE_OK;
    if (!bytes || !out) return fail(RE_ERR_ARG, "null pointer");
    int rc = do_init();
    if (rc) return rc;
    void* d = nullptr;
    const size_t src_off = (count * sizeof(float) + 255) / 256 * 256;
    HIP_TRY(hipMalloc(&d, src_off + nbytes));
    hipError_t e = hipMemcpy((uint8_t*)d + src_off, bytes, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_dense_to_f32(ggml_type, (uint8_t*)d + src_off, (float*)d, count, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, d, count * sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return fail(RE_ERR_HIP, "dequant: %s", hipGetErrorString(e));
    return RE_OK;
  }
  const TypeInfo* ti = type_info(ggml_type);
  if (!ti) return fail(RE_ERR_TYPE, "no scalar dequant for ggml type %u", ggml_type);
  if (nbytes % ti->bb)
    return fail(RE_ERR_SIZE, "%s data len %zu not a multiple of %d", type_name(ggml_type), nbytes, ti->bb);
  const size_t blocks = nbytes / ti->bb;
  if (out_len != blocks * ti->qk) return fail(RE_ERR_SIZE, "out needs %zu floats, got %zu", blocks * ti->qk, out_len);
  if (blocks == 0) return RE_OK;
  if (!bytes || !out) return fail(RE_ERR_ARG, "null pointer");
  // a flat stream is a (blocks x QK) matrix with one block per row
  re_qmat* q = nullptr;
  int rc = re_qmat_create(ggml_type, bytes, nbytes, blocks, ti->qk, &q);
  if (rc) return rc;
  float* d_out = nullptr;
  if (hipMalloc(&d_out, blocks * ti->qk * sizeof(float)) != hipSuccess) {
    re_qmat_destroy(q);
    return fail(RE_ERR_HIP, "hipMalloc failed");
  }
  rc = re_qmat_dequant_dev(q, d_out, q->stream);
  if (!rc && hipMemcpyAsync(out, d_out, blocks * ti->qk * sizeof(float), hipMemcpyDeviceToHost, q->stream) != hipSuccess)
    rc = fail(RE_ERR_HIP, "copy back failed");
  if (!rc && hipStreamSynchronize(q->stream) != hipSuccess) rc = fail(RE_ERR_HIP, "sync failed");
  (void)hipFree(d_out);
  re_qmat_destroy(q);
  return rc;
}

// ---- MoE ---------------------------------------------------------------------------------
int re_moe_create(uint32_t gate_type, const uint8_t* gate, size_t gate_bytes, uint32_t up_type, const uint8_t* up,
                  size_t up_bytes, uint32_t down_type, const uint8_t* down, size_t down_bytes, size_t n_experts,
                  size_t hidden, size_t inter, re_moe** out) {
  if (!out || !gate || !up || !down) return fail(RE_ERR_ARG, "null pointer");
  *out = nullptr;
  if (n_experts == 0 || n_experts > 65536) return fail(RE_ERR_SIZE, "n_experts = %zu", n_experts);
  MatGeom gg, gu, gd;
  int rc;
  if (gate_bytes % n_experts || up_bytes % n_experts || down_bytes % n_experts)
    return fail(RE_ERR_SIZE, "expert tensors must hold n_experts equal slices");
  if ((rc = check_matrix(gate_type, gate_bytes / n_experts, inter, hidden, &gg))) return rc;
  if ((rc = check_matrix(up_type, up_bytes / n_experts, inter, hidden, &gu))) return rc;
  if ((rc = check_matrix(down_type, down_bytes / n_experts, hidden, inter, &gd))) return rc;
  if ((rc = do_init())) return rc;
  re_moe* e = new (std::nothrow) re_moe();
  if (!e) return fail(RE_ERR_ARG, "out of memory");
  e->n_experts = n_experts;
  e->hidden = hidden;
  e->inter = inter;
  e->gg = gg;
  e->gu = gu;
  e->gd = gd;
  auto cleanup = [&](int code) {
    re_moe_destroy(e);
    return code;
  };
  struct P { const MatGeom* g; const uint8_t* src; size_t slice; uint8_t** dst; };
  P parts[3] = {{&gg, gate, gate_bytes / n_experts, &e->d_gate}, {&gu, up, up_bytes / n_experts, &e->d_up},
                {&gd, down, down_bytes / n_experts, &e->d_down}};
  for (auto& pt : parts) {
    if (hipMalloc(pt.dst, pt.g->bytes * n_experts) != hipSuccess)
      return cleanup(fail(RE_ERR_HIP, "hipMalloc(%zu) failed", pt.g->bytes * n_experts));
    if ((rc = upload_tiled(*pt.g, pt.src, n_experts, *pt.dst, pt.g->bytes))) return cleanup(rc);
  }
  if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess)
    return cleanup(fail(RE_ERR_HIP, "hipStreamCreate failed"));
  if (hipEventCreateWithFlags(&e->meta_ev, hipEventDisableTiming) != hipSuccess)
    return cleanup(fail(RE_ERR_HIP, "hipEventCreate failed"));
  *out = e;
  return RE_OK;
}

namespace {
// drops the shared expert's matrices and scratch (the caller holds e->mu or owns e exclusively,
// and no queued launch uses them any more)
void moe_clear_shared(re_moe* e) {
  for (re_qmat** q : {&e->sh_gate, &e->sh_up, &e->sh_down}) {
    re_qmat_destroy(*q);
    *q = nullptr;
  }
  for (Staging* st : {&e->ssg, &e->ssu, &e->ssh, &e->ssy}) st->release();
  e->sh_inter = 0;
}
}  // namespace

void re_moe_destroy(re_moe* e) {
  if (!e) return;
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  moe_clear_shared(e);
  e->dmeta.release();
  e->droute.release();
  if (e->d_gate) (void)hipFree(e->d_gate);
  if (e->d_up) (void)hipFree(e->d_up);
  if (e->d_down) (void)hipFree(e->d_down);
  for (Staging* s : {&e->sx, &e->sout, &e->sg, &e->su, &e->sh, &e->syp, &e->smeta, &e->sxb}) s->release();
  e->hx.release();
  e->hout.release();
  if (e->meta_ev) (void)hipEventSynchronize(e->meta_ev);
  if (e->meta_ev) (void)hipEventDestroy(e->meta_ev);
  if (e->hmeta) (void)hipHostFree(e->hmeta);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

// Shared expert (moe.rs:380-385, 424-429): down(silu(gate x) * up x) of every token, added to the
// routed sum (out[t] = routed[t] + shared[t]). The three matrices are QMats (any type QMat takes).
int re_moe_set_shared(re_moe* e, uint32_t gate_type, const uint8_t* gate, size_t gate_bytes, uint32_t up_type,
                      const uint8_t* up, size_t up_bytes, uint32_t down_type, const uint8_t* down, size_t down_bytes,
                      size_t inter) {
  if (!e) return fail(RE_ERR_ARG, "null moe");
  if ((gate || up || down) && (!gate || !up || !down)) return fail(RE_ERR_ARG, "shared expert: null pointer");
  // a host forward holds e->mu while it runs the shared expert; launches already queued by any
  // forward (host or device-pointer, on any stream) may still read the old matrices, so the device
  // drains before they are freed (a set-up call, not a hot path)
  std::lock_guard<std::mutex> lk(e->mu);
  HIP_TRY(hipDeviceSynchronize());
  moe_clear_shared(e);
  if (!gate) return RE_OK;
  int rc;
  if ((rc = re_qmat_create(gate_type, gate, gate_bytes, inter, e->hidden, &e->sh_gate)) ||
      (rc = re_qmat_create(up_type, up, up_bytes, inter, e->hidden, &e->sh_up)) ||
      (rc = re_qmat_create(down_type, down, down_bytes, e->hidden, inter, &e->sh_down))) {
    const std::string msg = re_last_error();
    moe_clear_shared(e);
    return fail(rc, "shared expert: %s", msg.c_str());
  }
  e->sh_inter = inter;
  return RE_OK;
}

namespace {

int moe_add_shared(re_moe* e, const float* d_x, size_t tokens, float* d_out, int mode, hipStream_t s) {
  if (!e->sh_gate) return RE_OK;
  const size_t act = tokens * e->sh_inter * sizeof(float), out = tokens * e->hidden * sizeof(float);
  int rc;
  if ((rc = e->ssg.ensure(act)) || (rc = e->ssu.ensure(act)) || (rc = e->ssh.ensure(act)) || (rc = e->ssy.ensure(out)))
    return rc;
  float *g = (float*)e->ssg.p, *u = (float*)e->ssu.p, *h = (float*)e->ssh.p, *y = (float*)e->ssy.p;
  if ((rc = re_qmat_matmul_dev(e->sh_gate, d_x, tokens, g, mode, s)) ||
      (rc = re_qmat_matmul_dev(e->sh_up, d_x, tokens, u, mode, s)))
    return rc;
  HIP_TRY(launch_swiglu(g, u, h, tokens * e->sh_inter, s));
  if ((rc = re_qmat_matmul_dev(e->sh_down, h, tokens, y, mode, s))) return rc;
  HIP_TRY(launch_add(d_out, y, tokens * e->hidden, tokens * e->hidden, d_out, s));
  return RE_OK;
}

// One token routed to k <= 8 experts with one gate/up type: the gate/up GEMV tasks come straight
// from the ids (no planning launch) and the down projection and the combine are one launch.
// REHIP_MOE_ONE=0 keeps the general path.
static bool moe_one_token_ok(const re_moe* e, size_t tokens, size_t top_k) {
  return tokens == 1 && top_k <= (size_t)kMoeOneTokenMaxK && e->gg.type == e->gu.type && moe_gemv_fits(e) &&
         moe_down_combine_lds(e->gd.type, (int)e->gd.kb, (int)top_k) <= kMaxLdsBytes &&
         env_size("REHIP_MOE_ONE", 1) != 0;
}

// d_ids / d_w: device ids and weights, or nullptr with h_ids / h_w on the host (passed by value)
static int moe_one_token(re_moe* e, const float* d_x, size_t top_k, const int* d_ids, const float* d_w,
                         const uint32_t* h_ids, const float* h_w, float* d_out, int mode, hipStream_t s) {
  int rc;
  if ((rc = e->sh.ensure(top_k * e->inter * sizeof(float)))) return rc;
  const int rgu = moe_gemv_rows_gu1();
  MoeGemvArgs g{};
  g.rows_per_task = rgu;
  g.max_rows = 1;
  g.X = d_x;
  g.ids = d_ids;
  g.id_inline = d_ids ? 0 : 1;
  if (g.id_inline)
    for (size_t j = 0; j < top_k; ++j) g.id_v[j] = (int)h_ids[j];
  g.id_tiles = (int)((e->inter + rgu - 1) / rgu);
  g.n_experts = (int)e->n_experts;
  g.m = (int)e->inter;
  g.K = (int)e->hidden;
  g.KB = (int)e->gg.kb;
  g.ldy = (int)e->inter;
  g.w_stride = e->gg.bytes;
  g.W0 = e->d_gate;
  g.W1 = e->d_up;
  g.Y = (float*)e->sh.p;
  HIP_TRY(launch_moe_gemv(e->gg.type, true, g, (int)top_k * g.id_tiles, s));
  MoeDownCombineArgs d{};
  d.W = e->d_down;
  d.w_stride = e->gd.bytes;
  d.H = (const float*)e->sh.p;
  d.ids = d_ids;
  d.wts = d_w;
  if (!d_ids)
    for (size_t j = 0; j < top_k; ++j) {
      d.id_v[j] = (int)h_ids[j];
      d.w_v[j] = h_w[j];
    }
  d.out = d_out;
  d.m = (int)e->hidden;
  d.K = (int)e->inter;
  d.KB = (int)e->gd.kb;
  d.k = (int)top_k;
  d.n_experts = (int)e->n_experts;
  HIP_TRY(launch_moe_down_combine(e->gd.type, d, s));
  return moe_add_shared(e, d_x, 1, d_out, mode, s);
}

}  // namespace

namespace {

// With 64-row chunks the down projection's tasks cover 128 weight rows (two tiles per wave, each
// activation load feeding twice the weights); with 32-row chunks one tile (more, shorter tasks
// suit the few rows). REHIP_QMMA_DOWN2 = 0 / 1 overrides.
int moe_qmma_down_pair(int chunk) {
  const size_t v = env_size("REHIP_QMMA_DOWN2", 2);
  if (v == 0 || v == 1) return v ? kQmmaTwoTiles : kQmmaOneTile;
  return chunk > 32 ? kQmmaTwoTiles : kQmmaOneTile;
}
int moe_qmma_down_rows(int chunk) { return moe_qmma_down_pair(chunk) == kQmmaTwoTiles ? 128 : 64; }

// gate/up pair (h = silu(gate x) * up x as bf16, rows gathered through xrow from the bf16 copy of x
// in e->sxb) then down (syp, f32) with the register-decoded grouped GEMMs; the task lists and
// their device counts (nullptr: the launch count is exact) come from the host or device planner
hipError_t moe_qmma_ffn(re_moe* e, size_t tokens, size_t pairs, int chunk, const int* xrow, const GemmTask* t_gu,
                        const int* n_gu_dev, int n_gu, const GemmTask* t_d, const int* n_d_dev, int n_d,
                        hipStream_t s, bool split = false) {
  // split: e->sxb holds x's hi then lo halves, and h goes to e->sh as hi then lo (the f32 size)
  GemmArgs a{};
  a.W = e->d_gate;
  a.W2 = e->d_up;
  a.w_bytes = (uint32_t)(e->gg.bytes * e->n_experts);
  a.w_stride = e->gg.bytes;
  a.X = e->sxb.p;
  a.x_bytes = (uint32_t)(tokens * e->hidden * 2 * (split ? 2 : 1));
  a.x_lo = (uint32_t)(tokens * e->hidden * 2);
  a.y_lo = pairs * e->inter;
  a.xrow = xrow;
  a.Y = (float*)e->sh.p;
  a.m = (int)e->inter;
  a.K = (int)e->hidden;
  a.KB = (int)e->gg.kb;
  a.tiles = (int)e->gg.tiles;
  a.ldy = (int)e->inter;
  a.tasks = t_gu;
  a.ntasks = n_gu_dev;
  hipError_t err = launch_moe_qmma(e->gg.type, kQmmaGateUp, chunk, a, n_gu, s, split);
  if (err != hipSuccess) return err;
  GemmArgs d{};
  d.W = e->d_down;
  d.w_bytes = (uint32_t)(e->gd.bytes * e->n_experts);
  d.w_stride = e->gd.bytes;
  d.X = e->sh.p;
  d.x_bytes = (uint32_t)(pairs * e->inter * 2 * (split ? 2 : 1));
  d.x_lo = (uint32_t)(pairs * e->inter * 2);
  d.xrow = nullptr;
  d.Y = (float*)e->syp.p;
  d.m = (int)e->hidden;
  d.K = (int)e->inter;
  d.KB = (int)e->gd.kb;
  d.tiles = (int)e->gd.tiles;
  d.ldy = (int)e->hidden;
  d.tasks = t_d;
  d.ntasks = n_d_dev;
  return launch_moe_qmma(e->gd.type, moe_qmma_down_pair(chunk), chunk, d, n_d, s, split);
}

}  // namespace

// ---- MoE with the routing on the device (row F3: no host round trip) ------------------------
int re_moe_route_dev(const float* d_logits, size_t tokens, size_t n_experts, size_t top_k, int gate, int* d_ids,
                     float* d_weights, void* stream) {
  if (!d_logits || !d_ids || !d_weights) return fail(RE_ERR_ARG, "null pointer");
  if (tokens == 0) return RE_OK;
  if (n_experts == 0 || n_experts > 1024 || top_k == 0 || top_k > n_experts || tokens > (1u << 24))
    return fail(RE_ERR_SIZE, "route: %zu experts (<= 1024), top_k %zu, %zu tokens", n_experts, top_k, tokens);
  if (gate != RE_GATE_SOFTMAX && gate != RE_GATE_SIGMOID) return fail(RE_ERR_ARG, "unknown gate %d", gate);
  HIP_TRY(launch_moe_route(d_logits, (int)tokens, (int)n_experts, (int)top_k, gate, d_ids, d_weights,
                           (hipStream_t)stream));
  return RE_OK;
}

int re_moe_route_group_dev(const float* d_logits, size_t tokens, size_t n_experts, size_t top_k, int gate,
                           const float* d_bias, size_t bias_len, size_t n_groups, size_t top_k_group, int* d_ids,
                           float* d_weights, void* stream) {
  if (!d_logits || !d_ids || !d_weights) return fail(RE_ERR_ARG, "null pointer");
  if (bias_len && !d_bias) return fail(RE_ERR_ARG, "null bias with bias_len %zu", bias_len);
  if (gate != RE_GATE_GROUP && gate != RE_GATE_NOAUX_TC) return fail(RE_ERR_ARG, "unknown group gate %d", gate);
  if (tokens == 0) return RE_OK;
  if (n_experts == 0 || n_experts > 1024 || top_k == 0 || top_k > n_experts || tokens > (1u << 24))
    return fail(RE_ERR_SIZE, "route: %zu experts (<= 1024), top_k %zu, %zu tokens", n_experts, top_k, tokens);
  // the reference clamps the group count to 1 ..= n (n_groups.max(1).min(n), moe.rs:150, 217)
  const size_t ng = std::min(std::max<size_t>(n_groups, 1), n_experts);
  HIP_TRY(launch_moe_route_group(d_logits, (int)tokens, (int)n_experts, (int)top_k, gate == RE_GATE_NOAUX_TC ? 1 : 0,
                                 d_bias, (int)std::min(bias_len, n_experts), (int)ng,
                                 (int)std::min(top_k_group, ng), d_ids, d_weights, (hipStream_t)stream));
  return RE_OK;
}

int re_moe_router_logits_dev(const float* d_x, const float* d_router_w, size_t tokens, size_t hidden,
                             size_t n_experts, float* d_logits, void* stream) {
  if (!d_x || !d_router_w || !d_logits) return fail(RE_ERR_ARG, "null pointer");
  if (tokens == 0) return RE_OK;
  if (hidden == 0 || hidden > 16384 || n_experts == 0 || n_experts > 65535 * 4 || tokens > 65535)
    return fail(RE_ERR_SIZE, "router: %zu tokens x %zu hidden, %zu experts", tokens, hidden, n_experts);
  HIP_TRY(launch_moe_router_logits(d_x, d_router_w, (int)tokens, (int)hidden, (int)n_experts, d_logits,
                                   (hipStream_t)stream));
  return RE_OK;
}

int re_moe_forward_routed_dev(re_moe* e, const float* d_x, size_t tokens, size_t top_k, const int* d_ids,
                              const float* d_weights, float* d_out, int mode, void* stream) {
  if (!e) return fail(RE_ERR_ARG, "null moe");
  if (mode != RE_MODE_BF16 && mode != RE_MODE_F32) return fail(RE_ERR_ARG, "unknown mode %d", mode);
  if (tokens == 0) return RE_OK;
  if (!d_x || !d_out || !d_ids || !d_weights || top_k == 0) return fail(RE_ERR_ARG, "null pointer or top_k = 0");
  const size_t pairs = tokens * top_k;
  if (pairs > (size_t)kMoeMaxDevicePairs || e->n_experts > 1024)
    return fail(RE_ERR_SIZE, "device routing takes <= %d (token, expert) pairs and <= 1024 experts",
                kMoeMaxDevicePairs);
  if (tokens * e->hidden * sizeof(float) >= (1ull << 31) || e->gg.bytes * e->n_experts >= (1ull << 31) ||
      e->gu.bytes * e->n_experts >= (1ull << 31) || e->gd.bytes * e->n_experts >= (1ull << 31) ||
      pairs * e->inter * sizeof(float) >= (1ull << 31))
    return fail(RE_ERR_SIZE, "MoE operands must stay below 2 GiB");
  hipStream_t s = (hipStream_t)stream;
  if (moe_one_token_ok(e, tokens, top_k))
    return moe_one_token(e, d_x, top_k, d_ids, d_weights, nullptr, nullptr, d_out, mode, s);
  // the grouping runs on the device, so the path is chosen from the batch size alone: the
  // grouped GEMV while an expert would get few rows on average (pairs <= 2 x experts); the
  // register-decoded grouped GEMMs take 32-row chunks there (one token tile) and 64 beyond
  const bool few = pairs <= 2 * e->n_experts;
  const bool qmma = moe_qmma_path(e, d_x, tokens, mode);
  const bool split = !qmma && moe_split_path(e, d_x, tokens, mode, few);
  const bool gemv = !qmma && !split && few && moe_gemv_fits(e);
  MoePlanShape sh{};
  sh.pairs = (int)pairs;
  sh.k = (int)top_k;
  sh.n_experts = (int)e->n_experts;
  sh.gemv = gemv;
  sh.chunk = gemv ? (tokens == 1 ? 1 : kMoeGemvBatch) : moe_qmma_chunk(qmma || split, few);
  if (gemv) {
    const int rd = moe_gemv_rows_down();
    const int rgu = tokens == 1 && e->gg.type == e->gu.type ? moe_gemv_rows_gu1() : kMoeGemvRows;
    sh.rows_gu = rgu;
    sh.rows_d = rd;
    sh.tiles_gu = (int)((e->inter + rgu - 1) / rgu);
    sh.tiles_d = (int)((e->hidden + rd - 1) / rd);
  } else {
    sh.rows_gu = sh.rows_d = kMoeTile;
    sh.tiles_gu = (int)((e->inter + kMoeTile - 1) / kMoeTile);
    const int rows_d = qmma || split ? moe_qmma_down_rows(sh.chunk) : kMoeTile;
    sh.tiles_d = (int)((e->hidden + rows_d - 1) / rows_d);
  }
  const int max_chunks = (int)((pairs + sh.chunk - 1) / sh.chunk + std::min(pairs, e->n_experts));
  sh.max_gu = max_chunks * sh.tiles_gu;
  sh.max_d = max_chunks * sh.tiles_d;
  int rc;
  const size_t act = pairs * e->inter * sizeof(float);
  if ((rc = e->dmeta.ensure(moe_meta_bytes(sh))) || (rc = e->sh.ensure(act)) ||
      (rc = e->syp.ensure(pairs * e->hidden * sizeof(float))))
    return rc;
  const bool dual = gemv && e->gg.type == e->gu.type;
  if (!dual && ((rc = e->sg.ensure(act)) || (rc = e->su.ensure(act)))) return rc;
  // the bf16 copy of X (grouped GEMMs in bf16 mode) is made by the planning launch
  const bool xb = !gemv && moe_bf16_acts(e, d_x, mode);
  if ((xb || split) && (rc = e->sxb.ensure(tokens * e->hidden * 2 * (split ? 2 : 1)))) return rc;
  int* dm = (int*)e->dmeta.p;
  HIP_TRY(launch_moe_plan(d_ids, sh, dm, d_x, xb || split ? e->sxb.p : nullptr, tokens * e->hidden, s, split));
  const int* xrow = dm;
  const int* pos = dm + pairs;
  const int* ntasks = dm + 2 * pairs;
  const uint8_t* tasks = (const uint8_t*)(dm + 2 * pairs + 4);
  if (gemv) {
    const MoeGemvTask* tg = (const MoeGemvTask*)tasks;
    MoeGemvArgs g{};
    g.rows_per_task = sh.rows_gu;
    g.max_rows = sh.chunk;
    g.X = d_x;
    g.xrow = xrow;
    g.tasks = tg;
    g.ntasks = ntasks;
    g.m = (int)e->inter;
    g.K = (int)e->hidden;
    g.KB = (int)e->gg.kb;
    g.ldy = (int)e->inter;
    g.w_stride = e->gg.bytes;
    if (dual) {
      g.W0 = e->d_gate;
      g.W1 = e->d_up;
      g.Y = (float*)e->sh.p;
      HIP_TRY(launch_moe_gemv(e->gg.type, true, g, sh.max_gu, s));
    } else {
      g.W0 = e->d_gate;
      g.Y = (float*)e->sg.p;
      HIP_TRY(launch_moe_gemv(e->gg.type, false, g, sh.max_gu, s));
      g.W0 = e->d_up;
      g.w_stride = e->gu.bytes;
      g.KB = (int)e->gu.kb;
      g.Y = (float*)e->su.p;
      HIP_TRY(launch_moe_gemv(e->gu.type, false, g, sh.max_gu, s));
      HIP_TRY(launch_swiglu((const float*)e->sg.p, (const float*)e->su.p, (float*)e->sh.p, pairs * e->inter, s));
    }
    MoeGemvArgs d{};
    d.rows_per_task = moe_gemv_rows_down();
    d.max_rows = sh.chunk;
    d.W0 = e->d_down;
    d.w_stride = e->gd.bytes;
    d.X = (const float*)e->sh.p;
    d.xrow = nullptr;
    d.Y = (float*)e->syp.p;
    d.tasks = tg + sh.max_gu;
    d.ntasks = ntasks + 1;
    d.m = (int)e->hidden;
    d.K = (int)e->inter;
    d.KB = (int)e->gd.kb;
    d.ldy = (int)e->hidden;
    HIP_TRY(launch_moe_gemv(e->gd.type, false, d, sh.max_d, s));
  } else if (qmma || split) {
    const GemmTask* tg = (const GemmTask*)tasks;
    HIP_TRY(moe_qmma_ffn(e, tokens, pairs, sh.chunk, xrow, tg, ntasks, sh.max_gu, tg + sh.max_gu, ntasks + 1,
                         sh.max_d, s, split));
  } else {
    const GemmTask* tg = (const GemmTask*)tasks;
    GemmArgs a{};
    a.X = d_x;
    a.x_bytes = (uint32_t)(tokens * e->hidden * sizeof(float));
    a.splits = 1;
    a.steps_per_split = 1 << 30;
    a.tasks = tg;
    a.ntasks = ntasks;
    a.xrow = xrow;
    a.m = (int)e->inter;
    a.K = (int)e->hidden;
    a.KB = (int)e->gg.kb;
    a.tiles = (int)e->gg.tiles;
    a.ldy = (int)e->inter;
    a.w_stride = e->gg.bytes;
    a.w_bytes = (uint32_t)(e->gg.bytes * e->n_experts);
    a.W = e->d_gate;
    a.Y = (float*)e->sg.p;
    if (xb) {
      a.X = e->sxb.p;
      a.x_bytes = (uint32_t)(tokens * e->hidden * 2);
      a.x_bf16 = 1;
    }
    const int kg_gu = gemm_kgroups(GemmTile::k64x64, mode, (long)sh.max_gu, (int)((e->hidden + kGemmBK - 1) / kGemmBK));
    const int kg_d = gemm_kgroups(GemmTile::k64x64, mode, (long)sh.max_d, (int)((e->inter + kGemmBK - 1) / kGemmBK));
    // bf16 activations and one gate/up type: one launch decodes both tiles against one staging of
    // the rows and writes h = silu(gate) * up as bf16 (the same values as the separate GEMMs and
    // SwiGLU below). REHIP_MOE_PAIR=0 turns it off.
    const bool pair = xb && e->gg.type == e->gu.type && kg_gu == 1 && env_size("REHIP_MOE_PAIR", 1) != 0;
    if (pair) {
      a.W2 = e->d_up;
      a.Y = (float*)e->sh.p;
      HIP_TRY(launch_gemm(e->gg.type, mode, a, sh.max_gu, GemmTile::k64x64, 1, s));
    } else {
      HIP_TRY(launch_gemm(e->gg.type, mode, a, sh.max_gu, GemmTile::k64x64, kg_gu, s));
      a.W = e->d_up;
      a.w_stride = e->gu.bytes;
      a.w_bytes = (uint32_t)(e->gu.bytes * e->n_experts);
      a.KB = (int)e->gu.kb;
      a.tiles = (int)e->gu.tiles;
      a.Y = (float*)e->su.p;
      HIP_TRY(launch_gemm(e->gu.type, mode, a, sh.max_gu, GemmTile::k64x64, kg_gu, s));
      if (xb) HIP_TRY(launch_swiglu_bf16((const float*)e->sg.p, (const float*)e->su.p, e->sh.p, pairs * e->inter, s));
      else HIP_TRY(launch_swiglu((const float*)e->sg.p, (const float*)e->su.p, (float*)e->sh.p, pairs * e->inter, s));
    }
    GemmArgs d{};
    d.X = e->sh.p;
    d.x_bytes = (uint32_t)(xb ? act / 2 : act);
    d.x_bf16 = xb;
    d.splits = 1;
    d.steps_per_split = 1 << 30;
    d.tasks = tg + sh.max_gu;
    d.ntasks = ntasks + 1;
    d.xrow = nullptr;
    d.m = (int)e->hidden;
    d.K = (int)e->inter;
    d.KB = (int)e->gd.kb;
    d.tiles = (int)e->gd.tiles;
    d.ldy = (int)e->hidden;
    d.w_stride = e->gd.bytes;
    d.w_bytes = (uint32_t)(e->gd.bytes * e->n_experts);
    d.W = e->d_down;
    d.Y = (float*)e->syp.p;
    HIP_TRY(launch_gemm(e->gd.type, mode, d, sh.max_d, GemmTile::k64x64, kg_d, s));
  }
  HIP_TRY(launch_combine((const float*)e->syp.p, pos, d_weights, d_out, (int)tokens, (int)top_k, (int)e->hidden, s));
  return moe_add_shared(e, d_x, tokens, d_out, mode, s);
}

}  // extern "C"

namespace {
// router logits -> route (`route(logits, ids, weights)`) -> the FFN, in one stream; the scratch
// for the logits, ids and weights is kept by e
template <typename Route>
int moe_layer(re_moe* e, const float* d_x, size_t tokens, const float* d_router_w, size_t top_k, float* d_out,
              int mode, void* stream, Route route) {
  if (!e || !d_x || !d_router_w || !d_out) return fail(RE_ERR_ARG, "null pointer");
  if (tokens == 0) return RE_OK;
  if (tokens > 65535) return fail(RE_ERR_SIZE, "%zu tokens", tokens);
  const size_t E = e->n_experts;
  const size_t logit_bytes = (tokens * E * sizeof(float) + 255) / 256 * 256;
  const size_t id_bytes = (tokens * top_k * sizeof(int) + 255) / 256 * 256;
  int rc;
  if ((rc = e->droute.ensure(logit_bytes + 2 * id_bytes))) return rc;
  float* logits = (float*)e->droute.p;
  int* ids = (int*)((uint8_t*)e->droute.p + logit_bytes);
  float* w = (float*)((uint8_t*)e->droute.p + logit_bytes + id_bytes);
  if ((rc = re_moe_router_logits_dev(d_x, d_router_w, tokens, e->hidden, E, logits, stream))) return rc;
  if ((rc = route(logits, ids, w))) return rc;
  return re_moe_forward_routed_dev(e, d_x, tokens, top_k, ids, w, d_out, mode, stream);
}
}  // namespace

extern "C" {

int re_moe_layer_dev(re_moe* e, const float* d_x, size_t tokens, const float* d_router_w, size_t top_k, int gate,
                     float* d_out, int mode, void* stream) {
  return moe_layer(e, d_x, tokens, d_router_w, top_k, d_out, mode, stream, [&](const float* lg, int* ids, float* w) {
    return re_moe_route_dev(lg, tokens, e->n_experts, top_k, gate, ids, w, stream);
  });
}

int re_moe_layer_group_dev(re_moe* e, const float* d_x, size_t tokens, const float* d_router_w, size_t top_k,
                           int gate, const float* d_bias, size_t bias_len, size_t n_groups, size_t top_k_group,
                           float* d_out, int mode, void* stream) {
  return moe_layer(e, d_x, tokens, d_router_w, top_k, d_out, mode, stream, [&](const float* lg, int* ids, float* w) {
    return re_moe_route_group_dev(lg, tokens, e->n_experts, top_k, gate, d_bias, bias_len, n_groups, top_k_group,
                                  ids, w, stream);
  });
}

int re_moe_forward_dev(re_moe* e, const float* d_x, size_t tokens, size_t top_k, const uint32_t* ids,
                       const float* weights, float* d_out, int mode, void* stream) {
  if (!e) return fail(RE_ERR_ARG, "null moe");
  if (mode != RE_MODE_BF16 && mode != RE_MODE_F32) return fail(RE_ERR_ARG, "unknown mode %d", mode);
  if (tokens == 0) return RE_OK;
  if (!d_x || !d_out || !ids || !weights || top_k == 0) return fail(RE_ERR_ARG, "null pointer or top_k = 0");
  const size_t pairs = tokens * top_k;
  if (pairs > (1u << 24)) return fail(RE_ERR_SIZE, "too many (token, expert) pairs");
  for (size_t p = 0; p < pairs; ++p)
    if (ids[p] >= e->n_experts) return fail(RE_ERR_ARG, "expert id %u out of range (%zu experts)", ids[p], e->n_experts);
  hipStream_t s = (hipStream_t)stream;

  // one token: its ids and weights ride in the kernel arguments (no upload)
  if (moe_one_token_ok(e, tokens, top_k))
    return moe_one_token(e, d_x, top_k, nullptr, nullptr, ids, weights, d_out, mode, s);

  // up to 2048 (token, expert) pairs: one pinned upload of the ids and weights, then the
  // device-routed launches (grouping, bf16 rounding of X and task lists in one planning launch,
  // task counts read on the device), so both entries run the same kernels and give the same
  // bits. Measured back to back on the Qwen3-30B-A3B expert shape: 32 tokens 113 -> 103 us and
  // 128 tokens 130 -> 119 us per call; at 512 tokens the host grouping (which overlaps the
  // previous call's kernels) is faster, 168 against 176 us, as the device planning launch sits on
  // the GPU's critical path. REHIP_MOE_HOST_GROUP=1 keeps the host grouping for every batch.
  if (pairs <= 2048 && e->n_experts <= 1024 && env_size("REHIP_MOE_HOST_GROUP", 0) == 0) {
    const size_t bytes = pairs * (sizeof(int) + sizeof(float));
    int rc;
    if ((rc = e->smeta.ensure(bytes))) return rc;
    // the pinned staging is rewritten once its previous upload has completed
    if (e->meta_pending) {
      HIP_TRY(hipEventSynchronize(e->meta_ev));
      e->meta_pending = false;
    }
    if (bytes > e->hmeta_cap) {
      if (e->hmeta) (void)hipHostFree(e->hmeta);
      e->hmeta = nullptr;
      e->hmeta_cap = 0;
      HIP_TRY(hipHostMalloc(&e->hmeta, bytes, hipHostMallocDefault));
      e->hmeta_cap = bytes;
    }
    std::memcpy(e->hmeta, ids, pairs * sizeof(int));   // ids < n_experts <= 1024: the same bits as int
    std::memcpy((uint8_t*)e->hmeta + pairs * sizeof(int), weights, pairs * sizeof(float));
    uint8_t* dm = (uint8_t*)e->smeta.p;
    HIP_TRY(hipMemcpyAsync(dm, e->hmeta, bytes, hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(e->meta_ev, s));
    e->meta_pending = true;
    return re_moe_forward_routed_dev(e, d_x, tokens, top_k, (const int*)dm, (const float*)(dm + pairs * sizeof(int)),
                                     d_out, mode, stream);
  }

  // group the pairs by expert, keeping (token, slot) order inside an expert
  std::vector<int> count(e->n_experts + 1, 0), start(e->n_experts + 1, 0);
  for (size_t p = 0; p < pairs; ++p) count[ids[p]]++;
  for (size_t x = 0; x < e->n_experts; ++x) start[x + 1] = start[x] + count[x];
  size_t touched = 0;
  for (size_t x = 0; x < e->n_experts; ++x) touched += count[x] > 0;
  std::vector<int> fill(start.begin(), start.end() - 1);
  std::vector<int> xrow(pairs), pos(pairs);
  for (size_t p = 0; p < pairs; ++p) {
    const int at = fill[ids[p]]++;
    xrow[at] = (int)(p / top_k);
    pos[p] = at;
  }
  if (tokens * e->hidden * sizeof(float) >= (1ull << 31) || e->gg.bytes * e->n_experts >= (1ull << 31) ||
      e->gu.bytes * e->n_experts >= (1ull << 31) || e->gd.bytes * e->n_experts >= (1ull << 31) ||
      pairs * e->inter * sizeof(float) >= (1ull << 31))
    return fail(RE_ERR_SIZE, "MoE operands must stay below 2 GiB");

  // Few rows per expert (decode-sized batches): grouped GEMV tasks that read each weight once
  // per kMoeGemvBatch rows. Otherwise MFMA tiles of kMoeTile gathered rows. The register-decoded
  // grouped GEMMs (bf16 mode) take chunks of 32 rows while the rows per expert are few, else 64.
  const bool few = pairs <= (size_t)kMoeGemvBatch * touched;
  const bool qmma = moe_qmma_path(e, d_x, tokens, mode);
  const bool split = !qmma && moe_split_path(e, d_x, tokens, mode, few);
  const bool gemv = !qmma && !split && few && moe_gemv_fits(e);
  const int chunk = moe_qmma_chunk(qmma || split, few);
  int max_rows = 0;
  for (size_t x = 0; x < e->n_experts; ++x) max_rows = std::max(max_rows, std::min(count[x], kMoeGemvBatch));
  // 16-row gate/up tasks exist for single-row tasks only (a repeated expert id gives 2+ rows)
  const int rgu = tokens == 1 && max_rows <= 1 && e->gg.type == e->gu.type ? moe_gemv_rows_gu1() : kMoeGemvRows;
  std::vector<MoeGemvTask> v_gu, v_d;
  std::vector<GemmTask> t_gu, t_d;
  if (gemv) {
    for (size_t x = 0; x < e->n_experts; ++x)
      for (int r = 0; r < count[x]; r += kMoeGemvBatch) {
        const int np = std::min(kMoeGemvBatch, count[x] - r);
        for (size_t row = 0; row < e->inter; row += (size_t)rgu) v_gu.push_back({(int)x, (int)row, start[x] + r, np});
        for (size_t row = 0; row < e->hidden; row += (size_t)moe_gemv_rows_down())
          v_d.push_back({(int)x, (int)row, start[x] + r, np});
      }
  } else {
    const int rows_d = qmma || split ? moe_qmma_down_rows(chunk) : kMoeTile;
    const int mt_gu = (int)((e->inter + kMoeTile - 1) / kMoeTile), mt_d = (int)((e->hidden + rows_d - 1) / rows_d);
    for (size_t x = 0; x < e->n_experts; ++x) {
      for (int r = 0; r < count[x]; r += chunk) {
        const int rn = std::min(chunk, count[x] - r);
        for (int mt = 0; mt < mt_gu; ++mt) t_gu.push_back({(int)x, mt, start[x] + r, rn});
        for (int mt = 0; mt < mt_d; ++mt) t_d.push_back({(int)x, mt, start[x] + r, rn});
      }
    }
  }
  // metadata block: xrow | pos | weights | tasks_gu | tasks_d
  const size_t task_sz = gemv ? sizeof(MoeGemvTask) : sizeof(GemmTask);
  const size_t n_gu = gemv ? v_gu.size() : t_gu.size(), n_d = gemv ? v_d.size() : t_d.size();
  const size_t off_pos = pairs * sizeof(int), off_w = 2 * pairs * sizeof(int);
  const size_t off_tgu = (off_w + pairs * sizeof(float) + 15) / 16 * 16;
  const size_t off_td = off_tgu + n_gu * task_sz;
  const size_t meta_bytes = off_td + n_d * task_sz;

  int rc;
  const size_t act = pairs * e->inter * sizeof(float);
  if ((rc = e->smeta.ensure(meta_bytes)) || (rc = e->sh.ensure(act)) ||
      (rc = e->syp.ensure(pairs * e->hidden * sizeof(float))))
    return rc;
  const bool dual = gemv && e->gg.type == e->gu.type;
  if (!dual && ((rc = e->sg.ensure(act)) || (rc = e->su.ensure(act)))) return rc;
  // the pinned staging is rewritten once its previous upload has completed
  if (e->meta_pending) {
    HIP_TRY(hipEventSynchronize(e->meta_ev));
    e->meta_pending = false;
  }
  if (meta_bytes > e->hmeta_cap) {
    if (e->hmeta) (void)hipHostFree(e->hmeta);
    e->hmeta = nullptr;
    e->hmeta_cap = 0;
    HIP_TRY(hipHostMalloc(&e->hmeta, meta_bytes, hipHostMallocDefault));
    e->hmeta_cap = meta_bytes;
  }
  uint8_t* meta = (uint8_t*)e->hmeta;
  std::memcpy(meta, xrow.data(), pairs * sizeof(int));
  std::memcpy(meta + off_pos, pos.data(), pairs * sizeof(int));
  std::memcpy(meta + off_w, weights, pairs * sizeof(float));
  std::memcpy(meta + off_tgu, gemv ? (const void*)v_gu.data() : (const void*)t_gu.data(), n_gu * task_sz);
  std::memcpy(meta + off_td, gemv ? (const void*)v_d.data() : (const void*)t_d.data(), n_d * task_sz);
  uint8_t* dm = (uint8_t*)e->smeta.p;
  HIP_TRY(hipMemcpyAsync(dm, meta, meta_bytes, hipMemcpyHostToDevice, s));
  HIP_TRY(hipEventRecord(e->meta_ev, s));
  e->meta_pending = true;

  if (gemv) {
    MoeGemvArgs g{};
    g.rows_per_task = rgu;
    g.max_rows = max_rows;
    g.X = d_x;
    g.xrow = (const int*)dm;
    g.tasks = (const MoeGemvTask*)(dm + off_tgu);
    g.m = (int)e->inter;
    g.K = (int)e->hidden;
    g.KB = (int)e->gg.kb;
    g.ldy = (int)e->inter;
    g.w_stride = e->gg.bytes;
    if (dual) {
      g.W0 = e->d_gate;
      g.W1 = e->d_up;
      g.Y = (float*)e->sh.p;
      HIP_TRY(launch_moe_gemv(e->gg.type, true, g, (int)n_gu, s));
    } else {
      g.W0 = e->d_gate;
      g.Y = (float*)e->sg.p;
      HIP_TRY(launch_moe_gemv(e->gg.type, false, g, (int)n_gu, s));
      g.W0 = e->d_up;
      g.w_stride = e->gu.bytes;
      g.KB = (int)e->gu.kb;
      g.Y = (float*)e->su.p;
      HIP_TRY(launch_moe_gemv(e->gu.type, false, g, (int)n_gu, s));
      HIP_TRY(launch_swiglu((const float*)e->sg.p, (const float*)e->su.p, (float*)e->sh.p, pairs * e->inter, s));
    }
    MoeGemvArgs d{};
    d.rows_per_task = moe_gemv_rows_down();
    d.max_rows = max_rows;
    d.W0 = e->d_down;
    d.w_stride = e->gd.bytes;
    d.X = (const float*)e->sh.p;
    d.xrow = nullptr;
    d.Y = (float*)e->syp.p;
    d.tasks = (const MoeGemvTask*)(dm + off_td);
    d.m = (int)e->hidden;
    d.K = (int)e->inter;
    d.KB = (int)e->gd.kb;
    d.ldy = (int)e->hidden;
    HIP_TRY(launch_moe_gemv(e->gd.type, false, d, (int)n_d, s));
  } else if (qmma || split) {
    if ((rc = e->sxb.ensure(tokens * e->hidden * 2 * (split ? 2 : 1)))) return rc;
    if (split) HIP_TRY(launch_x_to_bf16_split(d_x, e->sxb.p, tokens * e->hidden, s));
    else HIP_TRY(launch_x_to_bf16(d_x, e->sxb.p, tokens * e->hidden, s));
    HIP_TRY(moe_qmma_ffn(e, tokens, pairs, chunk, (const int*)dm, (const GemmTask*)(dm + off_tgu), nullptr, (int)n_gu,
                         (const GemmTask*)(dm + off_td), nullptr, (int)n_d, s, split));
  } else {
    GemmArgs a{};
    a.X = d_x;
    a.x_bytes = (uint32_t)(tokens * e->hidden * sizeof(float));
    a.splits = 1;
    a.steps_per_split = 1 << 30;
    a.tasks = (const GemmTask*)(dm + off_tgu);
    a.xrow = (const int*)dm;
    a.m = (int)e->inter;
    a.K = (int)e->hidden;
    a.KB = (int)e->gg.kb;
    a.tiles = (int)e->gg.tiles;
    a.ldy = (int)e->inter;
    a.W = e->d_gate;
    a.w_bytes = (uint32_t)(e->gg.bytes * e->n_experts);
    a.w_stride = e->gg.bytes;
    a.Y = (float*)e->sg.p;
    const int kg_gu = gemm_kgroups(GemmTile::k64x64, mode, (long)n_gu, (int)((e->hidden + kGemmBK - 1) / kGemmBK));
    const int kg_d = gemm_kgroups(GemmTile::k64x64, mode, (long)n_d, (int)((e->inter + kGemmBK - 1) / kGemmBK));
    if ((rc = e->sg.ensure(act)) || (rc = e->su.ensure(act))) return rc;
    a.Y = (float*)e->sg.p;
    const bool xb = moe_bf16_acts(e, d_x, mode);
    if (xb) {
      if ((rc = e->sxb.ensure(tokens * e->hidden * 2))) return rc;
      HIP_TRY(launch_x_to_bf16(d_x, e->sxb.p, tokens * e->hidden, s));
      a.X = e->sxb.p;
      a.x_bytes = (uint32_t)(tokens * e->hidden * 2);
      a.x_bf16 = 1;
    }
    // bf16 activations and one gate/up type: one launch decodes both tiles against one staging of
    // the rows and writes h = silu(gate) * up as bf16 (the same values as the separate GEMMs and
    // SwiGLU below). REHIP_MOE_PAIR=0 turns it off.
    const bool pair = xb && e->gg.type == e->gu.type && kg_gu == 1 && env_size("REHIP_MOE_PAIR", 1) != 0;
    if (pair) {
      a.W2 = e->d_up;
      a.Y = (float*)e->sh.p;
      HIP_TRY(launch_gemm(e->gg.type, mode, a, (int)n_gu, GemmTile::k64x64, 1, s));
    } else {
      HIP_TRY(launch_gemm(e->gg.type, mode, a, (int)n_gu, GemmTile::k64x64, kg_gu, s));
      a.W = e->d_up;
      a.w_bytes = (uint32_t)(e->gu.bytes * e->n_experts);
      a.w_stride = e->gu.bytes;
      a.KB = (int)e->gu.kb;
      a.tiles = (int)e->gu.tiles;
      a.Y = (float*)e->su.p;
      HIP_TRY(launch_gemm(e->gu.type, mode, a, (int)n_gu, GemmTile::k64x64, kg_gu, s));
      if (xb) HIP_TRY(launch_swiglu_bf16((const float*)e->sg.p, (const float*)e->su.p, e->sh.p, pairs * e->inter, s));
      else HIP_TRY(launch_swiglu((const float*)e->sg.p, (const float*)e->su.p, (float*)e->sh.p, pairs * e->inter, s));
    }
    GemmArgs d{};
    d.W = e->d_down;
    d.w_bytes = (uint32_t)(e->gd.bytes * e->n_experts);
    d.w_stride = e->gd.bytes;
    d.X = e->sh.p;
    d.x_bytes = (uint32_t)(pairs * e->inter * (xb ? 2 : sizeof(float)));
    d.x_bf16 = xb;
    d.splits = 1;
    d.steps_per_split = 1 << 30;
    d.Y = (float*)e->syp.p;
    d.m = (int)e->hidden;
    d.K = (int)e->inter;
    d.KB = (int)e->gd.kb;
    d.tiles = (int)e->gd.tiles;
    d.ldy = (int)e->hidden;
    d.tasks = (const GemmTask*)(dm + off_td);
    d.xrow = nullptr;
    HIP_TRY(launch_gemm(e->gd.type, mode, d, (int)n_d, GemmTile::k64x64, kg_d, s));
  }
  HIP_TRY(launch_combine((const float*)e->syp.p, (const int*)(dm + off_pos), (const float*)(dm + off_w), d_out,
                         (int)tokens, (int)top_k, (int)e->hidden, s));
  return moe_add_shared(e, d_x, tokens, d_out, mode, s);
}

int re_moe_forward(re_moe* e, const float* x, size_t tokens, size_t top_k, const uint32_t* ids,
                   const float* weights, float* out, int mode) {
  if (!e) return fail(RE_ERR_ARG, "null moe");
  if (tokens == 0) return RE_OK;
  if (!x || !out) return fail(RE_ERR_ARG, "null pointer");
  std::lock_guard<std::mutex> lk(e->mu);
  int rc;
  const size_t xb = tokens * e->hidden * sizeof(float);
  if ((rc = e->sx.ensure(xb)) || (rc = e->sout.ensure(xb)) || (rc = e->hx.ensure(xb)) || (rc = e->hout.ensure(xb)))
    return rc;
  // through pinned staging: the copies are DMA transfers without a pageable bounce
  std::memcpy(e->hx.h, x, xb);
  HIP_TRY(hipMemcpyAsync(e->sx.p, e->hx.h, xb, hipMemcpyHostToDevice, e->stream));
  if ((rc = re_moe_forward_dev(e, (const float*)e->sx.p, tokens, top_k, ids, weights, (float*)e->sout.p, mode,
                               e->stream)))
    return rc;
  HIP_TRY(hipMemcpyAsync(e->hout.h, e->sout.p, xb, hipMemcpyDeviceToHost, e->stream));
  HIP_TRY(hipStreamSynchronize(e->stream));
  std::memcpy(out, e->hout.h, xb);
  return RE_OK;
}


// ---- device-resident transformer steps ----------------------------------------------------------
struct re_ffn {
  re_qmat *gate = nullptr, *up = nullptr;
  int ntasks = 0;
  float* d_tmp = nullptr;                 // dense gate/up: normed x, gate and up outputs
  size_t x_off = 0, g_off = 0, u_off = 0;
};

int re_rmsnorm_dev(const float* d_x, const float* d_w, size_t rows, size_t d, float eps, float* d_out, void* stream) {
  if (!d_x || !d_w || !d_out) return fail(RE_ERR_ARG, "null pointer");
  if (rows == 0) return RE_OK;
  if (d == 0 || d > (1u << 24) || rows > (1u << 24)) return fail(RE_ERR_SIZE, "rmsnorm shape %zu x %zu", rows, d);
  HIP_TRY(launch_rmsnorm(d_x, d_w, (int)rows, (int)d, eps, d_out, (hipStream_t)stream));
  return RE_OK;
}

int re_rope_dev(float* d_x, size_t rows, size_t heads, size_t head_dim, float theta, const int* d_pos, int pos_offset,
                void* stream) {
  if (!d_x || !d_pos) return fail(RE_ERR_ARG, "null pointer");
  if (rows == 0 || heads == 0) return RE_OK;
  if (head_dim == 0 || head_dim % 2 || head_dim > 128 || rows > 65535 || heads > 65535)
    return fail(RE_ERR_SIZE, "rope shape rows %zu heads %zu head_dim %zu (even, <= 128)", rows, heads, head_dim);
  HIP_TRY(launch_rope(d_x, (int)rows, (int)heads, (int)head_dim, theta, d_pos, pos_offset, (hipStream_t)stream));
  return RE_OK;
}

int re_kv_append_dev(const float* d_k, const float* d_v, size_t rows, size_t kv_dim, float* d_kcache, float* d_vcache,
                     size_t max_seq, const int* d_pos, void* stream) {
  if (!d_k || !d_v || !d_kcache || !d_vcache || !d_pos) return fail(RE_ERR_ARG, "null pointer");
  if (rows == 0) return RE_OK;
  if (kv_dim == 0 || rows > (1u << 24) || max_seq == 0 || max_seq > (1u << 24))
    return fail(RE_ERR_SIZE, "kv append shape %zu x %zu, %zu cache rows", rows, kv_dim, max_seq);
  HIP_TRY(launch_kv_append(d_k, d_v, (int)rows, (int)kv_dim, d_kcache, d_vcache, (int)max_seq, d_pos,
                           (hipStream_t)stream));
  return RE_OK;
}

size_t re_attention_work_bytes(size_t rows, size_t n_heads, size_t head_dim, size_t max_seq) {
  if (rows == 0 || n_heads == 0 || head_dim == 0 || max_seq == 0 || rows > 65535 || n_heads > 65535 ||
      head_dim > 256 || max_seq > 32768)
    return 0;
  return attention_work_floats((int)rows, (int)n_heads, (int)head_dim, (int)max_seq) * sizeof(float);
}

int re_attention_dev(const float* d_q, const float* d_kcache, const float* d_vcache, size_t rows, size_t n_heads,
                     size_t n_kv_heads, size_t head_dim, size_t max_seq, const int* d_pos, float* d_work,
                     size_t work_bytes, float* d_ctx, void* stream) {
  if (!d_q || !d_kcache || !d_vcache || !d_pos || !d_ctx) return fail(RE_ERR_ARG, "null pointer");
  if (rows == 0) return RE_OK;
  if (n_heads == 0 || n_kv_heads == 0 || n_heads % n_kv_heads || head_dim == 0 || head_dim % 4 || head_dim > 256 ||
      max_seq == 0 || max_seq > 32768 || rows > 65535 || n_heads > 65535)
    return fail(RE_ERR_SIZE, "attention shape heads %zu/%zu head_dim %zu max_seq %zu", n_heads, n_kv_heads, head_dim,
                max_seq);
  if (!aligned16(d_q) || !aligned16(d_kcache) || !aligned16(d_vcache) || !aligned16(d_ctx))
    return fail(RE_ERR_ARG, "attention buffers must be 16-byte aligned");
  if (d_work && work_bytes < re_attention_work_bytes(rows, n_heads, head_dim, max_seq))
    return fail(RE_ERR_SIZE, "attention workspace of %zu bytes, need %zu", work_bytes,
                re_attention_work_bytes(rows, n_heads, head_dim, max_seq));
  HIP_TRY(launch_attention(d_q, d_kcache, d_vcache, (int)rows, (int)n_heads, (int)n_kv_heads, (int)head_dim,
                           (int)max_seq, d_pos, d_work, d_ctx, (hipStream_t)stream));
  return RE_OK;
}

int re_rope_table_dev(float theta, size_t head_dim, size_t rows, float* d_table, void* stream) {
  if (!d_table) return fail(RE_ERR_ARG, "null pointer");
  if (head_dim == 0 || head_dim % 2 || head_dim > 256 || rows == 0 || rows > 32768)
    return fail(RE_ERR_SIZE, "rope table head_dim %zu rows %zu", head_dim, rows);
  HIP_TRY(launch_rope_table(theta, (int)head_dim, (int)rows, d_table, (hipStream_t)stream));
  return RE_OK;
}

int re_attention_decode_dev(const float* d_q, const float* d_k, const float* d_v, const float* d_bq, const float* d_bk,
                            const float* d_bv, size_t n_heads, size_t n_kv_heads, size_t head_dim, float theta,
                            const float* d_rope, const int* d_pos, float* d_kcache, float* d_vcache, size_t max_seq,
                            float* d_work, size_t work_bytes, float* d_ctx, void* stream) {
  if (!d_q || !d_k || !d_v || !d_pos || !d_kcache || !d_vcache || !d_work || !d_ctx)
    return fail(RE_ERR_ARG, "null pointer");
  if (n_heads == 0 || n_kv_heads == 0 || n_heads % n_kv_heads || head_dim == 0 || head_dim % 4 || head_dim > 256 ||
      max_seq == 0 || max_seq > 32768 || n_heads > 65535)
    return fail(RE_ERR_SIZE, "attention shape heads %zu/%zu head_dim %zu max_seq %zu", n_heads, n_kv_heads, head_dim,
                max_seq);
  if (!aligned16(d_kcache) || !aligned16(d_vcache) || !aligned16(d_ctx))
    return fail(RE_ERR_ARG, "caches and ctx must be 16-byte aligned");
  if (work_bytes < re_attention_work_bytes(1, n_heads, head_dim, max_seq))
    return fail(RE_ERR_SIZE, "attention workspace of %zu bytes, need %zu", work_bytes,
                re_attention_work_bytes(1, n_heads, head_dim, max_seq));
  HIP_TRY(launch_attention_decode(d_q, d_k, d_v, d_bq, d_bk, d_bv, (int)n_heads, (int)n_kv_heads, (int)head_dim, theta,
                                  d_rope, d_pos, d_kcache, d_vcache, (int)max_seq, d_work, d_ctx, (hipStream_t)stream));
  return RE_OK;
}

int re_qkv_rope_append_dev(const float* d_q, size_t ldq, const float* d_k, size_t ldk, const float* d_v, size_t ldv,
                           const float* d_bq, const float* d_bk, const float* d_bv, size_t rows, size_t n_heads,
                           size_t n_kv_heads, size_t head_dim, float theta, const int* d_pos, float* d_qout,
                           float* d_kcache, float* d_vcache, size_t max_seq, void* stream) {
  if (!d_q || !d_k || !d_v || !d_pos || !d_qout || !d_kcache || !d_vcache) return fail(RE_ERR_ARG, "null pointer");
  if (rows == 0) return RE_OK;
  if (n_heads == 0 || n_kv_heads == 0 || head_dim == 0 || head_dim % 2 || head_dim > 256 || rows > 65535 ||
      n_heads + n_kv_heads > 65535 || max_seq == 0 || max_seq > (1u << 24) || ldq < n_heads * head_dim ||
      ldk < n_kv_heads * head_dim || ldv < n_kv_heads * head_dim || ldq > (1u << 30) || ldk > (1u << 30) ||
      ldv > (1u << 30))
    return fail(RE_ERR_SIZE, "qkv shape rows %zu heads %zu/%zu head_dim %zu strides %zu/%zu/%zu", rows, n_heads,
                n_kv_heads, head_dim, ldq, ldk, ldv);
  HIP_TRY(launch_qkv_rope_append(d_q, (int)ldq, d_k, (int)ldk, d_v, (int)ldv, d_bq, d_bk, d_bv, (int)rows,
                                 (int)n_heads, (int)n_kv_heads, (int)head_dim, theta, d_pos, d_qout, d_kcache,
                                 d_vcache, (int)max_seq, (hipStream_t)stream));
  return RE_OK;
}

int re_decode_advance_dev(unsigned long long* d_best, int* d_tok, int* d_pos, int delta, int* d_hist,
                          size_t hist_len, void* stream) {
  if (!d_best || !d_tok || !d_pos) return fail(RE_ERR_ARG, "null pointer");
  if (hist_len > (1u << 30)) return fail(RE_ERR_SIZE, "history of %zu tokens", hist_len);
  HIP_TRY(launch_decode_advance(d_best, d_tok, d_pos, delta, d_hist, (int)hist_len, (hipStream_t)stream));
  return RE_OK;
}

int re_add_dev(const float* d_a, const float* d_b, size_t n, size_t nb, float* d_out, void* stream) {
  if (!d_a || !d_b || !d_out) return fail(RE_ERR_ARG, "null pointer");
  if (n == 0) return RE_OK;
  if (nb == 0 || n % nb) return fail(RE_ERR_SIZE, "add: %zu values with a %zu-value operand", n, nb);
  HIP_TRY(launch_add(d_a, d_b, n, nb, d_out, (hipStream_t)stream));
  return RE_OK;
}

int re_swiglu_dev(const float* d_g, const float* d_u, float* d_h, size_t n, void* stream) {
  if (!d_g || !d_u || !d_h) return fail(RE_ERR_ARG, "null pointer");
  HIP_TRY(launch_swiglu(d_g, d_u, d_h, n, (hipStream_t)stream));
  return RE_OK;
}

int re_argmax_dev(const float* d_x, size_t n, int* d_idx, void* stream) {
  if (!d_x || !d_idx) return fail(RE_ERR_ARG, "null pointer");
  if (n == 0 || n > (1u << 30)) return fail(RE_ERR_SIZE, "argmax over %zu values", n);
  HIP_TRY(launch_argmax(d_x, (int)n, d_idx, (hipStream_t)stream));
  return RE_OK;
}

int re_embed_dev(const float* d_table, size_t n_vocab, size_t d, const int* d_tok, size_t rows, float* d_out,
                 void* stream) {
  if (!d_table || !d_tok || !d_out) return fail(RE_ERR_ARG, "null pointer");
  if (rows == 0) return RE_OK;
  if (d == 0 || rows > (1u << 24) || n_vocab == 0 || n_vocab > (1u << 30))
    return fail(RE_ERR_SIZE, "embed shape %zu x %zu of %zu tokens", rows, d, n_vocab);
  HIP_TRY(launch_embed(d_table, (int)n_vocab, (int)d, d_tok, (int)rows, d_out, (hipStream_t)stream));
  return RE_OK;
}

int re_pos_add_dev(int* d_pos, int delta, void* stream) {
  if (!d_pos) return fail(RE_ERR_ARG, "null pointer");
  HIP_TRY(launch_pos_add(d_pos, delta, (hipStream_t)stream));
  return RE_OK;
}

int re_ffn_create(re_qmat* gate, re_qmat* up, re_ffn** out) {
  if (!gate || !up || !out) return fail(RE_ERR_ARG, "null pointer");
  *out = nullptr;
  if (gate->dense != up->dense) return fail(RE_ERR_TYPE, "ffn: gate and up both quantized or both dense");
  if (gate->g.type != up->g.type || gate->g.m != up->g.m || gate->g.n != up->g.n)
    return fail(RE_ERR_SIZE, "ffn: gate and up must share type and shape");
  if (!gate->dense && gate->g.n > (size_t)kGemvRowsMaxK)
    return fail(RE_ERR_SIZE, "ffn: rows longer than %d", kGemvRowsMaxK);
  re_ffn* f = new (std::nothrow) re_ffn();
  if (!f) return fail(RE_ERR_ARG, "out of memory");
  f->gate = gate;
  f->up = up;
  if (gate->dense) {
    // dense weights: RMS-norm, the two products and SwiGLU as four launches, through a buffer
    // owned by the pair (so a captured decode step allocates nothing)
    auto pad = [](size_t v) { return (v + 63) / 64 * 64; };
    f->x_off = 0;
    f->g_off = pad(gate->g.n);
    f->u_off = f->g_off + pad(gate->g.m);
    if (hipMalloc(&f->d_tmp, (f->u_off + pad(gate->g.m)) * sizeof(float)) != hipSuccess) {
      delete f;
      return fail(RE_ERR_HIP, "ffn: hipMalloc failed");
    }
  }
  // one workgroup per kFfnGemvRows weight rows; the kernel derives its rows from the workgroup
  // index (no task list to load)
  f->ntasks = (int)((gate->g.m + kFfnGemvRows - 1) / kFfnGemvRows);
  *out = f;
  return RE_OK;
}

void re_ffn_destroy(re_ffn* f) {
  if (!f) return;
  if (f->d_tmp) {
    (void)hipDeviceSynchronize();
    (void)hipFree(f->d_tmp);
  }
  delete f;
}

int re_ffn_forward_dev(re_ffn* f, const float* d_x, const float* d_norm_w, float eps, float* d_h, void* stream) {
  if (!f || !d_x || !d_h) return fail(RE_ERR_ARG, "null pointer");
  if (!aligned16(d_x) || !aligned16(d_norm_w)) return fail(RE_ERR_ARG, "x and norm weights must be 16-byte aligned");
  if (f->gate->dense) {
    const hipStream_t s = (hipStream_t)stream;
    const int m = (int)f->gate->g.m, n = (int)f->gate->g.n;
    const float* xin = d_x;
    if (d_norm_w) {
      HIP_TRY(launch_rmsnorm(d_x, d_norm_w, 1, n, eps, f->d_tmp + f->x_off, s));
      xin = f->d_tmp + f->x_off;
    }
    float* gy = f->d_tmp + f->g_off;
    float* uy = f->d_tmp + f->u_off;
    HIP_TRY(launch_dense_gemm(f->gate->g.type, f->gate->d_w, xin, gy, m, n, 1, nullptr, RE_MODE_F32, nullptr, nullptr,
                              1, s));
    HIP_TRY(launch_dense_gemm(f->up->g.type, f->up->d_w, xin, uy, m, n, 1, nullptr, RE_MODE_F32, nullptr, nullptr, 1,
                              s));
    HIP_TRY(launch_swiglu(gy, uy, d_h, (size_t)m, s));
    return RE_OK;
  }
  MoeGemvArgs g{};
  g.rows_per_task = kFfnGemvRows;
  g.norm_w = d_norm_w;
  g.norm_eps = eps;
  g.W0 = f->gate->d_w;
  g.W1 = f->up->d_w;
  g.w_stride = 0;
  g.X = d_x;
  g.xrow = nullptr;
  g.Y = d_h;
  g.tasks = nullptr;                    // rows from the workgroup index
  g.m = (int)f->gate->g.m;
  g.K = (int)f->gate->g.n;
  g.KB = (int)f->gate->g.kb;
  g.ldy = (int)f->gate->g.m;
  g.max_rows = 1;
  HIP_TRY(launch_moe_gemv(f->gate->g.type, true, g, f->ntasks, (hipStream_t)stream));
  return RE_OK;
}

}  // extern "C"
