// Decode GEMV (N = 1) and the bit-exact dequant kernel over the tiled-slab layout.
//
// GEMV mapping: a workgroup owns one 64-row tile; lane r of every wave owns row r of the tile,
// so no cross-lane reduction is needed. The waves of a workgroup, and optionally several
// workgroups ("splits"), divide the tile's block columns. x is wave-uniform (every lane reads the
// same element), so it is fetched with scalar loads; only the weight planes use vector loads,
// each a contiguous 1 KiB (16-byte planes) / 256 B / 128 B per wavefront.
//
// Per 32-quant chunk the lane folds
//   scale * sum(q_i x_i) - offset * sum(x_i)
// where sum(x_i) over each 16-element run comes from a per-workgroup table in LDS.
//
// Long rows of small matrices are split over several workgroups so the whole chip works on
// them. Each split writes its partial row sums with plain stores and a second small kernel adds
// them in split order (deterministic): the kernel boundary publishes the partials, which is far
// cheaper on gfx950 than an agent-scope release per workgroup (an L2 write-back).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "deq.hpp"
#include "kernels.hpp"

namespace rehip {

// Work unit = one 32-quant chunk (two 16-element runs) of one block column for the 64 rows of
// a tile. Units of a tile are numbered u = kb * NCH + c; a workgroup owns the units of its
// block-column range, its waves take every WAVES-th unit, and each wave keeps DEPTH units'
// raw planes in flight (a ring of registers) so small matrices issue every load up front.
constexpr int kGemvDepth = 4;

template <int T, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs p) {
  using B = Blk<T>;
  constexpr int NCH = B::NCH;
  constexpr int D = kGemvDepth;
  // LDS: x[kb_per_split * QK] (zero past K), xs16[kb_per_split * QK / 16], red[WAVES * 64]
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int tile = blockIdx.x;
  const int split = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kb0 = split * p.kb_per_split;
  const int kb1 = min(p.KB, kb0 + p.kb_per_split);
  const int nx = p.kb_per_split * B::QK;
  float* xl = smem;
  float* xs16 = smem + nx;
  float* red = xs16 + nx / 16;

  // the first DEPTH units' planes go out before anything else
  const uint8_t* tbase = p.W + (size_t)tile * p.KB * B::SLAB;
  const int u_end = kb1 * NCH;
  const int u0 = kb0 * NCH + wave;
  // ring loads go through a buffer resource over the tile: a chunk past the end reads at an
  // offset past the resource (zeros, no memory traffic) instead of being skipped under a branch,
  // which made the compiler wait for each load where the branch joins (one round trip per entry)
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(tbase, (uint32_t)p.KB * (uint32_t)B::SLAB);
  auto load = [&](int u, typename B::CR& r) {
    const uint32_t off = u < u_end ? (uint32_t)(u / NCH) * (uint32_t)B::SLAB : 0x80000000u;
    B::bload_chunk(wr, off, lane, u % NCH, r);
  };
  typename B::CR ring[D];
#pragma unroll
  for (int i = 0; i < D; ++i) load(u0 + i * WAVES, ring[i]);

  // stage this split's x (float4, zero past K) and its per-16 sums
  const int x0 = kb0 * B::QK;
  const int nv = (kb1 - kb0) * B::QK / 4;
  float inv = 1.0f;
  if (p.norm_w) {                        // RMS over the whole row (every split reads all of x)
    float ss = 0.0f;
    for (int k = threadIdx.x; k < p.K; k += WAVES * 64) ss = __builtin_fmaf(p.x[k], p.x[k], ss);
    ss = wg_sum<WAVES>(ss, red);
    inv = 1.0f / sqrtf(ss / (float)p.K + p.norm_eps);
  }
  for (int i = threadIdx.x; i < nv; i += WAVES * 64) {
    const int k = x0 + 4 * i;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (k < p.K) {
      v = *reinterpret_cast<const float4*>(p.x + k);
      if (p.norm_w) {
        const float4 w = *reinterpret_cast<const float4*>(p.norm_w + k);
        v = make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
      }
    }
    reinterpret_cast<float4*>(xl)[i] = v;
  }
  __syncthreads();
  if constexpr (kNeedXs16<T>) {   // per-16 sums of x: only the dots that take out an offset use them
    for (int i = threadIdx.x; i < nv / 4; i += WAVES * 64) {
      const float4* q = reinterpret_cast<const float4*>(xl + 16 * i);
      float s = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) { const float4 t = q[v]; s += t.x; s += t.y; s += t.z; s += t.w; }
      xs16[i] = s;
    }
    __syncthreads();
  }

  float acc = 0.0f;
  for (int base = u0; base < u_end; base += D * WAVES) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int u = base + i * WAVES;
      if (u < u_end) {
        const int kb = u / NCH, c = u - kb * NCH;
        Run a, b;
        B::decode_chunk(ring[i], c, a, b);
        const int un = u + D * WAVES;
        if (un < u_end) load(un, ring[i]);
        const float* xb = xl + (kb - kb0) * B::QK;
        const float* xs = xs16 + (kb - kb0) * (B::QK / 16);
        const int valid = p.K - kb * B::QK;   // K is a multiple of 32: a run is wholly in or out
        if (a.e < valid) acc += run_dot<T>(a, xb, xs);
        if (b.e < valid) acc += run_dot<T>(b, xb, xs);
      }
    }
  }

  // fixed-order reduction over the waves
  red[threadIdx.x] = acc;
  __syncthreads();
  if (wave == 0) {
    float s = red[lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) s += red[w * 64 + lane];
    const int row = tile * 64 + lane;
    if (p.splits == 1) {
      unsigned long long key = 0;
      if (row < p.m) {
        const float y = p.add ? s + p.add[row] : s;
        p.y[row] = y;
        key = argmax_key(y, row);
      }
      if (p.best) wave_argmax_fold(key, p.best);
    } else {
      p.partial[(size_t)split * p.m_pad + row] = s;
    }
  }
}

// Row-group GEMV: a workgroup owns R consecutive rows of one 64-row tile (R = 64, 16, 8 or 4)
// and the whole row length, so a matrix with few rows still spreads over hundreds of
// workgroups and needs no second reduction kernel. Lane l of a wave serves row l % R of the
// group; the 64 / R lane groups of every wave ("slots") take the units of the row in turn, so
// one load instruction reads 64 / R runs of R * 16 contiguous bytes. Partial sums are folded
// over the lane groups with a fixed xor-shuffle tree, then over the waves in wave order
// (deterministic). Row groups that share cache lines are given to the same XCD (workgroup w
// runs on XCD w % 8).
// ONE: every slot has at most one chunk (KB * NCH <= slots per workgroup, the usual case for
// decode-sized matrices): a one-entry ring, no refill.
template <int T, int R, int WAVES, bool ONE>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_kernel(GemvArgs p) {
  using B = Blk<T>;
  constexpr int NCH = B::NCH;
  constexpr int D = ONE ? 1 : (WAVES == 16 ? 2 : kGemvDepth);   // 16 waves: 128 VGPRs per lane
  constexpr int G = 64 / R;              // lane groups per wave
  constexpr int S = WAVES * G;           // slots per workgroup
  // LDS: x[KB * QK] (zero past K), xs16[KB * QK / 16], red[WAVES * R], ssred[WAVES]
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int nb = p.batch > 1 ? p.batch : 1;
  const int per = (p.groups * nb + 7) / 8;
  const int gq = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (gq >= p.groups * nb) return;
  const int mb = gq / p.groups, gi = gq - mb * p.groups;     // matrix of the stack, its row group
  const float* xin = p.x + (size_t)mb * p.x_stride;
  float* yout = p.y + (size_t)mb * p.y_stride;
  constexpr int GPT = 64 / R;            // row groups per tile
  const int tile = gi / GPT;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rr = (gi - tile * GPT) * R + (lane % R);    // row inside the tile
  const int slot = wave * G + lane / R;
  const int nx = p.KB * B::QK;
  float* xl = smem;
  float* xs16 = smem + nx;
  float* red = xs16 + nx / 16;
  float* ssred = red + WAVES * R;

  const uint8_t* tbase = p.W + (size_t)mb * p.w_stride + (size_t)tile * p.KB * B::SLAB;
  const int u_end = p.KB * NCH;
  // this thread's first activation (and norm weight) goes out before the weight loads: loads
  // retire in order, so the staging below then waits for it alone and overlaps the weights'
  // round trip
  const int nv = nx / 4;
  float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), w0 = x0;
  if ((int)threadIdx.x < nv && 4 * (int)threadIdx.x < p.K) {
    x0 = *reinterpret_cast<const float4*>(xin + 4 * threadIdx.x);
    if (p.norm_w) w0 = *reinterpret_cast<const float4*>(p.norm_w + 4 * threadIdx.x);
  }
  __builtin_amdgcn_sched_barrier(0);
  // ring loads through a buffer resource over the tile, as in gemv_kernel: a slot past the end
  // reads at an offset past the resource (no branch, one round trip for the whole ring)
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(tbase, (uint32_t)p.KB * (uint32_t)B::SLAB);
  auto load = [&](int u, typename B::CR& r) {
    const uint32_t off = u < u_end ? (uint32_t)(u / NCH) * (uint32_t)B::SLAB : 0x80000000u;
    B::bload_chunk(wr, off, rr, u % NCH, r);
  };
  typename B::CR ring[D];
#pragma unroll
  for (int i = 0; i < D; ++i) load(slot + i * S, ring[i]);
  __builtin_amdgcn_sched_barrier(0);

  // RMS-norm prologue: x * w is staged and the sum of squares kept per thread; the row's
  // 1/rms multiplies the finished dot (W (x inv w) = inv W (x w)), so the norm adds no pass or
  // barrier before the weights are consumed.
  float ss = 0.0f;
  for (int i = threadIdx.x; i < nv; i += WAVES * 64) {
    const int k = 4 * i;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (k < p.K) {
      const bool first = i == (int)threadIdx.x;
      v = first ? x0 : *reinterpret_cast<const float4*>(xin + k);
      if (p.norm_w) {
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
        const float4 w = first ? w0 : *reinterpret_cast<const float4*>(p.norm_w + k);
        v = make_float4(v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w);
      }
    }
    reinterpret_cast<float4*>(xl)[i] = v;
  }
  __syncthreads();
  if constexpr (kNeedXs16<T>) {   // per-16 sums of x: only the dots that take out an offset use them
    for (int i = threadIdx.x; i < nv / 4; i += WAVES * 64) {
      const float4* q = reinterpret_cast<const float4*>(xl + 16 * i);
      float s = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) { const float4 t = q[v]; s += t.x; s += t.y; s += t.z; s += t.w; }
      xs16[i] = s;
    }
    __syncthreads();
  }

  float acc = 0.0f;
  for (int base = slot; base < u_end; base += D * S) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int u = base + i * S;
      if (u < u_end) {
        const int kb = u / NCH, c = u - kb * NCH;
        Run a, b;
        B::decode_chunk(ring[i], c, a, b);
        const int un = u + D * S;
        if (!ONE && un < u_end) load(un, ring[i]);
        const float* xb = xl + kb * B::QK;
        const float* xs = xs16 + kb * (B::QK / 16);
        const int valid = p.K - kb * B::QK;   // K is a multiple of 32: a run is wholly in or out
        if (a.e < valid) acc += run_dot<T>(a, xb, xs);
        if (b.e < valid) acc += run_dot<T>(b, xb, xs);
      }
    }
  }

#pragma unroll
  for (int off = R; off < 64; off *= 2) acc += __shfl_xor(acc, off, 64);
  if (lane < R) red[wave * R + lane] = acc;
  if (p.norm_w) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (lane == 0) ssred[wave] = ss;
  }
  __syncthreads();
  if (wave == 0) {
    unsigned long long key = 0;
    float inv = 1.0f;
    if (p.norm_w) {
      float t = ssred[0];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) t += ssred[w];
      inv = 1.0f / sqrtf(t / (float)p.K + p.norm_eps);
    }
    if (lane < R) {
      float s = red[lane];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) s += red[w * R + lane];
      if (p.norm_w) s *= inv;
      const int row = tile * 64 + rr;
      if (row < p.m) {
        const float y = p.add ? s + p.add[row] : s;
        yout[row] = y;
        key = argmax_key(y, row);
      }
    }
    if (p.best) wave_argmax_fold(key, p.best);
  }
}

// Tile GEMV for many tiles (big matrices, stacks of matrices): a workgroup owns one 64-row tile
// (lane = row) and its waves take the tile's steps in turn (one 256-quant super-block, or four
// 32-blocks). A step's planes are loaded whole into registers through a buffer
// resource whose slab offset is a scalar, the next step's loads are in flight while the current
// one is decoded (two register sets, alternated by hand: no copies, no runtime index), and the
// weight loads of the first step go out before x is staged. Blocks past the row's end read as
// zero (resource bound) against zero x, so ragged block counts need no branches. Wave partial
// sums are folded in wave order (deterministic).
// 0, computed from v so that the compiler cannot move what uses it above the arrival of v (the
// x reads of a chunk then wait for the chunk's weights instead of all being hoisted to the top
// of the loop, where their registers would crowd out the weight prefetch)
__device__ __forceinline__ int after_data(uint32_t v) {
  int z;
  asm volatile("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(v));
  return z;
}

template <int T> inline constexpr int kTileStepBlocks = Blk<T>::QK == 256 ? 1 : 4;

template <int T, int WAVES, bool HALF>
__global__ __launch_bounds__(WAVES * 64) void gemv_tile_kernel(GemvArgs p) {
  using B = Blk<T>;
  constexpr int NCH = B::NCH;
  constexpr int G = kTileStepBlocks<T>;            // blocks per step
  constexpr int SQ = G * B::QK;                    // quants per step
  // LDS: x[nsteps * SQ] (zero past K), xs16[nsteps * SQ / 16], red[WAVES * 64], ssred[WAVES]
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int nb = p.batch > 1 ? p.batch : 1;
  const int total = p.tiles * nb;
  const int per = (total + 7) / 8;
  const int gq = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (gq >= total) return;
  const int mb = gq / p.tiles, tile = gq - mb * p.tiles;
  const float* xin = p.x + (size_t)mb * p.x_stride;
  float* yout = p.y + (size_t)mb * p.y_stride;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nsteps = (p.KB + G - 1) / G;
  const int nx = nsteps * SQ;
  float* xl = smem;
  float* xs16 = smem + nx;
  float* red = xs16 + nx / 16;
  float* ssred = red + WAVES * 64;

  const uint8_t* tb = p.W + (size_t)mb * p.w_stride + (size_t)tile * p.KB * B::SLAB;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(tb, (uint32_t)(p.KB * B::SLAB));
  typename B::R r0[G], r1[G];
  auto load_step = [&](int st, typename B::R (&r)[G]) {
#pragma unroll
    for (int g = 0; g < G; ++g) B::sload(rs, (uint32_t)((st * G + g) * B::SLAB), lane, r[g]);
  };
  if (wave < nsteps) {
    if constexpr (B::NCH == 8 && HALF) B::template sload_half<0>(rs, (uint32_t)(wave * B::SLAB), lane, r0[0]);
    else load_step(wave, r0);
  }

  // stage x * norm_w (zero past K) and its per-16 sums; sum of squares per thread
  float ss = 0.0f;
  for (int i = threadIdx.x; i < nx / 4; i += WAVES * 64) {
    const int k = 4 * i;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (k < p.K) {
      v = *reinterpret_cast<const float4*>(xin + k);
      if (p.norm_w) {
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
        const float4 w = *reinterpret_cast<const float4*>(p.norm_w + k);
        v = make_float4(v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w);
      }
    }
    reinterpret_cast<float4*>(xl)[i] = v;
  }
  __syncthreads();
  if constexpr (kNeedXs16<T>) {   // per-16 sums of x: only the dots that take out an offset use them
    for (int i = threadIdx.x; i < nx / 16; i += WAVES * 64) {
      const float4* q = reinterpret_cast<const float4*>(xl + 16 * i);
      float t = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) { const float4 u = q[v]; t += u.x; t += u.y; t += u.z; t += u.w; }
      xs16[i] = t;
    }
    __syncthreads();
  }

  float acc = 0.0f;
  auto step = [&](int st, const typename B::R (&r)[G]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float* xb = xl + (st * G + g) * B::QK;
      const float* xs = xs16 + (st * G + g) * (B::QK / 16);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        Run a, b;
        B::decode(r[g], c, a, b);
        const int z = after_data(__float_as_uint(acc));
        acc += run_dot<T>(a, xb + z, xs + z);
        acc += run_dot<T>(b, xb + z, xs + z);
      }
    }
  };
  if constexpr (B::NCH == 8 && HALF) {
    // super-blocks: the pipeline runs on half blocks (chunks 0-3 / 4-7), so one block's worth
    // of registers keeps the next half in flight
    // one step: its second half loads while the first is consumed, then (PF) the next step's
    // first half while the second is. The last step runs as a copy without the prefetch: with
    // the prefetch under a branch, the two paths left different loads outstanding and the
    // compiler waited for all of them (the prefetch included) before the second half.
    auto half_step = [&](int st, auto pf) {
      const uint32_t so = (uint32_t)(st * B::SLAB);
      B::template sload_half<1>(rs, so, lane, r1[0]);
      __builtin_amdgcn_sched_barrier(0);   // the loads go out before any of the first half's decode
      const float* xb = xl + st * B::QK;
      const float* xs = xs16 + st * (B::QK / 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        Run a, b;
        B::decode(r0[0], c, a, b);
        const int z = after_data(__float_as_uint(acc));
        acc += run_dot<T>(a, xb + z, xs + z);
        acc += run_dot<T>(b, xb + z, xs + z);
      }
      if constexpr (decltype(pf)::value) B::template sload_half<0>(rs, (uint32_t)((st + WAVES) * B::SLAB), lane, r0[0]);
#pragma unroll
      for (int c = 4; c < 8; ++c) {
        Run a, b;
        B::decode(r1[0], c, a, b);
        const int z = after_data(__float_as_uint(acc));
        acc += run_dot<T>(a, xb + z, xs + z);
        acc += run_dot<T>(b, xb + z, xs + z);
      }
    };
    int st = wave;
#pragma unroll 1
    for (; st + WAVES < nsteps; st += WAVES) half_step(st, std::true_type{});
    if (st < nsteps) half_step(st, std::false_type{});
  } else {
    // steady state while both prefetches exist (unconditional: a prefetch under a branch left
    // the two paths with different loads outstanding, and the compiler then waited for all of
    // them, the prefetch included, inside the current step), then the last one or two steps
    int st = wave;
#pragma unroll 1
    for (; st + 2 * WAVES < nsteps; st += 2 * WAVES) {
      load_step(st + WAVES, r1);
      step(st, r0);
      load_step(st + 2 * WAVES, r0);
      step(st + WAVES, r1);
    }
    if (st + WAVES < nsteps) {
      load_step(st + WAVES, r1);
      step(st, r0);
      step(st + WAVES, r1);
    } else if (st < nsteps) {
      step(st, r0);
    }
  }

  red[wave * 64 + lane] = acc;
  if (p.norm_w) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (lane == 0) ssred[wave] = ss;
  }
  __syncthreads();
  if (wave == 0) {
    float sum = red[lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += red[w * 64 + lane];
    if (p.norm_w) {
      float t = ssred[0];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) t += ssred[w];
      sum *= 1.0f / sqrtf(t / (float)p.K + p.norm_eps);
    }
    const int row = tile * 64 + lane;
    unsigned long long key = 0;
    if (row < p.m) {
      const float y = p.add ? sum + p.add[row] : sum;
      yout[row] = y;
      key = argmax_key(y, row);
    }
    if (p.best) wave_argmax_fold(key, p.best);
  }
}

// y[r] = sum over splits, in split order, of partial[split][r]
__global__ __launch_bounds__(256) void gemv_reduce_kernel(const float* __restrict__ partial,
                                                          float* y, int m, int m_pad,
                                                          int splits, const float* add,
                                                          unsigned long long* best) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  unsigned long long key = 0;
  if (r < m) {
    // eight splits' loads in flight at a time, added in split order
    float s = 0.0f;
    int sp = 0;
    for (; sp + 8 <= splits; sp += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = partial[(size_t)(sp + j) * m_pad + r];
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
    }
    for (; sp < splits; ++sp) s += partial[(size_t)sp * m_pad + r];
    const float v = add ? s + add[r] : s;
    y[r] = v;
    key = argmax_key(v, r);
  }
  if (best) wave_argmax_fold(key, best);
}

// Bit-exact dequant of the tiled weights into a row-major f32 matrix [m x n].
template <int T>
__global__ __launch_bounds__(64) void dequant_kernel(const uint8_t* __restrict__ W, float* __restrict__ out,
                                                     int m, int n, int KB) {
  using B = Blk<T>;
  const int tile = blockIdx.x, kb = blockIdx.y, lane = threadIdx.x;
  const int row = tile * 64 + lane;
  if (row >= m) return;
  const uint8_t* slab = W + ((size_t)tile * KB + kb) * B::SLAB;
  float* o = out + (size_t)row * n + (size_t)kb * B::QK;
  const int valid = n - kb * B::QK;
#pragma unroll
  for (int c = 0; c < B::NCH; ++c) {
    Run a, b;
    B::chunk(slab, lane, c, a, b);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (a.e + i < valid) o[a.e + i] = run_value_exact<T>(a, i);
      if (b.e + i < valid) o[b.e + i] = run_value_exact<T>(b, i);
    }
  }
}

template <int T, int R, bool ONE>
static void launch_rows_w(const GemvArgs& a, int waves, unsigned grid, size_t lds, hipStream_t s) {
  if (waves == 16) {
    hipLaunchKernelGGL((gemv_rows_kernel<T, R, 16, ONE>), dim3(grid), dim3(1024), lds, s, a);
  } else if (waves == 8) {
    hipLaunchKernelGGL((gemv_rows_kernel<T, R, 8, ONE>), dim3(grid), dim3(512), lds, s, a);
  } else {
    hipLaunchKernelGGL((gemv_rows_kernel<T, R, 4, ONE>), dim3(grid), dim3(256), lds, s, a);
  }
}

template <int T, int R>
static hipError_t launch_rows(const GemvArgs& a, int waves, hipStream_t s) {
  const size_t lds = ((size_t)a.KB * Blk<T>::QK * 17 / 16 + 16 * R + 16) * sizeof(float);
  const unsigned grid = (unsigned)(((size_t)a.groups * (a.batch > 1 ? a.batch : 1) + 7) / 8 * 8);
  const int w = waves == 16 || waves == 8 ? waves : 4;
  if ((size_t)a.KB * Blk<T>::NCH <= (size_t)w * 64 / R) launch_rows_w<T, R, true>(a, w, grid, lds, s);
  else launch_rows_w<T, R, false>(a, w, grid, lds, s);
  return hipGetLastError();
}

template <int T>
static hipError_t launch_tile(const GemvArgs& a, int waves, hipStream_t s) {
  constexpr int G = kTileStepBlocks<T>;
  constexpr int SQ = G * Blk<T>::QK;
  const size_t nx = (size_t)((a.KB + G - 1) / G) * SQ;
  const unsigned grid = (unsigned)(((size_t)a.tiles * (a.batch > 1 ? a.batch : 1) + 7) / 8 * 8);
  const int w = gemv_tile_waves(waves);
  const size_t lds = (nx + nx / 16 + (size_t)w * 64 + w) * sizeof(float);
  // super-blocks: half-block pipelining pays once a wave has two or more blocks to stream;
  // with one block per wave the whole block is loaded before x is staged
  const bool half = gemv_tile_half(Blk<T>::QK, a.KB, w);
  if (w == 8) {
    if (half) hipLaunchKernelGGL((gemv_tile_kernel<T, 8, true>), dim3(grid), dim3(512), lds, s, a);
    else hipLaunchKernelGGL((gemv_tile_kernel<T, 8, false>), dim3(grid), dim3(512), lds, s, a);
  } else if (w == 2) {
    if (half) hipLaunchKernelGGL((gemv_tile_kernel<T, 2, true>), dim3(grid), dim3(128), lds, s, a);
    else hipLaunchKernelGGL((gemv_tile_kernel<T, 2, false>), dim3(grid), dim3(128), lds, s, a);
  } else {
    if (half) hipLaunchKernelGGL((gemv_tile_kernel<T, 4, true>), dim3(grid), dim3(256), lds, s, a);
    else hipLaunchKernelGGL((gemv_tile_kernel<T, 4, false>), dim3(grid), dim3(256), lds, s, a);
  }
  return hipGetLastError();
}

template <int T>
static hipError_t launch_gemv_t(const GemvArgs& a, int waves, hipStream_t s) {
  if (a.rows_per_group) {
    switch (a.rows_per_group) {
      case 64: return launch_tile<T>(a, waves, s);
      case 16: return launch_rows<T, 16>(a, waves, s);
      case 8: return launch_rows<T, 8>(a, waves, s);
      case 4: return launch_rows<T, 4>(a, waves, s);
      default: return hipErrorInvalidValue;
    }
  }
  const int nx = a.kb_per_split * Blk<T>::QK;
  const int xs = nx + nx / 16;
  dim3 grid((unsigned)a.tiles, (unsigned)a.splits);
  if (waves == 16) {
    hipLaunchKernelGGL((gemv_kernel<T, 16>), grid, dim3(1024), (size_t)(xs + 16 * 64) * sizeof(float), s, a);
  } else if (waves == 8) {
    hipLaunchKernelGGL((gemv_kernel<T, 8>), grid, dim3(512), (size_t)(xs + 8 * 64) * sizeof(float), s, a);
  } else {
    hipLaunchKernelGGL((gemv_kernel<T, 4>), grid, dim3(256), (size_t)(xs + 4 * 64) * sizeof(float), s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  hipLaunchKernelGGL(gemv_reduce_kernel, dim3((unsigned)((a.m + 255) / 256)), dim3(256), 0, s, a.partial, a.y,
                     a.m, a.m_pad, a.splits, a.add, a.best);
  return hipGetLastError();
}

hipError_t launch_gemv(uint32_t type, const GemvArgs& a, int waves, hipStream_t s) {
  switch (type) {
    case T_Q4_0: return launch_gemv_t<T_Q4_0>(a, waves, s);
    case T_Q5_0: return launch_gemv_t<T_Q5_0>(a, waves, s);
    case T_Q8_0: return launch_gemv_t<T_Q8_0>(a, waves, s);
    case T_Q4_K: return launch_gemv_t<T_Q4_K>(a, waves, s);
    case T_Q5_K: return launch_gemv_t<T_Q5_K>(a, waves, s);
    case T_Q6_K: return launch_gemv_t<T_Q6_K>(a, waves, s);
    default: return hipErrorInvalidValue;
  }
}

template <int T>
static hipError_t launch_dequant_t(const uint8_t* W, float* out, int m, int n, int KB, int tiles,
                                   hipStream_t s) {
  hipLaunchKernelGGL((dequant_kernel<T>), dim3((unsigned)tiles, (unsigned)KB), dim3(64), 0, s, W, out, m,
                     n, KB);
  return hipGetLastError();
}

hipError_t launch_dequant(uint32_t type, const uint8_t* W, float* out, int m, int n, int KB, int tiles,
                          hipStream_t s) {
  switch (type) {
    case T_Q4_0: return launch_dequant_t<T_Q4_0>(W, out, m, n, KB, tiles, s);
    case T_Q5_0: return launch_dequant_t<T_Q5_0>(W, out, m, n, KB, tiles, s);
    case T_Q8_0: return launch_dequant_t<T_Q8_0>(W, out, m, n, KB, tiles, s);
    case T_Q4_K: return launch_dequant_t<T_Q4_K>(W, out, m, n, KB, tiles, s);
    case T_Q5_K: return launch_dequant_t<T_Q5_K>(W, out, m, n, KB, tiles, s);
    case T_Q6_K: return launch_dequant_t<T_Q6_K>(W, out, m, n, KB, tiles, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rehip
