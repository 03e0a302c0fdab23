// Decode GEMV (N = 1) and the bit-exact dequant kernel over the tiled-slab layout.
//
// GEMV mapping: a workgroup owns one 64-row tile; lane r of every wave owns row r of the tile,
// so no cross-lane reduction is needed. The waves of a workgroup, and optionally several
// workgroups ("splits"), divide the tile's block columns. x is wave-uniform (every lane reads the
// same element), so it is fetched with scalar loads; only the weight planes use vector loads,
// each a contiguous 1 KiB (16-byte planes) / 256 B / 128 B per wavefront.
//
// Per block the lane decodes chunk after chunk (deq.hpp) and folds
//   scale * sum(q_i x_i) - offset * sum(x_i)
// where sum(x_i) over each 16-element run comes from a per-workgroup table in LDS.
//
// Split reduction is deterministic: each split writes its partial row sums, the last workgroup
// of a tile (arrival counter) adds the partials in split order, writes y and re-arms the
// counter for the next launch.
#include <hip/hip_runtime.h>

#include "deq.hpp"
#include "kernels.hpp"

namespace rehip {

// x is read through the constant address space: it is not written while a kernel runs, and
// wave-uniform loads from that space compile to scalar loads (s_load) into SGPRs.
typedef const __attribute__((address_space(4))) float cfloat;

template <int T, bool GUARD>
__device__ __forceinline__ float block_dot(const typename Blk<T>::R& r, cfloat* __restrict__ xb,
                                           const float* __restrict__ xs, int valid) {
  using B = Blk<T>;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < B::NCH; ++c) {
    // keeps each chunk's wave-uniform x loads (scalar loads) next to their use, so a
    // 256-element super-block never holds all of its x in SGPRs at once
    if (B::NCH > 1) asm volatile("" ::: "memory");
    Run a, b;
    B::decode(r, c, a, b);
    // K is a multiple of 32, so a 16-element run is either wholly inside K or wholly past it
    if (!GUARD || a.e < valid) {
      float sa = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) sa = __builtin_fmaf(qbyte(a.q, i), xb[a.e + i], sa);
      acc += __builtin_fmaf(a.scale, sa, -a.offset * xs[a.e >> 4]);
    }
    if (!GUARD || b.e < valid) {
      float sb = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) sb = __builtin_fmaf(qbyte(b.q, i), xb[b.e + i], sb);
      acc += __builtin_fmaf(b.scale, sb, -b.offset * xs[b.e >> 4]);
    }
  }
  return acc;
}

template <int T, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs p) {
  using B = Blk<T>;
  extern __shared__ float smem[];          // xs16[kb_per_split * QK/16], then red[WAVES*64]
  const int tile = blockIdx.x;
  const int split = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kb0 = split * p.kb_per_split;
  const int kb1 = min(p.KB, kb0 + p.kb_per_split);
  float* xs16 = smem;
  float* red = smem + p.kb_per_split * (B::QK / 16);

  // per-16 sums of x over this split's columns (zero beyond K)
  const int n16 = (kb1 - kb0) * (B::QK / 16);
  for (int i = threadIdx.x; i < n16; i += WAVES * 64) {
    const int k = kb0 * B::QK + 16 * i;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += (k + j < p.K) ? p.x[k + j] : 0.0f;
    xs16[i] = s;
  }
  __syncthreads();

  const uint8_t* tbase = p.W + (size_t)tile * p.KB * B::SLAB;
  const int kb_full = min(kb1, p.K / B::QK);   // columns with no element beyond K
  float acc = 0.0f;
  int kb = kb0 + wave;
  // software pipeline: the planes of the next block column are in flight while this one
  // is decoded
  typename B::R cur, nxt;
  if (kb < kb1) B::load(tbase + (size_t)kb * B::SLAB, lane, cur);
  for (; kb < kb1; kb += WAVES) {
    const int kn = kb + WAVES;
    if (kn < kb1) B::load(tbase + (size_t)kn * B::SLAB, lane, nxt);
    cfloat* xb = (cfloat*)(p.x + (size_t)kb * B::QK);
    const float* xs = xs16 + (kb - kb0) * (B::QK / 16);
    if (kb < kb_full) acc += block_dot<T, false>(cur, xb, xs, B::QK);
    else acc += block_dot<T, true>(cur, xb, xs, p.K - kb * B::QK);
    cur = nxt;
  }

  // fixed-order reduction over the waves
  red[threadIdx.x] = acc;
  __syncthreads();
  const int row = tile * 64 + lane;
  if (p.splits == 1) {
    if (wave == 0) {
      float s = red[lane];
      for (int w = 1; w < WAVES; ++w) s += red[w * 64 + lane];
      if (row < p.m) p.y[row] = s;
    }
    return;
  }
  if (wave == 0) {
    float s = red[lane];
    for (int w = 1; w < WAVES; ++w) s += red[w * 64 + lane];
    p.partial[(size_t)split * p.m_pad + row] = s;
  }
  __threadfence();
  __syncthreads();
  __shared__ int last;
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(&p.counters[tile], 1u);
    last = (prev == (unsigned)(p.splits - 1));
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (wave == 0) {
    float s = 0.0f;
    for (int sp = 0; sp < p.splits; ++sp)
      s += __hip_atomic_load(&p.partial[(size_t)sp * p.m_pad + row], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    if (row < p.m) p.y[row] = s;
  }
  if (threadIdx.x == 0) p.counters[tile] = 0u;
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

template <int T>
static hipError_t launch_gemv_t(const GemvArgs& a, int waves, hipStream_t s) {
  const int xs = a.kb_per_split * (Blk<T>::QK / 16);
  dim3 grid((unsigned)a.tiles, (unsigned)a.splits);
  if (waves == 4) {
    const size_t shm = (size_t)(xs + 4 * 64) * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<T, 4>), grid, dim3(256), shm, s, a);
  } else {
    const size_t shm = (size_t)(xs + 64) * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<T, 1>), grid, dim3(64), shm, s, a);
  }
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
