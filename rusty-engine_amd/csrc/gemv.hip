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

// x comes from LDS: every lane of the wave reads the same address (a broadcast), so a run of
// 16 activations is four ds_read_b128.
template <int T, bool GUARD>
__device__ __forceinline__ float block_dot(const typename Blk<T>::R& r, const float* __restrict__ xb,
                                           const float* __restrict__ xs, int valid) {
  using B = Blk<T>;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < B::NCH; ++c) {
    // one chunk's 32 activations live at a time: stops the scheduler from hoisting all of a
    // super-block's LDS reads (256 values) above the first chunk
    if (B::NCH > 1) asm volatile("" ::: "memory");
    Run a, b;
    B::decode(r, c, a, b);
    // ... and the same for the quant-to-float conversions: pin this chunk's quant words here
    if (B::NCH > 1)
      asm volatile("" : "+v"(a.q[0]), "+v"(a.q[1]), "+v"(a.q[2]), "+v"(a.q[3]),
                        "+v"(b.q[0]), "+v"(b.q[1]), "+v"(b.q[2]), "+v"(b.q[3]));
    // K is a multiple of 32, so a 16-element run is either wholly inside K or wholly past it
    if (!GUARD || a.e < valid) {
      const float4* xv = reinterpret_cast<const float4*>(xb + a.e);
      float sa = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float4 q = xv[v];
        sa = __builtin_fmaf(qbyte(a.q, 4 * v + 0), q.x, sa);
        sa = __builtin_fmaf(qbyte(a.q, 4 * v + 1), q.y, sa);
        sa = __builtin_fmaf(qbyte(a.q, 4 * v + 2), q.z, sa);
        sa = __builtin_fmaf(qbyte(a.q, 4 * v + 3), q.w, sa);
      }
      acc += __builtin_fmaf(a.scale, sa, -a.offset * xs[a.e >> 4]);
    }
    if (!GUARD || b.e < valid) {
      const float4* xv = reinterpret_cast<const float4*>(xb + b.e);
      float sb = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float4 q = xv[v];
        sb = __builtin_fmaf(qbyte(b.q, 4 * v + 0), q.x, sb);
        sb = __builtin_fmaf(qbyte(b.q, 4 * v + 1), q.y, sb);
        sb = __builtin_fmaf(qbyte(b.q, 4 * v + 2), q.z, sb);
        sb = __builtin_fmaf(qbyte(b.q, 4 * v + 3), q.w, sb);
      }
      acc += __builtin_fmaf(b.scale, sb, -b.offset * xs[b.e >> 4]);
    }
  }
  return acc;
}

template <int T, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs p) {
  using B = Blk<T>;
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

  // the first block's planes go out before anything else
  const uint8_t* tbase = p.W + (size_t)tile * p.KB * B::SLAB;
  int kb = kb0 + wave;
  typename B::R cur, nxt;
  if (kb < kb1) B::load(tbase + (size_t)kb * B::SLAB, lane, cur);

  // stage this split's x (float4, zero past K) and its per-16 sums
  const int x0 = kb0 * B::QK;
  const int nv = (kb1 - kb0) * B::QK / 4;
  for (int i = threadIdx.x; i < nv; i += WAVES * 64) {
    const int k = x0 + 4 * i;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (k < p.K) v = *reinterpret_cast<const float4*>(p.x + k);
    reinterpret_cast<float4*>(xl)[i] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nv / 4; i += WAVES * 64) {
    const float4* q = reinterpret_cast<const float4*>(xl + 16 * i);
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) { const float4 t = q[v]; s += t.x; s += t.y; s += t.z; s += t.w; }
    xs16[i] = s;
  }
  __syncthreads();

  const int kb_full = min(kb1, p.K / B::QK);   // columns with no element beyond K
  float acc = 0.0f;
  // software pipeline: the planes of the next block column are in flight while this one
  // is decoded
  for (; kb < kb1; kb += WAVES) {
    const int kn = kb + WAVES;
    if (kn < kb1) B::load(tbase + (size_t)kn * B::SLAB, lane, nxt);
    const float* xb = xl + (kb - kb0) * B::QK;
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
  // acquire: the agent-scope fence invalidates this CU's vector L1, so the plain loads below
  // see every split's partial (all published before their arrival increment)
  __atomic_thread_fence(__ATOMIC_ACQUIRE);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (wave == 0) {
    const float* part = p.partial + row;
    float s = 0.0f;
    for (int sp = 0; sp < p.splits; ++sp) s += part[(size_t)sp * p.m_pad];
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
  const int nx = a.kb_per_split * Blk<T>::QK;
  const int xs = nx + nx / 16;
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
