// MoE kernels: SwiGLU between the gate/up and down projections, the weighted combine of the
// routed expert outputs (src/moe.rs:280-283, 376-383), and the grouped expert GEMV used when
// the experts receive few rows each.
#include <hip/hip_runtime.h>

#include "deq.hpp"
#include "kernels.hpp"

namespace rehip {

__device__ __forceinline__ float silu_mul(float x, float u) {
  const float sig = __frcp_rn(__fadd_rn(1.0f, expf(-x)));
  return __fmul_rn(__fmul_rn(x, sig), u);
}

// h = silu(g) * u, silu(x) = x * (1 / (1 + exp(-x)))  (moe.rs:44-51, 280-283)
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ h, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  h[i] = silu_mul(g[i], u[i]);
}

// out[t][c] = sum over j = 0..k-1, in order, of w[t*k+j] * yp[pos[t*k+j]][c]; the sum starts
// from 0 and every step is a rounded multiply then a rounded add (moe.rs:376-383).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ yp, const int* __restrict__ pos,
                                                      const float* __restrict__ w, float* __restrict__ out,
                                                      int k, int hidden) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= hidden) return;
  float o = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int p = pos[t * k + j];
    o = __fadd_rn(o, __fmul_rn(w[t * k + j], yp[(size_t)p * hidden + c]));
  }
  out[(size_t)t * hidden + c] = o;
}

hipError_t launch_swiglu(const float* g, const float* u, float* h, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, h, n);
  return hipGetLastError();
}

hipError_t launch_combine(const float* yp, const int* pos, const float* w, float* out, int tokens, int k,
                          int hidden, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((hidden + 255) / 256), (unsigned)tokens), dim3(256), 0, s,
                     yp, pos, w, out, k, hidden);
  return hipGetLastError();
}


// Grouped expert GEMV for experts that receive at most NB gathered rows per task (decode-sized
// batches). A task is (expert, R weight rows starting at row0, gathered rows p0..p0+np-1). The
// workgroup stages the np activation rows (and their per-16 sums) in LDS; lane l of a wave
// serves weight row l % R, and the 64/R lane groups of every wave take the row's 32-quant units
// in turn (the row-group GEMV mapping). Each decoded run is dotted with all np rows, so a weight
// is read once per task. DUAL: the gate and up matrices are read side by side and the task
// writes silu(gate) * up (SwiGLU, moe.rs:280-283) directly. Sums fold over lane groups by a
// fixed xor tree and over waves in wave order (deterministic).
template <int T, int R, int WAVES, int NB, bool DUAL>
__global__ __launch_bounds__(WAVES * 64) void moe_gemv_kernel(MoeGemvArgs a) {
  using B = Blk<T>;
  constexpr int NCH = B::NCH;
  constexpr int D = 2;                   // units in flight per slot
  constexpr int G = 64 / R;
  constexpr int S = WAVES * G;
  constexpr int NM = DUAL ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const MoeGemvTask task = a.tasks[blockIdx.x];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KP = a.KB * B::QK;
  float* xl = smem;                      // [NB][KP]
  float* xs16 = smem + NB * KP;          // [NB][KP/16]
  float* red = xs16 + NB * (KP / 16);    // [WAVES][NM][NB][R]
  float* ssred = red + WAVES * NM * NB * R;   // [WAVES][NB]

  const int row = task.row0 + (lane % R);          // weight row inside the expert
  const int tile = row >> 6, rr = row & 63;
  const size_t wofs = (size_t)task.expert * a.w_stride + (size_t)tile * a.KB * B::SLAB;
  const uint8_t* t0 = a.W0 + wofs;
  const uint8_t* t1 = DUAL ? a.W1 + wofs : nullptr;
  const int slot = wave * G + lane / R;
  const int u_end = a.KB * NCH;

  typename B::CR ring0[D], ring1[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int u = slot + i * S;
    if (u < u_end) {
      B::load_chunk(t0 + (size_t)(u / NCH) * B::SLAB, rr, u % NCH, ring0[i]);
      if constexpr (DUAL) B::load_chunk(t1 + (size_t)(u / NCH) * B::SLAB, rr, u % NCH, ring1[i]);
    }
  }

  // stage the task's activation rows (zero past K and past np); with an RMS-norm, x * w is
  // staged, each thread keeps its rows' sums of squares, and 1/rms scales the finished dots
  const int nv = KP / 4;
  float ss[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) ss[nb] = 0.0f;
  for (int i = threadIdx.x; i < NB * nv; i += WAVES * 64) {
    const int nb = i / nv, k = 4 * (i - nb * nv);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (nb < task.np && k < a.K) {
      const int p = task.p0 + nb;
      const int xr = a.xrow ? a.xrow[p] : p;
      v = *reinterpret_cast<const float4*>(a.X + (size_t)xr * a.K + k);
      if (a.norm_w) {
        float t = __builtin_fmaf(v.x, v.x, __builtin_fmaf(v.y, v.y, __builtin_fmaf(v.z, v.z, v.w * v.w)));
#pragma unroll
        for (int q = 0; q < NB; ++q)
          if (q == nb) ss[q] += t;
        const float4 w = *reinterpret_cast<const float4*>(a.norm_w + k);
        v = make_float4(v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w);
      }
    }
    reinterpret_cast<float4*>(xl)[i] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NB * (KP / 16); i += WAVES * 64) {
    const float4* q = reinterpret_cast<const float4*>(xl + 16 * i);
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) { const float4 t = q[v]; sum += t.x; sum += t.y; sum += t.z; sum += t.w; }
    xs16[i] = sum;
  }
  __syncthreads();

  float acc[NM][NB];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[m][nb] = 0.0f;
  for (int base = slot; base < u_end; base += D * S) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int u = base + i * S;
      if (u < u_end) {
        const int kb = u / NCH, c = u - kb * NCH;
        Run a0, b0, a1, b1;
        B::decode_chunk(ring0[i], c, a0, b0);
        if constexpr (DUAL) B::decode_chunk(ring1[i], c, a1, b1);
        const int un = u + D * S;
        if (un < u_end) {
          B::load_chunk(t0 + (size_t)(un / NCH) * B::SLAB, rr, un % NCH, ring0[i]);
          if constexpr (DUAL) B::load_chunk(t1 + (size_t)(un / NCH) * B::SLAB, rr, un % NCH, ring1[i]);
        }
        const int valid = a.K - kb * B::QK;   // K is a multiple of 32: a run is wholly in or out
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          if (nb >= task.np) break;            // uniform: the task's row count
          const float* xb = xl + nb * KP + kb * B::QK;
          const float* xs = xs16 + nb * (KP / 16) + kb * (B::QK / 16);
          if (a0.e < valid) acc[0][nb] += run_dot<T>(a0, xb, xs);
          if (b0.e < valid) acc[0][nb] += run_dot<T>(b0, xb, xs);
          if constexpr (DUAL) {
            if (a1.e < valid) acc[NM - 1][nb] += run_dot<T>(a1, xb, xs);
            if (b1.e < valid) acc[NM - 1][nb] += run_dot<T>(b1, xb, xs);
          }
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float v = acc[m][nb];
#pragma unroll
      for (int off = R; off < 64; off *= 2) v += __shfl_xor(v, off, 64);
      if (lane < R) red[((wave * NM + m) * NB + nb) * R + lane] = v;
    }
  if (a.norm_w) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float t = ss[nb];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
      if (lane == 0) ssred[wave * NB + nb] = t;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < R * NB) {
    const int r = threadIdx.x % R, nb = threadIdx.x / R;
    float inv = 1.0f;
    if (a.norm_w) {
      float t = ssred[nb];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) t += ssred[w * NB + nb];
      inv = 1.0f / sqrtf(t / (float)a.K + a.norm_eps);
    }
    float v[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      float sum = red[((0 * NM + m) * NB + nb) * R + r];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) sum += red[((w * NM + m) * NB + nb) * R + r];
      v[m] = a.norm_w ? sum * inv : sum;
    }
    const int wrow = task.row0 + r;
    if (nb < task.np && wrow < a.m) {
      float* y = a.Y + (size_t)(task.p0 + nb) * a.ldy + wrow;
      *y = DUAL ? silu_mul(v[0], v[NM - 1]) : v[0];
    }
  }
}

template <int T, bool DUAL, int NB>
static hipError_t launch_moe_gemv_nb(const MoeGemvArgs& a, int ntasks, hipStream_t s) {
  constexpr int R = kMoeGemvRows, W = kMoeGemvWaves;
  const int KP = a.KB * Blk<T>::QK;
  const size_t lds = ((size_t)NB * KP * 17 / 16 + (size_t)W * (DUAL ? 2 : 1) * NB * R + (size_t)W * NB) * sizeof(float);
  hipLaunchKernelGGL((moe_gemv_kernel<T, R, W, NB, DUAL>), dim3((unsigned)ntasks), dim3(W * 64), lds, s, a);
  return hipGetLastError();
}

// tasks of at most one gathered row use the single-row instance (no idle activation slots)
template <int T, bool DUAL>
static hipError_t launch_moe_gemv_t(const MoeGemvArgs& a, int ntasks, hipStream_t s) {
  return a.max_rows <= 1 ? launch_moe_gemv_nb<T, DUAL, 1>(a, ntasks, s)
                         : launch_moe_gemv_nb<T, DUAL, kMoeGemvBatch>(a, ntasks, s);
}

hipError_t launch_moe_gemv(uint32_t type, bool dual, const MoeGemvArgs& a, int ntasks, hipStream_t s) {
  if (ntasks == 0) return hipSuccess;
  switch (type) {
    case T_Q4_0: return dual ? launch_moe_gemv_t<T_Q4_0, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q4_0, false>(a, ntasks, s);
    case T_Q5_0: return dual ? launch_moe_gemv_t<T_Q5_0, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q5_0, false>(a, ntasks, s);
    case T_Q8_0: return dual ? launch_moe_gemv_t<T_Q8_0, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q8_0, false>(a, ntasks, s);
    case T_Q4_K: return dual ? launch_moe_gemv_t<T_Q4_K, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q4_K, false>(a, ntasks, s);
    case T_Q5_K: return dual ? launch_moe_gemv_t<T_Q5_K, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q5_K, false>(a, ntasks, s);
    case T_Q6_K: return dual ? launch_moe_gemv_t<T_Q6_K, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q6_K, false>(a, ntasks, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rehip
