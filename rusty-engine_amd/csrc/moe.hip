// MoE epilogue kernels: SwiGLU between the gate/up and down projections, and the weighted
// combine of the routed expert outputs (src/moe.rs:280-283, 376-383).
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace rehip {

// h = silu(g) * u, silu(x) = x * (1 / (1 + exp(-x)))  (moe.rs:44-51, 280-283)
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ h, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float x = g[i];
  const float sig = __frcp_rn(__fadd_rn(1.0f, expf(-x)));
  h[i] = __fmul_rn(__fmul_rn(x, sig), u[i]);
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

}  // namespace rehip
