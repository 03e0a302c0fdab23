// Device-resident steps of the dense transformer block around the quantized projections
// (src/forward.rs:100-586, src/infer.rs:72-223, src/runner.rs:105-282): RMS-norm, NeoX RoPE,
// K/V cache append, causal GQA attention, residual/bias add, SwiGLU, argmax, embedding gather.
// Positions come from a device integer so that one captured graph serves every decode step.
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace rehip {

// block-wide reductions for 256-thread workgroups (fixed tree: deterministic)
__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// out = x * (1 / sqrt(mean(x^2) + eps)) * w, one workgroup per row (infer.rs:72-82)
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      int d, float eps, float* __restrict__ out) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * d;
  float s = 0.0f;
  for (int i = threadIdx.x; i < d; i += 256) s = __builtin_fmaf(xr[i], xr[i], s);
  s = block_sum256(s, red);
  const float inv = 1.0f / sqrtf(s / (float)d + eps);
  float* o = out + (size_t)blockIdx.x * d;
  for (int i = threadIdx.x; i < d; i += 256) o[i] = xr[i] * inv * w[i];
}

// NeoX rotate-half of head h of row r at position *pos + off + r (infer.rs:90-139):
// angle = p * base^(-2i/d); (x0, x1) -> (x0 c - x1 s, x1 c + x0 s)
__global__ __launch_bounds__(64) void rope_kernel(float* __restrict__ x, int heads, int hd, float base,
                                                  const int* __restrict__ pos, int off) {
  const int r = blockIdx.y, h = blockIdx.x, i = threadIdx.x;
  const int half = hd >> 1;
  if (i >= half) return;
  const float p = (float)(*pos + off + r);
  const float f = 1.0f / powf(base, (float)(2 * i) / (float)hd);
  const float a = p * f;
  const float c = cosf(a), s = sinf(a);
  float* v = x + ((size_t)r * heads + h) * hd;
  const float x0 = v[i], x1 = v[i + half];
  v[i] = x0 * c - x1 * s;
  v[i + half] = x1 * c + x0 * s;
}

__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                        int kv_dim, float* __restrict__ kc, float* __restrict__ vc,
                                                        int max_seq, const int* __restrict__ pos) {
  const int r = blockIdx.x;
  const int row = *pos + r;
  if (row < 0 || row >= max_seq) return;
  const size_t dst = (size_t)row * kv_dim;
  for (int i = threadIdx.x; i < kv_dim; i += 256) {
    kc[dst + i] = k[(size_t)r * kv_dim + i];
    vc[dst + i] = v[(size_t)r * kv_dim + i];
  }
}

// Causal GQA attention for one (query head, query row) per workgroup (forward.rs:232-277):
// scores q.k * (1/sqrt(hd)) over keys 0..p (p = *pos + r), softmax as moe.rs:61-72 (exp of
// x - max, divided by the sum when it is non-zero), then the probability-weighted values.
__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                        const float* __restrict__ vc, int heads, int kv_heads,
                                                        int hd, int max_seq, const int* __restrict__ pos,
                                                        float* __restrict__ ctx) {
  extern __shared__ float sc[];          // scores[max_seq], then 4 x hd partial sums
  __shared__ float red[4];
  __shared__ float qs[256];
  const int h = blockIdx.x, r = blockIdx.y;
  const int kvh = h * kv_heads / heads;
  const int kv_dim = kv_heads * hd;
  const int L = min(max(*pos + r + 1, 1), max_seq);
  const float* qh = q + ((size_t)r * heads + h) * hd;
  for (int i = threadIdx.x; i < hd; i += 256) qs[i] = qh[i];
  __syncthreads();
  const float scale = 1.0f / sqrtf((float)hd);
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < L; j += 256) {
    const float* kr = kc + (size_t)j * kv_dim + (size_t)kvh * hd;
    float s = 0.0f;
    for (int d = 0; d < hd; d += 4) {
      const float4 kv = *reinterpret_cast<const float4*>(kr + d);
      s = __builtin_fmaf(qs[d], kv.x, s);
      s = __builtin_fmaf(qs[d + 1], kv.y, s);
      s = __builtin_fmaf(qs[d + 2], kv.z, s);
      s = __builtin_fmaf(qs[d + 3], kv.w, s);
    }
    s *= scale;
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max256(mx, red);
  float sum = 0.0f;
  for (int j = threadIdx.x; j < L; j += 256) {
    const float e = expf(sc[j] - mx);
    sc[j] = e;
    sum += e;
  }
  sum = block_sum256(sum, red);
  const float inv = sum != 0.0f ? 1.0f / sum : 1.0f;
  // values: thread (g, d) sums keys j = g (mod 4) for dimension d; groups folded in order
  float* part = sc + ((L + 3) & ~3);
  const int g = threadIdx.x / 64, dd = threadIdx.x & 63;
  for (int d = dd; d < hd; d += 64) {
    float acc = 0.0f;
    for (int j = g; j < L; j += 4) acc = __builtin_fmaf(sc[j] * inv, vc[(size_t)j * kv_dim + (size_t)kvh * hd + d], acc);
    part[g * hd + d] = acc;
  }
  __syncthreads();
  float* out = ctx + ((size_t)r * heads + h) * hd;
  for (int d = threadIdx.x; d < hd; d += 256) out[d] = ((part[d] + part[hd + d]) + part[2 * hd + d]) + part[3 * hd + d];
}

// out[i] = a[i] + b[i % nb]
__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                  size_t n, size_t nb, float* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i % nb];
}

// index of the largest value; among equal maxima the last (Iterator::max_by, infer.rs:217-223)
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int n, int* __restrict__ idx) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  float best = -INFINITY;
  int besti = -1;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float v = x[i];
    if (v > best || (v == best && i > besti)) { best = v; besti = i; }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(besti, off, 64);
    if (ov > best || (ov == best && oi > besti)) { best = ov; besti = oi; }
  }
  if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = besti; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (bv[w] > best || (bv[w] == best && bi[w] > besti)) { best = bv[w]; besti = bi[w]; }
    *idx = besti < 0 ? 0 : besti;
  }
}

__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ table, int n_vocab, int d,
                                                    const int* __restrict__ tok, float* __restrict__ out) {
  const int t = tok[blockIdx.x];
  float* o = out + (size_t)blockIdx.x * d;
  if (t < 0 || t >= n_vocab) {
    for (int i = threadIdx.x; i < d; i += 256) o[i] = 0.0f;
    return;
  }
  const float* src = table + (size_t)t * d;
  for (int i = threadIdx.x; i < d; i += 256) o[i] = src[i];
}

__global__ void pos_add_kernel(int* pos, int delta) {
  if (threadIdx.x == 0) *pos += delta;
}

hipError_t launch_rmsnorm(const float* x, const float* w, int rows, int d, float eps, float* out, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, w, d, eps, out);
  return hipGetLastError();
}
hipError_t launch_rope(float* x, int rows, int heads, int hd, float base, const int* pos, int off, hipStream_t s) {
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)heads, (unsigned)rows), dim3(64), 0, s, x, heads, hd, base, pos, off);
  return hipGetLastError();
}
hipError_t launch_kv_append(const float* k, const float* v, int rows, int kv_dim, float* kc, float* vc,
                            int max_seq, const int* pos, hipStream_t s) {
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)rows), dim3(256), 0, s, k, v, kv_dim, kc, vc, max_seq, pos);
  return hipGetLastError();
}
hipError_t launch_attention(const float* q, const float* kc, const float* vc, int rows, int heads, int kv_heads,
                            int hd, int max_seq, const int* pos, float* ctx, hipStream_t s) {
  const size_t lds = ((size_t)((max_seq + 3) & ~3) + 4 * (size_t)hd) * sizeof(float);
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)heads, (unsigned)rows), dim3(256), lds, s, q, kc, vc, heads,
                     kv_heads, hd, max_seq, pos, ctx);
  return hipGetLastError();
}
hipError_t launch_add(const float* a, const float* b, size_t n, size_t nb, float* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, b, n, nb, out);
  return hipGetLastError();
}
hipError_t launch_argmax(const float* x, int n, int* idx, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, x, n, idx);
  return hipGetLastError();
}
hipError_t launch_embed(const float* table, int n_vocab, int d, const int* tok, int rows, float* out,
                        hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)rows), dim3(256), 0, s, table, n_vocab, d, tok, out);
  return hipGetLastError();
}
hipError_t launch_pos_add(int* pos, int delta, hipStream_t s) {
  hipLaunchKernelGGL(pos_add_kernel, dim3(1), dim3(64), 0, s, pos, delta);
  return hipGetLastError();
}

}  // namespace rehip
