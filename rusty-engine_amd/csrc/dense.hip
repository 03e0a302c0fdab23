// Dense (unquantized) weights: F32, F16 and BF16 matrices stored row-major as the GGUF file holds
// them (QMat::F32 and the no-fused-kernel fallback of src/qmat.rs:128-151, the float arms of
// quant::dequant, src/quant.rs:363-392). Every element widens exactly to f32 (F16 by bit
// widening with subnormals and NaN payloads kept, BF16 by a 16-bit shift); products accumulate in
// f32 per lane in element order and fold over the wave with a fixed xor tree (deterministic).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "deq.hpp"
#include "kernels.hpp"

namespace rehip {

namespace {

template <uint32_t T> struct DenseElem;
template <> struct DenseElem<0> {
  using S = float;
  __device__ static float get(float v) { return v; }
};
// The hardware widening quiets a signalling NaN; a dequantized F16 value is an output in its own
// right (no scale multiplies it), so NaNs are rebuilt bit for bit: sign, all-ones exponent, the
// ten payload bits on top of the mantissa (quant.rs:25-45).
template <> struct DenseElem<1> {
  using S = uint16_t;
  __device__ static float get(uint16_t h) {
    const float v = f16_bits_to_f32(h);
    const uint32_t nan = (((uint32_t)h & 0x8000u) << 16) | 0x7F800000u | (((uint32_t)h & 0x3FFu) << 13);
    return ((h & 0x7C00u) == 0x7C00u && (h & 0x3FFu)) ? __uint_as_float(nan) : v;
  }
};
template <> struct DenseElem<30> {
  using S = uint16_t;
  __device__ static float get(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
};

template <uint32_t T>
__global__ __launch_bounds__(256) void dense_to_f32_kernel(const typename DenseElem<T>::S* __restrict__ src,
                                                           float* __restrict__ dst, size_t count) {
  const size_t step = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += step) dst[i] = DenseElem<T>::get(src[i]);
}

__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Y[t][r] = sum_k W[r][k] x[t][k] (+ add[r] when given): one wave per weight row, TT activation
// rows per workgroup, lanes striding the row so every weight load is a contiguous 64-element run.
template <uint32_t T, int TT>
__global__ __launch_bounds__(256) void dense_gemm_kernel(const typename DenseElem<T>::S* __restrict__ W,
                                                         const float* __restrict__ x, float* __restrict__ y, int m,
                                                         int n, int rows, const float* __restrict__ add) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x * 4 + wave;
  if (r >= m) return;                    // no workgroup barrier below
  const int t0 = blockIdx.y * TT;
  const int nt = min(TT, rows - t0);
  const typename DenseElem<T>::S* wr = W + (size_t)r * n;
  float acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = 0.0f;
  for (int k = lane; k < n; k += 64) {
    const float w = DenseElem<T>::get(wr[k]);
#pragma unroll
    for (int t = 0; t < TT; ++t)
      if (t < nt) acc[t] = __builtin_fmaf(w, x[(size_t)(t0 + t) * n + k], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = wave_sum_xor(acc[t]);
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < TT; ++t)
      if (t < nt) y[(size_t)(t0 + t) * m + r] = add ? acc[t] + add[r] : acc[t];
  }
}

template <uint32_t T>
hipError_t launch_dense_t(const void* W, const float* x, float* y, int m, int n, int rows, const float* add,
                          hipStream_t s) {
  using S = typename DenseElem<T>::S;
  const unsigned gx = (unsigned)((m + 3) / 4);
  // 1, 4 or 16 activation rows per workgroup: W is read once per row group, and every output keeps
  // the same per-lane order and fold whatever the group
  if (rows == 1)
    hipLaunchKernelGGL((dense_gemm_kernel<T, 1>), dim3(gx, 1u), dim3(256), 0, s, (const S*)W, x, y, m, n, rows, add);
  else if (rows < 16)
    hipLaunchKernelGGL((dense_gemm_kernel<T, 4>), dim3(gx, (unsigned)((rows + 3) / 4)), dim3(256), 0, s, (const S*)W,
                       x, y, m, n, rows, add);
  else
    hipLaunchKernelGGL((dense_gemm_kernel<T, 16>), dim3(gx, (unsigned)((rows + 15) / 16)), dim3(256), 0, s,
                       (const S*)W, x, y, m, n, rows, add);
  return hipGetLastError();
}

}  // namespace

bool dense_type(uint32_t type) { return type == 0 || type == 1 || type == 30; }
size_t dense_elem_bytes(uint32_t type) { return type == 0 ? 4 : 2; }

hipError_t launch_dense_gemm(uint32_t type, const void* W, const float* x, float* y, int m, int n, int rows,
                             const float* add, hipStream_t s) {
  if (rows == 0 || m == 0) return hipSuccess;
  switch (type) {
    case 0: return launch_dense_t<0>(W, x, y, m, n, rows, add, s);
    case 1: return launch_dense_t<1>(W, x, y, m, n, rows, add, s);
    case 30: return launch_dense_t<30>(W, x, y, m, n, rows, add, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dense_to_f32(uint32_t type, const void* src, float* dst, size_t count, hipStream_t s) {
  if (count == 0) return hipSuccess;
  const dim3 grid((unsigned)std::min<size_t>((count + 255) / 256, 8192));   // grid-stride beyond 2M elements
  switch (type) {
    case 0: hipLaunchKernelGGL(dense_to_f32_kernel<0>, grid, dim3(256), 0, s, (const float*)src, dst, count); break;
    case 1: hipLaunchKernelGGL(dense_to_f32_kernel<1>, grid, dim3(256), 0, s, (const uint16_t*)src, dst, count); break;
    case 30: hipLaunchKernelGGL(dense_to_f32_kernel<30>, grid, dim3(256), 0, s, (const uint16_t*)src, dst, count); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace rehip
