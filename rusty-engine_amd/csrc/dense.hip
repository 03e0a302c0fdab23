// Dense (unquantized) weights: F32, F16 and BF16 matrices stored row-major as the GGUF file holds
// them (QMat::F32 and the no-fused-kernel fallback of src/qmat.rs:128-151, the float arms of
// quant::dequant, src/quant.rs:363-392). Every element widens exactly to f32 (F16 by bit
// widening with subnormals and NaN payloads kept, BF16 by a 16-bit shift). Up to 15 activation
// rows: products accumulate in f32 per lane in element order and fold over the wave with a fixed
// xor tree (deterministic); from 16 rows, an MFMA GEMM (bf16 operands in bf16 mode, f32 in f32
// mode).
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
// One row (TT = 1) may also fold the greedy argmax of y into best (the quantized GEMV's slots).
template <uint32_t T, int TT>
__global__ __launch_bounds__(256) void dense_gemm_kernel(const typename DenseElem<T>::S* __restrict__ W,
                                                         const float* __restrict__ x, float* __restrict__ y, int m,
                                                         int n, int rows, const float* __restrict__ add,
                                                         unsigned long long* __restrict__ best) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x * 4 + wave;
  if (r >= m) return;                    // no workgroup barrier below
  const int t0 = blockIdx.y * TT;
  const int nt = min(TT, rows - t0);
  const typename DenseElem<T>::S* wr = W + (size_t)r * n;
  float acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = 0.0f;
  // U of the lane's k at a time: their weight and activation loads go out together (a loop that
  // loads and multiplies one k at a time waits a memory round trip per k), then the FMAs in the
  // same ascending-k order, so the sums keep their bits. Activation rows past nt read row nt - 1
  // (their sums are not stored).
  // A k past the row loads index n - 1 and skips its FMAs (a branch around arithmetic only).
  constexpr int U = TT >= 16 ? 2 : TT >= 4 ? 4 : 8;
  for (int k = lane; k < n; k += 64 * U) {
    float w[U], xv[U][TT];
#pragma unroll
    for (int j = 0; j < U; ++j) w[j] = DenseElem<T>::get(wr[min(k + 64 * j, n - 1)]);
#pragma unroll
    for (int j = 0; j < U; ++j)
#pragma unroll
      for (int t = 0; t < TT; ++t) xv[j][t] = x[(size_t)(t0 + min(t, nt - 1)) * n + min(k + 64 * j, n - 1)];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      if (k + 64 * j < n) {
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = __builtin_fmaf(w[j], xv[j][t], acc[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = wave_sum_xor(acc[t]);
  unsigned long long key = 0;
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t < nt) {
        const float v = add ? acc[t] + add[r] : acc[t];
        y[(size_t)(t0 + t) * m + r] = v;
        if (TT == 1) key = argmax_key(v, r);
      }
    }
  }
  if (TT == 1 && best) wave_argmax_fold(key, best);
}

// Many activation rows: an MFMA GEMM over 64 x 64 output tiles (64 weight rows x 64 activation
// rows), four waves of one 32 x 32 tile each, K in steps of 32. Each step's weights and activations
// go through LDS: every element is widened exactly to f32 and, in bf16 mode, rounded to bf16 (RNE)
// for v_mfma_f32_32x32x16_bf16; f32 mode keeps f32 and uses v_mfma_f32_32x32x2_f32. The next
// step's global loads are in flight while a step multiplies. Needs n % 8 == 0 (whole 8-element
// runs per thread) and 16-byte aligned activation rows; K beyond n and rows beyond m / rows read
// zeros. The result of an output depends only on its row, column and the mode (fixed K order).
constexpr int kDenseBM = 64, kDenseBN = 64, kDenseBK = 32;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

template <bool F32> struct DenseLds;
template <> struct DenseLds<false> {
  using E = __bf16;
  static constexpr int LD = kDenseBK + 8;     // 80 bytes per row: 16-byte aligned, banks spread
};
template <> struct DenseLds<true> {
  using E = float;
  static constexpr int LD = kDenseBK + 4;     // 144 bytes per row
};

// the 8 elements k0 .. k0 + 7 of weight row r (zeros past the matrix), widened to f32
template <uint32_t T>
__device__ __forceinline__ void dense_load8(const typename DenseElem<T>::S* W, int m, int n, int r, int k0, float (&v)[8]) {
  if (r >= m || k0 >= n) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    return;
  }
  const typename DenseElem<T>::S* p = W + (size_t)r * n + k0;
  if constexpr (T == 0) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = DenseElem<T>::get((uint16_t)(w[i] & 0xFFFFu));
      v[2 * i + 1] = DenseElem<T>::get((uint16_t)(w[i] >> 16));
    }
  }
}

__device__ __forceinline__ void dense_loadx8(const float* x, int rows, int n, int t, int k0, float (&v)[8]) {
  if (t >= rows || k0 >= n) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    return;
  }
  const float* p = x + (size_t)t * n + k0;
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// 8 raw elements through a buffer resource (F32: two 16-byte loads, F16/BF16: one); an offset past
// the resource reads zeros, so the tile edges need no branch
struct DenseRaw { i32x4_t a, b; };
template <uint32_t T>
__device__ __forceinline__ DenseRaw dense_bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  DenseRaw v;
  v.a = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  if constexpr (T == 0) v.b = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off + 16u), 0, 0);
  else v.b = i32x4_t{0, 0, 0, 0};
  return v;
}
// the 8 elements widened exactly to f32
template <uint32_t T>
__device__ __forceinline__ void dense_widen8(const DenseRaw& u, float (&v)[8]) {
  if constexpr (T == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = __int_as_float(u.a[i]);
      v[4 + i] = __int_as_float(u.b[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = (uint32_t)u.a[i];
      v[2 * i] = DenseElem<T>::get((uint16_t)(w & 0xFFFFu));
      v[2 * i + 1] = DenseElem<T>::get((uint16_t)(w >> 16));
    }
  }
}

// the bf16 roundings of 8 values into hi and (LO) the bf16 roundings of their remainders into lo
template <bool LO>
__device__ __forceinline__ void dense_store8_split(__bf16* hi, __bf16* lo, const float (&v)[8]) {
  bf16x8_t h, l;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    h[i] = (__bf16)v[i];
    l[i] = (__bf16)(v[i] - (float)h[i]);
  }
  *reinterpret_cast<bf16x8_t*>(hi) = h;
  if constexpr (LO) *reinterpret_cast<bf16x8_t*>(lo) = l;
}

template <bool F32>
__device__ __forceinline__ void dense_store8(typename DenseLds<F32>::E* dst, const float (&v)[8]) {
  if constexpr (F32) {
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    bf16x8_t b;
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = (__bf16)v[i];
    *reinterpret_cast<bf16x8_t*>(dst) = b;
  }
}

// SP (f32 mode on bf16 MFMAs, split operands): the weights and activations are staged as their
// bf16 roundings (hi) and, in a second plane, the bf16 roundings of what hi leaves (lo); each
// product is w_hi x_hi + w_hi x_lo + w_lo x_hi, each term within 2^-16 relative (BF16 weights are
// their own rounding: w_lo = 0, two MFMAs)
template <uint32_t T, bool F32, bool SP = false>
__global__ __launch_bounds__(256) void dense_mma_kernel(const typename DenseElem<T>::S* __restrict__ W,
                                                        const float* __restrict__ x, float* __restrict__ y, int m,
                                                        int n, int rows, const float* __restrict__ add,
                                                        float* __restrict__ partial, int steps_per_split) {
  using L = DenseLds<F32>;
  using E = typename L::E;
  constexpr int LD = L::LD;
  static_assert(!(F32 && SP), "split operands run on bf16 MFMAs");
  constexpr bool WLO = SP && T != 30;                  // the weights have a remainder (not BF16)
  __shared__ __attribute__((aligned(16))) E ws[kDenseBM * LD * (WLO ? 2 : 1)];
  __shared__ __attribute__((aligned(16))) E xs[kDenseBN * LD * (SP ? 2 : 1)];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;             // the wave's 32 weight rows / 32 activation rows
  const int m0 = blockIdx.x * kDenseBM, t0 = blockIdx.y * kDenseBN;
  // K slice of this workgroup (blockIdx.z; one slice when the grid has no z)
  const int steps_all = (n + kDenseBK - 1) / kDenseBK;
  const int s0 = blockIdx.z * steps_per_split, s1 = min(steps_all, s0 + steps_per_split);
  // staging: thread t takes row t / 4 of both tiles, elements 8 (t % 4) .. + 7 of the step
  const int sr = tid >> 2, sk = 8 * (tid & 3);
  // buffer resources over the workgroup's weight rows and activation rows: a row past the matrix
  // lies past the resource, a k past the row (or past the split) takes an offset past it, so
  // every load is unconditional. Loaded under branches, the next step's loads had been waited for
  // right away (the compiler copied them where the branches join), before this step's MFMAs.
  using S = typename DenseElem<T>::S;
  const int wrows = min(kDenseBM, m - m0), xrows = min(kDenseBN, rows - t0);
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W + (size_t)m0 * n, (uint32_t)((size_t)wrows * n * sizeof(S)));
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x + (size_t)t0 * n, (uint32_t)((size_t)xrows * n * sizeof(float)));
  auto off = [&](int st, uint32_t es) -> uint32_t {
    const int k0 = st * kDenseBK + sk;
    return st < s1 && k0 < n ? ((uint32_t)sr * (uint32_t)n + (uint32_t)k0) * es : 0x80000000u;
  };
  DenseRaw wraw = dense_bload8<T>(wrs, off(s0, sizeof(S)));
  DenseRaw xraw = dense_bload8<0>(xrs, off(s0, sizeof(float)));
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  for (int st = s0; st < s1; ++st) {
    float wv[8], xv[8];
    dense_widen8<T>(wraw, wv);
    dense_widen8<0>(xraw, xv);
    if constexpr (SP) {
      dense_store8_split<WLO>(ws + sr * LD + sk, ws + kDenseBM * LD + sr * LD + sk, wv);
      dense_store8_split<true>(xs + sr * LD + sk, xs + kDenseBN * LD + sr * LD + sk, xv);
    } else {
      dense_store8<F32>(ws + sr * LD + sk, wv);
      dense_store8<F32>(xs + sr * LD + sk, xv);
    }
    __syncthreads();
    wraw = dense_bload8<T>(wrs, off(st + 1, sizeof(S)));     // the next step's loads fly under this
    xraw = dense_bload8<0>(xrs, off(st + 1, sizeof(float)));  // step's MFMAs (past s1: zeros)
    const E* wa = ws + (32 * wm + (lane & 31)) * LD;
    const E* xb = xs + (32 * wn + (lane & 31)) * LD;
    if constexpr (F32) {
      // MFMA q of the 8-k slice kk takes k = 8 kk + q (lanes 0-31) and 8 kk + 4 + q (lanes 32-63)
#pragma unroll
      for (int kk = 0; kk < kDenseBK / 8; ++kk) {
        const float4 a = *reinterpret_cast<const float4*>(wa + 8 * kk + 4 * (lane >> 5));
        const float4 b = *reinterpret_cast<const float4*>(xb + 8 * kk + 4 * (lane >> 5));
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < kDenseBK / 16; ++kk) {
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(wa + 16 * kk + 8 * (lane >> 5));
        const bf16x8_t b = *reinterpret_cast<const bf16x8_t*>(xb + 16 * kk + 8 * (lane >> 5));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        if constexpr (SP) {
          const bf16x8_t bl = *reinterpret_cast<const bf16x8_t*>(xb + kDenseBN * LD + 16 * kk + 8 * (lane >> 5));
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bl, acc, 0, 0, 0);
          if constexpr (WLO) {
            const bf16x8_t al = *reinterpret_cast<const bf16x8_t*>(wa + kDenseBM * LD + 16 * kk + 8 * (lane >> 5));
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b, acc, 0, 0, 0);
          }
        }
      }
    }
    __syncthreads();                     // every wave is done reading the step
  }
  // D[i][j]: weight row i = 8 (r / 4) + 4 (lane / 32) + r % 4 of the wave's 32, activation row
  // j = lane % 32: four consecutive registers are four consecutive outputs of one activation row
  // (K slices: each writes its partial tile; the reduce adds them in slice order)
  const int t = t0 + 32 * wn + (lane & 31);
  if (t >= rows) return;
  float* yr = (gridDim.z > 1 ? partial + (size_t)blockIdx.z * rows * m : y) + (size_t)t * m;
  const float* ad = gridDim.z > 1 ? nullptr : add;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int r0 = m0 + 32 * wm + 8 * g + 4 * (lane >> 5);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = r0 + e;
      if (r < m) yr[r] = ad ? acc[4 * g + e] + ad[r] : acc[4 * g + e];
    }
  }
}

template <uint32_t T>
hipError_t launch_dense_t(const void* W, const float* x, float* y, int m, int n, int rows, const float* add, int mode,
                          unsigned long long* best, float* partial, int splits, hipStream_t s) {
  using S = typename DenseElem<T>::S;
  if (best && rows != 1) return hipErrorInvalidValue;
  if (dense_mma_rows(n, rows, x)) {
    const int steps = (n + kDenseBK - 1) / kDenseBK;
    if (splits < 1 || (splits > 1 && (!partial || add))) return hipErrorInvalidValue;
    const int sps = (steps + splits - 1) / splits;
    splits = (steps + sps - 1) / sps;
    const dim3 grid((unsigned)((m + kDenseBM - 1) / kDenseBM), (unsigned)((rows + kDenseBN - 1) / kDenseBN),
                    (unsigned)splits);
    if (mode == kGemmModeSplit)
      hipLaunchKernelGGL((dense_mma_kernel<T, false, true>), grid, dim3(256), 0, s, (const S*)W, x, y, m, n, rows,
                         add, partial, sps);
    else if (mode == 1)
      hipLaunchKernelGGL((dense_mma_kernel<T, true>), grid, dim3(256), 0, s, (const S*)W, x, y, m, n, rows, add,
                         partial, sps);
    else
      hipLaunchKernelGGL((dense_mma_kernel<T, false>), grid, dim3(256), 0, s, (const S*)W, x, y, m, n, rows, add,
                         partial, sps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_gemm_reduce(partial, y, (size_t)rows * m, splits, s);
  }
  const unsigned gx = (unsigned)((m + 3) / 4);
  // 1, 4 or 16 activation rows per workgroup: W is read once per row group, and every output keeps
  // the same per-lane order and fold whatever the group
  if (rows == 1)
    hipLaunchKernelGGL((dense_gemm_kernel<T, 1>), dim3(gx, 1u), dim3(256), 0, s, (const S*)W, x, y, m, n, rows, add,
                       best);
  else if (rows < 16)
    hipLaunchKernelGGL((dense_gemm_kernel<T, 4>), dim3(gx, (unsigned)((rows + 3) / 4)), dim3(256), 0, s, (const S*)W,
                       x, y, m, n, rows, add, nullptr);
  else
    hipLaunchKernelGGL((dense_gemm_kernel<T, 16>), dim3(gx, (unsigned)((rows + 15) / 16)), dim3(256), 0, s,
                       (const S*)W, x, y, m, n, rows, add, nullptr);
  return hipGetLastError();
}

}  // namespace

bool dense_type(uint32_t type) { return type == 0 || type == 1 || type == 30; }
size_t dense_elem_bytes(uint32_t type) { return type == 0 ? 4 : 2; }

bool dense_mma_rows(int n, int rows, const float* x) {
  return rows >= kDenseMmaMinRows && n % 8 == 0 && ((uintptr_t)x & 15) == 0;
}

int dense_mma_splits(int m, int n, int rows) {
  // K slices until ~512 workgroups run (two per CU: a workgroup's K loop is bound by its load
  // latency), each slice at least 4 steps of 32
  const long tiles = (long)((m + kDenseBM - 1) / kDenseBM) * ((rows + kDenseBN - 1) / kDenseBN);
  const int steps = (n + kDenseBK - 1) / kDenseBK;
  if (tiles >= 512) return 1;
  return (int)std::max<long>(1, std::min<long>((512 + tiles - 1) / tiles, steps / 4));
}

hipError_t launch_dense_gemm(uint32_t type, const void* W, const float* x, float* y, int m, int n, int rows,
                             const float* add, int mode, unsigned long long* best, float* partial, int splits,
                             hipStream_t s) {
  if (rows == 0 || m == 0) return hipSuccess;
  switch (type) {
    case 0: return launch_dense_t<0>(W, x, y, m, n, rows, add, mode, best, partial, splits, s);
    case 1: return launch_dense_t<1>(W, x, y, m, n, rows, add, mode, best, partial, splits, s);
    case 30: return launch_dense_t<30>(W, x, y, m, n, rows, add, mode, best, partial, splits, s);
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
