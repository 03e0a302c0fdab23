// Prefill / MoE GEMM: Y[N x m] = X[N x K] * W[m x K]^T with W dequantized on the fly.
//
// Workgroup = 256 threads (4 waves) computing a BM(128 weight rows) x BN(128 activation rows)
// tile in K steps of 128 elements (4 32-element blocks, or half a 256-element super-block).
// Per step:
//   * W: 128 rows x 4 chunks; each thread decodes two (row, chunk) pairs from the tiled slabs
//     (consecutive threads = consecutive rows, so each plane read is a contiguous 1 KiB) and
//     writes the 32 values to LDS as bf16 (or f32 in strict mode);
//   * X: 128 rows x 128 f32, coalesced float4 loads (32 lanes per 512-byte row segment),
//     converted to bf16 (RNE) into LDS;
//   * MFMA: waves in a 2 x 2 grid, each 64 x 64 = 2 x 2 tiles of v_mfma_f32_32x32x16_bf16
//     (strict mode: v_mfma_f32_32x32x2_f32), f32 accumulators.
// LDS rows are padded by 16 bytes so the 32 lanes reading one k-slice hit different banks.
//
// Grouped launch (MoE): one task per workgroup names the expert, the weight tile and a run of
// gathered activation rows; `xrow` maps a gathered row to its activation row.
#include <hip/hip_runtime.h>

#include "deq.hpp"
#include "kernels.hpp"

namespace rehip {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

template <bool F32> struct Elem;
template <> struct Elem<false> { using T = __bf16; static constexpr int PAD = 8; };
template <> struct Elem<true> { using T = float; static constexpr int PAD = 4; };

// 16 decoded values of a run -> LDS (two 16-byte bf16 stores, or four float4 stores)
template <bool F32>
__device__ __forceinline__ void store_run(typename Elem<F32>::T* dst, const Run& r) {
  if constexpr (F32) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      reinterpret_cast<float4*>(dst)[v] = make_float4(run_value(r, 4 * v), run_value(r, 4 * v + 1),
                                                      run_value(r, 4 * v + 2), run_value(r, 4 * v + 3));
  } else {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      bf16x8_t o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (__bf16)run_value(r, 8 * v + i);
      reinterpret_cast<bf16x8_t*>(dst)[v] = o;
    }
  }
}

template <bool F32>
__device__ __forceinline__ void store_zero32(typename Elem<F32>::T* dst) {
  if constexpr (F32) {
#pragma unroll
    for (int v = 0; v < 8; ++v) reinterpret_cast<float4*>(dst)[v] = make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    bf16x8_t z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (__bf16)0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) reinterpret_cast<bf16x8_t*>(dst)[v] = z;
  }
}

template <bool F32>
__device__ __forceinline__ void store4(typename Elem<F32>::T* dst, float4 v) {
  if constexpr (F32) {
    *reinterpret_cast<float4*>(dst) = v;
  } else {
    bf16x4_t o;
    o[0] = (__bf16)v.x; o[1] = (__bf16)v.y; o[2] = (__bf16)v.z; o[3] = (__bf16)v.w;
    *reinterpret_cast<bf16x4_t*>(dst) = o;
  }
}

template <int T, bool F32, bool GROUPED>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  using B = Blk<T>;
  using E = typename Elem<F32>::T;
  constexpr int LD = kGemmBK + Elem<F32>::PAD;   // LDS row stride (elements)
  __shared__ __attribute__((aligned(16))) E Ws[kGemmBM * LD];
  __shared__ __attribute__((aligned(16))) E Xs[kGemmBN * LD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int mtile, r0, rn;
  const uint8_t* W = p.W;
  if constexpr (GROUPED) {
    const GemmTask t = p.tasks[blockIdx.x];
    mtile = t.mtile;
    r0 = t.r0;
    rn = t.rn;
    W += (size_t)t.expert * p.w_stride;
  } else {
    mtile = blockIdx.x;
    r0 = blockIdx.y * kGemmBN;
    rn = min(kGemmBN, p.N - r0);
  }

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // activation rows this thread stages: rows 8*jj + tid/32, k offset 4*(tid%32)
  const int xk = 4 * (tid & 31);
  const float* xptr[16];
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    const int rl = 8 * jj + (tid >> 5);
    int xr = -1;
    if (rl < rn) {
      const int g = r0 + rl;
      xr = (GROUPED && p.xrow) ? p.xrow[g] : g;
    }
    xptr[jj] = xr >= 0 ? p.X + (size_t)xr * p.K : nullptr;
  }

  const int steps = (p.K + kGemmBK - 1) / kGemmBK;
  for (int s = 0; s < steps; ++s) {
    __syncthreads();
    // ---- stage W: 128 rows x 4 chunks, two per thread
#pragma unroll
    for (int rep = 0; rep < 2; ++rep) {
      const int j = tid + 256 * rep;
      const int rl = j & 127, c = j >> 7;
      const int tile = 2 * mtile + (rl >> 6), tl = rl & 63;
      E* dst = Ws + rl * LD;
      int kb, cc, kl;
      if constexpr (B::QK == 32) {
        kb = 4 * s + c; cc = 0; kl = 32 * c;
      } else {
        kb = s >> 1; cc = 4 * (s & 1) + c; kl = -128 * (s & 1);
      }
      if (tile < p.tiles && kb < p.KB) {
        Run a, b;
        B::chunk(W + ((size_t)tile * p.KB + kb) * B::SLAB, tl, cc, a, b);
        store_run<F32>(dst + kl + a.e, a);
        store_run<F32>(dst + kl + b.e, b);
      } else {
        // missing rows/columns: the four chunk jobs of this row zero all 128 slots
        store_zero32<F32>(dst + 32 * c);
      }
    }
    // ---- stage X: 128 rows x 128 k, float4 per lane
    const int k = s * kGemmBK + xk;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int rl = 8 * jj + (tid >> 5);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (xptr[jj] && k < p.K) v = *reinterpret_cast<const float4*>(xptr[jj] + k);
      store4<F32>(Xs + rl * LD + xk, v);
    }
    __syncthreads();
    // ---- MFMA
    if constexpr (!F32) {
#pragma unroll
      for (int kk = 0; kk < kGemmBK / 16; ++kk) {
        bf16x8_t av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          av[i] = *reinterpret_cast<const bf16x8_t*>(Ws + (64 * wm + 32 * i + (lane & 31)) * LD + 16 * kk + 8 * (lane >> 5));
#pragma unroll
        for (int j = 0; j < 2; ++j)
          bv[j] = *reinterpret_cast<const bf16x8_t*>(Xs + (64 * wn + 32 * j + (lane & 31)) * LD + 16 * kk + 8 * (lane >> 5));
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    } else {
#pragma unroll 8
      for (int kk = 0; kk < kGemmBK / 2; ++kk) {
        float av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) av[i] = Ws[(64 * wm + 32 * i + (lane & 31)) * LD + 2 * kk + (lane >> 5)];
#pragma unroll
        for (int j = 0; j < 2; ++j) bv[j] = Xs[(64 * wn + 32 * j + (lane & 31)) * LD + 2 * kk + (lane >> 5)];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: D[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), register 4*(i/8) + i%4
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int xl = 64 * wn + 32 * j + (lane & 31);
      if (xl >= rn) continue;
      float* yrow = p.Y + (size_t)(r0 + xl) * p.ldy;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int wr = kGemmBM * mtile + 64 * wm + 32 * i + 8 * q + 4 * (lane >> 5);
        if (wr + 3 < p.m) {
          *reinterpret_cast<float4*>(yrow + wr) =
              make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (wr + e < p.m) yrow[wr + e] = acc[i][j][4 * q + e];
        }
      }
    }
  }
}

template <int T, bool F32>
static hipError_t launch_t(const GemmArgs& a, int ntasks, hipStream_t s) {
  if (a.tasks) {
    hipLaunchKernelGGL((gemm_kernel<T, F32, true>), dim3((unsigned)ntasks), dim3(256), 0, s, a);
  } else {
    dim3 grid((unsigned)((a.m + kGemmBM - 1) / kGemmBM), (unsigned)((a.N + kGemmBN - 1) / kGemmBN));
    hipLaunchKernelGGL((gemm_kernel<T, F32, false>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

template <int T>
static hipError_t launch_mode(int mode, const GemmArgs& a, int ntasks, hipStream_t s) {
  return mode == 1 ? launch_t<T, true>(a, ntasks, s) : launch_t<T, false>(a, ntasks, s);
}

hipError_t launch_gemm(uint32_t type, int mode, const GemmArgs& a, int ntasks, hipStream_t s) {
  switch (type) {
    case T_Q4_0: return launch_mode<T_Q4_0>(mode, a, ntasks, s);
    case T_Q5_0: return launch_mode<T_Q5_0>(mode, a, ntasks, s);
    case T_Q8_0: return launch_mode<T_Q8_0>(mode, a, ntasks, s);
    case T_Q4_K: return launch_mode<T_Q4_K>(mode, a, ntasks, s);
    case T_Q5_K: return launch_mode<T_Q5_K>(mode, a, ntasks, s);
    case T_Q6_K: return launch_mode<T_Q6_K>(mode, a, ntasks, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rehip
