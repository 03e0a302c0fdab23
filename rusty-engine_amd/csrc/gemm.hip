// Prefill / MoE GEMM: Y[N x m] = X[N x K] * W[m x K]^T with W dequantized on the fly.
//
// Workgroup = 256 threads (4 waves, 2 x 2) computing a BM (weight rows) x BN (activation rows)
// tile in K steps of 128 elements (4 32-element blocks, or half a 256-element super-block).
// Per step:
//   * W: BM rows x 4 chunks; a thread decodes (row, chunk) pairs from the tiled slabs
//     (consecutive threads = consecutive rows, so each plane read is a contiguous 1 KiB) and
//     writes the 32 values to LDS as bf16 (or f32 in strict mode);
//   * X: BN rows x 128 f32, float4 loads (32 lanes cover one 512-byte row segment), converted
//     to bf16 (RNE) into LDS;
//   * MFMA: each wave owns (BM/2) x (BN/2) as 32 x 32 tiles of v_mfma_f32_32x32x16_bf16
//     (strict mode: v_mfma_f32_32x32x2_f32), f32 accumulators.
// Global loads are double-buffered in registers: the raw weight chunks and X of step s+1 are in
// flight while the MFMAs of step s run; decoding happens when they are written to LDS.
// LDS rows are padded by 16 bytes so the 32 lanes reading one k-slice hit different banks.
//
// Dense launches use a 1-D grid ordered so that each of the 8 XCDs (workgroup w runs on XCD
// w % 8) processes a contiguous band of activation-row tiles for every weight tile: the X band
// stays in that XCD's L2 while the (small) quantized weights stream through.
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

template <int T, bool F32, bool GROUPED, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  using B = Blk<T>;
  using E = typename Elem<F32>::T;
  constexpr int BK = kGemmBK;
  constexpr int LD = BK + Elem<F32>::PAD;          // LDS row stride (elements)
  constexpr int WJOBS = BM * 4 / 256;              // (row, chunk) jobs per thread per step
  constexpr int XV = BN * BK / 4 / 256;            // float4 of X per thread per step
  constexpr int TM = BM / 64, TN = BN / 64;        // 32x32 MFMA tiles per wave
  __shared__ __attribute__((aligned(16))) E Ws[BM * LD];
  __shared__ __attribute__((aligned(16))) E Xs[BN * LD];

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
    // XCD-aware order: XCD (blockIdx % 8) takes a contiguous run of tiles, n-tile major
    const int mt = (p.m + BM - 1) / BM, nt = (p.N + BN - 1) / BN;
    const int total = mt * nt;
    const int per = (total + 7) / 8;
    const int t = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (t >= total) return;
    const int ntile = t / mt;
    mtile = t - ntile * mt;
    r0 = ntile * BN;
    rn = min(BN, p.N - r0);
  }

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // activation rows this thread stages: rows (256/32)*jj + tid/32, k offset 4*(tid%32)
  const int xk = 4 * (tid & 31);
  int xrow_off[XV];
#pragma unroll
  for (int jj = 0; jj < XV; ++jj) {
    const int rl = 8 * jj + (tid >> 5);
    int xr = -1;
    if (rl < rn) {
      const int g = r0 + rl;
      xr = (GROUPED && p.xrow) ? p.xrow[g] : g;
    }
    xrow_off[jj] = xr;
  }

  typename B::CR wraw[WJOBS];
  bool wok[WJOBS];
  float4 xraw[XV];

  auto prefetch = [&](int s) {
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) {
      const int j = tid + 256 * rep;
      const int rl = j % BM, c = j / BM;
      const int tile = BM / 64 * mtile + (rl >> 6), tl = rl & 63;
      int kb, cc;
      if constexpr (B::QK == 32) { kb = 4 * s + c; cc = 0; }
      else { kb = s >> 1; cc = 4 * (s & 1) + c; }
      wok[rep] = tile < p.tiles && kb < p.KB;
      if (wok[rep]) B::load_chunk(W + ((size_t)tile * p.KB + kb) * B::SLAB, tl, cc, wraw[rep]);
    }
    const int k = s * BK + xk;
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) {
      xraw[jj] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (xrow_off[jj] >= 0 && k < p.K)
        xraw[jj] = *reinterpret_cast<const float4*>(p.X + (size_t)xrow_off[jj] * p.K + k);
    }
  };

  auto commit = [&](int s) {
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) {
      const int j = tid + 256 * rep;
      const int rl = j % BM, c = j / BM;
      E* dst = Ws + rl * LD;
      if (wok[rep]) {
        int cc, kl;
        if constexpr (B::QK == 32) { cc = 0; kl = 32 * c; }
        else { cc = 4 * (s & 1) + c; kl = -128 * (s & 1); }
        Run a, b;
        B::decode_chunk(wraw[rep], cc, a, b);
        store_run<F32>(dst + kl + a.e, a);
        store_run<F32>(dst + kl + b.e, b);
      } else {
        // missing rows/columns: the four chunk jobs of this row zero all 128 slots
        store_zero32<F32>(dst + 32 * c);
      }
    }
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) store4<F32>(Xs + (8 * jj + (tid >> 5)) * LD + xk, xraw[jj]);
  };

  const int steps = (p.K + BK - 1) / BK;
  prefetch(0);
  for (int s = 0; s < steps; ++s) {
    if (s > 0) __syncthreads();          // previous step's MFMA reads are done
    commit(s);
    __syncthreads();
    if (s + 1 < steps) prefetch(s + 1);  // in flight during the MFMAs below
    if constexpr (!F32) {
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        bf16x8_t av[TM], bv[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          av[i] = *reinterpret_cast<const bf16x8_t*>(Ws + (BM / 2 * wm + 32 * i + (lane & 31)) * LD + 16 * kk + 8 * (lane >> 5));
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bv[j] = *reinterpret_cast<const bf16x8_t*>(Xs + (BN / 2 * wn + 32 * j + (lane & 31)) * LD + 16 * kk + 8 * (lane >> 5));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    } else {
#pragma unroll 8
      for (int kk = 0; kk < BK / 2; ++kk) {
        float av[TM], bv[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) av[i] = Ws[(BM / 2 * wm + 32 * i + (lane & 31)) * LD + 2 * kk + (lane >> 5)];
#pragma unroll
        for (int j = 0; j < TN; ++j) bv[j] = Xs[(BN / 2 * wn + 32 * j + (lane & 31)) * LD + 2 * kk + (lane >> 5)];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: D[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), register 4*(i/8) + i%4
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int xl = BN / 2 * wn + 32 * j + (lane & 31);
      if (xl >= rn) continue;
      float* yrow = p.Y + (size_t)(r0 + xl) * p.ldy;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int wr = BM * mtile + BM / 2 * wm + 32 * i + 8 * q + 4 * (lane >> 5);
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

template <int T, bool F32, int BM, int BN>
static hipError_t launch_shape(const GemmArgs& a, int ntasks, hipStream_t s) {
  if (a.tasks) {
    hipLaunchKernelGGL((gemm_kernel<T, F32, true, BM, BN>), dim3((unsigned)ntasks), dim3(256), 0, s, a);
  } else {
    const int total = ((a.m + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const int grid = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((gemm_kernel<T, F32, false, BM, BN>), dim3((unsigned)grid), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

// Tile choice: 128 x 128 when that already gives about a workgroup per CU, else 64 x 64.
template <int T, bool F32>
static hipError_t launch_t(const GemmArgs& a, int ntasks, int tile, hipStream_t s) {
  if (tile == 128) return launch_shape<T, F32, 128, 128>(a, ntasks, s);
  return launch_shape<T, F32, 64, 64>(a, ntasks, s);
}

template <int T>
static hipError_t launch_mode(int mode, const GemmArgs& a, int ntasks, int tile, hipStream_t s) {
  return mode == 1 ? launch_t<T, true>(a, ntasks, tile, s) : launch_t<T, false>(a, ntasks, tile, s);
}

int gemm_tile_for(int m, int n) {
  const long big = (long)((m + 127) / 128) * ((n + 127) / 128);
  return big >= 200 ? 128 : 64;
}

hipError_t launch_gemm(uint32_t type, int mode, const GemmArgs& a, int ntasks, int tile, hipStream_t s) {
  switch (type) {
    case T_Q4_0: return launch_mode<T_Q4_0>(mode, a, ntasks, tile, s);
    case T_Q5_0: return launch_mode<T_Q5_0>(mode, a, ntasks, tile, s);
    case T_Q8_0: return launch_mode<T_Q8_0>(mode, a, ntasks, tile, s);
    case T_Q4_K: return launch_mode<T_Q4_K>(mode, a, ntasks, tile, s);
    case T_Q5_K: return launch_mode<T_Q5_K>(mode, a, ntasks, tile, s);
    case T_Q6_K: return launch_mode<T_Q6_K>(mode, a, ntasks, tile, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rehip
