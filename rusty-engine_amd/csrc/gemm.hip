// Prefill / MoE GEMM: Y[N x m] = X[N x K] * W[m x K]^T with W dequantized on the fly.
//
// A workgroup of NW waves computes a BM (weight rows) x BN (activation rows) tile in K steps of
// 128 elements (4 32-element blocks, or half a 256-element super-block). The waves form a
// WM x WN grid; each owns (BM/WM) x (BN/WN) as 32 x 32 tiles of v_mfma_f32_32x32x16_bf16
// (strict mode: v_mfma_f32_32x32x2_f32) with f32 accumulators. Per step:
//   * W: BM rows x 4 chunks; a thread decodes (row, chunk) pairs from the tiled slabs
//     (consecutive threads = consecutive rows: each plane read is a contiguous 1 KiB) and
//     writes the 32 values to LDS as bf16 (or f32);
//   * X: BN rows x 128 f32, 16-byte loads (32 lanes per 512-byte row segment), converted to
//     bf16 (RNE) into LDS.
// Both are fetched with raw buffer loads: 32-bit offsets, and a read past the end of the buffer
// returns zero, so missing rows and columns cost no branches (zero weight bytes decode to 0).
// Global loads are double-buffered in registers: the raw chunks and X of step s+1 are in flight
// while the MFMAs of step s run; decoding happens when they are written to LDS. LDS rows are
// padded by 16 bytes so the 32 lanes reading one k-slice hit different banks.
//
// Dense launches use a 1-D grid ordered so that each of the 8 XCDs (workgroup w runs on XCD
// w % 8) processes a contiguous band of activation-row tiles for every weight tile, keeping that
// band of X in its L2. With `splits` > 1 the K steps are divided among workgroups, each writes
// its partial tile, and a second kernel sums the partials in split order (deterministic).
//
// Grouped launch (MoE): one task per workgroup names the expert, the weight tile and a run of
// gathered activation rows; `xrow` maps a gathered row to its activation row.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "deq.hpp"
#include "kernels.hpp"

namespace rehip {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

template <bool F32> struct Elem;
template <> struct Elem<false> { using T = __bf16; static constexpr int PAD = 8; };
template <> struct Elem<true> { using T = float; static constexpr int PAD = 4; };

// the 16 values of a run, scale*q - offset; 4-bit quants convert two per instruction (deq.hpp)
template <int T>
__device__ __forceinline__ void run_values(const Run& r, float v[16]) {
  if constexpr (kNibble<T>) {
    const float sc = r.scale * 512.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(r.q[i], false);
      const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(r.q[i], true);
      v[4 * i + 0] = __builtin_fmaf(sc, lo[0], -r.offset);
      v[4 * i + 1] = __builtin_fmaf(sc, lo[1], -r.offset);
      v[4 * i + 2] = __builtin_fmaf(sc, hi[0], -r.offset);
      v[4 * i + 3] = __builtin_fmaf(sc, hi[1], -r.offset);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = run_value(r, i);
  }
}

// 16 decoded values of a run -> LDS (two 16-byte bf16 stores, or four float4 stores)
template <int T, bool F32>
__device__ __forceinline__ void store_run(typename Elem<F32>::T* dst, const Run& r) {
  float v[16];
  run_values<T>(r, v);
  if constexpr (F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      reinterpret_cast<float4*>(dst)[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bf16x8_t o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (__bf16)v[8 * h + i];
      reinterpret_cast<bf16x8_t*>(dst)[h] = o;
    }
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

constexpr uint32_t kOob = 0x80000000u;   // a byte offset past every buffer: the load returns 0

template <int T, bool F32, bool GROUPED, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(GemmArgs p) {
  using B = Blk<T>;
  using E = typename Elem<F32>::T;
  constexpr int NT = WM * WN * 64;                 // threads
  constexpr int BK = kGemmBK;
  constexpr int LD = BK + Elem<F32>::PAD;          // LDS row stride (elements)
  constexpr int WJOBS = BM * 4 / NT;               // (row, chunk) jobs per thread per step
  constexpr int XV = BN * BK / 4 / NT;             // 16-byte X loads per thread per step
  constexpr int XR = NT / 32;                      // X rows covered by one pass of the workgroup
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(WJOBS >= 1 && XV >= 1 && TM >= 1 && TN >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) E Ws[BM * LD];
  __shared__ __attribute__((aligned(16))) E Xs[BN * LD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  int mtile, r0, rn, split = 0;
  uint32_t wbase = 0;
  if constexpr (GROUPED) {
    const GemmTask t = p.tasks[blockIdx.x];
    mtile = t.mtile;
    r0 = t.r0;
    rn = t.rn;
    wbase = (uint32_t)((size_t)t.expert * p.w_stride);
  } else {
    // XCD-aware order: XCD (blockIdx % 8) takes a contiguous run of (split, n-tile, m-tile)
    const int mt = (p.m + BM - 1) / BM, nt = (p.N + BN - 1) / BN;
    const int total = mt * nt * p.splits;
    const int per = (total + 7) / 8;
    int t = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (t >= total) return;
    split = t / (mt * nt);
    t -= split * (mt * nt);
    const int ntile = t / mt;
    mtile = t - ntile * mt;
    r0 = ntile * BN;
    rn = min(BN, p.N - r0);
  }
  const int steps_all = (p.K + BK - 1) / BK;
  const int s_begin = split * p.steps_per_split;
  const int s_end = min(steps_all, s_begin + p.steps_per_split);

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.X, p.x_bytes);

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // activation rows this thread stages: rows XR*jj + tid/32, k offset 4*(tid%32)
  const int xk = 4 * (tid & 31);
  uint32_t xoff[XV];
#pragma unroll
  for (int jj = 0; jj < XV; ++jj) {
    const int rl = XR * jj + (tid >> 5);
    uint32_t o = kOob;
    if (rl < rn) {
      const int g = r0 + rl;
      const int row = (GROUPED && p.xrow) ? p.xrow[g] : g;
      o = (uint32_t)row * (uint32_t)p.K * 4u + (uint32_t)xk * 4u;
    }
    xoff[jj] = o;
  }
  // weight jobs: row rl = j % BM of tile (BM/64)*mtile + rl/64, chunk c = j / BM
  uint32_t wrow[WJOBS];
  int wc[WJOBS];
#pragma unroll
  for (int rep = 0; rep < WJOBS; ++rep) {
    const int j = tid + NT * rep;
    const int rl = j % BM;
    const int tile = BM / 64 * mtile + (rl >> 6);
    wc[rep] = j / BM;
    wrow[rep] = tile < p.tiles ? wbase + (uint32_t)tile * (uint32_t)p.KB * (uint32_t)B::SLAB : kOob;
  }

  typename B::CR wraw[WJOBS];
  float4 xraw[XV];

  auto prefetch = [&](int s) {
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) {
      const int j = tid + NT * rep;
      const int tl = (j % BM) & 63;
      int kb, cc;
      if constexpr (B::QK == 32) { kb = 4 * s + wc[rep]; cc = 0; }
      else { kb = s >> 1; cc = 4 * (s & 1) + wc[rep]; }
      const uint32_t slab = (kb < p.KB && wrow[rep] != kOob) ? wrow[rep] + (uint32_t)kb * (uint32_t)B::SLAB : kOob;
      B::bload_chunk(wr, slab, tl, cc, wraw[rep]);
    }
    const bool kin = s * BK + xk < p.K;
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) {
      const uint32_t o = (kin && xoff[jj] != kOob) ? xoff[jj] + (uint32_t)(s * BK) * 4u : kOob;
      const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)o, 0, 0);
      xraw[jj] = make_float4(__int_as_float(v[0]), __int_as_float(v[1]), __int_as_float(v[2]), __int_as_float(v[3]));
    }
  };

  auto commit = [&](int s) {
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) {
      const int j = tid + NT * rep;
      const int rl = j % BM, c = j / BM;
      E* dst = Ws + rl * LD;
      int cc, kl;
      if constexpr (B::QK == 32) { cc = 0; kl = 32 * c; }
      else { cc = 4 * (s & 1) + c; kl = -128 * (s & 1); }
      Run a, b;
      B::decode_chunk(wraw[rep], cc, a, b);
      store_run<T, F32>(dst + kl + a.e, a);
      store_run<T, F32>(dst + kl + b.e, b);
    }
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) store4<F32>(Xs + (XR * jj + (tid >> 5)) * LD + xk, xraw[jj]);
  };

  if (s_begin < s_end) prefetch(s_begin);
  for (int s = s_begin; s < s_end; ++s) {
    if (s > s_begin) __syncthreads();    // previous step's MFMA reads are done
    commit(s);
    __syncthreads();
    if (s + 1 < s_end) prefetch(s + 1);  // in flight during the MFMAs below
    if constexpr (!F32) {
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        bf16x8_t av[TM], bv[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          av[i] = *reinterpret_cast<const bf16x8_t*>(Ws + (BM / WM * wm + 32 * i + (lane & 31)) * LD + 16 * kk + 8 * (lane >> 5));
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bv[j] = *reinterpret_cast<const bf16x8_t*>(Xs + (BN / WN * wn + 32 * j + (lane & 31)) * LD + 16 * kk + 8 * (lane >> 5));
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
        for (int i = 0; i < TM; ++i) av[i] = Ws[(BM / WM * wm + 32 * i + (lane & 31)) * LD + 2 * kk + (lane >> 5)];
#pragma unroll
        for (int j = 0; j < TN; ++j) bv[j] = Xs[(BN / WN * wn + 32 * j + (lane & 31)) * LD + 2 * kk + (lane >> 5)];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: D[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), register 4*(i/8) + i%4
  float* Y = p.splits > 1 ? p.partial + (size_t)split * p.N * p.ldy : p.Y;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int xl = BN / WN * wn + 32 * j + (lane & 31);
      if (xl >= rn) continue;
      float* yrow = Y + (size_t)(r0 + xl) * p.ldy;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int wr0 = BM * mtile + BM / WM * wm + 32 * i + 8 * q + 4 * (lane >> 5);
        if (wr0 + 3 < p.m) {
          *reinterpret_cast<float4*>(yrow + wr0) =
              make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (wr0 + e < p.m) yrow[wr0 + e] = acc[i][j][4 * q + e];
        }
      }
    }
  }
}

// Y[i] = sum over splits, in split order, of partial[split][i]  (i over N * ldy)
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float* __restrict__ partial, float* __restrict__ y,
                                                          size_t n, int splits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float s = partial[i];
  for (int sp = 1; sp < splits; ++sp) s += partial[(size_t)sp * n + i];
  y[i] = s;
}

template <int T, bool F32, int BM, int BN, int WM, int WN>
static hipError_t launch_shape(const GemmArgs& a, int ntasks, hipStream_t s) {
  constexpr int NT = WM * WN * 64;
  if (a.tasks) {
    hipLaunchKernelGGL((gemm_kernel<T, F32, true, BM, BN, WM, WN>), dim3((unsigned)ntasks), dim3(NT), 0, s, a);
    return hipGetLastError();
  }
  const int total = ((a.m + BM - 1) / BM) * ((a.N + BN - 1) / BN) * a.splits;
  const int grid = (total + 7) / 8 * 8;
  hipLaunchKernelGGL((gemm_kernel<T, F32, false, BM, BN, WM, WN>), dim3((unsigned)grid), dim3(NT), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  const size_t n = (size_t)a.N * a.ldy;
  hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a.partial, a.Y, n,
                     a.splits);
  return hipGetLastError();
}

template <int T, bool F32>
static hipError_t launch_t(const GemmArgs& a, int ntasks, GemmTile tile, hipStream_t s) {
  switch (tile) {
    case GemmTile::k128x256:
      // bf16 only: the f32 tile pair would need 198 KiB of LDS
      if constexpr (F32) return hipErrorInvalidValue;
      else return launch_shape<T, F32, 128, 256, 2, 4>(a, ntasks, s);
    case GemmTile::k128x128: return launch_shape<T, F32, 128, 128, 2, 2>(a, ntasks, s);
    default: return launch_shape<T, F32, 64, 64, 2, 2>(a, ntasks, s);
  }
}

template <int T>
static hipError_t launch_mode(int mode, const GemmArgs& a, int ntasks, GemmTile tile, hipStream_t s) {
  return mode == 1 ? launch_t<T, true>(a, ntasks, tile, s) : launch_t<T, false>(a, ntasks, tile, s);
}

GemmPlan plan_gemm(int m, int n, int K, int mode) {
  GemmPlan pl;
  const int steps = (K + kGemmBK - 1) / kGemmBK;
  const long t128 = (long)((m + 127) / 128) * ((n + 127) / 128);
  const long t256 = (long)((m + 127) / 128) * ((n + 255) / 256);
  const long t64 = (long)((m + 63) / 64) * ((n + 63) / 64);
  if (mode == 0 && n >= 512 && t256 >= 200) {
    pl.tile = GemmTile::k128x256;
  } else if (t128 >= 200) {
    pl.tile = GemmTile::k128x128;
  } else {
    pl.tile = GemmTile::k64x64;
    // few tiles over a deep K: split the K steps when the partial tiles stay small
    if (t64 < 128 && steps >= 8) {
      long splits = (256 + t64 - 1) / t64;
      splits = std::min<long>(splits, steps / 2);
      const long partial_bytes = splits * (long)n * m * 4;
      if (partial_bytes <= (16l << 20) && splits > 1) pl.splits = (int)splits;
    }
  }
  pl.steps_per_split = (steps + pl.splits - 1) / pl.splits;
  pl.splits = (steps + pl.steps_per_split - 1) / pl.steps_per_split;
  return pl;
}

hipError_t launch_gemm(uint32_t type, int mode, const GemmArgs& a, int ntasks, GemmTile tile, hipStream_t s) {
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
