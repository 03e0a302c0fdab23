// Few-row dense GEMM: Y[N x m] = X[N x K] W^T for 2 <= N <= 64 activation rows (QMat::matmul,
// src/qmat.rs:169-272, at the row counts of a short prompt or a batched decode), bf16 or f32 mode.
//
// One workgroup of four waves per (64-row weight tile, K slice of whole blocks). The slice of
// every activation row (zero-padded to 64 rows and to K) is staged once in LDS as bf16 (f32 mode:
// the bf16 rounding and, beside it, the bf16 rounding of the remainder). The waves then take the
// slice's 32-element chunks in turn: lane r loads weight row r's chunk from the tiled slab (one
// contiguous plane read per wave), decodes it straight into MFMA B operands (qfrag.hpp), and each
// of the chunk's two runs feeds v_mfma_f32_32x32x16_bf16 for both 32-row weight groups and both
// 32-row token tiles (f32 mode: three MFMAs per product, x_hi w_hi + x_hi w_lo + x_lo w_hi). A
// weight is read once and decoded once per launch; nothing but the activations touches LDS.
//
// The four waves' sums are added in wave order through LDS, each wave adding and writing a quarter
// of the tile. With one K slice the tile's output is final and goes out with streaming stores;
// otherwise each slice writes its partial tile and the split-K reduce sums them in slice order, so
// results do not depend on scheduling.
//
// The 1-D grid is ordered slice-major across the XCDs (workgroup w runs on XCD w % 8): the tiles
// that share one slice of X run on one XCD, so the slice is fetched into that XCD's L2 once.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "deq.hpp"
#include "kernels.hpp"
#include "qfrag.hpp"

namespace rehip {

namespace {

constexpr int kSkinnyRows = 64;                  // activation rows per launch (two token tiles)
constexpr int kSkinnyPad = 8;                    // bf16 of padding per staged row (bank spread)

template <int T, bool SP>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(SkinnyArgs p) {
  using B = Blk<T>;
  constexpr int NCH = B::NCH;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const int total = p.tiles * p.splits;
  const int per = (total + 7) / 8;
  const int u = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (u >= total) return;
  const int split = u / p.tiles, tile = u - split * p.tiles;
  const int kb0 = split * p.blocks_per_split;
  const int kb1 = min(p.KB, kb0 + p.blocks_per_split);
  const int ks = p.blocks_per_split * B::QK;     // staged k per row
  const int ld = ks + kSkinnyPad;                // LDS row stride (bf16)
  __bf16* xh = reinterpret_cast<__bf16*>(smem);
  __bf16* xl = xh + kSkinnyRows * ld;            // remainders (f32 mode)

  // the wave's first two chunks of weights go out before the activations are staged
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  const uint32_t tbase = (uint32_t)tile * (uint32_t)p.KB * (uint32_t)B::SLAB;
  const int c0 = kb0 * NCH, c1 = kb1 * NCH;
  auto load = [&](int c, typename B::CR& raw) {
    const int kb = c / NCH, cc = c - kb * NCH;
    const uint32_t slab = c < c1 ? tbase + (uint32_t)kb * (uint32_t)B::SLAB : 0x80000000u;
    B::bload_chunk(wr, slab, lane, cc, raw);
  };
  typename B::CR rawA, rawB;
  load(c0 + wave, rawA);
  load(c0 + wave + 4, rawB);

  // stage the slice: row r < N, k = kb0 * QK + j < K, else zero (bf16 RNE; f32 mode also the
  // remainder)
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.X, p.x_bytes);
  const int nt = (p.N + 31) >> 5;                // 32-row token tiles holding rows (uniform)
  const int q4 = ks / 4;                         // float4 per staged row
  const int nq = 32 * nt * q4;                   // rows past N inside the last tile read zeros
  // sixteen loads per thread in flight before any is converted (a loop that waits for each load
  // in turn costs a memory round trip per iteration)
  constexpr int SU = 16;
  for (int i0 = 0; i0 < nq; i0 += SU * 256) {
    i32x4_t v[SU];
#pragma unroll
    for (int uu = 0; uu < SU; ++uu) {
      const int i = i0 + uu * 256 + (int)threadIdx.x;
      const int r = i / q4, j = 4 * (i - r * q4);
      const int k = kb0 * B::QK + j;
      const uint32_t off =
          i < nq && r < p.N && k < p.K ? ((uint32_t)r * (uint32_t)p.K + (uint32_t)k) * 4u : 0x80000000u;
      v[uu] = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0);
    }
#pragma unroll
    for (int uu = 0; uu < SU; ++uu) {
      const int i = i0 + uu * 256 + (int)threadIdx.x;
      if (i >= nq) break;
      const int r = i / q4, j = 4 * (i - r * q4);
      const float f[4] = {__int_as_float(v[uu][0]), __int_as_float(v[uu][1]), __int_as_float(v[uu][2]),
                          __int_as_float(v[uu][3])};
      uint32_t h[2], l[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        h[e] = pack_bf16(f[2 * e], f[2 * e + 1]);
        if constexpr (SP) {
          const bf16x2_t hb = __builtin_bit_cast(bf16x2_t, h[e]);
          l[e] = pack_bf16(f[2 * e] - (float)hb[0], f[2 * e + 1] - (float)hb[1]);
        }
      }
      *reinterpret_cast<uint2*>(xh + r * ld + j) = make_uint2(h[0], h[1]);
      if constexpr (SP) *reinterpret_cast<uint2*>(xl + r * ld + j) = make_uint2(l[0], l[1]);
    }
  }
  __syncthreads();

  f32x16_t acc[2][2];                            // [weight row group][token tile]
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][j][r] = 0.0f;

  // A operand of a run at element e of block kb: token row 32 j + lane % 32, k e + 8 (lane / 32)
  auto xop = [&](const __bf16* src, int kb, int e, int j) {
    const int row = 32 * j + (lane & 31);
    return *reinterpret_cast<const bf16x8_t*>(src + row * ld + (kb - kb0) * B::QK + e + 8 * (lane >> 5));
  };
  auto step = [&](int c, const typename B::CR& raw) {
    const int kb = c / NCH, cc = c - kb * NCH;
    if constexpr (SP) {
      Frags f, fr;
      decode_frags_split<T>(raw, cc, f, fr);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j >= nt) break;
        const bf16x8_t xa = xop(xh, kb, f.ea, j), xb = xop(xh, kb, f.eb, j);
        const bf16x8_t xal = xop(xl, kb, f.ea, j), xbl = xop(xl, kb, f.eb, j);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, f.a0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, f.a1, acc[1][j], 0, 0, 0);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, f.b0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, f.b1, acc[1][j], 0, 0, 0);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, fr.a0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, fr.a1, acc[1][j], 0, 0, 0);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xal, f.a0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xal, f.a1, acc[1][j], 0, 0, 0);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, fr.b0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, fr.b1, acc[1][j], 0, 0, 0);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xbl, f.b0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xbl, f.b1, acc[1][j], 0, 0, 0);
      }
    } else {
      Frags f;
      decode_frags<T>(raw, cc, f);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j >= nt) break;
        const bf16x8_t xa = xop(xh, kb, f.ea, j), xb = xop(xh, kb, f.eb, j);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, f.a0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, f.a1, acc[1][j], 0, 0, 0);
        acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, f.b0, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, f.b1, acc[1][j], 0, 0, 0);
      }
    }
  };
  // chunks wave, wave + 4, ... of the slice, two in flight: a chunk's buffer is refilled as soon
  // as it has been decoded
  for (int c = c0 + wave; c < c1; c += 8) {
    step(c, rawA);
    if (c + 4 >= c1) break;
    if (c + 8 < c1) load(c + 8, rawA);
    step(c + 4, rawB);
    if (c + 12 < c1) load(c + 12, rawB);
  }

  // the four waves' sums: every wave parks its accumulators in LDS (four floats per lane per
  // weight group, token tile and quad of accumulator registers; the staging is no longer read),
  // then wave q adds quad q of the four waves in wave order and writes it
  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(smem);
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (j >= nt) break;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        red[((wave * 4 + g * 2 + j) * 4 + q) * 64 + lane] =
            f32x4_t{acc[g][j][4 * q], acc[g][j][4 * q + 1], acc[g][j][4 * q + 2], acc[g][j][4 * q + 3]};
    }
  __syncthreads();
  // D[token][row]: lane holds weight row 32 g + lane % 32 and, in quad q, tokens
  // 32 j + 8 q + 4 (lane / 32) + e for e < 4
  float* out = p.splits > 1 ? p.partial + (size_t)split * p.N * p.ldy : p.Y;
  const int q = wave;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int row = tile * 64 + 32 * g + (lane & 31);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (j >= nt) break;
      const int tok0 = 32 * j + 8 * q + 4 * (lane >> 5);
      if (tok0 >= p.N || row >= p.m) continue;
      f32x4_t v = red[((0 * 4 + g * 2 + j) * 4 + q) * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += red[((w * 4 + g * 2 + j) * 4 + q) * 64 + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = tok0 + e;
        if (tok >= p.N) break;
        float* dst = out + (size_t)tok * p.ldy + row;
        if (p.splits > 1) *dst = v[e];
        else __builtin_nontemporal_store(v[e], dst);
      }
    }
  }
}

template <int T>
hipError_t launch_skinny_t(const SkinnyArgs& a, bool split_operands, hipStream_t s) {
  const size_t lds = skinny_lds_bytes(Blk<T>::QK * a.blocks_per_split, split_operands);
  const unsigned grid = (unsigned)((a.tiles * a.splits + 7) / 8 * 8);
  if (split_operands)
    hipLaunchKernelGGL((gemm_skinny_kernel<T, true>), dim3(grid), dim3(256), lds, s, a);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<T, false>), dim3(grid), dim3(256), lds, s, a);
  return hipGetLastError();
}

}  // namespace

size_t skinny_lds_bytes(int staged_k, bool split_operands) {
  const size_t stage = (size_t)kSkinnyRows * (staged_k + kSkinnyPad) * 2 * (split_operands ? 2 : 1);
  return std::max<size_t>(stage, 4 * 64 * 64 * sizeof(float));   // the wave fold reuses it
}

SkinnyPlan plan_skinny(int m, int K, int qk) {
  SkinnyPlan pl;
  const int tiles = (m + 63) / 64, kb = (K + qk - 1) / qk;
  // K slices until ~256 workgroups run, a slice at most kSkinnyMaxK elements (LDS)
  const int max_bps = std::max(1, kSkinnyMaxK / qk);
  int splits = std::max(1, std::min(kb, (256 + tiles - 1) / tiles));
  int bps = std::min(max_bps, (kb + splits - 1) / splits);
  pl.blocks_per_split = bps;
  pl.splits = (kb + bps - 1) / bps;
  return pl;
}

hipError_t launch_gemm_skinny(uint32_t type, const SkinnyArgs& a, bool split_operands, hipStream_t s) {
  if (a.N < 1 || a.N > kSkinnyRows || a.blocks_per_split < 1 || a.splits < 1) return hipErrorInvalidValue;
  switch (type) {
    case T_Q4_0: return launch_skinny_t<T_Q4_0>(a, split_operands, s);
    case T_Q5_0: return launch_skinny_t<T_Q5_0>(a, split_operands, s);
    case T_Q8_0: return launch_skinny_t<T_Q8_0>(a, split_operands, s);
    case T_Q4_K: return launch_skinny_t<T_Q4_K>(a, split_operands, s);
    case T_Q5_K: return launch_skinny_t<T_Q5_K>(a, split_operands, s);
    case T_Q6_K: return launch_skinny_t<T_Q6_K>(a, split_operands, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rehip
