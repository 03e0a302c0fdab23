// Weights decoded in registers straight into bf16 MFMA operands, shared by the register-decoded
// expert GEMMs (moe_qmma.hip) and the few-row dense GEMM (skinny.hip).
//
// Lane r of a wave loads row r's raw 32-element chunk from the tiled slab (lane = row), decodes
// both 16-element runs (scale * q - offset in f32, exactly as the reference's dequantizer), rounds
// them to bf16 (or splits them into bf16 roundings and remainders for the f32 mode), and
// v_permlane32_swap exchanges lane halves so that lanes 0-31 / 32-63 hold k 0-7 / 8-15 of rows
// 0-31 (the B operand of row group 0) and of rows 32-63 (row group 1) of a v_mfma_f32_32x32x16_bf16.
#pragma once

#include <hip/hip_runtime.h>

#include "deq.hpp"

namespace rehip {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

constexpr uint32_t kQOob = 0x80000000u;   // a byte offset past every buffer: the load returns 0

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// The 16 values of a run (scale * q - offset, each exact in f32 as in the reference's
// dequantizer) in f32.
template <int T>
__device__ __forceinline__ void run_f32(const Run& r, float v[16]) {
  if constexpr (kNibble<T>) {
    // 4-bit quants as fp8 e4m3 bytes are exactly q * 2^-9 (two per instruction)
    const float sc = r.scale * 512.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8(r.q[i], false);
      const f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8(r.q[i], true);
      v[4 * i + 0] = __builtin_fmaf(sc, a[0], -r.offset);
      v[4 * i + 1] = __builtin_fmaf(sc, a[1], -r.offset);
      v[4 * i + 2] = __builtin_fmaf(sc, b[0], -r.offset);
      v[4 * i + 3] = __builtin_fmaf(sc, b[1], -r.offset);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = run_value(r, i);
  }
}

// The run rounded to bf16 pairs: lo = elements 0-7, hi = elements 8-15.
template <int T>
__device__ __forceinline__ void run_bf16(const Run& r, uint32_t lo[4], uint32_t hi[4]) {
  float v[16];
  run_f32<T>(r, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
    hi[i] = pack_bf16(v[8 + 2 * i], v[8 + 2 * i + 1]);
  }
}

// Split form (f32 mode): the bf16 rounding of each value (lo / hi as run_bf16) and the bf16
// rounding of what that leaves (rlo / rhi), so each value is held to 2^-16 relative.
template <int T>
__device__ __forceinline__ void run_bf16_split(const Run& r, uint32_t lo[4], uint32_t hi[4], uint32_t rlo[4],
                                               uint32_t rhi[4]) {
  float v[16];
  run_f32<T>(r, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
    hi[i] = pack_bf16(v[8 + 2 * i], v[8 + 2 * i + 1]);
    const bf16x2_t l = __builtin_bit_cast(bf16x2_t, lo[i]), h = __builtin_bit_cast(bf16x2_t, hi[i]);
    rlo[i] = pack_bf16(v[2 * i] - (float)l[0], v[2 * i + 1] - (float)l[1]);
    rhi[i] = pack_bf16(v[8 + 2 * i] - (float)h[0], v[8 + 2 * i + 1] - (float)h[1]);
  }
}

// lo/hi of this lane's row -> B operands of row group 0 (rows 0-31) and 1 (rows 32-63): lanes
// 0-31 take k 0-7 (lo), lanes 32-63 k 8-15 (hi) of row lane % 32 of the group.
__device__ __forceinline__ void halves_to_frags(const uint32_t lo[4], const uint32_t hi[4], bf16x8_t& g0,
                                                bf16x8_t& g1) {
  uint32_t a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // swaps lanes 32-63 of lo with lanes 0-31 of hi: lo becomes group 0's operand, hi group 1's
    const auto s = __builtin_amdgcn_permlane32_swap(lo[i], hi[i], false, false);
    a[i] = s[0];
    b[i] = s[1];
  }
  g0 = __builtin_bit_cast(bf16x8_t, make_uint4(a[0], a[1], a[2], a[3]));
  g1 = __builtin_bit_cast(bf16x8_t, make_uint4(b[0], b[1], b[2], b[3]));
}

// B operands of both runs of a decoded chunk, both row groups
struct Frags {
  bf16x8_t a0, a1, b0, b1;   // run a (groups 0, 1), run b (groups 0, 1)
  int ea, eb;                // element offsets of runs a and b inside the block
};

template <int T>
__device__ __forceinline__ void decode_frags(const typename Blk<T>::CR& raw, int cc, Frags& f) {
  Run a, b;
  Blk<T>::decode_chunk(raw, cc, a, b);
  uint32_t lo[4], hi[4];
  run_bf16<T>(a, lo, hi);
  halves_to_frags(lo, hi, f.a0, f.a1);
  run_bf16<T>(b, lo, hi);
  halves_to_frags(lo, hi, f.b0, f.b1);
  f.ea = a.e;
  f.eb = b.e;
}

// both parts of the split form: f (the bf16 roundings) and fr (the remainders)
template <int T>
__device__ __forceinline__ void decode_frags_split(const typename Blk<T>::CR& raw, int cc, Frags& f, Frags& fr) {
  Run a, b;
  Blk<T>::decode_chunk(raw, cc, a, b);
  uint32_t lo[4], hi[4], rlo[4], rhi[4];
  run_bf16_split<T>(a, lo, hi, rlo, rhi);
  halves_to_frags(lo, hi, f.a0, f.a1);
  halves_to_frags(rlo, rhi, fr.a0, fr.a1);
  run_bf16_split<T>(b, lo, hi, rlo, rhi);
  halves_to_frags(lo, hi, f.b0, f.b1);
  halves_to_frags(rlo, rhi, fr.b0, fr.b1);
  f.ea = fr.ea = a.e;
  f.eb = fr.eb = b.e;
}

}  // namespace
}  // namespace rehip
