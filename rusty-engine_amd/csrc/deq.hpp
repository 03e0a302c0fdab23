// Device-side block decoding for the tiled-slab layout (common.hpp).
//
// Every block is read as "chunks" of 32 quants. A chunk is two runs of 16 elements, run A at
// element offset eA and run B at eB inside the block; each run has an affine map
//     value = scale * q - offset,   q an unsigned integer quant (0..255)
// which reproduces the reference dequantizers (src/quant.rs:106-357) exactly: every product
// involved is exact in f32 and the subtraction rounds once, where the reference rounds.
//   Q4_0  d*(q-8)        -> scale d,       offset 8d          (1 chunk, runs 0/16)
//   Q5_0  d*(q-16)       -> scale d,       offset 16d         (1 chunk, runs 0/16)
//   Q8_0  d*qs (signed)  -> q = qs+128,    offset 128d        (1 chunk, runs 0/16)
//   Q4_K  d*sc*q - dmin*m                                     (8 chunks)
//   Q5_K  same with the 5th bit                               (8 chunks)
//   Q6_K  d*sc*(q-32)    -> scale d*sc,    offset 32*d*sc     (8 chunks)
// The affine form lets a dot product factor the scale out of the 16-element sum:
//   sum(v_i x_i) = scale * sum(q_i x_i) - offset * sum(x_i).
// Quants are delivered four per dword (one byte each) so they convert with v_cvt_f32_ubyte.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "common.hpp"

namespace rehip {

// binary16 -> f32 (src/quant.rs:25-45): v_cvt_f32_f16 widens every finite value and infinity
// exactly, subnormals included (f16 denormals are kept in the kernel float mode). A signalling NaN
// comes out quieted with its payload; the reference's value keeps the signalling bit, but every
// dequantized value multiplies the scale, and that multiplication quiets it on both sides.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

template <int T> struct Blk;

struct Run {
  uint32_t q[4];    // 16 quants, one per byte, element order
  float scale, offset;
  int e;            // element offset of the run inside the block
};

// Quants of at most 4 bits (Q4_0, Q4_K): a byte 0000qqqq read as an OCP E4M3 value is exactly
// q * 2^-9 (subnormal for q < 8, exponent 1 for q >= 8), so v_cvt_pk_f32_fp8 turns two of them
// into floats with one instruction; the 2^9 goes into the run's scale (exact).
template <int T> inline constexpr bool kNibble = (T == T_Q4_0 || T == T_Q4_K);
constexpr float kNibbleUnit = 1.0f / 512.0f;

// Quant bias of the types whose reference formula multiplies a signed quant, (q - bias) * d
// (Q4_0 8, Q5_0 16, Q8_0 128, Q6_K 32); 0 for Q4_K/Q5_K (d*sc*q - dmin*m).
template <int T> inline constexpr int kBias = 0;
template <> inline constexpr int kBias<T_Q4_0> = 8;
template <> inline constexpr int kBias<T_Q5_0> = 16;
template <> inline constexpr int kBias<T_Q8_0> = 128;
template <> inline constexpr int kBias<T_Q6_K> = 32;
// run_dot reads the per-16 sums of x only where it takes an offset out after the products: the
// 4-bit types (their bias or min) and Q5_K (its min)
template <int T> inline constexpr bool kNeedXs16 = kNibble<T> || kBias<T> == 0;

// Plane slab offsets: plane p of a 64-row slab starts at 64 * (sum of widths before p).
//
// Each Blk<T> offers two ways in:
//   chunk(slab, lane, c, a, b)   loads only the planes chunk c needs, then decodes it
//                                (GEMM staging and the dequant kernel, c may be a runtime value);
//   load(slab, lane, r) + decode(r, c, a, b)
//                                loads every plane of the block into registers first, then
//                                decodes chunk after chunk (GEMV; c is a compile-time constant
//                                after unrolling, so r.p[...] stays in registers).

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Raw buffer loads through a resource covering a whole matrix (or all experts): byte offsets are
// 32-bit and a read past num_records returns zero, so padding rows/columns need no branches
// (zero bytes decode to zero weights for every type: every scale is then 0).
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bld2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
// Streaming weight loads: the uniform part of the offset in soffset (a scalar register, so no
// per-lane address arithmetic when the base moves) and the nontemporal cache policy (weights are
// read once per launch; on MI355X a plain streaming read tops out near 6.2 TB/s and a
// nontemporal one near 7.0 TB/s).
constexpr int kLoadNT = 2;   // buffer load aux: nontemporal
__device__ __forceinline__ uint4 sld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kLoadNT);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
__device__ __forceinline__ uint32_t sld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, kLoadNT);
}
__device__ __forceinline__ uint32_t sld2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, kLoadNT);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// nibble split of 16 quant bytes: low nibbles -> run a, high nibbles -> run b
__device__ __forceinline__ void split_nibbles(const uint4& qs, Run& a, Run& b) {
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) { a.q[i] = w[i] & 0x0F0F0F0Fu; b.q[i] = (w[i] >> 4) & 0x0F0F0F0Fu; }
}

template <> struct Blk<T_Q4_0> {
  static constexpr int QK = 32, BB = 18, NCH = 1, NP = 1;
  static constexpr int SLAB = 64 * BB;
  struct R { uint4 p[NP]; uint32_t t0, t1; };
  __device__ static void load(const uint8_t* slab, int lane, R& r) {
    r.p[0] = ld16(slab + lane * 16);
    r.t0 = ld2(slab + 1024 + lane * 2);
    r.t1 = 0;
  }
  __device__ static void bload_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, int c, R& r) {
    (void)c;
    r.p[0] = bld16(rs, slab + lane * 16);
    r.t0 = bld2(rs, slab + 1024 + lane * 2);
    r.t1 = 0;
  }
  // whole block through a buffer resource, slab at scalar offset soff
  __device__ static void sload(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
    r.p[0] = sld16(rs, lane * 16, soff);
    r.t0 = sld2(rs, lane * 2, soff + 1024);
    r.t1 = 0;
  }
  __device__ static void decode(const R& r, int c, Run& a, Run& b) {
    (void)c;
    split_nibbles(r.p[0], a, b);
    const float d = f16_bits_to_f32(r.t0);
    a.scale = b.scale = d;
    a.offset = b.offset = 8.0f * d;
    a.e = 0; b.e = 16;
  }
  // raw data of one chunk (the whole block for 32-element types)
  using CR = R;
  __device__ static void load_chunk(const uint8_t* slab, int lane, int c, CR& r) { (void)c; load(slab, lane, r); }
  __device__ static void decode_chunk(const CR& r, int c, Run& a, Run& b) { decode(r, c, a, b); }
  __device__ static void chunk(const uint8_t* slab, int lane, int c, Run& a, Run& b) {
    R r; load(slab, lane, r); decode(r, c, a, b);
  }
};

// spread bits 0..3 of v to bit 4 of bytes 0..3: the nibble moved to bits 4..7, times
// 1 + 2^7 + 2^14 + 2^21, puts copies at shifts 0, 7, 14, 21 (no overlap, so no carries) and bit b
// of copy b at 4 + b + 7b = 8b + 4. Both factors fit 24 bits, so this is the full-rate
// v_mul_u32_u24 (a shift-or chain was folded by the compiler into the quarter-rate v_mul_lo_u32).
__device__ __forceinline__ uint32_t bits4_to_byte_bit4(uint32_t v) {
  return __umul24((v & 0xFu) << 4, 0x00204081u) & 0x10101010u;
}

template <> struct Blk<T_Q5_0> {
  static constexpr int QK = 32, BB = 22, NCH = 1, NP = 1;
  static constexpr int SLAB = 64 * BB;
  struct R { uint4 p[NP]; uint32_t t0, t1; };
  __device__ static void load(const uint8_t* slab, int lane, R& r) {
    r.p[0] = ld16(slab + lane * 16);
    r.t0 = ld4(slab + 1024 + lane * 4);      // qh
    r.t1 = ld2(slab + 1280 + lane * 2);      // d
  }
  __device__ static void bload_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, int c, R& r) {
    (void)c;
    r.p[0] = bld16(rs, slab + lane * 16);
    r.t0 = bld4(rs, slab + 1024 + lane * 4);
    r.t1 = bld2(rs, slab + 1280 + lane * 2);
  }
  __device__ static void sload(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
    r.p[0] = sld16(rs, lane * 16, soff);
    r.t0 = sld4(rs, lane * 4, soff + 1024);
    r.t1 = sld2(rs, lane * 2, soff + 1280);
  }
  __device__ static void decode(const R& r, int c, Run& a, Run& b) {
    (void)c;
    const uint32_t w[4] = {r.p[0].x, r.p[0].y, r.p[0].z, r.p[0].w};
    const uint32_t qh = r.t0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a.q[i] = (w[i] & 0x0F0F0F0Fu) | bits4_to_byte_bit4(qh >> (4 * i));
      b.q[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) | bits4_to_byte_bit4(qh >> (16 + 4 * i));
    }
    const float d = f16_bits_to_f32(r.t1);
    a.scale = b.scale = d;
    a.offset = b.offset = 16.0f * d;
    a.e = 0; b.e = 16;
  }
  // raw data of one chunk (the whole block for 32-element types)
  using CR = R;
  __device__ static void load_chunk(const uint8_t* slab, int lane, int c, CR& r) { (void)c; load(slab, lane, r); }
  __device__ static void decode_chunk(const CR& r, int c, Run& a, Run& b) { decode(r, c, a, b); }
  __device__ static void chunk(const uint8_t* slab, int lane, int c, Run& a, Run& b) {
    R r; load(slab, lane, r); decode(r, c, a, b);
  }
};

template <> struct Blk<T_Q8_0> {
  static constexpr int QK = 32, BB = 34, NCH = 1, NP = 2;
  static constexpr int SLAB = 64 * BB;
  struct R { uint4 p[NP]; uint32_t t0, t1; };
  __device__ static void load(const uint8_t* slab, int lane, R& r) {
    r.p[0] = ld16(slab + lane * 16);
    r.p[1] = ld16(slab + 1024 + lane * 16);
    r.t0 = ld2(slab + 2048 + lane * 2);
    r.t1 = 0;
  }
  __device__ static void bload_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, int c, R& r) {
    (void)c;
    r.p[0] = bld16(rs, slab + lane * 16);
    r.p[1] = bld16(rs, slab + 1024 + lane * 16);
    r.t0 = bld2(rs, slab + 2048 + lane * 2);
    r.t1 = 0;
  }
  __device__ static void sload(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
    r.p[0] = sld16(rs, lane * 16, soff);
    r.p[1] = sld16(rs, lane * 16, soff + 1024);
    r.t0 = sld2(rs, lane * 2, soff + 2048);
    r.t1 = 0;
  }
  __device__ static void decode(const R& r, int c, Run& a, Run& b) {
    (void)c;
    a.q[0] = r.p[0].x ^ 0x80808080u; a.q[1] = r.p[0].y ^ 0x80808080u;
    a.q[2] = r.p[0].z ^ 0x80808080u; a.q[3] = r.p[0].w ^ 0x80808080u;
    b.q[0] = r.p[1].x ^ 0x80808080u; b.q[1] = r.p[1].y ^ 0x80808080u;
    b.q[2] = r.p[1].z ^ 0x80808080u; b.q[3] = r.p[1].w ^ 0x80808080u;
    const float d = f16_bits_to_f32(r.t0);
    a.scale = b.scale = d;
    a.offset = b.offset = 128.0f * d;
    a.e = 0; b.e = 16;
  }
  // raw data of one chunk (the whole block for 32-element types)
  using CR = R;
  __device__ static void load_chunk(const uint8_t* slab, int lane, int c, CR& r) { (void)c; load(slab, lane, r); }
  __device__ static void decode_chunk(const CR& r, int c, Run& a, Run& b) { decode(r, c, a, b); }
  __device__ static void chunk(const uint8_t* slab, int lane, int c, Run& a, Run& b) {
    R r; load(slab, lane, r); decode(r, c, a, b);
  }
};

// src/quant.rs:250-258 on the 12 scale bytes held in three dwords s0 (bytes 0-3), s1 (4-7),
// s2 (8-11) of the head plane.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = (s0 >> (8 * j)) & 63u;
    m = (s1 >> (8 * j)) & 63u;
  } else {
    const int k = j - 4;
    const uint32_t hi = (s2 >> (8 * k)) & 0xFFu;
    sc = (hi & 0xFu) | (((s0 >> (8 * k + 6)) & 3u) << 4);
    m = (hi >> 4) | (((s1 >> (8 * k + 6)) & 3u) << 4);
  }
}

// Q4_K/Q5_K head plane: d, dmin and the packed (scale, min) of sub-blocks 2g, 2g+1
__device__ __forceinline__ void k4_scales(const uint4& head, int g, Run& a, Run& b) {
  const float d = f16_bits_to_f32(head.x & 0xFFFFu);
  const float dmin = f16_bits_to_f32(head.x >> 16);
  uint32_t sc0, m0, sc1, m1;
  scale_min_k4(2 * g, head.y, head.z, head.w, sc0, m0);
  scale_min_k4(2 * g + 1, head.y, head.z, head.w, sc1, m1);
  a.scale = d * (float)sc0; a.offset = dmin * (float)m0;
  b.scale = d * (float)sc1; b.offset = dmin * (float)m1;
}

template <> struct Blk<T_Q4_K> {
  static constexpr int QK = 256, BB = 144, NCH = 8, NP = 9;
  static constexpr int SLAB = 64 * BB;
  struct R { uint4 p[NP]; uint32_t t0, t1; };
  // chunk c = 2g + h: qs bytes 32g + 16h .. +16 (plane 1 + c); low nibbles -> elements
  // 64g + 16h + i (sub-block 2g), high nibbles -> 64g + 32 + 16h + i (sub-block 2g + 1)
  __device__ static void dec(const uint4& head, const uint4& qs, int c, Run& a, Run& b) {
    const int g = c >> 1, h = c & 1;
    split_nibbles(qs, a, b);
    k4_scales(head, g, a, b);
    a.e = 64 * g + 16 * h; b.e = a.e + 32;
  }
  __device__ static void load(const uint8_t* slab, int lane, R& r) {
#pragma unroll
    for (int p = 0; p < NP; ++p) r.p[p] = ld16(slab + 1024 * p + lane * 16);
    r.t0 = r.t1 = 0;
  }
  __device__ static void sload(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
#pragma unroll
    for (int p = 0; p < NP; ++p) r.p[p] = sld16(rs, lane * 16, soff + 1024 * p);
    r.t0 = r.t1 = 0;
  }
  // the planes chunks 4H .. 4H + 3 read (head and their four qs planes)
  template <int H> __device__ static void sload_half(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
    r.p[0] = sld16(rs, lane * 16, soff);
#pragma unroll
    for (int j = 0; j < 4; ++j) r.p[1 + 4 * H + j] = sld16(rs, lane * 16, soff + 1024 * (1 + 4 * H + j));
  }
  __device__ static void decode(const R& r, int c, Run& a, Run& b) { dec(r.p[0], r.p[1 + c], c, a, b); }
  struct CR { uint4 head, qs; };
  __device__ static void load_chunk(const uint8_t* slab, int lane, int c, CR& r) {
    r.head = ld16(slab + lane * 16);
    r.qs = ld16(slab + 1024 * (1 + c) + lane * 16);
  }
  __device__ static void bload_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, int c, CR& r) {
    r.head = bld16(rs, slab + lane * 16);
    r.qs = bld16(rs, slab + 1024 * (1 + c) + lane * 16);
  }
  __device__ static void decode_chunk(const CR& r, int c, Run& a, Run& b) { dec(r.head, r.qs, c, a, b); }
  __device__ static void chunk(const uint8_t* slab, int lane, int c, Run& a, Run& b) {
    CR r; load_chunk(slab, lane, c, r); decode_chunk(r, c, a, b);
  }
};

template <> struct Blk<T_Q5_K> {
  static constexpr int QK = 256, BB = 176, NCH = 8, NP = 11;
  static constexpr int SLAB = 64 * BB;
  struct R { uint4 p[NP]; uint32_t t0, t1; };
  // planes: head(0) qh(1,2) qs(3..10); chunk c = 2g + h as Q4_K plus the 5th bit, which for
  // element l of group g (l = 16h + i) is bit 2g (low run) / 2g+1 (high run) of qh[l]
  __device__ static void dec(const uint4& head, const uint4& qh, const uint4& qs, int c, Run& a, Run& b) {
    const int g = c >> 1, h = c & 1;
    const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
    const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a.q[i] = (w[i] & 0x0F0F0F0Fu) | (((hw[i] >> (2 * g)) & 0x01010101u) << 4);
      b.q[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) | (((hw[i] >> (2 * g + 1)) & 0x01010101u) << 4);
    }
    k4_scales(head, g, a, b);
    a.e = 64 * g + 16 * h; b.e = a.e + 32;
  }
  __device__ static void load(const uint8_t* slab, int lane, R& r) {
#pragma unroll
    for (int p = 0; p < NP; ++p) r.p[p] = ld16(slab + 1024 * p + lane * 16);
    r.t0 = r.t1 = 0;
  }
  __device__ static void sload(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
#pragma unroll
    for (int p = 0; p < NP; ++p) r.p[p] = sld16(rs, lane * 16, soff + 1024 * p);
    r.t0 = r.t1 = 0;
  }
  // the planes chunks 4H .. 4H + 3 read (head, both qh planes, their four qs planes)
  template <int H> __device__ static void sload_half(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
#pragma unroll
    for (int p = 0; p < 3; ++p) r.p[p] = sld16(rs, lane * 16, soff + 1024 * p);
#pragma unroll
    for (int j = 0; j < 4; ++j) r.p[3 + 4 * H + j] = sld16(rs, lane * 16, soff + 1024 * (3 + 4 * H + j));
  }
  __device__ static void decode(const R& r, int c, Run& a, Run& b) {
    dec(r.p[0], r.p[1 + (c & 1)], r.p[3 + c], c, a, b);
  }
  struct CR { uint4 head, qh, qs; };
  __device__ static void load_chunk(const uint8_t* slab, int lane, int c, CR& r) {
    r.head = ld16(slab + lane * 16);
    r.qh = ld16(slab + 1024 * (1 + (c & 1)) + lane * 16);
    r.qs = ld16(slab + 1024 * (3 + c) + lane * 16);
  }
  __device__ static void bload_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, int c, CR& r) {
    r.head = bld16(rs, slab + lane * 16);
    r.qh = bld16(rs, slab + 1024 * (1 + (c & 1)) + lane * 16);
    r.qs = bld16(rs, slab + 1024 * (3 + c) + lane * 16);
  }
  __device__ static void decode_chunk(const CR& r, int c, Run& a, Run& b) { dec(r.head, r.qh, r.qs, c, a, b); }
  __device__ static void chunk(const uint8_t* slab, int lane, int c, Run& a, Run& b) {
    CR r; load_chunk(slab, lane, c, r); decode_chunk(r, c, a, b);
  }
};

template <> struct Blk<T_Q6_K> {
  static constexpr int QK = 256, BB = 210, NCH = 8, NP = 13;
  static constexpr int SLAB = 64 * BB;
  struct R { uint4 p[NP]; uint32_t t0, t1; };
  // planes: ql(0..7) qh(8..11) sc(12) d(13, 2 bytes). Chunk c = ql plane c: half hh = c/4,
  // byte l = 16(c%2) + i of the half's ql[32*ih + l] with ih = (c%4)/2. Low nibble -> element
  // 128hh + 32ih + l (qh bits 2ih, scale 8hh + l/16 + 2ih); high nibble -> element + 64
  // (qh bits 2ih + 4, scale index + 4). qh byte = qh[32hh + l] = plane 8 + 2hh + c%2.
  __device__ static void dec(const uint4& ql, const uint4& qh, const uint4& sc, uint32_t dbits, int c,
                             Run& a, Run& b) {
    const int hh = c >> 2, ih = (c >> 1) & 1, lo = c & 1;
    const float d = f16_bits_to_f32(dbits);
    // sub-scale ia = 8hh + 2ih + lo is byte (c & 3) of dword 2hh; ib = ia + 4 the same byte of
    // dword 2hh + 1 (selected, not indexed: a runtime index into a register array goes to scratch)
    const uint32_t wa = hh ? sc.z : sc.x, wb = hh ? sc.w : sc.y;
    const int sh = 24 - 8 * (c & 3);
    const float sca = (float)((int)(wa << sh) >> 24);
    const float scb = (float)((int)(wb << sh) >> 24);
    const uint32_t w[4] = {ql.x, ql.y, ql.z, ql.w};
    const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
    const int sha = 2 * ih, shb = 2 * ih + 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a.q[i] = (w[i] & 0x0F0F0F0Fu) | (((hw[i] >> sha) & 0x03030303u) << 4);
      b.q[i] = ((w[i] >> 4) & 0x0F0F0F0Fu) | (((hw[i] >> shb) & 0x03030303u) << 4);
    }
    a.scale = d * sca; a.offset = 32.0f * a.scale;
    b.scale = d * scb; b.offset = 32.0f * b.scale;
    a.e = 128 * hh + 32 * ih + 16 * lo; b.e = a.e + 64;
  }
  __device__ static void load(const uint8_t* slab, int lane, R& r) {
#pragma unroll
    for (int p = 0; p < NP; ++p) r.p[p] = ld16(slab + 1024 * p + lane * 16);
    r.t0 = ld2(slab + 1024 * 13 + lane * 2);
    r.t1 = 0;
  }
  __device__ static void sload(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
#pragma unroll
    for (int p = 0; p < NP; ++p) r.p[p] = sld16(rs, lane * 16, soff + 1024 * p);
    r.t0 = sld2(rs, lane * 2, soff + 1024 * 13);
    r.t1 = 0;
  }
  // the planes chunks 4H .. 4H + 3 read (sc, d, then their ql planes and qh planes 8 + 2H and
  // 9 + 2H). The scales go first: loads complete in order, and the compiler converts d as soon as
  // it can, so a d issued last made that conversion wait for the whole half.
  template <int H> __device__ static void sload_half(__amdgpu_buffer_rsrc_t rs, uint32_t soff, int lane, R& r) {
    r.p[12] = sld16(rs, lane * 16, soff + 1024 * 12);
    r.t0 = sld2(rs, lane * 2, soff + 1024 * 13);
    __builtin_amdgcn_sched_barrier(0);   // keeps the scale loads ahead of the planes
#pragma unroll
    for (int j = 0; j < 4; ++j) r.p[4 * H + j] = sld16(rs, lane * 16, soff + 1024 * (4 * H + j));
    r.p[8 + 2 * H] = sld16(rs, lane * 16, soff + 1024 * (8 + 2 * H));
    r.p[9 + 2 * H] = sld16(rs, lane * 16, soff + 1024 * (9 + 2 * H));
  }
  __device__ static void decode(const R& r, int c, Run& a, Run& b) {
    dec(r.p[c], r.p[8 + 2 * (c >> 2) + (c & 1)], r.p[12], r.t0, c, a, b);
  }
  struct CR { uint4 ql, qh, sc; uint32_t d; };
  __device__ static void load_chunk(const uint8_t* slab, int lane, int c, CR& r) {
    r.ql = ld16(slab + 1024 * c + lane * 16);
    r.qh = ld16(slab + 1024 * (8 + 2 * (c >> 2) + (c & 1)) + lane * 16);
    r.sc = ld16(slab + 1024 * 12 + lane * 16);
    r.d = ld2(slab + 1024 * 13 + lane * 2);
  }
  __device__ static void bload_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, int c, CR& r) {
    r.ql = bld16(rs, slab + 1024 * c + lane * 16);
    r.qh = bld16(rs, slab + 1024 * (8 + 2 * (c >> 2) + (c & 1)) + lane * 16);
    r.sc = bld16(rs, slab + 1024 * 12 + lane * 16);
    r.d = bld2(rs, slab + 1024 * 13 + lane * 2);
  }
  __device__ static void decode_chunk(const CR& r, int c, Run& a, Run& b) { dec(r.ql, r.qh, r.sc, r.d, c, a, b); }
  __device__ static void chunk(const uint8_t* slab, int lane, int c, Run& a, Run& b) {
    CR r; load_chunk(slab, lane, c, r); decode_chunk(r, c, a, b);
  }
};

__device__ __forceinline__ float qbyte(const uint32_t* q, int i) {
  return (float)((q[i >> 2] >> (8 * (i & 3))) & 0xFFu);
}

// Value of element i of a run as scale*q - offset: exact for every type, signed zeros aside
// (used where values are summed).
__device__ __forceinline__ float run_value(const Run& r, int i) {
  return __builtin_fmaf(r.scale, qbyte(r.q, i), -r.offset);
}

// Value of element i with the reference's own operation order, bit for bit including the sign
// of zero: scale * (q - bias) for the biased types (quant.rs:113, 138, 153, 348-351), and
// (d*sc)*q - dmin*m for Q4_K/Q5_K (quant.rs:280-284, 314-318).
template <int T>
__device__ __forceinline__ float run_value_exact(const Run& r, int i) {
  const uint32_t q = (r.q[i >> 2] >> (8 * (i & 3))) & 0xFFu;
  if constexpr (kBias<T> != 0) {
    return r.scale * (float)((int)q - kBias<T>);
  } else {
    return __builtin_fmaf(r.scale, (float)q, -r.offset);
  }
}

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
typedef _Float16 h16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Dot of one decoded run (16 quants) with x from LDS: every lane of the wave reads the same
// address (a broadcast), so 16 activations are four ds_read_b128.
template <int T>
__device__ __forceinline__ float run_dot(const Run& r, const float* __restrict__ xb,
                                         const float* __restrict__ xs) {
  const float4* xv = reinterpret_cast<const float4*>(xb + r.e);
  float s = 0.0f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float4 q = xv[v];
    if constexpr (kNibble<T>) {
      const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(r.q[v], false);   // quants 4v, 4v+1
      const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(r.q[v], true);    // quants 4v+2, 4v+3
      s = __builtin_fmaf(lo[0], q.x, s);
      s = __builtin_fmaf(lo[1], q.y, s);
      s = __builtin_fmaf(hi[0], q.z, s);
      s = __builtin_fmaf(hi[1], q.w, s);
    } else {
      // bytes b -> binary16 1024 + b (0x64 as the high byte: exact), two per v_perm_b32; one
      // v_pk_add_f16 of -(1024 + bias) leaves the signed quant b - bias, exact in binary16, and the
      // multiply-add takes the half operand directly (v_fma_mix_f32): 2 instructions per quant
      // instead of a convert, a subtract and an FMA. Subtracting the offset here, before the
      // products, keeps the sum free of the cancellation a 1024 * sum(x) correction would bring.
      constexpr _Float16 kSub = (_Float16)(-(1024 + kBias<T>));
      const h16x2_t sub = {kSub, kSub};
      const h16x2_t p01 =
          __builtin_bit_cast(h16x2_t, __builtin_amdgcn_perm(0x64646464u, r.q[v], 0x04010400u)) + sub;
      const h16x2_t p23 =
          __builtin_bit_cast(h16x2_t, __builtin_amdgcn_perm(0x64646464u, r.q[v], 0x04030402u)) + sub;
      s = __builtin_fmaf((float)p01[0], q.x, s);
      s = __builtin_fmaf((float)p01[1], q.y, s);
      s = __builtin_fmaf((float)p23[0], q.z, s);
      s = __builtin_fmaf((float)p23[1], q.w, s);
    }
  }
  if constexpr (kNibble<T>) return __builtin_fmaf(r.scale * 512.0f, s, -r.offset * xs[r.e >> 4]);
  if constexpr (kBias<T> != 0) return r.scale * s;          // offset = bias * scale, taken out above
  return __builtin_fmaf(r.scale, s, -r.offset * xs[r.e >> 4]);
}

// Sum of one value per thread over a workgroup of WAVES waves: xor tree inside each wave, then
// the wave sums in wave order (deterministic). `red` holds WAVES floats; all threads get the sum.
template <int WAVES>
__device__ __forceinline__ float wg_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) s += red[w];
  return s;
}

// silu(x) * u with silu(x) = x * (1 / (1 + exp(-x))), each step rounded (moe.rs:44-51, 280-283);
// shared by the SwiGLU kernel, the expert GEMV and the fused gate/up GEMM epilogue
__device__ __forceinline__ float silu_mul(float x, float u) {
  const float sig = __frcp_rn(__fadd_rn(1.0f, expf(-x)));
  return __fmul_rn(__fmul_rn(x, sig), u);
}

}  // namespace rehip
