// Grouped expert GEMM with register-decoded weights, bf16 mode (moe.rs:288-300, 360-388): the
// gate/up pair (SwiGLU written as bf16 h) and the down projection of the experts the router hit.
//
// One wave per task (GemmTask: expert, 64-row weight tile, up to 64 gathered activation rows),
// over the whole K. Lane r loads row r's raw 32-element chunk from the tiled slab (one
// contiguous 1 KiB plane read per wave, lane = row), decodes both 16-element runs to bf16
// (scale * q - offset in f32, as the reference's dequantizer, then rounded), and
// v_permlane32_swap exchanges lane halves so that lanes 0-31 / 32-63 hold k 0-7 / 8-15 of rows
// 0-31 (B operand of row group 0) and of rows 32-63 (row group 1). Each run is then one
// v_mfma_f32_32x32x16_bf16 per (row group, 32-row token tile), the A operand (tokens x 16 k) read
// straight from the bf16 activation rows in L2. Weights never touch LDS: a weight is decoded once
// and feeds every token of the task, so the decode costs ~2-3 VALU operations per weight
// whatever the batch, against ~5-8 for the LDS-staged grouped GEMM and the expert GEMV.
//
// The K order inside a chunk follows the block format (the A operand of run a reads the
// activations at the run's own k offset), so X needs no reordering.
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "deq.hpp"
#include "kernels.hpp"
#include "qfrag.hpp"

namespace rehip {

namespace {

// Half tile (32 weight rows per wave): lanes 0-31 decode run a of rows 0-31, lanes 32-63 run b of
// the same rows; one v_permlane32_swap per dword then leaves run a's B operand in a0 (lanes 0-31
// k 0-7, lanes 32-63 k 8-15) and run b's in b0. Every weight is still decoded once.
template <int T>
__device__ __forceinline__ void decode_frags_half(const typename Blk<T>::CR& raw, int cc, Frags& f) {
  Run a, b;
  Blk<T>::decode_chunk(raw, cc, a, b);
  const bool up = (threadIdx.x & 32) != 0;
  Run r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r.q[i] = up ? b.q[i] : a.q[i];
  r.scale = up ? b.scale : a.scale;
  r.offset = up ? b.offset : a.offset;
  uint32_t lo[4], hi[4];
  run_bf16<T>(r, lo, hi);
  halves_to_frags(lo, hi, f.a0, f.b0);
  f.ea = a.e;
  f.eb = b.e;
}

// vector memory instructions of one Blk<T>::bload_chunk
template <int T> inline constexpr int kChunkLoads = 0;
template <> inline constexpr int kChunkLoads<T_Q4_0> = 2;
template <> inline constexpr int kChunkLoads<T_Q5_0> = 3;
template <> inline constexpr int kChunkLoads<T_Q8_0> = 3;
template <> inline constexpr int kChunkLoads<T_Q4_K> = 2;
template <> inline constexpr int kChunkLoads<T_Q5_K> = 3;
template <> inline constexpr int kChunkLoads<T_Q6_K> = 4;

// K-quant blocks: the block-wide planes (Q4_K / Q5_K: d, dmin and the scales; Q6_K: the scales and
// d) are loaded once per block and shared by its eight chunks, so a chunk loads only its quant
// planes and the scales of a pair of chunks are computed once (the decode sees the same values)
template <int T> inline constexpr bool kBlockHead = Blk<T>::QK == 256;
template <int T> inline constexpr int kChunkOwnLoads = kBlockHead<T> ? (T == T_Q4_K ? 1 : 2) : kChunkLoads<T>;
struct BlockHead {
  uint4 h;       // Q4_K / Q5_K: the head plane; Q6_K: the scales plane
  uint32_t d;    // Q6_K: d
};
template <int T>
__device__ __forceinline__ void load_head(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, BlockHead& h) {
  if constexpr (T == T_Q6_K) {
    h.h = bld16(rs, slab + 1024 * 12 + lane * 16);
    h.d = bld2(rs, slab + 1024 * 13 + lane * 2);
  } else {
    h.h = bld16(rs, slab + lane * 16);
    h.d = 0;
  }
}
// the chunk's own planes only
template <int T>
__device__ __forceinline__ void load_own(__amdgpu_buffer_rsrc_t rs, uint32_t slab, int lane, int cc,
                                         typename Blk<T>::CR& r) {
  if constexpr (T == T_Q4_K) {
    r.qs = bld16(rs, slab + 1024 * (1 + cc) + lane * 16);
  } else if constexpr (T == T_Q5_K) {
    r.qh = bld16(rs, slab + 1024 * (1 + (cc & 1)) + lane * 16);
    r.qs = bld16(rs, slab + 1024 * (3 + cc) + lane * 16);
  } else if constexpr (T == T_Q6_K) {
    r.ql = bld16(rs, slab + 1024 * cc + lane * 16);
    r.qh = bld16(rs, slab + 1024 * (8 + 2 * (cc >> 2) + (cc & 1)) + lane * 16);
  } else {
    Blk<T>::bload_chunk(rs, slab, lane, cc, r);
  }
}
template <int T>
__device__ __forceinline__ typename Blk<T>::CR with_head(typename Blk<T>::CR r, const BlockHead& h) {
  if constexpr (T == T_Q6_K) {
    r.sc = h.h;
    r.d = h.d;
  } else if constexpr (kBlockHead<T>) {
    r.head = h.h;
  }
  return r;
}

typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with only the vector-memory counter bounded (expcnt and lgkmcnt at their maximum)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Activations staged in LDS (XL): a stage is two consecutive chunks of K, 64 bf16 of each row
// (128 bytes: one cache line, or for Q6_K two half lines) in eight 16-byte units. Unit u of stage
// st starts at K index xl_unit_k<T>(st, u); the A operand of run a / b of chunk 2 st + cl starts at
// unit xl_run_unit<T>(cl, b) (plus lane / 32).
template <int T>
__device__ __forceinline__ int xl_unit_k(int st, int u) {
  if constexpr (Blk<T>::QK == 32) {
    return 64 * st + 8 * u;                                   // blocks 2 st, 2 st + 1
  } else if constexpr (T == T_Q6_K) {
    const int kb = st >> 2, m = (st & 3) >> 1, half = st & 1;  // chunks 4m + 2 half + {0, 1}
    const int k0 = 256 * kb + 128 * m + 32 * half;
    return u < 4 ? k0 + 8 * u : k0 + 64 + 8 * (u - 4);
  } else {
    return 256 * (st >> 2) + 64 * (st & 3) + 8 * u;          // chunks 2g, 2g + 1 of a block
  }
}
template <int T>
__device__ __forceinline__ constexpr int xl_run_unit(int cl, bool b) {
  if constexpr (Blk<T>::QK == 32) return 4 * cl + (b ? 2 : 0);
  else return 2 * cl + (b ? 4 : 0);
}

__device__ __forceinline__ bf16x8_t ld_x(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return __builtin_bit_cast(bf16x8_t, v);
}

}  // namespace

// NT token tiles of 32 (tasks of up to 32 * NT rows). PAIR selects the weights of a task:
//   kOneTile   one 64-row tile (mtile) of W, Y receives f32;
//   kGateUp    the tile of W (gate) and of W2 (up) side by side, Y receives h = silu(gate) * up
//              as bf16;
//   kTwoTiles  tiles 2 mtile and 2 mtile + 1 of W (128 rows per task: every activation operand
//              load feeds twice the weights), Y receives f32.
// KS waves per task split the blocks of K between them (wave w takes blocks w, w + KS, ...);
// their sums are added in wave order through LDS at the end (deterministic).
// H (staged activations only, one K wave): two waves share the task, each taking 32 of the
// tile's rows (half = wave), and one staging of the activation rows in LDS, each wave copying
// half of every stage.
// SP (f32 mode): split operands, three MFMAs per product (the activations' and the weights' bf16
// roundings and remainders: hi hi + hi lo + lo hi), activations read from L2.
constexpr int kOneTile = 0, kGateUp = 1, kTwoTiles = 2;
template <int T, int PAIR, int NT, int KS, bool XL, bool H, bool SP>
__device__ __forceinline__ void qmma_task(const GemmArgs& p, const GemmTask& t, uint8_t* xs) {
  using B = Blk<T>;
  static_assert(!H || (XL && KS == 1 && PAIR != kTwoTiles), "half tiles: staged activations, one K wave, one tile");
  static_assert(!SP || (!XL && !H), "split operands: activations from L2, whole tiles");
  constexpr int NCH = B::NCH;                       // 32-element chunks per block
  constexpr int RG = H ? 1 : 2;                     // 32-row groups per weight set
  const int lane = threadIdx.x & 63;
  const int half = H ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
  const int wave = H ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = H ? 32 * half + (lane & 31) : lane;   // the slab row this lane loads
  const int rn = t.rn;
  const int nt = (rn + 31) >> 5;                    // token tiles holding rows (uniform)

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  constexpr bool DUAL = PAIR != kOneTile;           // a second set of weight registers
  const __amdgpu_buffer_rsrc_t wr2 = make_rsrc(PAIR == kGateUp ? p.W2 : p.W, p.w_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.X, p.x_bytes);
  const int tile0 = PAIR == kTwoTiles ? 2 * t.mtile : t.mtile;
  const uint32_t wbase = (uint32_t)((size_t)t.expert * p.w_stride) +
                         (uint32_t)tile0 * (uint32_t)p.KB * (uint32_t)B::SLAB;
  // second set: the up tile (same offset, other matrix) or the next tile of W (a tile past the
  // expert's last one reads the following bytes of the stack; its rows are not stored)
  const uint32_t wbase2 = PAIR == kTwoTiles ? wbase + (uint32_t)p.KB * (uint32_t)B::SLAB : wbase;

  // this lane's activation row in each token tile (A operand row lane % 32), k half lane / 32
  uint32_t xoff[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int rl = 32 * j + (lane & 31);
    uint32_t o = kQOob;
    if (rl < rn) {
      const int row = p.xrow ? p.xrow[t.r0 + rl] : t.r0 + rl;
      o = ((uint32_t)row * (uint32_t)p.K + 8u * (uint32_t)(lane >> 5)) * 2u;
    }
    xoff[j] = o;
  }

  f32x16_t acc[RG][NT], acc2[DUAL ? RG : 1][DUAL ? NT : 1];
#pragma unroll
  for (int g = 0; g < RG; ++g)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][j][r] = 0.0f;
  if constexpr (DUAL) {
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc2[g][j][r] = 0.0f;
  }

  const int nch = p.KB * NCH;
  auto load = [&](int c, typename B::CR& raw, const __amdgpu_buffer_rsrc_t& rs, uint32_t base) {
    const int kb = c / NCH, cc = c - kb * NCH;
    const uint32_t slab = c < nch ? base + (uint32_t)kb * (uint32_t)B::SLAB : kQOob;
    load_own<T>(rs, slab, lrow, cc, raw);
  };
  // the block heads of the block holding chunk c (first chunk of a block), both weight sets
  BlockHead hc{}, hc2{}, hn{}, hn2{};
  auto load_heads = [&](int c, BlockHead& h, BlockHead& h2) {
    if constexpr (kBlockHead<T>) {
      const int kb = c / NCH;
      load_head<T>(wr, c < nch ? wbase + (uint32_t)kb * (uint32_t)B::SLAB : kQOob, lrow, h);
      if constexpr (DUAL) load_head<T>(wr2, c < nch ? wbase2 + (uint32_t)kb * (uint32_t)B::SLAB : kQOob, lrow, h2);
    }
  };
  // A operands of chunk c: runs a and b of every token tile
  struct XOps { bf16x8_t a[NT], b[NT], al[SP ? NT : 1], bl[SP ? NT : 1]; };
  // (runs at or past K, the padding of rows stored as whole blocks, read zeros: K % 16 == 0, so a
  // run is wholly inside or outside)
  auto load_x = [&](int c, int ea, int eb, XOps& x) {
    const int kb = c / NCH;
    const int ka = kb * B::QK + ea, kbe = kb * B::QK + eb;
    const bool in_a = c < nch && ka < p.K, in_b = c < nch && kbe < p.K;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const uint32_t oa = j < nt && in_a ? xoff[j] + (uint32_t)ka * 2u : kQOob;
      const uint32_t ob = j < nt && in_b ? xoff[j] + (uint32_t)kbe * 2u : kQOob;
      x.a[j] = ld_x(xr, oa);
      x.b[j] = ld_x(xr, ob);
      if constexpr (SP) {
        x.al[j] = ld_x(xr, oa == kQOob ? kQOob : oa + p.x_lo);
        x.bl[j] = ld_x(xr, ob == kQOob ? kQOob : ob + p.x_lo);
      }
    }
  };
  // run element offsets of chunk cc (the Blk<T>::dec layouts; the same for every row)
  auto run_e = [&](int c, int& ea, int& eb) {
    const int cc = c % NCH;
    if constexpr (B::QK == 32) {
      ea = 0; eb = 16;
    } else if constexpr (T == T_Q6_K) {
      ea = 128 * (cc >> 2) + 32 * ((cc >> 1) & 1) + 16 * (cc & 1); eb = ea + 64;
    } else {
      ea = 64 * (cc >> 1) + 16 * (cc & 1); eb = ea + 32;
    }
  };

  // Two register sets, A and B, take alternate chunks: while chunk c is decoded from set A, the
  // loads of chunk c + 1 (set B) are in flight, and set A is refilled with chunk c + 2 right after
  // its decode. Named sets (not a rotated copy) let the waits count only the older loads. Chunks
  // past the end load zeros and add nothing, so an odd chunk count needs no tail.
  auto mma = [&](const XOps& x, const Frags& f, f32x16_t (&a)[RG][NT]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      a[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.a[j], f.a0, a[0][j], 0, 0, 0);
      if constexpr (!H) a[RG - 1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.a[j], f.a1, a[RG - 1][j], 0, 0, 0);
      a[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.b[j], f.b0, a[0][j], 0, 0, 0);
      if constexpr (!H) a[RG - 1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.b[j], f.b1, a[RG - 1][j], 0, 0, 0);
    }
  };
  // split operands: the cross terms x_hi w_lo and x_lo w_hi after the x_hi w_hi products
  auto mma_rest = [&](const XOps& x, const Frags& f, const Frags& fr, f32x16_t (&a)[RG][NT]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      a[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.a[j], fr.a0, a[0][j], 0, 0, 0);
      a[RG - 1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.a[j], fr.a1, a[RG - 1][j], 0, 0, 0);
      a[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.al[j], f.a0, a[0][j], 0, 0, 0);
      a[RG - 1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.al[j], f.a1, a[RG - 1][j], 0, 0, 0);
      a[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.b[j], fr.b0, a[0][j], 0, 0, 0);
      a[RG - 1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.b[j], fr.b1, a[RG - 1][j], 0, 0, 0);
      a[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.bl[j], f.b0, a[0][j], 0, 0, 0);
      a[RG - 1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x.bl[j], f.b1, a[RG - 1][j], 0, 0, 0);
    }
  };
  auto decode = [&](const typename B::CR& raw, int cc, Frags& f) {
    if constexpr (H) decode_frags_half<T>(raw, cc, f);
    else decode_frags<T>(raw, cc, f);
  };
  auto load_all = [&](int c, typename B::CR& r, typename B::CR& q, XOps& x) {
    load(c, r, wr, wbase);
    if constexpr (DUAL) load(c, q, wr2, wbase2);
    int ea, eb;
    run_e(c, ea, eb);
    load_x(c, ea, eb, x);
  };
  auto step = [&](int c, const typename B::CR& r, const typename B::CR& q, const XOps& x) {
    if constexpr (SP) {
      Frags f, fr;
      decode_frags_split<T>(with_head<T>(r, hc), c % NCH, f, fr);
      mma(x, f, acc);
      mma_rest(x, f, fr, acc);
      if constexpr (DUAL) {
        Frags f2, fr2;
        decode_frags_split<T>(with_head<T>(q, hc2), c % NCH, f2, fr2);
        mma(x, f2, acc2);
        mma_rest(x, f2, fr2, acc2);
      }
    } else {
      Frags f;
      decode(with_head<T>(r, hc), c % NCH, f);
      mma(x, f, acc);
      if constexpr (DUAL) {
        Frags f2;
        decode(with_head<T>(q, hc2), c % NCH, f2);
        mma(x, f2, acc2);
      }
    }
  };
  // U chunks per iteration, a whole number of blocks, unrolled so that every chunk's position in
  // its block (and so its decode) is a compile-time constant
  constexpr int U = NCH >= 2 ? NCH : 2;
  // this wave's groups of U chunks: c0 = (i * KS + wave) * U for i = 0, 1, ...
  typename B::CR r[2], q[2];
  const int first = wave * U;
  if constexpr (XL) {
    // Activations through LDS: each stage (two chunks) of this wave's token rows is copied by
    // LDS DMA, one stage ahead, as whole 128-byte runs of a row (a line per row instead of a
    // 16-byte operand load per lane and run). Instruction i puts rows 8 i .. 8 i + 7 in the stage
    // buffer, row-major at 128 bytes a row, 16-byte unit u of a row at position u ^ ((row >> 1) & 7)
    // (so the 32 rows an operand read touches spread over the banks); lane l copies row
    // 8 i + l / 8, position l % 8. Rows past the task and K past the end read zeros.
    constexpr int LW = kChunkOwnLoads<T> * (DUAL ? 2 : 1);   // weight loads per chunk (heads not counted:
                                                              // a head load among them only waits longer)
    constexpr int ND = NT * 4;                            // LDS DMA instructions per stage
    constexpr int NDW = H ? ND / 2 : ND;                  // of them, issued by this wave
    constexpr int SB = NT * 32 * 128;                     // stage buffer bytes
    const int i0 = H ? half * NDW : 0;                    // this wave's first instruction
    uint32_t xo[NDW];
#pragma unroll
    for (int ii = 0; ii < NDW; ++ii) {
      const int rl = 8 * (i0 + ii) + (lane >> 3);
      uint32_t o = kQOob;
      if (rl < rn) {
        const int row = p.xrow ? p.xrow[t.r0 + rl] : t.r0 + rl;
        o = (uint32_t)row * (uint32_t)p.K * 2u;
      }
      xo[ii] = o;
    }
    const int pos = lane & 7;
    auto dma = [&](int c, int buf) {                      // the stage of chunks c, c + 1
      uint8_t* dst = xs + buf * SB;
      const int st = c >> 1;
#pragma unroll
      for (int ii = 0; ii < NDW; ++ii) {
        const int rl = 8 * (i0 + ii) + (lane >> 3);
        const int k = xl_unit_k<T>(st, pos ^ ((rl >> 1) & 7));
        const uint32_t o = c < nch && xo[ii] != kQOob && k < p.K ? xo[ii] + (uint32_t)k * 2u : kQOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void_t*)(dst + 1024 * (i0 + ii)), 16, (int)o, 0, 0, 0);
      }
    };
    auto read_x = [&](int buf, int cl, XOps& x) {
      const uint8_t* src = xs + buf * SB;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int row = 32 * j + (lane & 31);
        const int ua = xl_run_unit<T>(cl, false) + (lane >> 5), ub = xl_run_unit<T>(cl, true) + (lane >> 5);
        x.a[j] = *reinterpret_cast<const bf16x8_t*>(src + row * 128 + ((ua ^ ((row >> 1) & 7)) << 4));
        x.b[j] = *reinterpret_cast<const bf16x8_t*>(src + row * 128 + ((ub ^ ((row >> 1) & 7)) << 4));
      }
    };
    auto load_w = [&](int c, typename B::CR& rr, typename B::CR& qq) {
      load(c, rr, wr, wbase);
      if constexpr (DUAL) load(c, qq, wr2, wbase2);
    };
    // chunk u of this wave's chunks from c0 on (u may reach two groups ahead: U is 2 for the
    // 32-element blocks, and the stage DMA looks four chunks ahead)
    auto next_c = [&](int c0, int u) { return c0 + (u / U) * U * KS + u % U; };
    // issue order DMA(s), W(2s), W(2s + 1), DMA(s + 1), ...: when stage s is read, the loads
    // younger than its DMA are at most two chunks of weights and one stage of DMA. H: three stage
    // buffers; both waves pass a barrier before reading a stage (the other wave's half of the
    // copy has landed), and a buffer is refilled only two stages after it was read, so that
    // barrier also orders the refill after the other wave's reads.
    dma(first, 0);
    load_heads(first, hc, hc2);
    load_w(first, r[0], q[0]);
    load_w(first + 1, r[1], q[1]);
    dma(next_c(first, 2), 1);
    int buf = 0;
    for (int c0 = first; c0 < nch; c0 += U * KS) {
#pragma unroll
      for (int u = 0; u < U; u += 2) {
        wait_vmcnt<2 * LW + NDW>();
        if constexpr (H) {
          asm volatile("" ::: "memory");
          __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          XOps x;
          read_x(buf, h, x);
          step(c0 + u + h, r[h], q[h], x);
          __builtin_amdgcn_sched_barrier(0);
          if (u + h + 2 == U) load_heads(next_c(c0, U), hn, hn2);
          load_w(next_c(c0, u + h + 2), r[h], q[h]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (H) {
          dma(next_c(c0, u + 4), buf == 0 ? 2 : buf - 1);
          __builtin_amdgcn_sched_barrier(0);
          buf = buf == 2 ? 0 : buf + 1;
        } else {
          dma(next_c(c0, u + 4), buf);
          __builtin_amdgcn_sched_barrier(0);
          buf ^= 1;
        }
      }
      hc = hn;
      hc2 = hn2;
    }
    wait_vmcnt<0>();                                      // no LDS DMA outlives the task
  } else {
    XOps x[2];
    load_heads(first, hc, hc2);
    load_all(first, r[0], q[0], x[0]);
    load_all(first + 1, r[1], q[1], x[1]);
    for (int c0 = first; c0 < nch; c0 += U * KS) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        step(c0 + u, r[u & 1], q[u & 1], x[u & 1]);
        // keep the loads in program order behind the step that frees their registers, so the wait
        // before the next step counts only these (younger) loads
        __builtin_amdgcn_sched_barrier(0);
        if (u + 2 == U) load_heads(c0 + U * KS, hn, hn2);
        load_all(u + 2 < U ? c0 + u + 2 : c0 + U * KS + u + 2 - U, r[u & 1], q[u & 1], x[u & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      hc = hn;
      hc2 = hn2;
    }
  }
  if constexpr (KS > 1) {
    // waves 1 .. KS-1 hand their sums to wave 0, which adds them in wave order
    constexpr int NACC = RG * NT * 16 * (DUAL ? 2 : 1);
    __shared__ float red[(KS - 1) * NACC * 64];
    if (wave > 0) {
      float* dst = red + (wave - 1) * NACC * 64 + lane;
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            dst[((g * NT + j) * 16 + e) * 64] = acc[g][j][e];
            if constexpr (DUAL) dst[(((RG + g) * NT + j) * 16 + e) * 64] = acc2[g][j][e];
          }
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 1; w < KS; ++w) {
      const float* src = red + (w - 1) * NACC * 64 + lane;
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            acc[g][j][e] += src[((g * NT + j) * 16 + e) * 64];
            if constexpr (DUAL) acc2[g][j][e] += src[(((RG + g) * NT + j) * 16 + e) * 64];
          }
    }
  }

  // D[token i][row n]: lane holds row n = 32 g + lane % 32 and tokens 8 (r / 4) + 4 (lane / 32) + r % 4
  const int col = tile0 * 64 + (H ? 32 * half : 0) + (lane & 31);
#pragma unroll
  for (int g = 0; g < (PAIR == kTwoTiles ? 4 : RG); ++g) {
    const int row = col + 32 * g;
    if (row >= p.m) continue;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      if (j >= nt) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * j + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (i >= rn) continue;
        const size_t o = (size_t)(t.r0 + i) * (size_t)p.ldy + (size_t)row;
        if constexpr (PAIR == kGateUp) {
          const float hv = silu_mul(acc[g][j][r], acc2[g][j][r]);
          const __bf16 hh = (__bf16)hv;
          reinterpret_cast<__bf16*>(p.Y)[o] = hh;
          if constexpr (SP) reinterpret_cast<__bf16*>(p.Y)[o + p.y_lo] = (__bf16)(hv - (float)hh);
        } else if constexpr (PAIR == kTwoTiles) {
          p.Y[o] = g < 2 ? acc[g & 1][j][r] : acc2[g & 1][j][r];
        } else {
          p.Y[o] = acc[g][j][r];
        }
      }
    }
  }
}

// A task of at most 32 rows runs the one-tile body (no MFMAs on an empty second token tile).
// XL: activations staged in LDS (two stage buffers per wave).
// H: two waves per task (32 weight rows each) sharing three stage buffers.
template <int T, int PAIR, int NT, int KS, bool XL, bool H, bool SP = false>
__global__ __launch_bounds__(64 * KS * (H ? 2 : 1)) void moe_qmma_kernel(GemmArgs p) {
  if (p.ntasks && (int)blockIdx.x >= *p.ntasks) return;   // grid sized for the most tasks
  const GemmTask t = p.tasks[blockIdx.x];
  __shared__ __attribute__((aligned(16))) uint8_t xs[!XL ? 16 : H ? 3 * NT * 32 * 128 : KS * 2 * NT * 32 * 128];
  uint8_t* mine = xs + (XL && !H ? (threadIdx.x >> 6) * 2 * NT * 32 * 128 : 0);
  if constexpr (NT == 2) {
    if (t.rn <= 32) {
      qmma_task<T, PAIR, 1, KS, XL, H, SP>(p, t, mine);
      return;
    }
  }
  qmma_task<T, PAIR, NT, KS, XL, H, SP>(p, t, mine);
}

template <int T, int PA, int NT, int KS>
static void launch_qmma_v(bool xl, bool h, int ntasks, hipStream_t s, const GemmArgs& a, bool sp) {
  const dim3 grid((unsigned)ntasks);
  if (sp) {
    hipLaunchKernelGGL((moe_qmma_kernel<T, PA, NT, KS, false, false, true>), grid, dim3(64 * KS), 0, s, a);
    return;
  }
  if constexpr (PA != kTwoTiles && KS == 1) {
    if (h) {
      hipLaunchKernelGGL((moe_qmma_kernel<T, PA, NT, 1, true, true>), grid, dim3(128), 0, s, a);
      return;
    }
  }
  if (xl) hipLaunchKernelGGL((moe_qmma_kernel<T, PA, NT, KS, true, false>), grid, dim3(64 * KS), 0, s, a);
  else hipLaunchKernelGGL((moe_qmma_kernel<T, PA, NT, KS, false, false>), grid, dim3(64 * KS), 0, s, a);
}

hipError_t launch_moe_qmma(uint32_t type, int pair, int max_rows, const GemmArgs& a, int ntasks, hipStream_t s,
                           bool split) {
  if (ntasks <= 0) return hipSuccess;
  if (max_rows < 1 || max_rows > 64 || pair < kOneTile || pair > kTwoTiles) return hipErrorInvalidValue;
  const bool one = max_rows <= 32;
  // waves per task: two split K where the tasks are few rows each (more waves in flight), one
  // for 64-row tasks; REHIP_QMMA_KS = 1 / 2 overrides
  int ks = one ? 2 : 1;
  if (const char* v = std::getenv("REHIP_QMMA_KS"); v && (v[0] == '1' || v[0] == '2') && !v[1]) ks = v[0] - '0';
  // activations staged in LDS for the two-tile tasks of 64 rows (each staged run feeds 128
  // weight rows; measured at 512 tokens on the Qwen3-30B-A3B shape: down 61.1 against 65.8 us,
  // while the gate/up pair and the 32-row tasks ran slower staged), else read from L2 per run;
  // REHIP_QMMA_XL = 1 / 0 forces either
  const char* xv = std::getenv("REHIP_QMMA_XL");
  bool xl = pair == kTwoTiles && !one;
  if (xv && (xv[0] == '0' || xv[0] == '1') && !xv[1]) xl = xv[0] == '1';
  // the gate/up pair of 64-row tasks: two 32-row waves per task sharing one staging of the rows.
  // One-wave whole-tile tasks hold 233 VGPRs (two per SIMD), so at 512 tokens on the
  // Qwen3-30B-A3B shape 1536 tasks sit 1.5 per SIMD and half the SIMDs idle at the end; the
  // halves hold 150 (all 3072 waves resident): 154.2 -> 151.7 us per call, the same bits.
  // REHIP_QMMA_H = 1 / 0 forces either (never with a K split or two tiles)
  const char* hv = std::getenv("REHIP_QMMA_H");
  bool h = pair == kGateUp && !one;
  if (hv && (hv[0] == '0' || hv[0] == '1') && !hv[1]) h = hv[0] == '1';
  h = h && ks == 1 && pair != kTwoTiles;
#define REHIP_QMMA_P(TT, PA)                                                               \
  if (one) { if (ks == 2) launch_qmma_v<TT, PA, 1, 2>(xl, h, ntasks, s, a, split);           \
             else launch_qmma_v<TT, PA, 1, 1>(xl, h, ntasks, s, a, split); }                 \
  else { if (ks == 2) launch_qmma_v<TT, PA, 2, 2>(xl, h, ntasks, s, a, split);               \
         else launch_qmma_v<TT, PA, 2, 1>(xl, h, ntasks, s, a, split); }
#define REHIP_QMMA(TT)                                                     \
  case TT:                                                                 \
    if (pair == kGateUp) { REHIP_QMMA_P(TT, kGateUp) }                     \
    else if (pair == kTwoTiles) { REHIP_QMMA_P(TT, kTwoTiles) }            \
    else { REHIP_QMMA_P(TT, kOneTile) }                                    \
    break;
  switch (type) {
    REHIP_QMMA(T_Q4_0)
    REHIP_QMMA(T_Q5_0)
    REHIP_QMMA(T_Q8_0)
    REHIP_QMMA(T_Q4_K)
    REHIP_QMMA(T_Q5_K)
    REHIP_QMMA(T_Q6_K)
    default:
      return hipErrorInvalidValue;
  }
#undef REHIP_QMMA
#undef REHIP_QMMA_P
  return hipGetLastError();
}

}  // namespace rehip
