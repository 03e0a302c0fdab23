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
// Software pipeline (one LDS stage per K-group, two barriers per step): while the MFMAs of step s
// read LDS, the same waves decode the weight chunks of step s+1 (loaded one step earlier) into
// registers, and the raw chunks of step s+2 and the activations of step s+1 are in flight; after
// the MFMAs the decoded step s+1 is written to LDS. The dequantization VALU work thereby runs
// under the matrix-core time of the previous step. Steps past the end of a K range load from
// an out-of-range offset (zeros), so every iteration has the same branch-free body. LDS rows are
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
#include <type_traits>

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

// A decoded chunk held in registers: runs a and b, 16 values each (bf16 or f32)
template <bool F32> struct DecChunk;
template <> struct DecChunk<false> { bf16x8_t v[4]; int ea, eb; };
template <> struct DecChunk<true> { float4 v[8]; int ea, eb; };

template <int T, bool F32>
__device__ __forceinline__ void pack_run(const Run& r, DecChunk<F32>& d, int h) {
  float v[16];
  run_values<T>(r, v);
  if constexpr (F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) d.v[4 * h + i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      bf16x8_t o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (__bf16)v[8 * k + i];
      d.v[2 * h + k] = o;
    }
  }
}

// split form (f32 mode on bf16 MFMAs): the bf16 rounding of each value into hi, the bf16 rounding
// of what it leaves into lo, so hi + lo holds the value to 2^-16 relative
template <int T>
__device__ __forceinline__ void pack_run_split(const Run& r, DecChunk<false>& hi, DecChunk<false>& lo, int h) {
  float v[16];
  run_values<T>(r, v);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    bf16x8_t oh, ol;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      oh[i] = (__bf16)v[8 * k + i];
      ol[i] = (__bf16)(v[8 * k + i] - (float)oh[i]);
    }
    hi.v[2 * h + k] = oh;
    lo.v[2 * h + k] = ol;
  }
}

template <bool F32>
__device__ __forceinline__ void store_dec(typename Elem<F32>::T* row, const DecChunk<F32>& d) {
  if constexpr (F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<float4*>(row + d.ea)[i] = d.v[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<float4*>(row + d.eb)[i] = d.v[4 + i];
  } else {
    reinterpret_cast<bf16x8_t*>(row + d.ea)[0] = d.v[0];
    reinterpret_cast<bf16x8_t*>(row + d.ea)[1] = d.v[1];
    reinterpret_cast<bf16x8_t*>(row + d.eb)[0] = d.v[2];
    reinterpret_cast<bf16x8_t*>(row + d.eb)[1] = d.v[3];
  }
}

template <bool F32> struct DecX;
template <> struct DecX<false> { using T = bf16x4_t; };
template <> struct DecX<true> { using T = float4; };

template <bool F32>
__device__ __forceinline__ typename DecX<F32>::T cvt_x(float4 v) {
  if constexpr (F32) {
    return v;
  } else {
    bf16x4_t o;
    o[0] = (__bf16)v.x; o[1] = (__bf16)v.y; o[2] = (__bf16)v.z; o[3] = (__bf16)v.w;
    return o;
  }
}

constexpr uint32_t kOob = 0x80000000u;   // a byte offset past every buffer: the load returns 0

template <int T, bool F32, bool GROUPED, int BM, int BN, int WM, int WN, int KG, bool XB = false, bool DUAL = false,
          bool SP = false>
__global__ __launch_bounds__(WM* WN * 64 * KG) void gemm_kernel(GemmArgs p) {
  using B = Blk<T>;
  using E = typename Elem<F32>::T;
  static_assert(!XB || !F32, "bf16 activations feed the bf16 mode only");
  static_assert(!SP || (!F32 && !GROUPED && !XB && !DUAL && KG == 1), "split operands: dense bf16-MFMA launches");
  static_assert(!DUAL || (GROUPED && XB && KG == 1), "gate/up pairs: grouped bf16 launches, one K-group");
  constexpr int NW = DUAL ? 2 : 1;                 // weight tiles per step (gate, up)
  constexpr int GT = WM * WN * 64;                 // threads of one K-group
  constexpr int BK = kGemmBK;
  constexpr int LD = BK + Elem<F32>::PAD;          // LDS row stride (elements)
  constexpr int WJOBS = BM * 4 / GT;               // (row, chunk) jobs per thread per step
  constexpr int XE = XB ? 8 : 4;                   // X elements per 16-byte load
  constexpr uint32_t XS = XB ? 2 : 4;              // bytes per X element
  constexpr int XV = BN * BK / XE / GT;            // 16-byte X loads per thread per step
  constexpr int XR = GT / (BK / XE);               // X rows covered by one pass of a group
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  constexpr int STAGE = (NW * BM + BN) * LD;       // LDS elements of one group
  static_assert(WJOBS >= 1 && XV >= 1 && TM >= 1 && TN >= 1, "tile shape");
  static_assert((KG - 1) * BM * BN * 4 <= KG * STAGE * (int)sizeof(E), "K-group partials fit in LDS");
  // SP: a second stage of the same shape holds the remainders (lo) of the weights and activations
  __shared__ __attribute__((aligned(16))) E smem[KG * STAGE * (SP ? 2 : 1)];

  const int grp = __builtin_amdgcn_readfirstlane(threadIdx.x / GT);
  const int tid = threadIdx.x - grp * GT;          // thread inside the K-group
  const int lane = threadIdx.x & 63;
  const int wave = tid >> 6;                       // wave inside the K-group
  const int wm = wave / WN, wn = wave % WN;
  E* const Ws = smem + grp * STAGE;
  E* const Ws2 = Ws + BM * LD;                     // up tile (pairs only)
  E* const Xs = Ws + NW * BM * LD;
  E* const Wl = Ws + STAGE;                       // SP: remainder planes
  E* const Xl = Xs + STAGE;

  int mtile, r0, rn, split = 0;
  uint32_t wbase = 0;
  if constexpr (GROUPED) {
    if (p.ntasks && (int)blockIdx.x >= *p.ntasks) return;   // grid sized for the most tasks
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
  // K-group g takes steps s_begin + g, s_begin + g + KG, ...; every group runs `iters`
  // iterations (barriers are workgroup-wide); a step past s_end loads zeros and adds nothing
  const int iters = (s_end - s_begin + KG - 1) / KG;
  const int s0 = s_begin + grp;

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.W, p.w_bytes);
  const __amdgpu_buffer_rsrc_t wr2 = make_rsrc(DUAL ? p.W2 : p.W, p.w_bytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.X, p.x_bytes);

  f32x16_t acc[TM][TN], acc2[DUAL ? TM : 1][DUAL ? TN : 1];   // acc2: the up tile of a pair
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  if constexpr (DUAL) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc2[i][j][r] = 0.0f;
  }

  // activation rows this thread stages: rows XR*jj + tid/32, k offset 4*(tid%32). Dense launches
  // address row r0 + XR*jj + tid/32 as one per-thread offset plus a scalar jj*XR*K*4 (rows past
  // N lie past the end of X and read zeros); grouped launches gather rows through xrow.
  const int xk = XE * (tid % (BK / XE));
  constexpr int XOFFS = GROUPED ? XV : 1;
  uint32_t xoff[XOFFS];
  if constexpr (GROUPED) {
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) {
      const int rl = XR * jj + tid / (BK / XE);
      uint32_t o = kOob;
      if (rl < rn) {
        const int row = p.xrow ? p.xrow[r0 + rl] : r0 + rl;
        o = (uint32_t)row * (uint32_t)p.K * XS + (uint32_t)xk * XS;
      }
      xoff[jj] = o;
    }
  } else {
    xoff[0] = (uint32_t)(r0 + tid / (BK / XE)) * (uint32_t)p.K * XS + (uint32_t)xk * XS;
  }
  const uint32_t xrow_step = (uint32_t)XR * (uint32_t)p.K * XS;   // bytes between a thread's rows
  // weight jobs: row rl = j % BM of tile (BM/64)*mtile + rl/64, chunk c = j / BM
  uint32_t wrow[WJOBS];
  int wc[WJOBS];
#pragma unroll
  for (int rep = 0; rep < WJOBS; ++rep) {
    const int j = tid + GT * rep;
    const int rl = j % BM;
    const int tile = BM / 64 * mtile + (rl >> 6);
    wc[rep] = j / BM;
    wrow[rep] = tile < p.tiles ? wbase + (uint32_t)tile * (uint32_t)p.KB * (uint32_t)B::SLAB : kOob;
  }

  auto load_w = [&](int s, typename B::CR (&raw)[WJOBS], const __amdgpu_buffer_rsrc_t& rsrc) {
    const bool in = s < s_end;
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) {
      const int j = tid + GT * rep;
      const int tl = (j % BM) & 63;
      int kb, cc;
      if constexpr (B::QK == 32) { kb = 4 * s + wc[rep]; cc = 0; }
      else { kb = s >> 1; cc = 4 * (s & 1) + wc[rep]; }
      const uint32_t slab = (in && kb < p.KB) ? wrow[rep] + (uint32_t)kb * (uint32_t)B::SLAB : kOob;
      B::bload_chunk(rsrc, slab, tl, cc, raw[rep]);
    }
  };
  auto load_x = [&](int s, i32x4_t (&xv)[XV]) {
    const bool in = s < s_end && s * BK + xk < p.K;
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) {
      i32x4_t v;
      if constexpr (GROUPED) {
        const uint32_t o = in ? xoff[jj] + (uint32_t)(s * BK) * XS : kOob;
        v = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)o, 0, 0);
      } else {
        const uint32_t o = in ? xoff[0] + (uint32_t)(s * BK) * XS : kOob;
        v = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)o, (int)(jj * xrow_step), 0);
      }
      xv[jj] = v;
    }
  };
  // staged X element pack: bf16 activations are stored as loaded; f32 ones are rounded (bf16
  // mode, RNE) or kept (f32 mode)
  using XD = std::conditional_t<XB, bf16x8_t, typename DecX<F32>::T>;
  auto cvt = [&](const i32x4_t& v) -> XD {
    if constexpr (XB) {
      return __builtin_bit_cast(bf16x8_t, v);
    } else {
      return cvt_x<F32>(make_float4(__int_as_float(v[0]), __int_as_float(v[1]), __int_as_float(v[2]),
                                    __int_as_float(v[3])));
    }
  };
  // SP: the remainders' decoded chunks and activations (one element otherwise, unused)
  DecChunk<F32> dec_lo[SP ? WJOBS : 1];
  XD xdec_lo[SP ? XV : 1];
  // SP: the remainder of an activation after its bf16 rounding, rounded to bf16
  auto cvt_lo = [&](const i32x4_t& v, const XD& hi) -> XD {
    XD o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (__bf16)(__int_as_float(v[i]) - (float)hi[i]);
    return o;
  };
  auto decode = [&](int s, const typename B::CR (&raw)[WJOBS], DecChunk<F32> (&dec)[WJOBS]) {
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) {
      const int c = (tid + GT * rep) / BM;
      int cc, kl;
      if constexpr (B::QK == 32) { cc = 0; kl = 32 * c; }
      else { cc = 4 * (s & 1) + c; kl = -128 * (s & 1); }
      Run a, b;
      B::decode_chunk(raw[rep], cc, a, b);
      if constexpr (SP) {
        pack_run_split<T>(a, dec[rep], dec_lo[rep], 0);
        pack_run_split<T>(b, dec[rep], dec_lo[rep], 1);
        dec_lo[rep].ea = kl + a.e;
        dec_lo[rep].eb = kl + b.e;
      } else {
        pack_run<T, F32>(a, dec[rep], 0);
        pack_run<T, F32>(b, dec[rep], 1);
      }
      dec[rep].ea = kl + a.e;
      dec[rep].eb = kl + b.e;
    }
  };
  auto write_lds = [&](const DecChunk<F32> (&dec)[WJOBS], const DecChunk<F32> (&dec2)[WJOBS], const XD (&xd)[XV]) {
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) store_dec<F32>(Ws + ((tid + GT * rep) % BM) * LD, dec[rep]);
    if constexpr (DUAL) {
#pragma unroll
      for (int rep = 0; rep < WJOBS; ++rep) store_dec<F32>(Ws2 + ((tid + GT * rep) % BM) * LD, dec2[rep]);
    }
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) *reinterpret_cast<XD*>(Xs + (XR * jj + tid / (BK / XE)) * LD + xk) = xd[jj];
    if constexpr (SP) {
#pragma unroll
      for (int rep = 0; rep < WJOBS; ++rep) store_dec<false>(Wl + ((tid + GT * rep) % BM) * LD, dec_lo[rep]);
#pragma unroll
      for (int jj = 0; jj < XV; ++jj)
        *reinterpret_cast<XD*>(Xl + (XR * jj + tid / (BK / XE)) * LD + xk) = xdec_lo[jj];
    }
  };

  typename B::CR rawA[WJOBS], rawB[WJOBS];
  DecChunk<F32> dec[WJOBS];
  // up tile of a gate/up pair (unused otherwise)
  typename B::CR rawA2[WJOBS], rawB2[WJOBS];
  DecChunk<F32> dec2[WJOBS];
  i32x4_t xraw[XV];
  XD xdec[XV];

  // prologue: step s0 into LDS, raw chunks of s0 + KG in flight
  load_w(s0, rawA, wr);
  if constexpr (DUAL) load_w(s0, rawA2, wr2);
  load_x(s0, xraw);
  load_w(s0 + KG, rawB, wr);
  if constexpr (DUAL) load_w(s0 + KG, rawB2, wr2);
  decode(s0, rawA, dec);
  if constexpr (DUAL) decode(s0, rawA2, dec2);
#pragma unroll
  for (int jj = 0; jj < XV; ++jj) xdec[jj] = cvt(xraw[jj]);
  if constexpr (SP) {
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) xdec_lo[jj] = cvt_lo(xraw[jj], xdec[jj]);
  }
  write_lds(dec, dec2, xdec);
#pragma unroll
  for (int rep = 0; rep < WJOBS; ++rep) rawA[rep] = rawB[rep];
  if constexpr (DUAL) {
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) rawA2[rep] = rawB2[rep];
  }
  __syncthreads();

  for (int it = 0; it < iters; ++it) {
    const int s = s0 + KG * it;
    load_x(s + KG, xraw);
    load_w(s + 2 * KG, rawB, wr);
    if constexpr (DUAL) load_w(s + 2 * KG, rawB2, wr2);
    decode(s + KG, rawA, dec);             // VALU under the MFMAs below
    if constexpr (DUAL) decode(s + KG, rawA2, dec2);
    if constexpr (!F32) {
      // operands of k-slice kk+1 are read from LDS while the MFMAs of slice kk run
      const E* wsrc = Ws + (BM / WM * wm + (lane & 31)) * LD + 8 * (lane >> 5);
      const E* wsrc2 = wsrc + BM * LD;     // the up tile's same row and slice (pairs only)
      const E* xsrc = Xs + (BN / WN * wn + (lane & 31)) * LD + 8 * (lane >> 5);
      bf16x8_t av[2][TM], bv[2][TN], av2[2][DUAL ? TM : 1];
      // SP: the remainder fragments at the same places of the remainder stage
      bf16x8_t al[2][SP ? TM : 1], bl[2][SP ? TN : 1];
      if constexpr (SP) {
#pragma unroll
        for (int i = 0; i < TM; ++i) al[0][i] = *reinterpret_cast<const bf16x8_t*>(wsrc + STAGE + 32 * i * LD);
#pragma unroll
        for (int j = 0; j < TN; ++j) bl[0][j] = *reinterpret_cast<const bf16x8_t*>(xsrc + STAGE + 32 * j * LD);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) av[0][i] = *reinterpret_cast<const bf16x8_t*>(wsrc + 32 * i * LD);
      if constexpr (DUAL) {
#pragma unroll
        for (int i = 0; i < TM; ++i) av2[0][i] = *reinterpret_cast<const bf16x8_t*>(wsrc2 + 32 * i * LD);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[0][j] = *reinterpret_cast<const bf16x8_t*>(xsrc + 32 * j * LD);
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int cur = kk & 1, nxt = cur ^ 1;
        if (kk + 1 < BK / 16) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
            av[nxt][i] = *reinterpret_cast<const bf16x8_t*>(wsrc + 32 * i * LD + 16 * (kk + 1));
          if constexpr (DUAL) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
              av2[nxt][i] = *reinterpret_cast<const bf16x8_t*>(wsrc2 + 32 * i * LD + 16 * (kk + 1));
          }
#pragma unroll
          for (int j = 0; j < TN; ++j)
            bv[nxt][j] = *reinterpret_cast<const bf16x8_t*>(xsrc + 32 * j * LD + 16 * (kk + 1));
          if constexpr (SP) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
              al[nxt][i] = *reinterpret_cast<const bf16x8_t*>(wsrc + STAGE + 32 * i * LD + 16 * (kk + 1));
#pragma unroll
            for (int j = 0; j < TN; ++j)
              bl[nxt][j] = *reinterpret_cast<const bf16x8_t*>(xsrc + STAGE + 32 * j * LD + 16 * (kk + 1));
          }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[cur][i], bv[cur][j], acc[i][j], 0, 0, 0);
        if constexpr (SP) {
          // w_hi x_lo + w_lo x_hi after the w_hi x_hi products (the lo x lo term, ~2^-16
          // relative, is left out)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[cur][i], bl[cur][j], acc[i][j], 0, 0, 0);
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[cur][i], bv[cur][j], acc[i][j], 0, 0, 0);
            }
        }
        if constexpr (DUAL) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av2[cur][i], bv[cur][j], acc2[i][j], 0, 0, 0);
        }
      }
    } else {
      // each lane reads four consecutive k of its row (one 16-byte LDS read: the 32 rows of a
      // read, 132 floats apart, cover all banks) and feeds four v_mfma_f32_32x32x2f32: MFMA q of
      // the eight-k slice kk takes k = 8 kk + q (lanes 0-31) and 8 kk + 4 + q (lanes 32-63), for
      // the weights and the activations alike
      const float* wsrc = Ws + (BM / WM * wm + (lane & 31)) * LD + 4 * (lane >> 5);
      const float* xsrc = Xs + (BN / WN * wn + (lane & 31)) * LD + 4 * (lane >> 5);
      // slice kk + 1 is read from LDS while the MFMAs of slice kk run
      float4 av[2][TM], bv[2][TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[0][i] = *reinterpret_cast<const float4*>(wsrc + 32 * i * LD);
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[0][j] = *reinterpret_cast<const float4*>(xsrc + 32 * j * LD);
#pragma unroll
      for (int kk = 0; kk < BK / 8; ++kk) {
        const int cur = kk & 1, nxt = cur ^ 1;
        if (kk + 1 < BK / 8) {
#pragma unroll
          for (int i = 0; i < TM; ++i) av[nxt][i] = *reinterpret_cast<const float4*>(wsrc + 32 * i * LD + 8 * (kk + 1));
#pragma unroll
          for (int j = 0; j < TN; ++j) bv[nxt][j] = *reinterpret_cast<const float4*>(xsrc + 32 * j * LD + 8 * (kk + 1));
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cur][i].x, bv[cur][j].x, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cur][i].y, bv[cur][j].y, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cur][i].z, bv[cur][j].z, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cur][i].w, bv[cur][j].w, acc[i][j], 0, 0, 0);
          }
      }
    }
#pragma unroll
    for (int jj = 0; jj < XV; ++jj) xdec[jj] = cvt(xraw[jj]);
    if constexpr (SP) {
#pragma unroll
      for (int jj = 0; jj < XV; ++jj) xdec_lo[jj] = cvt_lo(xraw[jj], xdec[jj]);
    }
    __syncthreads();                      // every wave is done reading step s
    write_lds(dec, dec2, xdec);           // step s + KG (zeros past the end)
    __syncthreads();
#pragma unroll
    for (int rep = 0; rep < WJOBS; ++rep) rawA[rep] = rawB[rep];
    if constexpr (DUAL) {
#pragma unroll
      for (int rep = 0; rep < WJOBS; ++rep) rawA2[rep] = rawB2[rep];
    }
  }
  if constexpr (DUAL) {
    // h = silu(gate) * up, elementwise on the finished accumulators
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = silu_mul(acc[i][j][r], acc2[i][j][r]);
  }

  if constexpr (KG > 1) {
    // fold the K-groups into group 0 in group order (deterministic), through LDS
    float* red = reinterpret_cast<float*>(smem);
    constexpr int WG_ACC = TM * TN * 16 * 64;   // accumulator floats of one wave
    if (grp > 0) {
      float* dst = red + ((grp - 1) * (WM * WN) + wave) * WG_ACC;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[((i * TN + j) * 16 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll 1
    for (int g = 1; g < KG; ++g) {
      const float* src = red + ((g - 1) * (WM * WN) + wave) * WG_ACC;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += src[((i * TN + j) * 16 + r) * 64 + lane];
    }
  }

  // ---- epilogue: D[i][j] of a 32x32 tile sits in lane j + 32*((i/4)%2), register 4*(i/8) + i%4,
  // i.e. a lane holds 4-float pieces of one output row. Each wave turns its tiles around through
  // its own LDS scratch (32 rows x 36 floats, past the K-group partials) so that 8 consecutive
  // lanes store one output row's 128 contiguous bytes.
  float* Y = p.splits > 1 ? p.partial + (size_t)split * p.N * p.ldy : p.Y;
  constexpr int SROW = 36;
  static_assert((KG - 1) * BM * BN * 4 + WM * WN * 32 * SROW * 4 <= KG * STAGE * (int)sizeof(E),
                "epilogue scratch fits in LDS");
  float* scr = reinterpret_cast<float*>(smem) + (KG - 1) * BM * BN + wave * 32 * SROW;
  const int xr8 = lane >> 3, c4 = 4 * (lane & 7);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4*>(scr + (lane & 31) * SROW + 8 * q + 4 * (lane >> 5)) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
      __builtin_amdgcn_wave_barrier();
      const int xl0 = BN / WN * wn + 32 * j;
      const int wr = BM * mtile + BM / WM * wm + 32 * i + c4;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int xr = 8 * t + xr8;
        const float4 v = *reinterpret_cast<const float4*>(scr + xr * SROW + c4);
        if constexpr (DUAL) {
          if (xl0 + xr < rn) {
            __bf16* hrow = reinterpret_cast<__bf16*>(p.Y) + (size_t)(r0 + xl0 + xr) * p.ldy;
            const float vv[4] = {v.x, v.y, v.z, v.w};
            if (wr + 3 < p.m) {
              bf16x4_t o;
              o[0] = (__bf16)v.x; o[1] = (__bf16)v.y; o[2] = (__bf16)v.z; o[3] = (__bf16)v.w;
              *reinterpret_cast<bf16x4_t*>(hrow + wr) = o;
            } else {
#pragma unroll
              for (int e = 0; e < 3; ++e)
                if (wr + e < p.m) hrow[wr + e] = (__bf16)vv[e];
            }
          }
          continue;
        }
        if (xl0 + xr < rn) {
          float* yrow = Y + (size_t)(r0 + xl0 + xr) * p.ldy;
          if (wr + 3 < p.m) {
            if (!GROUPED && p.splits == 1) {
              // the finished output of a dense launch is not read again by this launch: streaming
              // (nontemporal) stores keep it from occupying L2 (C1 N = 961: 25.0 -> 21.2 us)
              __builtin_nontemporal_store(f32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4_t*>(yrow + wr));
            } else {
              *reinterpret_cast<float4*>(yrow + wr) = v;
            }
          } else {
            if (wr < p.m) yrow[wr] = v.x;
            if (wr + 1 < p.m) yrow[wr + 1] = v.y;
            if (wr + 2 < p.m) yrow[wr + 2] = v.z;
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// Y[i] = sum over splits, in split order, of partial[split][i]  (i over N * ldy). The loads of
// eight splits are in flight together (a loop of dependent load-add steps waited one memory
// round trip per split); the adds keep split order, so the sums are the same bits.
template <typename V>
__device__ __forceinline__ V vadd(V a, V b);
template <> __device__ __forceinline__ float vadd(float a, float b) { return a + b; }
template <> __device__ __forceinline__ float4 vadd(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
// the reduced output is final: streaming (nontemporal) stores
__device__ __forceinline__ void store_final(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_final(float4* p, float4 v) {
  __builtin_nontemporal_store(f32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4_t*>(p));
}
template <typename V>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const V* __restrict__ partial, V* __restrict__ y, size_t n,
                                                          int splits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  // up to sixteen slices' loads in flight per round trip (the slice count is uniform, so the
  // guards are scalar branches); the sum runs in slice order
  V s = partial[i];
  for (int sp = 1; sp < splits; sp += 16) {
    V v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (sp + j < splits) v[j] = partial[(size_t)(sp + j) * n + i];
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (sp + j < splits) s = vadd(s, v[j]);
  }
  store_final(y + i, s);
}

static hipError_t launch_reduce(const float* partial, float* y, size_t n, int splits, hipStream_t s) {
  if (n % 4 == 0 && ((uintptr_t)partial & 15) == 0 && ((uintptr_t)y & 15) == 0) {
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(gemm_reduce_kernel<float4>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       (const float4*)partial, (float4*)y, n4, splits);
  } else {
    hipLaunchKernelGGL(gemm_reduce_kernel<float>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, partial, y, n,
                       splits);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_reduce(const float* partial, float* y, size_t n, int splits, hipStream_t s) {
  return launch_reduce(partial, y, n, splits, s);
}

// x[i] -> bf16 with round to nearest even (the rounding the bf16-mode GEMM applies to f32 X), 8
// elements (two 16-byte loads, one store) per thread
__global__ __launch_bounds__(256) void x_to_bf16_kernel(const float4* __restrict__ x, bf16x8_t* __restrict__ xb,
                                                        size_t n8) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256) {
    const float4 a = x[2 * i], b = x[2 * i + 1];
    bf16x8_t o;
    o[0] = (__bf16)a.x; o[1] = (__bf16)a.y; o[2] = (__bf16)a.z; o[3] = (__bf16)a.w;
    o[4] = (__bf16)b.x; o[5] = (__bf16)b.y; o[6] = (__bf16)b.z; o[7] = (__bf16)b.w;
    xb[i] = o;
  }
}

// the split form: hi = bf16(x) at xb[i], lo = bf16(x - hi) at xb[n8 + i] (8 elements per unit)
__global__ __launch_bounds__(256) void x_to_bf16_split_kernel(const float4* __restrict__ x, bf16x8_t* __restrict__ xb,
                                                              size_t n8) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256) {
    const float4 a = x[2 * i], b = x[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    bf16x8_t hi, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      hi[j] = (__bf16)v[j];
      lo[j] = (__bf16)(v[j] - (float)hi[j]);
    }
    xb[i] = hi;
    xb[n8 + i] = lo;
  }
}

template <int T, bool F32, int BM, int BN, int WM, int WN, int KG, bool GROUPED, bool SP = false>
static hipError_t launch_shape(const GemmArgs& a, int ntasks, hipStream_t s) {
  constexpr int NT = WM * WN * 64 * KG;
  if constexpr (GROUPED) {
    if constexpr (!F32) {
      if (a.W2) {
        if constexpr (KG == 1) {
          if (!a.x_bf16) return hipErrorInvalidValue;
          hipLaunchKernelGGL((gemm_kernel<T, false, true, BM, BN, WM, WN, 1, true, true>), dim3((unsigned)ntasks),
                             dim3(NT), 0, s, a);
          return hipGetLastError();
        } else {
          return hipErrorInvalidValue;
        }
      }
      if (a.x_bf16) {
        hipLaunchKernelGGL((gemm_kernel<T, false, true, BM, BN, WM, WN, KG, true>), dim3((unsigned)ntasks), dim3(NT),
                           0, s, a);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((gemm_kernel<T, F32, true, BM, BN, WM, WN, KG>), dim3((unsigned)ntasks), dim3(NT), 0, s, a);
    return hipGetLastError();
  } else {
    const int total = ((a.m + BM - 1) / BM) * ((a.N + BN - 1) / BN) * a.splits;
    const int grid = (total + 7) / 8 * 8;
    hipLaunchKernelGGL((gemm_kernel<T, F32, false, BM, BN, WM, WN, KG, false, false, SP>), dim3((unsigned)grid),
                       dim3(NT), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splits == 1) return e;
    return launch_reduce(a.partial, a.Y, (size_t)a.N * a.ldy, a.splits, s);
  }
}

// tile x K-group instances: dense 64x64 (KG 1/2) in both modes, 128x128, 128x192, 128x256 and
// 256x128 (KG 1) in bf16; grouped (MoE) 64x64 (KG 1/2) in both modes.
template <int T, bool F32>
static hipError_t launch_t(const GemmArgs& a, int ntasks, GemmTile tile, int kg, hipStream_t s) {
  if ((a.x_bf16 || a.W2) && (F32 || !a.tasks)) return hipErrorInvalidValue;   // grouped bf16 launches only
  if (a.tasks) {
    if (tile != GemmTile::k64x64) return hipErrorInvalidValue;
    if (kg == 1) return launch_shape<T, F32, 64, 64, 2, 2, 1, true>(a, ntasks, s);
    if (kg == 2) return launch_shape<T, F32, 64, 64, 2, 2, 2, true>(a, ntasks, s);
    return hipErrorInvalidValue;
  }
  switch (tile) {
    case GemmTile::k128x256:
      if constexpr (F32) return hipErrorInvalidValue;   // the f32 tile pair would need 198 KiB of LDS
      else return kg != 1 ? hipErrorInvalidValue : launch_shape<T, F32, 128, 256, 2, 4, 1, false>(a, ntasks, s);
    case GemmTile::k256x128:
      if constexpr (F32) return hipErrorInvalidValue;
      else return kg != 1 ? hipErrorInvalidValue : launch_shape<T, F32, 256, 128, 4, 2, 1, false>(a, ntasks, s);
    case GemmTile::k128x192:
      if constexpr (F32) return hipErrorInvalidValue;
      else return kg != 1 ? hipErrorInvalidValue : launch_shape<T, F32, 128, 192, 4, 2, 1, false>(a, ntasks, s);
    case GemmTile::k128x128:
      if constexpr (F32) return hipErrorInvalidValue;
      else return kg != 1 ? hipErrorInvalidValue : launch_shape<T, F32, 128, 128, 2, 2, 1, false>(a, ntasks, s);
    default:
      if (kg == 1) return launch_shape<T, F32, 64, 64, 2, 2, 1, false>(a, ntasks, s);
      if (kg == 2) return launch_shape<T, F32, 64, 64, 2, 2, 2, false>(a, ntasks, s);
      return hipErrorInvalidValue;
  }
}

// f32 mode on bf16 MFMAs (split operands): dense launches, 128 x 128 or 64 x 64 tiles, one K-group
template <int T>
static hipError_t launch_t_split(const GemmArgs& a, GemmTile tile, int kg, hipStream_t s) {
  if (a.tasks || a.x_bf16 || a.W2 || kg != 1) return hipErrorInvalidValue;
  if (tile == GemmTile::k128x128) return launch_shape<T, false, 128, 128, 2, 2, 1, false, true>(a, 0, s);
  if (tile == GemmTile::k64x64) return launch_shape<T, false, 64, 64, 2, 2, 1, false, true>(a, 0, s);
  return hipErrorInvalidValue;
}

template <int T>
static hipError_t launch_mode(int mode, const GemmArgs& a, int ntasks, GemmTile tile, int kg, hipStream_t s) {
  if (mode == kGemmModeSplit) return launch_t_split<T>(a, tile, kg, s);
  return mode == 1 ? launch_t<T, true>(a, ntasks, tile, kg, s) : launch_t<T, false>(a, ntasks, tile, kg, s);
}

int gemm_kgroups(GemmTile tile, int mode, long workgroups, int steps) {
  // K-groups multiply the waves of a workgroup so that small grids still put ~4 waves on
  // every SIMD; each group keeps at least 2 K steps
  const int cap = tile == GemmTile::k64x64 ? 2 : 1;
  const long waves_per_group = tile == GemmTile::k64x64 ? 4 : (tile == GemmTile::k128x128 ? 4 : 8);
  int kg = 1;
  while (kg * 2 <= cap && workgroups * waves_per_group * kg * 2 <= 4096 && steps >= 2 * kg * 2) kg *= 2;
  return kg;
}

GemmPlan plan_gemm(int m, int n, int K, int mode) {
  GemmPlan pl;
  const int steps = (K + kGemmBK - 1) / kGemmBK;
  if (mode == kGemmModeSplit) {
    // split operands (f32 mode on bf16 MFMAs). Many tiles: 64 x 64 (two workgroups per CU; C1 at
    // 961 rows 50.7 us against 61.3 on 128 x 128). Fewer: 128 x 128 on four waves of 64 x 64 (the
    // tiles and their remainders fill 139 KiB of LDS), K split toward 224 workgroups while the
    // partial tiles stay <= 32 MiB (C2 at 961 rows: 4 splits 50.2 us, 3 59.5, 5 75.7, 8 57.2)
    pl.kgroups = 1;
    const long t64 = (long)((m + 63) / 64) * ((n + 63) / 64);
    if (t64 >= 512) {
      pl.tile = GemmTile::k64x64;
    } else {
      pl.tile = GemmTile::k128x128;
      const long tiles = (long)((m + 127) / 128) * ((n + 127) / 128);
      if (tiles < 200 && steps >= 4) {
        long splits = std::min<long>((224 + tiles - 1) / tiles, steps / 2);
        while (splits > 1 && splits * (long)n * m * 4 > (32l << 20)) --splits;
        pl.splits = (int)std::max<long>(1, splits);
      }
    }
    pl.steps_per_split = (steps + pl.splits - 1) / pl.splits;
    pl.splits = (steps + pl.steps_per_split - 1) / pl.steps_per_split;
    return pl;
  }
  const long t128 = (long)((m + 127) / 128) * ((n + 127) / 128);
  const long t256 = (long)((m + 127) / 128) * ((n + 255) / 256);
  const long t64 = (long)((m + 63) / 64) * ((n + 63) / 64);
  if (mode == 0 && n >= 384) {
    // bf16 with many activation rows: 128 weight rows x 256 activation rows, 8 waves (the
    // 256 x 128 transpose measured no faster on the prefill shapes). Split K over workgroups
    // until ~200 workgroups run, while the partial tiles stay <= 32 MiB.
    pl.tile = GemmTile::k128x256;
    pl.kgroups = 1;
    const long tw = t256;
    if (tw < 200 && steps >= 4) {
      long splits = std::min<long>((200 + tw - 1) / tw, steps / 2);
      while (splits > 1 && splits * (long)n * m * 4 > (32l << 20)) --splits;
      pl.splits = (int)std::max<long>(1, splits);
    }
    // unsplit, and 192-row tiles still fit one workgroup per CU: the smaller tile puts more CUs
    // to work (C1: 228 instead of 152 workgroups, 23.8 instead of 25.0 us)
    const long t192 = (long)((m + 127) / 128) * ((n + 191) / 192);
    if (pl.splits == 1 && t192 > tw && t192 <= 256) pl.tile = GemmTile::k128x192;
  } else if (t128 >= 200) {
    // many tiles already: 64 x 64 with one K-group (the 128 x 128 bf16 tile measured slower)
    pl.tile = GemmTile::k64x64;
    pl.kgroups = 1;
  } else {
    pl.tile = GemmTile::k64x64;
    // f32 over many tiles: spread K over workgroups rather than over K-groups inside them (C2 at
    // N = 961: 224 tiles, two K splits of one group each, 116 instead of 129 us for one K-group
    // pair per split)
    const bool wide = mode == 1 && t64 >= 128;
    pl.kgroups = wide ? 1 : gemm_kgroups(pl.tile, mode, t64, steps);
    // few tiles over a deep K: also split the K steps over workgroups when the partial tiles stay
    // small (each split keeps >= 2 steps per K-group)
    const long groups = t64 * pl.kgroups;
    const long target = wide ? 448 : 512;
    if (groups < target && steps >= 4 * pl.kgroups) {
      long splits = (target + groups - 1) / groups;
      splits = std::min<long>(splits, steps / (2 * pl.kgroups));
      const long partial_bytes = splits * (long)n * m * 4;
      if (partial_bytes <= (16l << 20) && splits > 1) pl.splits = (int)splits;
    }
  }
  pl.steps_per_split = (steps + pl.splits - 1) / pl.splits;
  pl.splits = (steps + pl.steps_per_split - 1) / pl.steps_per_split;
  return pl;
}

hipError_t launch_x_to_bf16(const float* x, void* xb, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  if (n % 8) return hipErrorInvalidValue;
  const size_t n8 = n / 8;
  const unsigned grid = (unsigned)std::min<size_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(x_to_bf16_kernel, dim3(grid), dim3(256), 0, s, (const float4*)x, (bf16x8_t*)xb, n8);
  return hipGetLastError();
}

hipError_t launch_x_to_bf16_split(const float* x, void* xb, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  if (n % 8) return hipErrorInvalidValue;
  const size_t n8 = n / 8;
  const unsigned grid = (unsigned)std::min<size_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(x_to_bf16_split_kernel, dim3(grid), dim3(256), 0, s, (const float4*)x, (bf16x8_t*)xb, n8);
  return hipGetLastError();
}

hipError_t launch_gemm(uint32_t type, int mode, const GemmArgs& a, int ntasks, GemmTile tile, int kgroups,
                       hipStream_t s) {
  switch (type) {
    case T_Q4_0: return launch_mode<T_Q4_0>(mode, a, ntasks, tile, kgroups, s);
    case T_Q5_0: return launch_mode<T_Q5_0>(mode, a, ntasks, tile, kgroups, s);
    case T_Q8_0: return launch_mode<T_Q8_0>(mode, a, ntasks, tile, kgroups, s);
    case T_Q4_K: return launch_mode<T_Q4_K>(mode, a, ntasks, tile, kgroups, s);
    case T_Q5_K: return launch_mode<T_Q5_K>(mode, a, ntasks, tile, kgroups, s);
    case T_Q6_K: return launch_mode<T_Q6_K>(mode, a, ntasks, tile, kgroups, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rehip
