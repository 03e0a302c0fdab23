// Int8 activation path (src/kernel.rs:70-166, Q8Activation / dot_q8_0_i8 / matmul_q8_0_i8):
// activations quantized per 32-value block to i8 with an f32 scale, multiplied against Q8_0
// weights with i8 MFMAs. Results are bit-identical to the reference's scalar integer dot: the
// i32 block sums are exact whatever the order, and each output's blocks are folded by one lane,
// in block order, as s += ((f32)isum * dw) * dx with no fused multiply-add.
#include <hip/hip_runtime.h>

#include "deq.hpp"
#include "kernels.hpp"

namespace rehip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// One thread per (row, 32-value block): Q8Activation::from_f32 (kernel.rs:88-105). d = max|x|/127
// (NaN never wins the max), inv = 1/d or 0, q = round-half-away(x * inv) clamped to [-127, 127],
// a NaN product gives 0. Division and rounding are the IEEE-exact device operations.
__global__ __launch_bounds__(256) void quantize_q8_act_kernel(const float* __restrict__ x, int rows, int n,
                                                              float* __restrict__ scales, int8_t* __restrict__ qs) {
  const int nb = n >> 5;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)rows * nb) return;
  const int row = (int)(i / nb), kb = (int)(i - (long long)row * nb);
  const float4* src = reinterpret_cast<const float4*>(x + (size_t)row * n + (size_t)kb * 32);
  float v[32];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float4 f = src[j];
    v[4 * j] = f.x;
    v[4 * j + 1] = f.y;
    v[4 * j + 2] = f.z;
    v[4 * j + 3] = f.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  const float d = amax / 127.0f;
  const float inv = d > 0.0f ? 1.0f / d : 0.0f;
  uint32_t packed[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      float r = roundf(v[4 * j + b] * inv);
      r = r != r ? 0.0f : fminf(fmaxf(r, -127.0f), 127.0f);
      w |= ((uint32_t)(uint8_t)(int8_t)(int)r) << (8 * b);
    }
    packed[j] = w;
  }
  uint4* dst = reinterpret_cast<uint4*>(qs + (size_t)row * n + (size_t)kb * 32);
  dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  scales[i] = d;
}

constexpr int kI8Chunk = 256;  // blocks of activation scales staged in LDS at a time (n <= 8192: one)
constexpr int kI8Ahead = 4;    // blocks whose operands are in flight ahead of the MFMA

// Y (rows x m) = Q8_0 W (m x n, tiled slabs) times quantized activations. Workgroup = 2 waves =
// one 64-row weight tile x 32 activation rows; wave w owns weight rows 32w..32w+31 of the tile.
// Per block one v_mfma_i32_32x32x32_i8 (A = 32 activation rows x 32 i8, B = 32 i8 x 32 weight
// rows; lane l supplies row/column l%32 and bytes 16(l/32)..+15 of the block to both, so the
// i32 sums are the exact block dot products) and the f32 fold of the 16 results the lane holds:
// activation rows 8(i/4) + 4(l/32) + i%4 of weight row l%32. The activation scales of up to 256
// blocks are staged in LDS (block-major) once; blocks then go in groups of kI8Ahead with no
// branch inside a group, the operands of the next group loading while this one is folded (a
// branch between an MFMA and the reads of its result, or between a load and its use, makes the
// compiler wait for every outstanding load, or miscount the MFMA's result latency).
__global__ __launch_bounds__(128) void q8_i8_gemm_kernel(const uint8_t* __restrict__ W, const float* __restrict__ xs,
                                                         const int8_t* __restrict__ xq, float* __restrict__ y, int m,
                                                         int n, int rows) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float dxs_flat[];     // min(nb, kI8Chunk) x 32
  float (*dxs)[32] = reinterpret_cast<float (*)[32]>(dxs_flat);
  const int nb = n >> 5;
  const int tile = blockIdx.x, r0 = blockIdx.y * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, c = lane & 31;
  const int trow = wave * 32 + c;                       // weight row inside the tile
  const uint8_t* wb = W + (size_t)tile * nb * (64 * 34) + h * (64 * 16) + trow * 16;
  const uint8_t* wd = W + (size_t)tile * nb * (64 * 34) + 2 * (64 * 16) + trow * 2;
  const int8_t* arow = xq + (size_t)min(r0 + c, rows - 1) * n + 16 * h;
  v4i A[kI8Ahead], Bw[kI8Ahead];
  uint32_t D[kI8Ahead];
#pragma unroll
  for (int j = 0; j < kI8Ahead; ++j) {
    const int kn = min(j, nb - 1);
    A[j] = *reinterpret_cast<const v4i*>(arow + (size_t)kn * 32);
    Bw[j] = *reinterpret_cast<const v4i*>(wb + (size_t)kn * (64 * 34));
    D[j] = *reinterpret_cast<const uint16_t*>(wd + (size_t)kn * (64 * 34));
  }
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = 0.0f;

  // one block: MFMA on slot j, refill slot j with block kb + kI8Ahead (clamped), fold
  auto step = [&](const int j, const int kb, const float* dxrow) __attribute__((always_inline)) {
    const v16i z = {};
    const v16i acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[j], Bw[j], z, 0, 0, 0);
    const float dw = f16_bits_to_f32(D[j]);
    const int kn = min(kb + kI8Ahead, nb - 1);
    A[j] = *reinterpret_cast<const v4i*>(arow + (size_t)kn * 32);
    Bw[j] = *reinterpret_cast<const v4i*>(wb + (size_t)kn * (64 * 34));
    D[j] = *reinterpret_cast<const uint16_t*>(wd + (size_t)kn * (64 * 34));
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 dx = *reinterpret_cast<const float4*>(dxrow + 8 * g + 4 * h);
      const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int i = 4 * g + jj;
        const float t = ((float)acc[i] * dw) * dxv[jj];   // no contraction: fp contract(off) above
        s[i] = s[i] + t;
      }
    }
  };

  for (int kb0 = 0; kb0 < nb; kb0 += kI8Chunk) {
    const int kc = min(kI8Chunk, nb - kb0);
    __syncthreads();
    // scales of 32 activation rows x kc blocks -> dxs[block][row]; loads issued 8 at a time
    for (int e0 = threadIdx.x; e0 < kc * 32; e0 += 128 * 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + 128 * u;
        const int t = e / kc, k = e - t * kc;
        v[u] = e < kc * 32 ? xs[(size_t)min(r0 + t, rows - 1) * nb + kb0 + k] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + 128 * u;
        const int t = e / kc, k = e - t * kc;
        if (e < kc * 32) dxs[k][t] = v[u];
      }
    }
    __syncthreads();
    const int full = kc & ~(kI8Ahead - 1);
    for (int k = 0; k < full; k += kI8Ahead) {
#pragma unroll
      for (int j = 0; j < kI8Ahead; ++j) step(j, kb0 + k + j, dxs[k + j]);
    }
    // blocks past the last whole group (only in the last chunk: kI8Chunk is a multiple of 4)
#pragma unroll
    for (int j = 0; j < kI8Ahead - 1; ++j)
      if (full + j < kc) step(j, kb0 + full + j, dxs[full + j]);
  }
  const int wr = tile * 64 + trow;
  if (wr >= m) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = r0 + 8 * (i >> 2) + 4 * h + (i & 3);
    if (r < rows) y[(size_t)r * m + wr] = s[i];
  }
}

constexpr int kSegWaves = 4;    // K segments (one per wave) of one output tile
constexpr int kSegBlocks = 4;   // blocks per wave per round

// Long rows over few output tiles: one 32 x 32 output tile per workgroup of kSegWaves waves. A
// round covers kSegWaves * kSegBlocks consecutive blocks; wave w takes kSegBlocks of them and
// computes their terms ((f32)isum * dw) * dx in parallel with the other waves (one i8 MFMA per
// block, as q8_i8_gemm_kernel), then the running sums (16 per lane) pass from wave to wave
// through LDS, each wave adding its terms in block order: the same fold, in the same order, as
// one lane walking all blocks, with only the adds serial. The next round's operands load during
// the folds (keeping two rounds in flight measured no faster: the compiler's wait counts then
// drain every outstanding load at the round's first MFMA).
__global__ __launch_bounds__(64 * kSegWaves) void q8_i8_gemm_seg_kernel(const uint8_t* __restrict__ W,
                                                                         const float* __restrict__ xs,
                                                                         const int8_t* __restrict__ xq,
                                                                         float* __restrict__ y, int m, int n,
                                                                         int rows) {
#pragma clang fp contract(off)
  constexpr int S = kSegWaves, KBs = kSegBlocks, RB = S * KBs;
  static_assert(kI8Chunk % RB == 0, "scale chunks hold whole rounds");
  extern __shared__ __align__(16) float dxs_flat[];   // min(nb, kI8Chunk) x 32 scales
  float (*dxs)[32] = reinterpret_cast<float (*)[32]>(dxs_flat);
  __shared__ float sbuf[16][64];          // running sums, [result register][lane]
  const int nb = n >> 5;
  const int grp = blockIdx.x;             // 32 weight rows: tile grp/2, rows 32 (grp%2) ..
  const int tile = grp >> 1;
  const int r0 = blockIdx.y * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, c = lane & 31;
  const int trow = (grp & 1) * 32 + c;
  const uint8_t* wb = W + (size_t)tile * nb * (64 * 34) + h * (64 * 16) + trow * 16;
  const uint8_t* wd = W + (size_t)tile * nb * (64 * 34) + 2 * (64 * 16) + trow * 2;
  const int8_t* arow = xq + (size_t)min(r0 + c, rows - 1) * n + 16 * h;
  const int rounds = (nb + RB - 1) / RB;
  v4i A[KBs], Bw[KBs];
  uint32_t D[KBs];
  auto load = [&](int rr, v4i (&a)[KBs], v4i (&b)[KBs], uint32_t (&d)[KBs]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < KBs; ++j) {
      const int kb = min(rr * RB + wave * KBs + j, nb - 1);
      a[j] = *reinterpret_cast<const v4i*>(arow + (size_t)kb * 32);
      b[j] = *reinterpret_cast<const v4i*>(wb + (size_t)kb * (64 * 34));
      d[j] = *reinterpret_cast<const uint16_t*>(wd + (size_t)kb * (64 * 34));
    }
  };
  load(0, A, Bw, D);
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = 0.0f;
  auto round = [&](int rr, v4i (&a)[KBs], v4i (&b)[KBs], uint32_t (&d)[KBs]) __attribute__((always_inline)) {
    const int b0 = rr * RB;
    const int kc0 = b0 / kI8Chunk * kI8Chunk;     // first block of the staged scale chunk
    if (b0 == kc0) {
      // scales of 32 activation rows x the chunk's blocks -> dxs[block][row], 8 loads in flight
      const int kc = min(kI8Chunk, nb - kc0);
      __syncthreads();                    // the previous chunk's readers are done
      for (int e0 = threadIdx.x; e0 < kc * 32; e0 += 64 * S * 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int e = e0 + 64 * S * u;
          const int t = e / kc, k = e - t * kc;
          v[u] = e < kc * 32 ? xs[(size_t)min(r0 + t, rows - 1) * nb + kc0 + k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int e = e0 + 64 * S * u;
          const int t = e / kc, k = e - t * kc;
          if (e < kc * 32) dxs[k][t] = v[u];
        }
      }
      __syncthreads();
    }
    float tm[KBs][16];
#pragma unroll
    for (int j = 0; j < KBs; ++j) {
      const v16i acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], b[j], v16i{}, 0, 0, 0);
      const float dw = f16_bits_to_f32(d[j]);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int kl = min(b0 + wave * KBs + j, nb - 1) - kc0;   // clamped blocks are not folded
        const float4 dx = *reinterpret_cast<const float4*>(&dxs[kl][8 * g + 4 * h]);
        const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) tm[j][4 * g + jj] = ((float)acc[4 * g + jj] * dw) * dxv[jj];
      }
    }
    if (rr + 1 < rounds) load(rr + 1, a, b, d);   // the next round's operands load during the folds
    // ordered fold: waves 0 .. S-1 in turn, each continuing the running sums of the one before
    for (int w = 0; w < S; ++w) {
      if (wave == w) {
        if (rr > 0 || w > 0) {
#pragma unroll
          for (int i = 0; i < 16; ++i) s[i] = sbuf[i][lane];
        }
#pragma unroll
        for (int j = 0; j < KBs; ++j) {
          if (b0 + w * KBs + j < nb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) s[i] = s[i] + tm[j][i];
          }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sbuf[i][lane] = s[i];
      }
      __syncthreads();
    }
  };
  for (int rr = 0; rr < rounds; ++rr) round(rr, A, Bw, D);
  if (wave != 0) return;
  const int wr = tile * 64 + trow;
  if (wr >= m) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = r0 + 8 * (i >> 2) + 4 * h + (i & 3);
    if (r < rows) y[(size_t)r * m + wr] = sbuf[i][lane];
  }
}

constexpr int kI8GemvRows = 16;       // weight rows per workgroup
constexpr int kI8GemvMaxBlocks = 960; // 16 x (nb + 1) f32 terms in LDS, at most 61.5 KB (n <= 30720)

// One activation row (matvec_q8_0_i8, kernel.rs:145-154). Workgroup = 256 threads = 16 weight
// rows x 16 block lanes: thread (row, j) computes the terms ((f32)isum * dw) * dx of blocks
// j, j + 16, ... of its row (isum by v_dot4_i32_i8, exact) into LDS; then one lane per row adds
// its row's terms in block order.
__global__ __launch_bounds__(256) void q8_i8_gemv_kernel(const uint8_t* __restrict__ W, const float* __restrict__ xs,
                                                         const int8_t* __restrict__ xq, float* __restrict__ y, int m,
                                                         int n) {
#pragma clang fp contract(off)
  extern __shared__ float terms[];               // kI8GemvRows x (nb + 1)
  const int nb = n >> 5;
  const int stride = nb + 1;
  const int r = threadIdx.x & (kI8GemvRows - 1), j = threadIdx.x >> 4;
  const int row = blockIdx.x * kI8GemvRows + r;         // may pass m: padding rows are zero
  const int tile = row >> 6, trow = row & 63;
  const uint8_t* slab0 = W + (size_t)tile * nb * (64 * 34);
  for (int kb = j; kb < nb; kb += 16) {
    const uint8_t* slab = slab0 + (size_t)kb * (64 * 34);
    const uint4 w0 = *reinterpret_cast<const uint4*>(slab + trow * 16);
    const uint4 w1 = *reinterpret_cast<const uint4*>(slab + 64 * 16 + trow * 16);
    const float dw = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(slab + 2 * (64 * 16) + trow * 2));
    const uint4 a0 = *reinterpret_cast<const uint4*>(xq + (size_t)kb * 32);
    const uint4 a1 = *reinterpret_cast<const uint4*>(xq + (size_t)kb * 32 + 16);
    int isum = 0;
    isum = __builtin_amdgcn_sdot4((int)w0.x, (int)a0.x, isum, false);
    isum = __builtin_amdgcn_sdot4((int)w0.y, (int)a0.y, isum, false);
    isum = __builtin_amdgcn_sdot4((int)w0.z, (int)a0.z, isum, false);
    isum = __builtin_amdgcn_sdot4((int)w0.w, (int)a0.w, isum, false);
    isum = __builtin_amdgcn_sdot4((int)w1.x, (int)a1.x, isum, false);
    isum = __builtin_amdgcn_sdot4((int)w1.y, (int)a1.y, isum, false);
    isum = __builtin_amdgcn_sdot4((int)w1.z, (int)a1.z, isum, false);
    isum = __builtin_amdgcn_sdot4((int)w1.w, (int)a1.w, isum, false);
    terms[r * stride + kb] = ((float)isum * dw) * xs[kb];
  }
  __syncthreads();
  if (j != 0 || row >= m) return;
  float acc = 0.0f;
  for (int kb = 0; kb < nb; ++kb) acc = acc + terms[r * stride + kb];
  y[row] = acc;
}

}  // namespace

hipError_t launch_quantize_q8_act(const float* x, int rows, int n, float* scales, int8_t* qs, hipStream_t s) {
  const long long blocks = (long long)rows * (n >> 5);
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_q8_act_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s, x, rows, n,
                     scales, qs);
  return hipGetLastError();
}

hipError_t launch_q8_i8_gemm(const uint8_t* W, int tiles, const float* xs, const int8_t* xq, float* y, int m, int n,
                             int rows, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  if (rows == 1 && (n >> 5) <= kI8GemvMaxBlocks) {
    const size_t lds = (size_t)kI8GemvRows * ((n >> 5) + 1) * sizeof(float);
    hipLaunchKernelGGL(q8_i8_gemv_kernel, dim3((unsigned)(tiles * (64 / kI8GemvRows))), dim3(256), lds, s, W, xs, xq,
                       y, m, n);
    return hipGetLastError();
  }
  const unsigned rgroups = (unsigned)((rows + 31) / 32);
  // long rows over few output tiles: split each tile's fold over the waves of a workgroup
  if ((n >> 5) >= 64 && (size_t)tiles * 2 * rgroups < 512) {
    const size_t lds = (size_t)min(n >> 5, kI8Chunk) * 32 * sizeof(float);
    hipLaunchKernelGGL(q8_i8_gemm_seg_kernel, dim3((unsigned)tiles * 2, rgroups), dim3(64 * kSegWaves), lds, s, W,
                       xs, xq, y, m, n, rows);
    return hipGetLastError();
  }
  const size_t lds = (size_t)min(n >> 5, kI8Chunk) * 32 * sizeof(float);
  hipLaunchKernelGGL(q8_i8_gemm_kernel, dim3((unsigned)tiles, rgroups), dim3(128), lds, s, W, xs, xq, y, m, n, rows);
  return hipGetLastError();
}

}  // namespace rehip
