// Kernel argument blocks and host-side launchers shared by the C ABI (api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace rehip {

struct GemvArgs {
  const uint8_t* W;      // tiled slabs of one matrix
  const float* x;        // K floats
  float* y;              // m floats
  float* partial;        // splits * m_pad floats (splits > 1), reduced by a second kernel
  int m, m_pad, K, KB, tiles;
  int kb_per_split, splits;
};

// waves per workgroup: 4 or 8
hipError_t launch_gemv(uint32_t type, const GemvArgs& a, int waves, hipStream_t s);
hipError_t launch_dequant(uint32_t type, const uint8_t* W, float* out, int m, int n, int KB, int tiles,
                          hipStream_t s);

// GEMM: K steps of 128 elements; square tiles of 128 or 64 (weight rows x activation rows).
constexpr int kGemmBK = 128;
constexpr int kMoeTile = 64;   // tile of the grouped (MoE) launches

// Work item of a grouped launch (MoE): one BM x BN output tile of one expert.
struct GemmTask {
  int expert;     // weight matrix index (byte offset expert * w_stride)
  int mtile;      // BM tile along the weight rows
  int r0;         // first gathered row of the tile
  int rn;         // valid rows in the tile (<= BN)
};

struct GemmArgs {
  const uint8_t* W;        // tiled slabs (expert 0)
  size_t w_stride;         // bytes between experts
  const float* X;          // activations, row-major, K floats per row
  float* Y;                // output, row stride ldy
  int m, K, KB, tiles;     // weight geometry (per expert)
  int N;                   // activation rows (dense launch)
  int ldy;
  const GemmTask* tasks;   // grouped launch: one task per workgroup (nullptr = dense 2-D grid)
  const int* xrow;         // grouped: X row of gathered row p (nullptr = p itself)
};

// mode 0 = bf16 MFMA with f32 accumulation, 1 = f32 MFMA (strict parity); tile 128 or 64
hipError_t launch_gemm(uint32_t type, int mode, const GemmArgs& a, int ntasks, int tile, hipStream_t s);
// tile a dense m x n-row launch uses
int gemm_tile_for(int m, int n);

// MoE helpers
hipError_t launch_swiglu(const float* g, const float* u, float* h, size_t n, hipStream_t s);
hipError_t launch_combine(const float* yp, const int* pos, const float* w, float* out, int tokens,
                          int k, int hidden, hipStream_t s);

}  // namespace rehip
