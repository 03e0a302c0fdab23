// Device-side repack of GGUF row-major blocks into the tiled-slab layout (the inverse order
// of layout.cpp's host repack, same result byte for byte): the GGUF loader copies a tensor's
// bytes to the device unchanged and the permutation runs here, so no host pass touches them.
// One 256-thread workgroup per slab (matrix, tile t, block column kb): the 64 rows' blocks are
// read into LDS (64 runs of BB contiguous bytes), then each plane of the slab is written with
// consecutive threads on consecutive 16-bit words. Rows past m write zero blocks.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "kernels.hpp"

namespace rehip {

struct RepackPlanes {
  int n;
  int off[16], width[16];
};

// Grid: mats x tiles x kb_count slabs. Matrix mi's GGUF rows start at src + mi * mat_src (m rows
// of kb_count * bb bytes) and its tiled slabs at dst + mi * dst_stride. Every block offset is even
// (bb is even), so the bytes move as 16-bit words.
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                     int m, int tiles, int kb_count, int bb, size_t mat_src,
                                                     size_t dst_stride, RepackPlanes pl) {
  __shared__ uint16_t blk[64 * 210 / 2];
  const int per_mat = tiles * kb_count;
  const int mi = blockIdx.x / per_mat;
  const int slab = blockIdx.x - mi * per_mat;   // t * kb_count + kb
  const int t = slab / kb_count, kb = slab - t * kb_count;
  const size_t row_bytes = (size_t)kb_count * bb;
  const int hw = bb / 2;                        // 16-bit words per block
  const uint8_t* msrc = src + (size_t)mi * mat_src;
  for (int i = threadIdx.x; i < 64 * hw; i += 256) {
    const int r = i / hw, c = i - r * hw;
    const int row = t * 64 + r;
    blk[i] = row < m ? *(const uint16_t*)(msrc + (size_t)row * row_bytes + (size_t)kb * bb + 2 * c) : 0;
  }
  __syncthreads();
  uint16_t* out = (uint16_t*)(dst + (size_t)mi * dst_stride + (size_t)slab * 64 * bb);
  for (int p = 0; p < pl.n; ++p) {
    const int w = pl.width[p] / 2, off = pl.off[p] / 2;
    for (int i = threadIdx.x; i < 64 * w; i += 256) {
      const int r = i / w, c = i - r * w;
      out[i] = blk[r * hw + off + c];
    }
    out += 64 * w;
  }
}

hipError_t launch_repack(uint32_t type, const uint8_t* src, uint8_t* dst, int m, int kb, int tiles, int mats,
                         size_t mat_src, size_t dst_stride, hipStream_t s) {
  const TypeInfo* ti = type_info(type);
  if (!ti) return hipErrorInvalidValue;
  RepackPlanes pl{};
  pl.n = ti->nplanes;
  for (int p = 0; p < ti->nplanes; ++p) {
    pl.off[p] = ti->planes[p].off;
    pl.width[p] = ti->planes[p].width;
  }
  hipLaunchKernelGGL(repack_kernel, dim3((unsigned)(mats * tiles * kb)), dim3(256), 0, s, src, dst, m, tiles, kb,
                     ti->bb, mat_src, dst_stride, pl);
  return hipGetLastError();
}

}  // namespace rehip
