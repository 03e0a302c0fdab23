// Host-side repack of GGUF row-major blocks into the tiled-slab layout (see common.hpp).
// The layout transform follows the idea of the reference's compute-friendly repack
// (src/repack.rs:1-16: split scales and quants into separate streams) but keeps every byte
// as stored, so the GPU reads exactly the GGUF byte count.
#include <cstring>

#include "common.hpp"

namespace rehip {

namespace {
template <bool kForward>
void permute(const MatGeom& g, const uint8_t* src, uint8_t* dst) {
  const TypeInfo* ti = type_info(g.type);
  const size_t row_bytes = g.kb * g.bb;
  if (kForward) std::memset(dst, 0, g.bytes);
  for (size_t t = 0; t < g.tiles; ++t) {
    for (size_t kb = 0; kb < g.kb; ++kb) {
      uint8_t* slab = (kForward ? dst : const_cast<uint8_t*>(src)) + (t * g.kb + kb) * g.slab_bytes;
      size_t plane_base = 0;
      for (int p = 0; p < ti->nplanes; ++p) {
        const int w = ti->planes[p].width, off = ti->planes[p].off;
        for (int r = 0; r < kTileRows; ++r) {
          const size_t row = t * kTileRows + r;
          if (row >= g.m) break;
          uint8_t* flat = (kForward ? const_cast<uint8_t*>(src) : dst) + row * row_bytes + kb * g.bb + off;
          uint8_t* tiled = slab + plane_base + (size_t)r * w;
          if (kForward) std::memcpy(tiled, flat, w);
          else std::memcpy(flat, tiled, w);
        }
        plane_base += (size_t)kTileRows * w;
      }
    }
  }
}
}  // namespace

void repack_host(const MatGeom& g, const uint8_t* src, uint8_t* dst) { permute<true>(g, src, dst); }
void unrepack_host(const MatGeom& g, const uint8_t* src, uint8_t* dst) { permute<false>(g, src, dst); }

}  // namespace rehip
