// Shared definitions for librehip: GGUF block geometry and the GPU-resident weight layout.
//
// Weight layout in HBM ("tiled slabs"). A quantized m x n matrix (row-major, each row
// ceil(n/QK) GGUF blocks; src/qmat.rs:30-42, src/kernel.rs:1983-1993) is stored as
//
//   tile t = rows 64t .. 64t+63 (m padded to a multiple of 64 with zero blocks)
//     block column kb = 0 .. KB-1 (KB = ceil(n/QK))
//       slab = 64 x BB bytes, split into the type's planes; plane p holds bytes
//              [off_p, off_p + w_p) of every row's block, row-major over the 64 rows.
//
// Slabs of one tile are contiguous in kb order, tiles follow each other. One lane of a
// wavefront owns one row of a tile, so a plane of width 16 is fetched by one wave-wide
// dwordx4 load covering 1 KiB of contiguous memory (eight full 128-byte lines), width 4 and
// 2 planes by dword/ushort loads covering 256/128 contiguous bytes. The bytes themselves are
// unchanged (same total as the GGUF stream, plus row padding); only their order differs.
#pragma once

#include <cstddef>
#include <cstdint>

namespace rehip {

enum GgmlType : uint32_t {
  T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14
};

constexpr int kTileRows = 64;   // rows per tile = lanes per wavefront

struct Plane { int off; int width; };

// Per-type block geometry and plane split (byte offsets inside the GGUF block).
//  Q4_0 [d 2][qs 16]                      -> qs(16) d(2)
//  Q5_0 [d 2][qh 4][qs 16]                -> qs(16) qh(4) d(2)
//  Q8_0 [d 2][qs 32]                      -> qs0(16) qs1(16) d(2)
//  Q4_K [d 2][dmin 2][sc 12][qs 128]      -> head(16) qs x8
//  Q5_K [d 2][dmin 2][sc 12][qh 32][qs128]-> head(16) qh x2 qs x8
//  Q6_K [ql 128][qh 64][sc 16][d 2]       -> ql x8 qh x4 sc(16) d(2)
struct TypeInfo {
  uint32_t type;
  int qk;        // elements per block
  int bb;        // bytes per block
  int nplanes;
  Plane planes[16];
};

inline const TypeInfo* type_info(uint32_t t) {
  static const TypeInfo q4_0 = {T_Q4_0, 32, 18, 2, {{2, 16}, {0, 2}}};
  static const TypeInfo q5_0 = {T_Q5_0, 32, 22, 3, {{6, 16}, {2, 4}, {0, 2}}};
  static const TypeInfo q8_0 = {T_Q8_0, 32, 34, 3, {{2, 16}, {18, 16}, {0, 2}}};
  static const TypeInfo q4_k = {T_Q4_K, 256, 144, 9,
      {{0, 16}, {16, 16}, {32, 16}, {48, 16}, {64, 16}, {80, 16}, {96, 16}, {112, 16}, {128, 16}}};
  static const TypeInfo q5_k = {T_Q5_K, 256, 176, 11,
      {{0, 16}, {16, 16}, {32, 16}, {48, 16}, {64, 16}, {80, 16}, {96, 16}, {112, 16}, {128, 16},
       {144, 16}, {160, 16}}};
  static const TypeInfo q6_k = {T_Q6_K, 256, 210, 14,
      {{0, 16}, {16, 16}, {32, 16}, {48, 16}, {64, 16}, {80, 16}, {96, 16}, {112, 16},
       {128, 16}, {144, 16}, {160, 16}, {176, 16}, {192, 16}, {208, 2}}};
  switch (t) {
    case T_Q4_0: return &q4_0;
    case T_Q5_0: return &q5_0;
    case T_Q8_0: return &q8_0;
    case T_Q4_K: return &q4_k;
    case T_Q5_K: return &q5_k;
    case T_Q6_K: return &q6_k;
    default: return nullptr;
  }
}

// Geometry of one uploaded matrix.
struct MatGeom {
  uint32_t type;
  size_t m, n;        // logical shape (rows, inner width)
  int qk, bb;
  size_t kb;          // block columns per row = ceil(n / qk)
  size_t tiles;       // ceil(m / 64)
  size_t slab_bytes;  // 64 * bb
  size_t bytes;       // tiles * kb * slab_bytes
};

inline bool make_geom(uint32_t t, size_t m, size_t n, MatGeom* g) {
  const TypeInfo* ti = type_info(t);
  if (!ti || m == 0 || n == 0) return false;
  g->type = t;
  g->m = m;
  g->n = n;
  g->qk = ti->qk;
  g->bb = ti->bb;
  g->kb = (n + ti->qk - 1) / ti->qk;
  g->tiles = (m + kTileRows - 1) / kTileRows;
  g->slab_bytes = (size_t)kTileRows * ti->bb;
  g->bytes = g->tiles * g->kb * g->slab_bytes;
  return true;
}

// Host repack: GGUF row-major blocks (m rows x kb blocks, `src`) -> tiled slabs (`dst`,
// g.bytes long; padding rows are zero). Pure byte permutation.
void repack_host(const MatGeom& g, const uint8_t* src, uint8_t* dst);
// Inverse of repack_host (used by tests of the layout).
void unrepack_host(const MatGeom& g, const uint8_t* src, uint8_t* dst);

}  // namespace rehip
