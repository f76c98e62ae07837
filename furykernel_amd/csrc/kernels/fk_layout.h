// fk_layout.h — the tile layout: how a matrix that feeds the matrix cores
// sits in HBM.
//
// A matrix X [R, K] of f16 (R a multiple of 256, K of 32) is held as slabs of
// 256 rows; a slab, for each step of 32 columns, as 16 chunks of 1 KB (rows
// 16 c .. 16 c + 15 of the slab); a chunk as 64 units of 16 bytes, unit L
// holding row L div 4 of the chunk and the 8 columns of logical unit
// (L mod 4) ^ ((row div 4) mod 4) of the step.  That is the image the GEMM
// stages in LDS, so one direct load of 1 KB of contiguous HBM fills a chunk.
// The XOR swizzle is for the matrix-operation fragment reads (32 rows × one
// 16-byte unit): a 16-byte LDS read serves 16 lanes a cycle from 64 banks
// (256 bytes), and in 64-byte rows, rows r, r + 4, r + 8, r + 12 of a chunk
// fall on the same banks; XORing the unit with row div 4 puts those four
// rows' units in four different places (measured: 1.65 times the read rate
// of the row div 2 swizzle, which leaves them 2-way conflicted).
//
// Offsets are in halves:
//   ((slab · K/32 + step) · 16 + chunk) · 512 + unit · 8 + half.
#pragma once

#include <stdint.h>

namespace fk {

// The swizzle of row r (0..15) of a chunk.
__host__ __device__ __forceinline__ uint32_t tile_swizzle(uint32_t r) { return (r >> 2) & 3u; }

// Offset in halves of element (row, col) of a tiled [R, K] matrix.
__host__ __device__ __forceinline__ size_t tile_offset(uint32_t row, uint32_t col, uint32_t k) {
  const uint32_t slab = row >> 8, chunk = (row >> 4) & 15u, r = row & 15u;
  const uint32_t step = col >> 5, unit = (col >> 3) & 3u, half = col & 7u;
  const uint32_t place = unit ^ tile_swizzle(r);
  return (((size_t)slab * (k >> 5) + step) * 16u + chunk) * 512u + (4u * r + place) * 8u + half;
}

}  // namespace fk
