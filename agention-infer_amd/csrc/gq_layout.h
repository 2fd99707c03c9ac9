// gq_layout.h -- the device-resident ("wave-tiled") weight layout.
//
// A weight matrix of R rows x K columns is cut into 256-element units
// (one super-block; for Q8_0 eight 32-element blocks).  Each unit's bytes
// ("logical unit bytes", below) are split into C chunks of 16 B.  Rows are
// grouped into tiles of RT rows; the RT*U units of a tile (U units per
// row, row-major) are dealt to the 64 lanes of one wave: unit j of the tile
// goes to lane j % 64 in iteration j / 64.  Memory holds, per tile and per
// iteration, chunk 0 of the 64 lanes' units (1 KiB), then chunk 1, ... so a
// wave-wide 128-bit load of chunk c reads 1 KiB of contiguous HBM.  The
// last iteration of a tile holds only its nv valid lanes, packed (nv*16 B
// per chunk), so the layout has no padding: its size is the ggml size
// (except a ragged Q8_0 row, padded with zero blocks to a whole unit).
//
// Logical unit bytes per format (all in ggml's order within a block):
//   Q4_K    the 144 B block                              C = 9
//   Q5_K    the 176 B block                              C = 11
//   Q6_K    bytes 0..207 (ql, qh, scales); d separately    C = 13
//   IQ3_XXS bytes 2..97 (qs, signs/scales); d separately   C = 6
//   Q8_0    qs of blocks 0..7 (8 x 32 B), then their 8 f16 d  C = 17
// "d separately": one f16 per unit at index (tile * RT * U + j).
//
// Quad layout (quad = 1; dense Q4_K / Q5_K / Q6_K / Q8_0 matrices, for the
// MFMA matvec): rows in groups of 16 (the last group has nr = R % 16 rows
// if that is not 0), units in quads of 4 (the last quad of a row has
// nq = U % 4 units if that is not 0).  An item is (row group g, quad t):
// its nv = nr * nq units sit in lanes nr * q + r (row 16g + r, unit
// 4t + q), and memory holds chunk 0 of the item's nv units (16 B each),
// then chunk 1, ...; items follow each other row group by row group, quad
// by quad.  A full item is one wave-wide 1 KiB load per chunk.  No padding;
// the d array (Q6_K) holds the units in the same item / lane order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gq {

struct Layout {
  int dtype;
  int rows;    // R
  int k;       // in_dim
  int units;   // U, units per row
  int chunks;  // C
  int rt;      // rows per tile: all rows (one tile) for matvec weights; a
               // power of two <= 64 dividing the rows per expert for stacked
               // expert tensors
  int quad;    // 1: the quad layout (row groups of 16 over all rows; with
               // stacked experts rt is a multiple of 16, so expert e's
               // matrix is a quad matrix of its own starting at unit e rt U)
};

constexpr int QROWS = 16;  // rows per row group of the quad layout

// Quad layout: first unit index (in the item / lane order of the body and
// d array) of item (g, t), its row count nr and unit count nq.
__host__ __device__ inline long quad_item_unit(const Layout &L, int g, int t, int &nr, int &nq) {
  nr = min(QROWS, L.rows - QROWS * g);
  nq = min(4, L.units - 4 * t);
  return (long)g * QROWS * L.units + (long)t * 4 * nr;
}

__host__ __device__ constexpr int unit_chunks(int t) {
  return t == 12 ? 9 : t == 13 ? 11 : t == 14 ? 13 : t == 18 ? 6 : t == 8 ? 17 : 0;
}

// Byte offset of chunk c of unit j (0 <= j < units in tile) of tile t.
__host__ __device__ inline long chunk_offset(const Layout &L, int t, int j, int c) {
  if (L.quad) {  // j = row * U + unit within tile t
    const int row = t * L.rt + j / L.units, u = j % L.units;
    int nr, nq;
    const long base = quad_item_unit(L, row / QROWS, u >> 2, nr, nq);
    return (base * L.chunks + (long)c * nr * nq + (long)nr * (u & 3) + row % QROWS) * 16;
  }
  const long tile_units = (long)L.rt * L.units;
  const int rows_here = min(L.rt, L.rows - t * L.rt);
  const int uit = rows_here * L.units;  // units in this tile
  const int iters = (uit + 63) >> 6;
  const int it = j >> 6, l = j & 63;
  const long base = (long)t * tile_units * L.chunks * 16;
  if (it < iters - 1) return base + ((long)it * L.chunks + c) * 1024 + 16 * l;
  const int nv = uit - 64 * (iters - 1);
  return base + (long)(iters - 1) * L.chunks * 1024 + (long)c * 16 * nv + 16 * l;
}

__host__ __device__ inline long unit_index(const Layout &L, int t, int j) {
  if (L.quad) {
    const int row = t * L.rt + j / L.units, u = j % L.units;
    int nr, nq;
    return quad_item_unit(L, row / QROWS, u >> 2, nr, nq) + (long)nr * (u & 3) + row % QROWS;
  }
  return (long)t * L.rt * L.units + j;
}

__host__ __device__ inline int num_tiles(const Layout &L) { return (L.rows + L.rt - 1) / L.rt; }

__host__ __device__ inline long body_bytes(const Layout &L) {
  return (long)L.rows * L.units * L.chunks * 16;
}

}  // namespace gq
