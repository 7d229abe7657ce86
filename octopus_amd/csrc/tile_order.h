// The GEMMs' workgroup -> tile order, as constexpr functions of plain integers: hipcc compiles them for the GPU
// (constexpr functions are callable from device code), and g++ for the CPU check of the order
// (tests/plan_check.cpp, under -fsanitize=address,undefined).
//
// Block -> (mt, nt). Blocks run on XCD b % 8. The first 8 * floor(M-tiles / 8) M-tiles are dealt to the XCDs
// round-robin (XCD x owns mt = x, x + 8, ...), and each XCD walks its own in groups of group_m across all N-tiles, so
// the ~32 workgroups resident on an XCD run 4 M-tiles x 8 N-tiles and share A and B K-slices in its L2, while the 8
// XCDs sweep the N-tiles in step (at 114,688 hidden rows, 0.59 GB, more than the 256 MB Infinity Cache, XCDs out of
// step made the forward 6% slower). The tiles of the last M-tiles % 8 M-tiles are cut into 8 contiguous segments of
// equal length (+-1), one per XCD, so every XCD holds the same number of tiles whatever the shape (whole M-tile rows
// for those too gave an XCD with one more row a whole extra round: 99 M-tiles x 10 N-tiles ran 5 rounds of 32 tiles on
// three XCDs against 4 on the others). Per XCD that is floor(M / 8) N + ceil((M % 8) N / 8) = ceil(M N / 8) tiles.
// A device-side row count that bounds M or N shrinks the tile grid (read once per block), so the idle blocks all come
// after the working ones instead of between them: interleaved idle blocks retire instantly and stagger the working
// workgroups at every group start, which breaks their L2 sharing. The grid is 8 * ceil(bound-free tiles / 8); blocks
// past their XCD's tiles return false.
#pragma once

#include <stdint.h>

namespace octo_tiles {

// Workgroups of the one-shot grid of mtiles x ntiles tiles: 8 ceil(tiles / 8).
constexpr int64_t tile_grid(int64_t mtiles, int64_t ntiles) { return 8 * ((mtiles * ntiles + 7) / 8); }

// Tiles XCD x holds in the order below.
constexpr int64_t xcd_tiles(int x, int64_t mtiles, int64_t ntiles) {
  const int64_t T = (mtiles % 8) * ntiles;
  return (mtiles / 8) * ntiles + (x + 1) * T / 8 - x * T / 8;
}

// XCD x's k-th tile (mt, nt) of an mtiles x ntiles grid walked in groups of group_m M-tiles; false past its tiles.
constexpr bool tile_at(int group_m, int x, int64_t k, int64_t mtiles, int64_t ntiles, int &mt, int &nt) {
  const int64_t mfull = mtiles / 8;  // M-tiles every XCD owns: x, x + 8, ..., x + 8 (mfull - 1)
  const int64_t main = mfull * ntiles;
  if (k < main) {
    const int64_t span = (int64_t)group_m * ntiles;
    const int64_t gid = k / span;
    const int64_t first = gid * group_m;
    const int64_t gsize = (mfull - first) < group_m ? (mfull - first) : group_m;
    const int64_t local = k - gid * span;
    mt = (int)(x + 8 * (first + local % gsize));
    nt = (int)(local / gsize);
    return true;
  }
  const int64_t r = mtiles - 8 * mfull, T = r * ntiles;  // the last r M-tiles, M fastest, cut into 8 segments
  const int64_t L = x * T / 8 + (k - main);
  if (L >= (x + 1) * T / 8) return false;
  mt = (int)(8 * mfull + L % r);
  nt = (int)(L / r);
  return true;
}

}  // namespace octo_tiles
