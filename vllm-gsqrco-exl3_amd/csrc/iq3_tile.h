// The build's IQ3_S tile layout (its own; the reference's iq3_pack.py layout serves its CUDA
// mma fragments and is not reproduced).
//
// Rows are grouped in tiles of 16. Tile t's bytes stay where rows 16t..16t+15 were; block b of
// the tile becomes one 1760-byte "tile-block" at byte 1760*b of the tile. Inside a tile-block,
// lane L = 8p + s of the decode GEMV (p = row pair 0..7, s = slice 0..7) finds its data as
//   [   0, 1024)  16 B at 16L : qs[8s..8s+8) of row 2p, then of row 2p+1
//   [1024, 1536)   8 B at 8L  : signs[4s..4s+4) of row 2p, then of row 2p+1
//   [1536, 1664)   2 B at 2L  : qh[s] of row 2p, then of row 2p+1
//   [1664, 1728)   2 B at 2(4p + j) : scales[j] of row 2p, then of row 2p+1 (j = 0..3)
//   [1728, 1760)   4 B at 4p  : d of row 2p, then of row 2p+1
// (block_iq3_s byte offsets: d 0, qs 2, qh 66, signs 74, scales 106.) A pure byte permutation:
// bijective, same size, each load of the GEMV 16-byte aligned and contiguous across lanes.
#pragma once

#include "gguf_common.h"

namespace gguf {

constexpr int kTileRows = 16;
constexpr int kTileBlockBytes = kTileRows * 110;  // 1760
constexpr int kTqs = 0, kTsg = 1024, kTqh = 1536, kTsc = 1664, kTd = 1728;

// tile-block byte j -> (row within the tile, byte within that row's block)
__host__ __device__ inline void iq3_tile_source(int j, int& r, int& o) {
  if (j < kTsg) {
    const int L = j >> 4, i = j & 15;
    r = 2 * (L >> 3) + (i >> 3);
    o = 2 + 8 * (L & 7) + (i & 7);
  } else if (j < kTqh) {
    const int jj = j - kTsg, L = jj >> 3, i = jj & 7;
    r = 2 * (L >> 3) + (i >> 2);
    o = 74 + 4 * (L & 7) + (i & 3);
  } else if (j < kTsc) {
    const int jj = j - kTqh, L = jj >> 1;
    r = 2 * (L >> 3) + (jj & 1);
    o = 66 + (L & 7);
  } else if (j < kTd) {
    const int jj = j - kTsc, m = jj >> 1;
    r = 2 * (m >> 2) + (jj & 1);
    o = 106 + (m & 3);
  } else {
    const int jj = j - kTd;
    r = 2 * (jj >> 2) + ((jj >> 1) & 1);
    o = jj & 1;
  }
}

// Decode of values 8q..8q+7 (groups 2q, 2q+1) of slice u of row li (0..15) from a tile-block,
// for the MFMA kernel's lane mapping.
__device__ __forceinline__ void decode_iq3s_tile_q(const uint8_t* t, int li, int u, int q, const uint32_t* grid,
                                                   int (&w)[2], float& d, int& ls) {
  const int L = 8 * (li >> 1) + u, ri = li & 1;
  const uint32_t qs = *(const uint16_t*)(t + kTqs + 16 * L + 8 * ri + 2 * q);
  const uint32_t qh = t[kTqh + 2 * L + ri] >> (2 * q);
  const uint32_t sg = t[kTsg + 8 * L + 4 * ri + q];
  w[0] = apply_signs(grid[(qs & 0xFF) | ((qh & 1u) << 8)], sg);
  w[1] = apply_signs(grid[(qs >> 8) | ((qh & 2u) << 7)], sg >> 4);
  d = half_bits_to_float(*(const uint16_t*)(t + kTd + 4 * (li >> 1) + 2 * ri));
  ls = 1 + 2 * ((t[kTsc + 2 * (4 * (li >> 1) + (u >> 1)) + ri] >> (4 * (u & 1))) & 0xF);
}

}  // namespace gguf
