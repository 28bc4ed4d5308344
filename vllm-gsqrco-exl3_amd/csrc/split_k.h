// K split over workgroups for the int8 small GEMMs (gemm_raw_kernel, gemm_iq3s_tile_kernel) on
// grids of few 16-row tiles: each of the S workgroups of one (row tile, column group) sums its
// part of K, writes the sums to its own slot of the workspace and counts itself in; the one that
// brings the count to S adds the S slots in slot order and writes the output, so the result does
// not depend on which one finishes last.
//
// Workspace (after the xq copy of X): per (tile, column group) S slots of NT x 4 x 64 floats (NT
// column tiles, 4 values per lane, 64 lanes), then one uint32 counter per (tile, column group),
// which the quantise launch before the GEMM clears. The slots and counters are agent-scope
// atomics: written through to the device-coherent level and read from it. A device-scope fence
// would do the same by writing back and invalidating the whole L2 of the workgroup's XCD, which
// also drops every other workgroup's cached activations there.
#pragma once

#include "xq.h"

namespace gguf {

constexpr int kMaxSplit = 4;  // most workgroups one tile's K is split over

// Column tiles per workgroup of both GEMMs' plans (1..4), and the y extent of their grids.
inline int64_t split_nt(int64_t n) {
  const int64_t nct = xq_col_tiles(n);
  return nct < 4 ? nct : 4;
}
inline int64_t split_groups(int64_t tiles, int64_t n) { return tiles * ((xq_col_tiles(n) + split_nt(n) - 1) / split_nt(n)); }

// Slot bytes of a split over `split` workgroups (0 for no split); a multiple of 1 KiB.
inline size_t split_part_bytes(int split, int64_t tiles, int64_t n) {
  if (split <= 1 || n <= 0) return 0;
  return (size_t)(split_groups(tiles, n) * split * split_nt(n) * 4 * 64 * (int64_t)sizeof(float));
}
inline int split_counters(int split, int64_t tiles, int64_t n) {
  return split <= 1 || n <= 0 ? 0 : (int)split_groups(tiles, n);
}
// slots, then the counters padded to 256 B
inline size_t split_ws_bytes(int split, int64_t tiles, int64_t n) {
  if (split <= 1 || n <= 0) return 0;
  return split_part_bytes(split, tiles, n) + (((size_t)split_counters(split, tiles, n) * 4 + 255) & ~(size_t)255);
}

// Called by one wave (all 64 lanes) holding its workgroup's sums of slice z of S for (tile,
// column group) tg: publishes them and returns false, or, in the last workgroup to arrive,
// replaces them by the total over the S slots in slot order and returns true.
template <int NT>
__device__ __forceinline__ bool split_fixup(float (&sum)[NT][4], float* part, uint32_t* cnt, int S, int z, size_t tg,
                                            int lane) {
  constexpr int kSlot = NT * 4 * 64;
  float* slot = part + (tg * S + z) * kSlot;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v)
      __hip_atomic_store(slot + (t * 4 + v) * 64 + lane, sum[t][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the slot's stores are complete before the count
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(cnt + tg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __builtin_amdgcn_readfirstlane(prev);
  if (prev != (uint32_t)S - 1) return false;
  asm volatile("" ::: "memory");
  // all S x NT x 4 loads in flight at once, then the sums in slot order
  const float* first = part + tg * S * kSlot;
  float pv[kMaxSplit][NT][4];
#pragma unroll
  for (int zz = 0; zz < kMaxSplit; ++zz)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        pv[zz][t][v] = zz < S ? __hip_atomic_load(first + zz * kSlot + (t * 4 + v) * 64 + lane, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                              : 0.0f;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float tot = pv[0][t][v];
#pragma unroll
      for (int zz = 1; zz < kMaxSplit; ++zz)
        if (zz < S) tot += pv[zz][t][v];
      sum[t][v] = tot;
    }
  return true;
}

}  // namespace gguf
