// In-place conversion between GGUF IQ3_S / IQ3_XXS rows and the build's unit layouts (iq3_tile.h), the
// load-time repack behind GGUFLinearMethod._pack_iq3 (reference: quantization/iq3_pack.py
// pack_ / unpack, linear.py:437-457). Whole 4-row units are copied to scratch in chunks and
// converted back. IQ3_S: per unit-block of r K blocks, 16 r threads handle the lanes' QS / E8 / L2
// bytes and 24 r threads the scale and d bytes; IQ3_XXS (a plain byte permutation): one thread per
// byte.
#include "iq3_tile.h"

namespace gguf {

constexpr size_t kPackChunkCap = (size_t)64 << 20;
constexpr int kSlotsPerUnitBlock = 40 * 4;  // 16 r lane slots + 24 r scale / d bytes, r = 4

size_t iq3_pack_scratch_bytes(int64_t rows, int64_t row_bytes) {
  const size_t tile = (size_t)kTileRows * (size_t)row_bytes;
  const size_t total = (size_t)rows * (size_t)row_bytes;
  const size_t cap = total < kPackChunkCap ? total : kPackChunkCap;
  return cap < tile ? tile : cap / tile * tile;
}

__global__ void iq3_unit_convert_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t row_bytes,
                                        int64_t nunits, int nb, bool unpack) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_unit = 40 * nb;  // sum of 40 r over the unit-blocks
  if (i >= nunits * per_unit) return;
  const int64_t u = i / per_unit;
  const int slot = (int)(i - u * per_unit);
  const int kb = slot / kSlotsPerUnitBlock, rem = slot - kb * kSlotsPerUnitBlock;
  const int r = iq3_unit_blocks(nb, kb);
  const int64_t ubase = u * kUnitRows * row_bytes;                  // the unit's first byte, either layout
  const int64_t ub = ubase + (int64_t)kb * kUnitBlockBytes;         // unit-block kb
  if (rem < 16 * r) {
    const int L = rem, bi = L >> 4, rp = (L >> 3) & 1, s = L & 7;
    const int64_t blk = ubase + (int64_t)(4 * kb + bi) * 110;        // GGUF row 0 of the unit, block 4kb + bi
    if (!unpack) {
      const uint8_t* rows[2] = {src + blk + (2 * rp) * row_bytes, src + blk + (2 * rp + 1) * row_bytes};
      iq3_tile_pack_lane(rows, s, dst + ub + 16 * L, dst + ub + iq3_e8_base(r) + 8 * L, dst + ub + iq3_l2_base(r) + 2 * L);
    } else {
      uint8_t* rows[2] = {dst + blk + (2 * rp) * row_bytes, dst + blk + (2 * rp + 1) * row_bytes};
      iq3_tile_unpack_lane(src + ub + 16 * L, src + ub + iq3_e8_base(r) + 8 * L, src + ub + iq3_l2_base(r) + 2 * L, s,
                           rows);
    }
  } else {
    const int j = (int)iq3_sc_base(r) + (rem - 16 * r);
    int row, bi, o;
    iq3_tile_scale_source(j, r, row, bi, o);
    const int64_t g = ubase + row * row_bytes + (int64_t)(4 * kb + bi) * 110 + o;
    if (!unpack) dst[ub + j] = src[g];
    else dst[g] = src[ub + j];
  }
}

// IQ3_XXS: one thread per byte of the unit layout (xxs_unit_source names its GGUF byte); unpack
// writes each GGUF byte back from its place in the unit layout.
__global__ void iq3xxs_unit_convert_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                           int64_t row_bytes, int64_t nunits, int nb, bool unpack) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t unit_bytes = kUnitRows * row_bytes;
  if (i >= nunits * unit_bytes) return;
  const int64_t u = i / unit_bytes;
  const int jb = (int)(i - u * unit_bytes);  // byte of the unit (layout side)
  const int kb = jb / kXxsUnitBlockBytes, j = jb - kb * kXxsUnitBlockBytes;
  int row, bi, o;
  xxs_unit_source(j, iq3_unit_blocks(nb, kb), row, bi, o);
  const int64_t g = u * unit_bytes + row * row_bytes + (int64_t)(4 * kb + bi) * 98 + o;
  if (!unpack) dst[i] = src[g];
  else dst[g] = src[i];
}

hipError_t launch_iq3_pack(int type, uint8_t* w, int64_t rows, int64_t row_bytes, bool unpack, uint8_t* scratch,
                           size_t scratch_bytes, hipStream_t stream) {
  const int64_t unit_bytes = (int64_t)kUnitRows * row_bytes;
  const int64_t units_per_chunk = (int64_t)(scratch_bytes / (size_t)unit_bytes);
  const int64_t nunits = rows / kUnitRows;
  const bool xxs = type == kIQ3_XXS;
  const int nb = (int)(row_bytes / (xxs ? 98 : 110));
  for (int64_t u0 = 0; u0 < nunits; u0 += units_per_chunk) {
    const int64_t nu = nunits - u0 < units_per_chunk ? nunits - u0 : units_per_chunk;
    uint8_t* chunk = w + u0 * unit_bytes;
    hipError_t e = hipMemcpyAsync(scratch, chunk, (size_t)(nu * unit_bytes), hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return e;
    if (xxs) {
      const int64_t threads = nu * unit_bytes;
      iq3xxs_unit_convert_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(scratch, chunk, row_bytes, nu,
                                                                                        nb, unpack);
    } else {
      const int64_t threads = nu * 40 * nb;
      iq3_unit_convert_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(scratch, chunk, row_bytes, nu,
                                                                                     nb, unpack);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace gguf
