// In-place conversion between GGUF IQ3_S rows and the build's tile layout (iq3_tile.h), the
// load-time repack behind GGUFLinearMethod._pack_iq3 (reference: quantization/iq3_pack.py
// pack_ / unpack, linear.py:437-457). Whole 16-row tiles are copied to scratch in chunks and
// converted back; per tile-block, 64 threads handle the lanes' QS / E8 / L2 bytes and 96 threads
// the scale and d bytes.
#include "iq3_tile.h"

namespace gguf {

constexpr size_t kPackChunkCap = (size_t)64 << 20;
constexpr int kSlotsPerTileBlock = 64 + (kTileBlockBytes - kTsc);  // 160

size_t iq3_pack_scratch_bytes(int64_t rows, int64_t row_bytes) {
  const size_t tile = (size_t)kTileRows * (size_t)row_bytes;
  const size_t total = (size_t)rows * (size_t)row_bytes;
  const size_t cap = total < kPackChunkCap ? total : kPackChunkCap;
  return cap < tile ? tile : cap / tile * tile;
}

__global__ void iq3_tile_convert_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t row_bytes,
                                        int64_t ntileblocks, int nb, bool unpack) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ntileblocks * kSlotsPerTileBlock) return;
  const int64_t tbi = i / kSlotsPerTileBlock;
  const int slot = (int)(i - tbi * kSlotsPerTileBlock);
  const int64_t t = tbi / nb;
  const int b = (int)(tbi - t * nb);
  const int64_t tile_off = t * kTileRows * row_bytes;
  const uint8_t* g_src = src + tile_off + (int64_t)b * 110;       // GGUF row 0 of the tile, block b
  uint8_t* g_dst = dst + tile_off + (int64_t)b * 110;
  const int64_t tb_off = tile_off + (int64_t)b * kTileBlockBytes;  // tile-block b
  if (slot < 64) {
    const int p = slot >> 3;
    if (!unpack) {
      const uint8_t* rows[2] = {g_src + (2 * p) * row_bytes, g_src + (2 * p + 1) * row_bytes};
      iq3_tile_pack_lane(rows, slot, dst + tb_off);
    } else {
      uint8_t* rows[2] = {g_dst + (2 * p) * row_bytes, g_dst + (2 * p + 1) * row_bytes};
      iq3_tile_unpack_lane(src + tb_off, slot, rows);
    }
  } else {
    const int j = kTsc + (slot - 64);
    int r, o;
    iq3_tile_scale_source(j, r, o);
    if (!unpack) {
      dst[tb_off + j] = g_src[r * row_bytes + o];
    } else {
      g_dst[r * row_bytes + o] = src[tb_off + j];
    }
  }
}

hipError_t launch_iq3_pack(uint8_t* w, int64_t rows, int64_t row_bytes, bool unpack, uint8_t* scratch,
                           size_t scratch_bytes, hipStream_t stream) {
  const int64_t tile_bytes = (int64_t)kTileRows * row_bytes;
  const int64_t tiles_per_chunk = (int64_t)(scratch_bytes / (size_t)tile_bytes);
  const int64_t ntiles = rows / kTileRows;
  const int nb = (int)(row_bytes / 110);
  for (int64_t t0 = 0; t0 < ntiles; t0 += tiles_per_chunk) {
    const int64_t nt = ntiles - t0 < tiles_per_chunk ? ntiles - t0 : tiles_per_chunk;
    uint8_t* chunk = w + t0 * tile_bytes;
    hipError_t e = hipMemcpyAsync(scratch, chunk, (size_t)(nt * tile_bytes), hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return e;
    const int64_t threads = nt * nb * kSlotsPerTileBlock;
    iq3_tile_convert_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(scratch, chunk, row_bytes, nt * nb,
                                                                                   nb, unpack);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace gguf
