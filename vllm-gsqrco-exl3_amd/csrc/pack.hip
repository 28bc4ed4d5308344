// In-place conversion between GGUF IQ3_S rows and the build's tile layout (iq3_tile.h), the
// load-time repack behind GGUFLinearMethod._pack_iq3 (reference: quantization/iq3_pack.py
// pack_ / unpack, linear.py:437-457). Whole 16-row tiles are copied to scratch in chunks and
// gathered back permuted, one thread per byte.
#include "iq3_tile.h"

namespace gguf {

constexpr size_t kPackChunkCap = (size_t)64 << 20;

size_t iq3_pack_scratch_bytes(int64_t rows, int64_t row_bytes) {
  const size_t tile = (size_t)kTileRows * (size_t)row_bytes;
  const size_t total = (size_t)rows * (size_t)row_bytes;
  const size_t cap = total < kPackChunkCap ? total : kPackChunkCap;
  return cap < tile ? tile : cap / tile * tile;
}

// src/dst: whole tiles (ntiles x 16 rows x row_bytes). pack: dst tile-blocks <- src GGUF rows.
__global__ void iq3_tile_permute_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t row_bytes,
                                        int64_t total, bool unpack) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t tile_bytes = (int64_t)kTileRows * row_bytes;
  const int64_t t = i / tile_bytes;
  const int64_t rem = i - t * tile_bytes;
  const int64_t b = rem / kTileBlockBytes;
  const int j = (int)(rem - b * kTileBlockBytes);
  int r, o;
  iq3_tile_source(j, r, o);
  const int64_t g = t * tile_bytes + (int64_t)r * row_bytes + b * 110 + o;  // GGUF position
  if (unpack) {
    dst[g] = src[i];
  } else {
    dst[i] = src[g];
  }
}

hipError_t launch_iq3_pack(uint8_t* w, int64_t rows, int64_t row_bytes, bool unpack, uint8_t* scratch,
                           size_t scratch_bytes, hipStream_t stream) {
  const int64_t tile_bytes = (int64_t)kTileRows * row_bytes;
  const int64_t tiles_per_chunk = (int64_t)(scratch_bytes / (size_t)tile_bytes);
  const int64_t ntiles = rows / kTileRows;
  for (int64_t t0 = 0; t0 < ntiles; t0 += tiles_per_chunk) {
    const int64_t nt = ntiles - t0 < tiles_per_chunk ? ntiles - t0 : tiles_per_chunk;
    const int64_t bytes = nt * tile_bytes;
    uint8_t* chunk = w + t0 * tile_bytes;
    hipError_t e = hipMemcpyAsync(scratch, chunk, (size_t)bytes, hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return e;
    const unsigned blocks = (unsigned)((bytes + 255) / 256);
    iq3_tile_permute_kernel<<<blocks, 256, 0, stream>>>(scratch, chunk, row_bytes, bytes, unpack);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace gguf
