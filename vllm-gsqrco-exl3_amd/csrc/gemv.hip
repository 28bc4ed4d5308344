// Decode GEMV for 1..8 activation rows on GGUF bytes: Y[c, r] = sum_k X[c, k] * W[r, k].
//
// Replaces the reference's 1..8-row products (vendored MMVQ mul_mat_vec_q, mmvq.cu:600-760; the
// owned dp4a kernels lcpp_shim.cu:498-607 and lcpp_owned_k4.cu:116-269) with one wave64 design:
//  * a workgroup of 4 waves owns 4*RW weight rows; lane l of a wave takes the 32-value slices
//    l, l+64, ... of the K axis, so one q8_1 block of X per lane per step is loaded once and
//    reused for the wave's RW rows;
//  * each lane decodes its slice of each row into 8 int8x4 words (decode.h) and multiplies with
//    v_dot4_i32_i8 (__builtin_amdgcn_sdot4); the integer slice dot is scaled in fp32 and added to
//    a per-lane accumulator;
//  * a 64-lane xor butterfly sums each (row, column) accumulator at the end.
// The integer slice sums equal the reference's vec_dot sumi bit for bit; only the fp32 order in
// which a row's slice terms are added differs (lane-strided, then the butterfly).
#include "decode.h"
#include "iq3_tile.h"

namespace gguf {

constexpr int kGemvWaves = 4;

template <int TYPE, int NC, int RW>
__global__ void __launch_bounds__(256) gemv_raw_kernel(const uint8_t* __restrict__ W, int64_t row_bytes, int nrows,
                                                       int k, const uint8_t* __restrict__ q8, void* __restrict__ y,
                                                       int y_dtype) {
  __shared__ uint32_t grid[TYPE == kIQ3_S ? 512 : 1];
  if constexpr (TYPE == kIQ3_S) {
    for (int i = threadIdx.x; i < 512; i += blockDim.x) grid[i] = kIq3sGrid.v[i];
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * RW;
  if (row0 >= nrows) return;
  constexpr int BS = block_bytes(TYPE);
  const int nslices = k / kQ81;

  float acc[RW][NC];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;

  for (int s = lane; s < nslices; s += 64) {
    int xq[NC][8];
    float d8[NC];
    int sq[NC];  // Q4_K: sum of the slice's q8 values (the min term's integer part)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint8_t* xb = q8 + ((int64_t)c * nslices + s) * 36;
      d8[c] = half_bits_to_float(*(const uint16_t*)xb);
      const u32x4 a = ld128a4(xb + 4);
      const u32x4 b = ld128a4(xb + 20);
      xq[c][0] = (int)a.x; xq[c][1] = (int)a.y; xq[c][2] = (int)a.z; xq[c][3] = (int)a.w;
      xq[c][4] = (int)b.x; xq[c][5] = (int)b.y; xq[c][6] = (int)b.z; xq[c][7] = (int)b.w;
      if constexpr (TYPE == kQ4_K) {
        int t = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) t = dot4(0x01010101, xq[c][e], t);
        sq[c] = t;
      }
    }
    const int blk = s >> 3, u = s & 7;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int row = row0 + r;
      if (row >= nrows) break;
      const uint8_t* b = W + (int64_t)row * row_bytes + (int64_t)blk * BS;
      int w[8];
      SliceScale sc;
      if constexpr (TYPE == kIQ3_S) decode_iq3s(b, u, grid, w, sc);
      if constexpr (TYPE == kQ4_K) decode_q4k(b, u, w, sc);
      if constexpr (TYPE == kIQ4_XS) decode_iq4xs(b, u, w, sc);
      if constexpr (TYPE == kQ6_K) decode_q6k(b, u, w, sc);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if constexpr (TYPE == kQ6_K) {
          int sa = 0, sb = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) sa = dot4(w[e], xq[c][e], sa);
#pragma unroll
          for (int e = 4; e < 8; ++e) sb = dot4(w[e], xq[c][e], sb);
          const int sumi = sa * sc.ls + sb * sc.ls2;
          acc[r][c] += (float)sumi * (sc.d * d8[c]);
        } else {
          int sumi = 0;
#pragma unroll
          for (int e = 0; e < 8; ++e) sumi = dot4(w[e], xq[c][e], sumi);
          if constexpr (TYPE == kQ4_K) {
            const float t = (sc.d * (float)sc.ls) * (float)sumi - (sc.dmin * (float)sc.ls2) * (float)sq[c];
            acc[r][c] += t * d8[c];
          } else {
            acc[r][c] += (float)(sumi * sc.ls) * (sc.d * d8[c]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float v = acc[r][c];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      acc[r][c] = v;
    }
  }
  // lane (r * NC + c) writes output (c, row0 + r)
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (lane == r * NC + c && row0 + r < nrows) store_y(y, (int64_t)c * nrows + row0 + r, acc[r][c], y_dtype);
}

template <int TYPE, int NC>
static void launch_nc(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, void* y, int y_dtype,
                      hipStream_t stream) {
  constexpr int RW = NC <= 4 ? 4 : 2;
  const unsigned blocks = (unsigned)((nrows + kGemvWaves * RW - 1) / (kGemvWaves * RW));
  gemv_raw_kernel<TYPE, NC, RW><<<blocks, 64 * kGemvWaves, 0, stream>>>(W, row_bytes, nrows, k, q8, y, y_dtype);
}

template <int TYPE>
static void launch_type(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n, void* y,
                        int y_dtype, hipStream_t stream) {
  switch (n) {
    case 1: launch_nc<TYPE, 1>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 2: launch_nc<TYPE, 2>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 3: launch_nc<TYPE, 3>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 4: launch_nc<TYPE, 4>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 5: launch_nc<TYPE, 5>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 6: launch_nc<TYPE, 6>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 7: launch_nc<TYPE, 7>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    default: launch_nc<TYPE, 8>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
  }
}

// n in 1..8 activation rows; q8: block_q8_1 of X; y: [n, nrows] in y_dtype.
hipError_t launch_gemv_raw(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                           void* y, int y_dtype, hipStream_t stream) {
  switch (type) {
    case kIQ3_S: launch_type<kIQ3_S>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ4_K: launch_type<kQ4_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ4_XS: launch_type<kIQ4_XS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ6_K: launch_type<kQ6_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}


// ---------------------------------------------------------------------------------------------
// IQ3_S in the tile layout (iq3_tile.h): a workgroup owns one 16-row tile, its 4 waves split the
// K blocks, and lane L = 8p + s of a wave decodes slice s of rows 2p, 2p+1 of each block it
// visits, from one 16-byte, one 8-byte and three small loads, all contiguous across the wave.
// The q8_1 block of X for the slice is loaded once per lane and used for both rows. Partial sums
// are added over the 8 slice lanes (xor butterfly) and then over the 4 waves in wave order.
template <int NC>
__global__ void __launch_bounds__(256) gemv_iq3s_tile_kernel(const uint8_t* __restrict__ W, int64_t row_bytes,
                                                             int nrows, int k, const uint8_t* __restrict__ q8,
                                                             void* __restrict__ y, int y_dtype) {
  __shared__ uint32_t grid[512];
  __shared__ float red[kGemvWaves][NC][kTileRows];
  for (int i = threadIdx.x; i < 512; i += blockDim.x) grid[i] = kIq3sGrid.v[i];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int p = lane >> 3, s = lane & 7;
  const int nb = k / kQK;
  const int nslices = k / kQ81;
  const int b_begin = wave * nb / kGemvWaves, b_end = (wave + 1) * nb / kGemvWaves;
  const uint8_t* tb = W + (int64_t)blockIdx.x * kTileRows * row_bytes;

  float acc[2][NC];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[i][c] = 0.0f;

  for (int b = b_begin; b < b_end; ++b) {
    const uint8_t* t = tb + (int64_t)b * kTileBlockBytes;
    const uint4 qs = *(const uint4*)(t + kTqs + 16 * lane);
    const uint2 sg = *(const uint2*)(t + kTsg + 8 * lane);
    const uint32_t qh = *(const uint16_t*)(t + kTqh + 2 * lane);
    const uint32_t sc = *(const uint16_t*)(t + kTsc + 2 * (4 * p + (s >> 1)));
    const uint32_t dd = *(const uint32_t*)(t + kTd + 4 * p);

    int xq[NC][8];
    float d8[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint8_t* xb = q8 + ((int64_t)c * nslices + b * 8 + s) * 36;
      d8[c] = half_bits_to_float(*(const uint16_t*)xb);
      const u32x4 a = ld128a4(xb + 4);
      const u32x4 e = ld128a4(xb + 20);
      xq[c][0] = (int)a.x; xq[c][1] = (int)a.y; xq[c][2] = (int)a.z; xq[c][3] = (int)a.w;
      xq[c][4] = (int)e.x; xq[c][5] = (int)e.y; xq[c][6] = (int)e.z; xq[c][7] = (int)e.w;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint64_t q = i == 0 ? ((uint64_t)qs.y << 32 | qs.x) : ((uint64_t)qs.w << 32 | qs.z);
      const uint32_t sgn = i == 0 ? sg.x : sg.y;
      const uint32_t h = (qh >> (8 * i)) & 0xFF;
      int w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t idx = (uint32_t)((q >> (8 * e)) & 0xFF) | (((h >> e) & 1u) << 8);
        w[e] = apply_signs(grid[idx], sgn >> (4 * e));
      }
      const int ls = 1 + 2 * (((sc >> (8 * i)) >> (4 * (s & 1))) & 0xF);
      const float dw = half_bits_to_float((dd >> (16 * i)) & 0xFFFF);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        int sumi = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) sumi = dot4(w[e], xq[c][e], sumi);
        acc[i][c] += (float)(sumi * ls) * (dw * d8[c]);
      }
    }
  }

#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float v = acc[i][c];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      if (s == 0) red[wave][c][2 * p + i] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < NC * kTileRows) {
    const int c = threadIdx.x / kTileRows, r = threadIdx.x % kTileRows;
    float v = red[0][c][r];
#pragma unroll
    for (int wv = 1; wv < kGemvWaves; ++wv) v += red[wv][c][r];
    store_y(y, (int64_t)c * nrows + (int64_t)blockIdx.x * kTileRows + r, v, y_dtype);
  }
}

// nrows % 16 == 0, n in 1..8
hipError_t launch_gemv_packed(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                              void* y, int y_dtype, hipStream_t stream) {
  const unsigned blocks = (unsigned)(nrows / kTileRows);
#define GGUF_GT(NC) gemv_iq3s_tile_kernel<NC><<<blocks, 64 * kGemvWaves, 0, stream>>>(W, row_bytes, nrows, k, q8, y, y_dtype)
  switch (n) {
    case 1: GGUF_GT(1); break;
    case 2: GGUF_GT(2); break;
    case 3: GGUF_GT(3); break;
    case 4: GGUF_GT(4); break;
    case 5: GGUF_GT(5); break;
    case 6: GGUF_GT(6); break;
    case 7: GGUF_GT(7); break;
    default: GGUF_GT(8); break;
  }
#undef GGUF_GT
  return hipGetLastError();
}

}  // namespace gguf
