// q8_1 activation quantisation on gfx950.
//
// Three output layouts; the first two are the reference's, bit-exact with its arithmetic:
//  * block_q8_1 (decode GEMV input), lcpp_shim.cu:274-294: per 32 values d = amax/127 (IEEE
//    division), q = amax == 0 ? 0 : roundf(x/d), sum by a 32-lane xor butterfly with offsets
//    16, 8, 4, 2, 1, stored as half2(d, sum) followed by 32 int8; block (row, k/32) row-major.
//  * block_q8_1_mmq (GEMM input), lcpp_shim.cu:298-355: per 32 values (64 for Q2_K) d_inv =
//    127/amax, q = roundf(x*d_inv), d = 1/d_inv; 144-byte blocks of 128 values, block index
//    (k/128)*n + row, 16 bytes of scales (4 x fp32 d; 4 x half2(d, sum) for Q4_K; for Q2_K
//    half d of each 64 values and half sums of the first six 16-value groups) then 128 int8.
//    An all-zero scale group stores q = 0, d = 0 (the reference's NaN -> 0 conversion).
//  * the xq layout of the MFMA GEMMs (xq.h): either arithmetic above, values placed as MFMA B
//    operands (and a converter from block_q8_1 bytes).
//
// Wave64 mapping: the MMVQ kernel gives each 32-lane half-wave one block (one value per lane);
// the MMQ kernel gives each lane 4 consecutive values, 8 lanes per 32-block.
#include <algorithm>

#include "gguf_common.h"
#include "xq.h"

namespace gguf {

// activation rows per launch of the xq / xh quantisers (grid y)
constexpr int kQuantRowsPerLaunch = 65520;

template <int DT>
__device__ __forceinline__ float ldx(const void* x, int64_t i) {
  if constexpr (DT == kF32) {
    return ((const float*)x)[i];
  } else if constexpr (DT == kF16) {
    return half_bits_to_float(((const uint16_t*)x)[i]);
  } else {
    return __uint_as_float((uint32_t)((const uint16_t*)x)[i] << 16);
  }
}

template <int DT>
__global__ void __launch_bounds__(256) quantize_q8_1_kernel(const void* __restrict__ x, uint8_t* __restrict__ y,
                                                            int64_t k, int64_t s01) {
  const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;  // column
  const int64_t row = blockIdx.y;
  if (i0 >= k) return;  // k % 512 == 0: whole 32-lane groups exit together
  const float xi = ldx<DT>(x, row * s01 + i0);
  float amax = fabsf(xi);
  float sum = xi;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    sum += __shfl_xor(sum, off, 32);
  }
  const float d = amax / 127.0f;
  const int q = amax == 0.0f ? 0 : (int)roundf(xi / d);
  const int64_t blk = (row * k + i0) / kQ81;
  const int iqs = (int)(i0 % kQ81);
  uint8_t* b = y + blk * 36;
  b[4 + iqs] = (uint8_t)(int8_t)q;
  if (iqs == 0) {
    const uint32_t dh = __half_as_ushort(__float2half_rn(d));
    const uint32_t sh = __half_as_ushort(__float2half_rn(sum));
    *(uint32_t*)b = dh | (sh << 16);
  }
}

// block_q8_1_mmq scale layouts (mmq.cuh:60-100): D4 (IQ types, Q6_K), DS4 (Q4_K), D2S6 (Q2_K)
constexpr int kD4 = 0, kDS4 = 1, kD2S6 = 2;

__host__ __device__ constexpr int mmq_layout(int type) { return type == kQ4_K ? kDS4 : type == kQ2_K ? kD2S6 : kD4; }

// One lane per 4 values. D4 / DS4: scale per 32 values (8 lanes); D2S6: d per 64 values (16
// lanes) and the sums of 16 values (4 lanes) for the first 96 of each 128.
template <int DT, int LAYOUT>
__global__ void __launch_bounds__(128) quantize_q8_1_mmq_kernel(const void* __restrict__ x, uint8_t* __restrict__ y,
                                                                int64_t k, int64_t s01, int n) {
  constexpr int kScaleLanes = LAYOUT == kD2S6 ? 16 : 8;
  constexpr int kSumLanes = LAYOUT == kD2S6 ? 4 : 8;
  const int64_t row = blockIdx.x;
  const int64_t i0 = ((int64_t)blockIdx.y * 128 + threadIdx.x) * 4;
  if (i0 >= k) return;  // k % 512 == 0: whole blocks exit together
  const int64_t base = row * s01 + i0;
  const float x0 = ldx<DT>(x, base), x1 = ldx<DT>(x, base + 1), x2 = ldx<DT>(x, base + 2),
              x3 = ldx<DT>(x, base + 3);
  float amax = fmaxf(fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fabsf(x2)), fabsf(x3));
  float sum = ((x0 + x1) + x2) + x3;
#pragma unroll
  for (int off = kScaleLanes / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kScaleLanes));
  if constexpr (LAYOUT != kD4) {
#pragma unroll
    for (int off = kSumLanes / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kSumLanes);
  }
  int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
  float d = 0.0f;
  if (amax != 0.0f) {
    const float d_inv = 127.0f / amax;
    q0 = (int)roundf(x0 * d_inv);
    q1 = (int)roundf(x1 * d_inv);
    q2 = (int)roundf(x2 * d_inv);
    q3 = (int)roundf(x3 * d_inv);
    d = 1.0f / d_inv;
  }
  const int64_t ib = (i0 / 128) * n + row;
  const int iqs = (int)(i0 % 128);
  uint8_t* b = y + ib * 144;
  *(uint32_t*)(b + 16 + iqs) = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) |
                               ((uint32_t)(q2 & 0xFF) << 16) | ((uint32_t)(q3 & 0xFF) << 24);
  if constexpr (LAYOUT == kD2S6) {
    // halves: [d of values 0..63, d of 64..127, sums of the 16-value groups 0..5]
    if (iqs % 16 == 0 && iqs < 96) {
      ((__half*)b)[2 + iqs / 16] = __float2half_rn(sum);
      if (iqs % 64 == 0) ((__half*)b)[iqs / 64] = __float2half_rn(d);
    }
  } else if (iqs % 32 == 0) {
    if constexpr (LAYOUT == kDS4) {
      const uint32_t dh = __half_as_ushort(__float2half_rn(d));
      const uint32_t sh = __half_as_ushort(__float2half_rn(sum));
      *(uint32_t*)(b + 4 * (iqs / 32)) = dh | (sh << 16);
    } else {
      *(float*)(b + 4 * (iqs / 32)) = d;
    }
  }
}

// The MFMA GEMMs' layout (xq.h). Thread i takes 8 consecutive values (one quarter of a slice) of
// padded activation row c = i / (k/8); the 4 quarters of a slice are 4 consecutive lanes. Rows
// c >= n (padding of the last column tile) write zeros. VEC selects the block_q8_1 arithmetic of
// the reference's decode ops (d = amax/127, q = roundf(x/d), d kept as fp16) instead of the MMQ
// arithmetic. DS4 (Q4_K weights) stores fp16 d in the low half of the scale word and, above it,
// the activation side of the min term: with VEC the slice's int16 sum of q (the decode ops' MMVQ
// form, vecdotq.cuh:525: d8 * sum(q8)), else the fp16 of the slice's sum of x, the half2 sum of
// block_q8_1_mmq's DS4 layout (the product ops' MMQ form, vecdotq.cuh:549-552).
template <bool VEC, bool DS4>
__device__ __forceinline__ void xq_store(uint8_t* y, int k, int c, int kk, int nct, uint32_t lo, uint32_t hi, float d,
                                         int qsum, float xsum) {
  const int nb = k / kQK;
  const int b = kk / kQK;
  const int u = (kk / kQ81) & 7, q = (kk / 8) & 3;
  const int t = c / kXqCols, j = c % kXqCols;
  const int64_t unit = (int64_t)t * nb + b;
  *(uint2*)(y + unit * kXqUnit + (16 * q + j) * 64 + 8 * u) = make_uint2(lo, hi);
  if (q == 0) {
    const uint32_t dh = __half_as_ushort(__float2half_rn(d));
    uint32_t word = VEC ? __float_as_uint(half_bits_to_float(dh)) : __float_as_uint(d);
    if constexpr (DS4)
      word = dh | (VEC ? (uint32_t)qsum << 16 : (uint32_t)__half_as_ushort(__float2half_rn(xsum)) << 16);
    *(uint32_t*)(y + xq_scale_base(nct, nb) + (unit * kXqCols + j) * 32 + 4 * u) = word;
  }
}

// The prefill GEMM's fp16 layout (xq.h, "xh"); same thread mapping and values as xq_store (MMQ
// arithmetic: for DS4 the min term's activation side is the fp16 sum of x, widened to fp32).
template <bool DS4>
__device__ __forceinline__ void xh_store(uint8_t* y, int k, int c, int kk, int nct, uint32_t lo, uint32_t hi, float d,
                                         float xsum) {
  const int nb = k / kQK;
  const int b = kk / kQK;
  const int u = (kk / kQ81) & 7, q = (kk / 8) & 3;
  const int t = c / kXqCols, j = c % kXqCols;
  const int64_t unit = (int64_t)t * nb + b;
  uint32_t h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t w = e < 2 ? lo : hi;
    const int sh = 16 * (e & 1);
    const float f0 = (float)(int8_t)((w >> sh) & 0xFF), f1 = (float)(int8_t)((w >> (sh + 8)) & 0xFF);
    h[e] = (uint32_t)__half_as_ushort(__float2half_rn(f0)) | ((uint32_t)__half_as_ushort(__float2half_rn(f1)) << 16);
  }
  *(uint4*)(y + unit * kXhUnit + 1024 * u + 16 * (16 * q + j)) = make_uint4(h[0], h[1], h[2], h[3]);
  if (q == 0) {
    uint8_t* sc = y + xh_scale_base(nct, nb) + unit * kXhScaleUnit + 32 * j + 4 * u;
    const float dd = DS4 ? half_bits_to_float(__half_as_ushort(__float2half_rn(d))) : d;
    *(float*)sc = dd;
    if constexpr (DS4) *(float*)(sc + 512) = half_bits_to_float(__half_as_ushort(__float2half_rn(xsum)));
  }
}

// Workgroup (0, 0) of a quantise launch clears `zero_words` dwords at `zero` (the split GEMM's
// counters, which the GEMM that follows in stream order reads; null: none).
__device__ __forceinline__ void clear_words(uint32_t* zero, int zero_words) {
  if (zero != nullptr && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = (int)threadIdx.x; i < zero_words; i += (int)blockDim.x) zero[i] = 0u;
}

// Thread (x, y) of the grid: values 8 x .. 8 x + 7 of activation row c0 + y (rows past n, the last
// column tile's padding, quantise zeros). k % 32 == 0, so a slice's four threads exit together.
template <int DT, bool VEC, bool DS4, bool XH = false>
__global__ void __launch_bounds__(256) quantize_xq_kernel(const void* __restrict__ x, uint8_t* __restrict__ y, int k,
                                                          int64_t s01, int n, int nct, int c0, uint32_t* zero,
                                                          int zero_words) {
  clear_words(zero, zero_words);
  const int kk = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 8;
  if (kk >= k) return;
  const int c = c0 + (int)blockIdx.y;
  float v[8];
  if (c < n) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = ldx<DT>(x, c * s01 + kk + e);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  uint32_t lo = 0, hi = 0;
  float d = 0.0f;
  int qsum = 0;
  if (VEC) d = amax / 127.0f;
  if (amax != 0.0f) {
    const float d_inv = 127.0f / amax;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int qe = VEC ? (int)roundf(v[e] / d) : (int)roundf(v[e] * d_inv);
      if (e < 4) lo |= ((uint32_t)qe & 0xFFu) << (8 * e);
      else hi |= ((uint32_t)qe & 0xFFu) << (8 * (e - 4));
      qsum += qe;
    }
    if (!VEC) d = 1.0f / d_inv;
  }
  qsum += __shfl_xor(qsum, 1, 64);
  qsum += __shfl_xor(qsum, 2, 64);
  // the MMQ quantiser's DS4 sum in its order (lcpp_shim.cu:320-326): 4-value lane sums
  // ((x0 + x1) + x2) + x3, then xor-butterfly offsets 4, 2, 1 over the slice's 8 lanes; this
  // lane holds the reference's lanes 2q, 2q + 1, so that is xor 2 then xor 1 here, then one add
  float xsum = 0.0f;
  if constexpr (DS4 && !VEC) {
    float a = ((v[0] + v[1]) + v[2]) + v[3];
    float b = ((v[4] + v[5]) + v[6]) + v[7];
    a += __shfl_xor(a, 2, 64);
    b += __shfl_xor(b, 2, 64);
    a += __shfl_xor(a, 1, 64);
    b += __shfl_xor(b, 1, 64);
    xsum = a + b;
  }
  if constexpr (XH) xh_store<DS4>(y, k, c, kk, nct, lo, hi, d, xsum);
  else xq_store<VEC, DS4>(y, k, c, kk, nct, lo, hi, d, qsum, xsum);
}

// block_q8_1 bytes of X (a caller's x_q8) -> the xq layout with the same values and fp16 scales.
template <bool DS4>
__global__ void __launch_bounds__(256) q8_1_to_xq_kernel(const uint8_t* __restrict__ q8, uint8_t* __restrict__ y,
                                                         int k, int n, int nct, int c0, uint32_t* zero, int zero_words) {
  clear_words(zero, zero_words);
  const int kk = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 8;
  if (kk >= k) return;
  const int c = c0 + (int)blockIdx.y;
  uint32_t lo = 0, hi = 0;
  float d = 0.0f;
  if (c < n) {
    const uint8_t* blk = q8 + ((int64_t)c * (k / kQ81) + kk / kQ81) * 36;
    const uint32_t* qv = (const uint32_t*)(blk + 4 + (kk % kQ81));
    lo = qv[0];
    hi = qv[1];
    d = half_bits_to_float(*(const uint16_t*)blk);
  }
  int qsum = dot4((int)lo, 0x01010101, dot4((int)hi, 0x01010101, 0));
  qsum += __shfl_xor(qsum, 1, 64);
  qsum += __shfl_xor(qsum, 2, 64);
  xq_store<true, DS4>(y, k, c, kk, nct, lo, hi, d, qsum, 0.0f);
}

// X [n, k] -> the xq layout at y (xq_bytes(n, k) bytes) for weights of ggml type `type`; vec:
// the decode ops' q8_1 arithmetic, else the MMQ arithmetic. The first launch also clears
// zero_words dwords at zero (null: none).
hipError_t launch_quantize_xq(const void* x, int dtype, int64_t n, int64_t k, int64_t s01, int type, bool vec,
                              void* y, hipStream_t stream, uint32_t* zero, int zero_words) {
  if (n == 0) return hipSuccess;
  const int nct = (int)xq_col_tiles(n), rows = nct * kXqCols;
  const unsigned gx = (unsigned)((k / 8 + 255) / 256);
  const bool ds4 = type == kQ4_K;
  for (int c0 = 0; c0 < rows; c0 += kQuantRowsPerLaunch) {
    const dim3 grid(gx, (unsigned)std::min(rows - c0, kQuantRowsPerLaunch));
#define GGUF_QXQ(DT, V, D) \
  quantize_xq_kernel<DT, V, D><<<grid, 256, 0, stream>>>(x, (uint8_t*)y, (int)k, s01, (int)n, nct, c0, \
                                                         c0 == 0 ? zero : nullptr, zero_words)
#define GGUF_QXQ_DT(DT)                          \
  if (vec) {                                     \
    if (ds4) GGUF_QXQ(DT, true, true);           \
    else GGUF_QXQ(DT, true, false);              \
  } else {                                       \
    if (ds4) GGUF_QXQ(DT, false, true);          \
    else GGUF_QXQ(DT, false, false);             \
  }
    switch (dtype) {
      case kF32: GGUF_QXQ_DT(kF32) break;
      case kF16: GGUF_QXQ_DT(kF16) break;
      default: GGUF_QXQ_DT(kBF16) break;
    }
#undef GGUF_QXQ_DT
#undef GGUF_QXQ
  }
  return hipGetLastError();
}

// X [n, k] -> the xh layout at y (xh_bytes(n, k) bytes), MMQ arithmetic, for weights of `type`.
hipError_t launch_quantize_xh(const void* x, int dtype, int64_t n, int64_t k, int64_t s01, int type, void* y,
                              hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const int nct = (int)xq_col_tiles(n), rows = nct * kXqCols;
  const unsigned gx = (unsigned)((k / 8 + 255) / 256);
  const bool ds4 = type == kQ4_K;
  for (int c0 = 0; c0 < rows; c0 += kQuantRowsPerLaunch) {
    const dim3 grid(gx, (unsigned)std::min(rows - c0, kQuantRowsPerLaunch));
#define GGUF_QXH(DT)                                                                                               \
  if (ds4)                                                                                                         \
    quantize_xq_kernel<DT, false, true, true><<<grid, 256, 0, stream>>>(x, (uint8_t*)y, (int)k, s01, (int)n, nct, c0, \
                                                                        nullptr, 0);                              \
  else                                                                                                             \
    quantize_xq_kernel<DT, false, false, true><<<grid, 256, 0, stream>>>(x, (uint8_t*)y, (int)k, s01, (int)n, nct, c0, \
                                                                         nullptr, 0);
    switch (dtype) {
      case kF32: GGUF_QXH(kF32) break;
      case kF16: GGUF_QXH(kF16) break;
      default: GGUF_QXH(kBF16) break;
    }
#undef GGUF_QXH
  }
  return hipGetLastError();
}

// block_q8_1 of X [n, k] -> the xq layout at y; the first launch also clears zero_words dwords at
// zero (null: none).
hipError_t launch_q8_1_to_xq(const void* q8, int64_t n, int64_t k, int type, void* y, hipStream_t stream,
                             uint32_t* zero, int zero_words) {
  if (n == 0) return hipSuccess;
  const int nct = (int)xq_col_tiles(n), rows = nct * kXqCols;
  const unsigned gx = (unsigned)((k / 8 + 255) / 256);
  for (int c0 = 0; c0 < rows; c0 += kQuantRowsPerLaunch) {
    const dim3 grid(gx, (unsigned)std::min(rows - c0, kQuantRowsPerLaunch));
    if (type == kQ4_K)
      q8_1_to_xq_kernel<true><<<grid, 256, 0, stream>>>((const uint8_t*)q8, (uint8_t*)y, (int)k, (int)n, nct, c0,
                                                        c0 == 0 ? zero : nullptr, zero_words);
    else
      q8_1_to_xq_kernel<false><<<grid, 256, 0, stream>>>((const uint8_t*)q8, (uint8_t*)y, (int)k, (int)n, nct, c0,
                                                         c0 == 0 ? zero : nullptr, zero_words);
  }
  return hipGetLastError();
}

// X [n, k] (row stride s01 elements, dtype DT) -> q8 bytes at y.
hipError_t launch_quantize(const void* x, int dtype, int64_t n, int64_t k, int64_t s01, int type, bool mmq,
                           void* y, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  if (!mmq) {
    const dim3 grid((unsigned)((k + 255) / 256), (unsigned)n);
    switch (dtype) {
      case kF32: quantize_q8_1_kernel<kF32><<<grid, 256, 0, stream>>>(x, (uint8_t*)y, k, s01); break;
      case kF16: quantize_q8_1_kernel<kF16><<<grid, 256, 0, stream>>>(x, (uint8_t*)y, k, s01); break;
      default: quantize_q8_1_kernel<kBF16><<<grid, 256, 0, stream>>>(x, (uint8_t*)y, k, s01); break;
    }
    return hipGetLastError();
  }
  const dim3 grid((unsigned)n, (unsigned)((k + 511) / 512));
  const int layout = mmq_layout(type);
#define GGUF_QMMQ(DT)                                                                                           \
  if (layout == kDS4) quantize_q8_1_mmq_kernel<DT, kDS4><<<grid, 128, 0, stream>>>(x, (uint8_t*)y, k, s01, (int)n);   \
  else if (layout == kD2S6) quantize_q8_1_mmq_kernel<DT, kD2S6><<<grid, 128, 0, stream>>>(x, (uint8_t*)y, k, s01, (int)n); \
  else quantize_q8_1_mmq_kernel<DT, kD4><<<grid, 128, 0, stream>>>(x, (uint8_t*)y, k, s01, (int)n);
  switch (dtype) {
    case kF32: GGUF_QMMQ(kF32) break;
    case kF16: GGUF_QMMQ(kF16) break;
    default: GGUF_QMMQ(kBF16) break;
  }
#undef GGUF_QMMQ
  return hipGetLastError();
}

}  // namespace gguf
