// int8-MFMA GEMM for 9+ activation rows on GGUF bytes: Y[c, r] = sum_k X[c, k] * W[r, k].
//
// Replaces the reference's MMQ-class products on plain GGUF rows (vendored mul_mat_q via
// lcpp_shim.cu:626-671 and the owned mma_k kernel lcpp_owned_mma_k.cu:354-540) with a gfx950
// design on v_mfma_i32_16x16x32_i8 (IQ3_S in the tile layout has its own GEMM, gemm_tile.hip):
//  * X is quantised to q8_1 in the MMQ block layout (quantize.hip); one 32-value slice is one
//    MFMA K step, so every MFMA result is exactly the reference's per-slice int32 dot;
//  * a workgroup owns 16 weight rows and 16*NT columns of X; its 4 waves split the K slices;
//    lane l decodes values 8q..8q+7 (q = l/16) of the slice of weight row l%16 straight into
//    the MFMA A operand, and reads the same 8 K positions of X column l%16 as the B operand;
//  * per slice, each int32 result is scaled in fp32 by (weight scale x activation scale) and
//    added to the accumulator; Q6_K takes two MFMAs per slice, one per 16-value sub-scale,
//    combined in int32 as the reference does; Q4_K's min term uses the integer q8 sum;
//  * the 4 waves' partial sums are added in wave order through LDS (deterministic).
#include "decode.h"

namespace gguf {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma16x16x32(long a, long b) {
  const v4i z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

template <int TYPE, int NT>
__global__ void __launch_bounds__(256) gemm_mfma_kernel(const uint8_t* __restrict__ W, int64_t row_bytes, int nrows,
                                                        int k, const uint8_t* __restrict__ q8, int n,
                                                        void* __restrict__ y, int y_dtype) {
  __shared__ uint32_t grid[TYPE == kIQ3_S ? 512 : 1];
  __shared__ float part[3][NT][4][64];
  if constexpr (TYPE == kIQ3_S) {
    for (int i = threadIdx.x; i < 512; i += blockDim.x) grid[i] = kIq3sGrid.v[i];
    __syncthreads();
  }
  constexpr int BS = block_bytes(TYPE);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q = lane >> 4;     // K quarter of the slice this lane carries (values 8q..8q+7)
  const int li = lane & 15;    // A row / B column index within the 16x16 tile
  const int row = blockIdx.x * 16 + li;          // weight row this lane decodes
  const int col0 = blockIdx.y * 16 * NT;         // first X column of the workgroup
  const int nslices = k / kQ81;
  const int per = nslices / 4;                   // k % 512 == 0: whole multiples of 4
  const int s_begin = wave * per, s_end = s_begin + per;
  const bool row_ok = row < nrows;
  const uint8_t* wrow = W + (int64_t)(row_ok ? row : 0) * row_bytes;

  float acc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t][v] = 0.0f;

  for (int s = s_begin; s < s_end; ++s) {
    const uint8_t* b = wrow + (int64_t)(s >> 3) * BS;
    const int u = s & 7;
    int wa[2];
    SliceScale sc;
    if constexpr (TYPE == kIQ3_S) {
      decode_iq3s_q(b, u, q, grid, wa, sc);
    }
    if constexpr (TYPE == kQ4_K) decode_q4k_q(b, u, q, wa, sc);
    if constexpr (TYPE == kIQ4_XS) decode_iq4xs_q(b, u, q, wa, sc);
    if constexpr (TYPE == kQ6_K) decode_q6k_q(b, u, q, wa, sc);
    if (!row_ok) wa[0] = wa[1] = 0;
    const long a = (long)(((uint64_t)(uint32_t)wa[1] << 32) | (uint32_t)wa[0]);

    // scales of the 4 output rows 4*q + v this lane accumulates (held by lanes 4q+v)
    float rs[4], rm[4], rs2[4];
    float my_s, my_m = 0.0f, my_s2 = 0.0f;
    if constexpr (TYPE == kQ4_K) {
      my_s = sc.d * (float)sc.ls;
      my_m = sc.dmin * (float)sc.ls2;
    } else if constexpr (TYPE == kQ6_K) {
      my_s = sc.d;
      // sub-scales of both halves: quarters 0,1 hold the first, 2,3 the second
      my_s2 = (float)sc.ls;
    } else {
      my_s = sc.d * (float)sc.ls;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int src = 4 * q + v;
      rs[v] = __shfl(my_s, src, 64);
      if constexpr (TYPE == kQ4_K) rm[v] = __shfl(my_m, src, 64);
      if constexpr (TYPE == kQ6_K) {
        rm[v] = __shfl(my_s2, src, 64);        // first-half scale (lane src has q = 0)
        rs2[v] = __shfl(my_s2, src + 32, 64);  // second-half scale (lane src + 32 has q = 2)
      }
    }

#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = col0 + 16 * t + li;
      long bq = 0;
      float cd = 0.0f;
      if (col < n) {
        const uint8_t* xb = q8 + ((int64_t)(s >> 2) * n + col) * 144;
        bq = *(const long*)(xb + 16 + 32 * (s & 3) + 8 * q);
        if constexpr (TYPE == kQ4_K) {
          cd = half_bits_to_float(*(const uint16_t*)(xb + 4 * (s & 3)));
        } else {
          cd = *(const float*)(xb + 4 * (s & 3));
        }
      }
      if constexpr (TYPE == kQ6_K) {
        // two MFMAs: K positions of the first 16 values (quarters 0,1), then the second 16
        const long a0 = q < 2 ? a : 0;
        const long a1 = q < 2 ? 0 : a;
        const v4i c0 = mfma16x16x32(a0, bq);
        const v4i c1 = mfma16x16x32(a1, bq);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int isum = c0[v] * (int)rm[v] + c1[v] * (int)rs2[v];
          acc[t][v] += (float)isum * (rs[v] * cd);
        }
      } else {
        const v4i c = mfma16x16x32(a, bq);
        if constexpr (TYPE == kQ4_K) {
          // integer sum of the slice's q8 values of this column: 8 per quarter lane
          int sq = dot4(0x01010101, (int)(uint32_t)bq, dot4(0x01010101, (int)(uint32_t)((uint64_t)bq >> 32), 0));
          sq += __shfl_xor(sq, 16, 64);
          sq += __shfl_xor(sq, 32, 64);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[t][v] += ((float)c[v] * rs[v] - (float)sq * rm[v]) * cd;
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[t][v] += (float)c[v] * (rs[v] * cd);
        }
      }
    }
  }

  // K-split partial sums: waves 1..3 park theirs in LDS, wave 0 adds them in wave order
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[wave - 1][t][v][lane] = acc[t][v];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = col0 + 16 * t + li;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float r = acc[t][v];
        r += part[0][t][v][lane];
        r += part[1][t][v][lane];
        r += part[2][t][v][lane];
        const int orow = blockIdx.x * 16 + 4 * q + v;
        if (col < n && orow < nrows) store_y(y, (int64_t)col * nrows + orow, r, y_dtype);
      }
    }
  }
}

template <int TYPE>
static void launch_gemm_t(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n, void* y,
                          int y_dtype, hipStream_t stream) {
  const unsigned gx = (unsigned)((nrows + 15) / 16);
  const int tiles = (n + 15) / 16;
  if (tiles <= 1) {
    gemm_mfma_kernel<TYPE, 1><<<dim3(gx, 1), 256, 0, stream>>>(W, row_bytes, nrows, k, q8, n, y, y_dtype);
  } else if (tiles == 2) {
    gemm_mfma_kernel<TYPE, 2><<<dim3(gx, 1), 256, 0, stream>>>(W, row_bytes, nrows, k, q8, n, y, y_dtype);
  } else if (tiles == 3) {
    gemm_mfma_kernel<TYPE, 3><<<dim3(gx, 1), 256, 0, stream>>>(W, row_bytes, nrows, k, q8, n, y, y_dtype);
  } else {
    const unsigned gy = (unsigned)((tiles + 3) / 4);
    gemm_mfma_kernel<TYPE, 4><<<dim3(gx, gy), 256, 0, stream>>>(W, row_bytes, nrows, k, q8, n, y, y_dtype);
  }
}

// q8: block_q8_1_mmq of X (n columns); y: [n, nrows] in y_dtype.
hipError_t launch_gemm(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                       void* y, int y_dtype, hipStream_t stream) {
  switch (type) {
    case kIQ3_S: launch_gemm_t<kIQ3_S>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ4_K: launch_gemm_t<kQ4_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ4_XS: launch_gemm_t<kIQ4_XS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ6_K: launch_gemm_t<kQ6_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace gguf
