// Dense (F32 / F16 / BF16) products of small weights at few activation rows:
// Y[c, r] = sum_k X[c, k] * W[r, k], for the GGUF file's unquantized tensors.
//
// Replaces the reference's batched-GEMV route for such weights (quantization/linear.py:281-291:
// at most 128 weight rows times up to 8 activation rows, where a library GEMM picks a few tiny
// workgroups): one workgroup per weight row, its 4 waves split K; lane l takes 8 consecutive
// values at 8l + 512i of its wave's K range with one 16-byte (32-byte for fp32) load of W and of
// each activation row; products in fp32, a 64-lane xor butterfly, then the waves' sums in wave
// order through LDS; Y in X's dtype, rounded to nearest even.
#include "gguf_common.h"

namespace gguf {

namespace {

constexpr int kDenseWaves = 4;

template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float (&v)[8]) {
  if constexpr (DT == kF32) {
    const float4 a = *(const float4*)((const float*)p + i), b = *(const float4*)((const float*)p + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 a = *(const uint4*)((const uint16_t*)p + i);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (DT == kF16) {
        v[2 * e] = half_bits_to_float(w[e] & 0xFFFF);
        v[2 * e + 1] = half_bits_to_float(w[e] >> 16);
      } else {
        v[2 * e] = __uint_as_float(w[e] << 16);
        v[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
      }
    }
  }
}

template <int DT, int NC>
__global__ void __launch_bounds__(64 * kDenseWaves) dense_gemv_kernel(const void* __restrict__ W, int64_t ws0,
                                                                      int rows, int k, const void* __restrict__ X,
                                                                      int64_t xs0, void* __restrict__ y) {
  __shared__ float part[kDenseWaves][NC];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x;
  const int k0 = wave * (k / kDenseWaves), k1 = k0 + k / kDenseWaves;  // k % 32 == 0
  float acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
  for (int kk = k0 + 8 * lane; kk < k1; kk += 512) {
    float w[8];
    load8<DT>(W, (int64_t)row * ws0 + kk, w);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float x[8];
      load8<DT>(X, (int64_t)c * xs0 + kk, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[c] = fmaf(w[e], x[e], acc[c]);
    }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float v = acc[c];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) part[wave][c] = v;
  }
  __syncthreads();
  if (threadIdx.x < NC) {
    const int c = threadIdx.x;
    float v = part[0][c];
#pragma unroll
    for (int w2 = 1; w2 < kDenseWaves; ++w2) v += part[w2][c];
    store_y(y, (int64_t)c * rows + row, v, DT);
  }
}

template <int DT>
void launch_dense_dt(const void* W, int64_t ws0, int rows, int k, const void* X, int64_t xs0, int n, void* y,
                     hipStream_t stream) {
#define GGUF_DENSE(NC) dense_gemv_kernel<DT, NC><<<rows, 64 * kDenseWaves, 0, stream>>>(W, ws0, rows, k, X, xs0, y)
  switch (n) {
    case 1: GGUF_DENSE(1); break;
    case 2: GGUF_DENSE(2); break;
    case 3: GGUF_DENSE(3); break;
    case 4: GGUF_DENSE(4); break;
    case 5: GGUF_DENSE(5); break;
    case 6: GGUF_DENSE(6); break;
    case 7: GGUF_DENSE(7); break;
    default: GGUF_DENSE(8); break;
  }
#undef GGUF_DENSE
}

}  // namespace

// W [rows, k] and X [n, k] (1 <= n <= 8) of one float dtype with row strides ws0 / xs0 in
// elements; k % 32 == 0; data and row strides 16-byte aligned (checked by the caller).
hipError_t launch_dense(int dtype, const void* W, int64_t ws0, int rows, int k, const void* X, int64_t xs0, int n,
                        void* y, hipStream_t stream) {
  switch (dtype) {
    case kF32: launch_dense_dt<kF32>(W, ws0, rows, k, X, xs0, n, y, stream); break;
    case kF16: launch_dense_dt<kF16>(W, ws0, rows, k, X, xs0, n, y, stream); break;
    default: launch_dense_dt<kBF16>(W, ws0, rows, k, X, xs0, n, y, stream); break;
  }
  return hipGetLastError();
}

}  // namespace gguf
