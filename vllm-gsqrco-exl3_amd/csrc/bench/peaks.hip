// Measured denominators for bench.py: what one MI355X sustains on the two resources the
// path's kernels are bound by, timed the way the path's kernels are timed (graph replays of single
// launches). Not part of the product library or its C ABI: built into libgguf_peaks.so, which only
// bench.py loads.
//  * gguf_peak_read: a read-only stream over `bytes` of device memory in one launch, the access
//    pattern of the decode GEMV (each workgroup reads one contiguous equal share with 16-byte
//    buffer loads, U loads in flight per lane, optionally non-temporal), so that its time is the
//    floor of a weight-streaming launch of that size: launch and ramp included.
//  * gguf_peak_mfma: chains of independent MFMAs (or v_dot4 on the VALU) with operands in
//    registers and no memory traffic, one kernel per instruction shape: the dense MFMA rate each
//    shape sustains, for the rate the GEMMs are priced against.
// Results are kept live by a store that the data never triggers (the sum compared with a value
// the host passes), so no load or MFMA is dropped by the compiler.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Workgroup g reads [g * chunk, min((g + 1) * chunk, bytes)), chunk a multiple of 16 * blockDim.
template <int U, int CPOL>
__global__ void read_stream_kernel(const uint8_t* __restrict__ src, uint64_t bytes, uint64_t chunk, uint32_t key,
                                   uint32_t* __restrict__ sink) {
  const uint64_t b0 = (uint64_t)blockIdx.x * chunk;
  if (b0 >= bytes) return;
  const uint32_t mine = (uint32_t)(bytes - b0 < chunk ? bytes - b0 : chunk);
  const __amdgpu_buffer_rsrc_t rs = rsrc(src + b0, mine);
  const uint32_t step = 16u * blockDim.x;
  uint32_t acc = 0;
  uint32_t off = 16u * threadIdx.x;
  for (; off + (U - 1) * step < mine; off += U * step) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(off + u * step), 0, CPOL);
#pragma unroll
    for (int u = 0; u < U; ++u) acc += v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; off < mine; off += step) {  // the tail: loads past `mine` read zeros
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, CPOL);
    acc += v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == key) sink[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// CH independent accumulators per wave, `iters` rounds of CH MFMAs each.
template <int CH>
__global__ void __launch_bounds__(256) mfma_i8_kernel(int iters, int key, int* __restrict__ sink) {
  i32x4 a = {(int)threadIdx.x, (int)threadIdx.x * 3, 7, 11}, b = {5, (int)blockIdx.x, 13, 1};
  i32x4 c[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) c[i] = (i32x4){i, 0, 0, 0};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < CH; ++i) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[i], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int i = 0; i < CH; ++i) s += c[i].x + c[i].y + c[i].z + c[i].w;
  if (s == key) sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <int CH>
__global__ void __launch_bounds__(256) mfma_f16_kernel(int iters, int key, int* __restrict__ sink) {
  const _Float16 t = (_Float16)(threadIdx.x & 7) * (_Float16)0.125f;
  const f16x8 a = {t, t, t, t, t, t, t, t}, b = {(_Float16)1.0f, t, t, t, t, t, t, (_Float16)0.5f};
  f32x4 c[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) c[i] = (f32x4){(float)i, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < CH; ++i) c[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) s += c[i].x + c[i].y + c[i].z + c[i].w;
  if (__float_as_int(s) == key) sink[blockIdx.x * blockDim.x + threadIdx.x] = __float_as_int(s);
}

// the other shapes: K selects the instruction (see gguf_peak_mfma)
template <int K>
__global__ void __launch_bounds__(256) mfma_shape_kernel(int iters, int key, int* __restrict__ sink) {
  int s = 0;
  if constexpr (K == 2) {  // v_mfma_i32_32x32x32_i8: 4 chains of 16 accumulators
    const i32x4 a = {(int)threadIdx.x, 1, 2, 3}, b = {(int)blockIdx.x, 5, 6, 7};
    i32x16 c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = (i32x16){};
      c[i][0] = i;
    }
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[i & 3], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) s += c[i][0] + c[i][15];
  } else if constexpr (K == 3) {  // v_mfma_f32_32x32x16_f16
    const _Float16 t = (_Float16)(threadIdx.x & 7) * (_Float16)0.125f;
    const f16x8 a = {t, t, t, t, t, t, t, t}, b = {(_Float16)1.0f, t, t, t, t, t, t, (_Float16)0.5f};
    f32x16 c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = (f32x16){};
      c[i][0] = (float)i;
    }
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[i & 3], 0, 0, 0);
    float f = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) f += c[i][0] + c[i][15];
    s = __float_as_int(f);
  } else if constexpr (K == 4) {  // v_mfma_i32_16x16x32_i8
    const long a = threadIdx.x, b = blockIdx.x * 3 + 1;
    i32x4 c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = (i32x4){i, 0, 0, 0};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) s += c[i].x + c[i].w;
  } else if constexpr (K == 5) {  // v_mfma_i32_4x4x4_16b_i8
    const int a = threadIdx.x, b = blockIdx.x * 3 + 1;
    i32x4 c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = (i32x4){i, 0, 0, 0};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_mfma_i32_4x4x4i8(a, b, c[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) s += c[i].x + c[i].w;
  } else {  // v_dot4_i32_i8 on the VALU
    const int a = threadIdx.x, b = blockIdx.x * 3 + 1;
    int c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = i;
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_sdot4(a, b, c[i], false);
#pragma unroll
    for (int i = 0; i < 8; ++i) s += c[i];
  }
  if (s == key) sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

extern "C" {

// One read of `bytes` (at most 4 GiB per workgroup share) by `grid` workgroups of `threads`
// threads (64..1024, a multiple of 64), `unroll` loads in flight per lane (1, 2, 4 or 8),
// non-temporal when nt != 0. sink: grid * threads uint32 (written only if the data sums to key).
__attribute__((visibility("default"))) int gguf_peak_read(const void* src, uint64_t bytes, int grid, int threads,
                                                         int unroll, int nt, uint32_t key, void* sink,
                                                         void* stream) {
  if (!src || !sink || grid < 1 || threads < 64 || threads > 1024 || threads % 64) return 1;
  const uint64_t line = 16ull * threads;
  const uint64_t chunk = ((bytes + grid - 1) / grid + line - 1) / line * line;
  if (chunk >= (1ull << 32)) return 1;
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* p = (const uint8_t*)src;
  uint32_t* k = (uint32_t*)sink;
#define GGUF_RD(U)                                                                                   \
  if (nt) read_stream_kernel<U, 3><<<grid, threads, 0, s>>>(p, bytes, chunk, key, k);               \
  else read_stream_kernel<U, 0><<<grid, threads, 0, s>>>(p, bytes, chunk, key, k)
  switch (unroll) {
    case 1: GGUF_RD(1); break;
    case 2: GGUF_RD(2); break;
    case 4: GGUF_RD(4); break;
    case 8: GGUF_RD(8); break;
    default: return 1;
  }
#undef GGUF_RD
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// grid workgroups of 4 waves, each wave 8 instructions x iters (8 independent chains; 4 chains
// for the 32 x 32 shapes). Operations per instruction: kind 0 v_mfma_i32_16x16x64_i8 32,768;
// 1 v_mfma_f32_16x16x32_f16 16,384; 2 v_mfma_i32_32x32x32_i8 65,536; 3 v_mfma_f32_32x32x16_f16
// 32,768; 4 v_mfma_i32_16x16x32_i8 16,384; 5 v_mfma_i32_4x4x4_16b_i8 2,048; 6 v_dot4_i32_i8
// 512 (64 lanes x 4 multiply-adds). sink: grid * 256 int.
__attribute__((visibility("default"))) int gguf_peak_mfma(int kind, int grid, int iters, int key, void* sink,
                                                         void* stream) {
  if (!sink || grid < 1 || iters < 1) return 1;
  hipStream_t s = (hipStream_t)stream;
  int* k = (int*)sink;
  switch (kind) {
    case 0: mfma_i8_kernel<8><<<grid, 256, 0, s>>>(iters, key, k); break;
    case 1: mfma_f16_kernel<8><<<grid, 256, 0, s>>>(iters, key, k); break;
    case 2: mfma_shape_kernel<2><<<grid, 256, 0, s>>>(iters, key, k); break;
    case 3: mfma_shape_kernel<3><<<grid, 256, 0, s>>>(iters, key, k); break;
    case 4: mfma_shape_kernel<4><<<grid, 256, 0, s>>>(iters, key, k); break;
    case 5: mfma_shape_kernel<5><<<grid, 256, 0, s>>>(iters, key, k); break;
    case 6: mfma_shape_kernel<6><<<grid, 256, 0, s>>>(iters, key, k); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
