// int8-MFMA GEMM for 9+ activation rows on GGUF bytes: Y[c, r] = sum_k X[c, k] * W[r, k].
//
// Replaces the reference's MMQ-class products on plain GGUF rows (vendored mul_mat_q via
// lcpp_shim.cu:626-671 and the owned mma_k kernel lcpp_owned_mma_k.cu:354-540) with gfx950
// designs on v_mfma_i32_16x16x32_i8 (IQ3_S in the tile layout has its own GEMM, gemm_tile.hip).
//
// gemm_mfma_kernel (IQ3_S on plain rows; Q2_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ1_M):
//  * X is quantised to q8_1 in the MMQ block layout (quantize.hip); one 32-value slice is one
//    MFMA K step, so every MFMA result is exactly the reference's per-slice int32 dot;
//  * a workgroup owns 16 weight rows and 16*NT columns of X; its 4 waves split the K slices;
//    lane l decodes values 8q..8q+7 (q = l/16) of the slice of weight row l%16 straight into
//    the MFMA A operand, and reads the same 8 K positions of X column l%16 as the B operand;
//  * per slice, each int32 result is scaled in fp32 by (weight scale x activation scale) and
//    added to the accumulator; types with a sub-scale per 16 values take two MFMAs per slice;
//  * the 4 waves' partial sums are added in wave order through LDS (deterministic).
// gemm_raw_kernel (Q4_K, IQ4_XS, Q6_K) reads X in the xq layout; see its own description below.
#include "decode.h"
#include "iq3_tile.h"
#include "split_k.h"
#include "xq.h"

namespace gguf {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma16x16x32(long a, long b) {
  const v4i z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ float round_half(float v) { return __half2float(__float2half_rn(v)); }

// The per-slice MFMA GEMM on plain GGUF rows for IQ3_S and the types served only by the generic
// kernels, X in block_q8_1_mmq (D4; Q2_K D2S6). The slice terms are the reference's product-op
// (MMQ) arithmetic:
//   IQ3_S, IQ2_XXS, IQ3_XXS  C * (d * ls / den) * d4: the x_df of the MMQ tile loaders
//       (mmq-load-tiles.cuh:1150-1152, :1348-1352; den 8 for IQ2, 4 for IQ3_XXS), exact in fp32
//   IQ2_XS, IQ2_S, IQ1_M     per 16 values, ls_h = 2 * scale + 1: (C_a * ls_a + C_b * ls_b) *
//       (d / 8) * d4, the same products as x_df = ((scale * d + d / 2) / 4) (:1207-1208, :1284-1285)
//       combined in int32
//   Q2_K  per 16 values h with dm_h = (half(d * sc_h), half(dmin * m_h)) (:582-591) and D2S6 d4:
//       (C_h * dm_h.x) * d4 - dm_h.y * S_h, S_h the stored fp16 sum of x, for the groups 0..5 of
//       each 128 values, and (C_h * dm_h.x - sum_h(q8) * dm_h.y) * d4 for groups 6, 7
//       (ggml_cuda_mmq_vec_dot_q2_K_q8_1_mma, mmq-vec-dot.cuh:688-745)
template <int TYPE, int NT>
__global__ void __launch_bounds__(256) gemm_mfma_kernel(const uint8_t* __restrict__ W, int64_t row_bytes, int nrows,
                                                        int k, const uint8_t* __restrict__ q8, int n,
                                                        void* __restrict__ y, int y_dtype) {
  using G = typename Codebook<TYPE>::T;
  __shared__ G grid[Codebook<TYPE>::n];
  __shared__ float part[3][NT][4][64];
  if constexpr (Codebook<TYPE>::n > 1) {
    stage_codebook<TYPE>(grid);
    __syncthreads();
  }
  constexpr bool P16 = per16_type(TYPE);
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
    const int u = s & 7, s4 = s & 3;
    int wa[2];
    SliceScale sc;
    decode_quarter<TYPE>(b, u, q, grid, wa, sc);
    if (!row_ok) wa[0] = wa[1] = 0;
    const long a = (long)(((uint64_t)(uint32_t)wa[1] << 32) | (uint32_t)wa[0]);

    // A-side scales of the 4 C rows 4q + v: lane 4q + v decoded that row's first 16 values
    // (q = 0), lane 4q + v + 32 its second 16 (q = 2)
    float my_s, my_m = 0.0f;
    if constexpr (TYPE == kQ2_K) {
      my_s = round_half(sc.d * (float)sc.ls);
      my_m = round_half(sc.dmin * (float)sc.m);
    } else if constexpr (P16) {
      my_s = (float)sc.ls;
      my_m = sc.d * 0.125f;
    } else {
      my_s = (sc.d * (float)sc.ls) * (1.0f / (float)iq_den(TYPE));
    }
    float rs[4], rs2[4], rm[4], rm2[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int src = 4 * q + v;
      rs[v] = __shfl(my_s, src, 64);
      if constexpr (P16) {
        rs2[v] = __shfl(my_s, src + 32, 64);
        rm[v] = __shfl(my_m, src, 64);
        rm2[v] = __shfl(my_m, src + 32, 64);
      }
    }

#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = col0 + 16 * t + li;
      long bq = 0;
      float cd = 0.0f, sx0 = 0.0f, sx1 = 0.0f;
      if (col < n) {
        const uint8_t* xb = q8 + ((int64_t)(s >> 2) * n + col) * 144;
        bq = *(const long*)(xb + 16 + 32 * s4 + 8 * q);
        if constexpr (TYPE == kQ2_K) {
          cd = half_bits_to_float(ld16(xb + 2 * (s4 >> 1)));
          if (s4 < 3) {
            sx0 = half_bits_to_float(ld16(xb + 4 + 4 * s4));
            sx1 = half_bits_to_float(ld16(xb + 6 + 4 * s4));
          }
        } else {
          cd = *(const float*)(xb + 4 * s4);
        }
      }
      if constexpr (P16) {
        // two MFMAs: K positions of the first 16 values (quarters 0,1), then the second 16
        const long a0 = q < 2 ? a : 0;
        const long a1 = q < 2 ? 0 : a;
        const v4i c0 = mfma16x16x32(a0, bq);
        const v4i c1 = mfma16x16x32(a1, bq);
        if constexpr (TYPE == kQ2_K) {
          int m0 = 0, m1 = 0;  // groups 6, 7: integer sums of the column's q8 over each half
          if (s4 == 3) {
            const int sq = dot4(0x01010101, (int)(uint32_t)bq, dot4(0x01010101, (int)(uint32_t)((uint64_t)bq >> 32), 0));
            m0 = __shfl(sq, li, 64) + __shfl(sq, li + 16, 64);
            m1 = __shfl(sq, li + 32, 64) + __shfl(sq, li + 48, 64);
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float t0 = (float)c0[v] * rs[v];
            float t1 = (float)c1[v] * rs2[v];
            if (s4 == 3) {
              t0 -= (float)m0 * rm[v];
              t1 -= (float)m1 * rm2[v];
            }
            acc[t][v] += t0 * cd;
            acc[t][v] -= rm[v] * sx0;
            acc[t][v] += t1 * cd;
            acc[t][v] -= rm2[v] * sx1;
          }
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int isum = c0[v] * (int)rs[v] + c1[v] * (int)rs2[v];
            acc[t][v] += (float)isum * (rm[v] * cd);
          }
        }
      } else {
        const v4i c = mfma16x16x32(a, bq);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][v] += (float)c[v] * (rs[v] * cd);
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

// q8: block_q8_1_mmq of X (n columns; D4, Q2_K D2S6); y: [n, nrows] in y_dtype. IQ3_S on plain
// rows and the generic types.
hipError_t launch_gemm(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                       void* y, int y_dtype, hipStream_t stream) {
  switch (type) {
    case kIQ3_S: launch_gemm_t<kIQ3_S>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ2_K: launch_gemm_t<kQ2_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ2_XXS: launch_gemm_t<kIQ2_XXS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ2_XS: launch_gemm_t<kIQ2_XS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ2_S: launch_gemm_t<kIQ2_S>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ3_XXS: launch_gemm_t<kIQ3_XXS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ1_M: launch_gemm_t<kIQ1_M>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}


// ---------------------------------------------------------------------------------------------
// Q4_K / IQ4_XS / Q6_K on plain GGUF rows, activations in the xq layout (xq.h).
//  * a workgroup owns one 16-row tile and NT column tiles; its KS waves split the K blocks;
//  * per K block lane 16q + j loads, from weight row j, the bytes of values 8q..8q+7 of every
//    slice (Q4_K: four 8-byte loads, each holding two slices as low / high nibbles; IQ4_XS: one
//    8-byte load per slice, codebook through byte permutes; Q6_K: four ql and two qh loads), so
//    the decoded words are the MFMA A operands directly; the row headers of the four C rows
//    4q..4q+3 it accumulates come with 8- or 16-byte loads;
//  * one v_mfma_i32_16x16x32_i8 per (slice, column tile) is the reference's integer slice dot
//    (Q6_K: two, one per 16-value sub-scale, combined in int32 as the reference does);
//  * per slice the dot is scaled by the integer sub-scale and the fp32 activation scale, summed
//    over the block, then multiplied by the row's block scale (Q4_K: minus dmin times the
//    min-term sum over slices of m times the activation side: d8 * sum(q8) for the decode ops'
//    MMVQ arithmetic, the fp16 sum of x for the product ops' MMQ arithmetic, SX);
//  * next block's loads are issued before the current block is computed (two register sets);
//    the waves' partial sums are added in wave order;
//  * on weights of few 16-row tiles (fewer than two per CU) the K blocks are also split over S =
//    gridDim.z workgroups per tile (raw_split): each writes its sums to a slot of the workspace,
//    bumps the tile's counter, and the one that brings it to S adds the S slots in slot order and
//    writes the output (split_k.h).
namespace {

constexpr int kRawRows = 16;   // weight rows per workgroup (the MFMA A rows)
constexpr int kRawWaves = 4;   // waves per workgroup, splitting its K blocks

template <int TYPE>
struct RawFrag;
template <>
struct RawFrag<kQ4_K> {
  uint32_t qs[8];  // 8-byte quarter c = 0..3: slices 2c (low nibbles), 2c+1 (high)
  u32x4 hdr[4];    // d | dmin << 16, scales[0..3], scales[4..7], scales[8..11] of C row 4q + v
};
template <>
struct RawFrag<kIQ4_XS> {
  uint32_t qs[16];    // slice u: bytes 8 (q & 1) .. of qs[16u..], nibble q >> 1
  uint32_t hdr[4][2]; // d | scales_h << 16, scales_l of C row 4q + v
};
template <>
struct RawFrag<kQ6_K> {
  uint32_t ql[8];  // (n, h) = 2n + h: ql[64n + 32h + 8q ..], 8 bytes
  uint32_t qh[4];  // n: qh[32n + 8q ..], 8 bytes
  u32x4 sc[4];     // 16 int8 sub-scales of C row 4q + v
  uint32_t d[4];   // fp16 d of C row 4q + v
};

__device__ __forceinline__ void ld64w(__amdgpu_buffer_rsrc_t rs, int voff, int soff, uint32_t* dst) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0);
  dst[0] = v[0];
  dst[1] = v[1];
}

// row_off: j * row_bytes; crow_off[v]: (4q + v) * row_bytes; soff: block offset
template <int TYPE>
__device__ __forceinline__ void load_raw_frag(__amdgpu_buffer_rsrc_t rs, int row_off, const int (&crow_off)[4],
                                              int soff, int q, RawFrag<TYPE>& f) {
  if constexpr (TYPE == kQ4_K) {
#pragma unroll
    for (int c = 0; c < 4; ++c) ld64w(rs, row_off + 16 + 32 * c + 8 * q, soff, &f.qs[2 * c]);
#pragma unroll
    for (int v = 0; v < 4; ++v) f.hdr[v] = __builtin_amdgcn_raw_buffer_load_b128(rs, crow_off[v], soff, 0);
  } else if constexpr (TYPE == kIQ4_XS) {
#pragma unroll
    for (int u = 0; u < 8; ++u) ld64w(rs, row_off + 8 + 16 * u + 8 * (q & 1), soff, &f.qs[2 * u]);
#pragma unroll
    for (int v = 0; v < 4; ++v) ld64w(rs, crow_off[v], soff, f.hdr[v]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) ld64w(rs, row_off + 64 * (i >> 1) + 32 * (i & 1) + 8 * q, soff, &f.ql[2 * i]);
#pragma unroll
    for (int n = 0; n < 2; ++n) ld64w(rs, row_off + 128 + 32 * n + 8 * q, soff, &f.qh[2 * n]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      f.sc[v] = __builtin_amdgcn_raw_buffer_load_b128(rs, crow_off[v] + 192, soff, 0);
      f.d[v] = __builtin_amdgcn_raw_buffer_load_b16(rs, crow_off[v] + 208, soff, 0);
    }
  }
}

__device__ __forceinline__ long pack_a(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

// A operand of slice u (values 8q..8q+7 of the lane's row)
template <int TYPE>
__device__ __forceinline__ long raw_a(const RawFrag<TYPE>& f, int u, int q) {
  if constexpr (TYPE == kQ4_K) {
    const int c = u >> 1, sh = 4 * (u & 1);
    return pack_a((f.qs[2 * c] >> sh) & 0x0F0F0F0Fu, (f.qs[2 * c + 1] >> sh) & 0x0F0F0F0Fu);
  } else if constexpr (TYPE == kIQ4_XS) {
    const int sh = 4 * (q >> 1);
    return pack_a((uint32_t)iq4nl(f.qs[2 * u], sh),
                  (uint32_t)iq4nl(f.qs[2 * u + 1], sh));
  } else {
    const int n = u >> 2, sub = u & 3, i = 2 * n + (sub & 1);
    const int lsh = 4 * (sub >> 1), hsh = 2 * sub;
    const uint32_t w0 = (uint32_t)sub32_bytes(((f.ql[2 * i] >> lsh) & 0x0F0F0F0Fu) |
                                              (((f.qh[2 * n] >> hsh) & 0x03030303u) << 4));
    const uint32_t w1 = (uint32_t)sub32_bytes(((f.ql[2 * i + 1] >> lsh) & 0x0F0F0F0Fu) |
                                              (((f.qh[2 * n + 1] >> hsh) & 0x03030303u) << 4));
    return pack_a(w0, w1);
  }
}

// Q4_K 6-bit scale and min of sub-block u from scales[0..11] (get_scale_min_k4,
// csrc/gguf/dequantize.cuh:156-163)
__device__ __forceinline__ void q4k_sm(const u32x4& h, int u, int& sc, int& m) {
  const int jj = u & 3;
  const uint32_t a = (h[1] >> (8 * jj)) & 0xFF, c = (h[2] >> (8 * jj)) & 0xFF, e = (h[3] >> (8 * jj)) & 0xFF;
  if (u < 4) {
    sc = (int)(a & 63);
    m = (int)(c & 63);
  } else {
    sc = (int)((e & 0xF) | ((a >> 6) << 4));
    m = (int)((e >> 4) | ((c >> 6) << 4));
  }
}

template <int NT>
struct XRawFrag {
  u32x4 b[NT][4];  // B operands: slices 2i, 2i+1 in b[t][i]
  u32x4 d[NT][2];  // scale words of slices 0..7
};

template <int NT>
__device__ __forceinline__ void load_xraw(__amdgpu_buffer_rsrc_t rs, const int (&units)[NT], int b, int sbase, int lane,
                                          int j, XRawFrag<NT>& x) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int unit = units[t] + b;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      x.b[t][i] = __builtin_amdgcn_raw_buffer_load_b128(rs, 64 * lane + 16 * i, unit * kXqUnit, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      x.d[t][i] = __builtin_amdgcn_raw_buffer_load_b128(rs, 32 * j + 16 * i, sbase + unit * kXqScaleUnit, 0);
  }
}

template <int TYPE, int NT, bool SX>
__device__ __forceinline__ void raw_block(const RawFrag<TYPE>& f, const XRawFrag<NT>& x, int q, float (&acc)[NT][4]) {
  float accb[NT][4], accm[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) accb[t][v] = accm[t][v] = 0.0f;
  const v4i zero = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const long a = raw_a<TYPE>(f, u, q);
    int s1[4], s2[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (TYPE == kQ4_K) {
        q4k_sm(f.hdr[v], u, s1[v], s2[v]);
      } else if constexpr (TYPE == kIQ4_XS) {
        const uint32_t sl = (f.hdr[v][1] >> (8 * (u >> 1) + 4 * (u & 1))) & 0xF;
        const uint32_t shh = (f.hdr[v][0] >> (16 + 2 * u)) & 3u;
        s1[v] = (int)(sl | (shh << 4)) - 32;
      } else {
        const uint32_t word = f.sc[v][u >> 1];
        s1[v] = (int)(int8_t)((word >> (16 * (u & 1))) & 0xFF);
        s2[v] = (int)(int8_t)((word >> (16 * (u & 1) + 8)) & 0xFF);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const long b = xq_b_operand(x.b[t][u >> 1], u & 1);
      const uint32_t sw = x.d[t][u >> 2][u & 3];
      // Q4_K: fp16 d | (SX ? fp16 sum(x) : int16 sum(q)) << 16; other types: fp32 d
      const float cd = TYPE == kQ4_K ? half_bits_to_float(sw & 0xFFFF) : __uint_as_float(sw);
      if constexpr (TYPE == kQ6_K) {
        const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(q < 2 ? a : 0, b, zero, 0, 0, 0);
        const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(q < 2 ? 0 : a, b, zero, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v)
          accb[t][v] = fmaf((float)(__mul24(c0[v], s1[v]) + __mul24(c1[v], s2[v])), cd, accb[t][v]);
      } else {
        const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v) accb[t][v] = fmaf((float)__mul24(c[v], s1[v]), cd, accb[t][v]);
        if constexpr (TYPE == kQ4_K) {
          const float cs = SX ? half_bits_to_float(sw >> 16) : cd * (float)(int)(int16_t)(sw >> 16);
#pragma unroll
          for (int v = 0; v < 4; ++v) accm[t][v] = fmaf((float)s2[v], cs, accm[t][v]);
        }
      }
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float d, dmin = 0.0f;
    if constexpr (TYPE == kQ4_K) {
      d = half_bits_to_float(f.hdr[v][0] & 0xFFFF);
      dmin = half_bits_to_float(f.hdr[v][0] >> 16);
    } else if constexpr (TYPE == kIQ4_XS) {
      d = half_bits_to_float(f.hdr[v][0] & 0xFFFF);
    } else {
      d = half_bits_to_float(f.d[v] & 0xFFFF);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[t][v] = fmaf(accb[t][v], d, acc[t][v]);
      if constexpr (TYPE == kQ4_K) acc[t][v] = fmaf(-accm[t][v], dmin, acc[t][v]);
    }
  }
}

// Up to two column tiles the kernel is held to two workgroups per CU (256 registers per lane):
// Q4_K at two column tiles otherwise takes 257 and runs alone on its CU (measured, op level:
// 5120 x 17408 M = 24 / 32 52.4 / 51.8 -> 38.8 / 38.9 us, 6144 x 5120 22.2 / 22.0 -> 19.6 /
// 19.5). At three column tiles Q6_K's 263 registers squeezed to 256 spill 15 dwords and lose on
// K = 5120 / 6144 (33.6 -> 35.1 us, 37.1 -> 40.6 at M = 48), so three stay unconstrained.
template <int TYPE, int NT, int KS, bool SX>
__global__ void __launch_bounds__(64 * KS, NT <= 2 ? 2 : 1) gemm_raw_kernel(const uint8_t* __restrict__ W, int64_t row_bytes, int nrows,
                                                           int k, const uint8_t* __restrict__ xq, int nct, int n,
                                                           void* __restrict__ y, int y_dtype, float* part,
                                                           uint32_t* cnt) {
  constexpr int BS = block_bytes(TYPE);
  __shared__ float red[KS > 1 ? KS - 1 : 1][NT][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int row0 = blockIdx.x * kRawRows;
  const int rows_here = nrows - row0 < kRawRows ? nrows - row0 : kRawRows;
  const int ct0 = blockIdx.y * NT;
  const int nb = k / kQK;
  // this workgroup's part of K (split z of S), then the wave's part of that
  const int S = (int)gridDim.z, z = (int)blockIdx.z;
  const int zb0 = z * nb / S, zb1 = (z + 1) * nb / S;
  const int b_begin = zb0 + wave * (zb1 - zb0) / KS, b_end = zb0 + (wave + 1) * (zb1 - zb0) / KS;
  // rows past nrows lie past the descriptor's size and read zeros
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(W + (int64_t)row0 * row_bytes, (uint32_t)(rows_here * row_bytes));
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(xq, (uint32_t)xq_bytes((int64_t)nct * kXqCols, k));
  const int sbase = (int)xq_scale_base(nct, nb);
  const int row_off = j * (int)row_bytes;
  int crow_off[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) crow_off[v] = (4 * q + v) * (int)row_bytes;
  int units[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) units[t] = (ct0 + t < nct ? ct0 + t : nct - 1) * nb;

  float acc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t][v] = 0.0f;

  // Two blocks per iteration (an odd last block after the loop); every load feeds a use that is
  // not behind a branch of its own (a load whose only use is conditional is sunk to it); the
  // scheduling barriers keep the next block's decode below the loads just issued. The prefetch
  // past the wave's last block reads zeros through an empty descriptor and is never used.
  const __amdgpu_buffer_rsrc_t nrs = buffer_rsrc(W, 0);
  RawFrag<TYPE> fa, fb;
  XRawFrag<NT> xa, xb;
  const int b_last = b_end - 1;
  if (b_begin < b_end) {
    load_xraw<NT>(xrs, units, b_begin, sbase, lane, j, xa);
    load_raw_frag<TYPE>(wrs, row_off, crow_off, b_begin * BS, q, fa);
  }
  const int nblk = b_end - b_begin;
  int b = b_begin;
  for (int it = 0; it < nblk / 2; ++it, b += 2) {
    const int b2 = b + 2 < b_last ? b + 2 : b_last;
    const __amdgpu_buffer_rsrc_t rs2 = b + 2 < b_end ? wrs : nrs;
    load_xraw<NT>(xrs, units, b + 1, sbase, lane, j, xb);
    load_raw_frag<TYPE>(wrs, row_off, crow_off, (b + 1) * BS, q, fb);
    __builtin_amdgcn_sched_barrier(0);
    raw_block<TYPE, NT, SX>(fa, xa, q, acc);
    load_xraw<NT>(xrs, units, b2, sbase, lane, j, xa);
    load_raw_frag<TYPE>(rs2, row_off, crow_off, (b + 2) * BS, q, fa);
    __builtin_amdgcn_sched_barrier(0);
    raw_block<TYPE, NT, SX>(fb, xb, q, acc);
  }
  if (nblk & 1) raw_block<TYPE, NT, SX>(fa, xa, q, acc);

  if constexpr (KS > 1) {
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[wave - 1][t][v][lane] = acc[t][v];
    }
    __syncthreads();
  }
  if (wave != 0) return;
  float sum[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sum[t][v] = acc[t][v];
      for (int w2 = 1; w2 < KS; ++w2) sum[t][v] += red[w2 - 1][t][v][lane];
    }
  if (S > 1 && !split_fixup<NT>(sum, part, cnt, S, z, (size_t)blockIdx.x * gridDim.y + blockIdx.y, lane)) return;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int col = (ct0 + t) * kXqCols + j;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 4 * q + v;
      if (col < n && row < rows_here) store_y(y, (int64_t)col * nrows + row0 + row, sum[t][v], y_dtype);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// IQ2_XXS, IQ2_XS, IQ2_S and IQ3_XXS on GGUF rows, X in the xq layout (MMQ arithmetic, fp32 d per
// slice). A workgroup owns one 16-row tile and NT column tiles; its KS waves split the K blocks.
// Per K block a wave copies the tile's 16 block-rows into a wave-private LDS buffer (lane l: 32
// bytes of row l / 4, two 16-byte loads, contiguous along each row; the next block's copy is in
// flight while the current block is computed), then lane 16q + j decodes values 8q..8q+7 of every
// slice of row j from LDS (decode.h, codebook in LDS) straight into the MFMA A operand. The copy
// starts at the 4-byte aligned address at or below the block (rows are 4-byte multiples, blocks
// 2), so no dword it reads straddles the end of the tile's bytes; the block lies at byte 0 or 2
// of its staged row. The B
// operands and scales come from the xq unit as in gemm_raw_kernel. The slice terms are the product
// ops' MMQ forms: (C * ls) * d4 per slice (two MFMAs and C_a * ls_a + C_b * ls_b for the
// 16-value sub-scales), summed over the block, then times d / den of the row.
constexpr int kGenRowStride = 144;  // LDS bytes per staged block-row: 2 + 128 copied, 16-byte multiple

template <int TYPE>
__device__ __forceinline__ void gen_row_scales(const uint8_t* rowp, int u, int& la, int& lb) {
  if constexpr (TYPE == kIQ2_XXS) {
    la = lb = 2 * (int)(ld32(rowp + 6 + 8 * u) >> 28) + 1;
  } else if constexpr (TYPE == kIQ3_XXS) {
    la = lb = 2 * (int)(ld32(rowp + 66 + 4 * u) >> 28) + 1;
  } else {
    const uint32_t sc = rowp[(TYPE == kIQ2_XS ? 66 : 74) + u];
    la = 2 * (int)(sc & 0xF) + 1;
    lb = 2 * (int)(sc >> 4) + 1;
  }
}

// PK (IQ3_XXS only): W in the build's IQ3_XXS unit layout (iq3_tile.h). Lane 16u + 8rp + s loads
// unit u's QS 16 B, AUX 8 B and D 4 B of block b's lanes 8 (2 bi + rp) + s (rows 2rp, 2rp+1,
// slice s: each field contiguous across the 16 lanes of a unit) and writes them to the staged
// rows 4u + 2rp, 4u + 2rp + 1 as the GGUF block, at byte 2 of each (the fields are then at the
// same places as in the GGUF path: d at 2, the slice's indices at 4 + 8s, its sign / scale word at
// 68 + 4s).
// Up to three column tiles the kernel is held to two workgroups per CU (256 registers per lane):
// IQ2_S at three column tiles otherwise takes 271 and runs alone on its CU; squeezed it spills 3
// dwords and its 48-row op at 17408 x 5120 goes from 81.8 to 56.3 us (IQ2_XS 58.6 -> 55.0,
// IQ3_XXS at 16 rows 30.8 -> 28.8). IQ3_XXS at two column tiles is held to three per CU (172 ->
// 168 registers, 4 dwords spilled): 17408 x 5120 M = 24 / 32 43.8 / 43.5 -> 40.2 / 39.6 us, at a
// cost of 0.4-0.6 us on 5120 x 17408 and 6144 x 5120 (45.5 -> 45.9, 19.5 -> 20.0 at M = 32).
template <int TYPE, int NT, int KS, bool PK = false>
__global__ void __launch_bounds__(64 * KS, NT == 2 && TYPE == kIQ3_XXS ? 3 : NT <= 3 ? 2 : 1) gemm_generic_kernel(const uint8_t* __restrict__ W, int64_t row_bytes,
                                                               int nrows, int k, const uint8_t* __restrict__ xq,
                                                               int nct, int n, void* __restrict__ y, int y_dtype) {
  constexpr int BS = block_bytes(TYPE);
  constexpr bool P16 = per16_type(TYPE);
  __shared__ typename Codebook<TYPE>::T grid[Codebook<TYPE>::n];
  __shared__ uint4 stage[KS][2][16 * kGenRowStride / 16];
  __shared__ float red[KS > 1 ? KS - 1 : 1][NT][4][64];
  stage_codebook<TYPE>(grid);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int row0 = blockIdx.x * kRawRows;
  const int rows_here = nrows - row0 < kRawRows ? nrows - row0 : kRawRows;
  const int ct0 = blockIdx.y * NT;
  const int nb = k / kQK;
  const int b_begin = wave * nb / KS, b_end = (wave + 1) * nb / KS;
  // rows past nrows, and the copy's read past the tile's last block-row, lie past the
  // descriptor's size and read zeros: the block's byte offset goes into the lane offset, which
  // the hardware range check covers (a scalar offset is not checked)
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(W + (int64_t)row0 * row_bytes, (uint32_t)(rows_here * row_bytes));
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(xq, (uint32_t)xq_bytes((int64_t)nct * kXqCols, k));
  const int sbase = (int)xq_scale_base(nct, nb);
  const int copy_off = (lane >> 2) * (int)row_bytes + 32 * (lane & 3);  // lane's 32 bytes of its row
  int units[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) units[t] = (ct0 + t < nct ? ct0 + t : nct - 1) * nb;
  uint8_t* buf0 = (uint8_t*)stage[wave][0];
  uint8_t* buf1 = (uint8_t*)stage[wave][1];

  float acc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t][v] = 0.0f;

  static_assert(!PK || TYPE == kIQ3_XXS, "the packed layout is IQ3_XXS's");
  const int pu = lane >> 4, prp = (lane >> 3) & 1, ps = lane & 7;  // PK: unit, row pair, slice
  const int pk_off = pu * 4 * (int)row_bytes + 16 * (8 * prp + ps);
  auto load_rows = [&](int b, u32x4 (&r)[2]) {
    const int bb = b < b_end ? b : b_end - 1;  // past the wave's range: re-read its last block
    if constexpr (PK) {
      const XxsFields f = xxs_block_fields(nb, bb);
      r[0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, pk_off + (int)f.qs, 0, 0);
      const auto a = __builtin_amdgcn_raw_buffer_load_b64(wrs, pu * 4 * (int)row_bytes + (int)f.aux + 8 * (8 * prp + ps),
                                                         0, 0);
      const uint32_t d = __builtin_amdgcn_raw_buffer_load_b32(wrs, pu * 4 * (int)row_bytes + (int)f.d + 4 * prp, 0, 0);
      r[1] = u32x4{a[0], a[1], d, 0u};
    } else {
      const int bo = (bb * BS) & ~3;
      r[0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, copy_off + bo, 0, 0);
      r[1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, copy_off + bo + 16, 0, 0);
    }
  };
  // the block lands at byte 2 of its staged row whatever its alignment in W, so that its 4-byte
  // fields (at 2 mod 4 in every format here) are aligned LDS words
  auto store_rows = [&](uint8_t* buf, int b, const u32x4 (&r)[2]) {
    if constexpr (PK) {
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        uint8_t* row = buf + 2 + (4 * pu + 2 * prp + rr) * kGenRowStride;
        *(uint32_t*)(row + 2 + 8 * ps) = r[0][2 * rr];
        *(uint32_t*)(row + 6 + 8 * ps) = r[0][2 * rr + 1];
        *(uint32_t*)(row + 66 + 4 * ps) = r[1][rr];
        *(uint16_t*)row = (uint16_t)(r[1][2] >> (16 * rr));  // the 8 lanes of a row pair write the same d
      }
    } else {
      const int bb = b < b_end ? b : b_end - 1;
      uint4* d = (uint4*)(buf + 2 - ((bb * BS) & 3) + (lane >> 2) * kGenRowStride + 32 * (lane & 3));
      d[0] = make_uint4(r[0][0], r[0][1], r[0][2], r[0][3]);
      d[1] = make_uint4(r[1][0], r[1][1], r[1][2], r[1][3]);
    }
  };
  auto compute = [&](const uint8_t* buf0_, int b, const XRawFrag<NT>& x) {
    const uint8_t* buf = buf0_ + 2;  // the block's first byte in each staged row
    float accb[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) accb[t][v] = 0.0f;
    const uint8_t* rowj = buf + j * kGenRowStride;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int wa[2];
      SliceScale sc;
      decode_quarter<TYPE>(rowj, u, q, grid, wa, sc);
      const long a = (long)(((uint64_t)(uint32_t)wa[1] << 32) | (uint32_t)wa[0]);
      int la[4], lb[4];  // sub-scales of the C rows 4q + v
#pragma unroll
      for (int v = 0; v < 4; ++v) gen_row_scales<TYPE>(buf + (4 * q + v) * kGenRowStride, u, la[v], lb[v]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const long bq = xq_b_operand(x.b[t][u >> 1], u & 1);
        const float cd = __uint_as_float(x.d[t][u >> 2][u & 3]);
        const v4i zero = {0, 0, 0, 0};
        if constexpr (P16) {
          const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(q < 2 ? a : 0, bq, zero, 0, 0, 0);
          const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(q < 2 ? 0 : a, bq, zero, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 4; ++v)
            accb[t][v] = fmaf((float)(__mul24(c0[v], la[v]) + __mul24(c1[v], lb[v])), cd, accb[t][v]);
        } else {
          const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq, zero, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 4; ++v) accb[t][v] = fmaf((float)__mul24(c[v], la[v]), cd, accb[t][v]);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float dd = half_bits_to_float(ld16(buf + (4 * q + v) * kGenRowStride)) * (1.0f / (float)iq_den(TYPE));
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t][v] = fmaf(accb[t][v], dd, acc[t][v]);
    }
  };

  const int nblk = b_end - b_begin;
  u32x4 ra[2], rb[2];
  XRawFrag<NT> xa, xb;
  if (nblk > 0) {
    load_rows(b_begin, ra);
    load_xraw<NT>(xrs, units, b_begin, sbase, lane, j, xa);
  }
  __syncthreads();  // the codebook
  if (nblk > 0) {
    store_rows(buf0, b_begin, ra);
    load_rows(b_begin + 1, rb);
  }
  // block b is in buf[(b - b_begin) & 1] with its X in xa / xb; the next block's rows are in
  // flight in rb / ra; a wave's LDS accesses complete in issue order, so each buffer's reads
  // come before it is rewritten
  int b = b_begin;
  for (int it = 0; it < nblk / 2; ++it, b += 2) {
    load_xraw<NT>(xrs, units, b + 1 < b_end ? b + 1 : b_end - 1, sbase, lane, j, xb);
    __builtin_amdgcn_sched_barrier(0);
    compute(buf0, b, xa);
    store_rows(buf1, b + 1, rb);
    load_rows(b + 2, ra);
    load_xraw<NT>(xrs, units, b + 2 < b_end ? b + 2 : b_end - 1, sbase, lane, j, xa);
    __builtin_amdgcn_sched_barrier(0);
    compute(buf1, b + 1, xb);
    store_rows(buf0, b + 2, ra);
    load_rows(b + 3, rb);
  }
  if (nblk & 1) compute(buf0, b, xa);

  if constexpr (KS > 1) {
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[wave - 1][t][v][lane] = acc[t][v];
    }
    __syncthreads();
  }
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = (ct0 + t) * kXqCols + j;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float sum = acc[t][v];
        for (int w2 = 1; w2 < KS; ++w2) sum += red[w2 - 1][t][v][lane];
        const int row = 4 * q + v;
        if (col < n && row < rows_here) store_y(y, (int64_t)col * nrows + row0 + row, sum, y_dtype);
      }
    }
  }
}

template <int TYPE, int NT, bool PK = false>
void launch_generic_t(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n, void* y,
                      int y_dtype, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const dim3 grid((unsigned)((nrows + kRawRows - 1) / kRawRows), (unsigned)((nct + NT - 1) / NT));
  gemm_generic_kernel<TYPE, NT, 4, PK><<<grid, 256, 0, stream>>>(W, row_bytes, nrows, k, xq, nct, n, y, y_dtype);
}

template <int TYPE, bool PK = false>
void launch_generic_type(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n, void* y,
                         int y_dtype, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  if (nct == 1) launch_generic_t<TYPE, 1, PK>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream);
  else if (nct == 2) launch_generic_t<TYPE, 2, PK>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream);
  else if (nct == 3) launch_generic_t<TYPE, 3, PK>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream);
  else launch_generic_t<TYPE, 4, PK>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream);
}

template <int TYPE, int NT, int KS, bool SX>
void launch_raw_t(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n, void* y,
                  int y_dtype, int split, float* part, uint32_t* cnt, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const dim3 grid((unsigned)((nrows + kRawRows - 1) / kRawRows), (unsigned)((nct + NT - 1) / NT), (unsigned)split);
  gemm_raw_kernel<TYPE, NT, KS, SX><<<grid, 64 * KS, 0, stream>>>(W, row_bytes, nrows, k, xq, nct, n, y, y_dtype, part,
                                                                  cnt);
}

template <int TYPE, bool SX = false>
void launch_raw_type(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n, void* y,
                     int y_dtype, int split, float* part, uint32_t* cnt, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  if (nct == 1) launch_raw_t<TYPE, 1, kRawWaves, SX>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
  else if (nct == 2) launch_raw_t<TYPE, 2, kRawWaves, SX>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
  else if (nct == 3) {
    // Q4_K / Q6_K unsplit on fewer than two tiles per CU: groups of two column tiles (2 + 1), at
    // two workgroups per CU instead of one workgroup of three alone on its CU (263-354
    // registers). Measured on the op, M = 40 / 48: Q4_K 6144 x 5120 29.0 / 28.5 -> 25.7 / 25.2
    // us, 5120 x 6144 32.6 / 32.1 -> 30.1 / 29.5; Q6_K 6144 x 5120 34.2 / 33.7 -> 31.4 / 31.1.
    // On 768 tiles (12288 x 5120) it lost (Q4_K 41.9 -> 43.5, Q6_K 49.8 -> 53.9 at M = 48), and
    // IQ4_XS, whose three-tile workgroups already share a CU, lost everywhere (26.5 -> 27.1,
    // 37.2 -> 46.3).
    const bool pairs = TYPE != kIQ4_XS && split == 1 && (nrows + kRawRows - 1) / kRawRows < 2 * device_cus();
    if (pairs) launch_raw_t<TYPE, 2, kRawWaves, SX>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
    else launch_raw_t<TYPE, 3, kRawWaves, SX>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
  }
  else launch_raw_t<TYPE, 4, kRawWaves, SX>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
}

bool raw_type(int type) { return type == kQ4_K || type == kIQ4_XS || type == kQ6_K; }

}  // namespace

// The raw GEMM's K split over workgroups (1: none; split_k.h), for grids of fewer than two (tile,
// column group) workgroups per CU. From 3 column tiles a workgroup holds a CU alone (up to 256
// VGPRs per lane), so G of them run in ceil(G / CUs) rounds, and split s over K they take
// ceil(G s / CUs) rounds of 1/s the work; with fewer column tiles 2-3 workgroups share a CU and
// the same count still picks the measured best. s in {2, 4} is taken where that time drops, the
// smaller s on a tie; each wave keeps 3 blocks of its split (4 from 3 column tiles: the fixed
// costs of a workgroup outweigh fewer), or 1 where the time at least halves (most CUs idle
// otherwise). Measured on the op (quantise included, graph replayed), no split -> split: IQ4_XS
// 5120 x 17408 (320 tiles, s = 4) M = 16 / 32 / 48: 38.1 -> 30.4 / 50.2 -> 41.1 / 65.9 -> 52.8
// us; Q6_K 5120 x 6144 (s = 2) M = 16 / 32: 22.2 -> 19.2 / 28.3 -> 23.7; Q6_K 1024 x 5120 (64
// tiles, s = 4) M = 16: 11.7 -> 9.8. Left unsplit: 256 workgroups (one round either way: 4096 x
// 4096 IQ4_XS M = 8 11.2 -> 13.0 with s = 2), 20-block K at 320 or 384 tiles (Q4_K 5120 x 5120
// M = 48 27.0 -> 31.0), 24 blocks at 3 column tiles (Q6_K 5120 x 6144 M = 48 37.1 -> 37.8).
int raw_split(int type, int64_t nrows, int64_t k, int64_t n) {
  if (!raw_type(type) || n <= 0) return 1;
  const int64_t tiles = (nrows + kRawRows - 1) / kRawRows, nb = k / kQK, cus = device_cus();
  // Q4_K at three column tiles on fewer than two tiles per CU: unsplit, in two-column-tile groups
  // (launch_raw_type), which beat the split (M = 40 / 48: 5120 x 17408 69.0 / 68.3 -> 64.6 / 63.5
  // us, 2048 x 5120 14.5 / 14.3 -> 13.0 / 12.8); for Q6_K the split stays faster (5120 x 17408
  // 80.7 against 85.1 at M = 48)
  if (type == kQ4_K && xq_col_tiles(n) == 3 && tiles < 2 * cus) return 1;
  const int64_t groups = split_groups(tiles, n);
  if (groups >= 2 * cus) return 1;
  // time in quarter workgroup-times
  auto quarters = [&](int64_t s) { return (groups * s + cus - 1) / cus * 4 / s; };
  int best = 1;
  int64_t best_t = quarters(1);
  const int64_t per_wave = split_nt(n) >= 3 ? 4 : 3;
  for (int s = 2; s <= kMaxSplit; s *= 2) {
    const int64_t t = quarters(s);
    const int64_t min_blocks = 2 * t <= quarters(1) ? kRawWaves : per_wave * kRawWaves;
    if (t < best_t && nb / s >= min_blocks) best = s, best_t = t;
  }
  // IQ4_XS at three column tiles (whose workgroups share a CU two by two) on fewer than two tiles
  // per CU: two ways where the rule above leaves it unsplit (M = 40 / 48: 5120 x 6144 31.0 / 30.6
  // -> 26.4 / 25.8 us, 6144 x 5120 26.5 / 26.5 -> 26.1 / 25.7); Q6_K lost with it (30.9 -> 37.6)
  if (best == 1 && type == kIQ4_XS && split_nt(n) == 3 && tiles < 2 * cus && nb >= 2 * kRawWaves) return 2;
  return best;
}

// Q4_K / IQ4_XS / Q6_K rows; xq: X in the xq layout (launch_quantize_xq). mmq: X quantised with
// the product ops' MMQ arithmetic (for Q4_K the scale words then carry the fp16 sum of x).
// split_ws: the split's workspace (split_k.h) when raw_split(...) > 1, its counters zeroed
// (unused otherwise).
hipError_t launch_gemm_xq(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n,
                          void* y, int y_dtype, bool mmq, void* split_ws, hipStream_t stream) {
  const int split = raw_split(type, nrows, k, n);
  float* part = (float*)split_ws;
  uint32_t* cnt =
      (uint32_t*)((uint8_t*)split_ws + split_part_bytes(split, (nrows + kRawRows - 1) / kRawRows, n));
  if (split > 1 && split_ws == nullptr) return hipErrorInvalidValue;
  switch (type) {
    case kQ4_K:
      if (mmq) launch_raw_type<kQ4_K, true>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
      else launch_raw_type<kQ4_K, false>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
      break;
    case kIQ4_XS: launch_raw_type<kIQ4_XS>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream); break;
    case kQ6_K: launch_raw_type<kQ6_K>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream); break;
    case kIQ2_XXS: launch_generic_type<kIQ2_XXS>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream); break;
    case kIQ2_XS: launch_generic_type<kIQ2_XS>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream); break;
    case kIQ2_S: launch_generic_type<kIQ2_S>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream); break;
    case kIQ3_XXS: launch_generic_type<kIQ3_XXS>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// IQ3_XXS in the build's unit layout (rows % 16 == 0), the product ops' MMQ arithmetic; xq: X in
// the xq layout
hipError_t launch_gemm_iq3xxs_packed(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n,
                                     void* y, int y_dtype, hipStream_t stream) {
  if (nrows % kRawRows != 0) return hipErrorInvalidValue;
  launch_generic_type<kIQ3_XXS, true>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream);
  return hipGetLastError();
}

}  // namespace gguf
