// The build's q8 activation layout for the int8-MFMA GEMMs ("xq"), an internal workspace format
// (the reference's block_q8_1_mmq, mmq.cuh:27-56, serves its CUDA mma fragments; the values and
// scales here are the same, only their placement differs).
//
// Activation rows are grouped in column tiles of 16 (the B-operand width of
// v_mfma_i32_16x16x32_i8); rows past n in the last tile are zero. For column tile t and 256-value
// K block b (nb = K / 256 blocks):
//   values  4096 B at ((t * nb + b) * 4096): lane l = 16q + j of a wave owns, for the block's
//           slices u = 0..7, the eight q8 values 32u + 8q .. 32u + 8q + 7 of activation row
//           16t + j, 8 bytes at 64l + 8u. One wave reads a (t, b) unit with four contiguous
//           16-byte loads per lane, and those bytes are the MFMA B operands of the 8 slices.
//   scales  512 B at nct * nb * 4096 + ((t * nb + b) * 16 + j) * 32: one dword per slice
//           u = 0..7 of activation row 16t + j: fp32 d, or for Q4_K weights fp16 d in the low half
//           and, above it, the activation side of Q4_K's min term: with the decode ops' q8_1
//           arithmetic the slice's int16 sum of q (times d: the MMVQ form, |sum| <= 4064, exact
//           in fp32), with the MMQ arithmetic the fp16 of the slice's sum of x (the half2 sum of
//           block_q8_1_mmq's DS4 layout, the MMQ form, vecdotq.cuh:549-552).
// Quantisation per 32-value slice is the reference's MMQ arithmetic (lcpp_shim.cu:298-355):
// d_inv = 127 / amax, q = roundf(x * d_inv), d = 1 / d_inv, and q = 0, d = 0 for an all-zero
// slice; for Q4_K d is stored as fp16 as in the reference's half2 (DS4) MMQ layout.
#pragma once

#include "gguf_common.h"

namespace gguf {

constexpr int kXqCols = 16;         // activation rows per column tile
constexpr int kXqUnit = 4096;       // value bytes per (column tile, K block)
constexpr int kXqScaleUnit = 512;   // scale bytes per (column tile, K block)

__host__ __device__ inline int64_t xq_col_tiles(int64_t n) { return (n + kXqCols - 1) / kXqCols; }

__host__ __device__ inline int64_t xq_scale_base(int64_t nct, int64_t nb) { return nct * nb * kXqUnit; }

__host__ __device__ inline size_t xq_bytes(int64_t n, int64_t k) {
  const int64_t nct = xq_col_tiles(n), nb = k / kQK;
  return (size_t)(nct * nb * (kXqUnit + kXqScaleUnit));
}

// The prefill GEMM's fp16 variant of the layout ("xh"): the same q8 values held as fp16 (exact),
// the same column tiles and K blocks. For column tile t and block b:
//   values  8192 B at ((t * nb + b) * 8192): slice u at 1024u, lane l = 16q + j of a wave owns 16
//           bytes at 1024u + 16l: the fp16 values 32u + 8q .. 32u + 8q + 7 of activation row
//           16t + j (the f16 MFMA B operand of the slice). Slices 4h..4h+3 are 4 KB contiguous.
//   scales  1024 B at nct * nb * 8192 + (t * nb + b) * 1024: fp32 d of (row j, slice u) at 32j + 4u
//           (a lane reads the 4 scales of its half block with one 16-byte load); for Q4_K
//           weights, d is the fp16-rounded scale, and 512 + 32j + 4u holds the fp16 sum of the
//           slice's x values widened to fp32 (DS4's half2 sum), the activation side of the min
//           term.
constexpr int kXhUnit = 8192;       // fp16 value bytes per (column tile, K block)
constexpr int kXhScaleUnit = 1024;  // scale bytes per (column tile, K block)

__host__ __device__ inline int64_t xh_scale_base(int64_t nct, int64_t nb) { return nct * nb * kXhUnit; }

__host__ __device__ inline size_t xh_bytes(int64_t n, int64_t k) {
  const int64_t nct = xq_col_tiles(n), nb = k / kQK;
  return (size_t)(nct * nb * (kXhUnit + kXhScaleUnit));
}

// MFMA B operand of slice 2i + h from the 16 bytes b[t][i] of a lane's xq unit
__device__ __forceinline__ long xq_b_operand(const u32x4& v, int h) {
  return h == 0 ? (long)(((uint64_t)v[1] << 32) | v[0]) : (long)(((uint64_t)v[3] << 32) | v[2]);
}

}  // namespace gguf
