// Per-slice decoders of GGUF super-blocks into signed int8 words, the integer form the dot4
// and MFMA kernels multiply with q8_1 activations.
//
// A "slice" is 32 consecutive values of a 256-value block (one q8_1 block of X). A decoder
// fills w[0..7] with the slice's values as int8x4 words in value order and reports the slice's
// scales so that, with sumi = sum(w * q8):
//   IQ3_S : value = d * ls * w           ls = 1 + 2*nibble         (vecdotq.cuh:1211-1248)
//   IQ4_XS: value = d * ls * w           ls = 6-bit scale - 32     (vecdotq.cuh:1357-1380)
//   Q4_K  : value = d * sc * w - dmin * m, w = 4-bit quant         (vecdotq.cuh:508-530)
//   Q6_K  : value = d * sc_h * w, sc_h int8 per 16 values          (vecdotq.cuh:627-648)
// Byte offsets inside a block are the format's (ggml-common.h block structs, see gguf_common.h).
#pragma once

#include "gguf_common.h"

namespace gguf {

struct SliceScale {
  float d;     // block scale (IQ3_S / IQ4_XS / Q6_K: d; Q4_K: d)
  float dmin;  // Q4_K only
  int ls;      // IQ3_S / IQ4_XS sub-scale; Q4_K sc; Q6_K first 16-value scale
  int ls2;     // Q4_K m; Q6_K second 16-value scale
};

// Q6_K bytes are 6-bit unsigned codes; bytewise q - 32 without borrows between bytes.
__device__ __forceinline__ int sub32_bytes(uint32_t v) {
  return (int)(((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
}

// ---------------------------------------------------------------------------------- IQ3_S
// block_iq3_s: d[0:2] qs[2:66] qh[66:74] signs[74:106] scales[106:110]. Group e (4 values) of
// slice u: grid index qs[8u+e] | bit e of qh[u] << 8, signs = nibble e of the slice's 4 sign bytes.
__device__ __forceinline__ void decode_iq3s(const uint8_t* b, int u, const uint32_t* grid, int (&w)[8],
                                            SliceScale& s) {
  const uint64_t qs = ld64(b + 2 + 8 * u);
  const uint32_t qh = b[66 + u];
  const uint32_t sg = ld32(b + 74 + 4 * u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t idx = (uint32_t)((qs >> (8 * e)) & 0xFF) | (((qh >> e) & 1u) << 8);
    w[e] = apply_signs(grid[idx], sg >> (4 * e));
  }
  s.d = half_bits_to_float(ld16(b));
  s.ls = 1 + 2 * ((b[106 + (u >> 1)] >> (4 * (u & 1))) & 0xF);
}

// groups 2q, 2q+1 only (values 8q..8q+7 of the slice)
__device__ __forceinline__ void decode_iq3s_q(const uint8_t* b, int u, int q, const uint32_t* grid, int (&w)[2],
                                              SliceScale& s) {
  const uint32_t qs = ld16(b + 2 + 8 * u + 2 * q);
  const uint32_t qh = b[66 + u] >> (2 * q);
  const uint32_t sg = b[74 + 4 * u + q];
  w[0] = apply_signs(grid[(qs & 0xFF) | ((qh & 1u) << 8)], sg);
  w[1] = apply_signs(grid[(qs >> 8) | ((qh & 2u) << 7)], sg >> 4);
  s.d = half_bits_to_float(ld16(b));
  s.ls = 1 + 2 * ((b[106 + (u >> 1)] >> (4 * (u & 1))) & 0xF);
}

// ---------------------------------------------------------------------------------- Q4_K
// block_q4_K: d[0:2] dmin[2:4] scales[4:16] qs[16:144]; qs[32j+l] holds value 64j+l (low
// nibble) and 64j+32+l (high nibble). 6-bit scale/min of sub-block u as get_scale_min_k4
// (csrc/gguf/dequantize.cuh:156-163).
__device__ __forceinline__ void q4k_scale_min(const uint8_t* b, int u, int& sc, int& m) {
  const uint32_t s0 = ld32(b + 4), s1 = ld32(b + 8), s2 = ld32(b + 12);
  const int j = u & 3;
  const uint32_t a = (s0 >> (8 * j)) & 0xFF;   // scales[j]
  const uint32_t c = (s1 >> (8 * j)) & 0xFF;   // scales[j + 4]
  const uint32_t e = (s2 >> (8 * j)) & 0xFF;   // scales[j + 8]
  if (u < 4) {
    sc = (int)(a & 63);
    m = (int)(c & 63);
  } else {
    sc = (int)((e & 0xF) | ((a >> 6) << 4));
    m = (int)((e >> 4) | ((c >> 6) << 4));
  }
}

__device__ __forceinline__ void decode_q4k(const uint8_t* b, int u, int (&w)[8], SliceScale& s) {
  const uint4 lo = *(const uint4*)(b + 16 + 32 * (u >> 1));
  const uint4 hi = *(const uint4*)(b + 32 + 32 * (u >> 1));
  const int sh = 4 * (u & 1);
  w[0] = (int)((lo.x >> sh) & 0x0F0F0F0Fu);
  w[1] = (int)((lo.y >> sh) & 0x0F0F0F0Fu);
  w[2] = (int)((lo.z >> sh) & 0x0F0F0F0Fu);
  w[3] = (int)((lo.w >> sh) & 0x0F0F0F0Fu);
  w[4] = (int)((hi.x >> sh) & 0x0F0F0F0Fu);
  w[5] = (int)((hi.y >> sh) & 0x0F0F0F0Fu);
  w[6] = (int)((hi.z >> sh) & 0x0F0F0F0Fu);
  w[7] = (int)((hi.w >> sh) & 0x0F0F0F0Fu);
  const uint32_t dm = ld32(b);
  s.d = half_bits_to_float(dm & 0xFFFF);
  s.dmin = half_bits_to_float(dm >> 16);
  q4k_scale_min(b, u, s.ls, s.ls2);
}

__device__ __forceinline__ void decode_q4k_q(const uint8_t* b, int u, int q, int (&w)[2], SliceScale& s) {
  const uint2 v = *(const uint2*)(b + 16 + 32 * (u >> 1) + 8 * q);
  const int sh = 4 * (u & 1);
  w[0] = (int)((v.x >> sh) & 0x0F0F0F0Fu);
  w[1] = (int)((v.y >> sh) & 0x0F0F0F0Fu);
  const uint32_t dm = ld32(b);
  s.d = half_bits_to_float(dm & 0xFFFF);
  s.dmin = half_bits_to_float(dm >> 16);
  q4k_scale_min(b, u, s.ls, s.ls2);
}

// ---------------------------------------------------------------------------------- IQ4_XS
// block_iq4_xs: d[0:2] scales_h[2:4] scales_l[4:8] qs[8:136]; slice u value j (< 16) is the low
// nibble of qs[16u+j], value 16+j the high nibble, mapped through kvalues_iq4nl.
__device__ __forceinline__ int iq4xs_ls(const uint8_t* b, int u) {
  const uint32_t sh = ld16(b + 2);
  return (int)(((b[4 + (u >> 1)] >> (4 * (u & 1))) & 0xF) | (((sh >> (2 * u)) & 3u) << 4)) - 32;
}

__device__ __forceinline__ void decode_iq4xs(const uint8_t* b, int u, int (&w)[8], SliceScale& s) {
  const uint64_t a = ld64(b + 8 + 16 * u), c = ld64(b + 16 + 16 * u);
  const uint32_t q[4] = {(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)c, (uint32_t)(c >> 32)};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w[j] = iq4nl(q[j], 0);
    w[4 + j] = iq4nl(q[j], 4);
  }
  s.d = half_bits_to_float(ld16(b));
  s.ls = iq4xs_ls(b, u);
}

__device__ __forceinline__ void decode_iq4xs_q(const uint8_t* b, int u, int q, int (&w)[2], SliceScale& s) {
  const uint64_t a = ld64(b + 8 + 16 * u + 8 * (q & 1));
  const int sh = 4 * (q >> 1);
  w[0] = iq4nl((uint32_t)a, sh);
  w[1] = iq4nl((uint32_t)(a >> 32), sh);
  s.d = half_bits_to_float(ld16(b));
  s.ls = iq4xs_ls(b, u);
}

// ---------------------------------------------------------------------------------- Q6_K
// block_q6_K: ql[0:128] qh[128:192] scales[192:208] d[208:210]. Value v of half h (128 each):
// low 4 bits from ql[64h + v%64] (nibble v/64), high 2 bits from qh[32h + v%32] (bits 2(v/32)).
__device__ __forceinline__ void decode_q6k(const uint8_t* b, int u, int (&w)[8], SliceScale& s) {
  const int h = u >> 2, uu = u & 3;
  const uint8_t* ql = b + 64 * h + 32 * (uu & 1);
  const uint8_t* qh = b + 128 + 32 * h;
  const int lsh = 4 * (uu >> 1), hsh = 2 * uu;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const uint64_t l = ld64(ql + 4 * i), hh = ld64(qh + 4 * i);
    const uint32_t l0 = (uint32_t)l, l1 = (uint32_t)(l >> 32);
    const uint32_t h0 = (uint32_t)hh, h1 = (uint32_t)(hh >> 32);
    w[i] = sub32_bytes(((l0 >> lsh) & 0x0F0F0F0Fu) | (((h0 >> hsh) & 0x03030303u) << 4));
    w[i + 1] = sub32_bytes(((l1 >> lsh) & 0x0F0F0F0Fu) | (((h1 >> hsh) & 0x03030303u) << 4));
  }
  s.d = half_bits_to_float(ld16(b + 208));
  s.ls = (int)(int8_t)b[192 + 2 * u];
  s.ls2 = (int)(int8_t)b[193 + 2 * u];
}

__device__ __forceinline__ void decode_q6k_q(const uint8_t* b, int u, int q, int (&w)[2], SliceScale& s) {
  const int h = u >> 2, uu = u & 3;
  const uint64_t l = ld64(b + 64 * h + 32 * (uu & 1) + 8 * q);
  const uint64_t hh = ld64(b + 128 + 32 * h + 8 * q);
  const int lsh = 4 * (uu >> 1), hsh = 2 * uu;
  w[0] = sub32_bytes((((uint32_t)l >> lsh) & 0x0F0F0F0Fu) | ((((uint32_t)hh >> hsh) & 0x03030303u) << 4));
  w[1] = sub32_bytes((((uint32_t)(l >> 32) >> lsh) & 0x0F0F0F0Fu) |
                     ((((uint32_t)(hh >> 32) >> hsh) & 0x03030303u) << 4));
  s.d = half_bits_to_float(ld16(b + 208));
  s.ls = (int)(int8_t)b[192 + 2 * u + (q >> 1)];  // values 8q..8q+7 lie in one 16-value half
  s.ls2 = 0;
}

}  // namespace gguf
