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
//   Q2_K  : value = d * sc_h * w - dmin * m_h, w = 2-bit quant, sc_h, m_h per 16 values
//   IQ2_XXS, IQ3_XXS: value = d * ls * w / den, ls = 2 * nibble + 1 per 32 values, den = 8 (IQ2),
//           4 (IQ3_XXS), w = signed grid byte
//   IQ2_XS, IQ2_S, IQ1_M: value = d * ls_h * w / 8, ls_h = 2 * scale + 1 per 16 values;
//           IQ1_M's w = 8 * grid +- 1 (grid in {-1, 0, 1}, the +-1/8 delta folded in)
// The /den forms are the gguf-py dequant's d * (0.5 + s) * 0.25 (or * 0.5) and d * (2s + 1) *
// (grid +- 0.125) with the fractions moved into one power-of-two factor, so every slice dot
// stays an exact integer.
// Byte offsets inside a block are the format's (ggml-common.h block structs, see gguf_common.h).
#pragma once

#include "gguf_common.h"

namespace gguf {

struct SliceScale {
  float d;     // the block's fp16 d
  float dmin;  // Q4_K, Q2_K
  int ls;      // IQ sub-scale; Q4_K sc; Q6_K / Q2_K / per-16 IQ: first 16-value scale
  int ls2;     // Q4_K m; Q6_K / Q2_K / per-16 IQ: second 16-value scale
  int m, m2;   // Q2_K: the two 16-value mins
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

// ---------------------------------------------------------------------------------- IQ2 / IQ3_XXS / IQ1_M
// These decoders report the block's fp16 d in s.d; the value is d * ls * w / iq_den(type).
__host__ __device__ constexpr int iq_den(int type) {
  return type == kIQ3_XXS ? 4 : (type == kIQ2_XXS || type == kIQ2_XS || type == kIQ2_S || type == kIQ1_M) ? 8 : 1;
}

// ksigns_iq2xs: 7 sign bits and an eighth that makes the byte's parity even
__device__ __forceinline__ uint32_t ksigns8(uint32_t s7) { return s7 | ((__builtin_popcount(s7) & 1u) << 7); }

// the 8 bytes of a grid entry, the bytes flagged in signs (bit j: byte j) negated
__device__ __forceinline__ void signed_grid8(uint64_t g, uint32_t signs, int& w0, int& w1) {
  w0 = apply_signs((uint32_t)g, signs & 0xFu);
  w1 = apply_signs((uint32_t)(g >> 32), (signs >> 4) & 0xFu);
}

// block_iq2_xxs: d[0:2], per slice u 8 bytes at 2 + 8u: four grid indices, then a dword of four
// 7-bit sign indices (bits 7g) and the scale (bits 28..31)
__device__ __forceinline__ void decode_iq2xxs(const uint8_t* b, int u, const uint64_t* grid, int (&w)[8],
                                              SliceScale& s) {
  const uint32_t idx = ld32(b + 2 + 8 * u), aux = ld32(b + 6 + 8 * u);
#pragma unroll
  for (int g = 0; g < 4; ++g)
    signed_grid8(grid[(idx >> (8 * g)) & 0xFF], ksigns8((aux >> (7 * g)) & 127), w[2 * g], w[2 * g + 1]);
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)(aux >> 28) + 1;
}

__device__ __forceinline__ void decode_iq2xxs_q(const uint8_t* b, int u, int q, const uint64_t* grid, int (&w)[2],
                                                SliceScale& s) {
  const uint32_t aux = ld32(b + 6 + 8 * u);
  signed_grid8(grid[b[2 + 8 * u + q]], ksigns8((aux >> (7 * q)) & 127), w[0], w[1]);
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)(aux >> 28) + 1;
}

// block_iq2_xs: d[0:2], qs[2:66] 32 uint16 (9-bit grid index | 7-bit sign index << 9),
// scales[66:74] (slice u: low nibble values 0..15, high nibble 16..31)
__device__ __forceinline__ void decode_iq2xs(const uint8_t* b, int u, const uint64_t* grid, int (&w)[8],
                                             SliceScale& s) {
  const uint64_t q = ld64(b + 2 + 8 * u);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t v = (uint32_t)(q >> (16 * g)) & 0xFFFF;
    signed_grid8(grid[v & 511], ksigns8(v >> 9), w[2 * g], w[2 * g + 1]);
  }
  const uint32_t sc = b[66 + u];
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)(sc & 0xF) + 1;
  s.ls2 = 2 * (int)(sc >> 4) + 1;
}

__device__ __forceinline__ void decode_iq2xs_q(const uint8_t* b, int u, int q, const uint64_t* grid, int (&w)[2],
                                               SliceScale& s) {
  const uint32_t v = ld16(b + 2 + 8 * u + 2 * q);
  signed_grid8(grid[v & 511], ksigns8(v >> 9), w[0], w[1]);
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)((b[66 + u] >> (4 * (q >> 1))) & 0xF) + 1;  // the 16-value half of values 8q..8q+7
}

// block_iq2_s: d[0:2], qs[2:34] grid index low bytes, signs[34:66] (one byte per 8 values),
// qh[66:74] (index bits 8, 9 of group g at bits 2g), scales[74:82]
__device__ __forceinline__ void decode_iq2s(const uint8_t* b, int u, const uint64_t* grid, int (&w)[8], SliceScale& s) {
  const uint32_t lo = ld32(b + 2 + 4 * u), sg = ld32(b + 34 + 4 * u), qh = b[66 + u];
#pragma unroll
  for (int g = 0; g < 4; ++g)
    signed_grid8(grid[((lo >> (8 * g)) & 0xFF) | (((qh >> (2 * g)) & 3u) << 8)], (sg >> (8 * g)) & 0xFF, w[2 * g],
                 w[2 * g + 1]);
  const uint32_t sc = b[74 + u];
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)(sc & 0xF) + 1;
  s.ls2 = 2 * (int)(sc >> 4) + 1;
}

__device__ __forceinline__ void decode_iq2s_q(const uint8_t* b, int u, int q, const uint64_t* grid, int (&w)[2],
                                              SliceScale& s) {
  const uint32_t idx = b[2 + 4 * u + q] | (((uint32_t)(b[66 + u] >> (2 * q)) & 3u) << 8);
  signed_grid8(grid[idx], b[34 + 4 * u + q], w[0], w[1]);
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)((b[74 + u] >> (4 * (q >> 1))) & 0xF) + 1;
}

// block_iq3_xxs: d[0:2], qs[2:66] grid indices (one per 4 values), then per slice u a dword at
// 66 + 4u: four 7-bit sign indices (one per 8 values) and the scale (bits 28..31). grid: the
// signed table (kIq3xxsSigned), indexed by grid index | sign nibble << 8.
__device__ __forceinline__ void iq3xxs_words(uint32_t q2, uint32_t aux, int g, const uint32_t* grid, int& w0,
                                             int& w1) {  // q2: the two grid indices of group g
  const uint32_t sg = ksigns8((aux >> (7 * g)) & 127);
  w0 = (int)grid[(q2 & 0xFF) | ((sg & 0xF) << 8)];
  w1 = (int)grid[((q2 >> 8) & 0xFF) | ((sg >> 4) << 8)];
}

__device__ __forceinline__ void decode_iq3xxs(const uint8_t* b, int u, const uint32_t* grid, int (&w)[8],
                                              SliceScale& s) {
  const uint64_t qi = ld64(b + 2 + 8 * u);
  const uint32_t aux = ld32(b + 66 + 4 * u);
#pragma unroll
  for (int g = 0; g < 4; ++g) iq3xxs_words((uint32_t)(qi >> (16 * g)), aux, g, grid, w[2 * g], w[2 * g + 1]);
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)(aux >> 28) + 1;
}

__device__ __forceinline__ void decode_iq3xxs_q(const uint8_t* b, int u, int q, const uint32_t* grid, int (&w)[2],
                                                SliceScale& s) {
  const uint32_t aux = ld32(b + 66 + 4 * u);
  iq3xxs_words(ld16(b + 2 + 8 * u + 2 * q), aux, q, grid, w[0], w[1]);
  s.d = half_bits_to_float(ld16(b));
  s.ls = 2 * (int)(aux >> 28) + 1;
}

// block_iq1_m: qs[0:32] grid index low bytes (one per 8 values), qh[32:48] (a nibble per group:
// index bits 8..10 and, in bit 3, the delta's sign), scales[48:56] as 4 uint16 holding the
// 3-bit scale of every 16 values in bits 0..11 and the fp16 d in the four top nibbles. The grid
// digits (value + 1, kIq1sNib) go through a byte permute to 8 * value + 1 (delta +) or
// 8 * value - 1 (delta -).
__device__ __forceinline__ float iq1m_d(const uint8_t* b) {
  const uint64_t sc = ld64(b + 48);
  const uint32_t s0 = (uint32_t)sc & 0xFFFF, s1 = (uint32_t)(sc >> 16) & 0xFFFF, s2 = (uint32_t)(sc >> 32) & 0xFFFF,
                 s3 = (uint32_t)(sc >> 48);
  return half_bits_to_float((s0 >> 12) | ((s1 >> 8) & 0xF0) | ((s2 >> 4) & 0xF00) | (s3 & 0xF000));
}

__device__ __forceinline__ int iq1m_scale(const uint8_t* b, int h) {  // h: 16-value group 0..15
  return (int)((ld16(b + 48 + 2 * (h >> 2)) >> (3 * (h & 3))) & 7);
}

__device__ __forceinline__ void iq1m_group(const uint8_t* b, int grp, const uint32_t* grid, int& w0, int& w1) {
  const uint32_t nib = (b[32 + (grp >> 1)] >> (4 * (grp & 1))) & 0xF;
  const uint32_t g = grid[b[grp] | ((nib & 7) << 8)];
  const uint32_t t = (nib & 8) ? 0x0007FFF7u : 0x000901F9u;  // bytes 0, 1, 2: digit 0 (-1), 1 (0), 2 (+1)
  w0 = (int)__builtin_amdgcn_perm(t, t, g & 0x0F0F0F0Fu);
  w1 = (int)__builtin_amdgcn_perm(t, t, (g >> 4) & 0x0F0F0F0Fu);
}

__device__ __forceinline__ void decode_iq1m(const uint8_t* b, int u, const uint32_t* grid, int (&w)[8],
                                            SliceScale& s) {
#pragma unroll
  for (int g = 0; g < 4; ++g) iq1m_group(b, 4 * u + g, grid, w[2 * g], w[2 * g + 1]);
  s.d = iq1m_d(b);
  s.ls = 2 * iq1m_scale(b, 2 * u) + 1;
  s.ls2 = 2 * iq1m_scale(b, 2 * u + 1) + 1;
}

__device__ __forceinline__ void decode_iq1m_q(const uint8_t* b, int u, int q, const uint32_t* grid, int (&w)[2],
                                              SliceScale& s) {
  iq1m_group(b, 4 * u + q, grid, w[0], w[1]);
  s.d = iq1m_d(b);
  s.ls = 2 * iq1m_scale(b, 2 * u + (q >> 1)) + 1;
}

// ---------------------------------------------------------------------------------- Q2_K
// block_q2_K: scales[0:16] (low nibble scale, high nibble min, per 16 values), qs[16:80],
// d[80:82], dmin[82:84]; value 128n + 32j + l is bits 2j of qs[32n + l]
__device__ __forceinline__ void decode_q2k(const uint8_t* b, int u, int (&w)[8], SliceScale& s) {
  const uint8_t* qs = b + 16 + 32 * (u >> 2);
  const int sh = 2 * (u & 3);
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = (int)((ld32(qs + 4 * e) >> sh) & 0x03030303u);
  const uint32_t dm = ld32(b + 80), sc = ld16(b + 2 * u);
  s.d = half_bits_to_float(dm & 0xFFFF);
  s.dmin = half_bits_to_float(dm >> 16);
  s.ls = (int)(sc & 0xF);
  s.m = (int)((sc >> 4) & 0xF);
  s.ls2 = (int)((sc >> 8) & 0xF);
  s.m2 = (int)(sc >> 12);
}

__device__ __forceinline__ void decode_q2k_q(const uint8_t* b, int u, int q, int (&w)[2], SliceScale& s) {
  const uint64_t v = ld64(b + 16 + 32 * (u >> 2) + 8 * q);
  const int sh = 2 * (u & 3);
  w[0] = (int)(((uint32_t)v >> sh) & 0x03030303u);
  w[1] = (int)(((uint32_t)(v >> 32) >> sh) & 0x03030303u);
  const uint32_t dm = ld32(b + 80), sc = b[2 * u + (q >> 1)];
  s.d = half_bits_to_float(dm & 0xFFFF);
  s.dmin = half_bits_to_float(dm >> 16);
  s.ls = (int)(sc & 0xF);
  s.m = (int)(sc >> 4);
}

// ---------------------------------------------------------------------------------- dispatch
// The codebook a type's decoder reads, staged in LDS by the kernels: entries and entry word.
template <int TYPE>
struct Codebook {
  static constexpr int n = 1;  // no codebook
  using T = uint32_t;
  static __device__ T at(int) { return 0; }
};
template <>
struct Codebook<kIQ3_S> {
  static constexpr int n = 512;
  using T = uint32_t;
  static __device__ T at(int i) { return kIq3sGrid.v[i]; }
};
template <>
struct Codebook<kIQ3_XXS> {
  static constexpr int n = 4096;  // the signed table
  using T = uint32_t;
  static __device__ T at(int i) { return kIq3xxsSigned.v[i]; }
};
template <>
struct Codebook<kIQ2_XXS> {
  static constexpr int n = 256;
  using T = uint64_t;
  static __device__ T at(int i) { return kIq2xxsGrid.v[i]; }
};
template <>
struct Codebook<kIQ2_XS> {
  static constexpr int n = 512;
  using T = uint64_t;
  static __device__ T at(int i) { return kIq2xsGrid.v[i]; }
};
template <>
struct Codebook<kIQ2_S> {
  static constexpr int n = 1024;
  using T = uint64_t;
  static __device__ T at(int i) { return kIq2sGrid.v[i]; }
};
template <>
struct Codebook<kIQ1_M> {
  static constexpr int n = 2048;
  using T = uint32_t;
  static __device__ T at(int i) { return kIq1sNib.v[i]; }
};

// Copies TYPE's codebook into `lds` with the workgroup's threads (the caller synchronises).
template <int TYPE>
__device__ __forceinline__ void stage_codebook(typename Codebook<TYPE>::T* lds) {
  if constexpr (Codebook<TYPE>::n > 1)
    for (int i = threadIdx.x; i < Codebook<TYPE>::n; i += blockDim.x) lds[i] = Codebook<TYPE>::at(i);
}

// the 32 values of slice u of block b
template <int TYPE>
__device__ __forceinline__ void decode_slice(const uint8_t* b, int u, const typename Codebook<TYPE>::T* grid,
                                             int (&w)[8], SliceScale& s) {
  if constexpr (TYPE == kIQ3_S) decode_iq3s(b, u, grid, w, s);
  if constexpr (TYPE == kQ4_K) decode_q4k(b, u, w, s);
  if constexpr (TYPE == kIQ4_XS) decode_iq4xs(b, u, w, s);
  if constexpr (TYPE == kQ6_K) decode_q6k(b, u, w, s);
  if constexpr (TYPE == kQ2_K) decode_q2k(b, u, w, s);
  if constexpr (TYPE == kIQ2_XXS) decode_iq2xxs(b, u, grid, w, s);
  if constexpr (TYPE == kIQ2_XS) decode_iq2xs(b, u, grid, w, s);
  if constexpr (TYPE == kIQ2_S) decode_iq2s(b, u, grid, w, s);
  if constexpr (TYPE == kIQ3_XXS) decode_iq3xxs(b, u, grid, w, s);
  if constexpr (TYPE == kIQ1_M) decode_iq1m(b, u, grid, w, s);
}

// values 8q..8q+7 of slice u of block b; s.ls is the sub-scale of their 16-value half where the
// type has one per 16 values
template <int TYPE>
__device__ __forceinline__ void decode_quarter(const uint8_t* b, int u, int q, const typename Codebook<TYPE>::T* grid,
                                               int (&w)[2], SliceScale& s) {
  if constexpr (TYPE == kIQ3_S) decode_iq3s_q(b, u, q, grid, w, s);
  if constexpr (TYPE == kQ4_K) decode_q4k_q(b, u, q, w, s);
  if constexpr (TYPE == kIQ4_XS) decode_iq4xs_q(b, u, q, w, s);
  if constexpr (TYPE == kQ6_K) decode_q6k_q(b, u, q, w, s);
  if constexpr (TYPE == kQ2_K) decode_q2k_q(b, u, q, w, s);
  if constexpr (TYPE == kIQ2_XXS) decode_iq2xxs_q(b, u, q, grid, w, s);
  if constexpr (TYPE == kIQ2_XS) decode_iq2xs_q(b, u, q, grid, w, s);
  if constexpr (TYPE == kIQ2_S) decode_iq2s_q(b, u, q, grid, w, s);
  if constexpr (TYPE == kIQ3_XXS) decode_iq3xxs_q(b, u, q, grid, w, s);
  if constexpr (TYPE == kIQ1_M) decode_iq1m_q(b, u, q, grid, w, s);
}

// types with a sub-scale per 16 values (two integer dots per slice)
__host__ __device__ constexpr bool per16_type(int type) {
  return type == kQ6_K || type == kQ2_K || type == kIQ2_XS || type == kIQ2_S || type == kIQ1_M;
}

// ---------------------------------------------------------------------------------- raw slices
// The bytes one lane needs to decode slice u of a block of the generic types, loaded by
// raw_load and decoded by raw_decode into the same words and scales as decode_slice: a GEMV can
// issue the next block's loads before it computes the current one.
template <int TYPE>
struct RawSlice;
template <>
struct RawSlice<kIQ2_XXS> {
  uint32_t d, idx, aux;
};
template <>
struct RawSlice<kIQ2_XS> {
  uint32_t d, sc;
  uint64_t q;
};
template <>
struct RawSlice<kIQ2_S> {
  uint32_t d, lo, sg, qh, sc;
};
template <>
struct RawSlice<kIQ3_XXS> {
  uint32_t d, aux;
  uint64_t qi;
};
template <>
struct RawSlice<kIQ1_M> {
  uint32_t qs, qh;
  uint64_t sc;
};
template <>
struct RawSlice<kQ2_K> {
  uint32_t q[8], sc, dm;
};

template <int TYPE>
__device__ __forceinline__ void raw_load(const uint8_t* b, int u, RawSlice<TYPE>& r) {
  if constexpr (TYPE == kIQ2_XXS) {
    r.d = ld16(b);
    r.idx = ld32(b + 2 + 8 * u);
    r.aux = ld32(b + 6 + 8 * u);
  } else if constexpr (TYPE == kIQ2_XS) {
    r.d = ld16(b);
    r.q = ld64(b + 2 + 8 * u);
    r.sc = b[66 + u];
  } else if constexpr (TYPE == kIQ2_S) {
    r.d = ld16(b);
    r.lo = ld32(b + 2 + 4 * u);
    r.sg = ld32(b + 34 + 4 * u);
    r.qh = b[66 + u];
    r.sc = b[74 + u];
  } else if constexpr (TYPE == kIQ3_XXS) {
    r.d = ld16(b);
    r.qi = ld64(b + 2 + 8 * u);
    r.aux = ld32(b + 66 + 4 * u);
  } else if constexpr (TYPE == kIQ1_M) {
    r.qs = ld32(b + 4 * u);
    r.qh = ld16(b + 32 + 2 * u);
    r.sc = ld64(b + 48);
  } else {
    const uint8_t* qs = b + 16 + 32 * (u >> 2);
#pragma unroll
    for (int e = 0; e < 8; ++e) r.q[e] = ld32(qs + 4 * e);
    r.sc = ld16(b + 2 * u);
    r.dm = ld32(b + 80);
  }
}

template <int TYPE>
__device__ __forceinline__ void raw_decode(const RawSlice<TYPE>& r, int u, const typename Codebook<TYPE>::T* grid,
                                           int (&w)[8], SliceScale& s) {
  if constexpr (TYPE == kIQ2_XXS) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      signed_grid8(grid[(r.idx >> (8 * g)) & 0xFF], ksigns8((r.aux >> (7 * g)) & 127), w[2 * g], w[2 * g + 1]);
    s.d = half_bits_to_float(r.d);
    s.ls = 2 * (int)(r.aux >> 28) + 1;
  } else if constexpr (TYPE == kIQ2_XS) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t v = (uint32_t)(r.q >> (16 * g)) & 0xFFFF;
      signed_grid8(grid[v & 511], ksigns8(v >> 9), w[2 * g], w[2 * g + 1]);
    }
    s.d = half_bits_to_float(r.d);
    s.ls = 2 * (int)(r.sc & 0xF) + 1;
    s.ls2 = 2 * (int)(r.sc >> 4) + 1;
  } else if constexpr (TYPE == kIQ2_S) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      signed_grid8(grid[((r.lo >> (8 * g)) & 0xFF) | (((r.qh >> (2 * g)) & 3u) << 8)], (r.sg >> (8 * g)) & 0xFF,
                   w[2 * g], w[2 * g + 1]);
    s.d = half_bits_to_float(r.d);
    s.ls = 2 * (int)(r.sc & 0xF) + 1;
    s.ls2 = 2 * (int)(r.sc >> 4) + 1;
  } else if constexpr (TYPE == kIQ3_XXS) {
#pragma unroll
    for (int g = 0; g < 4; ++g) iq3xxs_words((uint32_t)(r.qi >> (16 * g)), r.aux, g, grid, w[2 * g], w[2 * g + 1]);
    s.d = half_bits_to_float(r.d);
    s.ls = 2 * (int)(r.aux >> 28) + 1;
  } else if constexpr (TYPE == kIQ1_M) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t nib = (r.qh >> (4 * g)) & 0xF;
      const uint32_t e = grid[((r.qs >> (8 * g)) & 0xFF) | ((nib & 7) << 8)];
      const uint32_t t = (nib & 8) ? 0x0007FFF7u : 0x000901F9u;
      w[2 * g] = (int)__builtin_amdgcn_perm(t, t, e & 0x0F0F0F0Fu);
      w[2 * g + 1] = (int)__builtin_amdgcn_perm(t, t, (e >> 4) & 0x0F0F0F0Fu);
    }
    const uint32_t s0 = (uint32_t)r.sc & 0xFFFF, s1 = (uint32_t)(r.sc >> 16) & 0xFFFF,
                   s2 = (uint32_t)(r.sc >> 32) & 0xFFFF, s3 = (uint32_t)(r.sc >> 48);
    s.d = half_bits_to_float((s0 >> 12) | ((s1 >> 8) & 0xF0) | ((s2 >> 4) & 0xF00) | (s3 & 0xF000));
    const uint32_t sw = (uint32_t)(r.sc >> (16 * (u >> 1)));  // scales of 16-value groups 2u, 2u + 1
    s.ls = 2 * (int)((sw >> (6 * (u & 1))) & 7) + 1;
    s.ls2 = 2 * (int)((sw >> (6 * (u & 1) + 3)) & 7) + 1;
  } else {
    const int sh = 2 * (u & 3);
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = (int)((r.q[e] >> sh) & 0x03030303u);
    s.d = half_bits_to_float(r.dm & 0xFFFF);
    s.dmin = half_bits_to_float(r.dm >> 16);
    s.ls = (int)(r.sc & 0xF);
    s.m = (int)((r.sc >> 4) & 0xF);
    s.ls2 = (int)((r.sc >> 8) & 0xF);
    s.m2 = (int)(r.sc >> 12);
  }
}

}  // namespace gguf
