// fp16 decode of weight blocks for the fp16-operand MFMA GEMMs (the prefill GEMM's fp16 variant
// and the small GEMM): IQ3_S and IQ3_XXS in their unit layouts (iq3_tile.h), Q4_K and Q6_K rows,
// decoded to fp16
// values with the slice (Q6_K: 16-value) sub-scale applied (exact integers: at most 465 for
// IQ3_S, 945 for Q4_K; Q6_K's up to 4064 round above 2048), in the A-operand order of
// v_mfma_f32_16x16x32_f16.
//
// A decoding lane (row j = lane & 15, part q = lane >> 4) handles one row of a 16-row tile for
// half a K block (4 slices): IQ3_S slice 4h + q of row j; Q4_K quarter q (8 values) of each of
// the half block's 4 slices of row j. The decoded half block of row tile t sits at h_off(t, ...)
// of the caller's A area.
//
// Block scales: each row's accumulator is held in units of e, the last nonzero d of the row's
// blocks so far (a block with d = 0 decodes to zeros). At a block start the decoder writes the
// ratio e_prev / e_cur (RT) and e_cur (EF) for the row; the GEMM multiplies the row's
// accumulators by RT before adding the block and by EF at the end.
#pragma once

#include "decode.h"
#include "iq3_tile.h"

namespace gguf {

namespace {  // each kernel file gets its own copy of the device tables

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kHRegion = 1040;                     // A bytes per (row tile, slice): 16 rows x 64 B + pad

// fp16 bits of a small positive integer
constexpr uint32_t small_int_half(uint32_t v) {
  int e = 0;
  while ((v >> (e + 1)) != 0) ++e;
  return ((uint32_t)(e + 15) << 10) | ((v - (1u << e)) << (10 - e));
}
static_assert(small_int_half(1) == 0x3C00 && small_int_half(15) == 0x4B80, "fp16 bits");

// The IQ3_S grid as fp16: entry i = the 4 grid values of index i, 2 per dword
struct Iq3sGridHalf {
  uint32_t v[1024];
};
constexpr Iq3sGridHalf make_iq3s_grid_half() {
  Iq3sGridHalf g{};
  for (int i = 0; i < 512; ++i) {
    const uint32_t w = kIq3sGrid.v[i];
    g.v[2 * i] = small_int_half(w & 0xFF) | (small_int_half((w >> 8) & 0xFF) << 16);
    g.v[2 * i + 1] = small_int_half((w >> 16) & 0xFF) | (small_int_half(w >> 24) << 16);
  }
  return g;
}
__device__ const Iq3sGridHalf kIq3sGridHalf = make_iq3s_grid_half();

// The IQ3_XXS grid as fp16 (entries 0..255 in the first 512 dwords)
constexpr Iq3sGridHalf make_iq3xxs_grid_half() {
  Iq3sGridHalf g{};
  for (int i = 0; i < 256; ++i) {
    const uint32_t w = kIq3xxsGrid.v[i];
    g.v[2 * i] = small_int_half(w & 0xFF) | (small_int_half((w >> 8) & 0xFF) << 16);
    g.v[2 * i + 1] = small_int_half((w >> 16) & 0xFF) | (small_int_half(w >> 24) << 16);
  }
  return g;
}
__device__ const Iq3sGridHalf kIq3xxsGridHalf = make_iq3xxs_grid_half();

// A slot of (row tile t, slice u of the half block, row j, quarter q): the quarter's 16 bytes sit
// in slot q ^ g(j) of the row, g(j) = ((j >> 1) ^ (j >> 3)) & 3, which keeps the operand reads
// (lane (j, q)) free of bank conflicts.
__device__ __forceinline__ int h_off(int t, int u, int j, int q) {
  return (t * 4 + u) * kHRegion + j * 64 + ((q ^ ((j >> 1) ^ (j >> 3))) & 3) * 16;
}

__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 bits_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

// A decoding lane's raw weight bytes for one step, loaded two steps ahead.
// (16- and 8-bit loads kept narrow: a 32-bit field is widened where the loop's register sets meet,
// at its head, which waits for every load in flight, the prefetch of the next steps included)
struct RawIq3 {
  uint2 qs;     // qs of the lane's row and slice
  uint32_t e8;  // E8 dword of the row
  uint16_t l2;  // L2 halfword of the row pair
  uint8_t sc;   // SC byte (two 4-bit sub-scales)
  uint16_t d;   // fp16 d of the row
};
struct RawXxsH {
  uint2 qs;      // the 8 grid indices of the lane's row and slice
  uint32_t aux;  // the slice's four 7-bit sign indices and 4-bit scale
  uint16_t d;    // fp16 d of the row
};
struct RawQ4k {
  u32x4 hdr;    // d, dmin, scales[12]
  uint2 v0, v1; // quarter q of the two 32-byte quant groups of the half block
};

// IQ3_S lane (row j, slice 4h + sp) of K block b of a 16-row tile in the unit layout (tile: the
// tile's first byte; tile row j is in unit j >> 2, row pair (j >> 1) & 1)
__device__ __forceinline__ void load_step(RawIq3& w, const uint8_t* tile, int64_t row_bytes, int nb, int b, int h,
                                          int j, int sp) {
  const int r = j & 1, s = 4 * h + sp;
  const Iq3Fields f = iq3_block_fields(nb, b), l = iq3_lane_fields((j >> 1) & 1, s);
  const uint8_t* u = tile + (int64_t)(j >> 2) * kUnitRows * row_bytes;
  w.qs = *(const uint2*)(u + f.qs + l.qs + 8 * r);
  w.e8 = *(const uint32_t*)(u + f.e8 + l.e8 + 4 * r);
  w.l2 = *(const uint16_t*)(u + f.l2 + l.l2);
  w.sc = u[f.sc + l.sc + 2 * (s >> 1) + r];
  w.d = *(const uint16_t*)(u + f.d + l.d + 2 * r);
}

// IQ3_XXS lane (row j, slice 4h + sp) of K block b of a 16-row tile in the IQ3_XXS unit layout:
// the block's 16 lanes 8 rp + s hold rows 2rp, 2rp+1 of the unit
__device__ __forceinline__ void load_step(RawXxsH& w, const uint8_t* tile, int64_t row_bytes, int nb, int b, int h,
                                          int j, int sp) {
  const int r = j & 1, rp = (j >> 1) & 1, s = 4 * h + sp, L = 8 * rp + s;
  const XxsFields f = xxs_block_fields(nb, b);
  const uint8_t* u = tile + (int64_t)(j >> 2) * kUnitRows * row_bytes;
  w.qs = *(const uint2*)(u + f.qs + 16 * L + 8 * r);
  w.aux = *(const uint32_t*)(u + f.aux + 8 * L + 4 * r);
  w.d = *(const uint16_t*)(u + f.d + 4 * rp + 2 * r);
}

// Q4_K lane (row j, quarter q) of the row's block
__device__ __forceinline__ void load_step(RawQ4k& w, const uint8_t* blk, int h, int q) {
  w.hdr = *(const u32x4*)blk;
  w.v0 = *(const uint2*)(blk + 16 + 64 * h + 8 * q);
  w.v1 = *(const uint2*)(blk + 48 + 64 * h + 8 * q);
}

// The row's running scale at a block start (h == 0): e_cur = d, or e_prev for d = 0; the ratio
// and the final scale go to LDS (the lanes of a row store the same values).
__device__ __forceinline__ float next_scale(float d, float& e, float* RT, float* EF, int row) {
  const float en = d != 0.0f ? d : e;
  RT[row] = e / en;
  EF[row] = en;
  e = en;
  return en;
}

__device__ __forceinline__ void decode_step(const RawIq3& w, int h, const uint32_t* gh, const uint2* sm, uint8_t* A,
                                            float* RT, float* EF, float& e, int t, int j, int sp) {
  const int s = 4 * h + sp;
  const float d = half_bits_to_float(w.d);
  if (h == 0) next_scale(d, e, RT, EF, t * 16 + j);
  uint32_t lo, hi;
  iq3_tile_ex(w.e8, w.l2, j & 1, lo, hi);
  const uint32_t nib = (w.sc >> (4 * (s & 1))) & 0xF;
  const _Float16 ls = d != 0.0f ? (_Float16)(float)(1 + 2 * nib) : (_Float16)0.0f;
  const h2 lsh = {ls, ls};
  uint32_t v[16];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint32_t qb = ((g < 4 ? w.qs.x : w.qs.y) >> (8 * (g & 3))) & 0xFF;
    const uint32_t ex = ((g < 4 ? lo : hi) >> (8 * (g & 3))) & 0xFF;
    const uint2 gv = *(const uint2*)(gh + 2 * (qb | ((ex >> 4) << 8)));
    const uint2 sg = sm[ex & 0xF];
    v[2 * g] = h2_bits(bits_h2(gv.x ^ sg.x) * lsh);
    v[2 * g + 1] = h2_bits(bits_h2(gv.y ^ sg.y) * lsh);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *(uint4*)(A + h_off(t, sp, j, q)) = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

// IQ3_XXS: value = d * ls * w / 4 (ls = 2 * scale + 1, w the signed grid byte): the operand is
// w * ls (at most 62 * 31 = 1922, exact in fp16) and the row's scale d / 4. The second word of
// each 8-value group takes bits 4..6 of the group's 7-bit sign index and their parity with bits
// 0..3 (ksigns_iq2xs), all four parities from two three-way xors (bit 7g of t ^ t >> 3 ^ a >> 6,
// t = a ^ a >> 1 ^ a >> 2, is the xor of bits 7g..7g+6).
__device__ __forceinline__ void decode_step(const RawXxsH& w, int h, const uint32_t* gh, const uint2* sm, uint8_t* A,
                                            float* RT, float* EF, float& e, int t, int j, int sp) {
  const float d = half_bits_to_float(w.d) * 0.25f;
  if (h == 0) next_scale(d, e, RT, EF, t * 16 + j);
  const uint32_t a = w.aux;
  const uint32_t t3 = a ^ (a >> 1) ^ (a >> 2);
  const uint32_t par = t3 ^ (t3 >> 3) ^ (a >> 6);
  const uint32_t hi = ((par << 3) & 0x01020408u) | ((a >> 4) & ~0x01020408u);
  const _Float16 ls = d != 0.0f ? (_Float16)(float)(2 * (a >> 28) + 1) : (_Float16)0.0f;
  const h2 lsh = {ls, ls};
  uint32_t v[16];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t qw = (g < 2 ? w.qs.x : w.qs.y) >> (16 * (g & 1));
    const uint2 g0 = *(const uint2*)(gh + 2 * (qw & 0xFF)), g1 = *(const uint2*)(gh + 2 * ((qw >> 8) & 0xFF));
    const uint2 s0 = sm[(a >> (7 * g)) & 0xF], s1 = sm[(hi >> (7 * g)) & 0xF];
    v[4 * g] = h2_bits(bits_h2(g0.x ^ s0.x) * lsh);
    v[4 * g + 1] = h2_bits(bits_h2(g0.y ^ s0.y) * lsh);
    v[4 * g + 2] = h2_bits(bits_h2(g1.x ^ s1.x) * lsh);
    v[4 * g + 3] = h2_bits(bits_h2(g1.y ^ s1.y) * lsh);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *(uint4*)(A + h_off(t, sp, j, q)) = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

// Q4_K: fp16 (1024 + nibble) by a byte permute, then one packed FMA gives nibble x sc exactly.
__device__ __forceinline__ void decode_step(const RawQ4k& w, int h, float* AM, uint8_t* A, float* RT, float* EF,
                                            float& e, int t, int j, int q) {
  const float d = half_bits_to_float(w.hdr[0] & 0xFFFF);
  const float dmin = half_bits_to_float(w.hdr[0] >> 16);
  // e: the running scale of the row; a lane decoding only the second half updates it itself
  const float en = h == 0 ? next_scale(d, e, RT, EF, t * 16 + j) : (e = d != 0.0f ? d : e);
  const float mf = -dmin / en;
  const bool nz = d != 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int us = 4 * h + u, jj = us & 3;
    const uint32_t a = (w.hdr[1] >> (8 * jj)) & 0xFF, c = (w.hdr[2] >> (8 * jj)) & 0xFF;
    uint32_t sc, m;
    if (us < 4) {
      sc = a & 63;
      m = c & 63;
    } else {
      const uint32_t ee = (w.hdr[3] >> (8 * jj)) & 0xFF;
      sc = (ee & 0xF) | ((a >> 6) << 4);
      m = (ee >> 4) | ((c >> 6) << 4);
    }
    const _Float16 scf = nz ? (_Float16)(float)sc : (_Float16)0.0f;
    const h2 mul = {scf, scf};
    const h2 off = mul * (_Float16)(-1024.0f);
    const uint2 vv = u < 2 ? w.v0 : w.v1;
    const int sh = 4 * (u & 1);
    const uint32_t x0 = (vv.x >> sh) & 0x0F0F0F0Fu, x1 = (vv.y >> sh) & 0x0F0F0F0Fu;
    const uint32_t w0 = h2_bits(__builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)), mul, off));
    const uint32_t w1 = h2_bits(__builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)), mul, off));
    const uint32_t w2 = h2_bits(__builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)), mul, off));
    const uint32_t w3 = h2_bits(__builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)), mul, off));
    *(uint4*)(A + h_off(t, u, j, q)) = make_uint4(w0, w1, w2, w3);
    AM[(t * 4 + u) * 16 + j] = mf * (float)m;  // the 4 lanes of row j store the same value
  }
}

// Q6_K lane (row j, part q) of the row's block for half block h (values 128h .. 128h + 127, slices
// 4h + sub): ql bytes [64h + 8q, + 8) (low nibbles: sub 0, high: sub 2) and [64h + 32 + 8q, + 8)
// (sub 1, 3), qh bytes [32h + 8q, + 8) (bit pair 2 sub), the half's 8 scales, d
// (dequantize_row_q6_K, ggml-quants.c). Blocks are 210 bytes: 2-byte aligned loads.
struct RawQ6k {
  uint64_t la, lb, qh, sc;
  uint16_t d;  // kept 16-bit (see RawIq3)
};

__device__ __forceinline__ void load_step(RawQ6k& w, const uint8_t* blk, int h, int q) {
  w.la = ld64(blk + 64 * h + 8 * q);
  w.lb = ld64(blk + 64 * h + 32 + 8 * q);
  w.qh = ld64(blk + 128 + 32 * h + 8 * q);
  w.sc = ld64(blk + 192 + 8 * h);
  w.d = ld16(blk + 208);
}

// Q6_K: fp16 (1024 + q) by a byte permute, q - 32 by one packed subtract (exact), then times the
// 16-value sub-scale by one packed multiply. The product (q - 32) * sc is exact in fp16 up to 2048
// in magnitude; beyond (sub-scales above 64) an odd product rounds to an even neighbour, 2^-12
// relative at most. The lane's 8 values of slice 4h + sub share sub-scale 2 sub + (q >> 1).
__device__ __forceinline__ void decode_step(const RawQ6k& w, int h, uint8_t* A, float* RT, float* EF, float& e,
                                            int t, int j, int q) {
  const float d = half_bits_to_float(w.d);
  if (h == 0) next_scale(d, e, RT, EF, t * 16 + j);
  else e = d != 0.0f ? d : e;
  const bool nz = d != 0.0f;
  const h2 bias = {(_Float16)-1056.0f, (_Float16)-1056.0f};
#pragma unroll
  for (int sub = 0; sub < 4; ++sub) {
    const uint64_t l = (sub & 1) ? w.lb : w.la;
    const int lsh = 4 * (sub >> 1), hsh = 2 * sub;
    const uint32_t x0 = (((uint32_t)l >> lsh) & 0x0F0F0F0Fu) | ((((uint32_t)w.qh >> hsh) & 0x03030303u) << 4);
    const uint32_t x1 = (((uint32_t)(l >> 32) >> lsh) & 0x0F0F0F0Fu) | ((((uint32_t)(w.qh >> 32) >> hsh) & 0x03030303u) << 4);
    const int scv = (int)(int8_t)((w.sc >> (8 * (2 * sub + (q >> 1)))) & 0xFF);
    const _Float16 scf = nz ? (_Float16)(float)scv : (_Float16)0.0f;
    const h2 mul = {scf, scf};
    const uint32_t w0 = h2_bits((bits_h2(__builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) + bias) * mul);
    const uint32_t w1 = h2_bits((bits_h2(__builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) + bias) * mul);
    const uint32_t w2 = h2_bits((bits_h2(__builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) + bias) * mul);
    const uint32_t w3 = h2_bits((bits_h2(__builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) + bias) * mul);
    *(uint4*)(A + h_off(t, sub, j, q)) = make_uint4(w0, w1, w2, w3);
  }
}

// The IQ3_S decode tables in LDS: the fp16 grid (GH, 1024 dwords) and the 16 sign masks (SM),
// written by threads tid = 0 .. nt - 1 of the workgroup; the caller synchronises.
__device__ __forceinline__ void iq3_half_tables_to_lds(uint32_t* GH, uint2* SM, int tid, int nt, bool xxs = false) {
  if (xxs) {
    for (int i = tid; i < 512; i += nt) GH[i] = kIq3xxsGridHalf.v[i];
  } else {
    for (int i = tid; i < 1024; i += nt) GH[i] = kIq3sGridHalf.v[i];
  }
  if (tid < 16) {
    const uint32_t nib = tid;
    SM[nib] = make_uint2(((nib & 1u) << 15) | ((nib & 2u) << 30), ((nib & 4u) << 13) | ((nib & 8u) << 28));
  }
}

}  // namespace

}  // namespace gguf
