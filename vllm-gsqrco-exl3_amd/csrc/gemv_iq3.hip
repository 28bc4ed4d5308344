// Decode GEMV for IQ3_S in the build's unit layout (iq3_tile.h): Y[c, r] = sum_k X[c, k] * W[r, k]
// for 1..8 activation rows.
//
// Replaces the reference's packed decode products (lcpp_owned_iq3_mma.cu:484-612, the
// lcpp_mul_mat_vec_iq3_mma_packed op) with two gfx950 kernels sharing one decode step: a lane
// turns every 4-value group of its two rows into one read of the 32 KB signed-grid table in LDS
// (a byte permute builds two table indices) and multiplies with v_dot4_i32_i8; the integer slice
// dot is scaled by the slice's sub-scale, the row's d and X's q8_1 d in fp32.
//  * gemv_iq3s_stream_kernel (weights of at least one unit per CU, 1-4 activation rows): one
//    workgroup per CU owns an equal run of 4-row units (17408 rows = 17 per CU, 5120 rows = 5),
//    and each of its 8 waves a contiguous run of the range's (unit, unit-block) items, so every
//    CU streams the same bytes with no cross-workgroup reduction. A wave keeps two unit-blocks in
//    flight while it computes a third. Partial row sums go to LDS when a wave leaves a unit and
//    are added in wave order at the end. X is staged in LDS first: the caller's q8_1 copied, or X
//    quantised there with the q8_1 quantiser's arithmetic (bit-identical bytes), while the first
//    weight loads are in flight.
//  * gemv_iq3s_tile_kernel (the other shapes): one 16-row tile per workgroup, its waves split the
//    K blocks; X as q8_1 or quantised block by block.
#include <algorithm>
#include <type_traits>

#include "gemv_x.h"
#include "iq3_tile.h"

namespace gguf {

__device__ const Iq3sSignedTable kIq3sSignedDev = make_iq3s_signed_table();
__device__ const Iq3sGrid kIq3sGridDev = kIq3sGrid;

struct TileFrag {
  uint4 qs;
  uint2 e8;
  uint16_t l2, sc;  // 16-bit loads kept 16-bit: widening them is left to their uses
  uint32_t dd;
};

// A lane's byte offsets inside one K block's (tile kernel) or one unit-block's (stream kernel)
// fields; the block's field bases (Iq3Fields) are added as scalar offsets.
struct TileOffs {
  uint32_t qs, e8, l2, sc, dd;
};

// tile kernel: lane L = 8p + s of a 16-row tile owns rows 2p, 2p+1 (unit p >> 1, its row pair
// p & 1) in slice s
__device__ __forceinline__ TileOffs tile_lane_offsets(int p, int s, int64_t row_bytes) {
  const uint32_t u = (uint32_t)((p >> 1) * kUnitRows * row_bytes);
  const Iq3Fields l = iq3_lane_fields(p & 1, s);
  return {u + l.qs, u + l.e8, u + l.l2, u + l.sc + 2u * (uint32_t)(s >> 1), u + l.d};
}

// stream kernel: lane L = 8p + s of a unit-block (p = 2 bi + rp)
__device__ __forceinline__ TileOffs unit_lane_offsets(int lane, int p, int s) {
  return {16u * lane, 8u * lane, 2u * lane, 2u * (uint32_t)(4 * p + (s >> 1)), 4u * p};
}

// the lane's bytes of one K block or unit-block: scalar field bases f (inside rs) + lane offsets o
__device__ __forceinline__ void load_tile_frag(__amdgpu_buffer_rsrc_t rs, const Iq3Fields& f, const TileOffs& o,
                                               TileFrag& t) {
  const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o.qs, (int)f.qs, kWeightCpol);
  t.qs = make_uint4(q.x, q.y, q.z, q.w);
  const auto e = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)o.e8, (int)f.e8, kWeightCpol);
  t.e8 = make_uint2(e[0], e[1]);
  t.l2 = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)o.l2, (int)f.l2, kWeightCpol);
  t.sc = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)o.sc, (int)f.sc, kWeightCpol);
  t.dd = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)o.dd, (int)f.d, kWeightCpol);
}

template <int NC>
struct XFrag {
  int q[NC][8];
  uint32_t d[NC];  // fp16 bits (converted where used, so a prefetch does not wait for its load)
};

// ---------------------------------------------------------------------------------------------
// IQ3_XXS in the build's unit layout (iq3_tile.h): the stream kernel below serves it with the
// lanes of the IQ3_S layout. Lane L = 8p + s loads its 16 QS bytes (row 2rp's 8 grid indices of
// slice s, then row 2rp+1's), its 8 AUX bytes (the two rows' sign / scale words) and the 4 D bytes
// of its row pair, each field contiguous across the wave.
__device__ const Lattice32<256> kIq3xxsGridDev = kIq3xxsGrid;

struct XxsFrag {
  uint4 qs;
  uint2 aux;
  uint32_t dd;  // fp16 d of row 2rp (low half) and 2rp+1 (high half)
};

// f: the unit-block's field bases inside rs (scalar offsets); o: the lane's offsets (unit_lane_offsets:
// qs 16L, e8 8L, dd 4p)
__device__ __forceinline__ void load_xxs_frag(__amdgpu_buffer_rsrc_t rs, const XxsFields& f, const TileOffs& o,
                                              XxsFrag& t) {
  const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o.qs, (int)f.qs, kWeightCpol);
  t.qs = make_uint4(q.x, q.y, q.z, q.w);
  const auto e = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)o.e8, (int)f.aux, kWeightCpol);
  t.aux = make_uint2(e[0], e[1]);
  t.dd = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)o.dd, (int)f.d, kWeightCpol);
}

// The 4096-entry IQ3_XXS signed table in LDS (entry g | n << 8: grid word g with the bytes whose
// bit is set in the nibble n negated; the kIq3xxsSigned entries), built from the 1 KB grid:
// thread i < 512 holds grid word i & 255 and writes the 8 entries of the nibbles 8 (i >> 8) ..
// 8 (i >> 8) + 7. Every grid byte is nonzero, so the bytewise negation is 0x01010100 - g.
constexpr bool iq3xxs_table_formula_holds() {
  for (int i = 0; i < 4096; ++i) {
    const uint32_t g = kIq3xxsGrid.v[i & 255], neg = 0x01010100u - g, n = (uint32_t)i >> 8;
    const uint32_t m = ((n & 1) ? 0xFFu : 0u) | ((n & 2) ? 0xFF00u : 0u) | ((n & 4) ? 0xFF0000u : 0u) |
                       ((n & 8) ? 0xFF000000u : 0u);
    if (((neg & m) | (g & ~m)) != kIq3xxsSigned.v[i]) return false;
  }
  return true;
}
static_assert(iq3xxs_table_formula_holds(), "IQ3_XXS signed table from the grid");

__device__ __forceinline__ void iq3xxs_table_from_grid(uint4* table, uint32_t gword, int i) {
  const uint32_t neg = 0x01010100u - gword;
  const uint32_t top = (i >> 8) & 1 ? 0xFF000000u : 0u;  // nibble bit 3
  uint32_t* t32 = (uint32_t*)table;
  const uint32_t base = (uint32_t)(i & 255) | ((uint32_t)((i >> 8) & 1) << 11);
#pragma unroll
  for (int sg = 0; sg < 8; ++sg) {
    const uint32_t m = ((sg & 1) ? 0xFFu : 0u) | ((sg & 2) ? 0xFF00u : 0u) | ((sg & 4) ? 0xFF0000u : 0u) | top;
    t32[base | ((uint32_t)sg << 8)] = (neg & m) | (gword & ~m);
  }
}

// byte B of v times 4 (a table entry's byte offset): one SDWA shift
template <int B>
__device__ __forceinline__ uint32_t byte_x4(uint32_t v) {
  uint32_t o;
  if constexpr (B == 0)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0" : "=v"(o) : "v"(v));
  else if constexpr (B == 1)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1" : "=v"(o) : "v"(v));
  else if constexpr (B == 2)
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2" : "=v"(o) : "v"(v));
  else
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3" : "=v"(o) : "v"(v));
  return o;
}

// a ^ b ^ c in one gfx950 three-input bit operation (truth table 0x96: odd parity)
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t o;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(o) : "v"(a), "v"(b), "v"(c));
  return o;
}

// bits 7g..7g+3 of v at bits 10..13 (the nibble's place in a table byte offset)
template <int G>
__device__ __forceinline__ uint32_t nib_x1024(uint32_t v) {
  constexpr int sh = 10 - 7 * G;
  return (sh >= 0 ? v << sh : v >> -sh) & 0x3C00u;
}

// The lane's two rows of one item. Sign index g (bits 7g..7g+6 of aux) gives the first word of
// group g its nibble (bits 7g..7g+3) and the second word bits 7g+4..7g+6 plus the parity of all
// seven as bit 3 (ksigns_iq2xs). The four parities come from two three-way xors: with
// t_i = a_i ^ a_i+1 ^ a_i+2, t_i ^ t_i+3 ^ a_i+6 is the xor of a_i..a_i+6, which at i = 7g reads
// only sign index g's bits. A table read's byte offset is (index byte) * 4 | nibble * 1024. The
// slice term is the decode ops' (s4 sumi + sumi / 2) / 2 with s4 = aux >> 28 (ls = 2 s4 + 1),
// times d and X's d.
template <int NC>
__device__ __forceinline__ void xxs_compute(const uint8_t* tbl, const XxsFrag& f, const XFrag<NC>& x,
                                            float (&acc)[2][NC]) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint32_t a = r == 0 ? f.aux.x : f.aux.y;
    const uint32_t t = xor3(a, a >> 1, a >> 2);
    const uint32_t par = xor3(t, t >> 3, a >> 6);                              // bit 7g: parity of index g
    const uint32_t hi = ((par << 3) & 0x01020408u) | ((a >> 4) & ~0x01020408u);  // bits 7g..7g+3
    const uint32_t q0 = r == 0 ? f.qs.x : f.qs.z, q1 = r == 0 ? f.qs.y : f.qs.w;
    int w[8];
    w[0] = *(const int*)(tbl + (byte_x4<0>(q0) | nib_x1024<0>(a)));
    w[1] = *(const int*)(tbl + (byte_x4<1>(q0) | nib_x1024<0>(hi)));
    w[2] = *(const int*)(tbl + (byte_x4<2>(q0) | nib_x1024<1>(a)));
    w[3] = *(const int*)(tbl + (byte_x4<3>(q0) | nib_x1024<1>(hi)));
    w[4] = *(const int*)(tbl + (byte_x4<0>(q1) | nib_x1024<2>(a)));
    w[5] = *(const int*)(tbl + (byte_x4<1>(q1) | nib_x1024<2>(hi)));
    w[6] = *(const int*)(tbl + (byte_x4<2>(q1) | nib_x1024<3>(a)));
    w[7] = *(const int*)(tbl + (byte_x4<3>(q1) | nib_x1024<3>(hi)));
    const float lsq = (float)(2 * (int)(a >> 28) + 1) * 0.25f;  // ls / 4
    const float dw = half_bits_to_float((f.dd >> (16 * r)) & 0xFFFFu);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      int sumi = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) sumi = dot4(w[e], x.q[c][e], sumi);
      // (s4 sumi + sumi / 2) / 2 in C's truncating division equals trunc(sumi ls / 4), and
      // sumi ls (|sumi| <= 32 * 62 * 127, ls <= 31) is below 2^24: exact in fp32
      const float v = truncf((float)sumi * lsq);
      acc[r][c] = fmaf(v, dw * half_bits_to_float(x.d[c]), acc[r][c]);
    }
  }
}

// q8_1 blocks of X at slice `slice0 + s` for every activation row c (row c starts nslices
// blocks after row c-1): rs describes the whole q8_1 buffer, lane_off = 36 * s
template <int NC>
__device__ __forceinline__ void load_x_frag(__amdgpu_buffer_rsrc_t rs, uint32_t lane_off, int nslices, int slice0,
                                            XFrag<NC>& x) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int so = (c * nslices + slice0) * 36;
    x.d[c] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)lane_off, so, 0);
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)lane_off, so + 4, 0);
    const u32x4 e = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)lane_off, so + 20, 0);
    x.q[c][0] = (int)a.x; x.q[c][1] = (int)a.y; x.q[c][2] = (int)a.z; x.q[c][3] = (int)a.w;
    x.q[c][4] = (int)e.x; x.q[c][5] = (int)e.y; x.q[c][6] = (int)e.z; x.q[c][7] = (int)e.w;
  }
}

// Fused quantisation of X (the decode ops' block_q8_1 arithmetic, done inside the GEMV): lane
// L = 8p + s loads values 4p..4p+3 of slice s of a block of every activation row; the 8 lanes of a
// slice exchange their partial amax and then their 4 q bytes through a 64-dword LDS area of the
// wave, so each lane ends up with the slice's 32 q values as the q8_1 path would load them.
template <int NC, int XDT>
struct XRawFrag {
  uint32_t v[NC][XDT == kF32 ? 4 : 2];
};

template <int NC, int XDT>
__device__ __forceinline__ void load_xraw_frag(const void* x, int64_t s01, int block, int p, int s,
                                               XRawFrag<NC, XDT>& r) {
  const int64_t e0 = (int64_t)block * kQK + 32 * s + 4 * p;  // values 4p..4p+3 of slice s
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if constexpr (XDT == kF32) {
      const uint4 v = *(const uint4*)((const float*)x + c * s01 + e0);
      r.v[c][0] = v.x; r.v[c][1] = v.y; r.v[c][2] = v.z; r.v[c][3] = v.w;
    } else {
      const uint2 v = *(const uint2*)((const uint16_t*)x + c * s01 + e0);
      r.v[c][0] = v.x; r.v[c][1] = v.y;
    }
  }
}

template <int XDT>
__device__ __forceinline__ float xraw_value(const uint32_t* v, int i) {
  if constexpr (XDT == kF32) return __uint_as_float(v[i]);
  const uint32_t h = (v[i >> 1] >> (16 * (i & 1))) & 0xFFFF;
  if constexpr (XDT == kF16) return half_bits_to_float(h);
  return __uint_as_float(h << 16);
}

// ex: the wave's 64-dword exchange area; the lane holds values 4p..4p+3 of slice s (the slice's
// 8 lanes are s, s+8, ..., s+56)
template <int NC, int XDT>
__device__ __forceinline__ void quantize_xraw(const XRawFrag<NC, XDT>& r, uint32_t* ex, int p, int s,
                                              XFrag<NC>& x) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = xraw_value<XDT>(r.v[c], i);
    ex[8 * s + p] = __float_as_uint(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    const uint4 a0 = *(const uint4*)(ex + 8 * s), a1 = *(const uint4*)(ex + 8 * s + 4);
    const float amax = fmaxf(fmaxf(fmaxf(__uint_as_float(a0.x), __uint_as_float(a0.y)),
                                   fmaxf(__uint_as_float(a0.z), __uint_as_float(a0.w))),
                             fmaxf(fmaxf(__uint_as_float(a1.x), __uint_as_float(a1.y)),
                                   fmaxf(__uint_as_float(a1.z), __uint_as_float(a1.w))));
    const float d = amax / 127.0f;
    uint32_t qw[1];
    quantize_q81<4>(v, amax, d, qw);
    ex[8 * s + p] = qw[0];  // after this wave's reads above: a wave's LDS operations complete in order
    const uint4 q0 = *(const uint4*)(ex + 8 * s), q1 = *(const uint4*)(ex + 8 * s + 4);
    x.q[c][0] = (int)q0.x; x.q[c][1] = (int)q0.y; x.q[c][2] = (int)q0.z; x.q[c][3] = (int)q0.w;
    x.q[c][4] = (int)q1.x; x.q[c][5] = (int)q1.y; x.q[c][6] = (int)q1.z; x.q[c][7] = (int)q1.w;
    x.d[c] = __half_as_ushort(__float2half_rn(d));
  }
}

template <int NC>
__device__ __forceinline__ void tile_compute(const uint8_t* tbl, const TileFrag& f, const XFrag<NC>& x, int s,
                                             float (&acc)[2][NC]) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint32_t q0 = r == 0 ? f.qs.x : f.qs.z;
    const uint32_t q1 = r == 0 ? f.qs.y : f.qs.w;
    uint32_t lo, hi;
    iq3_tile_ex(r == 0 ? f.e8.x : f.e8.y, f.l2, r, lo, hi);
    int w[8];
    tile_lookup2(tbl, __builtin_amdgcn_perm(lo, q0, 0x05010400u), w[0], w[1]);
    tile_lookup2(tbl, __builtin_amdgcn_perm(lo, q0, 0x07030602u), w[2], w[3]);
    tile_lookup2(tbl, __builtin_amdgcn_perm(hi, q1, 0x05010400u), w[4], w[5]);
    tile_lookup2(tbl, __builtin_amdgcn_perm(hi, q1, 0x07030602u), w[6], w[7]);
    const int ls = 1 + 2 * (((f.sc >> (8 * r)) >> (4 * (s & 1))) & 0xF);
    const float dl = half_bits_to_float((f.dd >> (16 * r)) & 0xFFFF) * (float)ls;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      int sumi = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) sumi = dot4(w[e], x.q[c][e], sumi);
      acc[r][c] = fmaf((float)sumi, dl * half_bits_to_float(x.d[c]), acc[r][c]);
    }
  }
}

// XDT < 0: X given as block_q8_1 (q8); else X itself (dtype XDT, row stride s01), quantised in the
// kernel with the same arithmetic.
template <int NC, int TPW, int WPT, int XDT>
__global__ void __launch_bounds__(64 * TPW * WPT) gemv_iq3s_tile_kernel(const uint8_t* __restrict__ W,
                                                                        int64_t row_bytes, int nrows, int k,
                                                                        const void* __restrict__ xsrc,
                                                                        int64_t s01, void* __restrict__ y,
                                                                        int y_dtype) {
  constexpr bool FUSED = XDT >= 0;
  __shared__ uint4 table[2048];  // the 8192-entry signed-grid table
  __shared__ float red[TPW][WPT][NC][kTileRows];
  __shared__ uint32_t xex[FUSED ? TPW * WPT : 1][64];  // per-wave exchange of the fused quantisation
  const uint8_t* q8 = (const uint8_t*)xsrc;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave index, scalar
  const int wave = wv % WPT;   // K part of the tile
  const int tw = wv / WPT;     // tile of the workgroup
  const int tile = blockIdx.x * TPW + tw;
  const int ntiles = nrows / kTileRows;
  const int p = lane >> 3, s = lane & 7;
  const int nb = k / kQK;
  const int nslices = k / kQ81;
  const bool active = tile < ntiles;
  const int b_begin = active ? wave * nb / WPT : 0, b_end = active ? (wave + 1) * nb / WPT : 0;
  const uint8_t* tb = W + (int64_t)(active ? tile : 0) * kTileRows * row_bytes;  // scalar
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(tb, (uint32_t)(kTileRows * row_bytes));
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(q8, FUSED ? 0u : (uint32_t)(NC * nslices * 36));
  const uint8_t* tbl = (const uint8_t*)table;
  const TileOffs off = tile_lane_offsets(p, s, row_bytes);
  const uint32_t xoff = 36u * (uint32_t)s;

  float acc[2][NC];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[i][c] = 0.0f;

  // Two named register sets (A, B) for the weight tile-block and the q8_1 blocks of X; the next
  // block's loads are issued before the current block is computed. Two blocks per iteration and
  // an odd last block after the loop, so that no load is behind a branch: a load under a branch
  // makes the compiler wait for it before the next compute (vmcnt(0) on the joined paths), and
  // one whose only use is conditional is sunk to that use. The weight prefetch past the wave's
  // last block reads zeros through an empty descriptor and is never used; the X prefetch is
  // clamped to the last block. The scheduling barriers keep the next block's decode below the
  // loads just issued.
  const __amdgpu_buffer_rsrc_t nrs = buffer_rsrc(W, 0);
  const int b_last = b_end - 1;
  const int nblk = b_end - b_begin;
  TileFrag fa, fb;
  if constexpr (!FUSED) {
    XFrag<NC> xa, xb;
    if (nblk > 0) {
      load_x_frag<NC>(xrs, xoff, nslices, b_begin * 8, xa);
      load_tile_frag(wrs, iq3_block_fields(nb, b_begin), off, fa);
    }
    iq3_table_to_lds<TPW * WPT>(table, &kIq3sSignedDev, wv, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int b = b_begin;
    for (int it = 0; it < nblk / 2; ++it, b += 2) {
      const int b2 = b + 2 < b_last ? b + 2 : b_last;
      const __amdgpu_buffer_rsrc_t rs2 = b + 2 < b_end ? wrs : nrs;
      load_x_frag<NC>(xrs, xoff, nslices, (b + 1) * 8, xb);
      load_tile_frag(wrs, iq3_block_fields(nb, b + 1), off, fb);
      __builtin_amdgcn_sched_barrier(0);
      tile_compute<NC>(tbl, fa, xa, s, acc);
      load_x_frag<NC>(xrs, xoff, nslices, b2 * 8, xa);
      load_tile_frag(rs2, iq3_block_fields(nb, b + 2), off, fa);
      __builtin_amdgcn_sched_barrier(0);
      tile_compute<NC>(tbl, fb, xb, s, acc);
    }
    if (nblk & 1) tile_compute<NC>(tbl, fa, xa, s, acc);
  } else {
    // Raw X runs two blocks ahead and is quantised one block ahead, so the slice exchange of
    // the next block overlaps the current block's decode.
    constexpr int XD = FUSED ? XDT : kBF16;
    uint32_t* ex = xex[wv];
    XRawFrag<NC, XD> ra, rb;
    XFrag<NC> qa, qb;
    auto clampb = [&](int bb) { return bb < b_last ? bb : b_last; };
    if (nblk > 0) {
      load_xraw_frag<NC, XD>(xsrc, s01, b_begin, p, s, ra);
      load_xraw_frag<NC, XD>(xsrc, s01, clampb(b_begin + 1), p, s, rb);
      load_tile_frag(wrs, iq3_block_fields(nb, b_begin), off, fa);
    }
    iq3_table_to_lds<TPW * WPT>(table, &kIq3sSignedDev, wv, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    quantize_xraw<NC, XD>(ra, ex, p, s, qa);
    int b = b_begin;
    for (int it = 0; it < nblk / 2; ++it, b += 2) {
      const __amdgpu_buffer_rsrc_t rs2 = b + 2 < b_end ? wrs : nrs;
      load_xraw_frag<NC, XD>(xsrc, s01, clampb(b + 2), p, s, ra);
      load_tile_frag(wrs, iq3_block_fields(nb, b + 1), off, fb);
      __builtin_amdgcn_sched_barrier(0);
      quantize_xraw<NC, XD>(rb, ex, p, s, qb);
      tile_compute<NC>(tbl, fa, qa, s, acc);
      load_xraw_frag<NC, XD>(xsrc, s01, clampb(b + 3), p, s, rb);
      load_tile_frag(rs2, iq3_block_fields(nb, b + 2), off, fa);
      __builtin_amdgcn_sched_barrier(0);
      quantize_xraw<NC, XD>(ra, ex, p, s, qa);
      tile_compute<NC>(tbl, fb, qb, s, acc);
    }
    if (nblk & 1) tile_compute<NC>(tbl, fa, qa, s, acc);
  }

#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float v = acc[i][c];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      if (s == 0) red[tw][wave][c][2 * p + i] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < TPW * NC * kTileRows) {
    const int t = threadIdx.x / (NC * kTileRows);
    const int c = (threadIdx.x / kTileRows) % NC, r = threadIdx.x % kTileRows;
    const int otile = blockIdx.x * TPW + t;
    if (otile < ntiles) {
      float v = red[t][0][c][r];
#pragma unroll
      for (int w2 = 1; w2 < WPT; ++w2) v += red[t][w2][c][r];
      store_y(y, (int64_t)c * nrows + (int64_t)otile * kTileRows + r, v, y_dtype);
    }
  }
}

// X of the stream GEMV, staged in LDS: q8 values [NC][slice][8 dwords], then each slice's fp16 d
// [NC][slice] (one dword, low half). Work unit: group g = 8 values, part g & 3 of slice row
// g >> 2 (= c * nslices + slice of activation row c). The four lanes of a slice are consecutive.
// group g of X into the LDS staging area (every lane of a slice takes part in the amax exchange);
// a group past the end (live false) is written to `sink`: a load whose only use is a conditional
// store is moved under the condition by the compiler and then waited for (vmcnt(0)) at the join
template <int XDT>
__device__ __forceinline__ void xgroup_store(const XGroup<XDT>& r, int g, bool live, uint32_t* xq, uint32_t* xd,
                                             uint4* sink) {
  const int sr = g >> 2, part = g & 3;
  uint32_t lo, hi, dbits;
  if constexpr (XDT < 0) {
    lo = r.v[1];
    hi = r.v[2];
    dbits = r.v[0] & 0xFFFFu;
  } else {
    xgroup_quantize<XDT>(r, lo, hi, dbits);
  }
  *(live ? (uint2*)(xq + sr * 8 + 2 * part) : (uint2*)sink) = make_uint2(lo, hi);
  *(live && part == 0 ? xd + sr : (uint32_t*)sink) = dbits;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  // every control used here reads a valid lane; bound_ctrl with old = 0 lets hipcc fold the move
  // into the add that consumes it (one v_add_f32 with a DPP source)
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

constexpr int kStreamWaves = 8;

// Stream GEMV over 4-row units. Workgroup g owns units [g U / G, (g + 1) U / G) (as one buffer
// range) and its items (unit, unit-block), unit-major; wave w takes items [w I / 8, (w + 1) I / 8)
// of them. Lane L = 8p + s (p = 2 bi + rp) decodes rows 2rp, 2rp+1 of the unit in slice s of K
// block 4 kb + bi and accumulates over the wave's unit-blocks of a unit; when the wave leaves a
// unit (or its run ends) the 8 slice lanes are summed by DPP (xor 1, xor 2, then the half-row
// mirror: the same sums, in the same order, as an xor-4 butterfly) and the lanes of slice 0 store
// 16 partial row sums to LDS, slot (unit, wave). The output adds, per row, the slots of the waves
// that touched the unit in wave order, the four bi partials in bi order within each. In a last
// unit-block of r < 4 blocks the lanes of bi >= r add nothing (d and X's d taken as 0). The slots
// start at zero, so every wave's slot of a unit is added (zeros where the wave did not touch it).
// X: XDT < 0 the caller's block_q8_1 copied into LDS, XDT >= 0 X itself (row stride s01)
// quantised into LDS with the q8_1 arithmetic. Each thread stages XPT groups of 8 values, their
// loads issued first, then the grid word, then the wave's first two unit-blocks.
// TYPE kIQ3_XXS: the same split, items and lanes over the IQ3_XXS unit layout (1568-B unit-blocks;
// XxsFrag), its 16 KB signed table built from the 1 KB grid.
// Y's activation rows are ys elements apart (the launch may cover a run of the weight's rows).
// RG: K's last unit-block is ragged (nb % 4 == 2); without it no lane needs the remapped offsets
// or the zeroed scales, and neither is computed (11 of 177 VALU instructions per item at 4 rows,
// 9 of 90 at one; in one run of graph replays 17408 x 5120 M = 1 10.9-11.2 against 11.3-11.9 us
// with the ragged code, 5120 x 17408 12.7 against 12.9-13.1).
template <int TYPE, int NC, int XDT, int XPT, bool RG, int NW = kStreamWaves>
__global__ void __launch_bounds__(64 * NW) gemv_iq3s_stream_kernel(const uint8_t* __restrict__ W,
                                                                              int64_t row_bytes, int nrows, int k,
                                                                              const void* __restrict__ xsrc,
                                                                              int64_t s01, void* __restrict__ y,
                                                                              int64_t ys, int y_dtype) {
  constexpr int NT = 64 * NW;
  constexpr bool XXS = TYPE == kIQ3_XXS;
  static_assert(TYPE == kIQ3_S || XXS, "IQ3_S or IQ3_XXS, each in its unit layout");
  static_assert(NT >= 512, "the table build takes 512 threads");
  using Frag = typename std::conditional<XXS, XxsFrag, TileFrag>::type;
  __shared__ uint4 table[XXS ? 1024 : 2048];
  __shared__ uint4 sink;    // staging writes of groups past the end of X
  extern __shared__ uint4 xdyn[];  // X: q [NC][slice][8 dwords], d [NC][slice]; then the partial sums
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = lane >> 3, s = lane & 7, bi = p >> 1;
  const int nb = k / kQK, nkb = (nb + 3) >> 2, nslices = k / kQ81;
  const int nslots_x = NC * nslices * 8;
  uint32_t* xq = (uint32_t*)xdyn;
  uint32_t* xd = xq + nslots_x;
  float* part = (float*)(xd + NC * nslices);  // [unit][wave][NC][16]
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(xsrc, XDT < 0 ? (uint32_t)(NC * nslices * 36) : 0u);
  const int ngroups = NC * nslices * 4;
  int xg[XPT];
  bool xlive[XPT];
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int g = threadIdx.x + j * NT;
    xlive[j] = g < ngroups;
    xg[j] = xlive[j] ? g : ngroups - 1;
  }
  // X and the grid word first; every wave's staging loads are issued before any weight load
  // (barrier below), since a CU's loads return in order
  XGroup<XDT> xa[XPT];
#pragma unroll
  for (int j = 0; j < XPT; ++j) xgroup_load<NC, XDT>(xsrc, xrs, s01, nslices, xg[j], xa[j]);
  const uint32_t gword =
      XXS ? __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(&kIq3xxsGridDev, 1024), 4 * (threadIdx.x & 255), 0, 0)
          : __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(&kIq3sGridDev, 2048), 4 * (threadIdx.x & 511), 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  // the workgroup's units [u0, u1) and the wave's run of items [j0, j1) (32-bit: units * grid
  // < 2^31 for any weight of fewer than 2^23 rows)
  const uint32_t nunits = (uint32_t)nrows / kUnitRows, G = gridDim.x;
  const int u0 = (int)(blockIdx.x * nunits / G), u1 = (int)((blockIdx.x + 1) * nunits / G);
  const int nu = u1 - u0, items = nu * nkb;
  const uint32_t ubytes = (uint32_t)(kUnitRows * row_bytes), rbytes = (uint32_t)nu * ubytes;
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(W + (int64_t)u0 * ubytes, rbytes);
  // a last unit-block of r = 2 blocks (nb % 4 == 2; K % 512 == 0 leaves r in {0, 2}): lanes of
  // bi >= 2 load lane L - 32's bytes instead of bytes past the block's fields, so every load of
  // the run stays inside it; their terms are zeroed below (d = 0)
  const TileOffs off = unit_lane_offsets(lane, p, s), off_r = unit_lane_offsets(lane & 31, p & 3, s);
  constexpr bool ragged = RG;  // the launch passes RG == (nb % 4 != 0)
  // an empty range: loads past the wave's run read zeros without touching memory (the hardware
  // range check sees only the lane offset, not the scalar field base)
  const __amdgpu_buffer_rsrc_t nrs = buffer_rsrc(W, 0u);
  const uint8_t* tbl = (const uint8_t*)table;
  const int j0 = wave * items / NW, j1 = (wave + 1) * items / NW;
  const int cu0 = (int)((uint32_t)j0 / (uint32_t)nkb);
  int lj = j0, lu = cu0, lkb = j0 - cu0 * nkb;  // the next item to load
  auto fields = [&](int u, int kb) {
    Iq3Fields f = iq3_unitblock_fields(nb, kb);
    const uint32_t ub = (uint32_t)u * ubytes;
    f.qs += ub; f.e8 += ub; f.l2 += ub; f.sc += ub; f.d += ub;
    return f;
  };
  // past the run: the empty range nrs (every lane's load reads zeros)
  auto load_next = [&](Frag& f) {
    const bool in_run = lj < j1;
    if constexpr (XXS) {
      XxsFields x = {0u, 0u, 0u};
      if (in_run) {
        x = xxs_unitblock_fields(nb, lkb);
        const uint32_t ub = (uint32_t)lu * ubytes;
        x.qs += ub; x.aux += ub; x.d += ub;
      }
      load_xxs_frag(in_run ? wrs : nrs, x, ragged && lkb == nkb - 1 ? off_r : off, f);
    } else {
      const Iq3Fields e = {0u, 0u, 0u, 0u, 0u};
      load_tile_frag(in_run ? wrs : nrs, in_run ? fields(lu, lkb) : e, ragged && lkb == nkb - 1 ? off_r : off, f);
    }
    ++lj;
    if (++lkb == nkb) {
      lkb = 0;
      ++lu;
    }
  };
  __syncthreads();
  Frag f0, f1, f2;
  load_next(f0);
  load_next(f1);
  __builtin_amdgcn_sched_barrier(0);
  if (NT == 512 || threadIdx.x < 512) {
    if constexpr (XXS) iq3xxs_table_from_grid(table, gword, threadIdx.x);
    else iq3_table_from_grid(table, gword, threadIdx.x);
  }
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    if (wave * 64 + j * NT < ngroups)  // waves with no group left skip the (fused) quantisation
      xgroup_store<XDT>(xa[j], xg[j], xlive[j], xq, xd, &sink);
  }
  // the partial-sum slots start at zero: the output adds every wave's slot of a unit
  for (int t = threadIdx.x; t < nu * NW * NC * 4; t += NT) ((float4*)part)[t] = make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  int cu = cu0, ckb = j0 - cu0 * nkb, j = j0;  // the item being computed
  const int xl = 8 * bi + s;
  float acc[2][NC];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
  auto step = [&](const Frag& fc, Frag& fl) {
    load_next(fl);
    __builtin_amdgcn_sched_barrier(0);
    // lanes of blocks past a last unit-block of r < 4 blocks: d = 0 and X's d = 0
    const bool live = !RG || bi < iq3_unit_blocks(nb, ckb);
    const int sl = live ? 32 * ckb + xl : 0;
    XFrag<NC> x;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int o = c * nslices + sl;
      const uint4 a0 = *(const uint4*)(xq + o * 8), a1 = *(const uint4*)(xq + o * 8 + 4);
      x.q[c][0] = (int)a0.x; x.q[c][1] = (int)a0.y; x.q[c][2] = (int)a0.z; x.q[c][3] = (int)a0.w;
      x.q[c][4] = (int)a1.x; x.q[c][5] = (int)a1.y; x.q[c][6] = (int)a1.z; x.q[c][7] = (int)a1.w;
      const uint32_t dv = xd[o];  // read unconditionally (o is in range) and selected: no branch
      x.d[c] = live ? dv : 0u;
    }
    Frag f = fc;
    f.dd = live ? f.dd : 0u;
    if constexpr (XXS) xxs_compute<NC>(tbl, f, x, acc);
    else tile_compute<NC>(tbl, f, x, s, acc);
    ++j;
    if (++ckb == nkb || j == j1) {  // leaving the unit: its partial sums to the wave's slot
      const int slot = cu * NW + wave;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float v0 = acc[0][c], v1 = acc[1][c];
        v0 += dpp_f<0xB1>(v0);
        v1 += dpp_f<0xB1>(v1);
        v0 += dpp_f<0x4E>(v0);
        v1 += dpp_f<0x4E>(v1);
        v0 += dpp_f<0x141>(v0);
        v1 += dpp_f<0x141>(v1);
        if (s == 0) *(float2*)(part + (slot * NC + c) * 16 + 2 * p) = make_float2(v0, v1);
        acc[0][c] = 0.0f;
        acc[1][c] = 0.0f;
      }
      if (ckb == nkb) {
        ckb = 0;
        ++cu;
      }
    }
  };
  const int nmine = j1 - j0;
  int i = 0;
  for (; i + 3 <= nmine; i += 3) {
    step(f0, f2);
    step(f1, f0);
    step(f2, f1);
  }
  if (i < nmine) step(f0, f2);
  if (i + 1 < nmine) step(f1, f0);
  __syncthreads();
  // output o = (unit, column, row) by the quad of lanes 4o + bi: each adds its bi partial of every
  // wave's slot in wave order, then the quad adds the four (xor 1, then xor 2)
  const int nout = nu * kUnitRows * NC;
  for (int t0 = 0; t0 < 4 * nout; t0 += NT) {
    const int t = t0 + (int)threadIdx.x, o = t >> 2, q = t & 3;
    const int uu = o / (kUnitRows * NC), c = (o >> 2) % NC, row = o & 3;
    float v = 0.0f;
    if (o < nout) {
      const float* pp = part + (uu * NW * NC + c) * 16 + 4 * q + 2 * (row >> 1) + (row & 1);
#pragma unroll
      for (int w = 0; w < NW; ++w) v += pp[w * NC * 16];
    }
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    if (q == 0 && o < nout)
      store_y(y, (int64_t)c * ys + (int64_t)(u0 + uu) * kUnitRows + row, v, y_dtype);
  }
}

// ---------------------------------------------------------------------------------------------
// Launch plans

constexpr size_t kStreamXMax = 96 * 1024;        // X staged in the stream kernel's LDS
constexpr size_t kStreamLdsMin = 82 * 1024;      // dynamic LDS floor: one workgroup per CU
constexpr int kStreamXpt[] = {1, 2, 3, 4, 5, 6, 9, 13, 17, 24};

// dynamic LDS of a stream launch: X's q8_1 plus the partial-sum slots of the most units a
// workgroup owns, at least kStreamLdsMin
static size_t stream_lds(int64_t nrows, int64_t k, int64_t n, int64_t grid) {
  const int64_t nu_max = (nrows / kUnitRows + grid - 1) / grid;
  const size_t part = (size_t)nu_max * kStreamWaves * (size_t)n * 16 * sizeof(float);
  return std::max(kStreamLdsMin, (size_t)n * (size_t)(k / kQ81) * 36 + part);
}

// the stream kernel's static LDS: the signed-grid table (IQ3_S 2048, IQ3_XXS 1024 x 16 B) and the
// 16-B sink; the dynamic LDS a workgroup may take beside it
template <int TYPE>
constexpr size_t stream_lds_max() {
  return 160 * 1024 - sizeof(uint4) * ((TYPE == kIQ3_XXS ? 1024 : 2048) + 1);
}

// The stream kernel takes 1..4 activation rows (fused X: 1..2 rows at K <= 8192) on weights of
// at least one 4-row unit per CU, with X's q8_1 and the partial sums within its LDS budget (a
// weight of many units per CU at 3-4 rows needs more partial-sum slots than fit: such shapes take
// the tile kernel). Quantising X in every workgroup costs more than the quantise launch at 3-4
// rows (17408 x 5120, M = 4: 19.5 against 18.3 us) and at K = 17408 (5120 x 17408, M = 1: 13.5
// against 12.8 us): those take the q8_1 path.
template <int TYPE = kIQ3_S>
static bool stream_supported(int64_t nrows, int64_t k, int64_t n, bool fused) {
  if (n < 1 || n > (fused ? 2 : 4) || (fused && k > 8192)) return false;
  if ((size_t)n * (size_t)(k / kQ81) * 36 > kStreamXMax) return false;
  const int64_t cus = device_cus();
  if (nrows / kUnitRows < cus) return false;
  return stream_lds(nrows, k, n, cus) <= stream_lds_max<TYPE>();
}

template <int TYPE, int NC, int XDT, int XPT>
static void launch_stream_k(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int64_t s01,
                            void* y, int64_t ys, int y_dtype, hipStream_t stream) {
  const unsigned g = (unsigned)std::min<int64_t>(nrows / kUnitRows, device_cus());
  const size_t lds = stream_lds(nrows, k, NC, g);
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    struct Tag;  // one set of per-device flags per kernel instantiation
    once_per_device<Tag>(dev, [] {
      (void)hipFuncSetAttribute((const void*)gemv_iq3s_stream_kernel<TYPE, NC, XDT, XPT, false>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)stream_lds_max<TYPE>());
      (void)hipFuncSetAttribute((const void*)gemv_iq3s_stream_kernel<TYPE, NC, XDT, XPT, true>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)stream_lds_max<TYPE>());
    });
  }
  if ((k / kQK) % 4 != 0)
    gemv_iq3s_stream_kernel<TYPE, NC, XDT, XPT, true><<<g, 64 * kStreamWaves, lds, stream>>>(W, row_bytes, nrows, k, x,
                                                                                            s01, y, ys, y_dtype);
  else
    gemv_iq3s_stream_kernel<TYPE, NC, XDT, XPT, false><<<g, 64 * kStreamWaves, lds, stream>>>(W, row_bytes, nrows, k, x,
                                                                                             s01, y, ys, y_dtype);
}

template <int TYPE, int NC, int XDT>
static hipError_t launch_stream_nc(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x,
                                   int64_t s01, void* y, int64_t ys, int y_dtype, hipStream_t stream) {
  const int need = (NC * (k / kQ81) * 4 + 64 * kStreamWaves - 1) / (64 * kStreamWaves);
#define GGUF_XPT(X)                                                                         \
  if (need <= X) {                                                                          \
    launch_stream_k<TYPE, NC, XDT, X>(W, row_bytes, nrows, k, x, s01, y, ys, y_dtype, stream);  \
    return hipSuccess;                                                                      \
  }
  if constexpr (XDT >= 0) {  // fused: K <= 8192, at most 4 groups per thread
    GGUF_XPT(1) GGUF_XPT(2) GGUF_XPT(3) GGUF_XPT(4)
  } else {
    GGUF_XPT(1) GGUF_XPT(2) GGUF_XPT(3) GGUF_XPT(4) GGUF_XPT(5) GGUF_XPT(6) GGUF_XPT(9) GGUF_XPT(13) GGUF_XPT(17)
    GGUF_XPT(24)
  }
#undef GGUF_XPT
  return hipErrorInvalidValue;  // no instantiation stages this much of X (stream_supported excludes it)
}

// ys: Y's row stride in elements (the weight's rows, or more where a launch covers a run of them)
template <int XDT, int TYPE = kIQ3_S>
static hipError_t launch_stream(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int64_t s01,
                                int n, void* y, int y_dtype, hipStream_t stream, int64_t ys = -1) {
  if (ys < 0) ys = nrows;
  if (n == 1) return launch_stream_nc<TYPE, 1, XDT>(W, row_bytes, nrows, k, x, s01, y, ys, y_dtype, stream);
  if (n == 2) return launch_stream_nc<TYPE, 2, XDT>(W, row_bytes, nrows, k, x, s01, y, ys, y_dtype, stream);
  if constexpr (XDT < 0) {
    if (n == 3) return launch_stream_nc<TYPE, 3, XDT>(W, row_bytes, nrows, k, x, s01, y, ys, y_dtype, stream);
    if (n == 4) return launch_stream_nc<TYPE, 4, XDT>(W, row_bytes, nrows, k, x, s01, y, ys, y_dtype, stream);
  }
  return hipErrorInvalidValue;
}

// one 16-row tile per workgroup: 8 waves split K for one or two activation rows, 4 from three on
template <int WPT, int XDT>
static void launch_tile(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int64_t s01, int n,
                        void* y, int y_dtype, hipStream_t stream) {
  const unsigned blocks = (unsigned)(nrows / kTileRows);
#define GGUF_GT(NC) \
  gemv_iq3s_tile_kernel<NC, 1, WPT, XDT><<<blocks, 64 * WPT, 0, stream>>>(W, row_bytes, nrows, k, x, s01, y, y_dtype)
  if constexpr (XDT >= 0) {  // the fused path serves one row
    GGUF_GT(1);
  } else {
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
  }
#undef GGUF_GT
}

// nrows % 16 == 0, n in 1..8; q8: block_q8_1 of X.
hipError_t launch_gemv_packed(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                              void* y, int y_dtype, hipStream_t stream) {
  if (stream_supported(nrows, k, n, false)) {
    const hipError_t e = launch_stream<-1>(W, row_bytes, nrows, k, q8, 0, n, y, y_dtype, stream);
    if (e != hipSuccess) return e;
  } else if (n <= 2) launch_tile<8, -1>(W, row_bytes, nrows, k, q8, 0, n, y, y_dtype, stream);
  else launch_tile<4, -1>(W, row_bytes, nrows, k, q8, 0, n, y, y_dtype, stream);
  return hipGetLastError();
}

// X [n, k] of dtype x_dtype quantised in the kernel (bit-identical to the q8_1 quantiser followed
// by the GEMV of launch_gemv_packed, which takes the same kernel structure for the shape): the
// stream kernel at 1-2 rows where it applies (K <= 8192); one row on weights of up to 32M values
// that the q8_1 path also gives the one-tile kernel, which quantises each block as it goes.
bool gemv_packed_x_supported(int64_t nrows, int64_t k, int64_t n) {
  if (stream_supported(nrows, k, n, true)) return true;
  return n == 1 && nrows * k <= ((int64_t)32 << 20) && !stream_supported(nrows, k, n, false);
}

hipError_t launch_gemv_packed_x(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int x_dtype,
                                int64_t s01, int n, void* y, int y_dtype, hipStream_t stream) {
  if (!gemv_packed_x_supported(nrows, k, n)) return hipErrorInvalidValue;
  const bool st = stream_supported(nrows, k, n, true);
  switch (x_dtype) {
    case kF32:
      if (st) {
        const hipError_t e = launch_stream<kF32>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream);
        if (e != hipSuccess) return e;
      } else {
        launch_tile<8, kF32>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream);
      }
      break;
    case kF16:
      if (st) {
        const hipError_t e = launch_stream<kF16>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream);
        if (e != hipSuccess) return e;
      } else {
        launch_tile<8, kF16>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream);
      }
      break;
    default:
      if (st) {
        const hipError_t e = launch_stream<kBF16>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream);
        if (e != hipSuccess) return e;
      } else {
        launch_tile<8, kBF16>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream);
      }
      break;
  }
  return hipGetLastError();
}

// IQ3_XXS decode in its unit layout (packed; rows % 16 == 0, K % 512 == 0) through the stream
// kernel, on any number of rows: launches take at most 4 activation rows (fused, X quantised
// inside: 1-2 rows at K <= 8192, bit-identical to the q8_1 quantiser followed by the q8_1
// launch), and a weight of more units per CU than the partial-sum slots of LDS hold runs in
// consecutive row ranges, one launch each. X's q8_1 of one activation row must fit the kernel's
// X staging (K <= 87,381).
static int64_t xxs_rows_per_launch(int64_t nrows, int64_t k, int64_t n) {
  const int64_t cus = device_cus();
  const size_t x = (size_t)n * (size_t)(k / kQ81) * 36;
  if (x > kStreamXMax) return 0;
  const size_t slot = (size_t)kStreamWaves * (size_t)n * 16 * sizeof(float);  // per unit
  const int64_t nu_fit = (int64_t)((stream_lds_max<kIQ3_XXS>() - x) / slot);
  if (nu_fit < 1) return 0;
  return std::min<int64_t>(nrows, nu_fit * cus * kUnitRows);
}

static int xxs_rows_per_group(int64_t k, bool fused) {
  int g = fused ? 2 : 4;
  while (g > 1 && (size_t)g * (size_t)(k / kQ81) * 36 > kStreamXMax) --g;
  return g;
}

bool gemv_iq3xxs_stream_supported(int64_t nrows, int64_t row_bytes, int64_t k, int64_t n, bool fused) {
  if (nrows < kTileRows || nrows % kTileRows != 0 || k < 512 || k % 512 != 0 || row_bytes != k / kQK * 98) return false;
  if (n < 1 || (fused && (n > 2 || k > 8192))) return false;
  return xxs_rows_per_launch(nrows, k, 1) > 0;
}

// x_dtype < 0: x is X's block_q8_1; else X itself (dtype x_dtype, row stride s01)
hipError_t launch_gemv_iq3xxs_stream(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x,
                                     int x_dtype, int64_t s01, int n, void* y, int y_dtype, hipStream_t stream) {
  const bool fused = x_dtype >= 0;
  if (!gemv_iq3xxs_stream_supported(nrows, row_bytes, k, n, fused)) return hipErrorInvalidValue;
  const int group = xxs_rows_per_group(k, fused);
  const int64_t ysz = y_dtype == kF32 ? 4 : 2, xsz = x_dtype == kF32 ? 4 : 2;
  for (int c0 = 0; c0 < n; c0 += group) {
    const int nc = std::min(group, n - c0);
    const int64_t run = xxs_rows_per_launch(nrows, k, nc);
    if (run <= 0) return hipErrorInvalidValue;
    const void* xc = fused ? (const void*)((const uint8_t*)x + (int64_t)c0 * s01 * xsz)
                           : (const void*)((const uint8_t*)x + (int64_t)c0 * (k / kQ81) * 36);
    for (int64_t r0 = 0; r0 < nrows; r0 += run) {
      const int rows = (int)std::min<int64_t>(run, nrows - r0);
      const uint8_t* wc = W + r0 * row_bytes;
      void* yc = (uint8_t*)y + ((int64_t)c0 * nrows + r0) * ysz;
      hipError_t e;
      switch (x_dtype) {
        case kF32: e = launch_stream<kF32, kIQ3_XXS>(wc, row_bytes, rows, k, xc, s01, nc, yc, y_dtype, stream, nrows); break;
        case kF16: e = launch_stream<kF16, kIQ3_XXS>(wc, row_bytes, rows, k, xc, s01, nc, yc, y_dtype, stream, nrows); break;
        case kBF16: e = launch_stream<kBF16, kIQ3_XXS>(wc, row_bytes, rows, k, xc, s01, nc, yc, y_dtype, stream, nrows); break;
        default: e = launch_stream<-1, kIQ3_XXS>(wc, row_bytes, rows, k, xc, 0, nc, yc, y_dtype, stream, nrows); break;
      }
      if (e != hipSuccess) return e;
    }
  }
  return hipGetLastError();
}

}  // namespace gguf
