// The build's IQ3_S unit layout (its own; the reference's iq3_pack.py layout serves its CUDA mma
// fragments and is not reproduced), and the signed-grid table the decode kernels read.
//
// Rows are grouped in units of 4. Unit u's bytes stay where rows 4u..4u+3 were; its K blocks are
// taken four at a time: blocks 4kb..4kb+3 of the unit become one 1760-byte unit-block at byte
// 1760*kb of the unit (when nb % 4 = r != 0 the last unit-block holds the r remaining blocks in
// 440*r bytes, with every field below scaled by r/4). A decode lane L = 8p + s (p = 2*bi + rp,
// s = 32-value slice 0..7) owns rows 2rp, 2rp+1 (r = 0, 1) of the unit in slice s of block
// 4kb + bi. For group e (values 4e..4e+3 of the slice, e = 0..7) of row r define the 5-bit
//   ex(r, e) = sign nibble e of the slice's 4 sign bytes | (bit e of qh[s]) << 4
// so that (qs byte | ex << 8) is a 13-bit index into the signed-grid table (below). A full
// unit-block holds, for every lane L:
//   [   0, 1024)  QS  16 B at 16L : qs[8s..8s+8) of row 2rp, then of row 2rp+1
//   [1024, 1536)  E8   8 B at 8L  : byte 4r+j (j = 0..3) = ex(r, j) | (ex(r, 4+j) & 7) << 5
//   [1536, 1664)  L2   2 B at 2L  : bits 8r+2j, 8r+2j+1 = ex(r, 4+j) >> 3
//   [1664, 1728)  SC   2 B at 2(4p + j) : scales[j] of row 2rp, then of row 2rp+1 (j = 0..3)
//   [1728, 1760)  D    4 B at 4p  : d of row 2rp, then of row 2rp+1
// (block_iq3_s byte offsets: d 0, qs 2, qh 66, signs 74, scales 106.) Same size, bijective,
// local to each unit, and every load of a decode wave is contiguous across the wave (16 / 8 / 2 B
// per lane). Fields are ordered by bi, so the data of one K block b = 4kb + bi is, inside its
// unit-block, QS at 256 bi, E8 at 1024 + 128 bi, L2 at 1536 + 32 bi, SC at 1664 + 16 bi and D at
// 1728 + 8 bi. The MFMA kernels work on 16-row tiles = 4 consecutive units and read one K block
// of each unit per step; the decode GEMV reads whole unit-blocks. 4-row units split the
// 27B-class shapes evenly over 256 CUs (17408 rows = 17 units per CU, 5120 rows = 5).
#pragma once

#include "gguf_common.h"

namespace gguf {

constexpr int kTileRows = 16;            // row tile of the MFMA kernels: 4 units
constexpr int kUnitRows = 4;
constexpr int kUnitBlockBytes = 4 * 4 * 110;  // 1760
constexpr int kTe8 = 1024, kTl2 = 1536, kTsc = 1664, kTd = 1728;  // field bases of a full unit-block

// field bases inside a unit-block of r blocks (r = 4 except a ragged last one)
__host__ __device__ constexpr uint32_t iq3_e8_base(int r) { return 256u * r; }
__host__ __device__ constexpr uint32_t iq3_l2_base(int r) { return 384u * r; }
__host__ __device__ constexpr uint32_t iq3_sc_base(int r) { return 416u * r; }
__host__ __device__ constexpr uint32_t iq3_d_base(int r) { return 432u * r; }

// blocks held by unit-block kb of a unit of nb blocks
__host__ __device__ constexpr int iq3_unit_blocks(int nb, int kb) { return kb < (nb >> 2) ? 4 : (nb & 3); }

// Byte offsets, from the unit's first byte, of the five fields of K block b (for every lane: add
// the lane's part, iq3_lane_fields)
struct Iq3Fields {
  uint32_t qs, e8, l2, sc, d;
};

__host__ __device__ inline Iq3Fields iq3_block_fields(int nb, int b) {
  const int kb = b >> 2, bi = b & 3, r = iq3_unit_blocks(nb, kb);
  const uint32_t u = (uint32_t)kUnitBlockBytes * kb;
  return {u + 256u * bi, u + iq3_e8_base(r) + 128u * bi, u + iq3_l2_base(r) + 32u * bi, u + iq3_sc_base(r) + 16u * bi,
          u + iq3_d_base(r) + 8u * bi};
}

// The whole unit-block kb (the decode GEMV's work item): field bases, lanes add 16L / 8L / 2L /
// 2(4p + j) / 4p
__host__ __device__ inline Iq3Fields iq3_unitblock_fields(int nb, int kb) {
  const int r = iq3_unit_blocks(nb, kb);
  const uint32_t u = (uint32_t)kUnitBlockBytes * kb;
  return {u, u + iq3_e8_base(r), u + iq3_l2_base(r), u + iq3_sc_base(r), u + iq3_d_base(r)};
}

// A lane's part of one K block's fields: rows 2rp, 2rp+1 of the unit, slice s (the SC byte of
// scales[j] of row r at sc + 2j + r, the d of row r at d + 2r)
__host__ __device__ inline Iq3Fields iq3_lane_fields(int rp, int s) {
  return {(uint32_t)(128 * rp + 16 * s), (uint32_t)(64 * rp + 8 * s), (uint32_t)(16 * rp + 2 * s), (uint32_t)(8 * rp),
          (uint32_t)(4 * rp)};
}

// Signed-grid table: entry (qs | ex << 8) = the grid word of index qs | (ex >> 4) << 8 with the
// bytes whose bit is set in ex & 0xF negated; 8192 x int8x4 = 32 KB, staged in LDS by the
// decode kernels.
struct Iq3sSignedTable {
  uint32_t v[8192];
};

constexpr Iq3sSignedTable make_iq3s_signed_table() {
  Iq3sSignedTable t{};
  for (int idx = 0; idx < 8192; ++idx) {
    const int ex = idx >> 8;
    const uint32_t g = kIq3sGrid.v[(idx & 0xFF) | ((ex >> 4) << 8)];
    uint32_t out = 0;
    for (int b = 0; b < 4; ++b) {
      uint32_t byte = (g >> (8 * b)) & 0xFF;
      if ((ex >> b) & 1) byte = (256u - byte) & 0xFF;
      out |= byte << (8 * b);
    }
    t.v[idx] = out;
  }
  return t;
}

// ---------------------------------------------------------------------------------------------
// Pack / unpack of one lane's share of a K block (host and device).

// ex of group e (0..7) of a slice, from its 4 sign bytes (as a dword) and its qh byte
__host__ __device__ inline uint32_t iq3_ex(uint32_t signs, uint32_t qh, int e) {
  return ((signs >> (4 * e)) & 0xF) | (((qh >> e) & 1u) << 4);
}

// GGUF block pointers of rows 2rp, 2rp+1 (slice s) -> the lane's QS / E8 / L2 bytes at qs / e8 / l2
__host__ __device__ inline void iq3_tile_pack_lane(const uint8_t* const rowblk[2], int s, uint8_t* qs, uint8_t* e8,
                                                   uint8_t* l2p) {
  uint32_t l2 = 0;
  for (int r = 0; r < 2; ++r) {
    const uint8_t* b = rowblk[r];
    for (int i = 0; i < 8; ++i) qs[8 * r + i] = b[2 + 8 * s + i];
    const uint32_t sg = (uint32_t)b[74 + 4 * s] | ((uint32_t)b[75 + 4 * s] << 8) | ((uint32_t)b[76 + 4 * s] << 16) |
                        ((uint32_t)b[77 + 4 * s] << 24);
    const uint32_t qh = b[66 + s];
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = iq3_ex(sg, qh, j), hi = iq3_ex(sg, qh, 4 + j);
      e8[4 * r + j] = (uint8_t)(lo | ((hi & 7u) << 5));
      l2 |= (hi >> 3) << (8 * r + 2 * j);
    }
  }
  l2p[0] = (uint8_t)(l2 & 0xFF);
  l2p[1] = (uint8_t)(l2 >> 8);
}

// the lane's QS / E8 / L2 bytes -> qs, qh and sign bytes of rows 2rp, 2rp+1 (GGUF blocks, slice s)
__host__ __device__ inline void iq3_tile_unpack_lane(const uint8_t* qs, const uint8_t* e8, const uint8_t* l2p, int s,
                                                     uint8_t* const rowblk[2]) {
  const uint32_t l2 = (uint32_t)l2p[0] | ((uint32_t)l2p[1] << 8);
  for (int r = 0; r < 2; ++r) {
    uint8_t* b = rowblk[r];
    for (int i = 0; i < 8; ++i) b[2 + 8 * s + i] = qs[8 * r + i];
    uint32_t sg = 0, qh = 0;
    for (int e = 0; e < 8; ++e) {
      const int j = e & 3;
      const uint32_t byte = e8[4 * r + j];
      const uint32_t ex = e < 4 ? (byte & 0x1F) : ((byte >> 5) | (((l2 >> (8 * r + 2 * j)) & 3u) << 3));
      sg |= (ex & 0xF) << (4 * e);
      qh |= ((ex >> 4) & 1u) << e;
    }
    for (int i = 0; i < 4; ++i) b[74 + 4 * s + i] = (uint8_t)(sg >> (8 * i));
    b[66 + s] = (uint8_t)qh;
  }
}

// SC and D bytes of a unit-block of r blocks: byte j in [iq3_sc_base(r), 440 r) <-> (row in the
// unit, block bi in the unit-block, byte in the row's block)
__host__ __device__ inline void iq3_tile_scale_source(int j, int r, int& row, int& bi, int& o) {
  if (j < (int)iq3_d_base(r)) {
    const int jj = j - (int)iq3_sc_base(r), rem = jj & 15;  // 16 bi + 8 rp + 2 jsc + rr
    bi = jj >> 4;
    row = 2 * (rem >> 3) + (rem & 1);
    o = 106 + ((rem >> 1) & 3);
  } else {
    const int jj = j - (int)iq3_d_base(r), rem = jj & 7;    // 8 bi + 4 rp + 2 rr + byte
    bi = jj >> 3;
    row = 2 * (rem >> 2) + ((rem >> 1) & 1);
    o = rem & 1;
  }
}

// ---------------------------------------------------------------------------------------------
// The build's IQ3_XXS unit layout (its own, as the IQ3_S one above): the same 4-row units and
// unit-blocks of 4 K blocks (4 x 4 x 98 = 1568 B; a last unit-block of r = nb % 4 blocks takes
// 392 r bytes, fields scaled by r/4), the same lanes L = 8p + s (p = 2 bi + rp: rows 2rp, 2rp+1 of
// the unit in slice s of block 4kb + bi). block_iq3_xxs is d[0:2], qs[2:66] (one grid index per 4
// values), then per slice s a dword at 66 + 4s (four 7-bit sign indices, the scale in bits 28..31).
//   [   0, 256 r) QS  16 B at 16L: qs[8s..8s+8) of row 2rp, then of row 2rp+1
//   [256 r, 384 r) AUX  8 B at 8L : the slice's dword of row 2rp, then of row 2rp+1
//   [384 r, 392 r) D    4 B at 4p : d of row 2rp, then of row 2rp+1
// A byte permutation local to each unit, bijective; every decode-wave load is contiguous across
// the wave (16 / 8 B per lane, 4 B per 8 lanes). The data of K block b = 4kb + bi sits, inside its
// unit-block, at QS 256 bi, AUX 128 bi and D 8 bi.
constexpr int kXxsUnitBlockBytes = 4 * 4 * 98;  // 1568

__host__ __device__ constexpr uint32_t xxs_aux_base(int r) { return 256u * r; }
__host__ __device__ constexpr uint32_t xxs_d_base(int r) { return 384u * r; }

struct XxsFields {
  uint32_t qs, aux, d;
};

// unit-block kb of a unit of nb blocks: field bases from the unit's first byte
__host__ __device__ inline XxsFields xxs_unitblock_fields(int nb, int kb) {
  const int r = iq3_unit_blocks(nb, kb);
  const uint32_t u = (uint32_t)kXxsUnitBlockBytes * kb;
  return {u, u + xxs_aux_base(r), u + xxs_d_base(r)};
}

// K block b of a unit of nb blocks: its QS / AUX / D bytes from the unit's first byte (QS: 16
// lanes x 16 B, AUX 16 x 8 B, D 2 x 4 B, lanes 16 bi .. 16 bi + 15 in order)
__host__ __device__ inline XxsFields xxs_block_fields(int nb, int b) {
  const int kb = b >> 2, bi = b & 3, r = iq3_unit_blocks(nb, kb);
  const uint32_t u = (uint32_t)kXxsUnitBlockBytes * kb;
  return {u + 256u * bi, u + xxs_aux_base(r) + 128u * bi, u + xxs_d_base(r) + 8u * bi};
}

// Byte j of a unit-block of r blocks <- (row in the unit, block bi in the unit-block, byte o of
// that row's GGUF block)
__host__ __device__ inline void xxs_unit_source(int j, int r, int& row, int& bi, int& o) {
  if (j < (int)xxs_aux_base(r)) {
    const int L = j >> 4, w = j & 15, s = L & 7;
    bi = L >> 4;
    row = 2 * ((L >> 3) & 1) + (w >> 3);
    o = 2 + 8 * s + (w & 7);
  } else if (j < (int)xxs_d_base(r)) {
    const int jj = j - (int)xxs_aux_base(r), L = jj >> 3, w = jj & 7, s = L & 7;
    bi = L >> 4;
    row = 2 * ((L >> 3) & 1) + (w >> 2);
    o = 66 + 4 * s + (w & 3);
  } else {
    const int jj = j - (int)xxs_d_base(r), p = jj >> 2, w = jj & 3;
    bi = p >> 1;
    row = 2 * (p & 1) + (w >> 1);
    o = w & 1;
  }
}

// ---------------------------------------------------------------------------------------------
// Decode helpers of the kernels

// ex of the 4 groups 0..3 (lo) and 4..7 (hi) of row r, one per byte, from a lane's E8 dword of
// row r and its L2 halfword
__device__ __forceinline__ void iq3_tile_ex(uint32_t e8, uint32_t l2, int r, uint32_t& lo, uint32_t& hi) {
  lo = e8 & 0x1F1F1F1Fu;
  const uint32_t b = (l2 >> (8 * r)) & 0xFF;
  const uint32_t t = (b | (b << 12)) & 0x000F000Fu;
  const uint32_t t2 = (t | (t << 6)) & 0x03030303u;
  hi = ((e8 >> 5) & 0x07070707u) | (t2 << 3);
}

// signed-grid words of the table entries for the two groups a byte permute pairs in P
// (P = qs0 | ex0 << 8 | qs1 << 16 | ex1 << 24; tbl is the table in LDS)
// The low index's byte offset (P & 0xFFFF) << 2 is one SDWA shift of P's low word (the compiler
// otherwise emits a shift and a mask).
__device__ __forceinline__ void tile_lookup2(const uint8_t* tbl, uint32_t P, int& w0, int& w1) {
  uint32_t o0;
  asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
      : "=v"(o0)
      : "v"(P));
  w0 = *(const int*)(tbl + o0);
  w1 = *(const int*)(tbl + (P >> 14));  // bits 14, 15 of P are zero (ex has 5 bits)
}

// The signed-grid table built in LDS from the 512-word grid (2 KB read instead of 32 KB): thread
// i < 512 holds grid word i (`gword`) and writes the 16 entries (i & 255) | (sign nibble | (i >> 8)
// << 4) << 8. Every grid byte is odd (1..15), so the bytewise negation 256 - b of all four bytes is
// the one subtraction 0x01010100 - g (each byte borrows from the next exactly once); the entry
// takes the negated bytes where the sign nibble has a bit.
constexpr bool iq3_grid_negation_is_bytewise() {
  for (int i = 0; i < 512; ++i) {
    const uint32_t g = kIq3sGrid.v[i], n = 0x01010100u - g;
    for (int b = 0; b < 4; ++b)
      if (((n >> (8 * b)) & 0xFF) != ((256u - ((g >> (8 * b)) & 0xFF)) & 0xFF)) return false;
  }
  return true;
}
static_assert(iq3_grid_negation_is_bytewise(), "0x01010100 - g negates every byte of every grid word");

__device__ __forceinline__ void iq3_table_from_grid(uint4* table, uint32_t gword, int i) {
  const uint32_t neg = 0x01010100u - gword;
  uint32_t* t32 = (uint32_t*)table;
  const uint32_t base = (uint32_t)(i & 255) | ((uint32_t)(i >> 8) << 12);
#pragma unroll
  for (int sg = 0; sg < 16; ++sg) {
    const uint32_t m = ((sg & 1) ? 0xFFu : 0u) | ((sg & 2) ? 0xFF00u : 0u) | ((sg & 4) ? 0xFF0000u : 0u) |
                       ((sg & 8) ? 0xFF000000u : 0u);
    t32[base | ((uint32_t)sg << 8)] = (neg & m) | (gword & ~m);
  }
}

// The 32 KB signed-grid table, global -> LDS without VGPRs: 32 wave-wide 1 KB DMA loads
// (global_load_lds_dwordx4) shared out over the workgroup's NW waves (wave < NW). The caller waits
// (vmcnt) and synchronises the workgroup before reading the table. When NW divides 32 every wave
// issues the same number of loads with no branch, so the compiler's count of outstanding loads
// stays exact past the copy.
template <int NW>
__device__ __forceinline__ void iq3_table_to_lds(uint4* table, const Iq3sSignedTable* src_table, int wave, int lane) {
  const uint4* src = (const uint4*)src_table->v;
  if constexpr (32 % NW == 0) {
#pragma unroll
    for (int j = 0; j < 32 / NW; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(src + (wave + j * NW) * 64 + lane),
                                       (__attribute__((address_space(3))) void*)(table + (wave + j * NW) * 64), 16, 0,
                                       0);
  } else {
#pragma unroll
    for (int i = wave; i < 32; i += NW)
      __builtin_amdgcn_global_load_lds((const void*)(src + i * 64 + lane),
                                       (__attribute__((address_space(3))) void*)(table + i * 64), 16, 0, 0);
  }
}

}  // namespace gguf
