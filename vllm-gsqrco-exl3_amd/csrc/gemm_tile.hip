// int8-MFMA GEMM for IQ3_S in the unit layout (iq3_tile.h) on activations in the xq layout (xq.h):
// Y[c, r] = sum_k X[c, k] * W[r, k] for 9+ activation rows.
//
// Replaces the reference's tiled IQ3 products on packed weights (lcpp_owned_iq3_mma.cu:769-1020,
// lcpp_mul_mat_iq3_packed / lcpp_mul_mat_vec_iq3_mma_packed above 8 rows) with a gfx950 design:
//  * a workgroup owns RW 16-row tiles and NT column tiles of 16 activation rows; its KS waves
//    split the K blocks;
//  * per K block a wave loads each tile's block with the decode GEMV's loads (lane L = 8p + s:
//    slice s of rows 2p, 2p+1, i.e. of row pair p & 1 of unit p >> 1), turns every 4-value group into one read of the 32 KB
//    signed-grid table in LDS, and writes the int8 values to a per-wave LDS buffer from which
//    lane 16q + j reads the MFMA A operand (values 8q..8q+7 of slice u of tile row j);
//  * the B operands of the block come from the xq unit with four 16-byte loads per lane and
//    serve all RW tiles; one v_mfma_i32_16x16x32_i8 per (tile, slice, column tile) gives the
//    reference's integer slice dot for 16 x 16 (row, column) pairs;
//  * each dot is scaled by its slice sub-scale (integer) and activation scale (fp32) and summed
//    over the block's 8 slices, then multiplied by the block scale d of its row;
//  * the next block's weight and activation loads are issued before the current block is
//    computed (two named register sets); the waves' partial sums are added in wave order.
#include "iq3_tile.h"
#include "split_k.h"
#include "xq.h"

namespace gguf {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ const Iq3sSignedTable kIq3sSignedMma = make_iq3s_signed_table();

// Per-wave transposition buffer: slice u at 528u (512 B + 16 B pad), tile row j at 32j, the
// four 8-byte quarters q of the row in slots q ^ (j >> 2). Lane 16q + j reads its A operand of
// slice u from slot q ^ (j >> 2) of row j; a writer lane stores a row's quarter pairs with
// 16-byte stores.
constexpr int kTrSlice = 528;
constexpr int kTrBytes = 8 * kTrSlice;

struct MmaFrag {
  u32x4 qs;     // decode view: qs of slice s, rows 2p, 2p+1
  uint32_t e8x, e8y, l2;
  u32x4 sc;     // MFMA view: scale bytes of rows 4q .. 4q+3
  uint32_t d01, d23;  // fp16 d of rows 4q .. 4q+3
};

// a lane's byte offsets in one K block: decode view (rows 2p, 2p+1 of the tile: unit p >> 1, row
// pair p & 1; slice s), MFMA view (the scale and d bytes of rows 4q..4q+3: unit q)
struct MmaOffs {
  uint32_t qs, e8, l2, sc, d;
};

__device__ __forceinline__ MmaOffs mma_offsets(int p, int s, int q, int64_t row_bytes) {
  const uint32_t u = (uint32_t)((p >> 1) * kUnitRows * row_bytes), uq = (uint32_t)(q * kUnitRows * row_bytes);
  const Iq3Fields l = iq3_lane_fields(p & 1, s);
  return {u + l.qs, u + l.e8, u + l.l2, uq, uq};
}

// K block b of the tile at byte toff of rs (scalar field bases) at the lane's offsets
__device__ __forceinline__ void load_mma_frag(__amdgpu_buffer_rsrc_t rs, uint32_t toff, int nb, int b, const MmaOffs& o,
                                              MmaFrag& f) {
  const Iq3Fields bf = iq3_block_fields(nb, b);
  f.qs = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o.qs, (int)(toff + bf.qs), 0);
  const auto e = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)o.e8, (int)(toff + bf.e8), 0);
  f.e8x = e[0];
  f.e8y = e[1];
  f.l2 = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)o.l2, (int)(toff + bf.l2), 0);
  f.sc = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o.sc, (int)(toff + bf.sc), 0);
  const auto d = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)o.d, (int)(toff + bf.d), 0);
  f.d01 = d[0];
  f.d23 = d[1];
}

template <int NT>
struct XqFrag {
  u32x4 b[NT][4];  // B operands: slices 2i, 2i+1 in b[t][i]
  u32x4 d[NT][2];  // fp32 activation scales of slices 0..7 (as bits)
};

// units[t] = (column tile) * nb of the workgroup's column tile t; block b
template <int NT>
__device__ __forceinline__ void load_xq_frag(__amdgpu_buffer_rsrc_t rs, const int (&units)[NT], int b, int sbase,
                                             int lane, int j, XqFrag<NT>& x) {
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

// decode one tile-block (decode view) into the wave's transposition buffer, then read the 8
// A operands (MFMA view)
__device__ __forceinline__ void tile_to_a(const uint8_t* tbl, uint8_t* tr, const MmaFrag& f, int p, int s, int q, int j,
                                          long (&a)[8]) {
  const int c = p >> 1;  // (row >> 2) of both rows of the lane
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint32_t q0 = r == 0 ? f.qs[0] : f.qs[2];
    const uint32_t q1 = r == 0 ? f.qs[1] : f.qs[3];
    uint32_t lo, hi;
    iq3_tile_ex(r == 0 ? f.e8x : f.e8y, f.l2, r, lo, hi);
    int w[8];
    tile_lookup2(tbl, __builtin_amdgcn_perm(lo, q0, 0x05010400u), w[0], w[1]);
    tile_lookup2(tbl, __builtin_amdgcn_perm(lo, q0, 0x07030602u), w[2], w[3]);
    tile_lookup2(tbl, __builtin_amdgcn_perm(hi, q1, 0x05010400u), w[4], w[5]);
    tile_lookup2(tbl, __builtin_amdgcn_perm(hi, q1, 0x07030602u), w[6], w[7]);
    const int row = 2 * p + r;
    uint8_t* dst = tr + s * kTrSlice + row * 32;
#pragma unroll
    for (int P = 0; P < 2; ++P) {
      // quarters 2P, 2P+1 go to slots (2P) ^ c and (2P+1) ^ c: the pair P ^ (c >> 1), swapped if c is odd
      const bool sw = c & 1;
      uint4 v;
      v.x = (uint32_t)(sw ? w[4 * P + 2] : w[4 * P + 0]);
      v.y = (uint32_t)(sw ? w[4 * P + 3] : w[4 * P + 1]);
      v.z = (uint32_t)(sw ? w[4 * P + 0] : w[4 * P + 2]);
      v.w = (uint32_t)(sw ? w[4 * P + 1] : w[4 * P + 3]);
      *(uint4*)(dst + 16 * (P ^ (c >> 1))) = v;
    }
  }
  // a wave's LDS operations complete in issue order, so the reads below see the writes above;
  // the compiler barriers keep the program order (and measured faster than free scheduling)
  __asm__ volatile("" ::: "memory");
  const int slot = (q ^ (j >> 2)) & 3;
#pragma unroll
  for (int u = 0; u < 8; ++u) a[u] = *(const long*)(tr + u * kTrSlice + j * 32 + slot * 8);
  __asm__ volatile("" ::: "memory");
}

// one K block of RW tiles: decode + MFMA + scale, added into acc
template <int NT, int RW>
__device__ __forceinline__ void mma_block(const uint8_t* tbl, uint8_t* tr, const MmaFrag (&f)[RW], const XqFrag<NT>& x,
                                          int p, int s, int q, int j, float (&acc)[RW][NT][4]) {
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    long a[8];
    tile_to_a(tbl, tr, f[r], p, s, q, j, a);
    float accb[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) accb[t][v] = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      // sub-scales ls = 1 + 2 * nibble of rows 4q + v: byte 8 (v >> 1) + 2 (u >> 1) + (v & 1), nibble u & 1
      int ls[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t word = f[r].sc[2 * (v >> 1) + (u >> 2)];
        const int sh = 8 * (2 * ((u >> 1) & 1) + (v & 1)) + 4 * (u & 1);
        ls[v] = 1 + 2 * (int)((word >> sh) & 0xFu);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const long b = xq_b_operand(x.b[t][u >> 1], u & 1);
        const v4i zero = {0, 0, 0, 0};
        const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[u], b, zero, 0, 0, 0);
        const float cd = __uint_as_float(x.d[t][u >> 2][u & 3]);
#pragma unroll
        for (int v = 0; v < 4; ++v) accb[t][v] = fmaf((float)__mul24(c[v], ls[v]), cd, accb[t][v]);
      }
    }
    const float d[4] = {half_bits_to_float(f[r].d01 & 0xFFFF), half_bits_to_float(f[r].d01 >> 16),
                        half_bits_to_float(f[r].d23 & 0xFFFF), half_bits_to_float(f[r].d23 >> 16)};
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[r][t][v] = fmaf(accb[t][v], d[v], acc[r][t][v]);
  }
}

// Two column tiles on four waves: held to three workgroups per CU (168 registers per lane, 3
// dwords spilled; the LDS admits three): 17408 x 5120 M = 20 / 32 39.1 / 38.6 -> 35.9 / 35.5 us,
// 5120 x 17408 39.3 / 38.4 -> 36.4 / 36.2 (172 registers and two workgroups per CU before).
template <int NT, int RW, int KS>
__global__ void __launch_bounds__(64 * KS, KS == 4 && NT == 2 ? 3 : 1) gemm_iq3s_tile_kernel(const uint8_t* __restrict__ W, int64_t row_bytes,
                                                                 int nrows, int k, const uint8_t* __restrict__ xq,
                                                                 int nct, int n, void* __restrict__ y, int y_dtype,
                                                                 float* part, uint32_t* cnt) {
  static_assert((KS - 1) * RW * NT * 4 * 64 * 4 <= 2048 * 16, "wave partials fit the table region");
  static_assert(RW == 1, "the K split's slots hold one row tile");
  __shared__ uint4 table[2048];  // signed-grid table; the waves' partial sums at the end
  __shared__ uint4 trbuf[KS][kTrBytes / 16];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = lane >> 3, s = lane & 7;   // decode view
  const int j = lane & 15, q = lane >> 4;  // MFMA view
  const int ntiles = nrows / kTileRows;
  const int tile0 = blockIdx.x * RW;
  const int ct0 = blockIdx.y * NT;
  const int nb = k / kQK;
  // this workgroup's part of K (split z of S), then the wave's part of that
  const int S = (int)gridDim.z, z = (int)blockIdx.z;
  const int zb0 = z * nb / S, zb1 = (z + 1) * nb / S;
  const int b_begin = zb0 + wave * (zb1 - zb0) / KS, b_end = zb0 + (wave + 1) * (zb1 - zb0) / KS;
  const int64_t tile_bytes = (int64_t)kTileRows * row_bytes;
  const int tiles_here = ntiles - tile0 < RW ? ntiles - tile0 : RW;
  // every load stays inside the workgroup's tiles and the xq buffer: a missing tile of the last
  // workgroup re-reads its last tile (never stored), the prefetch past the wave's last block
  // re-reads that block
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(W + tile0 * tile_bytes, (uint32_t)(tiles_here * tile_bytes));
  const int sbase = (int)xq_scale_base(nct, nb);
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(xq, (uint32_t)xq_bytes((int64_t)nct * kXqCols, k));
  const uint8_t* tbl = (const uint8_t*)table;
  uint8_t* tr = (uint8_t*)trbuf[wave];
  const MmaOffs mo = mma_offsets(p, s, q, row_bytes);

  float acc[RW][NT][4];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[r][t][v] = 0.0f;

  MmaFrag fa[RW], fb[RW];
  XqFrag<NT> xa, xb;
  // column tiles past nct (last workgroup of the y grid) re-read column tile nct - 1 (never stored)
  int units[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) units[t] = (ct0 + t < nct ? ct0 + t : nct - 1) * nb;
  uint32_t toff[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) toff[r] = (uint32_t)((r < tiles_here ? r : tiles_here - 1) * tile_bytes);
  // Two blocks per iteration (an odd last block after the loop); every load feeds a use that is
  // not behind a branch of its own (the compiler sinks a load whose only use is conditional to
  // that use, which would serialise the prefetch). The prefetch past the wave's last block reads
  // zeros through an empty descriptor and is never used.
  const __amdgpu_buffer_rsrc_t nrs = buffer_rsrc(W, 0);
  const int b_last = b_end - 1;
  if (b_begin < b_end) {
    load_xq_frag<NT>(xrs, units, b_begin, sbase, lane, j, xa);
#pragma unroll
    for (int r = 0; r < RW; ++r) load_mma_frag(wrs, toff[r], nb, b_begin, mo, fa[r]);
  }
  iq3_table_to_lds<KS>(table, &kIq3sSignedMma, wave, lane);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int nblk = b_end - b_begin;
  int b = b_begin;
  for (int it = 0; it < nblk / 2; ++it, b += 2) {
    const int b2 = b + 2 < b_last ? b + 2 : b_last;
    const __amdgpu_buffer_rsrc_t rs2 = b + 2 < b_end ? wrs : nrs;
    load_xq_frag<NT>(xrs, units, b + 1, sbase, lane, j, xb);
#pragma unroll
    for (int r = 0; r < RW; ++r) load_mma_frag(wrs, toff[r], nb, b + 1, mo, fb[r]);
    __builtin_amdgcn_sched_barrier(0);  // the scheduler hoists the next block's decode (and its
                                        // wait) above these loads otherwise
    mma_block<NT, RW>(tbl, tr, fa, xa, p, s, q, j, acc);
    load_xq_frag<NT>(xrs, units, b2, sbase, lane, j, xa);
#pragma unroll
    for (int r = 0; r < RW; ++r) load_mma_frag(rs2, toff[r], nb, b + 2, mo, fa[r]);
    __builtin_amdgcn_sched_barrier(0);
    mma_block<NT, RW>(tbl, tr, fb, xb, p, s, q, j, acc);
  }
  if (nblk & 1) mma_block<NT, RW>(tbl, tr, fa, xa, p, s, q, j, acc);

  // partial sums of waves 1.. through LDS (the table is no longer read), added in wave order
  __syncthreads();
  float* red = (float*)table;
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[((((wave - 1) * RW + r) * NT + t) * 4 + v) * 64 + lane] = acc[r][t][v];
  }
  __syncthreads();
  if (wave != 0) return;
  float sum[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sum[t][v] = acc[0][t][v];
      for (int w2 = 1; w2 < KS; ++w2) sum[t][v] += red[(((w2 - 1) * NT + t) * 4 + v) * 64 + lane];
    }
  if (S > 1 && !split_fixup<NT>(sum, part, cnt, S, z, (size_t)blockIdx.x * gridDim.y + blockIdx.y, lane)) return;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int col = (ct0 + t) * kXqCols + j;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (col < n) store_y(y, (int64_t)col * nrows + (int64_t)tile0 * kTileRows + 4 * q + v, sum[t][v], y_dtype);
  }
}

template <int NT, int RW, int KS>
void launch_tile_gemm(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n, void* y,
                      int y_dtype, int split, float* part, uint32_t* cnt, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const dim3 grid((unsigned)((nrows / kTileRows + RW - 1) / RW), (unsigned)((nct + NT - 1) / NT), (unsigned)split);
  gemm_iq3s_tile_kernel<NT, RW, KS>
      <<<grid, 64 * KS, 0, stream>>>(W, row_bytes, nrows, k, xq, nct, n, y, y_dtype, part, cnt);
}

}  // namespace

// The tile GEMM's K split over workgroups (1: none; split_k.h). Two or three of its workgroups
// share a CU (49.6 KB of LDS each), so an uneven grid costs less than on the raw GEMM; the split
// pays on long K and on grids that leave most CUs idle. Measured on the op (quantise included,
// graph replayed), no split -> split: IQ3_S 5120 x 17408 (320 tiles, 68 blocks) M = 8 / 16 (2
// ways): 29.5 -> 27.6 / 29.5 -> 27.7 us, M = 24 / 32 / 48 (4 ways): 42.8 -> 37.9 / 42.8 -> 38.0 /
// 56.7 -> 48.9; 1024 x 5120 (64 tiles, 2 ways) M = 16 / 48: 9.9 -> 9.7 / 16.7 -> 14.2. At 20
// blocks on 384 tiles (6144 x 5120) a 2-way split loses (12.9 -> 14.2 us at M = 16, measured
// without the fixup).
int tile_split(int64_t nrows, int64_t k, int64_t n) {
  if (n <= 0) return 1;
  const int64_t tiles = nrows / kTileRows, nb = k / kQK, cus = device_cus();
  const int64_t groups = split_groups(tiles, n);
  if (groups >= 2 * cus) return 1;
  if (nb >= 48) return xq_col_tiles(n) >= 2 ? 4 : 2;
  return 2 * groups < cus && nb >= 16 ? 2 : 1;
}

// IQ3_S in the unit layout; nrows % 16 == 0; xq: X in the xq layout (launch_quantize_xq).
// Launch shapes measured at 17408 x 5120, 5120 x 17408 and 5120 x 5120: four waves per tile,
// eight for one column tile on matrices of fewer than 512 tiles (more waves per tile to fill
// the GPU; on more tiles eight waves lost: 17408 x 5120 M = 16 26.5 -> 28.1 us, 12288 x 5120
// 19.5 -> 20.4); above 64 activation rows the y grid walks groups of four column tiles. split_ws: the
// split's workspace (split_k.h) when tile_split(...) > 1, its counters zeroed.
hipError_t launch_gemm_packed_xq(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n,
                                 void* y, int y_dtype, void* split_ws, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const bool few = nrows / kTileRows < 512;
  const int split = tile_split(nrows, k, n);
  if (split > 1 && split_ws == nullptr) return hipErrorInvalidValue;
  float* part = (float*)split_ws;
  uint32_t* cnt = (uint32_t*)((uint8_t*)split_ws + split_part_bytes(split, nrows / kTileRows, n));
  // 2-3 column tiles unsplit on fewer than two tiles per CU: one column tile per workgroup, two or
  // three times the workgroups (each decodes its tile again). Measured on the op (graph
  // replays): IQ3_S M = 48 5120 x 6144 26.9 -> 23.1 us, 6144 x 5120 24.0 -> 23.5 (groups of two
  // column tiles: 27.4, 24.7); M = 32 5120 x 6144 21.1 -> 19.9, 6144 x 5120 19.0 -> 18.4
  const bool one_ct = nct <= 3 && split == 1 && nrows / kTileRows < 2 * device_cus();
  if (nct == 1 || one_ct) {
    if (few && nct == 1) launch_tile_gemm<1, 1, 8>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
    else launch_tile_gemm<1, 1, 4>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
  } else if (nct == 2) {
    launch_tile_gemm<2, 1, 4>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
  } else if (nct == 3) {
    launch_tile_gemm<3, 1, 4>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
  } else {
    launch_tile_gemm<4, 1, 4>(W, row_bytes, nrows, k, xq, n, y, y_dtype, split, part, cnt, stream);
  }
  return hipGetLastError();
}

}  // namespace gguf
