// Prefill GEMM (many activation rows) on int8 MFMA: Y[c, r] = sum_k X[c, k] * W[r, k].
//
// Replaces the reference's large-M products (the IQ3 tiled kernel's wide plans,
// lcpp_owned_iq3_mma.cu:1022-1055, and vendored MMQ, mmq.cuh / mmq-load-tiles.cuh:711,946) with a
// gfx950 design whose point is operand reuse:
//  * a workgroup of 4 waves owns a 128-row x 128-column output tile (8 x 8 MFMA tiles of 16 x 16);
//    wave (wr, wc) accumulates row tiles 4wr..4wr+3 x column tiles 4wc..4wc+3, so every A and B
//    operand it reads from LDS feeds four MFMAs;
//  * per 256-value K block the workgroup stages, in LDS,
//      - A: the block of its 128 weight rows decoded to int8, in MFMA operand order (row tile,
//        slice, row, 8-byte quarter slot swizzled by row so both the decoders' stores and the
//        operand reads are free of bank conflicts); each wave decodes two 16-row tiles;
//      - the per-(row, slice) sub-scales and per-row block scales the epilogue needs;
//      - B: the xq units (xq.h) of its 8 column tiles, copied by LDS DMA;
//  * one v_mfma_i32_16x16x32_i8 per (row tile, column tile, slice) is the reference's integer
//    slice dot; the per-slice epilogue and the block scale are those of the small GEMMs
//    (Q6_K: two MFMAs per slice, one per 16-value sub-scale; Q4_K: the min term);
//  * IQ3_S decodes through the 2 KB unsigned grid with the signs applied by VALU (the 32 KB
//    signed table would leave room for one workgroup per CU).
// Single-buffered: two workgroups per CU overlap one's staging with the other's MFMAs.
#include <type_traits>

#include "decode.h"
#include "iq3_tile.h"
#include "xh_decode.h"
#include "xq.h"

namespace gguf {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kPfRowTiles = 8;                  // 128 weight rows per workgroup
constexpr int kPfColTiles = 8;                  // 128 activation rows per workgroup
constexpr int kPfSlice = 528;                   // A bytes per (row tile, slice): 16 rows x 32 B + pad
constexpr int kPfATile = 8 * kPfSlice;          // A bytes per row tile (one block)
constexpr int kPfA = kPfRowTiles * kPfATile;    // 33,792
constexpr int kPfB = kPfColTiles * kXqUnit;     // 32,768
constexpr int kPfBS = kPfColTiles * kXqScaleUnit;  // 4,096
constexpr int kPfS = kPfRowTiles * 8 * 32;      // sub-scales: [tile][slice][s1 x16 | s2 x16] bytes
constexpr int kPfD = kPfRowTiles * 16 * 2 * 4;  // [tile][row][d, dmin] fp32

__device__ const Iq3sGrid kIq3sGridPf = kIq3sGrid;

// A slot of (row tile t, slice u, row j, quarter q): byte offset in the A area. The quarter's
// slot is q ^ (j >> 2) (as the small GEMM's transposition buffer).
__device__ __forceinline__ int a_off(int t, int u, int j, int q) {
  return t * kPfATile + u * kPfSlice + j * 32 + ((q ^ (j >> 2)) & 3) * 8;
}

// ------------------------------------------------------------------------- A staging, IQ3_S
// The lane (decode view L = 8p + s) decodes slice s of rows 2p, 2p+1 of one tile-block and stores
// the 8 quarters of each row; ex = sign nibble | qh << 4 of each 4-value group.
__device__ __forceinline__ uint32_t grid_signed(const uint32_t* grid, uint32_t qs, uint32_t ex) {
  return (uint32_t)apply_signs(grid[qs | ((ex >> 4) << 8)], ex & 0xF);
}

__device__ __forceinline__ void stage_iq3_tile(const uint8_t* tile, int64_t row_bytes, int nb, int b,
                                               const uint32_t* grid, uint8_t* A, uint8_t* S, float* D, int t, int lane) {
  const int p = lane >> 3, s = lane & 7;
  const Iq3Fields f = iq3_block_fields(nb, b), l = iq3_lane_fields(p & 1, s);
  const uint8_t* u = tile + (int64_t)(p >> 1) * kUnitRows * row_bytes;  // rows 2p, 2p+1: unit p >> 1
  const u32x4 qs = *(const u32x4*)(u + f.qs + l.qs);
  const uint2 e8 = *(const uint2*)(u + f.e8 + l.e8);
  const uint32_t l2 = *(const uint16_t*)(u + f.l2 + l.l2);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    uint32_t lo, hi;
    iq3_tile_ex(r == 0 ? e8.x : e8.y, l2, r, lo, hi);
    const uint32_t q0 = r == 0 ? qs[0] : qs[2], q1 = r == 0 ? qs[1] : qs[3];
    uint32_t w[8];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      w[g] = grid_signed(grid, (q0 >> (8 * g)) & 0xFF, (lo >> (8 * g)) & 0xFF);
      w[4 + g] = grid_signed(grid, (q1 >> (8 * g)) & 0xFF, (hi >> (8 * g)) & 0xFF);
    }
    const int j = 2 * p + r;
#pragma unroll
    for (int q = 0; q < 4; ++q) *(uint2*)(A + a_off(t, s, j, q)) = make_uint2(w[2 * q], w[2 * q + 1]);
    // sub-scale ls = 1 + 2 * nibble of (row j, slice s); SC byte 2 (s/2) + r of the row pair, nibble s & 1
    const uint32_t scb = u[f.sc + l.sc + 2 * (s >> 1) + r];
    S[(t * 8 + s) * 32 + j] = (uint8_t)(1 + 2 * ((scb >> (4 * (s & 1))) & 0xF));
    if (s == 0) D[(t * 16 + j) * 2] = half_bits_to_float(*(const uint16_t*)(u + f.d + l.d + 2 * r));
  }
}

// ------------------------------------------------------------------------- A staging, raw rows
// The lane (j = lane & 15, q = lane >> 4) decodes values 8q..8q+7 of every slice of row j of a
// 16-row tile (blk: row j's block), as the small raw GEMM's A operands.
template <int TYPE>
__device__ __forceinline__ void stage_raw_tile(const uint8_t* blk, bool valid, uint8_t* A, uint8_t* S, float* D,
                                               int t, int lane) {
  const int j = lane & 15, q = lane >> 4;
  uint32_t w0[8], w1[8];
  int s1[8], s2[8];
  float d = 0.0f, dmin = 0.0f;
  if (valid) {
    if constexpr (TYPE == kQ4_K) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint2 v = *(const uint2*)(blk + 16 + 32 * c + 8 * q);
        w0[2 * c] = v.x & 0x0F0F0F0Fu;
        w1[2 * c] = v.y & 0x0F0F0F0Fu;
        w0[2 * c + 1] = (v.x >> 4) & 0x0F0F0F0Fu;
        w1[2 * c + 1] = (v.y >> 4) & 0x0F0F0F0Fu;
      }
      const uint32_t dm = *(const uint32_t*)blk;
      d = half_bits_to_float(dm & 0xFFFF);
      dmin = half_bits_to_float(dm >> 16);
#pragma unroll
      for (int u = 0; u < 8; ++u) q4k_scale_min(blk, u, s1[u], s2[u]);
    } else if constexpr (TYPE == kIQ4_XS) {
      const int sh = 4 * (q >> 1);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint2 v = *(const uint2*)(blk + 8 + 16 * u + 8 * (q & 1));
        w0[u] = (uint32_t)iq4nl(v.x, sh);
        w1[u] = (uint32_t)iq4nl(v.y, sh);
        s1[u] = iq4xs_ls(blk, u);
        s2[u] = 0;
      }
      d = half_bits_to_float(ld16(blk));
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int n = u >> 2, sub = u & 3;
        const uint64_t l = ld64(blk + 64 * n + 32 * (sub & 1) + 8 * q);
        const uint64_t h = ld64(blk + 128 + 32 * n + 8 * q);
        const int lsh = 4 * (sub >> 1), hsh = 2 * sub;
        w0[u] = (uint32_t)sub32_bytes((((uint32_t)l >> lsh) & 0x0F0F0F0Fu) | ((((uint32_t)h >> hsh) & 0x03030303u) << 4));
        w1[u] = (uint32_t)sub32_bytes((((uint32_t)(l >> 32) >> lsh) & 0x0F0F0F0Fu) |
                                      ((((uint32_t)(h >> 32) >> hsh) & 0x03030303u) << 4));
        s1[u] = (int)(int8_t)blk[192 + 2 * u];
        s2[u] = (int)(int8_t)blk[193 + 2 * u];
      }
      d = half_bits_to_float(ld16(blk + 208));
    }
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) w0[u] = w1[u] = 0, s1[u] = s2[u] = 0;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) *(uint2*)(A + a_off(t, u, j, q)) = make_uint2(w0[u], w1[u]);
  if (q == 0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      S[(t * 8 + u) * 32 + j] = (uint8_t)s1[u];
      S[(t * 8 + u) * 32 + 16 + j] = (uint8_t)s2[u];
    }
    D[(t * 16 + j) * 2] = d;
    D[(t * 16 + j) * 2 + 1] = dmin;
  }
}

// ------------------------------------------------------------------------- the kernel
// W: weight rows (IQ3_S: the tile layout); xq: X in the xq layout (nct column tiles).
template <int TYPE, bool TILE>
__global__ void __launch_bounds__(256, 2) gemm_prefill_kernel(const uint8_t* __restrict__ W, int64_t row_bytes,
                                                              int nrows, int k, const uint8_t* __restrict__ xq,
                                                              int nct, int n, void* __restrict__ y, int y_dtype) {
  __shared__ __attribute__((aligned(16))) uint8_t A[kPfA];
  __shared__ __attribute__((aligned(16))) uint8_t B[kPfB + kPfBS];
  __shared__ __attribute__((aligned(16))) uint8_t S[kPfS];
  __shared__ __attribute__((aligned(16))) float D[kPfD / 4];
  __shared__ uint32_t grid[TILE ? 512 : 1];
  constexpr int BS = block_bytes(TYPE);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave >> 1, wc = wave & 1;
  const int j = lane & 15, q = lane >> 4;
  const int ntiles = (nrows + 15) / 16;
  const int tile0 = blockIdx.x * kPfRowTiles;
  const int ct0 = blockIdx.y * kPfColTiles;
  const int nb = k / kQK;
  const int sbase = (int)xq_scale_base(nct, nb);
  if constexpr (TILE) {
    for (int i = threadIdx.x; i < 512; i += 256) grid[i] = kIq3sGridPf.v[i];
    __syncthreads();  // every wave's decoder reads the whole grid
  }

  float acc[4][4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[r][t][v] = 0.0f;

  for (int b = 0; b < nb; ++b) {
    // ---- stage: B by LDS DMA (16 B per lane per instruction; column tiles past nct re-read the
    // last one, never stored), A and the scales by the waves' decoders
#pragma unroll
    for (int i = 0; i < kPfColTiles / 4; ++i) {
      const int tt = wave * (kPfColTiles / 4) + i;  // this wave copies column tiles 2w, 2w+1
      const int ct = ct0 + tt < nct ? ct0 + tt : nct - 1;
      const uint8_t* src = xq + ((int64_t)ct * nb + b) * kXqUnit;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        __builtin_amdgcn_global_load_lds((const void*)(src + c * 1024 + 16 * lane),
                                         (__attribute__((address_space(3))) void*)(B + tt * kXqUnit + c * 1024), 16,
                                         0, 0);
      // scales: 512 B = 32 lanes x 16 B
      const uint8_t* ssrc = xq + sbase + ((int64_t)ct * nb + b) * kXqScaleUnit;
      if (lane < 32)
        __builtin_amdgcn_global_load_lds((const void*)(ssrc + 16 * lane),
                                         (__attribute__((address_space(3))) void*)(B + kPfB + tt * kXqScaleUnit), 16,
                                         0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int t = wave * 2 + i;
      const int gt = tile0 + t < ntiles ? tile0 + t : ntiles - 1;
      if constexpr (TILE) {
        stage_iq3_tile(W + (int64_t)gt * kTileRows * row_bytes, row_bytes, nb, b, grid, A, S, D, t, lane);
      } else {
        const int row = gt * 16 + j;
        const bool valid = row < nrows;
        stage_raw_tile<TYPE>(W + (int64_t)(valid ? row : 0) * row_bytes + (int64_t)b * BS, valid, A, S, D, t, lane);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // ---- compute: wave (wr, wc) over its 4 x 4 MFMA tiles; the row's block scale d (and Q4_K's
    // dmin) is folded into each slice's factor so that one set of accumulators is live
    float dr[4][4], dmr[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * wr + r;
      const float4 dd0 = *(const float4*)(D + (t * 16 + 4 * q) * 2);      // d, dmin of rows 4q, 4q+1
      const float4 dd1 = *(const float4*)(D + (t * 16 + 4 * q + 2) * 2);  // rows 4q+2, 4q+3
      dr[r][0] = dd0.x; dr[r][1] = dd0.z; dr[r][2] = dd1.x; dr[r][3] = dd1.z;
      dmr[r][0] = dd0.y; dmr[r][1] = dd0.w; dmr[r][2] = dd1.y; dmr[r][3] = dd1.w;
    }
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      long a[4], bo[4];
      uint32_t s1w[4], s2w[4];
      uint32_t cw[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 4 * wr + r;
        a[r] = *(const long*)(A + a_off(t, u, j, q));
        s1w[r] = *(const uint32_t*)(S + (t * 8 + u) * 32 + 4 * q);
        if constexpr (TYPE == kQ4_K || TYPE == kQ6_K) s2w[r] = *(const uint32_t*)(S + (t * 8 + u) * 32 + 16 + 4 * q);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int tt = 4 * wc + c;
        bo[c] = *(const long*)(B + tt * kXqUnit + 64 * lane + 8 * u);
        cw[c] = *(const uint32_t*)(B + kPfB + tt * kXqScaleUnit + 32 * j + 4 * u);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int s1[4], s2[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          if constexpr (TYPE == kIQ3_S || TYPE == kQ4_K) s1[v] = (int)((s1w[r] >> (8 * v)) & 0xFF);
          else s1[v] = (int)(int8_t)((s1w[r] >> (8 * v)) & 0xFF);
          if constexpr (TYPE == kQ4_K) s2[v] = (int)((s2w[r] >> (8 * v)) & 0xFF);
          if constexpr (TYPE == kQ6_K) s2[v] = (int)(int8_t)((s2w[r] >> (8 * v)) & 0xFF);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float cd = TYPE == kQ4_K ? half_bits_to_float(cw[c] & 0xFFFF) : __uint_as_float(cw[c]);
          if constexpr (TYPE == kQ6_K) {
            const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(q < 2 ? a[r] : 0, bo[c], zero, 0, 0, 0);
            const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(q < 2 ? 0 : a[r], bo[c], zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v)
              acc[r][c][v] = fmaf((float)(__mul24(c0[v], s1[v]) + __mul24(c1[v], s2[v])), cd * dr[r][v], acc[r][c][v]);
          } else {
            const v4i cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[r], bo[c], zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[r][c][v] = fmaf((float)__mul24(cc[v], s1[v]), cd * dr[r][v], acc[r][c][v]);
            if constexpr (TYPE == kQ4_K) {
              const float cs = cd * (float)(int)(int16_t)(cw[c] >> 16);
#pragma unroll
              for (int v = 0; v < 4; ++v) acc[r][c][v] = fmaf(-(float)s2[v] * dmr[r][v], cs, acc[r][c][v]);
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // the next block's staging overwrites A, B, S, D
  }

#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = tile0 + 4 * wr + r;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int col = (ct0 + 4 * wc + c) * kXqCols + j;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = t * 16 + 4 * q + v;
        if (col < n && t < ntiles && row < nrows) store_y(y, (int64_t)col * nrows + row, acc[r][c][v], y_dtype);
      }
    }
  }
}

// ------------------------------------------------------------------------- fp16-operand variant
// IQ3_S and Q4_K: the weight value times its slice sub-scale is an integer of at most 465 (IQ3_S)
// or 945 (Q4_K), exact in fp16, and so are the activation's q8 values (the xh layout). One
// v_mfma_f32_16x16x32_f16 with a zero accumulator then returns sub-scale x integer slice dot
// exactly (every partial sum is an integer below 2^24), already in fp32, and the per-slice
// epilogue is one FMA by the activation scale. Q6_K: the 16-value sub-scale goes into the decoded
// operand, (q - 32) * sc, so a 32-value slice with two sub-scales is one MFMA as well (the int8
// GEMM needs one per sub-scale); that product is exact up to 2048 in magnitude and rounds to
// fp16 beyond (xh_decode.h). The row's block scale d is not applied per
// slice: each row's accumulator is held in units of the d of the block being summed (e, the last
// nonzero d; a block with d = 0 decodes to zeros), and is multiplied by e_prev / e_cur when a new
// block starts and by the last e at the end. The Q4_K min term, sum over slices of
// (-dmin * m / e) x (the fp16 sum of the slice's x, the MMQ form), is a K = 4 fp32 product per
// half block: one v_mfma_f32_16x16x4f32 into the accumulator.
//
// Workgroup: NW waves over 128 weight rows x 32 NW activation rows. Wave w owns column tiles 2w,
// 2w+1 against all 8 row tiles (16 accumulator tiles); its B operands (4 KB per column tile and
// half block) come straight from global memory into registers one step ahead, so only the
// decoded weights are shared through LDS, double-buffered, with one barrier per step (half
// block). Each wave decodes 8 / NW row tiles per step from raw bytes it loaded two steps ahead.
constexpr int kHA = kPfRowTiles * 4 * kHRegion;    // 33,280 per buffer (half a K block)

template <int TYPE, int NW>
__global__ void __launch_bounds__(64 * NW, 8 / NW) gemm_prefill_h_kernel(const uint8_t* __restrict__ W,
                                                                         int64_t row_bytes, int nrows, int k,
                                                                         const uint8_t* __restrict__ xh, int nct,
                                                                         int n, void* __restrict__ y, int y_dtype) {
  constexpr bool XXS = TYPE == kIQ3_XXS;
  constexpr bool IQ3 = TYPE == kIQ3_S || XXS;  // the unit layouts: a 16-row tile is 4 units
  constexpr bool MIN = TYPE == kQ4_K;  // the min term
  constexpr int TPW = 8 / NW;  // row tiles a wave decodes per step
  using Raw = typename std::conditional<
      XXS, RawXxsH,
      typename std::conditional<IQ3, RawIq3, typename std::conditional<MIN, RawQ4k, RawQ6k>::type>::type>::type;
  __shared__ __attribute__((aligned(16))) uint8_t A[2 * kHA];
  __shared__ __attribute__((aligned(16))) float RT[128];
  __shared__ __attribute__((aligned(16))) float EF[128];
  __shared__ __attribute__((aligned(16))) float AM[MIN ? 2 * 512 : 4];
  __shared__ __attribute__((aligned(16))) uint32_t GH[IQ3 ? 1024 : 4];
  __shared__ __attribute__((aligned(16))) uint2 SM[16];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int ntiles = (nrows + 15) / 16;
  const int tile0 = blockIdx.x * kPfRowTiles;
  const int nb = k / kQK;
  if constexpr (IQ3) {
    iq3_half_tables_to_lds(GH, SM, threadIdx.x, 64 * NW, XXS);
  }

  // this wave's column tiles (past nct: the last one again, never stored)
  const uint8_t* xv[2];
  const uint8_t* xs[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int ct = min((int)blockIdx.y * 2 * NW + 2 * wave + c, nct - 1);
    xv[c] = xh + (int64_t)ct * nb * kXhUnit + 16 * lane;
    xs[c] = xh + xh_scale_base(nct, nb) + (int64_t)ct * nb * kXhScaleUnit + 32 * j;
  }
  // B operands of the current step: slice u of column tile c, refilled with the next step's as
  // soon as the slice's MFMAs are issued; its scales (and Q4_K's sums) in a second set
  u32x4 bq[2][4];
  float dx[2][4], dxn[2][4], sq[2], sqn[2];
  auto load_bq = [&](int c, int u, int b, int h) {
    bq[c][u] = *(const u32x4*)(xv[c] + (int64_t)b * kXhUnit + 4096 * h + 1024 * u);
  };
  auto load_scales = [&](int b, int h) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const f4 v = *(const f4*)(xs[c] + (int64_t)b * kXhScaleUnit + 16 * h);
      dxn[c][0] = v[0];
      dxn[c][1] = v[1];
      dxn[c][2] = v[2];
      dxn[c][3] = v[3];
      if constexpr (MIN) sqn[c] = *(const float*)(xs[c] + (int64_t)b * kXhScaleUnit + 512 + 16 * h + 4 * q);
    }
  };
  auto take_scales = [&]() {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int u = 0; u < 4; ++u) dx[c][u] = dxn[c][u];
      sq[c] = sqn[c];
    }
  };
  // this wave's decode rows (tiles past the weight's end, rows past nrows: copies, never stored)
  const uint8_t* wp[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int t = wave * TPW + i;
    if constexpr (IQ3) {
      wp[i] = W + (int64_t)min(tile0 + t, ntiles - 1) * kTileRows * row_bytes;
    } else {
      wp[i] = W + (int64_t)min((tile0 + t) * 16 + j, nrows - 1) * row_bytes;
    }
  }
  Raw raw[TPW];
  float e[TPW];
  auto load_w = [&](int b, int h) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      if constexpr (IQ3) load_step(raw[i], wp[i], row_bytes, nb, b, h, j, q);
      else load_step(raw[i], wp[i] + (int64_t)b * block_bytes(TYPE), h, q);
    }
  };
  auto decode = [&](int h) {
    uint8_t* Ab = A + h * kHA;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int t = wave * TPW + i;
      if constexpr (IQ3) decode_step(raw[i], h, GH, SM, Ab, RT, EF, e[i], t, j, q);
      else if constexpr (MIN) decode_step(raw[i], h, AM + h * 512, Ab, RT, EF, e[i], t, j, q);
      else decode_step(raw[i], h, Ab, RT, EF, e[i], t, j, q);
    }
  };

  f4 acc[8][2];
#pragma unroll
  for (int r = 0; r < 8; ++r) acc[r][0] = acc[r][1] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // One step: 4 slices x 8 row tiles x 2 column tiles. Software-pipelined: the next A operand is
  // read while the current pair of MFMAs runs, and a pair's results are folded into acc one
  // row tile later. nb_, nh: the step whose B operands refill the registers.
  auto compute = [&](int h, int bnext, int hnext) {
    const uint8_t* Ab = A + h * kHA;
    if (h == 0) {  // a new block: rescale every row to its e
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const f4 rt = *(const f4*)(RT + r * 16 + 4 * q);
        acc[r][0] *= rt;
        acc[r][1] *= rt;
      }
    }
    h8 a = *(const h8*)(Ab + h_off(0, 0, j, q));
    f4 p0 = zero, p1 = zero;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int rn = r == 7 ? 0 : r + 1, un = r == 7 ? u + 1 : u;
        h8 an = a;
        if (un < 4) an = *(const h8*)(Ab + h_off(rn, un, j, q));
        const f4 n0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8, bq[0][u]), zero, 0, 0, 0);
        const f4 n1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8, bq[1][u]), zero, 0, 0, 0);
        if (u > 0 || r > 0) {
          const int rp = r == 0 ? 7 : r - 1, upv = r == 0 ? u - 1 : u;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            acc[rp][0][v] = fmaf(p0[v], dx[0][upv], acc[rp][0][v]);
            acc[rp][1][v] = fmaf(p1[v], dx[1][upv], acc[rp][1][v]);
          }
        }
        p0 = n0;
        p1 = n1;
        a = an;
      }
      load_bq(0, u, bnext, hnext);  // slice u's operands are consumed: the next step's
      load_bq(1, u, bnext, hnext);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc[7][0][v] = fmaf(p0[v], dx[0][3], acc[7][0][v]);
      acc[7][1][v] = fmaf(p1[v], dx[1][3], acc[7][1][v]);
    }
    if constexpr (MIN) {  // the min term of the half block
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float am = AM[h * 512 + (r * 4 + q) * 16 + j];
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(am, sq[c], acc[r][c], 0, 0, 0);
      }
    }
  };

#pragma unroll
  for (int i = 0; i < TPW; ++i) e[i] = 1.0f;
  load_w(0, 0);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    load_bq(0, u, 0, 0);
    load_bq(1, u, 0, 0);
  }
  load_scales(0, 0);
  if constexpr (IQ3) __syncthreads();  // the decode tables
  decode(0);
  load_w(0, 1);
  take_scales();
  __syncthreads();
  for (int b = 0; b < nb; ++b) {
    const int bn = min(b + 1, nb - 1);  // past the end: block nb - 1 again (never computed)
    // sched_barrier: the decode's arithmetic on the raw bytes stays after the MFMAs (hoisted
    // into them it makes the whole step wait for the raw loads of the step after)
    load_scales(b, 1);
    compute(0, b, 1);
    __builtin_amdgcn_sched_barrier(0);
    decode(1);
    load_w(bn, 0);
    take_scales();
    __syncthreads();
    load_scales(bn, 0);
    compute(1, bn, 0);
    __builtin_amdgcn_sched_barrier(0);
    decode(0);  // at the last block a repeat of it, which leaves e and EF as they are
    load_w(bn, 1);
    take_scales();
    __syncthreads();
  }

  const int col0 = ((int)blockIdx.y * 2 * NW + 2 * wave) * kXqCols + j;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int t = tile0 + r;
    const f4 ef = *(const f4*)(EF + r * 16 + 4 * q);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int col = col0 + c * kXqCols;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = t * 16 + 4 * q + v;
        if (col < n && t < ntiles && row < nrows) store_y(y, (int64_t)col * nrows + row, acc[r][c][v] * ef[v], y_dtype);
      }
    }
  }
}

template <int TYPE, int NW>
void launch_prefill_h_t(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xh, int n, void* y,
                        int y_dtype, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const int ntiles = (nrows + 15) / 16;
  const dim3 grid((unsigned)((ntiles + kPfRowTiles - 1) / kPfRowTiles), (unsigned)((nct + 2 * NW - 1) / (2 * NW)));
  gemm_prefill_h_kernel<TYPE, NW><<<grid, 64 * NW, 0, stream>>>(W, row_bytes, nrows, k, xh, nct, n, y, y_dtype);
}

template <int TYPE>
void launch_prefill_h(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xh, int n, void* y,
                      int y_dtype, hipStream_t stream) {
  const int64_t groups = (int64_t)((nrows + 127) / 128) * ((xq_col_tiles(n) + 15) / 16);
  if (groups >= 256) launch_prefill_h_t<TYPE, 8>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
  else launch_prefill_h_t<TYPE, 4>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
}

template <int TYPE, bool TILE>
void launch_prefill_t(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n, void* y,
                      int y_dtype, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const int ntiles = (nrows + 15) / 16;
  const dim3 grid((unsigned)((ntiles + kPfRowTiles - 1) / kPfRowTiles), (unsigned)((nct + kPfColTiles - 1) / kPfColTiles));
  gemm_prefill_kernel<TYPE, TILE><<<grid, 256, 0, stream>>>(W, row_bytes, nrows, k, xq, nct, n, y, y_dtype);
}

}  // namespace

// Whether the prefill GEMM of this type takes X in the xh layout (else xq).
bool prefill_uses_xh(int type, bool packed) { return packed || type == kQ4_K || type == kQ6_K; }

// Large-M products; xq: X in the xq layout, or the xh layout where prefill_uses_xh. packed: IQ3_S
// or IQ3_XXS in its unit layout (nrows % 16 == 0).
hipError_t launch_gemm_prefill(int type, bool packed, const uint8_t* W, int64_t row_bytes, int nrows, int k,
                               const uint8_t* xq, int n, void* y, int y_dtype, hipStream_t stream) {
  if (packed) {
    if (type == kIQ3_XXS) launch_prefill_h<kIQ3_XXS>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream);
    else launch_prefill_h<kIQ3_S>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream);
  } else {
    switch (type) {
      case kQ4_K: launch_prefill_h<kQ4_K>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream); break;
      case kIQ4_XS: launch_prefill_t<kIQ4_XS, false>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream); break;
      case kQ6_K: launch_prefill_h<kQ6_K>(W, row_bytes, nrows, k, xq, n, y, y_dtype, stream); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

}  // namespace gguf
