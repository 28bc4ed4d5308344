// Small-batch GEMM on fp16 MFMA for IQ3_S (tile layout) and Q4_K rows: Y[c, r] = sum_k X[c, k] *
// W[r, k] for 64..255 activation rows (product ops below the prefill GEMM's rows).
//
// Replaces the reference's tiled products at these row counts (lcpp_owned_iq3_mma.cu:614-1096 for
// packed IQ3_S, vendored MMQ for Q4_K) with a gfx950 design on the exact fp16 route of the prefill
// GEMM (xh_decode.h): a weight value times its slice sub-scale is an exact fp16 integer, so one
// v_mfma_f32_16x16x32_f16 returns sub-scale x integer slice dot exactly in fp32 and the per-slice
// epilogue is one FMA by the activation scale (the int8-MFMA route needs an integer multiply, a
// conversion and an FMA per output element and slice).
//  * A workgroup owns RT (1 or 2) 16-row tiles and NM (1, 2 or 4) column tiles of 16 activation
//    rows (grid y walks groups of NM column tiles). Its 2 RT decoder waves and NM multiplier waves
//    work on consecutive K blocks: while the multipliers use block b from one LDS A area, decoder
//    w writes half block w & 1 of row tile w >> 1 of block b + 1 into the other (one row slice of
//    32 values per lane), with one LDS-only barrier per block. Each role runs its own loop, so no
//    load sits behind a branch.
//  * Multiplier w's B operands (xh layout, 1 KB per slice) and activation scales come from global
//    memory into two named register sets, each refilled two blocks ahead as its slices are
//    consumed: X is read once per workgroup, the weights once per column-tile group.
//  * IQ3_S decodes through the signed-grid table biased by 128, in LDS (one 4-byte read per 4
//    values); Q4_K by byte permutes. Q4_K's min term is one v_mfma_f32_16x16x4f32 per (tile,
//    half block).
#include <type_traits>

#include "xh_decode.h"
#include "xq.h"

namespace gguf {

namespace {

// The signed-grid table (iq3_tile.h) with every byte biased by 128 (grid value +- 15 -> 113..143):
// a byte permute turns two biased bytes into the fp16 numbers 1024 + byte, and one packed FMA by
// the sub-scale ls with addend -1152 ls gives value x ls exactly (|value x ls| <= 465; 1152 ls is
// a multiple of 128 below 2^16, exact in fp16). One 4-byte table read per 4 values: the fp16 grid
// plus sign masks of the prefill decode take two 8-byte reads, and LDS bandwidth bounds this GEMM.
constexpr Iq3sSignedTable make_iq3s_biased_table() {
  Iq3sSignedTable t = make_iq3s_signed_table();
  for (int i = 0; i < 8192; ++i) t.v[i] ^= 0x80808080u;
  return t;
}
__device__ const Iq3sSignedTable kIq3sBiased = make_iq3s_biased_table();

// decode_step for IQ3_S (same lane mapping, A layout and block-scale handling) through the
// biased table in LDS (tbl)
__device__ __forceinline__ void decode_step_tb(const RawIq3& w, int h, const uint8_t* tbl, uint8_t* A, float* RT,
                                               float* EF, float& e, int t, int j, int sp) {
  const int s = 4 * h + sp;
  const float d = half_bits_to_float(w.d);
  if (h == 0) next_scale(d, e, RT, EF, t * 16 + j);
  uint32_t lo, hi;
  iq3_tile_ex(w.e8, w.l2, j & 1, lo, hi);
  const uint32_t nib = (w.sc >> (4 * (s & 1))) & 0xF;
  const _Float16 ls = d != 0.0f ? (_Float16)(float)(1 + 2 * nib) : (_Float16)0.0f;
  const h2 mul = {ls, ls};
  const h2 off = mul * (_Float16)(-1152.0f);
  int g[8];
  tile_lookup2(tbl, __builtin_amdgcn_perm(lo, w.qs.x, 0x05010400u), g[0], g[1]);
  tile_lookup2(tbl, __builtin_amdgcn_perm(lo, w.qs.x, 0x07030602u), g[2], g[3]);
  tile_lookup2(tbl, __builtin_amdgcn_perm(hi, w.qs.y, 0x05010400u), g[4], g[5]);
  tile_lookup2(tbl, __builtin_amdgcn_perm(hi, w.qs.y, 0x07030602u), g[6], g[7]);
  uint32_t v[16];
#pragma unroll
  for (int gg = 0; gg < 8; ++gg) {
    const uint32_t x = (uint32_t)g[gg];
    v[2 * gg] = h2_bits(__builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)), mul, off));
    v[2 * gg + 1] = h2_bits(__builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)), mul, off));
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *(uint4*)(A + h_off(t, sp, j, q)) = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

// Workgroup barrier that orders LDS only: __syncthreads()'s fences also order global memory,
// for which the compiler waits for the loads still in flight (the prefetch of the next steps).
// The scheduling barriers keep the next step's arithmetic (and its waits for loads) after it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  __builtin_amdgcn_sched_barrier(0);
}

// RANGE: workgroup g owns the row tiles [g T / G, (g + 1) T / G) of the T tiles (at most RT; one
// workgroup per CU on the 27B-class weights, X read once per CU), else tiles [RT g, RT g + RT).
// DPT decoder waves per row tile: 2 (each one half block per step) or 1 (both halves).
template <int TYPE, int RT, int NM, int DPT, bool RANGE, int MW = 1>
__global__ void __launch_bounds__(64 * (DPT * RT + NM * MW), RANGE ? 1 : 4) gemm_small_h_kernel(
    const uint8_t* __restrict__ W, int64_t row_bytes, int nrows, int k, const uint8_t* __restrict__ xh, int nct, int n,
    void* __restrict__ y, int y_dtype) {
  constexpr bool IQ3 = TYPE == kIQ3_S;
  constexpr int ND = DPT * RT;     // decoding waves: tile w / DPT, half block w % DPT (DPT = 2) or both
  constexpr int NT = 64 * (ND + NM * MW);
  constexpr int TPM = (RT + MW - 1) / MW;  // row tiles per multiplier wave: MW waves share a column tile
  constexpr int kHalf = RT * 4 * kHRegion;  // A bytes of one half block of the RT tiles
  using Raw = typename std::conditional<IQ3, RawIq3, RawQ4k>::type;
  __shared__ __attribute__((aligned(16))) uint8_t A[2][2][kHalf];  // [block parity][half]
  __shared__ __attribute__((aligned(16))) float RTs[2][RT * 16];
  __shared__ __attribute__((aligned(16))) float EFs[2][RT * 16];
  __shared__ __attribute__((aligned(16))) float AM[IQ3 ? 1 : 2][2][RT * 64];
  __shared__ __attribute__((aligned(16))) uint4 TB[IQ3 ? 2048 : 1];  // the biased table
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int ntiles = (nrows + 15) / 16;
  int tile0, tile1;  // the workgroup's row tiles
  if constexpr (RANGE) {
    tile0 = (int)(blockIdx.x * (uint32_t)ntiles / gridDim.x);
    tile1 = (int)((blockIdx.x + 1) * (uint32_t)ntiles / gridDim.x);
  } else {
    tile0 = blockIdx.x * RT;
    tile1 = min(tile0 + RT, ntiles);
  }
  const int nb = k / kQK;
  if constexpr (IQ3) {
    // all loads first, then the stores (indices past the table repeat its last entry)
    constexpr int TPT = (2048 + NT - 1) / NT;
    uint4 tv[TPT];
#pragma unroll
    for (int i = 0; i < TPT; ++i) tv[i] = ((const uint4*)kIq3sBiased.v)[min((int)threadIdx.x + i * NT, 2047)];
#pragma unroll
    for (int i = 0; i < TPT; ++i) TB[min((int)threadIdx.x + i * NT, 2047)] = tv[i];
    lds_barrier();
  }

  if (wave < ND) {
    // ---- decoder: block b + 1 into the A area of its parity while the multipliers use block b.
    // Tiles past the workgroup's last re-read it, rows past the weight its last row (decoded,
    // never stored). Past the end, the loads re-read block nb - 1 and the decode repeats it, which
    // leaves e and EF as they are.
    const int dt = wave / DPT;
    const int dtile = min(tile0 + dt, tile1 - 1);
    const uint8_t* wp;
    if constexpr (IQ3) wp = W + (int64_t)dtile * kTileRows * row_bytes;
    else wp = W + (int64_t)min(dtile * 16 + j, nrows - 1) * row_bytes;
    float e = 1.0f;
    // the raw bytes of a block (per half this wave decodes): two named sets, each refilled right
    // after its decode and used two steps later
    constexpr int NH = 2 / DPT;
    const int h0 = DPT == 2 ? (wave & 1) : 0;
    struct RawSet {
      Raw r[NH];
    };
    auto load_w = [&](int b, RawSet& raw) {
#pragma unroll
      for (int i = 0; i < NH; ++i) {
        const int h = h0 + i;
        if constexpr (IQ3) load_step(raw.r[i], wp, row_bytes, nb, b, h, j, q);
        else load_step(raw.r[i], wp + (int64_t)b * block_bytes(kQ4_K), h, q);
      }
    };
    auto decode = [&](int par, const RawSet& raw) {
#pragma unroll
      for (int i = 0; i < NH; ++i) {
        const int h = h0 + i;
        uint8_t* Ab = A[par][h];
        if constexpr (IQ3) decode_step_tb(raw.r[i], h, (const uint8_t*)TB, Ab, RTs[par], EFs[par], e, dt, j, q);
        else decode_step(raw.r[i], h, AM[par][h], Ab, RTs[par], EFs[par], e, dt, j, q);
      }
    };
    if constexpr (DPT == 2) {
      RawSet r0, r1;
      load_w(0, r0);
      load_w(min(1, nb - 1), r1);
      decode(0, r0);
      __builtin_amdgcn_sched_barrier(0);
      load_w(min(2, nb - 1), r0);
      lds_barrier();
      auto step = [&](int b, RawSet& rdec) {
        decode((b & 1) ^ 1, rdec);
        __builtin_amdgcn_sched_barrier(0);
        load_w(min(b + 3, nb - 1), rdec);
        lds_barrier();
      };
      int b = 0;
      for (; b + 1 < nb; b += 2) {
        step(b, r1);
        step(b + 1, r0);
      }
      if (b < nb) step(b, r1);
    } else {
      // three named sets: block b + 1 decoded while blocks b + 2 and b + 3 load
      RawSet r0, r1, r2;
      load_w(0, r0);
      load_w(min(1, nb - 1), r1);
      load_w(min(2, nb - 1), r2);
      __builtin_amdgcn_sched_barrier(0);
      decode(0, r0);
      __builtin_amdgcn_sched_barrier(0);
      load_w(min(3, nb - 1), r0);
      __builtin_amdgcn_sched_barrier(0);
      lds_barrier();
      auto step = [&](int b, RawSet& rdec) {
        decode((b & 1) ^ 1, rdec);
        __builtin_amdgcn_sched_barrier(0);
        load_w(min(b + 4, nb - 1), rdec);
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();
      };
      int b = 0;
      for (; b + 2 < nb; b += 3) {
        step(b, r1);
        step(b + 1, r2);
        step(b + 2, r0);
      }
      if (b < nb) step(b, r1);
      if (b + 1 < nb) step(b + 1, r2);
    }
    return;
  }

  // ---- multiplier: column tile ct against its row tiles tm + MW i of the RT decoded tiles (past
  // nct: the last column tile again, past RT: tile RT - 1 again; never stored). The B operand and activation scale of each slice (and Q4_K's d x sum q per
  // half block) are refilled in place with the next block's once consumed: a copy of a value
  // still to be used would make the compiler wait for the refill.
  const int mw = wave - ND, tm = mw % MW;
  const int ctw = (int)blockIdx.y * NM + mw / MW;
  int tix[TPM];  // the multiplier's row tiles in the decoded set
#pragma unroll
  for (int i = 0; i < TPM; ++i) tix[i] = min(tm + MW * i, RT - 1);
  const int ct = min(ctw, nct - 1);
  const uint8_t* xv = xh + (int64_t)ct * nb * kXhUnit + 16 * lane;
  const uint8_t* xs = xh + xh_scale_base(nct, nb) + (int64_t)ct * nb * kXhScaleUnit + 32 * j;
  // two named sets (blocks of even and odd index), each refilled in place with the block two on
  // once consumed: one step of prefetch is shorter than the load latency under this traffic
  struct BSet {
    u32x4 bq[8];
    float dq[8], sqv[2];
  };
  auto load_b = [&](BSet& o, int s, int b) {
    o.bq[s] = *(const u32x4*)(xv + (int64_t)b * kXhUnit + 1024 * s);
    o.dq[s] = *(const float*)(xs + (int64_t)b * kXhScaleUnit + 4 * s);
    if constexpr (!IQ3)
      if ((s & 3) == 0) o.sqv[s >> 2] = *(const float*)(xs + (int64_t)b * kXhScaleUnit + 512 + 4 * (s + q));
  };
  f4 acc[TPM];
#pragma unroll
  for (int t = 0; t < TPM; ++t) acc[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // block b from the A area of parity b & 1 with operand set o, refilled with block bn's
  auto compute = [&](int b, int bn, BSet& o) {
    const int par = b & 1;
#pragma unroll
    for (int t = 0; t < TPM; ++t) acc[t] *= *(const f4*)(RTs[par] + tix[t] * 16 + 4 * q);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        // all A operands of a quarter block (2 slices), then its MFMAs back to back, then the
        // FMAs: a chain of LDS read, MFMA and FMA per slice would be paid 8 times per block
        h8 a[2][TPM];
#pragma unroll
        for (int uu = 0; uu < 2; ++uu)
#pragma unroll
          for (int t = 0; t < TPM; ++t) a[uu][t] = *(const h8*)(A[par][h] + h_off(tix[t], 2 * qq + uu, j, q));
        f4 p[2][TPM];
#pragma unroll
        for (int uu = 0; uu < 2; ++uu)
#pragma unroll
          for (int t = 0; t < TPM; ++t)
            p[uu][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[uu][t], __builtin_bit_cast(h8, o.bq[4 * h + 2 * qq + uu]),
                                                              zero, 0, 0, 0);
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
#pragma unroll
          for (int t = 0; t < TPM; ++t) {
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[t][v] = fmaf(p[uu][t][v], o.dq[4 * h + 2 * qq + uu], acc[t][v]);
            // keeps the FMAs here: the compiler otherwise sinks them to the next block's use of
            // acc, past the barrier, with every MFMA result live (and spilled) meanwhile
            asm volatile("" : "+v"(acc[t]));
          }
        }
      }
      if constexpr (!IQ3) {  // the min term of the half block
#pragma unroll
        for (int t = 0; t < TPM; ++t) {
          const float am = AM[par][h][(tix[t] * 4 + q) * 16 + j];
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(am, o.sqv[h], acc[t], 0, 0, 0);
          asm volatile("" : "+v"(acc[t]));
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) load_b(o, 4 * h + u, bn);
    }
  };
  BSet o0, o1;
#pragma unroll
  for (int s = 0; s < 8; ++s) load_b(o0, s, 0);
#pragma unroll
  for (int s = 0; s < 8; ++s) load_b(o1, s, min(1, nb - 1));
  lds_barrier();  // block 0 decoded
  // past the end the refills re-read block nb - 1 (never used)
  int b = 0;
  for (; b + 1 < nb; b += 2) {
    compute(b, min(b + 2, nb - 1), o0);
    lds_barrier();
    compute(b + 1, min(b + 3, nb - 1), o1);
    lds_barrier();
  }
  if (b < nb) {
    compute(b, nb - 1, o0);
    lds_barrier();
  }

  if (ctw >= nct) return;
  const float* EF = EFs[(nb - 1) & 1];
  const int col = ctw * kXqCols + j;
#pragma unroll
  for (int t = 0; t < TPM; ++t) {
    if (tm + MW * t >= RT) break;
    const int tile = tile0 + tix[t];
    const f4 ef = *(const f4*)(EF + tix[t] * 16 + 4 * q);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = tile * 16 + 4 * q + v;
      if (col < n && tile < tile1 && row < nrows) store_y(y, (int64_t)col * nrows + row, acc[t][v] * ef[v], y_dtype);
    }
  }
}

template <int TYPE, int RT, int NM, int DPT, bool RANGE, int MW = 1>
void launch_small_h_t(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xh, int n, void* y,
                      int y_dtype, unsigned gx, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const dim3 grid(gx, (unsigned)((nct + NM - 1) / NM));
  gemm_small_h_kernel<TYPE, RT, NM, DPT, RANGE, MW><<<grid, 64 * (DPT * RT + NM * MW), 0, stream>>>(
      W, row_bytes, nrows, k, xh, nct, n, y, y_dtype);
}

template <int TYPE, int RT>
void launch_small_h_rt(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xh, int n, void* y,
                       int y_dtype, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const unsigned gx = (unsigned)(((nrows + 15) / 16 + RT - 1) / RT);
  if (nct <= 1) launch_small_h_t<TYPE, RT, 1, 2, false>(W, row_bytes, nrows, k, xh, n, y, y_dtype, gx, stream);
  else if (nct <= 2) launch_small_h_t<TYPE, RT, 2, 2, false>(W, row_bytes, nrows, k, xh, n, y, y_dtype, gx, stream);
  else launch_small_h_t<TYPE, RT, 4, 2, false>(W, row_bytes, nrows, k, xh, n, y, y_dtype, gx, stream);
}

// one workgroup per CU over at most kRangeTiles row tiles each, 1..3 column tiles
constexpr int kRangeTiles = 5;

}  // namespace

// Types the fp16 small GEMM serves: IQ3_S in the unit layout (packed) and Q4_K rows.
bool small_h_supported(int type, bool packed) { return packed ? type == kIQ3_S : type == kQ4_K; }

// The range plan: 2..3 column tiles on weights of 4 to kRangeTiles row tiles per CU: every CU's
// workgroup decodes its 4-5 tiles once per block for all columns and reads X once. Measured at
// 17408 x 5120 (op level, quantise included) against the int8 small GEMM: IQ3_S packed 48 rows
// 42.9 against 50.1 us, 32 rows 40.2 against 39.3; Q4_K 48 rows 41.8 against 66.8, 32 rows 39.6
// against 51.4, 16 rows 36.8 against 28.7 (one column tile stays on the int8 GEMM). With fewer
// tiles per CU the int8 GEMM's grid is the faster one: 6144 x 5120 (1.5 tiles per CU), IQ3_S 48
// rows 39.8 us on the range plan against 19.0 us for 32 rows on the int8 GEMM.
bool small_h_range(int type, int64_t nrows, int64_t n) {
  const int64_t tiles = (nrows + 15) / 16, cus = device_cus();
  const int64_t from = type == kIQ3_S ? 33 : 17;
  return n >= from && n <= 3 * 16 && tiles >= 4 * cus && tiles <= kRangeTiles * cus;
}

// xh: X in the xh layout (launch_quantize_xh / launch_q8_1_to_xh). The range plan where it
// applies; else two row tiles per workgroup from 1024 tiles on (X read once per tile pair), one
// below (more workgroups on smaller weights).
hipError_t launch_gemm_small_h(int type, bool packed, const uint8_t* W, int64_t row_bytes, int nrows, int k,
                               const uint8_t* xh, int n, void* y, int y_dtype, hipStream_t stream) {
  if (!small_h_supported(type, packed)) return hipErrorInvalidValue;
  if (small_h_range(type, nrows, n)) {
    const int nct = (int)xq_col_tiles(n);
    const unsigned gx = (unsigned)device_cus();
#define GGUF_RANGE(T)                                                                                                      \
  if (nct <= 2) launch_small_h_t<T, kRangeTiles, 2, 1, true, 1>(W, row_bytes, nrows, k, xh, n, y, y_dtype, gx, stream); \
  else launch_small_h_t<T, kRangeTiles, 3, 1, true, 1>(W, row_bytes, nrows, k, xh, n, y, y_dtype, gx, stream);
    if (type == kIQ3_S) {
      GGUF_RANGE(kIQ3_S)
    } else {
      GGUF_RANGE(kQ4_K)
    }
#undef GGUF_RANGE
    return hipGetLastError();
  }
  const bool two = (nrows + 15) / 16 >= 1024;
  if (type == kIQ3_S) {
    if (two) launch_small_h_rt<kIQ3_S, 2>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
    else launch_small_h_rt<kIQ3_S, 1>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
  } else {
    if (two) launch_small_h_rt<kQ4_K, 2>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
    else launch_small_h_rt<kQ4_K, 1>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
  }
  return hipGetLastError();
}

}  // namespace gguf
