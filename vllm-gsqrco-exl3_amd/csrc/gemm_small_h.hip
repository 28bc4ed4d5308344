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

template <int TYPE, int RT, int NM>
__global__ void __launch_bounds__(64 * (2 * RT + NM), 4) gemm_small_h_kernel(const uint8_t* __restrict__ W,
                                                                             int64_t row_bytes, int nrows, int k,
                                                                             const uint8_t* __restrict__ xh, int nct,
                                                                             int n, void* __restrict__ y, int y_dtype) {
  constexpr bool IQ3 = TYPE == kIQ3_S;
  constexpr int ND = 2 * RT;       // decoding waves: tile w >> 1, half block w & 1
  constexpr int NT = 64 * (ND + NM);
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
  const int tile0 = blockIdx.x * RT;
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
    // Rows past the weight re-read its last tile / row (decoded, never stored). Past the end,
    // the loads re-read block nb - 1 and the decode repeats it, which leaves e and EF as they are.
    const int dt = wave >> 1, dh = wave & 1;
    const uint8_t* wp;
    if constexpr (IQ3) wp = W + (int64_t)min(tile0 + dt, ntiles - 1) * kTileRows * row_bytes;
    else wp = W + (int64_t)min((tile0 + dt) * 16 + j, nrows - 1) * row_bytes;
    float e = 1.0f;
    // the raw bytes of a block: two named sets, each refilled right after its decode and used
    // two steps later
    auto load_w = [&](int b, Raw& raw) {
      if constexpr (IQ3) load_step(raw, wp, row_bytes, nb, b, dh, j, q);
      else load_step(raw, wp + (int64_t)b * block_bytes(kQ4_K), dh, q);
    };
    auto decode = [&](int par, const Raw& raw) {
      uint8_t* Ab = A[par][dh];
      if constexpr (IQ3) decode_step_tb(raw, dh, (const uint8_t*)TB, Ab, RTs[par], EFs[par], e, dt, j, q);
      else decode_step(raw, dh, AM[par][dh], Ab, RTs[par], EFs[par], e, dt, j, q);
    };
    Raw r0, r1;
    load_w(0, r0);
    load_w(min(1, nb - 1), r1);
    decode(0, r0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(min(2, nb - 1), r0);
    lds_barrier();
    auto step = [&](int b, Raw& rdec) {
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
    return;
  }

  // ---- multiplier: column tile ct against the RT decoded tiles (past nct: the last one again,
  // never stored). The B operand and activation scale of each slice (and Q4_K's d x sum q per
  // half block) are refilled in place with the next block's once consumed: a copy of a value
  // still to be used would make the compiler wait for the refill.
  const int ctw = (int)blockIdx.y * NM + (wave - ND);
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
  f4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // block b from the A area of parity b & 1 with operand set o, refilled with block bn's
  auto compute = [&](int b, int bn, BSet& o) {
    const int par = b & 1;
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] *= *(const f4*)(RTs[par] + t * 16 + 4 * q);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        // all A operands of a quarter block (2 slices), then its MFMAs back to back, then the
        // FMAs: a chain of LDS read, MFMA and FMA per slice would be paid 8 times per block
        h8 a[2][RT];
#pragma unroll
        for (int uu = 0; uu < 2; ++uu)
#pragma unroll
          for (int t = 0; t < RT; ++t) a[uu][t] = *(const h8*)(A[par][h] + h_off(t, 2 * qq + uu, j, q));
        f4 p[2][RT];
#pragma unroll
        for (int uu = 0; uu < 2; ++uu)
#pragma unroll
          for (int t = 0; t < RT; ++t)
            p[uu][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[uu][t], __builtin_bit_cast(h8, o.bq[4 * h + 2 * qq + uu]),
                                                              zero, 0, 0, 0);
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
#pragma unroll
          for (int t = 0; t < RT; ++t) {
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
        for (int t = 0; t < RT; ++t) {
          const float am = AM[par][h][(t * 4 + q) * 16 + j];
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
  for (int t = 0; t < RT; ++t) {
    const int tile = tile0 + t;
    const f4 ef = *(const f4*)(EF + t * 16 + 4 * q);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = tile * 16 + 4 * q + v;
      if (col < n && tile < ntiles && row < nrows) store_y(y, (int64_t)col * nrows + row, acc[t][v] * ef[v], y_dtype);
    }
  }
}

template <int TYPE, int RT, int NM>
void launch_small_h_t(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xh, int n, void* y,
                      int y_dtype, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  const int ntiles = (nrows + 15) / 16;
  const dim3 grid((unsigned)((ntiles + RT - 1) / RT), (unsigned)((nct + NM - 1) / NM));
  gemm_small_h_kernel<TYPE, RT, NM><<<grid, 64 * (2 * RT + NM), 0, stream>>>(W, row_bytes, nrows, k, xh, nct, n, y,
                                                                             y_dtype);
}

template <int TYPE, int RT>
void launch_small_h_rt(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xh, int n, void* y,
                       int y_dtype, hipStream_t stream) {
  const int nct = (int)xq_col_tiles(n);
  if (nct <= 1) launch_small_h_t<TYPE, RT, 1>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
  else if (nct <= 2) launch_small_h_t<TYPE, RT, 2>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
  else launch_small_h_t<TYPE, RT, 4>(W, row_bytes, nrows, k, xh, n, y, y_dtype, stream);
}

}  // namespace

// Types the fp16 small GEMM serves: IQ3_S in the tile layout (packed) and Q4_K rows.
bool small_h_supported(int type, bool packed) { return packed ? type == kIQ3_S : type == kQ4_K; }

// xh: X in the xh layout (launch_quantize_xh / launch_q8_1_to_xh). Two row tiles per workgroup
// from 1024 tiles on (X read once per tile pair), one below (more workgroups on smaller weights).
hipError_t launch_gemm_small_h(int type, bool packed, const uint8_t* W, int64_t row_bytes, int nrows, int k,
                               const uint8_t* xh, int n, void* y, int y_dtype, hipStream_t stream) {
  if (!small_h_supported(type, packed)) return hipErrorInvalidValue;
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
