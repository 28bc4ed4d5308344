// Decode GEMV for 1..8 activation rows on GGUF bytes: Y[c, r] = sum_k X[c, k] * W[r, k].
//
// Replaces the reference's 1..8-row products (vendored MMVQ mul_mat_vec_q, mmvq.cu:600-760; the
// owned dp4a kernels lcpp_shim.cu:498-607 and lcpp_owned_k4.cu:116-269) with one wave64 design:
//  * a workgroup of 4 waves owns 4*RW weight rows; lane l of a wave takes the 32-value slices
//    l, l+64, ... of the K axis, so one q8_1 block of X per lane per step is loaded once and
//    reused for the wave's RW rows;
//  * each lane decodes its slice of each row into 8 int8x4 words (decode.h) and multiplies with
//    v_dot4_i32_i8 (__builtin_amdgcn_sdot4); the integer slice dot is scaled in fp32 and added to
//    a per-lane accumulator;
//  * a 64-lane xor butterfly sums each (row, column) accumulator at the end.
// The integer slice sums equal the reference's vec_dot sumi bit for bit; only the fp32 order in
// which a row's slice terms are added differs (lane-strided, then the butterfly).
#include <type_traits>

#include <algorithm>

#include "decode.h"
#include "gemv_x.h"

namespace gguf {

constexpr int kGemvWaves = 4;


// The slice term of one (row, column) pair in the reference's decode-op (MMVQ) arithmetic, from
// the slice's decoded words w, the column's q8 words x, d8 and (Q4_K, Q2_K) q8 sums:
//   IQ3_S, IQ4_XS  (float)(sumi * ls) * (d * d8)                    vecdotq.cuh:1211-1248,1357-1380
//   Q4_K           (d * sc * sumi - dmin * m * sum q8) * d8         vecdotq.cuh:508-530
//   Q6_K           (float)(sc_a * sumi_a + sc_b * sumi_b) * (d * d8) vecdotq.cuh:627-648
//   Q2_K           d8 * (d * sum sc_h sumi_h - dmin * sum m_h sum_h q8) (vecdotq.cuh:367-392)
//   IQ2_XXS        (float)(sumi * ls / 8) * (d * d8), C division     vecdotq.cuh:1074-1077
//   IQ2_XS, IQ2_S  (float)((sumi_a * s_a + sumi_b * s_b + (sumi_a + sumi_b) / 2) / 4) * (d * d8)
//                  with the raw 4-bit scales s                       vecdotq.cuh:1116-1118,1163-1166
//   IQ3_XXS        (float)((s * sumi + sumi / 2) / 2) * (d * d8)    vecdotq.cuh:1201-1204
//   IQ1_M          (float)(ls_a * sumi_a + ls_b * sumi_b) * ((d * d8) / 8), w = 8 grid +- 1: the
//                  reference's d * ((sumi + delta * sum q8) * ls ...) holds the same multiple
//                  of 1/8 exactly                                    vecdotq.cuh:1286-1328
// The truncating divisions make these the reference's slice values, not just equal in exact
// arithmetic; the fp32 order in which slices are added differs.
template <int TYPE>
__device__ __forceinline__ float mmvq_term(const int (&w)[8], const int (&x)[8], const SliceScale& sc, float d8,
                                           int sq, int sq2) {
  if constexpr (per16_type(TYPE)) {
    int sa = 0, sb = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) sa = dot4(w[e], x[e], sa);
#pragma unroll
    for (int e = 4; e < 8; ++e) sb = dot4(w[e], x[e], sb);
    // every integer product here has operands within 24 bits (slice dots below 2^20 in magnitude,
    // scales and half-slice sums of q8 below 2^12): __mul24 is exact and full rate (a 32-bit
    // v_mul_lo_u32 is quarter rate)
    if constexpr (TYPE == kQ6_K) return (float)(__mul24(sa, sc.ls) + __mul24(sb, sc.ls2)) * (sc.d * d8);
    if constexpr (TYPE == kQ2_K)
      return d8 * (sc.d * (float)(__mul24(sa, sc.ls) + __mul24(sb, sc.ls2)) -
                   sc.dmin * (float)(__mul24(sq, sc.m) + __mul24(sq2, sc.m2)));
    if constexpr (TYPE == kIQ1_M) return (float)(__mul24(sa, sc.ls) + __mul24(sb, sc.ls2)) * ((sc.d * d8) * 0.125f);
    const int s0 = (sc.ls - 1) >> 1, s1 = (sc.ls2 - 1) >> 1;  // IQ2_XS, IQ2_S
    return (float)((__mul24(sa, s0) + __mul24(sb, s1) + (sa + sb) / 2) / 4) * (sc.d * d8);
  } else {
    int sumi = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) sumi = dot4(w[e], x[e], sumi);
    if constexpr (TYPE == kQ4_K)
      return ((sc.d * (float)sc.ls) * (float)sumi - (sc.dmin * (float)sc.ls2) * (float)sq) * d8;
    if constexpr (TYPE == kIQ2_XXS) return (float)(__mul24(sumi, sc.ls) / 8) * (sc.d * d8);
    if constexpr (TYPE == kIQ3_XXS) {
      const int s4 = (sc.ls - 1) >> 1;
      return (float)((__mul24(s4, sumi) + sumi / 2) / 2) * (sc.d * d8);
    }
    return (float)__mul24(sumi, sc.ls) * (sc.d * d8);  // IQ3_S, IQ4_XS
  }
}

// Workgroups of the generic GEMV: one per group of 4*RW rows, at most kGemvRawGrid of them, each
// looping over groups (the types with a codebook stage it in LDS once per workgroup).
constexpr int kGemvRawGrid = 2048;

template <int TYPE, int NC, int RW>
__global__ void __launch_bounds__(256) gemv_raw_kernel(const uint8_t* __restrict__ W, int64_t row_bytes, int nrows,
                                                       int k, const uint8_t* __restrict__ q8, void* __restrict__ y,
                                                       int y_dtype) {
  using G = typename Codebook<TYPE>::T;
  __shared__ G grid[Codebook<TYPE>::n];
  if constexpr (Codebook<TYPE>::n > 1) {
    stage_codebook<TYPE>(grid);
    __syncthreads();
  }
  constexpr bool SUMS = TYPE == kQ4_K || TYPE == kQ2_K;  // the min term reads sums of q8
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ngroups = (nrows + kGemvWaves * RW - 1) / (kGemvWaves * RW);
  constexpr int BS = block_bytes(TYPE);
  const int nslices = k / kQ81;

  for (int grp = blockIdx.x; grp < ngroups; grp += gridDim.x) {
    const int row0 = (grp * kGemvWaves + wave) * RW;
    if (row0 >= nrows) continue;
    float acc[RW][NC];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;

    for (int s = lane; s < nslices; s += 64) {
      int xq[NC][8];
      float d8[NC];
      int sq[NC], sq2[NC];  // sums of the slice's q8 values: Q4_K all 32; Q2_K each 16-value half
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint8_t* xb = q8 + ((int64_t)c * nslices + s) * 36;
        d8[c] = half_bits_to_float(*(const uint16_t*)xb);
        const u32x4 a = ld128a4(xb + 4);
        const u32x4 b = ld128a4(xb + 20);
        xq[c][0] = (int)a.x; xq[c][1] = (int)a.y; xq[c][2] = (int)a.z; xq[c][3] = (int)a.w;
        xq[c][4] = (int)b.x; xq[c][5] = (int)b.y; xq[c][6] = (int)b.z; xq[c][7] = (int)b.w;
        sq[c] = sq2[c] = 0;
        if constexpr (SUMS) {
          int t0 = 0, t1 = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) t0 = dot4(0x01010101, xq[c][e], t0);
#pragma unroll
          for (int e = 4; e < 8; ++e) t1 = dot4(0x01010101, xq[c][e], t1);
          if constexpr (TYPE == kQ4_K) {
            sq[c] = t0 + t1;
          } else {
            sq[c] = t0;
            sq2[c] = t1;
          }
        }
      }
      const int blk = s >> 3, u = s & 7;
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int row = row0 + r;
        if (row >= nrows) break;
        const uint8_t* b = W + (int64_t)row * row_bytes + (int64_t)blk * BS;
        int w[8];
        SliceScale sc;
        decode_slice<TYPE>(b, u, grid, w, sc);
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] += mmvq_term<TYPE>(w, xq[c], sc, d8[c], sq[c], sq2[c]);
      }
    }

#pragma unroll
    for (int r = 0; r < RW; ++r) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float v = acc[r][c];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[r][c] = v;
      }
    }
    // lane (r * NC + c) writes output (c, row0 + r)
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (lane == r * NC + c && row0 + r < nrows) store_y(y, (int64_t)c * nrows + row0 + r, acc[r][c], y_dtype);
  }
}

// The generic types' decode GEMV with X in LDS: a persistent workgroup of 8 waves loops over
// 8-row tiles; the waves split each tile's K blocks; lane 8r + c decodes slice c of row r of each
// block of its share (decode.h, the codebook in LDS), so a row's 8 lanes read the block's bytes
// contiguously and each load instruction covers 8 rows. X's q8_1 (values, d8 and, for Q2_K, the
// int16 sums of each 16-value half) is copied into LDS once per workgroup and read by every tile;
// lanes of the same slice read the same LDS words (broadcast). The slice term is mmvq_term (the
// decode ops' arithmetic); partial sums over a row's 8 lanes by xor shuffles, then over the waves
// in wave order. X quantised inside the kernel (as the packed
// IQ3_S GEMV does) was measured slower at every row count: 24.1 against 18.5 us for IQ3_XXS
// 17408 x 5120 at one row, quantise launch included.
constexpr int kSlicesWaves = 8;
constexpr int kSlicesXBudget = 48 * 1024;  // LDS bytes for X (40 per slice and activation row)

template <int TYPE, int NC, int RPL>
__global__ void __launch_bounds__(64 * kSlicesWaves) gemv_slices_kernel(const uint8_t* __restrict__ W,
                                                                        int64_t row_bytes, int nrows, int k,
                                                                        const uint8_t* __restrict__ q8,
                                                                        void* __restrict__ y, int y_dtype) {
  constexpr int TR = 8 * RPL;  // rows per tile: lane 8r + c takes rows r, r + 8, ...
  __shared__ typename Codebook<TYPE>::T grid[Codebook<TYPE>::n];
  __shared__ float red[2][kSlicesWaves][NC][TR];
  extern __shared__ uint4 xdyn[];
  constexpr int BS = block_bytes(TYPE);
  const int nslices = k / kQ81, nb = k / kQK;
  uint32_t* xq = (uint32_t*)xdyn;                // [NC][nslices][8] q8 words
  float* xd = (float*)(xq + NC * nslices * 8);   // [NC][nslices] d8
  int* xs = (int*)(xd + NC * nslices);           // [NC][nslices] Q2_K: sums of the halves
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 3, c = lane & 7;
  const int ntiles = (nrows + TR - 1) / TR;
  const int G = gridDim.x;
  const int b0 = wave * nb / kSlicesWaves, per = (wave + 1) * nb / kSlicesWaves - b0;  // per >= 1
  const int my_tiles = (int)blockIdx.x < ntiles ? (ntiles - 1 - (int)blockIdx.x) / G + 1 : 0;
  const int items = my_tiles * per;  // (tile, block) pairs of this wave, tile-major
  // item it -> the block bytes of row r + 8i of its tile (rows past the end re-read the last row;
  // items past the end re-read the last item: the loads need no branch)
  auto block_ptr = [&](int it, int i) {
    it = min(it, items - 1);
    const int tile = (int)blockIdx.x + (it / per) * G;
    const int row = min(tile * TR + 8 * i + r, nrows - 1);
    return W + (int64_t)row * row_bytes + (int64_t)(b0 + it % per) * BS;
  };
  auto load = [&](int it, RawSlice<TYPE> (&raw)[RPL]) {
#pragma unroll
    for (int i = 0; i < RPL; ++i) raw_load<TYPE>(block_ptr(it, i), c, raw[i]);
  };
  float acc[RPL][NC];
#pragma unroll
  for (int i = 0; i < RPL; ++i)
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) acc[i][cc] = 0.0f;
  int par = 0;
  auto compute = [&](const RawSlice<TYPE> (&raw)[RPL], int it) {
    int w[RPL][8];
    SliceScale sc[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) raw_decode<TYPE>(raw[i], c, grid, w[i], sc[i]);
    const int s = (b0 + it % per) * 8 + c;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int xi = cc * nslices + s;
      const uint4 x0 = *(const uint4*)(xq + 8 * xi), x1 = *(const uint4*)(xq + 8 * xi + 4);
      const int xv[8] = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
      int sq = 0, sq2 = 0;
      if constexpr (TYPE == kQ2_K) {
        const int h = xs[xi];
        sq = (int)(int16_t)(h & 0xFFFF);
        sq2 = h >> 16;
      }
      const float d8 = xd[xi];
#pragma unroll
      for (int i = 0; i < RPL; ++i) acc[i][cc] += mmvq_term<TYPE>(w[i], xv, sc[i], d8, sq, sq2);
    }
    if (it % per == per - 1) {  // the wave's last block of the tile: reduce and store
      const int tile = (int)blockIdx.x + (it / per) * G;
#pragma unroll
      for (int i = 0; i < RPL; ++i)
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          float v = acc[i][cc];
          v += __shfl_xor(v, 1, 64);
          v += __shfl_xor(v, 2, 64);
          v += __shfl_xor(v, 4, 64);
          if (c == 0) red[par][wave][cc][8 * i + r] = v;
          acc[i][cc] = 0.0f;
        }
      __syncthreads();
      if (wave == 0) {
        for (int o = lane; o < TR * NC; o += 64) {
          const int rr = o % TR, cc = o / TR;
          float v = red[par][0][cc][rr];
#pragma unroll
          for (int ww = 1; ww < kSlicesWaves; ++ww) v += red[par][ww][cc][rr];
          const int orow = tile * TR + rr;
          if (orow < nrows) store_y(y, (int64_t)cc * nrows + orow, v, y_dtype);
        }
      }
      par ^= 1;
    }
  };
  // two blocks in flight: the next item's bytes load while the current one is computed; the
  // first item's are requested before X is copied
  RawSlice<TYPE> ra[RPL], rb[RPL];
  if (items > 0) load(0, ra);
  __builtin_amdgcn_sched_barrier(0);
  stage_codebook<TYPE>(grid);
  for (int i = threadIdx.x; i < NC * nslices; i += blockDim.x) {
    const uint8_t* src = q8 + (int64_t)i * 36;
    const u32x4 a = ld128a4(src + 4), b = ld128a4(src + 20);
    *(uint4*)(xq + 8 * i) = make_uint4(a.x, a.y, a.z, a.w);
    *(uint4*)(xq + 8 * i + 4) = make_uint4(b.x, b.y, b.z, b.w);
    xd[i] = half_bits_to_float(*(const uint16_t*)src);
  }
  if constexpr (TYPE == kQ2_K) {
    __syncthreads();
    for (int i = threadIdx.x; i < NC * nslices; i += blockDim.x) {
      const uint4 a = *(const uint4*)(xq + 8 * i), b = *(const uint4*)(xq + 8 * i + 4);
      const int s0 = dot4(0x01010101, (int)a.w, dot4(0x01010101, (int)a.z, dot4(0x01010101, (int)a.y,
                                                                                 dot4(0x01010101, (int)a.x, 0))));
      const int s1 = dot4(0x01010101, (int)b.w, dot4(0x01010101, (int)b.z, dot4(0x01010101, (int)b.y,
                                                                                 dot4(0x01010101, (int)b.x, 0))));
      xs[i] = (s0 & 0xFFFF) | (s1 << 16);
    }
  }
  __syncthreads();
  for (int it = 0; it < items; it += 2) {
    load(it + 1, rb);
    __builtin_amdgcn_sched_barrier(0);
    compute(ra, it);
    if (it + 1 >= items) break;
    load(it + 2, ra);
    __builtin_amdgcn_sched_barrier(0);
    compute(rb, it + 1);
  }
}

// The generic types at 1-4 activation rows on weights of at least one 4-row unit per CU: the
// stream GEMV's split (gemv_iq3.hip). One workgroup per CU owns an equal run of 4-row units; its
// items are (unit, pair of K blocks), unit-major, and each of its 8 waves a contiguous run of
// them, so every CU reads the same number of bytes and no barrier falls inside the loop. Lane
// l = 16r + 8kb + s decodes slice s of block kb of the pair in row r (raw_load / raw_decode, the
// codebook in LDS): a row's 16 lanes read its two blocks' bytes contiguously and one load
// instruction covers 4 rows. Three items are in flight while a fourth is computed. The codebook's
// and X's loads are issued before the first weight load (a CU's loads return in order); X's
// q8_1 goes to LDS as in gemv_slices_kernel. The slice term is mmvq_term; a lane adds its terms
// over the wave's items of a unit, and on leaving the unit the 16 lanes of each row are summed
// by DPP (xor 1, xor 2, half-row mirror, row mirror) into a (unit, wave) slot; the output adds
// the slots in wave order.
constexpr int kGsWaves = 8;
constexpr int kGsXpt[] = {1, 2, 3, 5};  // X slices staged per thread (NC * K / 32 <= XPT * 512)

template <int CTRL>
__device__ __forceinline__ float gs_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// X: XDT < 0 the caller's block_q8_1 (xsrc), XPT q8_1 blocks staged per thread; XDT >= 0 X itself
// (dtype XDT, row stride s01) quantised while staged, XPT groups of 8 values per thread, with the
// q8_1 quantiser's arithmetic (xgroup_quantize: bit-identical bytes, and for Q2_K the sums of
// each half formed from those bytes).
template <int TYPE, int NC, int XPT, int XDT>
__global__ void __launch_bounds__(64 * kGsWaves) gemv_generic_stream_kernel(const uint8_t* __restrict__ W,
                                                                            int64_t row_bytes, int nrows, int k,
                                                                            const void* __restrict__ xsrc,
                                                                            int64_t s01, void* __restrict__ y,
                                                                            int y_dtype) {
  constexpr int NW = kGsWaves, NT = 64 * NW, BS = block_bytes(TYPE);
  using CB = Codebook<TYPE>;
  constexpr int CPT = (CB::n + NT - 1) / NT;  // codebook entries staged per thread
  __shared__ typename CB::T grid[CB::n];
  __shared__ uint4 sink;  // staging writes past the end
  extern __shared__ uint4 xdyn[];
  const int nslices = k / kQ81, nb = k / kQK, npair = nb >> 1;
  uint32_t* xq = (uint32_t*)xdyn;               // [NC][nslices][8] q8 words
  float* xd = (float*)(xq + NC * nslices * 8);  // [NC][nslices] d8
  int* xs = (int*)(xd + NC * nslices);          // [NC][nslices] Q2_K: sums of the two halves
  float* part = (float*)(xs + NC * nslices);    // [unit][wave][row][NC]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4, kb = (lane >> 3) & 1, s = lane & 7;
  // staging loads first: the codebook entries and X's q8_1 blocks (indices clamped into range)
  typename CB::T cbv[CPT];
#pragma unroll
  for (int t = 0; t < CPT; ++t) cbv[t] = CB::at(min((int)threadIdx.x + t * NT, CB::n - 1));
  const int nx = NC * nslices;
  constexpr int QX = XDT < 0 ? XPT : 1, RX = XDT < 0 ? 1 : XPT;
  u32x4 xa[QX], xb[QX];
  uint32_t xdb[QX];
  XGroup<XDT < 0 ? kBF16 : XDT> xr[RX];
  if constexpr (XDT < 0) {
    const uint8_t* q8 = (const uint8_t*)xsrc;
#pragma unroll
    for (int t = 0; t < XPT; ++t) {
      const uint8_t* src = q8 + (int64_t)min((int)threadIdx.x + t * NT, nx - 1) * 36;
      xdb[t] = *(const uint16_t*)src;
      xa[t] = ld128a4(src + 4);
      xb[t] = ld128a4(src + 20);
    }
  } else {
    const __amdgpu_buffer_rsrc_t none = buffer_rsrc(xsrc, 0u);  // unused by the raw-X loads
#pragma unroll
    for (int t = 0; t < XPT; ++t)
      xgroup_load<NC, XDT>(xsrc, none, s01, nslices, min((int)threadIdx.x + t * NT, 4 * nx - 1), xr[t]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the workgroup's units [u0, u1), the wave's items [j0, j1)
  const uint32_t nunits = (uint32_t)nrows / 4, G = gridDim.x;
  const int u0 = (int)(blockIdx.x * nunits / G), u1 = (int)((blockIdx.x + 1) * nunits / G);
  const int nu = u1 - u0, items = nu * npair;
  const int j0 = wave * items / NW, j1 = (wave + 1) * items / NW;
  const int64_t ubytes = 4 * row_bytes;
  const uint8_t* wl = W + ((int64_t)u0 * 4 + r) * row_bytes + kb * BS;  // pair 0 of the lane's row, unit u0
  // the next item to load: unit lu, pair lp (past the run: the workgroup's last item again)
  const int cu0 = j0 / npair;
  int lj = j0, lu = cu0, lp = j0 - cu0 * npair;
  auto load_next = [&](RawSlice<TYPE>& f) {
    const bool in_run = lj < j1;
    const int uu = in_run ? lu : nu - 1, pp = in_run ? lp : npair - 1;
    raw_load<TYPE>(wl + (int64_t)uu * ubytes + (int64_t)pp * (2 * BS), s, f);
    ++lj;
    if (++lp == npair) {
      lp = 0;
      ++lu;
    }
  };
  RawSlice<TYPE> f0, f1, f2, f3;
  load_next(f0);
  load_next(f1);
  load_next(f2);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < CPT; ++t) {
    const int i = (int)threadIdx.x + t * NT;
    if (CB::n % NT == 0 || i < CB::n) grid[i] = cbv[t];
  }
  if constexpr (XDT >= 0) {  // group g: part g & 3 (8 values) of slice row g >> 2; a slice is a quad
#pragma unroll
    for (int t = 0; t < XPT; ++t) {
      const int g = (int)threadIdx.x + t * NT, sr = g >> 2, pt = g & 3;
      const bool live = g < 4 * nx;
      uint32_t lo, hi, dbits;
      xgroup_quantize<XDT>(xr[t], lo, hi, dbits);
      *(live ? (uint2*)(xq + 8 * sr + 2 * pt) : (uint2*)&sink) = make_uint2(lo, hi);
      *(live && pt == 0 ? xd + sr : (float*)&sink) = half_bits_to_float(dbits);
      if constexpr (TYPE == kQ2_K) {  // values 0..15 are parts 0, 1; 16..31 parts 2, 3
        int hs = dot4(0x01010101, (int)hi, dot4(0x01010101, (int)lo, 0));
        hs += __builtin_amdgcn_update_dpp(0, hs, 0xB1, 0xF, 0xF, true);             // quad xor 1
        const int other = __builtin_amdgcn_update_dpp(0, hs, 0x4E, 0xF, 0xF, true);  // quad xor 2
        *(live && pt == 0 ? xs + sr : (int*)&sink) = (hs & 0xFFFF) | (other << 16);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < QX && XDT < 0; ++t) {
    const int i = (int)threadIdx.x + t * NT;
    const bool live = i < nx;
    *(live ? (uint4*)(xq + 8 * i) : &sink) = make_uint4(xa[t][0], xa[t][1], xa[t][2], xa[t][3]);
    *(live ? (uint4*)(xq + 8 * i + 4) : &sink) = make_uint4(xb[t][0], xb[t][1], xb[t][2], xb[t][3]);
    *(live ? xd + i : (float*)&sink) = half_bits_to_float(xdb[t]);
    if constexpr (TYPE == kQ2_K) {
      int s0 = 0, s1 = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s0 = dot4(0x01010101, (int)xa[t][e], s0);
        s1 = dot4(0x01010101, (int)xb[t][e], s1);
      }
      *(live ? xs + i : (int*)&sink) = (s0 & 0xFFFF) | (s1 << 16);
    }
  }
  for (int t = threadIdx.x; t < nu * NW * NC; t += NT) ((float4*)part)[t] = make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  float acc[NC];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) acc[cc] = 0.0f;
  int cu = cu0, cp = j0 - cu0 * npair, j = j0;  // the item being computed
  auto step = [&](const RawSlice<TYPE>& fc, RawSlice<TYPE>& fl) {
    load_next(fl);
    __builtin_amdgcn_sched_barrier(0);
    int w[8];
    SliceScale sc;
    raw_decode<TYPE>(fc, s, grid, w, sc);
    const int sl = (2 * cp + kb) * 8 + s;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int xi = cc * nslices + sl;
      const uint4 x0 = *(const uint4*)(xq + 8 * xi), x1 = *(const uint4*)(xq + 8 * xi + 4);
      const int xv[8] = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
      int sq = 0, sq2 = 0;
      if constexpr (TYPE == kQ2_K) {
        const int hsum = xs[xi];
        sq = (int)(int16_t)(hsum & 0xFFFF);
        sq2 = hsum >> 16;
      }
      acc[cc] += mmvq_term<TYPE>(w, xv, sc, xd[xi], sq, sq2);
    }
    ++j;
    if (++cp == npair || j == j1) {  // leaving the unit: the row sums to the wave's slot
      const int slot = cu * NW + wave;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        float v = acc[cc];
        v += gs_dpp<0xB1>(v);   // quad xor 1
        v += gs_dpp<0x4E>(v);   // quad xor 2
        v += gs_dpp<0x141>(v);  // half-row mirror: the other quad of the 8
        v += gs_dpp<0x140>(v);  // row mirror: the other 8 of the 16
        if ((lane & 15) == 0) part[(slot * 4 + r) * NC + cc] = v;
        acc[cc] = 0.0f;
      }
      if (cp == npair) {
        cp = 0;
        ++cu;
      }
    }
  };
  const int nmine = j1 - j0;
  int i = 0;
  for (; i + 4 <= nmine; i += 4) {
    step(f0, f3);
    step(f1, f0);
    step(f2, f1);
    step(f3, f2);
  }
  if (i < nmine) step(f0, f3);
  if (i + 1 < nmine) step(f1, f0);
  if (i + 2 < nmine) step(f2, f1);
  __syncthreads();
  const int nout = nu * 4 * NC;
  for (int t = threadIdx.x; t < nout; t += NT) {
    const int uu = t / (4 * NC), cc = (t >> 2) % NC, row = t & 3;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += part[((uu * NW + w) * 4 + row) * NC + cc];
    store_y(y, (int64_t)cc * nrows + (int64_t)(u0 + uu) * 4 + row, v, y_dtype);
  }
}

// X of the row-chunk GEMV, staged in LDS: q8 values [NC][slice][8 dwords], then (d8, sum of q)
// [NC][slice]. Group g = part g & 3 (8 q bytes) of slice row g >> 2 of the block_q8_1 array; the
// four lanes of a slice are consecutive, so the slice's sum of q is a quad sum (DPP).
struct XGroupQ8 {
  uint32_t d, q0, q1;
};

__device__ __forceinline__ void xgroup_q8_load(__amdgpu_buffer_rsrc_t xrs, int g, XGroupQ8& r) {
  const int o = (g >> 2) * 36, part = g & 3;
  r.d = __builtin_amdgcn_raw_buffer_load_b32(xrs, o, 0, 0);
  r.q0 = __builtin_amdgcn_raw_buffer_load_b32(xrs, o + 4 + 8 * part, 0, 0);
  r.q1 = __builtin_amdgcn_raw_buffer_load_b32(xrs, o + 8 + 8 * part, 0, 0);
}


// SUMS: what the second word of a slice's (d8, .) pair holds. kSumSlice: the slice's sum of q (as
// float; Q4_K's min term). kSumHalves: the sums of q over values 0..15 and 16..31 as two int16 in
// the word's bits (Q6_K folds its -32 offset into them). A group past the end (live false) is
// written to `sink`, not skipped: a load whose only use is a conditional store is moved under the
// condition by the compiler, and a load under a branch is waited for (vmcnt(0)) where the paths
// join.
constexpr int kSumNone = 0, kSumSlice = 1, kSumHalves = 2;

template <int SUMS>
__device__ __forceinline__ void xgroup_q8_store(const XGroupQ8& r, int g, bool live, uint32_t* xq, float2* xs,
                                                uint4* sink) {
  const int sr = g >> 2, part = g & 3;
  float sum = 0.0f;
  if constexpr (SUMS != kSumNone) {
    int t = dot4(0x01010101, (int)r.q1, dot4(0x01010101, (int)r.q0, 0));
    t += __builtin_amdgcn_update_dpp(0, t, 0xB1, 0xF, 0xF, true);  // quad xor 1: this half's sum
    const int o = __builtin_amdgcn_update_dpp(0, t, 0x4E, 0xF, 0xF, true);  // quad xor 2: the other half's
    if constexpr (SUMS == kSumSlice) sum = (float)(t + o);
    else sum = __uint_as_float(((uint32_t)t & 0xFFFFu) | ((uint32_t)o << 16));
  }
  *(live ? (uint2*)(xq + sr * 8 + 2 * part) : (uint2*)sink) = make_uint2(r.q0, r.q1);
  *(live && part == 0 ? xs + sr : (float2*)sink) = make_float2(half_bits_to_float(r.d & 0xFFFF), sum);
}

// Q4_K, IQ4_XS and Q6_K on GGUF rows with loads that run along each row: lane L = 8 r + c (r = row
// in an 8-row group, c = 16-byte chunk of the row's 128 quant bytes) loads quant bytes
// [16c, 16c + 16) of the block of rows r and 8 + r of the tile, and what its values need of the
// block header. One load instruction then covers 8 rows' bytes contiguously (128 B per row); a
// lane per slice pair of a 16-row tile touches two to three times as many cache lines per block,
// and the L1 tag rate is what bounds such a layout. The chunk's values (ggml-common.h block
// layouts; the reference's MMVQ dots, vecdotq.cuh: Q4_K 508-530, IQ4_XS 1357-1380, Q6_K 627-648):
//   IQ4_XS  slice c (low nibbles values 0..15, high nibbles 16..31).
//   Q4_K    half h = c & 1 (values 16h..16h+15) of slice 2j (low nibbles) and of slice 2j + 1
//           (high nibbles), j = c >> 1.
//   Q6_K    half h = c & 1 of slice 4n + t (low nibbles) and of slice 4n + t + 2 (high nibbles),
//           c = 4n + 2t + h, with the high bits from the 16 qh bytes of the same positions; the
//           -32 offset is applied as 32 times X's half-slice sum.
// For Q4_K and Q6_K, lanes c and c ^ 1 hold the two halves of the same two slices; they exchange
// the integer sums by DPP and each finishes one slice. Every slice's term is the reference's
// arithmetic; partial sums over a row's 8 lanes by DPP, then over the waves in wave order.
template <int TYPE>
struct RowsFrag;
template <>
struct RowsFrag<kQ4_K> {
  u32x4 hdr[2], qs[2];  // rows r, 8 + r: d | dmin << 16, scales[0..12); the chunk
};
template <>
struct RowsFrag<kIQ4_XS> {
  uint2 hdr[2];  // d | scales_h << 16, scales_l
  u32x4 qs[2];
};
// Q6_K blocks are 210 bytes: every odd block starts 2 bytes past a dword boundary, and 16-byte
// loads there are split by the memory pipeline. The lane loads the dword-aligned 16 bytes at or
// 2 below each 16-byte field (mis = 2 on odd blocks, wave-uniform) and the dword after them, and
// takes the field with a byte align; the two scale bytes and d come from byte and 16-bit loads.
template <>
struct RowsFrag<kQ6_K> {
  u32x4 ql[2], qh[2];      // from ql[16c - mis], qh[32n + 16h - mis]
  uint32_t qlx[2], qhx[2];  // the dword after each
  uint8_t s0[2], s1[2];     // scales[8n + 2t + h], scales[8n + 4 + 2t + h]
  uint16_t d[2];            // fp16 d of rows r, 8 + r
  uint32_t mis;
};

// PH (kp_arg > 1): X's q8_1 does not fit the LDS budget, so K runs in kp phases of whole blocks;
// in each phase the 8 waves split its blocks, and the workgroup stages that phase's part of X
// (between two barriers) when its waves reach it. Every wave has at least one block in every
// phase. Without PH (one phase) the staging branch is compiled out: inside the K loop, a branch
// with loads makes the compiler wait for every load in flight at its join.
// XDT < 0: X given as block_q8_1 (xsrc). XDT >= 0 (one phase only): X itself (dtype XDT, row
// stride s01), quantised in the kernel with the q8_1 quantiser's arithmetic (bit-identical
// bytes, sums of q formed as from the q8_1 bytes): each wave stages the X its own K range reads,
// at most XPL groups of 8 values per lane, loaded before its first weight block.
template <int TYPE, int NC, int WPT, bool PH, int RPL, int XDT = -1, int XPL = 0>
__global__ void __launch_bounds__(64 * WPT) gemv_rows_kernel(const uint8_t* __restrict__ W, int64_t row_bytes,
                                                             int nrows, int k, const void* __restrict__ xsrc,
                                                             int64_t s01, void* __restrict__ y, int y_dtype, int kp_arg) {
  static_assert(XDT < 0 || (!PH && XPL > 0), "raw X: one phase, per-wave staging");
  const uint8_t* q8 = (const uint8_t*)xsrc;
  const int kp = PH ? kp_arg : 1;
  constexpr int TR = 8 * RPL;  // rows per tile: lane 8r + c takes rows r (and 8 + r)
  constexpr int BS = block_bytes(TYPE);
  constexpr int NT = 64 * WPT;
  constexpr int SUMS = TYPE == kQ4_K ? kSumSlice : (TYPE == kQ6_K ? kSumHalves : kSumNone);
  __shared__ float red[2][WPT][NC][TR];
  __shared__ uint4 sink;           // staging writes of groups past the end of X
  extern __shared__ uint4 xdyn[];  // q values [NC][slice][8 dwords], then (d8, sums) [NC][slice]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 3, c = lane & 7, h = c & 1;
  const int ntiles = (nrows + TR - 1) / TR;
  const int nb = k / kQK, nslices = k / kQ81;
  const int nsl = (nb + kp - 1) / kp * 8;  // LDS slices per activation row (the longest phase)
  const int G = gridDim.x;
  uint32_t* xq = (uint32_t*)xdyn;
  float2* xs = (float2*)(xq + NC * nsl * 8);
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(W, (uint32_t)((int64_t)nrows * row_bytes));
  const __amdgpu_buffer_rsrc_t nrs = buffer_rsrc(W, 0);
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(q8, XDT < 0 ? (uint32_t)(NC * nslices * 36) : 0u);
  auto load = [&](int t, int b, RowsFrag<TYPE>& f) {
    const __amdgpu_buffer_rsrc_t rs = t < ntiles ? wrs : nrs;
    const int t0 = (t < ntiles ? t : 0) * TR;
    const int bo = b * BS;
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const int o = min(t0 + 8 * i + r, nrows - 1) * (int)row_bytes;
      if constexpr (TYPE == kQ4_K) {
        f.hdr[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o, bo, 0);
        f.qs[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 16 + 16 * c, bo, 0);
      } else if constexpr (TYPE == kIQ4_XS) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, o, bo, 0);
        f.hdr[i] = make_uint2(v[0], v[1]);
        f.qs[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 8 + 16 * c, bo, 0);
      } else {  // row_bytes % 4 == 0 (an even number of blocks): mis = 2 on odd blocks
        const int n = c >> 2, sb = (c >> 1 & 1) * 2 + h, mis = bo & 3;
        f.ql[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 16 * c, bo - mis, 0);
        f.qlx[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, o + 16 * c + 16, bo - mis, 0);
        f.qh[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 128 + 16 * (2 * n + h), bo - mis, 0);
        f.qhx[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, o + 144 + 16 * (2 * n + h), bo - mis, 0);
        f.s0[i] = __builtin_amdgcn_raw_buffer_load_b8(rs, o + 192 + 8 * n + sb, bo, 0);
        f.s1[i] = __builtin_amdgcn_raw_buffer_load_b8(rs, o + 196 + 8 * n + sb, bo, 0);
        f.d[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, o + 208, bo, 0);
        f.mis = (uint32_t)mis;
      }
    }
  };
  // phase p: blocks [ph0(p), ph0(p + 1)); this wave's part of it: [wb(p), we(p))
  auto ph0 = [&](int pp) { return pp * nb / kp; };
  auto wb = [&](int pp) { return ph0(pp) + wave * (ph0(pp + 1) - ph0(pp)) / WPT; };
  auto we = [&](int pp) { return ph0(pp) + (wave + 1) * (ph0(pp + 1) - ph0(pp)) / WPT; };
  int per_tile = 0;
  for (int pp = 0; pp < kp; ++pp) per_tile += we(pp) - wb(pp);
  const int items = ((int)blockIdx.x < ntiles ? (ntiles - 1 - (int)blockIdx.x) / G + 1 : 0) * per_tile;
  auto next = [&](int& tt, int& pp, int& bb) {
    if (++bb == we(pp)) {
      if (++pp == kp) {
        pp = 0;
        tt += G;
      }
      bb = wb(pp);
    }
  };
  // X staging of phase pp: local group gl (8 values; 4 per slice) of activation row cc -> global
  // group of the block_q8_1 array, and the group index of the LDS layout (row stride nsl)
  auto groups = [&](int pp) { return NC * (ph0(pp + 1) - ph0(pp)) * 32; };
  auto gmap = [&](int pp, int gl, int& gg, int& gL) {
    const int per_row = (ph0(pp + 1) - ph0(pp)) * 32;
    int cc = 0, rem = gl;
#pragma unroll
    for (int i = 1; i < NC; ++i)
      if (rem >= per_row) rem -= per_row, ++cc;
    gg = (cc * nslices + ph0(pp) * 8) * 4 + rem;
    gL = cc * nsl * 4 + rem;
  };
  auto stage = [&](int pp) {  // the in-loop staging of a later phase (between barriers)
    const int ng = groups(pp);
    for (int gl = threadIdx.x; gl < ng; gl += NT) {
      int gg, gL;
      gmap(pp, gl, gg, gL);
      XGroupQ8 xc;
      xgroup_q8_load(xrs, gg, xc);
      xgroup_q8_store<SUMS>(xc, gL, true, xq, xs, &sink);
    }
  };
  // phase 0: X's first two groups per thread (raw X: the wave's own groups), then the first two
  // weight blocks, then X to LDS
  const int ng0 = groups(0);
  const int ga = threadIdx.x, gb = threadIdx.x + NT;
  int gga, gLa, ggb, gLb;
  gmap(0, ga < ng0 ? ga : ng0 - 1, gga, gLa);
  gmap(0, gb < ng0 ? gb : ng0 - 1, ggb, gLb);
  XGroupQ8 xa, xb;
  constexpr int XN = XDT >= 0 ? XPL : 1;
  XGroup<XDT> xr[XN];
  int xgl[XN];
  bool xlive[XN];
  if constexpr (XDT >= 0) {  // activation rows cc, slices [8 wb(0), 8 we(0)): NC * 32 * nblk groups
    const int nblk = we(0) - wb(0), wcnt = NC * 32 * nblk;
#pragma unroll
    for (int j = 0; j < XN; ++j) {
      const int li0 = lane + 64 * j;
      xlive[j] = li0 < wcnt;
      const int li = xlive[j] ? li0 : wcnt - 1;
      const int cc = li / (32 * nblk), rem = li - cc * 32 * nblk;
      const int sg = 32 * wb(0) + rem;  // group within the activation row
      xgl[j] = cc * nsl * 4 + sg;
      xgroup_load<NC, XDT>(xsrc, xrs, s01, nslices, cc * nslices * 4 + sg, xr[j]);
    }
  } else {
    xgroup_q8_load(xrs, gga, xa);
    xgroup_q8_load(xrs, ggb, xb);
  }
  __builtin_amdgcn_sched_barrier(0);
  RowsFrag<TYPE> f0, f1, f2;
  int lt = blockIdx.x, lp = 0, lb = wb(0);  // next item to load
  load(lt, lb, f0);
  next(lt, lp, lb);
  load(lt, lb, f1);
  next(lt, lp, lb);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (XDT >= 0) {
#pragma unroll
    for (int j = 0; j < XN; ++j) {
      XGroupQ8 xc;
      xgroup_quantize<XDT>(xr[j], xc.q0, xc.q1, xc.d);
      xgroup_q8_store<SUMS>(xc, xgl[j], xlive[j], xq, xs, &sink);
    }
  } else {
    xgroup_q8_store<SUMS>(xa, gLa, ga < ng0, xq, xs, &sink);
    xgroup_q8_store<SUMS>(xb, gLb, gb < ng0, xq, xs, &sink);
    for (int gl = threadIdx.x + 2 * NT; gl < ng0; gl += NT) {  // phase 0 beyond 2 groups per thread
      int gg, gL;
      gmap(0, gl, gg, gL);
      XGroupQ8 xc;
      xgroup_q8_load(xrs, gg, xc);
      xgroup_q8_store<SUMS>(xc, gL, true, xq, xs, &sink);
    }
  }
  __syncthreads();
  float acc[2][NC];
#pragma unroll
  for (int i = 0; i < RPL; ++i)
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) acc[i][cc] = 0.0f;
  // the lane's two (Q4_K, Q6_K) or one (IQ4_XS) slices of block b, for activation row cc
  auto slices = [&](int cc, int b, int& s1, int& s2) {  // b: block index within the staged phase
    const int base = cc * nsl + b * 8;
    if constexpr (TYPE == kQ4_K) {
      s1 = base + 2 * (c >> 1);
      s2 = s1 + 1;
    } else if constexpr (TYPE == kQ6_K) {
      s1 = base + 4 * (c >> 2) + ((c >> 1) & 1);
      s2 = s1 + 2;
    } else {
      s1 = s2 = base + c;
    }
  };
  // lanes h = 0 / 1 hold halves 0 / 1 of slices s1, s2: each sends its partner the integer sum of
  // the slice the partner finishes (h = 0 finishes s1, h = 1 s2); half 0's sum comes first
  auto join = [&](int p1, int p2) {
    const int mine = h == 0 ? p1 : p2, send = h == 0 ? p2 : p1;
    const int got = __builtin_amdgcn_mov_dpp(send, 0xB1, 0xF, 0xF, false);  // quad xor 1
    return h == 0 ? mine + got : got + mine;
  };
  auto compute = [&](const RowsFrag<TYPE>& f, int b) {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      int s1, s2;
      slices(cc, b, s1, s2);
      if constexpr (TYPE == kIQ4_XS) {
        const uint4 x0 = *(const uint4*)(xq + s1 * 8), x1 = *(const uint4*)(xq + s1 * 8 + 4);
        const int xv[8] = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        const float d8 = xs[s1].x;
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
          int sumi = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) sumi = dot4(iq4nl(f.qs[i][e], 0), xv[e], sumi);
#pragma unroll
          for (int e = 0; e < 4; ++e) sumi = dot4(iq4nl(f.qs[i][e], 4), xv[4 + e], sumi);
          const int ls = (int)(((f.hdr[i].y >> (4 * c)) & 0xF) | (((f.hdr[i].x >> (16 + 2 * c)) & 3u) << 4)) - 32;
          acc[i][cc] = fmaf(half_bits_to_float(f.hdr[i].x & 0xFFFF) * (float)__mul24(sumi, ls), d8, acc[i][cc]);
        }
      } else {
        const uint4 x1 = *(const uint4*)(xq + s1 * 8 + 4 * h), x2 = *(const uint4*)(xq + s2 * 8 + 4 * h);
        const int xv1[4] = {(int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        const int xv2[4] = {(int)x2.x, (int)x2.y, (int)x2.z, (int)x2.w};
        const int sf = h == 0 ? s1 : s2;  // the slice this lane finishes
        const float d8 = xs[sf].x;
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
          int a1 = 0, a2 = 0;
          if constexpr (TYPE == kQ4_K) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              a1 = dot4((int)(f.qs[i][e] & 0x0F0F0F0Fu), xv1[e], a1);
              a2 = dot4((int)((f.qs[i][e] >> 4) & 0x0F0F0F0Fu), xv2[e], a2);
            }
            const int sumi = join(a1, a2);
            const int u = sf & 7;  // slice within the block
            const int jj = u & 3;
            const uint32_t sa = (f.hdr[i][1] >> (8 * jj)) & 0xFF, sb = (f.hdr[i][2] >> (8 * jj)) & 0xFF;
            const uint32_t se = (f.hdr[i][3] >> (8 * jj)) & 0xFF;
            const uint32_t sc = u < 4 ? (sa & 63) : ((se & 0xF) | ((sa >> 6) << 4));
            const uint32_t m = u < 4 ? (sb & 63) : ((se >> 4) | ((sb >> 6) << 4));
            const float d = half_bits_to_float(f.hdr[i][0] & 0xFFFF), dmin = half_bits_to_float(f.hdr[i][0] >> 16);
            const float term = (d * (float)sc) * (float)sumi - (dmin * (float)m) * xs[sf].y;
            acc[i][cc] = fmaf(term, d8, acc[i][cc]);
          } else {
            const uint32_t t2 = 2 * ((c >> 1) & 1);  // qh bit pair of the low-nibble half slice
            const uint32_t hs1 = __float_as_uint(xs[s1].y), hs2 = __float_as_uint(xs[s2].y);
            const int sx1 = (int)(int16_t)((hs1 >> (16 * h)) & 0xFFFFu), sx2 = (int)(int16_t)((hs2 >> (16 * h)) & 0xFFFFu);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t l = __builtin_amdgcn_alignbyte(e < 3 ? f.ql[i][e + 1] : f.qlx[i], f.ql[i][e], f.mis);
              const uint32_t q = __builtin_amdgcn_alignbyte(e < 3 ? f.qh[i][e + 1] : f.qhx[i], f.qh[i][e], f.mis);
              const int w1 = (int)((l & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(q, q, (t2 + 28) & 31) & 0x30303030u));
              const int w2 = (int)(((l >> 4) & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(q, q, t2 & 31) & 0x30303030u));
              a1 = dot4(w1, xv1[e], a1);
              a2 = dot4(w2, xv2[e], a2);
            }
            const int sc1 = (int)(int8_t)f.s0[i], sc2 = (int)(int8_t)f.s1[i];  // 8n + 2t + h, and 4 above
            const int tot = join(__mul24(a1 - 32 * sx1, sc1), __mul24(a2 - 32 * sx2, sc2));  // 24-bit operands
            const float dr = half_bits_to_float(f.d[i]);
            acc[i][cc] = fmaf(dr * (float)tot, d8, acc[i][cc]);
          }
        }
      }
    }
  };
  int t = blockIdx.x, p = 0, b = wb(0), it = 0, staged = 0;  // item being computed
  auto step = [&](const RowsFrag<TYPE>& fc, RowsFrag<TYPE>& fl) {
    load(lt, lb, fl);
    next(lt, lp, lb);
    __builtin_amdgcn_sched_barrier(0);
    if (PH && p != staged) {  // the first block of a later phase (or of phase 0 of the next tile)
      __syncthreads();
      stage(p);
      __syncthreads();
      staged = p;
    }
    compute(fc, b - ph0(p));
    if (p == kp - 1 && b == we(kp - 1) - 1) {  // the wave's last block of tile t: reduce and store
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          float v = acc[i][cc];
          v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));   // xor 1
          v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));   // xor 2
          v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));  // 7 - lane
          if (c == 0) red[it & 1][wave][cc][8 * i + r] = v;
          acc[i][cc] = 0.0f;
        }
      }
      __syncthreads();
      if (threadIdx.x < NC * TR) {
        const int cc = threadIdx.x / TR, rr = threadIdx.x % TR;
        const int row = t * TR + rr;
        float v = red[it & 1][0][cc][rr];
#pragma unroll
        for (int w2 = 1; w2 < WPT; ++w2) v += red[it & 1][w2][cc][rr];
        if (row < nrows) store_y(y, (int64_t)cc * nrows + row, v, y_dtype);
      }
      ++it;
    }
    next(t, p, b);
  };
  int i = 0;
  for (; i + 3 <= items; i += 3) {
    step(f0, f2);
    step(f1, f0);
    step(f2, f1);
  }
  if (i < items) step(f0, f2);
  if (i + 1 < items) step(f1, f0);
}

// Q4_K / IQ4_XS / Q6_K at 1-4 rows on weights below 2 GiB: the row-chunk kernel. X's q8_1 takes
// 40 bytes of LDS per slice and row; kp: the fewest K phases that bring a phase within 48 KB
// with at least one block per wave and phase (0 if none does).
static int rows_phases(int64_t k, int64_t n) {
  const int64_t nb = k / kQK;
  for (int64_t kp = 1; nb / kp >= 8; ++kp)
    if (n * ((nb + kp - 1) / kp) * 8 * 40 <= 48 * 1024) return (int)kp;
  return 0;
}

// Q4_K at 4 rows in K phases stays on the int8-MFMA small GEMM (5120 x 17408: 34 against 51 us;
// at 3 rows the phased GEMV is the faster, 32 against 34 us).
bool gemv_rows_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n) {
  const int kp = rows_phases(k, n);
  return (type == kQ4_K || type == kIQ4_XS || type == kQ6_K) && n >= 1 && n <= 4 &&
         nrows * row_bytes < ((int64_t)1 << 31) && kp > 0 && !(type == kQ4_K && n == 4 && kp > 1);
}

template <int TYPE, int RPL>
static void launch_rows_rpl(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n, void* y,
                            int y_dtype, hipStream_t stream) {
  const int kp = rows_phases(k, n);
  const int tiles = (nrows + 8 * RPL - 1) / (8 * RPL);
  const unsigned g = (unsigned)std::min(tiles, persist_grid());
  const size_t lds = (size_t)n * ((k / kQK + kp - 1) / kp) * 8 * 40;
#define GGUF_ROWS(NC)                                                                                                   \
  (kp > 1 ? gemv_rows_kernel<TYPE, NC, 8, true, RPL><<<g, 512, lds, stream>>>(W, row_bytes, nrows, k, q8, 0, y, y_dtype, kp) \
          : gemv_rows_kernel<TYPE, NC, 8, false, RPL><<<g, 512, lds, stream>>>(W, row_bytes, nrows, k, q8, 0, y, y_dtype, 1))
  switch (n) {
    case 1: GGUF_ROWS(1); break;
    case 2: GGUF_ROWS(2); break;
    case 3: GGUF_ROWS(3); break;
    default: GGUF_ROWS(4); break;
  }
#undef GGUF_ROWS
}

template <int TYPE>
static bool launch_rows(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n, void* y,
                        int y_dtype, hipStream_t stream) {
  if (!gemv_rows_supported(TYPE, nrows, row_bytes, k, n)) return false;
  // 8-row tiles (one row per lane): twice the work items, shared out more evenly over the CUs
  // (measured at M = 1: 5120 x 17408 IQ4_XS 19.8 -> 16.3 us, Q6_K 31.1 -> 25.7; 17408 x 5120
  // IQ4_XS 18.3 -> 15.5). Over K phases X is staged once per phase and tile, and there IQ4_XS
  // keeps 16-row tiles (5120 x 17408 M = 4: 33.2 against 36.0 us; Q6_K 41.5 against 43.8).
  if (rows_phases(k, n) == 1 || TYPE == kQ6_K) launch_rows_rpl<TYPE, 1>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream);
  else launch_rows_rpl<TYPE, 2>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream);
  return true;
}

// X quantised inside the row-chunk kernel: one or two activation rows, one K phase, and each
// wave's own part of X within two (one row) or three (two rows) groups of 8 values per lane
// (K <= 8192 with eight waves). Larger K keeps quantise + GEMV: the per-lane quantisation then
// costs as much as the launch it saves (measured on the packed IQ3_S GEMV at K = 17408).
static int rows_x_groups(int64_t k, int64_t n) { return (int)((n * 32 * ((k / kQK + 7) / 8) + 63) / 64); }

bool gemv_rows_x_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n) {
  return n >= 1 && n <= 2 && gemv_rows_supported(type, nrows, row_bytes, k, n) && rows_phases(k, n) == 1 &&
         rows_x_groups(k, n) <= (n == 1 ? 2 : 3);
}

template <int TYPE, int XDT>
static void launch_rows_x_dt(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int64_t s01, int n,
                             void* y, int y_dtype, hipStream_t stream) {
  const unsigned g = (unsigned)std::min((nrows + 7) / 8, persist_grid());
  const size_t lds = (size_t)n * (k / kQK) * 8 * 40;
  if (n == 1)
    gemv_rows_kernel<TYPE, 1, 8, false, 1, XDT, 2><<<g, 512, lds, stream>>>(W, row_bytes, nrows, k, x, s01, y, y_dtype, 1);
  else
    gemv_rows_kernel<TYPE, 2, 8, false, 1, XDT, 3><<<g, 512, lds, stream>>>(W, row_bytes, nrows, k, x, s01, y, y_dtype, 1);
}

template <int TYPE>
static void launch_rows_x_type(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int x_dtype,
                               int64_t s01, int n, void* y, int y_dtype, hipStream_t stream) {
  switch (x_dtype) {
    case kF32: launch_rows_x_dt<TYPE, kF32>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream); break;
    case kF16: launch_rows_x_dt<TYPE, kF16>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream); break;
    default: launch_rows_x_dt<TYPE, kBF16>(W, row_bytes, nrows, k, x, s01, n, y, y_dtype, stream); break;
  }
}

template <int TYPE, int NC>
static void launch_nc(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, void* y, int y_dtype,
                      hipStream_t stream) {
  constexpr int RW = NC <= 4 ? 4 : 2;
  const unsigned blocks = (unsigned)std::min((nrows + kGemvWaves * RW - 1) / (kGemvWaves * RW), kGemvRawGrid);
  gemv_raw_kernel<TYPE, NC, RW><<<blocks, 64 * kGemvWaves, 0, stream>>>(W, row_bytes, nrows, k, q8, y, y_dtype);
}

// The generic types at up to 8 activation rows whose X fits the LDS budget, on weights of at
// least 8 K blocks (one per wave).
static bool slices_supported(int type, int64_t k, int64_t n) {
  return generic_type(type) && n >= 1 && n <= 8 && k / kQK >= kSlicesWaves &&
         n * (k / kQ81) * 40 <= kSlicesXBudget;
}

template <int TYPE>
static void launch_slices(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n, void* y,
                          int y_dtype, hipStream_t stream) {
  constexpr int RPL = 2;  // 16-row tiles: two rows' blocks per lane in flight
  const int tiles = (nrows + 8 * RPL - 1) / (8 * RPL);
  const unsigned g = (unsigned)std::min(tiles, persist_grid());
  const size_t lds = (size_t)n * (k / kQ81) * 40;
#define GGUF_SLICES(NC) \
  gemv_slices_kernel<TYPE, NC, RPL><<<g, 64 * kSlicesWaves, lds, stream>>>(W, row_bytes, nrows, k, q8, y, y_dtype)
  switch (n) {
    case 1: GGUF_SLICES(1); break;
    case 2: GGUF_SLICES(2); break;
    case 3: GGUF_SLICES(3); break;
    case 4: GGUF_SLICES(4); break;
    case 5: GGUF_SLICES(5); break;
    case 6: GGUF_SLICES(6); break;
    case 7: GGUF_SLICES(7); break;
    default: GGUF_SLICES(8); break;
  }
#undef GGUF_SLICES
}

// The generic stream GEMV: X slices staged per thread, its dynamic LDS (X, then the partial-sum
// slots of the most units a workgroup takes) and the most it may take beside the codebook.
static int gs_xpt(int64_t k, int64_t n) {
  const int64_t need = (n * (k / kQ81) + 511) / 512;
  for (int x : kGsXpt)
    if (x >= need) return x;
  return 0;
}

static size_t gs_lds(int64_t nrows, int64_t k, int64_t n, int64_t grid) {
  const int64_t units = (nrows / 4 + grid - 1) / grid;
  return (size_t)(n * (k / kQ81) * 40 + units * kGsWaves * 4 * n * 4);
}

// 256 bytes are left for the alignment padding of the static arrays (the codebook and the 16-byte
// sink); static plus dynamic LDS must stay within the 160 KB a workgroup may take.
template <int TYPE>
constexpr size_t gs_lds_max() {
  return 160 * 1024 - sizeof(typename Codebook<TYPE>::T) * Codebook<TYPE>::n - 256;
}

template <int TYPE>
static bool gs_supported(int64_t nrows, int64_t row_bytes, int64_t k, int64_t n) {
  if (!generic_type(TYPE) || n < 1 || n > 4 || nrows % 4 != 0 || k % 512 != 0) return false;
  if (row_bytes != k / kQK * block_bytes(TYPE) || gs_xpt(k, n) == 0) return false;
  const int64_t cus = device_cus();
  return nrows / 4 >= cus && gs_lds(nrows, k, n, cus) <= gs_lds_max<TYPE>();
}

template <int TYPE, int NC, int XPT, int XDT>
static void launch_gs_x(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int64_t s01, void* y,
                        int y_dtype, hipStream_t stream) {
  const int cus = device_cus();
  const size_t lds = gs_lds(nrows, k, NC, cus);
  int dev = 0;
  if (lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess) {
    struct Tag;
    once_per_device<Tag>(dev, [] {
      (void)hipFuncSetAttribute((const void*)gemv_generic_stream_kernel<TYPE, NC, XPT, XDT>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)gs_lds_max<TYPE>());
    });
  }
  gemv_generic_stream_kernel<TYPE, NC, XPT, XDT><<<cus, 64 * kGsWaves, lds, stream>>>(W, row_bytes, nrows, k, x, s01,
                                                                                      y, y_dtype);
}

template <int TYPE, int NC>
static void launch_gs_nc(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, void* y,
                         int y_dtype, hipStream_t stream) {
  switch (gs_xpt(k, NC)) {
    case 1: launch_gs_x<TYPE, NC, 1, -1>(W, row_bytes, nrows, k, q8, 0, y, y_dtype, stream); break;
    case 2: launch_gs_x<TYPE, NC, 2, -1>(W, row_bytes, nrows, k, q8, 0, y, y_dtype, stream); break;
    case 3: launch_gs_x<TYPE, NC, 3, -1>(W, row_bytes, nrows, k, q8, 0, y, y_dtype, stream); break;
    default: launch_gs_x<TYPE, NC, 5, -1>(W, row_bytes, nrows, k, q8, 0, y, y_dtype, stream); break;
  }
}

// X quantised inside the generic stream GEMV: 1-2 activation rows at K <= 8192 (at most 4 groups
// of 8 values per thread), where the quantisation each workgroup repeats costs less than the
// quantise launch it saves.
static int gs_fused_xpt(int64_t k, int64_t n) { return (int)((n * (k / kQ81) * 4 + 511) / 512); }

template <int TYPE>
static bool gs_x_supported(int64_t nrows, int64_t row_bytes, int64_t k, int64_t n) {
  return n <= 2 && k <= 8192 && gs_supported<TYPE>(nrows, row_bytes, k, n);
}

template <int TYPE, int NC, int XDT>
static void launch_gs_fused_dt(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int64_t s01,
                               void* y, int y_dtype, hipStream_t stream) {
  switch (gs_fused_xpt(k, NC)) {
    case 1: launch_gs_x<TYPE, NC, 1, XDT>(W, row_bytes, nrows, k, x, s01, y, y_dtype, stream); break;
    case 2: launch_gs_x<TYPE, NC, 2, XDT>(W, row_bytes, nrows, k, x, s01, y, y_dtype, stream); break;
    case 3: launch_gs_x<TYPE, NC, 3, XDT>(W, row_bytes, nrows, k, x, s01, y, y_dtype, stream); break;
    default: launch_gs_x<TYPE, NC, 4, XDT>(W, row_bytes, nrows, k, x, s01, y, y_dtype, stream); break;
  }
}

template <int TYPE, int NC>
static void launch_gs_fused_nc(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int x_dtype,
                               int64_t s01, void* y, int y_dtype, hipStream_t stream) {
  switch (x_dtype) {
    case kF32: launch_gs_fused_dt<TYPE, NC, kF32>(W, row_bytes, nrows, k, x, s01, y, y_dtype, stream); break;
    case kF16: launch_gs_fused_dt<TYPE, NC, kF16>(W, row_bytes, nrows, k, x, s01, y, y_dtype, stream); break;
    default: launch_gs_fused_dt<TYPE, NC, kBF16>(W, row_bytes, nrows, k, x, s01, y, y_dtype, stream); break;
  }
}

template <int TYPE>
static void launch_gs_fused(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int x_dtype,
                            int64_t s01, int n, void* y, int y_dtype, hipStream_t stream) {
  if (n == 1) launch_gs_fused_nc<TYPE, 1>(W, row_bytes, nrows, k, x, x_dtype, s01, y, y_dtype, stream);
  else launch_gs_fused_nc<TYPE, 2>(W, row_bytes, nrows, k, x, x_dtype, s01, y, y_dtype, stream);
}

template <int TYPE>
static void launch_type(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n, void* y,
                        int y_dtype, hipStream_t stream) {
  if constexpr (generic_type(TYPE)) {
    if (gs_supported<TYPE>(nrows, row_bytes, k, n)) {
      switch (n) {
        case 1: launch_gs_nc<TYPE, 1>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
        case 2: launch_gs_nc<TYPE, 2>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
        case 3: launch_gs_nc<TYPE, 3>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
        default: launch_gs_nc<TYPE, 4>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
      }
      return;
    }
    if (slices_supported(TYPE, k, n)) {
      launch_slices<TYPE>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream);
      return;
    }
  }
  switch (n) {
    case 1: launch_nc<TYPE, 1>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 2: launch_nc<TYPE, 2>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 3: launch_nc<TYPE, 3>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 4: launch_nc<TYPE, 4>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 5: launch_nc<TYPE, 5>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 6: launch_nc<TYPE, 6>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 7: launch_nc<TYPE, 7>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    default: launch_nc<TYPE, 8>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
  }
}

// Q4_K / IQ4_XS / Q6_K decode with X (dtype x_dtype, row stride s01) quantised in the GEMV, on
// the shapes gemv_rows_x_supported admits; bit-identical to the q8_1 quantiser + launch_gemv_raw.
hipError_t launch_gemv_rows_x(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x,
                              int x_dtype, int64_t s01, int n, void* y, int y_dtype, hipStream_t stream) {
  if (!gemv_rows_x_supported(type, nrows, row_bytes, k, n)) return hipErrorInvalidValue;
  switch (type) {
    case kQ4_K: launch_rows_x_type<kQ4_K>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
    case kIQ4_XS: launch_rows_x_type<kIQ4_XS>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
    default: launch_rows_x_type<kQ6_K>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
  }
  return hipGetLastError();
}

bool gemv_mfma4_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n);
hipError_t launch_gemv_mfma4(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                             void* y, int y_dtype, hipStream_t stream);

// n in 1..8 activation rows; q8: block_q8_1 of X; y: [n, nrows] in y_dtype.
hipError_t launch_gemv_raw(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                           void* y, int y_dtype, hipStream_t stream) {
  // Q4_K / IQ4_XS / Q6_K at 1-4 rows on weights of at least 8 K blocks (one per wave) below 2 GiB:
  // the row-chunk kernel (measured 17408 x 5120 M = 1 against a 16-row tile kernel with a lane per
  // slice pair: Q4_K 13.8 us against 16.0, and 16.9 against 20.5 on 5120 x 17408; at 3-4 rows it
  // replaces the generic GEMV and the MMA small GEMM: IQ4_XS M = 4 18.8 us against 25.6, Q6_K
  // 26.2 against 37.1 + quantise)
  // Q4_K / IQ4_XS / Q6_K at 2-4 rows (Q4_K / IQ4_XS also at one row on K > 8192): the MFMA decode
  // GEMV where it applies (gemv_mfma4.hip)
  if (gemv_mfma4_supported(type, nrows, row_bytes, k, n))
    return launch_gemv_mfma4(type, W, row_bytes, nrows, k, q8, n, y, y_dtype, stream);
  bool done = false;
  if (type == kQ4_K) done = launch_rows<kQ4_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream);
  if (type == kIQ4_XS) done = launch_rows<kIQ4_XS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream);
  if (type == kQ6_K) done = launch_rows<kQ6_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream);
  if (done) return hipGetLastError();
  switch (type) {
    case kIQ3_S: launch_type<kIQ3_S>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ4_K: launch_type<kQ4_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ4_XS: launch_type<kIQ4_XS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ6_K: launch_type<kQ6_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kQ2_K: launch_type<kQ2_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ2_XXS: launch_type<kIQ2_XXS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ2_XS: launch_type<kIQ2_XS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ2_S: launch_type<kIQ2_S>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ3_XXS: launch_type<kIQ3_XXS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ1_M: launch_type<kIQ1_M>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The generic types' decode GEMV with X (dtype x_dtype, row stride s01) quantised inside the
// stream GEMV, on the shapes gs_x_supported admits; bit-identical to the q8_1 quantiser +
// launch_gemv_raw.
bool gemv_generic_x_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n) {
  switch (type) {
    case kQ2_K: return gs_x_supported<kQ2_K>(nrows, row_bytes, k, n);
    case kIQ2_XXS: return gs_x_supported<kIQ2_XXS>(nrows, row_bytes, k, n);
    case kIQ2_XS: return gs_x_supported<kIQ2_XS>(nrows, row_bytes, k, n);
    case kIQ2_S: return gs_x_supported<kIQ2_S>(nrows, row_bytes, k, n);
    case kIQ3_XXS: return gs_x_supported<kIQ3_XXS>(nrows, row_bytes, k, n);
    case kIQ1_M: return gs_x_supported<kIQ1_M>(nrows, row_bytes, k, n);
    default: return false;
  }
}

hipError_t launch_gemv_generic_x(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x,
                                 int x_dtype, int64_t s01, int n, void* y, int y_dtype, hipStream_t stream) {
  if (!gemv_generic_x_supported(type, nrows, row_bytes, k, n)) return hipErrorInvalidValue;
  switch (type) {
    case kQ2_K: launch_gs_fused<kQ2_K>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
    case kIQ2_XXS: launch_gs_fused<kIQ2_XXS>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
    case kIQ2_XS: launch_gs_fused<kIQ2_XS>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
    case kIQ2_S: launch_gs_fused<kIQ2_S>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
    case kIQ3_XXS: launch_gs_fused<kIQ3_XXS>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
    default: launch_gs_fused<kIQ1_M>(W, row_bytes, nrows, k, x, x_dtype, s01, n, y, y_dtype, stream); break;
  }
  return hipGetLastError();
}

}  // namespace gguf
