// Decode GEMV on v_mfma_i32_4x4x4_16b_i8 for 2-4 activation rows of Q4_K, IQ4_XS and Q6_K on GGUF
// rows (and one row of Q4_K / IQ4_XS on long K): Y[c, r] = sum_k X[c, k] * W[r, k], X given as
// block_q8_1.
//
// Replaces the reference's 2..4-row decode products of these types (vendored MMVQ
// mul_mat_vec_q, mmvq.cu:600-760; the owned dp4a kernel lcpp_owned_k4.cu:116-269) where the
// row-chunk GEMV's v_dot4 work bounds it. v_mfma_i32_4x4x4_16b_i8 computes 16 independent
// 4 x 4 x 4 products per wave: with A = X (row i of block b from lane 4b + i, one activation row)
// and B = W (column j from lane 4b + j, one weight row), lane 4b + j receives the 4 activation
// rows' sums of weight row j, so at 4 activation rows every output lane is useful and the integer
// dot products leave the VALU.
//
// Work: the stream GEMV's split (gemv_iq3.hip). Rows form units of 4; one workgroup per CU owns
// an equal run of units, its items are (unit, pair of K blocks), unit-major, and each of its 8
// waves takes a contiguous run of items. Lane l = 4b + r (r = l & 3, b = l >> 2 = 8 kb + c) loads
// 16-byte chunk c of the quant bytes of block kb of row r and what its values need of the block
// header (ggml-common.h block layouts), so one load instruction covers 4 rows x 2 blocks of quant
// bytes contiguously. What chunk c holds, and the slice term (the reference's MMVQ arithmetic):
//   Q4_K    half h = c & 1 of slices 2q (low nibbles) and 2q + 1 (high), q = c >> 1;
//           ((d * sc) * sumi - (dmin * m) * sum q8) * d8                 (vecdotq.cuh:508-530)
//   IQ4_XS  slice c: values 0..15 (low nibbles), 16..31 (high), through the IQ4_NL codebook;
//           (float)(sumi * ls) * (d * d8)                                (vecdotq.cuh:1357-1380)
//   Q6_K    half h of slices 4n + t (low nibbles) and 4n + t + 2 (high), c = 4n + 2t + h, with
//           the high bits from qh and the -32 offset in the operand; d * (float)(sc_a * sumi_a +
//           sc_b * sumi_b) * d8 over the slice's two 16-value halves     (vecdotq.cuh:627-648)
// Q4_K and Q6_K accumulate their two slices' halves in two sets (4 MFMAs each); lanes h = 0 and
// h = 1 (l and l ^ 4) then exchange integer half sums by DPP, and lane h finishes slice 2q + h
// (Q4_K) or the low / high slice (Q6_K). IQ4_XS lanes finish their slice from one set (8 MFMAs).
// The integer slice sums equal the reference's sumi bit for bit; the fp32 order in which a row's
// slice terms are added differs (per lane over its items, then lanes, then waves, in fixed order).
#include <algorithm>

#include "gemv_x.h"

namespace gguf {

typedef int m4_i32x4 __attribute__((ext_vector_type(4)));

constexpr int kM4Waves = 8;
constexpr int kM4UnitRows = 4;

// The bytes a lane loads per item (block kb of the pair, its chunk c = b & 7).
template <int TYPE>
struct M4Frag;
template <>
struct M4Frag<kQ4_K> {
  u32x4 hdr;  // d | dmin << 16, then scales[0..12)
  u32x4 qs;   // quant bytes [16c, +16)
};
template <>
struct M4Frag<kIQ4_XS> {
  uint2 hdr;  // d | scales_h << 16, scales_l
  u32x4 qs;   // quant bytes [16c, +16): slice c
};
// Q6_K blocks are 210 bytes, so block kb = 1 of a pair starts 2 bytes past a dword boundary, and
// 16-byte loads there are split by the memory pipeline (measured: 30.4 against 20.0 us for
// 17408 x 5120 at 2 rows). The lane loads the dword-aligned 16 bytes at or 2 below each 16-byte
// field and the dword after them, and takes the field with a byte align; the scale bytes and d
// come from byte and 16-bit loads (narrow fields, so no widening waits at the loop head).
template <>
struct M4Frag<kQ6_K> {
  u32x4 ql;      // from ql[16c - mis]
  u32x4 qh;      // from qh[32n + 16h - mis]
  uint32_t qlx;  // the dword after each
  uint32_t qhx;
  uint8_t s0, s1;  // scales[8n + 2t + h], scales[8n + 4 + 2t + h]
  uint16_t d;      // fp16 d
};

// one group of 8 q8_1 values (block g >> 2 of the block_q8_1 array, part g & 3): the block's
// d | sum word and the part's 8 bytes
struct M4XGroup {
  uint32_t d, q0, q1;
};

__device__ __forceinline__ void m4_xgroup_load(__amdgpu_buffer_rsrc_t xrs, int g, M4XGroup& r) {
  const int o = (g >> 2) * 36, part = g & 3;
  r.d = __builtin_amdgcn_raw_buffer_load_b32(xrs, o, 0, 0);
  r.q0 = __builtin_amdgcn_raw_buffer_load_b32(xrs, o + 4 + 8 * part, 0, 0);
  r.q1 = __builtin_amdgcn_raw_buffer_load_b32(xrs, o + 8 + 8 * part, 0, 0);
}

// DPP move with every lane's source valid for the controls used here
template <int CTRL>
__device__ __forceinline__ int m4_dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float m4_dpp_f(float v) {
  return __int_as_float(m4_dpp<CTRL>(__float_as_int(v)));
}

// lanes l and l ^ 4 (h = 0, 1: the halves of the same slices) exchange one integer each: the
// value of the slice the other finishes (h = 0 reads lane l + 4, h = 1 lane l - 4)
__device__ __forceinline__ int m4_partner(int send, int h) {
  const int up = m4_dpp<0x104>(send);  // row_shl:4
  const int dn = m4_dpp<0x114>(send);  // row_shr:4
  return h ? dn : up;
}

// bytewise v - 32 of 6-bit values (Q6_K's offset), as int8
__device__ __forceinline__ int m4_minus32(uint32_t v) {
  return (int)(((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
}

// LDS of the kernel, in dwords: X's q values [NC][slice][8], X's (d8, sum of q) pairs [slice][4]
// (activation rows NC..3 unused), 16 zero dwords (the A operands of absent activation rows), then
// the partial sums [unit][wave][lane group g = l >> 4][row][NC].
__host__ __device__ constexpr size_t m4_lds_bytes(int nc, int64_t nslices, int64_t units_per_wg) {
  return (size_t)nc * nslices * 32 + (size_t)nslices * 32 + 64 + (size_t)units_per_wg * kM4Waves * 4 * 4 * nc * 4;
}

// XPT: groups of 8 X values staged per thread (NC * K / 8 <= XPT * 512).
template <int TYPE, int NC, int XPT>
__global__ void __launch_bounds__(64 * kM4Waves) gemv_mfma4_kernel(const uint8_t* __restrict__ W, int row_bytes,
                                                                   int nrows, int k, const uint8_t* __restrict__ q8,
                                                                   void* __restrict__ y, int y_dtype) {
  constexpr int NW = kM4Waves, NT = 64 * NW, BS = block_bytes(TYPE);
  extern __shared__ uint4 m4dyn[];
  __shared__ uint4 sink;  // staging writes of groups past the end of X
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 3, b = lane >> 2, kb = b >> 3, c = b & 7, h = c & 1;
  // the lane's two operand slices of block kb (A / B: dwords da..da+3 of slice s0, of slice s1)
  // and the slice it finishes
  int s0, s1, da, uf;
  if constexpr (TYPE == kQ4_K) {  // half h of slices 2q (low nibbles), 2q + 1 (high), q = c >> 1
    s0 = c & ~1; s1 = s0 + 1; da = 4 * h; uf = c;
  } else if constexpr (TYPE == kIQ4_XS) {  // slice c: values 0..15 (low nibbles), 16..31 (high)
    s0 = s1 = c; da = 0; uf = c;
  } else {  // Q6_K: half h of slices 4n + t (low nibbles), 4n + t + 2 (high), c = 4n + 2t + h
    s0 = 4 * (c >> 2) + ((c >> 1) & 1); s1 = s0 + 2; da = 4 * h; uf = h ? s1 : s0;
  }
  const int nb = k / kQK, npair = nb >> 1, nslices = k / kQ81;
  uint32_t* xq = (uint32_t*)m4dyn;
  float2* xs = (float2*)(xq + NC * nslices * 8);
  uint32_t* xz = (uint32_t*)(xs + nslices * 4);
  float* part = (float*)(xz + 16);
  // X: every thread issues its groups' loads before any weight load (a CU's loads return in order)
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(q8, (uint32_t)(NC * nslices * 36));
  const int ngroups = NC * nslices * 4;
  M4XGroup xg[XPT];
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int g = (int)threadIdx.x + j * NT;
    m4_xgroup_load(xrs, g < ngroups ? g : ngroups - 1, xg[j]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the workgroup's units [u0, u1) and the wave's items [j0, j1)
  const uint32_t nunits = (uint32_t)nrows / kM4UnitRows, G = gridDim.x;
  const int u0 = (int)(blockIdx.x * nunits / G), u1 = (int)((blockIdx.x + 1) * nunits / G);
  const int nu = u1 - u0, items = nu * npair;
  const uint32_t ubytes = (uint32_t)(kM4UnitRows * row_bytes);
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(W + (int64_t)u0 * ubytes, (uint32_t)nu * ubytes);
  // loads past the wave's run read zeros from an empty range (the range check sees only the lane
  // offset, which stays inside the unit's bytes)
  const __amdgpu_buffer_rsrc_t nrs = buffer_rsrc(W, 0u);
  const int ob = r * row_bytes + kb * BS;  // the lane's block, first item
  const int mis = (kb * BS) & 3;            // its byte offset past a dword boundary (row_bytes % 4 == 0)
  const int j0 = wave * items / NW, j1 = (wave + 1) * items / NW;
  const int cu0 = j0 / npair;
  int lj = j0, lu = cu0, lp = j0 - cu0 * npair;  // the next item to load
  auto load_next = [&](M4Frag<TYPE>& f) {
    const bool in_run = lj < j1;
    const __amdgpu_buffer_rsrc_t rs = in_run ? wrs : nrs;
    const int so = in_run ? lu * (int)ubytes + lp * (2 * BS) : 0;
    if constexpr (TYPE == kQ4_K) {
      f.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, ob, so, 0);
      f.qs = __builtin_amdgcn_raw_buffer_load_b128(rs, ob + 16 + 16 * c, so, 0);
    } else if constexpr (TYPE == kIQ4_XS) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, ob, so, 0);
      f.hdr = make_uint2(v[0], v[1]);
      f.qs = __builtin_amdgcn_raw_buffer_load_b128(rs, ob + 8 + 16 * c, so, 0);
    } else {  // mis = 2 kb: every offset stays inside the lane's row (ob - mis >= 208 when kb = 1)
      const int n = c >> 2, oql = ob + 16 * c - mis, oqh = ob + 128 + 32 * n + 16 * h - mis;
      f.ql = __builtin_amdgcn_raw_buffer_load_b128(rs, oql, so, 0);
      f.qlx = __builtin_amdgcn_raw_buffer_load_b32(rs, oql + 16, so, 0);
      f.qh = __builtin_amdgcn_raw_buffer_load_b128(rs, oqh, so, 0);
      f.qhx = __builtin_amdgcn_raw_buffer_load_b32(rs, oqh + 16, so, 0);
      f.s0 = __builtin_amdgcn_raw_buffer_load_b8(rs, ob + 192 + 8 * n + 2 * ((c >> 1) & 1) + h, so, 0);
      f.s1 = __builtin_amdgcn_raw_buffer_load_b8(rs, ob + 196 + 8 * n + 2 * ((c >> 1) & 1) + h, so, 0);
      f.d = __builtin_amdgcn_raw_buffer_load_b16(rs, ob + 208, so, 0);
    }
    ++lj;
    if (++lp == npair) {
      lp = 0;
      ++lu;
    }
  };
  M4Frag<TYPE> f0, f1, f2, f3;
  load_next(f0);
  load_next(f1);
  load_next(f2);
  __builtin_amdgcn_sched_barrier(0);
  // X to LDS: q bytes to xq, (d8, integer sum of the slice's q) to xs[slice][activation row]; the
  // 4 parts of a slice are the 4 lanes of a quad (g & 3 = lane & 3)
#pragma unroll
  for (int j = 0; j < XPT; ++j) {
    const int g = (int)threadIdx.x + j * NT;
    const bool live = g < ngroups;
    int t = dot4(0x01010101, (int)xg[j].q1, dot4(0x01010101, (int)xg[j].q0, 0));
    t += m4_dpp<0xB1>(t);  // quad xor 1
    t += m4_dpp<0x4E>(t);  // quad xor 2
    const int sr = g >> 2, pt = g & 3;
    *(live ? (uint2*)(xq + sr * 8 + 2 * pt) : (uint2*)&sink) = make_uint2(xg[j].q0, xg[j].q1);
    const int cc = sr / nslices, sl = sr - cc * nslices;
    *(live && pt == 0 ? xs + sl * 4 + cc : (float2*)&sink) =
        make_float2(half_bits_to_float(xg[j].d & 0xFFFFu), (float)t);
  }
  if (threadIdx.x < 16) xz[threadIdx.x] = 0u;
  for (int t = threadIdx.x; t < nu * NW * 4 * NC; t += NT) ((float4*)part)[t] = make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  // per-lane LDS bases of the first block pair: the A operands (activation row r), absent rows
  // read zeros; the (d8, sum) pairs of the finished slice
  const bool xlive = r < NC;
  const uint32_t* xa0 = xlive ? xq + (r * nslices + kb * 8 + s0) * 8 + da : xz;
  const uint32_t* xa1 = xlive ? xq + (r * nslices + kb * 8 + s1) * 8 + da + (TYPE == kIQ4_XS ? 4 : 0) : xz;
  const int xstep = xlive ? 16 * 8 : 0;  // dwords per block pair
  const float2* xsl = xs + (kb * 8 + uf) * 4;
  float acc[NC];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) acc[cc] = 0.0f;
  int cu = cu0, cp = j0 - cu0 * npair, j = j0;  // the item being computed
  auto step = [&](const M4Frag<TYPE>& fc, M4Frag<TYPE>& fl) {
    load_next(fl);
    __builtin_amdgcn_sched_barrier(0);
    const uint4 a0 = *(const uint4*)(xa0 + cp * xstep), a1 = *(const uint4*)(xa1 + cp * xstep);
    const int alo[4] = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w};
    const int ahi[4] = {(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
    const float4 x0 = *(const float4*)(xsl + cp * 64), x1 = *(const float4*)(xsl + cp * 64 + 2);
    const float d8[4] = {x0.x, x0.z, x1.x, x1.z};
    const float sq[4] = {x0.y, x0.w, x1.y, x1.w};
    m4_i32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
    if constexpr (TYPE == kQ4_K) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo = __builtin_amdgcn_mfma_i32_4x4x4i8(alo[e], (int)(fc.qs[e] & 0x0F0F0F0Fu), lo, 0, 0, 0);
        hi = __builtin_amdgcn_mfma_i32_4x4x4i8(ahi[e], (int)((fc.qs[e] >> 4) & 0x0F0F0F0Fu), hi, 0, 0, 0);
      }
      // vecdotq.cuh:508-530: ((d * sc) * sumi - (dmin * m) * sum q8) * d8, slice uf of the block
      const uint32_t sh = 8 * (uf & 3);
      const uint32_t sa = (fc.hdr[1] >> sh) & 0xFFu, sb = (fc.hdr[2] >> sh) & 0xFFu, se = (fc.hdr[3] >> sh) & 0xFFu;
      const uint32_t sc = uf < 4 ? (sa & 63u) : ((se & 0xFu) | ((sa >> 6) << 4));
      const uint32_t m = uf < 4 ? (sb & 63u) : ((se >> 4) | ((sb >> 6) << 4));
      const float d = half_bits_to_float(fc.hdr[0] & 0xFFFFu), dmin = half_bits_to_float(fc.hdr[0] >> 16);
      const float dsc = d * (float)sc, dm = dmin * (float)m;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const int got = m4_partner(h ? lo[cc] : hi[cc], h);
        const int sumi = h ? got + hi[cc] : lo[cc] + got;
        const float term = dsc * (float)sumi - dm * sq[cc];
        acc[cc] = fmaf(term, d8[cc], acc[cc]);
      }
    } else if constexpr (TYPE == kIQ4_XS) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo = __builtin_amdgcn_mfma_i32_4x4x4i8(alo[e], iq4nl(fc.qs[e], 0), lo, 0, 0, 0);
        lo = __builtin_amdgcn_mfma_i32_4x4x4i8(ahi[e], iq4nl(fc.qs[e], 4), lo, 0, 0, 0);
      }
      // vecdotq.cuh:1357-1380: (float)(sumi * ls) * (d * d8)
      const int ls = (int)(((fc.hdr.y >> (4 * c)) & 0xF) | (((fc.hdr.x >> (16 + 2 * c)) & 3u) << 4)) - 32;
      const float d = half_bits_to_float(fc.hdr.x & 0xFFFFu);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) acc[cc] = fmaf(d * (float)__mul24(lo[cc], ls), d8[cc], acc[cc]);
    } else {
      const int t2 = 2 * ((c >> 1) & 1);  // qh bit pair of the low-nibble slice
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t l = __builtin_amdgcn_alignbyte(e < 3 ? fc.ql[e + 1] : fc.qlx, fc.ql[e], mis);
        const uint32_t q = __builtin_amdgcn_alignbyte(e < 3 ? fc.qh[e + 1] : fc.qhx, fc.qh[e], mis);
        const uint32_t w0 = (l & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(q, q, (t2 + 28) & 31) & 0x30303030u);
        const uint32_t w1 = ((l >> 4) & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(q, q, t2 & 31) & 0x30303030u);
        lo = __builtin_amdgcn_mfma_i32_4x4x4i8(alo[e], m4_minus32(w0), lo, 0, 0, 0);
        hi = __builtin_amdgcn_mfma_i32_4x4x4i8(ahi[e], m4_minus32(w1), hi, 0, 0, 0);
      }
      // vecdotq.cuh:627-648: (sc_a * sumi_a + sc_b * sumi_b) with the 16-value scales of the two
      // halves, then d * d8; the -32 offset is in the operand
      const int sc0 = (int)(int8_t)fc.s0, sc1 = (int)(int8_t)fc.s1;
      const float dr = half_bits_to_float(fc.d);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const int p0 = __mul24(lo[cc], sc0), p1 = __mul24(hi[cc], sc1);
        const int got = m4_partner(h ? p0 : p1, h);
        const int tot = h ? got + p1 : p0 + got;
        acc[cc] = fmaf(dr * (float)tot, d8[cc], acc[cc]);
      }
    }
    ++j;
    if (++cp == npair || j == j1) {  // leaving the unit: the wave's partial sums to its slot
      const int slot = cu * NW + wave;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        float v = acc[cc];
        v += m4_dpp_f<0x124>(v);  // row_ror:4
        v += m4_dpp_f<0x128>(v);  // row_ror:8: the 4 lanes of row r in this 16-lane group
        if ((lane & 12) == 0) part[((slot * 4 + (lane >> 4)) * 4 + r) * NC + cc] = v;
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
  // output (unit, activation row, row): the slots of every wave in wave order, each over the 4
  // lane groups in order
  const int nout = nu * kM4UnitRows * NC;
  for (int t = threadIdx.x; t < nout; t += NT) {
    const int uu = t / (kM4UnitRows * NC), cc = (t / kM4UnitRows) % NC, row = t % kM4UnitRows;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float* pp = part + ((uu * NW + w) * 4 * 4 + row) * NC + cc;
      v += ((pp[0] + pp[4 * NC]) + (pp[8 * NC] + pp[12 * NC]));
    }
    store_y(y, (int64_t)cc * nrows + (int64_t)(u0 + uu) * kM4UnitRows + row, v, y_dtype);
  }
}

// ---------------------------------------------------------------------------------------------
// Launch plan

constexpr int kM4Xpt[] = {2, 3, 5, 9, 13, 17};
// the dynamic LDS a workgroup may take: 160 KB less the static sink and its alignment padding
constexpr size_t kM4LdsMax = 160 * 1024 - 256;

static int m4_xpt(int64_t k, int64_t n) {
  const int64_t need = (n * (k / kQ81) * 4 + 511) / 512;
  for (int x : kM4Xpt)
    if (x >= need) return x;
  return 0;
}

static int64_t m4_units_per_wg(int64_t nrows, int64_t grid) { return (nrows / kM4UnitRows + grid - 1) / grid; }

// Q4_K, IQ4_XS and Q6_K at 2-4 activation rows, and Q4_K / IQ4_XS at one row on K > 8192 (where
// the row-chunk GEMV does not quantise X itself and its 8-row tiles leave CUs uneven: 5120 x 17408
// at one row 16.1 -> 14.7 us for Q4_K, 17.2 -> 16.5 for IQ4_XS; Q6_K's row-chunk GEMV stays
// faster there); rows % 4 == 0 with at least one unit per CU, K % 512 == 0 (whole block pairs), a
// weight below 2 GiB, X within the staged groups and the LDS.
bool gemv_mfma4_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n) {
  if (!(type == kQ4_K || type == kIQ4_XS || type == kQ6_K)) return false;
  if (n == 1 && (k <= 8192 || type == kQ6_K)) return false;
  // Q6_K at two rows: the row-chunk GEMV (X quantised inside at K <= 8192) is faster, measured
  // in graph replays (op with X): 17408 x 5120 22.1-22.8 against 23.8 us, 5120 x 17408 24.1-24.3
  // against 26.9; from three rows this kernel is (24.8 against 24.2-24.6 us and 28.0 against
  // 36.9 at three, 24.7 / 29.0 against 27.1 / 40.7 at four). Q4_K and IQ4_XS at two rows stay
  // here: the row-chunk GEMV measured 19.1 / 20.1 against 14.5 / 16.8 us (Q4_K 17408 x 5120 /
  // 5120 x 17408) and 17.9 / 19.6 against 16.3 / 17.2 (IQ4_XS).
  if (type == kQ6_K && n == 2) return false;
  if (n < 1 || n > 4 || k % 512 != 0 || nrows % kM4UnitRows != 0) return false;
  if (row_bytes != k / kQK * block_bytes(type) || nrows * row_bytes >= ((int64_t)1 << 31)) return false;
  const int64_t cus = device_cus();
  if (nrows / kM4UnitRows < cus || m4_xpt(k, n) == 0) return false;
  return m4_lds_bytes((int)n, k / kQ81, m4_units_per_wg(nrows, cus)) <= kM4LdsMax;
}

template <int TYPE, int NC, int XPT>
static void launch_m4_x(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, void* y, int y_dtype,
                        hipStream_t stream) {
  const int cus = device_cus();
  const size_t lds = m4_lds_bytes(NC, k / kQ81, m4_units_per_wg(nrows, cus));
  int dev = 0;
  if (lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess) {
    struct Tag;
    once_per_device<Tag>(dev, [] {
      (void)hipFuncSetAttribute((const void*)gemv_mfma4_kernel<TYPE, NC, XPT>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kM4LdsMax);
    });
  }
  gemv_mfma4_kernel<TYPE, NC, XPT><<<cus, 64 * kM4Waves, lds, stream>>>(W, (int)row_bytes, nrows, k, q8, y, y_dtype);
}

template <int TYPE, int NC>
static void launch_m4_nc(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, void* y,
                         int y_dtype, hipStream_t stream) {
  switch (m4_xpt(k, NC)) {
    case 2: launch_m4_x<TYPE, NC, 2>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 3: launch_m4_x<TYPE, NC, 3>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 5: launch_m4_x<TYPE, NC, 5>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 9: launch_m4_x<TYPE, NC, 9>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 13: launch_m4_x<TYPE, NC, 13>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    default: launch_m4_x<TYPE, NC, 17>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
  }
}

template <int TYPE>
static void launch_m4_type(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n, void* y,
                           int y_dtype, hipStream_t stream) {
  switch (n) {
    case 1: launch_m4_nc<TYPE, 1>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 2: launch_m4_nc<TYPE, 2>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 3: launch_m4_nc<TYPE, 3>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    default: launch_m4_nc<TYPE, 4>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
  }
}

// n in 1..4 activation rows on the shapes gemv_mfma4_supported admits; q8: block_q8_1 of X;
// y: [n, nrows] in y_dtype.
hipError_t launch_gemv_mfma4(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                             void* y, int y_dtype, hipStream_t stream) {
  if (!gemv_mfma4_supported(type, nrows, row_bytes, k, n)) return hipErrorInvalidValue;
  switch (type) {
    case kQ4_K: launch_m4_type<kQ4_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    case kIQ4_XS: launch_m4_type<kIQ4_XS>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
    default: launch_m4_type<kQ6_K>(W, row_bytes, nrows, k, q8, n, y, y_dtype, stream); break;
  }
  return hipGetLastError();
}

}  // namespace gguf
