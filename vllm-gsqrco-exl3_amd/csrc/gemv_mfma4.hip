// Decode GEMV on v_mfma_i32_4x4x4_16b_i8 for 2-4 activation rows of Q4_K on GGUF rows:
// Y[c, r] = sum_k X[c, k] * W[r, k], X given as block_q8_1.
//
// Replaces the reference's 2..4-row Q4_K decode products (vendored MMVQ mul_mat_vec_q,
// mmvq.cu:600-760; the owned dp4a kernel lcpp_owned_k4.cu:116-269) where the row-chunk GEMV's
// v_dot4 work bounds it. v_mfma_i32_4x4x4_16b_i8 computes 16 independent 4 x 4 x 4 products per
// wave: with A = X (row i of block b from lane 4b + i, one activation row) and B = W (column j from
// lane 4b + j, one weight row), lane 4b + j receives the 4 activation rows' sums of weight row j,
// so at 4 activation rows every output lane is useful and the integer dot products leave the VALU.
//
// Work: the stream GEMV's split (gemv_iq3.hip). Rows form units of 4; one workgroup per CU owns
// an equal run of units, its items are (unit, pair of K blocks), unit-major, and each of its 8
// waves takes a contiguous run of items. An item is 4 rows x 2 blocks = 1152 bytes; lane
// l = 4b + r (r = l & 3, b = l >> 2 = 8 kb + 2 q + h) loads the 16-byte header and quant bytes
// [32q + 16h, +16) of block kb of row r: values 16h .. 16h + 15 of slice 2q (low nibbles) and of
// slice 2q + 1 (high nibbles) (ggml-common.h block_q4_K). One load instruction covers 4 rows x
// 256 contiguous quant bytes. Two accumulator sets take the low and high nibbles (4 MFMAs each);
// lanes h = 0 and h = 1 (l and l ^ 4) then exchange the half sums by DPP, and lane h finishes
// slice 2q + h of its row for each activation row with the reference's MMVQ arithmetic:
//   ((d * sc) * sumi - (dmin * m) * sum q8) * d8                      (vecdotq.cuh:508-530)
// The integer slice sums equal the reference's sumi bit for bit; the fp32 order in which a row's
// slice terms are added differs (per lane over its items, then lanes, then waves, in fixed order).
#include <algorithm>

#include "gemv_x.h"

namespace gguf {

typedef int m4_i32x4 __attribute__((ext_vector_type(4)));

constexpr int kM4Waves = 8;
constexpr int kM4UnitRows = 4;

struct M4Frag {
  u32x4 hdr;  // d | dmin << 16, then scales[0..12)
  u32x4 qs;   // quant bytes [32q + 16h, +16) of the block
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

// LDS of the kernel, in dwords: X's q values [NC][slice][8], X's (d8, sum of q) pairs [slice][4]
// (activation rows NC..3 unused), 16 zero dwords (the A operands of absent activation rows), then
// the partial sums [unit][wave][lane group g = l >> 4][row][NC].
__host__ __device__ constexpr size_t m4_lds_bytes(int nc, int64_t nslices, int64_t units_per_wg) {
  return (size_t)nc * nslices * 32 + (size_t)nslices * 32 + 64 + (size_t)units_per_wg * kM4Waves * 4 * 4 * nc * 4;
}

// XPT: groups of 8 X values staged per thread (NC * K / 8 <= XPT * 512).
template <int NC, int XPT>
__global__ void __launch_bounds__(64 * kM4Waves) gemv_q4k_mfma4_kernel(const uint8_t* __restrict__ W, int row_bytes,
                                                                       int nrows, int k,
                                                                       const uint8_t* __restrict__ q8,
                                                                       void* __restrict__ y, int y_dtype) {
  constexpr int NW = kM4Waves, NT = 64 * NW;
  extern __shared__ uint4 m4dyn[];
  __shared__ uint4 sink;  // staging writes of groups past the end of X
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 3, b = lane >> 2, kb = b >> 3, q = (b >> 1) & 3, h = b & 1;
  const int u = 2 * q + h;  // the slice of block kb this lane finishes
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
  const int off_h = r * row_bytes + kb * 144, off_q = off_h + 16 + 32 * q + 16 * h;
  const int j0 = wave * items / NW, j1 = (wave + 1) * items / NW;
  const int cu0 = j0 / npair;
  int lj = j0, lu = cu0, lp = j0 - cu0 * npair;  // the next item to load
  auto load_next = [&](M4Frag& f) {
    const bool in_run = lj < j1;
    const __amdgpu_buffer_rsrc_t rs = in_run ? wrs : nrs;
    const int so = in_run ? lu * (int)ubytes + lp * 288 : 0;
    f.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, off_h, so, 0);
    f.qs = __builtin_amdgcn_raw_buffer_load_b128(rs, off_q, so, 0);
    ++lj;
    if (++lp == npair) {
      lp = 0;
      ++lu;
    }
  };
  M4Frag f0, f1, f2;
  load_next(f0);
  load_next(f1);
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
    const int c = sr / nslices, sl = sr - c * nslices;
    *(live && pt == 0 ? xs + sl * 4 + c : (float2*)&sink) = make_float2(half_bits_to_float(xg[j].d & 0xFFFFu), (float)t);
  }
  if (threadIdx.x < 16) xz[threadIdx.x] = 0u;
  for (int t = threadIdx.x; t < nu * NW * 4 * NC; t += NT) ((float4*)part)[t] = make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  // per-lane LDS bases: A operands (activation row r, slices 2q / 2q + 1 of block kb, dwords
  // 4h..4h+3), absent rows read zeros; the (d8, sum) pairs of slice u of block kb
  const bool xlive = r < NC;
  const uint32_t* xa = xlive ? xq + (r * nslices + kb * 8 + 2 * q) * 8 + 4 * h : xz;
  const int xstep = xlive ? 16 * 8 : 0;  // dwords per block pair
  const float2* xsl = xs + (kb * 8 + u) * 4;
  const uint32_t sh = 8 * (u & 3);
  float acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
  int cu = cu0, cp = j0 - cu0 * npair, j = j0;  // the item being computed
  auto step = [&](const M4Frag& fc, M4Frag& fl) {
    load_next(fl);
    __builtin_amdgcn_sched_barrier(0);
    const uint4 a0 = *(const uint4*)(xa + cp * xstep), a1 = *(const uint4*)(xa + cp * xstep + 8);
    const int alo[4] = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w};
    const int ahi[4] = {(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
    m4_i32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo = __builtin_amdgcn_mfma_i32_4x4x4i8(alo[e], (int)(fc.qs[e] & 0x0F0F0F0Fu), lo, 0, 0, 0);
      hi = __builtin_amdgcn_mfma_i32_4x4x4i8(ahi[e], (int)((fc.qs[e] >> 4) & 0x0F0F0F0Fu), hi, 0, 0, 0);
    }
    // lane h = 0 finishes slice 2q with the partner's (l + 4) low half; h = 1 slice 2q + 1 with
    // the partner's (l - 4) high half
    const float4 s0 = *(const float4*)(xsl + cp * 64), s1 = *(const float4*)(xsl + cp * 64 + 2);
    const float2 xsv[4] = {make_float2(s0.x, s0.y), make_float2(s0.z, s0.w), make_float2(s1.x, s1.y),
                           make_float2(s1.z, s1.w)};
    const uint32_t sa = (fc.hdr[1] >> sh) & 0xFFu, sb = (fc.hdr[2] >> sh) & 0xFFu, se = (fc.hdr[3] >> sh) & 0xFFu;
    const uint32_t sc = u < 4 ? (sa & 63u) : ((se & 0xFu) | ((sa >> 6) << 4));
    const uint32_t m = u < 4 ? (sb & 63u) : ((se >> 4) | ((sb >> 6) << 4));
    const float d = half_bits_to_float(fc.hdr[0] & 0xFFFFu), dmin = half_bits_to_float(fc.hdr[0] >> 16);
    const float dsc = d * (float)sc, dm = dmin * (float)m;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int send = h ? lo[c] : hi[c];
      const int up = m4_dpp<0x104>(send);  // row_shl:4, lane l reads l + 4
      const int dn = m4_dpp<0x114>(send);  // row_shr:4, lane l reads l - 4
      const int sumi = h ? dn + hi[c] : lo[c] + up;
      const float term = dsc * (float)sumi - dm * xsv[c].y;
      acc[c] = fmaf(term, xsv[c].x, acc[c]);
    }
    ++j;
    if (++cp == npair || j == j1) {  // leaving the unit: the wave's partial sums to its slot
      const int slot = cu * NW + wave;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float v = acc[c];
        v += m4_dpp_f<0x124>(v);  // row_ror:4
        v += m4_dpp_f<0x128>(v);  // row_ror:8: the 4 lanes of row r in this 16-lane group
        if ((lane & 12) == 0) part[((slot * 4 + (lane >> 4)) * 4 + r) * NC + c] = v;
        acc[c] = 0.0f;
      }
      if (cp == npair) {
        cp = 0;
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
  // output (unit, activation row, row): the slots of every wave in wave order, each over the 4
  // lane groups in order
  const int nout = nu * kM4UnitRows * NC;
  for (int t = threadIdx.x; t < nout; t += NT) {
    const int uu = t / (kM4UnitRows * NC), c = (t / kM4UnitRows) % NC, row = t % kM4UnitRows;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float* pp = part + ((uu * NW + w) * 4 * 4 + row) * NC + c;
      v += ((pp[0] + pp[4 * NC]) + (pp[8 * NC] + pp[12 * NC]));
    }
    store_y(y, (int64_t)c * nrows + (int64_t)(u0 + uu) * kM4UnitRows + row, v, y_dtype);
  }
}

// ---------------------------------------------------------------------------------------------
// Launch plan

constexpr int kM4Xpt[] = {2, 3, 5, 9, 13, 17};
constexpr size_t kM4LdsMax = 160 * 1024 - sizeof(uint4);  // the dynamic LDS a workgroup may take

static int m4_xpt(int64_t k, int64_t n) {
  const int64_t need = (n * (k / kQ81) * 4 + 511) / 512;
  for (int x : kM4Xpt)
    if (x >= need) return x;
  return 0;
}

static int64_t m4_units_per_wg(int64_t nrows, int64_t grid) { return (nrows / kM4UnitRows + grid - 1) / grid; }

// Q4_K at 2-4 activation rows, rows % 4 == 0 with at least one unit per CU, K % 512 == 0 (whole
// block pairs), a weight below 2 GiB, X within the staged groups and the LDS.
bool gemv_mfma4_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n) {
  if (type != kQ4_K || n < 2 || n > 4 || k % 512 != 0 || nrows % kM4UnitRows != 0) return false;
  if (row_bytes != k / kQK * 144 || nrows * row_bytes >= ((int64_t)1 << 31)) return false;
  const int64_t cus = device_cus();
  if (nrows / kM4UnitRows < cus || m4_xpt(k, n) == 0) return false;
  return m4_lds_bytes((int)n, k / kQ81, m4_units_per_wg(nrows, cus)) <= kM4LdsMax;
}

template <int NC, int XPT>
static void launch_m4_x(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, void* y, int y_dtype,
                        hipStream_t stream) {
  const int cus = device_cus();
  const size_t lds = m4_lds_bytes(NC, k / kQ81, m4_units_per_wg(nrows, cus));
  int dev = 0;
  if (lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess) {
    struct Tag;
    once_per_device<Tag>(dev, [] {
      (void)hipFuncSetAttribute((const void*)gemv_q4k_mfma4_kernel<NC, XPT>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kM4LdsMax);
    });
  }
  gemv_q4k_mfma4_kernel<NC, XPT><<<cus, 64 * kM4Waves, lds, stream>>>(W, (int)row_bytes, nrows, k, q8, y, y_dtype);
}

template <int NC>
static void launch_m4_nc(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, void* y,
                         int y_dtype, hipStream_t stream) {
  switch (m4_xpt(k, NC)) {
    case 2: launch_m4_x<NC, 2>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 3: launch_m4_x<NC, 3>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 5: launch_m4_x<NC, 5>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 9: launch_m4_x<NC, 9>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 13: launch_m4_x<NC, 13>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    default: launch_m4_x<NC, 17>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
  }
}

// n in 2..4 activation rows on the shapes gemv_mfma4_supported admits; q8: block_q8_1 of X;
// y: [n, nrows] in y_dtype.
hipError_t launch_gemv_mfma4(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                             void* y, int y_dtype, hipStream_t stream) {
  if (!gemv_mfma4_supported(type, nrows, row_bytes, k, n)) return hipErrorInvalidValue;
  switch (n) {
    case 2: launch_m4_nc<2>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    case 3: launch_m4_nc<3>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
    default: launch_m4_nc<4>(W, row_bytes, nrows, k, q8, y, y_dtype, stream); break;
  }
  return hipGetLastError();
}

}  // namespace gguf
