// X staging helpers of the decode GEMVs: the q8_1 quantiser's arithmetic on groups of 8 values
// (bit-identical bytes), used where a GEMV quantises X itself, and the persistent grid size.
#pragma once

#include "gguf_common.h"

namespace gguf {

// workgroups of the persistent GEMVs: two per CU of the current device
inline int persist_grid() { return 2 * device_cus(); }

// q8_1 bytes of N (4 or 8) values of one slice, given the slice's amax and d = amax / 127: q =
// roundf(v / d) (q = 0 when amax == 0), bit for bit as the q8_1 quantiser computes them. The
// quotient comes from the product v * rcp(d): for |v| <= amax it lies within 2^-15 of v / d (rcp
// within 1 ulp), and the fp32 rounding of v / d moves that by less than 2^-16, so when the product
// lies more than 2^-12 from every half-integer, roundf(v / d) is the integer nearest to it. Adding
// 1.5 * 2^23 rounds to that integer and leaves it in the low mantissa bits. The largest distance
// is taken over the bit patterns of |a - n|, where a NaN (a NaN or infinite value) ranks above
// every number. A lane with a value near a tie, a non-finite product or a tiny amax (rcp of a
// subnormal d) takes the IEEE division. out[j] holds the bytes of values 4j..4j+3.
template <int N>
__device__ __forceinline__ void quantize_q81(const float (&v)[N], float amax, float d, uint32_t (&out)[N / 4]) {
  constexpr float kMagic = 12582912.0f;
  const float r = __builtin_amdgcn_rcpf(d);
  uint32_t m[N], dev = 0;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float a = v[e] * r;
    const float t = a + kMagic;
    m[e] = __float_as_uint(t);
    dev = max(dev, __float_as_uint(a - (t - kMagic)) & 0x7FFFFFFFu);
  }
#pragma unroll
  for (int j = 0; j < N / 4; ++j)
    out[j] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(m[4 * j + 3], m[4 * j + 2], 0x0c0c0400u),
                                   __builtin_amdgcn_perm(m[4 * j + 1], m[4 * j], 0x0c0c0400u), 0x05040100u);
  if (!(amax >= 0x1p-100f) || dev > __float_as_uint(0.5f - 0x1p-12f)) {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) out[j] = 0;
    if (amax != 0.0f) {
#pragma unroll
      for (int e = 0; e < N; ++e) out[e >> 2] |= ((uint32_t)(int)roundf(v[e] / d) & 0xFFu) << (8 * (e & 3));
    }
  }
}

template <int XDT>
struct XGroup {
  uint32_t v[XDT == kF32 ? 8 : (XDT < 0 ? 3 : 4)];
};

template <int NC, int XDT>
__device__ __forceinline__ void xgroup_load(const void* x, __amdgpu_buffer_rsrc_t xrs, int64_t s01, int nslices, int g,
                                            XGroup<XDT>& r) {
  const int sr = g >> 2, part = g & 3;
  if constexpr (XDT < 0) {  // block_q8_1: d (fp16) and s, then 32 q bytes
    const int o = sr * 36;
    r.v[0] = __builtin_amdgcn_raw_buffer_load_b32(xrs, o, 0, 0);
    r.v[1] = __builtin_amdgcn_raw_buffer_load_b32(xrs, o + 4 + 8 * part, 0, 0);
    r.v[2] = __builtin_amdgcn_raw_buffer_load_b32(xrs, o + 8 + 8 * part, 0, 0);
  } else {
    int c = 0, sl = sr;
#pragma unroll
    for (int i = 1; i < NC; ++i)
      if (sl >= nslices) sl -= nslices, ++c;
    const int64_t e0 = c * s01 + (int64_t)sl * kQ81 + 8 * part;
    if constexpr (XDT == kF32) {
      const uint4 a = *(const uint4*)((const float*)x + e0), b = *(const uint4*)((const float*)x + e0 + 4);
      r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
      r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
    } else {
      const uint4 a = *(const uint4*)((const uint16_t*)x + e0);
      r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
    }
  }
}

// max over the four lanes of a quad, exchanged by DPP quad permutes (xor 1, then xor 2)
__device__ __forceinline__ float quad_fmax(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true)));
  return v;
}

// q8_1 bytes (lo: values 0..3, hi: 4..7) and fp16 d of the group of 8 raw values in r: the four
// lanes of the slice exchange their amax (the quantiser's arithmetic, bit-identical bytes)
template <int XDT>
__device__ __forceinline__ void xgroup_quantize(const XGroup<XDT>& r, uint32_t& lo, uint32_t& hi, uint32_t& dbits) {
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (XDT == kF32) v[e] = __uint_as_float(r.v[e]);
    else {
      const uint32_t h = (r.v[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      v[e] = XDT == kF16 ? half_bits_to_float(h) : __uint_as_float(h << 16);
    }
  }
  float amax = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))),
                     fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7]))));
  amax = quad_fmax(amax);
  const float d = amax / 127.0f;
  uint32_t qw[2];
  quantize_q81<8>(v, amax, d, qw);
  lo = qw[0];
  hi = qw[1];
  dbits = __half_as_ushort(__float2half_rn(d));
}

}  // namespace gguf
