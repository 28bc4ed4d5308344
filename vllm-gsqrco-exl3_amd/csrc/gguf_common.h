// GGUF block formats, codebooks and small device helpers shared by the gfx950 kernels.
//
// Block layouts follow the reference's ggml-common.h (plugin/vllm_gguf_plugin/csrc/lcpp/ggml/
// src/ggml-common.h): block_q8_1 :259-268, block_q4_K :327-338, block_q6_K :362-368,
// block_iq3_s :415-422, block_iq4_xs :454-460. They are a storage format, so the byte offsets
// below are the format's, written as offsets rather than structs (the kernels read blocks that
// are only 2-byte aligned, with explicit unaligned loads).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gguf {

// ggml type ids (gguf GGMLQuantizationType)
constexpr int kQ4_K = 12;
constexpr int kQ6_K = 14;
constexpr int kIQ3_S = 21;
constexpr int kIQ4_XS = 23;

constexpr int kQK = 256;   // values per super-block
constexpr int kQ81 = 32;   // values per q8_1 block ("slice")

// dtype codes at the C-ABI (include/gguf_mi355x.h)
constexpr int kF32 = 0, kF16 = 1, kBF16 = 2, kU8 = 3;

__host__ __device__ constexpr int block_bytes(int type) {
  return type == kQ4_K ? 144 : type == kQ6_K ? 210 : type == kIQ3_S ? 110 : type == kIQ4_XS ? 136 : 0;
}

// ---------------------------------------------------------------------------------------------
// IQ3_S codebook (ggml-common.h:1052 iq3s_grid). The grid is the ascending list of the 512
// points of {1,3,...,15}^4 the format uses; it is stored here as a 4096-bit membership set over
// codes c = sum_b ((byte_b - 1) / 2) << 3b and expanded at compile time. Enumerating members in
// ascending c yields the reference table in its own (ascending uint32) order.
struct Iq3sGrid {
  uint32_t v[512];
};

constexpr uint64_t kIq3sMembers[64] = {
    0x92050aa5082357a7ull, 0x0422001022892317ull, 0x09000aa4112249a3ull, 0x228005104a052208ull,
    0x0100020904128801ull, 0x084000a208450014ull, 0x0200040002000a40ull, 0x0000110008450015ull,
    0x040250005205ab17ull, 0x410005020902114bull, 0x040120090411a401ull, 0x0104000211820992ull,
    0x000011440a001428ull, 0x0000020005020902ull, 0x0000005000910000ull, 0x010400022002050aull,
    0x2980052a058a55abull, 0x0000020412248905ull, 0x12008802810a0092ull, 0x004001040a140225ull,
    0x2400000224090082ull, 0x0100080180040210ull, 0x0002200000020085ull, 0x0000010801400220ull,
    0x020802942a04aa04ull, 0x44010001000a102aull, 0x0000010014010401ull, 0x0800208a018a1102ull,
    0x0011040002044208ull, 0x0800401004200502ull, 0x0000000200004000ull, 0x000000002005000aull,
    0x0100010204910411ull, 0x0000220821040a84ull, 0x010480010802210aull, 0x0000000022050a10ull,
    0x0200000180100005ull, 0x00040000000200a0ull, 0x0001000010000800ull, 0x0000020801002100ull,
    0x1040049100041104ull, 0x040000000402042aull, 0x0000080041080201ull, 0x0820021000800184ull,
    0x0000004004010012ull, 0x00000a0000400400ull, 0x0000000400000000ull, 0x0000000000040014ull,
    0x000100000a002a00ull, 0x0010000000810001ull, 0x0104200410000400ull, 0x0000000100021001ull,
    0x0004000800200000ull, 0x0001000010000009ull, 0x0000000100000020ull, 0x0000000000000a00ull,
    0x0004100140050091ull, 0x0000002800100204ull, 0x0000020001024112ull, 0x0000080024000004ull,
    0x0000010000010822ull, 0x0000000400040000ull, 0x0000000002000004ull, 0x0000000000000001ull,
};

constexpr Iq3sGrid make_iq3s_grid() {
  Iq3sGrid g{};
  int n = 0;
  for (int c = 0; c < 4096; ++c) {
    if ((kIq3sMembers[c >> 6] >> (c & 63)) & 1) {
      uint32_t e = 0;
      for (int b = 0; b < 4; ++b) e |= (uint32_t)(2 * ((c >> (3 * b)) & 7) + 1) << (8 * b);
      g.v[n++] = e;
    }
  }
  return g;
}

constexpr Iq3sGrid kIq3sGrid = make_iq3s_grid();
static_assert(kIq3sGrid.v[0] == 0x01010101u && kIq3sGrid.v[511] == 0x0f0f0101u, "iq3s grid");

// kvalues_iq4nl (ggml-common.h:1120), packed 4 per dword for byte permutes
constexpr uint32_t kIq4nl[4] = {0xbfad9881u, 0xf6eaddcfu, 0x26190d01u, 0x71594535u};

// ---------------------------------------------------------------------------------------------
// Device helpers

// unaligned little-endian loads from global memory (gfx950 serves unaligned dword loads; the
// aligned(1/2) types make hipcc emit them instead of byte loads)
typedef uint32_t __attribute__((aligned(2))) u32a2;
typedef uint64_t __attribute__((aligned(2))) u64a2;
typedef uint16_t __attribute__((aligned(1))) u16a1;

__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const u32a2*)p; }
__device__ __forceinline__ uint64_t ld64(const uint8_t* p) { return *(const u64a2*)p; }
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *(const uint16_t*)p; }
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4a4 __attribute__((aligned(4)));
// 16 bytes from a 4-byte aligned address (q8_1 blocks are 36 bytes)
__device__ __forceinline__ u32x4 ld128a4(const uint8_t* p) { return *(const u32x4a4*)p; }

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return __half2float(__ushort_as_half((unsigned short)h));
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Buffer-descriptor loads (raw buffer loads: SGPR descriptor + VGPR lane offset + SGPR offset +
// immediate), so K loops spend no vector instructions on addresses; a load past `bytes` returns
// zero. gfx9 descriptor word 3.
constexpr int kBufDword3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufDword3);
}

// fp32 -> storage dtype with round-to-nearest-even (as torch's casts)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float load_x(const void* p, int64_t i, int dtype) {
  if (dtype == kF32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  if (dtype == kF16) return half_bits_to_float(h);
  return __uint_as_float((uint32_t)h << 16);
}

__device__ __forceinline__ void store_y(void* p, int64_t i, float v, int dtype) {
  if (dtype == kF32) {
    ((float*)p)[i] = v;
  } else if (dtype == kF16) {
    ((__half*)p)[i] = __float2half_rn(v);
  } else {
    ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
  }
}

// bytewise negation of the grid bytes whose sign bit is set in the low nibble of s. Grid bytes
// are odd and below 16, so the per-byte two's complement (~g + 1) never carries across bytes.
__device__ __forceinline__ int apply_signs(uint32_t g, uint32_t s) {
  const uint32_t one = ((s & 0xFu) * 0x00204081u) & 0x01010101u;  // bit i -> byte i
  const uint32_t mask = (one << 8) - one;                            // 0xFF in flagged bytes
  return (int)((g ^ mask) + one);
}

// IQ4_NL codebook values of the 4 nibbles q >> sh (sh = 0: the low nibble of each byte, 4: the
// high one), one per byte: two byte permutes over entries 0-7 and 8-15, then the per-byte choice
// on the nibble's bit 3, as a third permute: with that bit moved to bit 7 of its byte (t), the
// selectors 8-11 of v_perm_b32 replicate the sign bits of bytes 1, 3 of t and of t << 8.
__device__ __forceinline__ int iq4nl(uint32_t q, int sh) {
  const uint32_t i = (q >> sh) & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(kIq4nl[1], kIq4nl[0], i);
  const uint32_t hi = __builtin_amdgcn_perm(kIq4nl[3], kIq4nl[2], i);
  const uint32_t t = q << (4 - sh);
  const uint32_t sel = __builtin_amdgcn_perm(t << 8, t, 0x090B080Au);  // 0xFF where bit 3 is set
  return (int)((hi & sel) | (lo & ~sel));
}

}  // namespace gguf
