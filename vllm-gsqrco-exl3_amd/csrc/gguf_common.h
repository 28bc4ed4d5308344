// GGUF block formats, codebooks and small device helpers shared by the gfx950 kernels.
//
// Block layouts follow the reference's ggml-common.h (plugin/vllm_gguf_plugin/csrc/lcpp/ggml/
// src/ggml-common.h): block_q8_1 :259-268, block_q2_K :296-309, block_q4_K :327-338,
// block_q6_K :362-368, block_iq2_xxs :381-385, block_iq2_xs :388-393, block_iq2_s :396-402,
// block_iq3_xxs :407-411, block_iq3_s :415-422, block_iq1_m :433-444, block_iq4_xs :454-460.
// They are a storage format, so the byte offsets below are the format's, written as offsets
// rather than structs (the kernels read blocks that are only 2-byte aligned, with explicit
// unaligned loads).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

namespace gguf {

// ggml type ids (gguf GGMLQuantizationType)
constexpr int kQ2_K = 10;
constexpr int kQ4_K = 12;
constexpr int kQ6_K = 14;
constexpr int kIQ2_XXS = 16;
constexpr int kIQ2_XS = 17;
constexpr int kIQ3_XXS = 18;
constexpr int kIQ3_S = 21;
constexpr int kIQ2_S = 22;
constexpr int kIQ4_XS = 23;
constexpr int kIQ1_M = 29;

constexpr int kQK = 256;   // values per super-block
constexpr int kQ81 = 32;   // values per q8_1 block ("slice")

// dtype codes at the C-ABI (include/gguf_mi355x.h)
constexpr int kF32 = 0, kF16 = 1, kBF16 = 2, kU8 = 3;

__host__ __device__ constexpr int block_bytes(int type) {
  return type == kQ4_K     ? 144
         : type == kQ6_K   ? 210
         : type == kIQ3_S  ? 110
         : type == kIQ4_XS ? 136
         : type == kQ2_K   ? 84
         : type == kIQ2_XXS ? 66
         : type == kIQ2_XS ? 74
         : type == kIQ2_S  ? 82
         : type == kIQ3_XXS ? 98
         : type == kIQ1_M  ? 56
                           : 0;
}

// types served on GGUF rows by the generic decode GEMV and per-slice MFMA GEMM only
__host__ __device__ constexpr bool generic_type(int type) {
  return type == kQ2_K || type == kIQ2_XXS || type == kIQ2_XS || type == kIQ2_S || type == kIQ3_XXS || type == kIQ1_M;
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

// The IQ2 / IQ3_XXS / IQ1 codebooks of ggml-common.h (iq2xxs_grid, iq2xs_grid, iq2s_grid,
// iq3xxs_grid, iq1s_grid) are ascending lists of points of a small lattice: 8 bytes from
// {8, 25, 43}; 4 bytes from {4, 12, 20, 28, 36, 44, 52, 62}; 8 bytes from {-1, 0, 1} (ascending as
// signed bytes). Each is stored here as a membership set over the lattice codes
// c = sum_b digit(byte_b) * base^b and expanded at compile time, like the IQ3_S grid.
constexpr uint64_t kIq2xxsMembers[103] = {
    0x4141441055141555ull, 0x0000100044140400ull, 0x0040001400400400ull, 0x1050000004000000ull,
    0x4004140100114140ull, 0x0500001000400450ull, 0x0001000050000010ull, 0x4004144100004000ull,
    0x0400000400001414ull, 0x0000000000040000ull, 0x0000000000100400ull, 0x0010100414000000ull,
    0x1001040011040040ull, 0x0000000100404000ull, 0x0000000004010000ull, 0x0000400440041000ull,
    0x0000100000000004ull, 0x1000400000001000ull, 0x0000000000000000ull, 0x0040000004000105ull,
    0x0000000000110000ull, 0x0000000001000000ull, 0x0414000000000040ull, 0x0000050100010000ull,
    0x0000001010000000ull, 0x0000000000500000ull, 0x0000414000000000ull, 0x0040000000004001ull,
    0x0000004000040000ull, 0x0000000000000000ull, 0x0000040040000040ull, 0x0000000004000000ull,
    0x0000000000000000ull, 0x0000000001000000ull, 0x0110104144105000ull, 0x0000400010000414ull,
    0x0040400000440400ull, 0x4000000100404000ull, 0x0010000000010010ull, 0x0000001004000010ull,
    0x0000000100000000ull, 0x0414000000000000ull, 0x0000000000011000ull, 0x0401100000000004ull,
    0x0004000000000000ull, 0x0050441000040000ull, 0x0100000104000000ull, 0x0000000000040000ull,
    0x0000000000000001ull, 0x0000000000000040ull, 0x0001000001400000ull, 0x0400000000000000ull,
    0x0000000100000000ull, 0x0400000004100400ull, 0x0040000000000000ull, 0x0004000000000000ull,
    0x0000000000000000ull, 0x0001000001000041ull, 0x0040000000004000ull, 0x0000400000000000ull,
    0x0011000000001000ull, 0x0000000000000000ull, 0x0400000000001400ull, 0x0000000000000000ull,
    0x0000000000000000ull, 0x0000000000000001ull, 0x0000000000000000ull, 0x0000000000000000ull,
    0x0004000041400000ull, 0x0040040000004000ull, 0x0000000000000004ull, 0x0000000000000004ull,
    0x0040001000441400ull, 0x0400000004000000ull, 0x0004000010000000ull, 0x4000000001000040ull,
    0x0000000000000000ull, 0x0000000000010000ull, 0x0000010000000000ull, 0x0104000000000000ull,
    0x0100000000000410ull, 0x0040000000004000ull, 0x0001000000000000ull, 0x0040000400000000ull,
    0x0000000000000001ull, 0x0000000001000000ull, 0x0000000000000000ull, 0x0000000000000000ull,
    0x0100000000001000ull, 0x0000000000000000ull, 0x0000000000000000ull, 0x0000100000000400ull,
    0x0000000100000004ull, 0x0000040000000000ull, 0x0000000000000000ull, 0x0000000000000400ull,
    0x0000000000000000ull, 0x0000000000000000ull, 0x0000000000000000ull, 0x0000000000040000ull,
    0x0000000000000004ull, 0x0000000000000000ull, 0x0000000000000000ull,
};
constexpr uint64_t kIq2xsMembers[103] = {
    0x1541455551555555ull, 0x4145505555540145ull, 0x4010515400010510ull, 0x5550000101000441ull,
    0x0004140115154145ull, 0x0404010500414550ull, 0x0005100041400000ull, 0x1105554000004000ull,
    0x0540400010010414ull, 0x0010400000040001ull, 0x0000000104000100ull, 0x4550515554011000ull,
    0x1051540001054041ull, 0x5000500100004140ull, 0x0000010000400011ull, 0x1001450041455000ull,
    0x0100004140000004ull, 0x0400400000000000ull, 0x0000000000010000ull, 0x0400004004000505ull,
    0x0000000000110000ull, 0x0000000000000004ull, 0x5555000000000040ull, 0x0400010000414010ull,
    0x0010001040001050ull, 0x0000010000100000ull, 0x4000414400000400ull, 0x0040000000000001ull,
    0x1000000010040000ull, 0x0000000001000100ull, 0x0000040141100000ull, 0x0000000400100001ull,
    0x0000010010000000ull, 0x0144000000001001ull, 0x1105554145555000ull, 0x0500414550000414ull,
    0x0141404000440001ull, 0x4000000000000140ull, 0x0010000414014515ull, 0x0000041001050001ull,
    0x4000010100400000ull, 0x0414000000000010ull, 0x0000000101011000ull, 0x0040004100001004ull,
    0x0000000000400000ull, 0x1041455000000000ull, 0x4140000004000105ull, 0x0000000000050004ull,
    0x0000001000000040ull, 0x0004040105400000ull, 0x0000410100004010ull, 0x0000001040000000ull,
    0x0000100000001000ull, 0x0000404000400404ull, 0x0140100000010000ull, 0x0000000000000000ull,
    0x4000004000000000ull, 0x0100101001000041ull, 0x0000000000005000ull, 0x0010000000000000ull,
    0x4001000100000004ull, 0x0000000000000000ull, 0x0000000110000400ull, 0x0000000000001000ull,
    0x0000001000000000ull, 0x0000000001000000ull, 0x0000000000000400ull, 0x0010100000000400ull,
    0x0415010515400000ull, 0x0001155000005000ull, 0x0100000000041004ull, 0x0001400000000400ull,
    0x0040001000541441ull, 0x0100000004000040ull, 0x0400004000000000ull, 0x1000000100000000ull,
    0x0014010000040004ull, 0x0000000000040400ull, 0x0004000000000000ull, 0x0105100404100000ull,
    0x0000010001000400ull, 0x0001000000100001ull, 0x0400000000000000ull, 0x0000004400004000ull,
    0x0000000000001041ull, 0x0014000000001000ull, 0x0000000100000000ull, 0x0400000000000000ull,
    0x0000000400000000ull, 0x0000000000000100ull, 0x0000001000000010ull, 0x0000000404014500ull,
    0x4000000000010000ull, 0x0001144000000010ull, 0x0004000100000010ull, 0x4000000000400000ull,
    0x0000000000000000ull, 0x0000000000000000ull, 0x0040000400004000ull, 0x1040000000000045ull,
    0x0500000000000004ull, 0x0000050000000000ull, 0x0000000100010000ull,
};
constexpr uint64_t kIq2sMembers[103] = {
    0x1555455551555555ull, 0x5545505155551105ull, 0x5010515414150514ull, 0x5550101111000455ull,
    0x5145541555555545ull, 0x5414555514555550ull, 0x1451000455401051ull, 0x1155154000105004ull,
    0x0540010110515555ull, 0x0040401051440455ull, 0x0000100510140100ull, 0x4551515554004000ull,
    0x5555541451151555ull, 0x5000145505155545ull, 0x0414000504414114ull, 0x1455551455455000ull,
    0x5505155540105154ull, 0x0514400010500414ull, 0x4000001000041401ull, 0x0140105154045155ull,
    0x0010500414550000ull, 0x1000041004000010ull, 0x5154000000000400ull, 0x0011010405415115ull,
    0x1401050540415054ull, 0x0104510010100004ull, 0x0514554400050000ull, 0x1440001050041455ull,
    0x0000110004140105ull, 0x0004000400010500ull, 0x1050001411000000ull, 0x0004150000400000ull,
    0x0000100000000000ull, 0x0140040000004004ull, 0x1555554555555000ull, 0x5505554550514414ull,
    0x1541401051541455ull, 0x4000005004145104ull, 0x4550515554555555ull, 0x1051541455550041ull,
    0x5004145500004150ull, 0x5514100000400010ull, 0x0001040041455051ull, 0x0100004140105154ull,
    0x0000400010500040ull, 0x1555455000000000ull, 0x5540005154145555ull, 0x0010500414550515ull,
    0x1400041401051440ull, 0x5154145555000000ull, 0x0414550000414010ull, 0x1400000040001050ull,
    0x0000000000110004ull, 0x0040414010515400ull, 0x0040001050000001ull, 0x1000100000000000ull,
    0x4400004000000000ull, 0x1040041451051545ull, 0x0004140105154000ull, 0x0400010400100010ull,
    0x1451010000000100ull, 0x0000004000105004ull, 0x0010001010000414ull, 0x0000000000040004ull,
    0x0000105000100000ull, 0x0010010000100000ull, 0x0000000000004000ull, 0x0000000400000000ull,
    0x5414114515404000ull, 0x1455450001411011ull, 0x1140004140005154ull, 0x0000000010500015ull,
    0x0041455011555400ull, 0x4140105154000105ull, 0x0010500001010000ull, 0x1000000000000050ull,
    0x0000000105000141ull, 0x4000010000014040ull, 0x0004000000000000ull, 0x5545010000400500ull,
    0x0000414010515410ull, 0x0000101050001411ull, 0x0000100004140000ull, 0x4010515440000000ull,
    0x1050004001000041ull, 0x1100000000004000ull, 0x0010001000000010ull, 0x0001100041400000ull,
    0x0000005000000000ull, 0x0000000000001100ull, 0x0040000000000000ull, 0x0000105410111100ull,
    0x0010000001040000ull, 0x4004100000000400ull, 0x5100014400000014ull, 0x0100000000400010ull,
    0x0000000010001040ull, 0x0000000000000000ull, 0x0040000000000004ull, 0x0100000000000040ull,
    0x0400004000000000ull, 0x0000011401400000ull, 0x0000000100001000ull,
};
constexpr uint64_t kIq3xxsMembers[64] = {
    0x2800000402058a15ull, 0x010010020522050aull, 0x200082008a050215ull, 0x0100000000200582ull,
    0x2800801080000800ull, 0x0000040004000082ull, 0x0010000020000000ull, 0x0002000800005100ull,
    0x00000180150a050aull, 0x0000000000050205ull, 0x040000000102050aull, 0x0040004002010005ull,
    0x0000010000000022ull, 0x0200004000110000ull, 0x0000000000000020ull, 0x0000000100040000ull,
    0x0000000402450a05ull, 0x018800000102052aull, 0x0000200180058205ull, 0x1100000000001102ull,
    0x0000080020000000ull, 0x1000000200800008ull, 0x0000000000000000ull, 0x000000200000400aull,
    0x04200100000a0502ull, 0x0000005002010005ull, 0x040004000020010aull, 0x0000000008000200ull,
    0x0400008001000000ull, 0x0000200000040041ull, 0x0008000040001000ull, 0x0001000008000000ull,
    0x00008800a0008010ull, 0x1000000000000000ull, 0x0041000180010000ull, 0x0000002000000080ull,
    0x0010020000000010ull, 0x0100000800200000ull, 0x0000000000000000ull, 0x0000000001000520ull,
    0x0100000200000400ull, 0x0000200000400041ull, 0x0400000004001000ull, 0x0000080000000004ull,
    0x0400000000880100ull, 0x0000000002000004ull, 0x0000010000000000ull, 0x0000000400100000ull,
    0x0010005000100000ull, 0x0002000000020000ull, 0x0010000000008000ull, 0x0000000041000000ull,
    0x0000001000000000ull, 0x0000040000000020ull, 0x0000000008000000ull, 0x0000000000020008ull,
    0x00000400040001a8ull, 0x0000000100400000ull, 0x0000042000000400ull, 0x0001000008002001ull,
    0x0000000200020000ull, 0x0000000000100005ull, 0x0000000001000000ull, 0x0000000000000000ull,
};
constexpr uint64_t kIq1sMembers[103] = {
    0x514202a085142555ull, 0xa28a2086a8314508ull, 0x14508514202a081aull, 0xa005152545442082ull,
    0x8208001888208202ull, 0x0aaabb88a02a03a0ull, 0xaa0a0022000baa90ull, 0x4508514008a0828cull,
    0x0851421450808821ull, 0x2a8008a09808308aull, 0x4248208514214508ull, 0x20a0c22c01450855ull,
    0xa2aaa8242a00268aull, 0x0028280808afe208ull, 0xa82028aa284202a0ull, 0xa8bab9089b0a2080ull,
    0x3aaaaea289aeca20ull, 0xb80e82bbbaeaeb7cull, 0x2202920ed3caba22ull, 0x820aba8aa8202200ull,
    0x3ba2e04a2a000802ull, 0x81408100a22b2022ull, 0x8514012208288aaaull, 0x5421450920821550ull,
    0x203aa8230208a085ull, 0xa208514254208284ull, 0x082a021450950820ull, 0x200248a08082a8b8ull,
    0xab2802a268a28208ull, 0x083082082085082aull, 0xa085142145004045ull, 0x8229014500514200ull,
    0x1430a1082a828a00ull, 0x2145082882145005ull, 0x2aaa200202208514ull, 0xa828ae8ab1122000ull,
    0x0a820070a8aaa1baull, 0x8200840222280208ull, 0xaa2ab0eaa0804800ull, 0xa7daea22ba8b20c2ull,
    0xaa2ab092a86e8b8bull, 0x48202a0c448a8b72ull, 0x20aa082a8a284084ull, 0xa09aafa222a2ccc8ull,
    0xa82a00020002a8e8ull, 0xa2a28ba080200088ull, 0xba0a328280a0ba28ull, 0x2ba0a2ebfebab8beull,
    0x00a2ea280a8a08a2ull, 0xdeeaa4fa0c0232a1ull, 0xeb7ebe8d2ea82befull, 0xdeba7de6bf7ff7faull,
    0x12fa26bfff27fb69ull, 0x0ebeaa10228ae1e9ull, 0xae820ba8b208aa84ull, 0x62048083e924baffull,
    0x002ba40aa8f2682cull, 0x0012aae208082a02ull, 0x82c920a60a2a8202ull, 0x8c00a20028829089ull,
    0x6c00080882001380ull, 0x8abea602bbaaaa8aull, 0xd02e976b8002caa0ull, 0xdeaa2e108210e9b2ull,
    0x820a0004a5d11528ull, 0x20a1010820828a00ull, 0xa0843222ba39aa82ull, 0x0262a28a00188009ull,
    0xac21450051441481ull, 0x20aa085142145082ull, 0x45082a120a87aa28ull, 0x08514208a0051421ull,
    0x22a240a002200145ull, 0x8a6a08a208008800ull, 0x0a200080aaaab86eull, 0x5044082122c8e282ull,
    0x8515208a09514214ull, 0x2a2aaa080a861450ull, 0x21450851420a0080ull, 0xe2085142145000a8ull,
    0x082a82180a828820ull, 0x0a028bb08aaaa2aaull, 0x0aaa80822820aa2aull, 0x220288a900280828ull,
    0xba8a08b8280bbea0ull, 0xaef8a4baffaeb24bull, 0x30a0b668285220aaull, 0x6a220828020a80e6ull,
    0x2baaaa020a208062ull, 0x0808a2a0a9a2eaaaull, 0x0e8200228aa02010ull, 0x400aa08514214500ull,
    0x4a0006a921450851ull, 0x440d1000a50802aaull, 0x0514214508288214ull, 0x0020f2ac82820800ull,
    0x20ba0a280aaa0000ull, 0x280948820002a2eaull, 0x0051454b110014e9ull, 0x5142145002a80145ull,
    0x400a288808248808ull, 0x02a0051401450008ull, 0x0000000145085140ull,
};

template <int N>
struct Lattice64 {
  uint64_t v[N];
};
template <int N>
struct Lattice32 {
  uint32_t v[N];
};

// N points of {levels}^8 (base 3) named by a membership bitmap, bytes little-endian in a uint64
template <int N>
constexpr Lattice64<N> make_lattice8(const uint64_t* members, int l0, int l1, int l2) {
  Lattice64<N> g{};
  const int lv[3] = {l0, l1, l2};
  int n = 0;
  for (int c = 0; c < 6561 && n < N; ++c) {
    if ((members[c >> 6] >> (c & 63)) & 1) {
      uint64_t e = 0;
      int r = c;
      for (int b = 0; b < 8; ++b, r /= 3) e |= (uint64_t)(lv[r % 3] & 0xFF) << (8 * b);
      g.v[n++] = e;
    }
  }
  return g;
}

constexpr Lattice32<256> make_iq3xxs_grid() {
  Lattice32<256> g{};
  const int lv[8] = {4, 12, 20, 28, 36, 44, 52, 62};
  int n = 0;
  for (int c = 0; c < 4096 && n < 256; ++c) {
    if ((kIq3xxsMembers[c >> 6] >> (c & 63)) & 1) {
      uint32_t e = 0;
      for (int b = 0; b < 4; ++b) e |= (uint32_t)lv[(c >> (3 * b)) & 7] << (8 * b);
      g.v[n++] = e;
    }
  }
  return g;
}

constexpr Lattice64<256> kIq2xxsGrid = make_lattice8<256>(kIq2xxsMembers, 8, 25, 43);
constexpr Lattice64<512> kIq2xsGrid = make_lattice8<512>(kIq2xsMembers, 8, 25, 43);
constexpr Lattice64<1024> kIq2sGrid = make_lattice8<1024>(kIq2sMembers, 8, 25, 43);
constexpr Lattice32<256> kIq3xxsGrid = make_iq3xxs_grid();
static_assert(kIq2xxsGrid.v[0] == 0x0808080808080808ull && kIq2sGrid.v[1023] != 0, "iq2 grids");
static_assert(kIq3xxsGrid.v[0] == 0x04040404u, "iq3xxs grid");

// iq3xxs_grid with the signs applied: entry g | n << 8 is grid word g with the bytes flagged in
// the 4-bit sign nibble n negated (16 KB), so one lookup yields four signed int8 weights
constexpr Lattice32<4096> make_iq3xxs_signed() {
  Lattice32<4096> t{};
  for (int n = 0; n < 16; ++n)
    for (int g = 0; g < 256; ++g) {
      uint32_t e = 0;
      for (int b = 0; b < 4; ++b) {
        const uint32_t v = (kIq3xxsGrid.v[g] >> (8 * b)) & 0xFF;
        e |= (((n >> b) & 1) ? ((0x100u - v) & 0xFF) : v) << (8 * b);
      }
      t.v[g | (n << 8)] = e;
    }
  return t;
}
constexpr Lattice32<4096> kIq3xxsSigned = make_iq3xxs_signed();
static_assert(kIq3xxsSigned.v[0x100] == 0x040404fcu, "iq3xxs signed grid");

// iq1s_grid (values -1, 0, 1; base-3 digit = value + 1) in nibble form: byte j of entry e holds
// the digit of value j in its low nibble and that of value j + 4 in its high nibble, so one
// 32-bit word carries the 8 values and a byte permute maps the digits to weights.
constexpr Lattice32<2048> make_iq1_nibbles() {
  Lattice32<2048> g{};
  int n = 0;
  for (int c = 0; c < 6561 && n < 2048; ++c) {
    if ((kIq1sMembers[c >> 6] >> (c & 63)) & 1) {
      int dg[8] = {};
      for (int b = 0, r = c; b < 8; ++b, r /= 3) dg[b] = r % 3;
      uint32_t e = 0;
      for (int j = 0; j < 4; ++j) e |= (uint32_t)(dg[j] | (dg[j + 4] << 4)) << (8 * j);
      g.v[n++] = e;
    }
  }
  return g;
}
constexpr Lattice32<2048> kIq1sNib = make_iq1_nibbles();
static_assert(kIq1sNib.v[0] == 0u && kIq1sNib.v[2047] != 0u, "iq1s grid");

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

// Cache policy of the IQ3_S decode GEMVs' weight loads (the aux operand of a raw buffer load on
// gfx950: bit 0 sc0, bit 1 nt). Each weight byte is read once per launch by one lane, so the loads
// are marked non-temporal; on the 17408 x 5120 and 5120 x 17408 stream GEMV this took 4-5 % off
// each launch at 1 and 4 activation rows (sc0 alone changed nothing). The row-chunk GEMV of the
// GGUF-row types keeps the default policy: its lanes read the header bytes of a block from lines
// that other loads of the same block also touch, and nt made it slower (Q4_K 17408 x 5120 M = 1
// 12.6 -> 14.1 us, Q6_K 5120 x 17408 23.6 -> 28.6 us).
constexpr int kWeightCpol = 3;

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

// bytewise negation of the grid bytes whose sign bit is set in the low nibble of s. No grid byte
// of the IQ2 / IQ3 codebooks is zero, so the per-byte two's complement (~g + 1) never carries
// across bytes.
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

// Per-device one-time set-up (device queries, kernel attributes) runs lazily, on a product's first
// call on a device, and that call may be made inside a caller's stream capture (a CUDA-graph
// capture in torch). The set-up is run with this thread's capture mode exchanged for relaxed, so
// that no capture in global mode (torch's default) rejects it, and is restored afterwards. The
// reference makes the same first-call-in-capture promise (lcpp_owned_iq3_mma.cu:333-346,
// lcpp_owned_mma_k.cu:551-569).
template <class F>
inline void outside_capture(F&& fn) {
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
  fn();
  if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
}

constexpr int kMaxDevices = 64;

// fn() once per device (device index dev < kMaxDevices), thread-safe: concurrent first calls from
// several host threads run it once and the others wait for it.
template <class Tag, class F>
inline void once_per_device(int dev, F&& fn) {
  static std::once_flag flags[kMaxDevices];
  if (dev < 0 || dev >= kMaxDevices) return;
  std::call_once(flags[dev], [&] { outside_capture(fn); });
}

// compute units of the current device (256 on MI355X; 256 when the query fails), cached per device
inline int device_cus() {
  static std::atomic<int> cus[kMaxDevices];  // zero-initialised (static storage)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    outside_capture([&] {
      if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    });
    cus[dev].store(n, std::memory_order_relaxed);  // every thread that races here stores the same value
  }
  return n;
}

}  // namespace gguf
