"""CPU oracle for the GGUF quantized-matmul path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker (or, in bench.py, as the timed CPU baseline). The
product path (vllm-gsqrco-exl3_amd/) never imports it and has no CPU fallback.

A numpy restatement of the reference's arithmetic, each function citing the reference
file:line it follows (paths relative to the reference repository root):

  formats     plugin/vllm_gguf_plugin/csrc/lcpp/ggml/src/ggml-common.h:259-268 (block_q8_1),
              :296-309 (block_q2_K), :327-338 (block_q4_K), :362-368 (block_q6_K),
              :381-385 (block_iq2_xxs), :388-393 (block_iq2_xs), :396-402 (block_iq2_s),
              :407-411 (block_iq3_xxs), :415-422 (block_iq3_s), :433-444 (block_iq1_m),
              :454-460 (block_iq4_xs); codebooks iq3s_grid :1052, kvalues_iq4nl :1120, and
              iq2xxs_grid, iq2xs_grid, iq2s_grid, iq3xxs_grid, iq1s_grid, ksigns_iq2xs
  dequant     gguf-py b11211 gguf.quants.<T>.dequantize_blocks (a third-party dependency of
              the reference, absent here; called from tests/gpu/_refs.py:33-37 and pinned by
              the golden rows tests/fixtures/dequant/*.npz); the same formulas as
              plugin/vllm_gguf_plugin/csrc/gguf/dequantize.cuh:102-120 (Q2_K), :156-197,233-256,
              :259-329 (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS), :335-353, :377-398 (IQ1_M), :421-434
  q8_1        plugin/vllm_gguf_plugin/csrc/lcpp_shim.cu:274-294 (MMVQ layout) and :298-355
              (MMQ layout, block_q8_1_mmq of ggml-cuda/mmq.cuh:27-56, ds layout :60-100);
              warp reductions ggml-cuda/common.cuh:468-474,528-534
  slice dots  ggml-cuda/vecdotq.cuh:365-393 (Q2_K MMVQ), :396-445 (Q2_K MMQ), :508-530 (Q4_K
              MMVQ), :627-648 (Q6_K MMVQ), :1211-1248 (IQ3_S), :1357-1380 (IQ4_XS) and the IQ2 /
              IQ3_XXS / IQ1_M vec_dot functions of the same file
  q81 model   tests/gpu/_refs.py:40-54,78-91 (y = dequant(q8_1(x)) @ dequant(W).T, float64)

How each part is pinned (tests/test_oracle.py):
  dequant     bit-exact against the reference's golden rows (tests/golden/dequant, fp32 gguf-py
              output on real GGUF rows) for all ten types.
  tables      every codebook against the reference header itself when oracle/_ref is built
              (the recipe in oracle/Makefile compiles ggml-common.h's tables), else against the
              golden rows (the entries they reach) and the codebooks' invariants.
  q8_1        closed form: d = amax/127 exactly as IEEE fp32 division, roundf ties away from
              zero, |q| <= 127, all-zero block -> (0, 0, 0), the xor-butterfly sum order
              checked against brute-force float32 trees, dequant(q8_1(x)) within d/2 of x.
  slice dots  brute force: int64 sum of decoded int8 weight x q8 per slice, and the identity
              d_w*scale*sumi*d8 == sum(dequant(w) * q*d8) up to fp32 rounding.
The reference's q8_1 bytes have no golden vectors in the reference repository (its checks
are GPU-vs-GPU), so the q8_1 bytes are pinned by the closed form only.
"""

from __future__ import annotations

import numpy as np

QK_K = 256
QK8_1 = 32

# ggml type ids (gguf-py GGMLQuantizationType, restated from tests/cpu/test_lcpp_guards.py:22 and
# the golden rows' ggml_type)
Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 10, 12, 14, 16, 17, 18, 21, 22, 23, 29
TYPE_NAMES = {Q2_K: "Q2_K", Q4_K: "Q4_K", Q6_K: "Q6_K", IQ2_XXS: "IQ2_XXS", IQ2_XS: "IQ2_XS", IQ3_XXS: "IQ3_XXS",
              IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ4_XS: "IQ4_XS", IQ1_M: "IQ1_M"}
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}
# bytes per 256-value block (ggml-common.h static_asserts)
BLOCK_BYTES = {Q2_K: 84, Q4_K: 144, Q6_K: 210, IQ2_XXS: 66, IQ2_XS: 74, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82,
               IQ4_XS: 136, IQ1_M: 56}

# --------------------------------------------------------------------------- tables
# iq3s_grid (ggml-common.h:1052) is the ascending list of the 512 points of {1,3,..,15}^4
# that IQ3_S uses. Encoded here as a 4096-bit membership set over codes
# c = sum_i ((byte_i - 1) / 2) << 3i; enumerating members in ascending c gives the table in
# its ascending uint32 order (byte 3 is the most significant in both).
_IQ3S_MEMBERS = (
    0x92050aa5082357a7, 0x0422001022892317, 0x09000aa4112249a3, 0x228005104a052208,
    0x0100020904128801, 0x084000a208450014, 0x0200040002000a40, 0x0000110008450015,
    0x040250005205ab17, 0x410005020902114b, 0x040120090411a401, 0x0104000211820992,
    0x000011440a001428, 0x0000020005020902, 0x0000005000910000, 0x010400022002050a,
    0x2980052a058a55ab, 0x0000020412248905, 0x12008802810a0092, 0x004001040a140225,
    0x2400000224090082, 0x0100080180040210, 0x0002200000020085, 0x0000010801400220,
    0x020802942a04aa04, 0x44010001000a102a, 0x0000010014010401, 0x0800208a018a1102,
    0x0011040002044208, 0x0800401004200502, 0x0000000200004000, 0x000000002005000a,
    0x0100010204910411, 0x0000220821040a84, 0x010480010802210a, 0x0000000022050a10,
    0x0200000180100005, 0x00040000000200a0, 0x0001000010000800, 0x0000020801002100,
    0x1040049100041104, 0x040000000402042a, 0x0000080041080201, 0x0820021000800184,
    0x0000004004010012, 0x00000a0000400400, 0x0000000400000000, 0x0000000000040014,
    0x000100000a002a00, 0x0010000000810001, 0x0104200410000400, 0x0000000100021001,
    0x0004000800200000, 0x0001000010000009, 0x0000000100000020, 0x0000000000000a00,
    0x0004100140050091, 0x0000002800100204, 0x0000020001024112, 0x0000080024000004,
    0x0000010000010822, 0x0000000400040000, 0x0000000002000004, 0x0000000000000001,
)


def _iq3s_grid() -> np.ndarray:
    codes = [w * 64 + j for w, bits in enumerate(_IQ3S_MEMBERS) for j in range(64) if bits >> j & 1]
    out = np.zeros((len(codes), 4), dtype=np.uint8)
    for i, c in enumerate(codes):
        for b in range(4):
            out[i, b] = 2 * ((c >> (3 * b)) & 7) + 1
    return out


IQ3S_GRID = _iq3s_grid()                     # [512, 4] uint8, byte b of entry i
IQ3S_GRID_U32 = IQ3S_GRID.astype(np.uint32) @ (1 << (8 * np.arange(4, dtype=np.uint32)))
# The IQ2 / IQ3_XXS / IQ1 codebooks of ggml-common.h are ascending lists of points of a small
# lattice: 8 bytes from {8, 25, 43} (iq2xxs_grid, iq2xs_grid, iq2s_grid), 4 bytes from
# {4, 12, 20, 28, 36, 44, 52, 62} (iq3xxs_grid), 8 bytes from {-1, 0, 1} (iq1s_grid, ascending as
# signed bytes). Each is stored as a membership set over the lattice codes
# c = sum_b digit(byte_b) * base**b (byte 7, or 3, most significant); enumerating members in
# ascending c gives the table in its own order.
_IQ2XXS_MEMBERS = (
    0x4141441055141555, 0x0000100044140400, 0x0040001400400400, 0x1050000004000000,
    0x4004140100114140, 0x0500001000400450, 0x0001000050000010, 0x4004144100004000,
    0x0400000400001414, 0x0000000000040000, 0x0000000000100400, 0x0010100414000000,
    0x1001040011040040, 0x0000000100404000, 0x0000000004010000, 0x0000400440041000,
    0x0000100000000004, 0x1000400000001000, 0x0000000000000000, 0x0040000004000105,
    0x0000000000110000, 0x0000000001000000, 0x0414000000000040, 0x0000050100010000,
    0x0000001010000000, 0x0000000000500000, 0x0000414000000000, 0x0040000000004001,
    0x0000004000040000, 0x0000000000000000, 0x0000040040000040, 0x0000000004000000,
    0x0000000000000000, 0x0000000001000000, 0x0110104144105000, 0x0000400010000414,
    0x0040400000440400, 0x4000000100404000, 0x0010000000010010, 0x0000001004000010,
    0x0000000100000000, 0x0414000000000000, 0x0000000000011000, 0x0401100000000004,
    0x0004000000000000, 0x0050441000040000, 0x0100000104000000, 0x0000000000040000,
    0x0000000000000001, 0x0000000000000040, 0x0001000001400000, 0x0400000000000000,
    0x0000000100000000, 0x0400000004100400, 0x0040000000000000, 0x0004000000000000,
    0x0000000000000000, 0x0001000001000041, 0x0040000000004000, 0x0000400000000000,
    0x0011000000001000, 0x0000000000000000, 0x0400000000001400, 0x0000000000000000,
    0x0000000000000000, 0x0000000000000001, 0x0000000000000000, 0x0000000000000000,
    0x0004000041400000, 0x0040040000004000, 0x0000000000000004, 0x0000000000000004,
    0x0040001000441400, 0x0400000004000000, 0x0004000010000000, 0x4000000001000040,
    0x0000000000000000, 0x0000000000010000, 0x0000010000000000, 0x0104000000000000,
    0x0100000000000410, 0x0040000000004000, 0x0001000000000000, 0x0040000400000000,
    0x0000000000000001, 0x0000000001000000, 0x0000000000000000, 0x0000000000000000,
    0x0100000000001000, 0x0000000000000000, 0x0000000000000000, 0x0000100000000400,
    0x0000000100000004, 0x0000040000000000, 0x0000000000000000, 0x0000000000000400,
    0x0000000000000000, 0x0000000000000000, 0x0000000000000000, 0x0000000000040000,
    0x0000000000000004, 0x0000000000000000, 0x0000000000000000,
)
_IQ2XS_MEMBERS = (
    0x1541455551555555, 0x4145505555540145, 0x4010515400010510, 0x5550000101000441,
    0x0004140115154145, 0x0404010500414550, 0x0005100041400000, 0x1105554000004000,
    0x0540400010010414, 0x0010400000040001, 0x0000000104000100, 0x4550515554011000,
    0x1051540001054041, 0x5000500100004140, 0x0000010000400011, 0x1001450041455000,
    0x0100004140000004, 0x0400400000000000, 0x0000000000010000, 0x0400004004000505,
    0x0000000000110000, 0x0000000000000004, 0x5555000000000040, 0x0400010000414010,
    0x0010001040001050, 0x0000010000100000, 0x4000414400000400, 0x0040000000000001,
    0x1000000010040000, 0x0000000001000100, 0x0000040141100000, 0x0000000400100001,
    0x0000010010000000, 0x0144000000001001, 0x1105554145555000, 0x0500414550000414,
    0x0141404000440001, 0x4000000000000140, 0x0010000414014515, 0x0000041001050001,
    0x4000010100400000, 0x0414000000000010, 0x0000000101011000, 0x0040004100001004,
    0x0000000000400000, 0x1041455000000000, 0x4140000004000105, 0x0000000000050004,
    0x0000001000000040, 0x0004040105400000, 0x0000410100004010, 0x0000001040000000,
    0x0000100000001000, 0x0000404000400404, 0x0140100000010000, 0x0000000000000000,
    0x4000004000000000, 0x0100101001000041, 0x0000000000005000, 0x0010000000000000,
    0x4001000100000004, 0x0000000000000000, 0x0000000110000400, 0x0000000000001000,
    0x0000001000000000, 0x0000000001000000, 0x0000000000000400, 0x0010100000000400,
    0x0415010515400000, 0x0001155000005000, 0x0100000000041004, 0x0001400000000400,
    0x0040001000541441, 0x0100000004000040, 0x0400004000000000, 0x1000000100000000,
    0x0014010000040004, 0x0000000000040400, 0x0004000000000000, 0x0105100404100000,
    0x0000010001000400, 0x0001000000100001, 0x0400000000000000, 0x0000004400004000,
    0x0000000000001041, 0x0014000000001000, 0x0000000100000000, 0x0400000000000000,
    0x0000000400000000, 0x0000000000000100, 0x0000001000000010, 0x0000000404014500,
    0x4000000000010000, 0x0001144000000010, 0x0004000100000010, 0x4000000000400000,
    0x0000000000000000, 0x0000000000000000, 0x0040000400004000, 0x1040000000000045,
    0x0500000000000004, 0x0000050000000000, 0x0000000100010000,
)
_IQ2S_MEMBERS = (
    0x1555455551555555, 0x5545505155551105, 0x5010515414150514, 0x5550101111000455,
    0x5145541555555545, 0x5414555514555550, 0x1451000455401051, 0x1155154000105004,
    0x0540010110515555, 0x0040401051440455, 0x0000100510140100, 0x4551515554004000,
    0x5555541451151555, 0x5000145505155545, 0x0414000504414114, 0x1455551455455000,
    0x5505155540105154, 0x0514400010500414, 0x4000001000041401, 0x0140105154045155,
    0x0010500414550000, 0x1000041004000010, 0x5154000000000400, 0x0011010405415115,
    0x1401050540415054, 0x0104510010100004, 0x0514554400050000, 0x1440001050041455,
    0x0000110004140105, 0x0004000400010500, 0x1050001411000000, 0x0004150000400000,
    0x0000100000000000, 0x0140040000004004, 0x1555554555555000, 0x5505554550514414,
    0x1541401051541455, 0x4000005004145104, 0x4550515554555555, 0x1051541455550041,
    0x5004145500004150, 0x5514100000400010, 0x0001040041455051, 0x0100004140105154,
    0x0000400010500040, 0x1555455000000000, 0x5540005154145555, 0x0010500414550515,
    0x1400041401051440, 0x5154145555000000, 0x0414550000414010, 0x1400000040001050,
    0x0000000000110004, 0x0040414010515400, 0x0040001050000001, 0x1000100000000000,
    0x4400004000000000, 0x1040041451051545, 0x0004140105154000, 0x0400010400100010,
    0x1451010000000100, 0x0000004000105004, 0x0010001010000414, 0x0000000000040004,
    0x0000105000100000, 0x0010010000100000, 0x0000000000004000, 0x0000000400000000,
    0x5414114515404000, 0x1455450001411011, 0x1140004140005154, 0x0000000010500015,
    0x0041455011555400, 0x4140105154000105, 0x0010500001010000, 0x1000000000000050,
    0x0000000105000141, 0x4000010000014040, 0x0004000000000000, 0x5545010000400500,
    0x0000414010515410, 0x0000101050001411, 0x0000100004140000, 0x4010515440000000,
    0x1050004001000041, 0x1100000000004000, 0x0010001000000010, 0x0001100041400000,
    0x0000005000000000, 0x0000000000001100, 0x0040000000000000, 0x0000105410111100,
    0x0010000001040000, 0x4004100000000400, 0x5100014400000014, 0x0100000000400010,
    0x0000000010001040, 0x0000000000000000, 0x0040000000000004, 0x0100000000000040,
    0x0400004000000000, 0x0000011401400000, 0x0000000100001000,
)
_IQ3XXS_MEMBERS = (
    0x2800000402058a15, 0x010010020522050a, 0x200082008a050215, 0x0100000000200582,
    0x2800801080000800, 0x0000040004000082, 0x0010000020000000, 0x0002000800005100,
    0x00000180150a050a, 0x0000000000050205, 0x040000000102050a, 0x0040004002010005,
    0x0000010000000022, 0x0200004000110000, 0x0000000000000020, 0x0000000100040000,
    0x0000000402450a05, 0x018800000102052a, 0x0000200180058205, 0x1100000000001102,
    0x0000080020000000, 0x1000000200800008, 0x0000000000000000, 0x000000200000400a,
    0x04200100000a0502, 0x0000005002010005, 0x040004000020010a, 0x0000000008000200,
    0x0400008001000000, 0x0000200000040041, 0x0008000040001000, 0x0001000008000000,
    0x00008800a0008010, 0x1000000000000000, 0x0041000180010000, 0x0000002000000080,
    0x0010020000000010, 0x0100000800200000, 0x0000000000000000, 0x0000000001000520,
    0x0100000200000400, 0x0000200000400041, 0x0400000004001000, 0x0000080000000004,
    0x0400000000880100, 0x0000000002000004, 0x0000010000000000, 0x0000000400100000,
    0x0010005000100000, 0x0002000000020000, 0x0010000000008000, 0x0000000041000000,
    0x0000001000000000, 0x0000040000000020, 0x0000000008000000, 0x0000000000020008,
    0x00000400040001a8, 0x0000000100400000, 0x0000042000000400, 0x0001000008002001,
    0x0000000200020000, 0x0000000000100005, 0x0000000001000000, 0x0000000000000000,
)
_IQ1S_MEMBERS = (
    0x514202a085142555, 0xa28a2086a8314508, 0x14508514202a081a, 0xa005152545442082,
    0x8208001888208202, 0x0aaabb88a02a03a0, 0xaa0a0022000baa90, 0x4508514008a0828c,
    0x0851421450808821, 0x2a8008a09808308a, 0x4248208514214508, 0x20a0c22c01450855,
    0xa2aaa8242a00268a, 0x0028280808afe208, 0xa82028aa284202a0, 0xa8bab9089b0a2080,
    0x3aaaaea289aeca20, 0xb80e82bbbaeaeb7c, 0x2202920ed3caba22, 0x820aba8aa8202200,
    0x3ba2e04a2a000802, 0x81408100a22b2022, 0x8514012208288aaa, 0x5421450920821550,
    0x203aa8230208a085, 0xa208514254208284, 0x082a021450950820, 0x200248a08082a8b8,
    0xab2802a268a28208, 0x083082082085082a, 0xa085142145004045, 0x8229014500514200,
    0x1430a1082a828a00, 0x2145082882145005, 0x2aaa200202208514, 0xa828ae8ab1122000,
    0x0a820070a8aaa1ba, 0x8200840222280208, 0xaa2ab0eaa0804800, 0xa7daea22ba8b20c2,
    0xaa2ab092a86e8b8b, 0x48202a0c448a8b72, 0x20aa082a8a284084, 0xa09aafa222a2ccc8,
    0xa82a00020002a8e8, 0xa2a28ba080200088, 0xba0a328280a0ba28, 0x2ba0a2ebfebab8be,
    0x00a2ea280a8a08a2, 0xdeeaa4fa0c0232a1, 0xeb7ebe8d2ea82bef, 0xdeba7de6bf7ff7fa,
    0x12fa26bfff27fb69, 0x0ebeaa10228ae1e9, 0xae820ba8b208aa84, 0x62048083e924baff,
    0x002ba40aa8f2682c, 0x0012aae208082a02, 0x82c920a60a2a8202, 0x8c00a20028829089,
    0x6c00080882001380, 0x8abea602bbaaaa8a, 0xd02e976b8002caa0, 0xdeaa2e108210e9b2,
    0x820a0004a5d11528, 0x20a1010820828a00, 0xa0843222ba39aa82, 0x0262a28a00188009,
    0xac21450051441481, 0x20aa085142145082, 0x45082a120a87aa28, 0x08514208a0051421,
    0x22a240a002200145, 0x8a6a08a208008800, 0x0a200080aaaab86e, 0x5044082122c8e282,
    0x8515208a09514214, 0x2a2aaa080a861450, 0x21450851420a0080, 0xe2085142145000a8,
    0x082a82180a828820, 0x0a028bb08aaaa2aa, 0x0aaa80822820aa2a, 0x220288a900280828,
    0xba8a08b8280bbea0, 0xaef8a4baffaeb24b, 0x30a0b668285220aa, 0x6a220828020a80e6,
    0x2baaaa020a208062, 0x0808a2a0a9a2eaaa, 0x0e8200228aa02010, 0x400aa08514214500,
    0x4a0006a921450851, 0x440d1000a50802aa, 0x0514214508288214, 0x0020f2ac82820800,
    0x20ba0a280aaa0000, 0x280948820002a2ea, 0x0051454b110014e9, 0x5142145002a80145,
    0x400a288808248808, 0x02a0051401450008, 0x0000000145085140,
)


def _lattice_grid(members, nbytes, levels) -> np.ndarray:
    """[N, nbytes] int16 table of the lattice points named by a membership bitmap."""
    base = len(levels)
    codes = [w * 64 + j for w, bits in enumerate(members) for j in range(64) if bits >> j & 1]
    out = np.zeros((len(codes), nbytes), dtype=np.int16)
    for i, c in enumerate(codes):
        for b in range(nbytes):
            out[i, b] = levels[c // base ** b % base]
    return out


IQ2XXS_GRID = _lattice_grid(_IQ2XXS_MEMBERS, 8, (8, 25, 43))                    # [256, 8]
IQ2XS_GRID = _lattice_grid(_IQ2XS_MEMBERS, 8, (8, 25, 43))                      # [512, 8]
IQ2S_GRID = _lattice_grid(_IQ2S_MEMBERS, 8, (8, 25, 43))                        # [1024, 8]
IQ3XXS_GRID = _lattice_grid(_IQ3XXS_MEMBERS, 4, (4, 12, 20, 28, 36, 44, 52, 62))  # [256, 4]
IQ1S_GRID = _lattice_grid(_IQ1S_MEMBERS, 8, (-1, 0, 1))                         # [2048, 8]
# ksigns_iq2xs: 7 sign bits and an eighth that makes the byte's parity even
KSIGNS_IQ2XS = np.array([i | ((bin(i).count("1") & 1) << 7) for i in range(128)], dtype=np.uint8)
IQ1M_DELTA = np.float32(0.125)   # IQ1M_DELTA / IQ1S_DELTA of ggml-common.h


def grid_words(grid: np.ndarray) -> np.ndarray:
    """A codebook as the reference header stores it: each entry's bytes little-endian in one
    unsigned integer (uint64 for 8 bytes, uint32 for 4)."""
    g = grid.astype(np.int64) & 0xFF
    return (g << (8 * np.arange(g.shape[1], dtype=np.int64))).sum(1).astype(np.uint64)


# kvalues_iq4nl (ggml-common.h:1120): the IQ4_NL / IQ4_XS non-linear codebook
KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                         dtype=np.int8)


# --------------------------------------------------------------------------- helpers
def _blocks(raw: np.ndarray, qt: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    bs = BLOCK_BYTES[qt]
    assert raw.size % bs == 0, (raw.shape, qt)
    return raw.reshape(-1, bs)


def _f16(b: np.ndarray) -> np.ndarray:
    """[..., 2] uint8 little-endian -> float32 (fp16 widened, exact)."""
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)[..., 0]


def _q4k_scale_min(sc12: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """get_scale_min_k4 (csrc/gguf/dequantize.cuh:156-163) for j = 0..7: 6-bit scale and min."""
    s = sc12.astype(np.int32)
    j = np.arange(8)
    lo = j < 4
    sc = np.where(lo, s[:, np.minimum(j, 3)] & 63,
                  (s[:, np.minimum(j + 4, 11)] & 0xF) | ((s[:, np.maximum(j - 4, 0)] >> 6) << 4))
    mn = np.where(lo, s[:, np.minimum(j + 4, 11)] & 63,
                  (s[:, np.minimum(j + 4, 11)] >> 4) | ((s[:, np.minimum(j, 7)] >> 6) << 4))
    return sc, mn


# --------------------------------------------------------------------------- integer decode
def decode_int(raw: np.ndarray, qt: int) -> dict:
    """Blocks -> integer codes and scales, the form the kernels' integer dots use.

    Returns (per block b, value i in 0..255):
      IQ3_S : w[b,i] = sign * grid (odd, |w| <= 15); ls[b,s] = 1 + 2*scale nibble (per 32); d[b]
      IQ4_XS: w = kvalues_iq4nl[q]; ls[b,s] = scale - 32 (per 32); d[b]
      Q4_K  : w = 4-bit quant (0..15); sc[b,s], m[b,s] (6-bit, per 32); d[b], dmin[b]
      Q6_K  : w = q - 32 (in [-32, 31]); sc[b,t] int8 per 16; d[b]
    """
    b = _blocks(raw, qt)
    nb = b.shape[0]
    if qt == IQ3_S:
        # block_iq3_s: d[0:2] qs[2:66] qh[66:74] signs[74:106] scales[106:110]
        d = _f16(b[:, 0:2])
        qs = b[:, 2:66].astype(np.int32)                   # [nb, 64] one per 4-value group
        qh = b[:, 66:74].astype(np.int32)                  # [nb, 8] bit e of qh[s] -> group 8s+e
        g = np.arange(64)
        idx = qs | (((qh[:, g // 8] >> (g % 8)) & 1) << 8)
        vals = IQ3S_GRID[idx].astype(np.int32)             # [nb, 64, 4]
        sg = b[:, 74:106].astype(np.int32)                 # [nb, 32]: byte t -> values 8t..8t+7
        v = np.arange(256)
        sbit = (sg[:, v // 8] >> (v % 8)) & 1
        w = vals.reshape(nb, 256) * (1 - 2 * sbit)
        sc = b[:, 106:110].astype(np.int32)
        s = np.arange(8)
        ls = 1 + 2 * ((sc[:, s // 2] >> (4 * (s % 2))) & 0xF)
        return {"w": w.astype(np.int8), "ls": ls, "d": d}
    if qt == IQ4_XS:
        # block_iq4_xs: d[0:2] scales_h[2:4] scales_l[4:8] qs[8:136]
        d = _f16(b[:, 0:2])
        sh = b[:, 2].astype(np.int32) | (b[:, 3].astype(np.int32) << 8)
        sl = b[:, 4:8].astype(np.int32)
        s = np.arange(8)
        ls = ((sl[:, s // 2] >> (4 * (s % 2))) & 0xF) | (((sh[:, None] >> (2 * s)) & 3) << 4)
        qs = b[:, 8:136].astype(np.int32).reshape(nb, 8, 16)   # slice s: 16 bytes
        q = np.concatenate([qs & 0xF, qs >> 4], axis=2)          # values 0..15 low, 16..31 high
        w = KVALUES_IQ4NL[q.reshape(nb, 256)]
        return {"w": w, "ls": ls - 32, "d": d}
    if qt == Q4_K:
        # block_q4_K: d[0:2] dmin[2:4] scales[4:16] qs[16:144]
        d = _f16(b[:, 0:2])
        dmin = _f16(b[:, 2:4])
        sc, m = _q4k_scale_min(b[:, 4:16])
        qs = b[:, 16:144].astype(np.int32).reshape(nb, 4, 32)  # qs[32j+l]: values 64j+l, 64j+32+l
        q = np.concatenate([qs & 0xF, qs >> 4], axis=2)         # [nb, 4, 64]
        return {"w": q.reshape(nb, 256).astype(np.int8), "sc": sc, "m": m, "d": d, "dmin": dmin}
    if qt == Q6_K:
        # block_q6_K: ql[0:128] qh[128:192] scales[192:208] (int8) d[208:210]
        ql = b[:, 0:128].astype(np.int32).reshape(nb, 2, 64)
        qh = b[:, 128:192].astype(np.int32).reshape(nb, 2, 32)
        sc = b[:, 192:208].view(np.int8).astype(np.int32)
        d = _f16(b[:, 208:210])
        l = np.arange(32)
        q = np.empty((nb, 2, 128), dtype=np.int32)
        q[:, :, l] = (ql[:, :, l] & 0xF) | ((qh[:, :, l] & 3) << 4)
        q[:, :, l + 32] = (ql[:, :, l + 32] & 0xF) | (((qh[:, :, l] >> 2) & 3) << 4)
        q[:, :, l + 64] = (ql[:, :, l] >> 4) | (((qh[:, :, l] >> 4) & 3) << 4)
        q[:, :, l + 96] = (ql[:, :, l + 32] >> 4) | (((qh[:, :, l] >> 6) & 3) << 4)
        return {"w": (q.reshape(nb, 256) - 32).astype(np.int8), "sc": sc, "d": d}
    return _decode_int_more(b, qt)


def _sign_bits(signs8: np.ndarray) -> np.ndarray:
    """[..., k] sign bytes -> [..., k, 8] of +1 / -1 (bit j negates value j)."""
    bits = (signs8[..., None].astype(np.int32) >> np.arange(8)) & 1
    return (1 - 2 * bits).astype(np.int32)


def _decode_int_more(b: np.ndarray, qt: int) -> dict:
    """decode_int of Q2_K and the IQ2 / IQ3_XXS / IQ1_M formats. Value = d * ls * w / den with an
    integer sub-scale ls per 32 values ('ls') or per 16 ('ls16'); Q2_K: d * sc * w - dmin * m with
    sc, m per 16 values ('sc16', 'm16')."""
    nb = b.shape[0]
    if qt == Q2_K:
        # block_q2_K: scales[0:16] (low nibble scale, high nibble min, per 16 values) qs[16:80]
        # d[80:82] dmin[82:84]; value 128n + 32j + l is bits 2j of qs[32n + l]
        sc = b[:, 0:16].astype(np.int32)
        qs = b[:, 16:80].astype(np.int32).reshape(nb, 2, 1, 32)
        q = (qs >> (2 * np.arange(4)).reshape(1, 1, 4, 1)) & 3
        return {"w": q.reshape(nb, 256).astype(np.int8), "sc16": sc & 0xF, "m16": sc >> 4,
                "d": _f16(b[:, 80:82]), "dmin": _f16(b[:, 82:84]), "den": 1}
    if qt == IQ2_XXS:
        # d[0:2], then per 32-value slice 8 bytes: 4 grid indices, then a uint32 of four 7-bit
        # sign indices (bits 7g) and the 4-bit scale (bits 28..31)
        d = _f16(b[:, 0:2])
        q = b[:, 2:66].reshape(nb, 8, 8)
        aux = q[:, :, 4:8].copy().view(np.uint32)[..., 0].astype(np.int64)     # [nb, 8]
        grid = IQ2XXS_GRID[q[:, :, 0:4].astype(np.int64)]                      # [nb, 8, 4, 8]
        sidx = (aux[..., None] >> (7 * np.arange(4))) & 127
        sg = _sign_bits(KSIGNS_IQ2XS[sidx])                                    # [nb, 8, 4, 8]
        return {"w": (grid * sg).reshape(nb, 256).astype(np.int8), "ls": (2 * (aux >> 28) + 1).astype(np.int32),
                "d": d, "den": 8}
    if qt == IQ2_XS:
        # d[0:2], qs[2:66] 32 uint16 (9-bit grid index | 7-bit sign index << 9), scales[66:74]
        # (low nibble values 0..15, high nibble 16..31 of slice s)
        d = _f16(b[:, 0:2])
        qs = b[:, 2:66].copy().view(np.uint16).astype(np.int64).reshape(nb, 8, 4)
        grid = IQ2XS_GRID[qs & 511]
        sg = _sign_bits(KSIGNS_IQ2XS[qs >> 9])
        sc = b[:, 66:74].astype(np.int32)
        ls16 = np.stack([sc & 0xF, sc >> 4], -1).reshape(nb, 16)
        return {"w": (grid * sg).reshape(nb, 256).astype(np.int8), "ls16": 2 * ls16 + 1, "d": d, "den": 8}
    if qt == IQ2_S:
        # d[0:2], qs[2:34] grid index low bytes, signs[34:66], qh[66:74] (2 index bits per
        # group), scales[74:82]
        d = _f16(b[:, 0:2])
        lo = b[:, 2:34].astype(np.int64).reshape(nb, 8, 4)
        qh = b[:, 66:74].astype(np.int64).reshape(nb, 8, 1)
        idx = lo | (((qh >> (2 * np.arange(4))) & 3) << 8)
        grid = IQ2S_GRID[idx]
        sg = _sign_bits(b[:, 34:66].reshape(nb, 8, 4))
        sc = b[:, 74:82].astype(np.int32)
        ls16 = np.stack([sc & 0xF, sc >> 4], -1).reshape(nb, 16)
        return {"w": (grid * sg).reshape(nb, 256).astype(np.int8), "ls16": 2 * ls16 + 1, "d": d, "den": 8}
    if qt == IQ3_XXS:
        # d[0:2], qs[2:66] grid indices (one per 4 values), then 8 uint32 (one per slice): four
        # 7-bit sign indices (per 8 values) and the 4-bit scale
        d = _f16(b[:, 0:2])
        grid = IQ3XXS_GRID[b[:, 2:66].astype(np.int64)].reshape(nb, 8, 4, 8)     # [nb, slice, group8, 8]
        aux = b[:, 66:98].copy().view(np.uint32).astype(np.int64).reshape(nb, 8)
        sidx = (aux[..., None] >> (7 * np.arange(4))) & 127
        sg = _sign_bits(KSIGNS_IQ2XS[sidx])
        return {"w": (grid * sg).reshape(nb, 256).astype(np.int8), "ls": (2 * (aux >> 28) + 1).astype(np.int32),
                "d": d, "den": 4}
    if qt == IQ1_M:
        # qs[0:32] grid index low bytes (one per 8 values), qh[32:48] (per group a nibble: index
        # bits 8..10, bit 3 the delta's sign), scales[48:56] as 4 uint16: 3-bit scales per 16
        # values in bits 0..11, the fp16 d in the four top nibbles
        sc = b[:, 48:56].copy().view(np.uint16).astype(np.int64).reshape(nb, 4)
        dbits = ((sc[:, 0] >> 12) | ((sc[:, 1] >> 8) & 0xF0) | ((sc[:, 2] >> 4) & 0xF00) | (sc[:, 3] & 0xF000))
        d = dbits.astype(np.uint16).view(np.float16).astype(np.float32)
        ls16 = ((sc[..., None] >> (3 * np.arange(4))) & 7).reshape(nb, 16)
        qh = b[:, 32:48].astype(np.int64)
        nib = np.stack([qh & 0xF, qh >> 4], -1).reshape(nb, 32)
        idx = b[:, 0:32].astype(np.int64) | ((nib & 7) << 8)
        delta = np.where(nib & 8, -1, 1)                                        # in units of 1/8
        w = 8 * IQ1S_GRID[idx].astype(np.int32) + delta[..., None]
        return {"w": w.reshape(nb, 256).astype(np.int8), "ls16": 2 * ls16 + 1, "d": d, "den": 8}
    raise ValueError(f"decode_int: type {qt} not served")


# --------------------------------------------------------------------------- dequant (gguf-py)
def dequantize(raw: np.ndarray, qt: int) -> np.ndarray:
    """GGUF blocks -> float32 values, the gguf-py b11211 arithmetic (products in float32, the
    same order; every product below is exact in float32 except Q6_K's d*sc*q and Q4_K's
    difference, each a single rounding of the exact value)."""
    t = decode_int(raw, qt)
    nb = t["w"].shape[0]
    w = t["w"].astype(np.float32)
    if qt == IQ3_S:
        db = (t["d"][:, None] * t["ls"].astype(np.float32))          # [nb, 8]
        return (np.repeat(db, 32, axis=1) * w).reshape(-1)
    if qt == IQ4_XS:
        dl = (t["d"][:, None] * t["ls"].astype(np.float32))
        return (np.repeat(dl, 32, axis=1) * w).reshape(-1)
    if qt == Q4_K:
        dd = t["d"][:, None] * t["sc"].astype(np.float32)
        dm = t["dmin"][:, None] * t["m"].astype(np.float32)
        return (np.repeat(dd, 32, axis=1) * w - np.repeat(dm, 32, axis=1)).reshape(-1)
    if qt == Q6_K:
        dd = t["d"][:, None] * t["sc"].astype(np.float32)            # [nb, 16]
        return (np.repeat(dd, 16, axis=1) * w).reshape(nb * 256)
    f32 = np.float32
    if qt == Q2_K:  # dl * q - ml
        dl = t["d"][:, None] * t["sc16"].astype(f32)
        ml = t["dmin"][:, None] * t["m16"].astype(f32)
        return (np.repeat(dl, 16, axis=1) * w - np.repeat(ml, 16, axis=1)).reshape(-1)
    # the IQ formats: gguf-py multiplies a per-group float scale by the grid value, then the sign
    b = _blocks(raw, qt)
    mag = np.abs(w)
    sign = np.where(w < 0, f32(-1), f32(1))
    if qt in (IQ2_XXS, IQ3_XXS):
        s4 = ((t["ls"] - 1) // 2).astype(f32)                          # the 4-bit scale
        db = (t["d"][:, None] * (f32(0.5) + s4)) * (f32(0.25) if qt == IQ2_XXS else f32(0.5))
        return (np.repeat(db, 32, axis=1) * mag * sign).reshape(-1)
    if qt in (IQ2_XS, IQ2_S):
        s4 = ((t["ls16"] - 1) // 2).astype(f32)
        db = (t["d"][:, None] * (f32(0.5) + s4)) * f32(0.25)
        return (np.repeat(db, 16, axis=1) * mag * sign).reshape(-1)
    if qt == IQ1_M:  # dl * (grid + delta)
        dl = t["d"][:, None] * t["ls16"].astype(f32)
        gd = (w.astype(f32) / f32(8))                                  # grid +- 0.125, exact
        return (np.repeat(dl, 16, axis=1) * gd).reshape(-1)
    raise ValueError(qt)


# --------------------------------------------------------------------------- q8_1
def _roundf(t: np.ndarray) -> np.ndarray:
    """C roundf on float32: nearest integer, ties away from zero (t - trunc(t) is exact)."""
    r = np.trunc(t)
    frac = np.abs(t - r)
    return r + np.where(frac >= 0.5, np.sign(t), 0).astype(np.float32)


def _xor_tree_sum(v: np.ndarray, offsets) -> np.ndarray:
    """Lane 0 of a float32 xor-butterfly sum over the last axis (x += shfl_xor(x, off))."""
    n = v.shape[-1]
    lanes = np.arange(n)
    for off in offsets:
        v = (v + v[..., lanes ^ off]).astype(np.float32)
    return v[..., 0]


def _as_f32(x) -> np.ndarray:
    if hasattr(x, "detach"):  # torch tensor of any float dtype: widening to fp32 is exact
        x = x.detach().cpu().float().numpy()
    return np.ascontiguousarray(x, dtype=np.float32)


def quantize_q8_1(x) -> np.ndarray:
    """X [n, K] -> block_q8_1 bytes (n*K/32 blocks of 36 B, row-major by (row, block)):
    half d, half sum, 32 x int8. lcpp_shim.cu:274-294: d = amax/127.0f, q = amax == 0 ? 0 :
    roundf(x/d), sum by a 32-lane xor butterfly (offsets 16..1), ds = make_half2(d, sum)."""
    xf = _as_f32(x)
    n, k = xf.shape
    assert k % QK8_1 == 0
    b = xf.reshape(n, k // QK8_1, QK8_1)
    amax = np.abs(b).max(-1)
    s = _xor_tree_sum(b, (16, 8, 4, 2, 1))
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (b / d[..., None]).astype(np.float32)
    q = np.where(amax[..., None] == 0, 0, _roundf(t)).astype(np.int8)
    out = np.zeros((n, k // QK8_1, 36), dtype=np.uint8)
    with np.errstate(over="ignore"):
        out[..., 0:2] = d.astype(np.float16)[..., None].view(np.uint8)
        out[..., 2:4] = s.astype(np.float16)[..., None].view(np.uint8)
    out[..., 4:36] = q.view(np.uint8)
    return out.reshape(-1)


def dequant_q8_1(q8: np.ndarray, n: int, k: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """block_q8_1 bytes -> (q int8 [n, K], d float32 [n, K/32] (from half), sum float32)."""
    blk = np.ascontiguousarray(q8, dtype=np.uint8).reshape(n, k // QK8_1, 36)
    d = blk[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    s = blk[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float32)
    q = blk[..., 4:36].copy().view(np.int8).reshape(n, k)
    return q, d, s


# ds layouts of block_q8_1_mmq (mmq.cuh:60-100) for the served types
MMQ_DS4_TYPES = (Q4_K,)


def _quantize_q8_1_mmq_d2s6(xf: np.ndarray) -> np.ndarray:
    """block_q8_1_mmq with the D2S6 scale layout (Q2_K, mmq.cuh:60-100; lcpp_shim.cu:298-355 with
    vals_per_scale 64 and vals_per_sum 16): per 64 values d_inv = 127 / amax, q = roundf(x *
    d_inv), d = 1 / d_inv; per 16 values the sum ((x0 + x1) + x2) + x3 per 4-value lane, then xor
    offsets 2, 1; header halves [d of values 0..63, d of 64..127, sums of the 16-value groups
    0..5]."""
    n, k = xf.shape
    b = xf.reshape(n, k // 64, 64)
    amax = np.abs(b).max(-1)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        d_inv = (np.float32(127.0) / amax).astype(np.float32)
        t = (b * d_inv[..., None]).astype(np.float32)
        d = (np.float32(1.0) / d_inv).astype(np.float32)
    q = np.where(amax[..., None] == 0, 0, _roundf(np.nan_to_num(t))).astype(np.int8)
    d = np.where(amax == 0, np.float32(0), d).astype(np.float32)
    lane = xf.reshape(n, k // 16, 4, 4)
    ls = (((lane[..., 0] + lane[..., 1]).astype(np.float32) + lane[..., 2]).astype(np.float32)
          + lane[..., 3]).astype(np.float32)
    sums = _xor_tree_sum(ls, (2, 1))                                     # [n, k/16]
    out = np.zeros((k // 128, n, 144), dtype=np.uint8)
    hdr = np.zeros((k // 128, n, 8), dtype=np.float16)
    with np.errstate(over="ignore"):
        hdr[..., 0:2] = d.reshape(n, k // 128, 2).transpose(1, 0, 2).astype(np.float16)
        hdr[..., 2:8] = sums.reshape(n, k // 128, 8)[..., :6].transpose(1, 0, 2).astype(np.float16)
    out[..., 0:16] = hdr.view(np.uint8).reshape(k // 128, n, 16)
    out[..., 16:144] = q.reshape(n, k // 128, 128).transpose(1, 0, 2).view(np.uint8)
    return out.reshape(-1)


def mmq_d2s6_sums(q8: np.ndarray, n: int, k: int) -> np.ndarray:
    """The six stored half sums of D2S6 block_q8_1_mmq bytes per 128 values, widened: float32
    [n, K/16] with NaN for the two unstored groups (values 96..127 of each block)."""
    blk = np.ascontiguousarray(q8, dtype=np.uint8).reshape(k // 128, n, 144)
    h = blk[..., :16].copy().view(np.float16).reshape(k // 128, n, 8)[..., 2:8].astype(np.float32)
    out = np.full((n, k // 128, 8), np.nan, dtype=np.float32)
    out[..., :6] = h.transpose(1, 0, 2)
    return out.reshape(n, k // 16)


def quantize_q8_1_mmq(x, qt: int) -> np.ndarray:
    """X [n, K] -> block_q8_1_mmq bytes: 144-B blocks of 128 values, block index
    (k/128)*n + row; bytes 0..15 = 4 x fp32 d (D4) or 4 x half2(d, sum) (DS4, Q4_K), bytes
    16..143 = 128 x int8. lcpp_shim.cu:298-355: per 32 values d_inv = 127/amax,
    q = roundf(x*d_inv), d = 1/d_inv; sum = ((x0+x1)+x2)+x3 per lane, then xor offsets 4,2,1.
    amax == 0 gives q = 0 and d = 0 (the reference's NaN -> 0 int8 conversion and 1/inf)."""
    xf = _as_f32(x)
    n, k = xf.shape
    assert k % 128 == 0
    if qt == Q2_K:
        return _quantize_q8_1_mmq_d2s6(xf)
    b = xf.reshape(n, k // 32, 32)
    amax = np.abs(b).max(-1)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        d_inv = (np.float32(127.0) / amax).astype(np.float32)
        t = (b * d_inv[..., None]).astype(np.float32)
        d = (np.float32(1.0) / d_inv).astype(np.float32)
    q = np.where(amax[..., None] == 0, 0, _roundf(np.nan_to_num(t))).astype(np.int8)
    d = np.where(amax == 0, np.float32(0), d).astype(np.float32)
    lane = b.reshape(n, k // 32, 8, 4)
    ls = (((lane[..., 0] + lane[..., 1]).astype(np.float32) + lane[..., 2]).astype(np.float32)
          + lane[..., 3]).astype(np.float32)
    s = _xor_tree_sum(ls, (4, 2, 1))
    out = np.zeros((k // 128, n, 144), dtype=np.uint8)
    d4 = d.reshape(n, k // 128, 4).transpose(1, 0, 2)
    q4 = q.reshape(n, k // 128, 128).transpose(1, 0, 2)
    s4 = s.reshape(n, k // 128, 4).transpose(1, 0, 2)
    if qt in MMQ_DS4_TYPES:
        with np.errstate(over="ignore"):
            ds = np.stack([d4.astype(np.float16), s4.astype(np.float16)], -1)  # [.., 4, 2]
        out[..., 0:16] = np.ascontiguousarray(ds).view(np.uint8).reshape(k // 128, n, 16)
    else:
        out[..., 0:16] = np.ascontiguousarray(d4).view(np.uint8).reshape(k // 128, n, 16)
    out[..., 16:144] = q4.view(np.uint8)
    return out.reshape(-1)


def mmq_ds4_sums(q8: np.ndarray, n: int, k: int) -> np.ndarray:
    """The half2 sum field of DS4 block_q8_1_mmq bytes (Q4_K), widened: float32 [n, K/32]."""
    blk = np.ascontiguousarray(q8, dtype=np.uint8).reshape(k // 128, n, 144)
    s = blk[..., :16].copy().view(np.float16).reshape(k // 128, n, 4, 2)[..., 1].astype(np.float32)
    return np.ascontiguousarray(s.transpose(1, 0, 2).reshape(n, k // 32))


def dequant_q8_1_mmq(q8: np.ndarray, n: int, k: int, qt: int) -> tuple[np.ndarray, np.ndarray]:
    """block_q8_1_mmq bytes -> (q int8 [n, K], d float32 [n, K/32]) (d from half for DS4)."""
    blk = np.ascontiguousarray(q8, dtype=np.uint8).reshape(k // 128, n, 144)
    q = blk[..., 16:].copy().view(np.int8).transpose(1, 0, 2).reshape(n, k)
    hdr = blk[..., :16].copy()
    if qt == Q2_K:  # D2S6: one half d per 64 values
        d64 = hdr.view(np.float16).reshape(k // 128, n, 8)[..., 0:2].astype(np.float32)
        return q, np.ascontiguousarray(np.repeat(d64.transpose(1, 0, 2).reshape(n, k // 64), 2, axis=1))
    if qt in MMQ_DS4_TYPES:
        d = hdr.view(np.float16).reshape(k // 128, n, 4, 2)[..., 0].astype(np.float32)
    else:
        d = hdr.view(np.float32).reshape(k // 128, n, 4)
    return q, np.ascontiguousarray(d.transpose(1, 0, 2).reshape(n, k // 32))


# --------------------------------------------------------------------------- integer slice dots
def slice_dots(raw: np.ndarray, qt: int, q: np.ndarray) -> dict:
    """Per (activation row, weight row, 32-value slice) integer dot products, int64, exactly as
    the reference's vec_dot functions form them before any float scale:
      IQ3_S : sumi * (1 + 2*ls)                        (vecdotq.cuh:1211-1248)
      IQ4_XS: sumi * (ls - 32)                         (vecdotq.cuh:1357-1380)
      Q6_K  : sc_a * sumi_a + sc_b * sumi_b, 16 each   (vecdotq.cuh:627-648)
      Q4_K  : 'd' = sc * sum(nib * q8), 'm' = m * sum(q8)  (vecdotq.cuh:508-530)
      Q2_K  : as Q4_K per 16 values: 'd' = sum_h sc_h * sumi_h, 'm' = sum_h m_h * sum(q8)_h
      IQ2_XXS, IQ3_XXS: sumi * (2s + 1); IQ2_XS, IQ2_S, IQ1_M: sum_h (2s_h + 1) * sumi_h, with
              the value d * that / den, den = 8 (IQ2, IQ1_M: w = 8 grid +- 1) or 4 (IQ3_XXS)
    raw: [rows, row_bytes]; q: int8 [n, K]. Returns dict of int64 [n, rows, K/32] (and 'den')."""
    rows = raw.shape[0]
    t = decode_int(raw.reshape(-1), qt)
    n, k = q.shape
    ns = k // 32
    w = t["w"].astype(np.int64).reshape(rows, ns, 32)
    qq = q.astype(np.int64).reshape(n, ns, 32)
    if qt == Q6_K:
        w16 = w.reshape(rows, ns, 2, 16)
        q16 = qq.reshape(n, ns, 2, 16)
        sumi = np.einsum("rstv,nstv->nrst", w16, q16)                   # [n, rows, ns, 2]
        sc = t["sc"].reshape(rows, ns, 2).astype(np.int64)
        return {"dot": (sumi * sc[None]).sum(-1)}
    sumi = np.einsum("rsv,nsv->nrs", w, qq)
    if qt == IQ3_S or qt == IQ4_XS:
        return {"dot": sumi * t["ls"].reshape(rows, ns).astype(np.int64)[None]}
    if qt == Q4_K:
        sq = qq.sum(-1)                                                 # [n, ns]
        return {"dot": sumi * t["sc"].reshape(rows, ns).astype(np.int64)[None],
                "m": sq[:, None, :] * t["m"].reshape(rows, ns).astype(np.int64)[None]}
    if "ls" in t:        # IQ2_XXS, IQ3_XXS: one sub-scale per slice; value = d * ls * w / den
        return {"dot": sumi * t["ls"].reshape(rows, ns).astype(np.int64)[None], "den": t["den"]}
    w16 = w.reshape(rows, ns, 2, 16)
    q16 = qq.reshape(n, ns, 2, 16)
    sumi16 = np.einsum("rstv,nstv->nrst", w16, q16)                     # [n, rows, ns, 2]
    if "ls16" in t:      # IQ2_XS, IQ2_S, IQ1_M: a sub-scale per 16 values
        return {"dot": (sumi16 * t["ls16"].reshape(rows, ns, 2).astype(np.int64)[None]).sum(-1), "den": t["den"]}
    if qt == Q2_K:       # sc and m per 16 values (vecdotq.cuh:365-393)
        sq16 = q16.sum(-1)                                              # [n, ns, 2]
        return {"dot": (sumi16 * t["sc16"].reshape(rows, ns, 2).astype(np.int64)[None]).sum(-1),
                "m": (sq16[:, None] * t["m16"].reshape(rows, ns, 2).astype(np.int64)[None]).sum(-1)}
    raise ValueError(qt)


def _cdiv(a: np.ndarray, b: int) -> np.ndarray:
    """C integer division of int64 values by a positive int: the quotient truncated toward zero."""
    return np.sign(a) * (np.abs(a) // b)


# the types whose slice value is d * (integer) / den with a single block d
UNIT_TYPES = (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ1_M)


def mmvq_slice_units(raw: np.ndarray, qt: int, q: np.ndarray) -> np.ndarray:
    """Per (activation row, weight row, 32-value slice) the decode ops' slice value in units of
    d_w * d8, float64, formed as the reference's vec_dot functions form it, truncating C
    divisions included (s: the raw 4-bit scale, ls = 2s + 1):
      IQ2_XXS        sumi * ls / 8                                    (vecdotq.cuh:1074-1077)
      IQ2_XS, IQ2_S  (sumi_a * s_a + sumi_b * s_b + (sumi_a + sumi_b) / 2) / 4, halves a, b
                                                                      (:1116-1118, :1163-1166)
      IQ3_XXS        (s * sumi + sumi / 2) / 2                         (:1201-1204)
      IQ1_M          ((sumi_a + delta_a sum q8_a) * ls_a + ...) with sumi over grid + 1 and delta
                     = -1 +- 1/8 (:1286-1328): exactly slice_dots' dot / 8 (no division)
    raw: [rows, row_bytes]; q: int8 [n, K]. Returns [n, rows, K/32]."""
    rows = raw.shape[0]
    t = decode_int(raw.reshape(-1), qt)
    n, k = q.shape
    ns = k // 32
    w = t["w"].astype(np.int64).reshape(rows, ns, 2, 16)
    qq = q.astype(np.int64).reshape(n, ns, 2, 16)
    s16 = np.einsum("rsth,nsth->nrst", w, qq)                          # [n, rows, ns, 2]
    s = s16.sum(-1)
    if qt == IQ2_XXS:
        return _cdiv(s * t["ls"].reshape(rows, ns)[None].astype(np.int64), 8).astype(np.float64)
    if qt == IQ3_XXS:
        s4 = ((t["ls"].reshape(rows, ns).astype(np.int64) - 1) // 2)[None]
        return _cdiv(s4 * s + _cdiv(s, 2), 2).astype(np.float64)
    if qt in (IQ2_XS, IQ2_S):
        s4 = ((t["ls16"].reshape(rows, ns, 2).astype(np.int64) - 1) // 2)[None]
        a, b = s16[..., 0], s16[..., 1]
        return _cdiv(a * s4[..., 0] + b * s4[..., 1] + _cdiv(a + b, 2), 4).astype(np.float64)
    if qt == IQ1_M:
        return (s16 * t["ls16"].reshape(rows, ns, 2)[None].astype(np.int64)).sum(-1) / 8.0
    raise ValueError(f"mmvq_slice_units: type {qt} has no single-scale slice value")


# --------------------------------------------------------------------------- reference models
def q81_model(raw: np.ndarray, qt: int, x, layout: str = "mmvq") -> np.ndarray:
    """float64 y[n, rows] = dequant(q8_1(x)) @ dequant(W).T (tests/gpu/_refs.py:40-54,83).
    layout 'mmvq': x' = q * half(d) (block_q8_1, lcpp_shim.cu:274-294); 'mmq': x' = q * d
    with the MMQ layout's rounding and fp32 d (half d for DS4 types, lcpp_shim.cu:298-355).
    Q4_K's min term follows the layout's vec_dot: with 'mmvq' it is dmin * m * d8 * sum(q8) per
    slice (vec_dot_q4_K_q8_1_impl_vmmq, vecdotq.cuh:508-530), which is what dequant(q8_1(x)) .
    dequant(W) gives; with 'mmq' it is dmin * m * half(sum(x)) per slice, the DS4 sum of the
    block_q8_1_mmq bytes (vec_dot_q4_K_q8_1_impl_mmq, vecdotq.cuh:533-557). Q2_K's 'mmq' layout
    is D2S6 (a scale per 64 values, stored sums per 16)."""
    xf = _as_f32(x)
    n, k = xf.shape
    rows = raw.shape[0]
    if layout == "mmvq":
        q, d, _ = dequant_q8_1(quantize_q8_1(xf), n, k)
    else:
        q8 = quantize_q8_1_mmq(xf, qt)
        q, d = dequant_q8_1_mmq(q8, n, k, qt)
    xq = (q.astype(np.float64).reshape(n, k // 32, 32) * d.astype(np.float64)[..., None]).reshape(n, k)
    if qt == Q2_K and layout == "mmq":
        # ggml_cuda_mmq_vec_dot_q2_K_q8_1_mma (mmq-vec-dot.cuh:688-745, the scalar form
        # vecdotq.cuh:396-445): the tile loader stores d * sc and dmin * m as fp16
        # (mmq-load-tiles.cuh:582-591); the min term per 16 values is dmin * m * half(sum x) where
        # D2S6 stores the sum (groups 0..5 of every 128 values), dmin * m * d8 * sum(q8) for
        # groups 6, 7
        t = decode_int(raw.reshape(-1), qt)
        f16 = np.float16
        dd = (t["d"][:, None] * t["sc16"].astype(np.float32)).astype(f16).astype(np.float64)    # [nb, 16]
        main = (np.repeat(dd, 16, axis=1) * t["w"].astype(np.float64)).reshape(rows, k)
        mins = (t["dmin"][:, None] * t["m16"].astype(np.float32)).astype(f16).astype(np.float64).reshape(rows, k // 16)
        S = mmq_d2s6_sums(q8, n, k).astype(np.float64)
        qsum = (q.astype(np.float64).reshape(n, k // 16, 16).sum(-1) * np.repeat(d.astype(np.float64), 2, axis=1))
        S = np.where(np.isnan(S), qsum, S)
        return xq @ main.T - S @ mins.T
    if qt == Q4_K and layout == "mmq":
        t = decode_int(raw.reshape(-1), qt)
        dd = (t["d"][:, None] * t["sc"].astype(np.float32)).astype(np.float64)        # [nb, 8]
        main = (np.repeat(dd, 32, axis=1) * t["w"].astype(np.float64)).reshape(rows, k)
        mins = (t["dmin"][:, None] * t["m"].astype(np.float32)).astype(np.float64).reshape(rows, k // 32)
        return xq @ main.T - mmq_ds4_sums(q8, n, k).astype(np.float64) @ mins.T
    W = dequantize(raw.reshape(-1), qt).astype(np.float64).reshape(rows, k)
    return xq @ W.T


def full_model(raw: np.ndarray, qt: int, x) -> np.ndarray:
    """float64 x @ dequant(W).T (no activation quantization)."""
    xf = _as_f32(x).astype(np.float64)
    rows = raw.shape[0]
    W = dequantize(raw.reshape(-1), qt).astype(np.float64).reshape(rows, xf.shape[1])
    return xf @ W.T


def rel_l2(y, ref) -> float:
    """max over activation rows of ||y - ref|| / ||ref|| (tests/gpu/_refs.py:94-99)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    num = np.linalg.norm(y - ref, axis=-1)
    den = np.maximum(np.linalg.norm(ref, axis=-1), 1e-30)
    return float((num / den).max())


# --------------------------------------------------------------------------- synthetic weights
def random_blocks(rng: np.random.Generator, qt: int, rows: int, k: int,
                  scale_sigma: float = 2e-3) -> np.ndarray:
    """Seeded synthetic GGUF rows [rows, k/256*bytes]: uniform random code bytes with every fp16
    scale replaced by |N(0, scale_sigma)| (the benchmark configs; the reference's recipe is
    kit/synth.py:70-87, uniform bytes with valid fp16 scales)."""
    bs = BLOCK_BYTES[qt]
    nb = rows * (k // QK_K)
    b = rng.integers(0, 256, size=(nb, bs), dtype=np.uint8)
    for off in SCALE_OFFSETS[qt]:
        s = np.abs(rng.normal(0.0, scale_sigma, nb)).astype(np.float16)
        b[:, off:off + 2] = s.view(np.uint8).reshape(nb, 2)
    if qt == IQ1_M:
        set_iq1m_d(b, np.abs(rng.normal(0.0, scale_sigma, nb)).astype(np.float16))
    return b.reshape(rows, -1)


# byte offsets of the fp16 block scales (d, and dmin for Q4_K / Q2_K); IQ1_M keeps d in nibbles
SCALE_OFFSETS = {IQ3_S: (0,), IQ4_XS: (0,), Q4_K: (0, 2), Q6_K: (208,), Q2_K: (80, 82), IQ2_XXS: (0,),
                 IQ2_XS: (0,), IQ2_S: (0,), IQ3_XXS: (0,), IQ1_M: ()}


def set_iq1m_d(blocks: np.ndarray, d: np.ndarray) -> None:
    """Write fp16 d into the four top nibbles of IQ1_M blocks' scale words, in place."""
    bits = np.ascontiguousarray(d, dtype=np.float16).view(np.uint16).astype(np.int64)
    sc = blocks[:, 48:56].copy().view(np.uint16).astype(np.int64).reshape(-1, 4)
    for j in range(4):
        sc[:, j] = (sc[:, j] & 0x0FFF) | (((bits >> (4 * j)) & 0xF) << 12)
    blocks[:, 48:56] = sc.astype(np.uint16).view(np.uint8).reshape(-1, 8)
