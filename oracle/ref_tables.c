/* Prints the reference's GGUF codebooks and block sizes, compiled from the reference's own header
 * (plugin/vllm_gguf_plugin/csrc/lcpp/ggml/src/ggml-common.h: iq3s_grid :1052, kvalues_iq4nl :1120,
 * iq2xxs_grid, iq2xs_grid, iq2s_grid, iq3xxs_grid, iq1s_grid, ksigns_iq2xs). Test infrastructure:
 * tests/test_oracle.py compares oracle/gguf_oracle.py's tables with this output when
 * oracle/_ref/ref_tables exists. Build recipe: oracle/Makefile. */
#include <stdio.h>
#include <stdint.h>
#define GGML_COMMON_DECL_C
#define GGML_COMMON_IMPL_C
#include "ggml-common.h"

int main(void) {
  for (int i = 0; i < 512; ++i) printf("iq3s_grid %d %u\n", i, (unsigned)iq3s_grid[i]);
  for (int i = 0; i < 16; ++i) printf("kvalues_iq4nl %d %d\n", i, (int)kvalues_iq4nl[i]);
  for (int i = 0; i < 256; ++i) printf("iq2xxs_grid %d %llu\n", i, (unsigned long long)iq2xxs_grid[i]);
  for (int i = 0; i < 512; ++i) printf("iq2xs_grid %d %llu\n", i, (unsigned long long)iq2xs_grid[i]);
  for (int i = 0; i < 1024; ++i) printf("iq2s_grid %d %llu\n", i, (unsigned long long)iq2s_grid[i]);
  for (int i = 0; i < 256; ++i) printf("iq3xxs_grid %d %u\n", i, (unsigned)iq3xxs_grid[i]);
  for (int i = 0; i < 2048; ++i) printf("iq1s_grid %d %llu\n", i, (unsigned long long)iq1s_grid[i]);
  for (int i = 0; i < 128; ++i) printf("ksigns_iq2xs %d %u\n", i, (unsigned)ksigns_iq2xs[i]);
  printf("sizeof block_iq3_s %zu block_q4_K %zu block_q6_K %zu block_iq4_xs %zu block_q8_1 %zu "
         "block_q2_K %zu block_iq2_xxs %zu block_iq2_xs %zu block_iq2_s %zu block_iq3_xxs %zu block_iq1_m %zu\n",
         sizeof(block_iq3_s), sizeof(block_q4_K), sizeof(block_q6_K), sizeof(block_iq4_xs), sizeof(block_q8_1),
         sizeof(block_q2_K), sizeof(block_iq2_xxs), sizeof(block_iq2_xs), sizeof(block_iq2_s), sizeof(block_iq3_xxs),
         sizeof(block_iq1_m));
  return 0;
}
