/* Prints the reference's IQ3_S grid and IQ4_NL codebook, compiled from the reference's own
 * header (plugin/vllm_gguf_plugin/csrc/lcpp/ggml/src/ggml-common.h:1052,1120). Test
 * infrastructure: tests/test_oracle.py compares oracle/gguf_oracle.py's tables with this
 * output when oracle/_ref/ref_tables exists. Build recipe: oracle/Makefile. */
#include <stdio.h>
#include <stdint.h>
#define GGML_COMMON_DECL_C
#define GGML_COMMON_IMPL_C
#include "ggml-common.h"

int main(void) {
  for (int i = 0; i < 512; ++i) printf("iq3s_grid %d %u\n", i, (unsigned)iq3s_grid[i]);
  for (int i = 0; i < 16; ++i) printf("kvalues_iq4nl %d %d\n", i, (int)kvalues_iq4nl[i]);
  printf("sizeof block_iq3_s %zu block_q4_K %zu block_q6_K %zu block_iq4_xs %zu block_q8_1 %zu\n",
         sizeof(block_iq3_s), sizeof(block_q4_K), sizeof(block_q6_K), sizeof(block_iq4_xs),
         sizeof(block_q8_1));
  return 0;
}
