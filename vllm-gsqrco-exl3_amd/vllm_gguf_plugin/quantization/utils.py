"""GGUF type ids and the type sets the linear method routes on
(reference: plugin/vllm_gguf_plugin/quantization/utils.py:46-75)."""

import enum

try:  # gguf-py, when installed, is the source of the ids
    from gguf import GGML_QUANT_SIZES
    from gguf import GGMLQuantizationType as WeightType
except ImportError:
    class WeightType(enum.IntEnum):
        """gguf-py GGMLQuantizationType ids (a file-format enumeration)."""
        F32 = 0
        F16 = 1
        Q4_0 = 2
        Q4_1 = 3
        Q5_0 = 6
        Q5_1 = 7
        Q8_0 = 8
        Q8_1 = 9
        Q2_K = 10
        Q3_K = 11
        Q4_K = 12
        Q5_K = 13
        Q6_K = 14
        Q8_K = 15
        IQ2_XXS = 16
        IQ2_XS = 17
        IQ3_XXS = 18
        IQ1_S = 19
        IQ4_NL = 20
        IQ3_S = 21
        IQ2_S = 22
        IQ4_XS = 23
        I8 = 24
        I16 = 25
        I32 = 26
        I64 = 27
        F64 = 28
        IQ1_M = 29
        BF16 = 30

    # (values per block, bytes per block) of the types this build serves, and the float types
    GGML_QUANT_SIZES = {
        WeightType.F32: (1, 4), WeightType.F16: (1, 2), WeightType.BF16: (1, 2),
        WeightType.Q2_K: (256, 84), WeightType.Q4_K: (256, 144), WeightType.Q6_K: (256, 210),
        WeightType.IQ2_XXS: (256, 66), WeightType.IQ2_XS: (256, 74), WeightType.IQ2_S: (256, 82),
        WeightType.IQ3_XXS: (256, 98), WeightType.IQ3_S: (256, 110), WeightType.IQ4_XS: (256, 136),
        WeightType.IQ1_M: (256, 56),
    }

UNQUANTIZED_TYPES = {WeightType.F32, WeightType.F16, WeightType.BF16}
STANDARD_QUANT_TYPES = {WeightType.Q4_0, WeightType.Q4_1, WeightType.Q5_0, WeightType.Q5_1,
                        WeightType.Q8_0, WeightType.Q8_1}
KQUANT_TYPES = {WeightType.Q2_K, WeightType.Q3_K, WeightType.Q4_K, WeightType.Q5_K, WeightType.Q6_K}
IMATRIX_QUANT_TYPES = {WeightType.IQ1_M, WeightType.IQ1_S, WeightType.IQ2_XXS, WeightType.IQ2_XS,
                       WeightType.IQ2_S, WeightType.IQ3_XXS, WeightType.IQ3_S, WeightType.IQ4_XS,
                       WeightType.IQ4_NL}
DEQUANT_TYPES = STANDARD_QUANT_TYPES | KQUANT_TYPES | IMATRIX_QUANT_TYPES
MMVQ_QUANT_TYPES = STANDARD_QUANT_TYPES | KQUANT_TYPES | IMATRIX_QUANT_TYPES
MMQ_QUANT_TYPES = STANDARD_QUANT_TYPES | KQUANT_TYPES
