"""Route L switch and type set (reference: plugin/vllm_gguf_plugin/ops.py:85-115).

In this build Route L is the only quantized path (the reference's stock CUDA / Triton dispatch is
not rebuilt), so it is on unless VLLM_GGUF_LCPP=0. Importing this module registers
torch.ops._C_gguf from libgguf_mi355x.so and fails loudly if the library is not built.
"""

import os

from . import _C_gguf
from .quantization.utils import WeightType

LCPP_ENABLED = os.environ.get("VLLM_GGUF_LCPP", "1") != "0"
# the Route L types (reference ops.py:85-115), all served by this build's kernels
LCPP_QUANT_TYPES = frozenset({
    WeightType.Q2_K, WeightType.Q4_K, WeightType.Q6_K, WeightType.IQ2_XXS, WeightType.IQ2_XS, WeightType.IQ2_S,
    WeightType.IQ3_XXS, WeightType.IQ3_S, WeightType.IQ4_XS, WeightType.IQ1_M})

_C_gguf.register()
