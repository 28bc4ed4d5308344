"""MI355X-native GGUF quantized-matmul path of the vllm_gguf_plugin surface.

The Python surface mirrors the reference plugin's (plugin/vllm_gguf_plugin): the GGUF linear
method (quantization/linear.py), its routing table and IQ3 repack hook, and the Route L ops
torch.ops._C_gguf.lcpp_* (_C_gguf.py), all served by the hand-written gfx950 HIP kernels of
libgguf_mi355x.so through its C ABI (include/gguf_mi355x.h).
"""
