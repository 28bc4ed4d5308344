"""The op registration shares the _C_gguf namespace with other libraries.

The reference defines `_C_gguf` once, for its stock ops (`STABLE_TORCH_LIBRARY(_C_gguf)`,
plugin/vllm_gguf_plugin/csrc/torch_bindings.cpp:22), and adds the Route L ops to it as a fragment
(`STABLE_TORCH_LIBRARY_FRAGMENT(_C_gguf)`, csrc/lcpp_shim.cu:973). The stock extension supplies
`ggml_dequantize` to the plugin's other callers, so this build's registration must load beside a
library that already defines the namespace, and the namespace must stay open to one that defines
it afterwards. Each case runs in a fresh child process with the GPU hidden: a second definition
of a namespace ends a process in std::terminate, not in a Python exception.
"""

import os
import subprocess
import sys

from conftest import PKG_ROOT

OPS_LIB = os.path.join(PKG_ROOT, "vllm_gguf_plugin", "_C_gguf_ops.so")
ROUTE_L = ("lcpp_mul_mat_vec_q", "lcpp_mul_mat_q", "lcpp_mul_mat_vec_iq3", "lcpp_mul_mat_vec_iq3_mma",
           "lcpp_mul_mat_vec_own", "lcpp_mul_mat_mma_k", "lcpp_mul_mat_vec_iq3_mma_packed",
           "lcpp_mul_mat_iq3_packed", "lcpp_quantize_q8_1")

# a stand-in for the stock extension's definition of the namespace (its op schema,
# torch_bindings.cpp: ggml_dequantize(Tensor W, int type, SymInt m, SymInt n, ScalarType? dtype))
DEFINE_STOCK = """
stock = torch.library.Library("_C_gguf", "DEF")
stock.define("ggml_dequantize(Tensor W, int type, SymInt m, SymInt n, ScalarType? dtype) -> Tensor")
"""

CHECK = """
for name in {ops!r}:
    assert hasattr(torch.ops._C_gguf, name), name
assert hasattr(torch.ops._C_gguf, "ggml_dequantize")
print("both", flush=True)
"""


def _child(body):
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="", ROCR_VISIBLE_DEVICES="")
    src = "import torch\n" + body + CHECK.format(ops=ROUTE_L)
    return subprocess.run([sys.executable, "-c", src], capture_output=True, text=True, env=env, timeout=300)


def test_loads_after_the_stock_namespace():
    """The stock ops define _C_gguf first (the reference's import order), then the Route L
    registration loads into it."""
    p = _child(DEFINE_STOCK + f"torch.ops.load_library({OPS_LIB!r})\n")
    assert p.returncode == 0, p.stderr[-2000:]
    assert "both" in p.stdout


def test_stock_namespace_defined_after_the_ops():
    """The Route L registration loads first and the namespace is defined afterwards."""
    p = _child(f"torch.ops.load_library({OPS_LIB!r})\n" + DEFINE_STOCK)
    assert p.returncode == 0, p.stderr[-2000:]
    assert "both" in p.stdout


def test_guards_still_run_beside_the_stock_ops():
    """With the stock namespace defined first, a Route L op still runs its guards on host tensors
    (the CPU registration) and raises the library's message."""
    body = DEFINE_STOCK + f"torch.ops.load_library({OPS_LIB!r})\n" + """
W = torch.zeros(16, 110, dtype=torch.uint8)
X = torch.zeros(1, 256)
try:
    torch.ops._C_gguf.lcpp_mul_mat_vec_q(W, X, 21, 16)
except RuntimeError as e:
    assert "lcpp_mul_mat_vec_q: K=256 must be a multiple of 512" in str(e), str(e)
    print("guard:", str(e).splitlines()[0], flush=True)
else:
    raise AssertionError("no guard raised")
"""
    p = _child(body)
    assert p.returncode == 0, p.stderr[-2000:]
    assert "guard:" in p.stdout and "both" in p.stdout
