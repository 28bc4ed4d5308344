"""Each kernel family's first call made inside a CUDA-graph capture, in a fresh process.

The reference promises that its kernels' one-time set-up (the max-dynamic-shared-memory attribute,
the first device query) may run inside a capture (lcpp_owned_iq3_mma.cu:333-346,
lcpp_owned_mma_k.cu:551-569) and tests it in a fresh process (tests/gpu/test_kernel_parity.py:
655-698). Here the set-up is the stream GEMVs' dynamic-LDS attributes (IQ3_S, the 4x4x4 MFMA
GEMV, the generic types' stream GEMV), the compute-unit count the launch plans read, and the
no-allocation entry point's scratch address. The child process touches
the GPU only through torch (inputs made and packed on the host, so that not even the repack
kernel runs first), then for each case captures one op call as the first call of its kernel
instance, replays the graph on new activations twice and compares both replays with an eager call
on the same activations: bit-identical. Needs an MI355X.
"""

import os
import subprocess
import sys

import pytest
from conftest import ORACLE, PKG_ROOT, ROOT

pytestmark = pytest.mark.gpu

CHILD = r"""
import ctypes, sys
import numpy as np
import torch
sys.path[:0] = [PKG_ROOT, ORACLE, TESTS]
import gguf_oracle as o
import _tile
from vllm_gguf_plugin import _capi, ops  # noqa: F401  loads the library and the ops: no GPU call
from vllm_gguf_plugin.quantization import linear

C = torch.ops._C_gguf
torch.zeros(1, device="cuda")  # the HIP context, but no library call before the captures
lib = _capi.load()

# (type, rows, k, n, packed): the routing table picks the op; the comments name the kernel plan
CASES = [
    (o.IQ3_S, 4096, 5120, 1, True),     # stream GEMV, X quantised in the kernel (bf16)
    (o.IQ3_S, 4096, 5120, 4, True),     # quantise + stream GEMV on q8_1
    (o.IQ3_S, 1024, 5120, 1, True),     # one-tile GEMV, X quantised block by block
    (o.IQ3_S, 1024, 5120, 3, True),     # quantise + one-tile GEMV
    (o.IQ3_S, 5120, 17408, 16, True),   # int8 tile GEMM with K split over workgroups
    (o.IQ3_S, 17408, 5120, 48, True),   # fp16 small GEMM, range plan (one workgroup per CU)
    (o.IQ3_S, 4096, 5120, 128, True),   # fp16 small GEMM
    (o.IQ3_S, 4096, 5120, 512, True),   # fp16 prefill GEMM
    (o.Q4_K, 5120, 17408, 16, False),   # int8 raw GEMM with K split
    (o.Q4_K, 4096, 5120, 1, False),     # row-chunk GEMV
    (o.Q6_K, 1024, 5120, 4, False),     # raw GEMV
    (o.IQ4_XS, 1024, 5120, 512, False), # int8 prefill GEMM
    (o.IQ2_S, 1024, 5120, 2, False),    # generic GEMV
    (o.IQ2_S, 1024, 5120, 16, False),   # generic MFMA GEMM
    (o.IQ3_S, 1024, 5120, 16, False),   # per-slice MFMA GEMM (unpacked IQ3_S)
    (o.Q4_K, 5120, 17408, 4, False),    # 4x4x4 MFMA GEMV, 97 KB of dynamic LDS (the attribute)
    (o.IQ4_XS, 1024, 17408, 3, False),  # 4x4x4 MFMA GEMV, 70 KB of dynamic LDS
    (o.Q4_K, 1024, 17408, 1, False),    # 4x4x4 MFMA GEMV at one row (K > 8192)
    (o.IQ2_XS, 1024, 17408, 3, False),  # generic stream GEMV, 65 KB of dynamic LDS
    (o.IQ3_XXS, 1024, 17408, 3, True),  # IQ3 stream GEMV on the IQ3_XXS unit layout, 82 KB of LDS
    (o.IQ3_XXS, 4096, 5120, 1, True),   # the same, X quantised in the kernel
    (o.IQ3_XXS, 1024, 5120, 16, True),  # generic GEMM staging the IQ3_XXS unit layout
    (o.IQ2_XXS, 1024, 2048, 1, False),  # generic stream GEMV, X quantised in the kernel
]

fails = []
for i, (qt, rows, k, n, packed) in enumerate(CASES):
    raw = o.random_blocks(np.random.default_rng(i), qt, rows, k)
    if packed:
        raw = _tile.pack_xxs(raw) if qt == o.IQ3_XXS else _tile.pack(raw)
    w = torch.from_numpy(raw).cuda()
    g = torch.Generator().manual_seed(100 + i)
    x1, x2 = (torch.randn(n, k, generator=g).bfloat16().cuda() for _ in range(2))
    op = getattr(C, linear._lcpp_op(n, qt, rows, k, packed))
    print(f"case {i}: type {qt} {rows}x{k} n={n} {op.__name__}", flush=True)
    static_x = x1.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_y = op(w, static_x, qt, rows)  # the first call of this kernel instance
    static_x.copy_(x2)
    graph.replay()
    torch.cuda.synchronize()
    first = static_y.clone()
    graph.replay()
    torch.cuda.synchronize()
    eager = op(w, x2, qt, rows)
    torch.cuda.synchronize()
    if not (torch.equal(first, eager) and torch.equal(static_y, eager)):
        fails.append(f"case {i}")
    del graph, static_y, first, eager

# the no-allocation entry point: its scratch address looked up inside the capture
qt, rows, k, n = o.IQ3_S, 4096, 5120, 4
print("case noalloc", flush=True)
w = torch.from_numpy(_tile.pack(o.random_blocks(np.random.default_rng(99), qt, rows, k))).cuda()
x2 = torch.randn(n, k, generator=torch.Generator().manual_seed(7)).bfloat16().cuda()
static_x = torch.zeros_like(x2)
y = torch.empty(n, rows, dtype=torch.bfloat16, device="cuda")
wv, xv = _capi.view(w), _capi.view(static_x)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = lib.gguf_mul_mat_noalloc(6, _capi.ref(wv), _capi.ref(xv), qt, rows, None, y.data_ptr(),
                                  y.numel() * 2, torch.cuda.current_stream().cuda_stream)
assert rc == 0, _capi.error(lib)
static_x.copy_(x2)
graph.replay()
torch.cuda.synchronize()
if not torch.equal(y, C.lcpp_mul_mat_vec_iq3_mma_packed(w, x2, qt, rows)):
    fails.append("noalloc")
print("FAILS", fails, flush=True)
"""


def test_first_call_of_every_kernel_family_inside_capture():
    src = (f"PKG_ROOT, ORACLE, TESTS = {PKG_ROOT!r}, {ORACLE!r}, {os.path.join(ROOT, 'tests')!r}\n" + CHILD)
    p = subprocess.run([sys.executable, "-u", "-c", src], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ))
    print(p.stdout[-3000:])
    assert p.returncode == 0, p.stdout[-1500:] + p.stderr[-3000:]
    assert "FAILS []" in p.stdout, p.stdout[-2000:]
