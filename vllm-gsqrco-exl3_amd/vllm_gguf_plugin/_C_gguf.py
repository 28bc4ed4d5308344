"""torch.ops._C_gguf: the reference's Route L op surface, served by libgguf_mi355x.so.

Same namespace, op names and schemas as the reference's registration
(plugin/vllm_gguf_plugin/csrc/lcpp_shim.cu:973-983), so plugin code that calls
torch.ops._C_gguf.<op> runs unchanged:

  lcpp_mul_mat_vec_q(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor
  lcpp_mul_mat_q(Tensor W, Tensor X, int type, SymInt row) -> Tensor
  lcpp_mul_mat_vec_iq3(...,  Tensor? x_q8=None) -> Tensor
  lcpp_mul_mat_vec_iq3_mma(..., Tensor? x_q8=None) -> Tensor
  lcpp_mul_mat_vec_own(..., Tensor? x_q8=None) -> Tensor
  lcpp_mul_mat_mma_k(Tensor W, Tensor X, int type, SymInt row) -> Tensor
  lcpp_mul_mat_vec_iq3_mma_packed(..., Tensor? x_q8=None) -> Tensor
  lcpp_mul_mat_iq3_packed(Tensor W, Tensor X, int type, SymInt row) -> Tensor
  lcpp_quantize_q8_1(Tensor X, int type, bool mmq, bool vendored) -> Tensor

and this build's own dense_mul_mat(Tensor W, Tensor X) -> Tensor, the small unquantized product of
quantization/linear.py's _unquantized_gemm.

The ops are defined and implemented in C++ (csrc/torch_ops.cpp, built into _C_gguf_ops.so next
to the library): for CUDA (HIP tensors on ROCm) and, as in the reference (lcpp_shim.cu:997-1008),
for CPU, where every guard runs in the library and the call then ends with "must be CUDA
tensors", so the guards are testable without a GPU. Each op returns a new [n, row] tensor in X's
dtype, allocated with torch's caching allocator, as is the workspace (the q8_1 copy of X), so
calls are safe under CUDA-graph capture. This module loads that registration and adds the fake
(meta) implementations torch.compile needs.
"""

from __future__ import annotations

import os

import torch

from . import _capi

NAMESPACE = "_C_gguf"
OPS_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_C_gguf_ops.so")

_Q8_OPS = ("lcpp_mul_mat_vec_q", "lcpp_mul_mat_vec_iq3", "lcpp_mul_mat_vec_iq3_mma", "lcpp_mul_mat_vec_own",
           "lcpp_mul_mat_vec_iq3_mma_packed")
_OWN_OPS = ("lcpp_mul_mat_q", "lcpp_mul_mat_mma_k", "lcpp_mul_mat_iq3_packed")


def _fake_q8(W, X, type, row, x_q8=None):
    return X.new_empty(X.shape[0], row)


def _fake_own(W, X, type, row):
    return X.new_empty(X.shape[0], row)


def _dense_fake(W, X):
    return X.new_empty(X.shape[0], W.shape[0])


def _quantize_fake(X, type, mmq, vendored):
    n, k = X.shape
    return X.new_empty((n * k // 128 * 144) if mmq else (n * k // 32 * 36), dtype=torch.uint8)


_registered = False


def register() -> None:
    """Load the ops once per process (import time of vllm_gguf_plugin.ops). Raises if the native
    library or its op registration is not built: there is no fallback path."""
    global _registered
    if _registered:
        return
    _capi.load()
    if not os.path.exists(OPS_LIB):
        raise ImportError(f"{OPS_LIB} is not built: run vllm-gsqrco-exl3_amd/build.py "
                          "(or __graft_entry__.build())")
    torch.ops.load_library(OPS_LIB)
    for name in _Q8_OPS:
        torch.library.register_fake(f"{NAMESPACE}::{name}", _fake_q8)
    for name in _OWN_OPS:
        torch.library.register_fake(f"{NAMESPACE}::{name}", _fake_own)
    torch.library.register_fake(f"{NAMESPACE}::lcpp_quantize_q8_1", _quantize_fake)
    torch.library.register_fake(f"{NAMESPACE}::dense_mul_mat", _dense_fake)
    _registered = True
