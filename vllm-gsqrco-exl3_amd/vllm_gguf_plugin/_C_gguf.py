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

Implementations are registered for CUDA (HIP tensors on ROCm) and, as in the reference
(lcpp_shim.cu:997-1008), for CPU: there every guard runs in the library and the call then ends
with "must be CUDA tensors", so the guards are testable without a GPU. Each op returns a new
[n, row] tensor in X's dtype, allocated with torch's caching allocator, as is the workspace
(the q8_1 copy of X), so calls are safe under CUDA-graph capture.
"""

from __future__ import annotations

import torch

from . import _capi

NAMESPACE = "_C_gguf"

_SCHEMAS = {
    "lcpp_mul_mat_vec_q": "(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor",
    "lcpp_mul_mat_q": "(Tensor W, Tensor X, int type, SymInt row) -> Tensor",
    "lcpp_mul_mat_vec_iq3": "(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor",
    "lcpp_mul_mat_vec_iq3_mma": "(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor",
    "lcpp_mul_mat_vec_own": "(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor",
    "lcpp_mul_mat_mma_k": "(Tensor W, Tensor X, int type, SymInt row) -> Tensor",
    "lcpp_mul_mat_vec_iq3_mma_packed": "(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor",
    "lcpp_mul_mat_iq3_packed": "(Tensor W, Tensor X, int type, SymInt row) -> Tensor",
}
QUANTIZE_SCHEMA = "(Tensor X, int type, bool mmq, bool vendored) -> Tensor"


def mul_mat(name: str, W: torch.Tensor, X: torch.Tensor, type: int, row: int,
            x_q8: torch.Tensor | None = None) -> torch.Tensor:
    """One product through the C ABI: Y[n, row] = X @ W[:row].T in X's dtype."""
    lib = _capi.load()
    op = _capi.OPS[name]
    wv, xv, qv = _capi.view(W), _capi.view(X), _capi.view(x_q8)
    _capi.check(lib, lib.gguf_check_op(op, _capi.ref(wv), _capi.ref(xv), int(type), int(row), _capi.ref(qv)))
    n, k = X.shape
    y = torch.empty(n, row, dtype=X.dtype, device=X.device)
    if n == 0:
        return y
    wsb = lib.gguf_op_workspace_bytes(op, int(type), int(row), k, n, int(x_q8 is not None))
    ws = torch.empty(wsb, dtype=torch.uint8, device=X.device) if wsb else None
    rc = lib.gguf_mul_mat(op, _capi.ref(wv), _capi.ref(xv), int(type), int(row), _capi.ref(qv),
                          y.data_ptr(), y.numel() * y.element_size(),
                          ws.data_ptr() if ws is not None else None, wsb, _capi.stream_of(X))
    _capi.check(lib, rc)
    return y


def quantize_q8_1(X: torch.Tensor, type: int, mmq: bool, vendored: bool) -> torch.Tensor:
    """X -> q8_1 bytes (block_q8_1, or block_q8_1_mmq when mmq), as lcpp_quantize_q8_1."""
    lib = _capi.load()
    xv = _capi.view(X)
    nbytes = lib.gguf_q8_1_bytes(X.shape[0], X.shape[1], int(mmq)) if X.dim() == 2 else 0
    out = torch.empty(nbytes, dtype=torch.uint8, device=X.device)
    rc = lib.gguf_lcpp_quantize_q8_1(_capi.ref(xv), int(type), int(mmq), int(vendored),
                                     out.data_ptr() if nbytes else None, nbytes,
                                     _capi.stream_of(X) if X.is_cuda else None)
    _capi.check(lib, rc)
    return out


def _make_impl(name):
    if "x_q8" in _SCHEMAS[name]:
        def impl(W, X, type, row, x_q8=None):
            return mul_mat(name, W, X, type, row, x_q8)
    else:
        def impl(W, X, type, row):
            return mul_mat(name, W, X, type, row)
    impl.__name__ = name
    return impl


def _make_fake(name):
    if "x_q8" in _SCHEMAS[name]:
        def fake(W, X, type, row, x_q8=None):
            return X.new_empty(X.shape[0], row)
    else:
        def fake(W, X, type, row):
            return X.new_empty(X.shape[0], row)
    return fake


def _quantize_fake(X, type, mmq, vendored):
    n, k = X.shape
    return X.new_empty((n * k // 128 * 144) if mmq else (n * k // 32 * 36), dtype=torch.uint8)


_lib = None


def register() -> None:
    """Define and implement the ops once per process (import time of vllm_gguf_plugin.ops)."""
    global _lib
    if _lib is not None:
        return
    _capi.load()  # fail loudly if the native library is missing: no fallback path exists
    lib = torch.library.Library(NAMESPACE, "FRAGMENT")
    for name, schema in _SCHEMAS.items():
        lib.define(name + schema)
        impl = _make_impl(name)
        lib.impl(name, impl, "CUDA")
        lib.impl(name, impl, "CPU")
        torch.library.register_fake(f"{NAMESPACE}::{name}", _make_fake(name), lib=lib)
    lib.define("lcpp_quantize_q8_1" + QUANTIZE_SCHEMA)
    lib.impl("lcpp_quantize_q8_1", quantize_q8_1, "CUDA")
    lib.impl("lcpp_quantize_q8_1", quantize_q8_1, "CPU")
    torch.library.register_fake(f"{NAMESPACE}::lcpp_quantize_q8_1", _quantize_fake, lib=lib)
    _lib = lib
