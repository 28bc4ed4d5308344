"""ctypes binding of libgguf_mi355x.so, the C ABI declared in include/gguf_mi355x.h.

The library is the product: there is no CPU or PyTorch fallback. load() raises if the built
library is missing, and every call that the library rejects raises RuntimeError with the
library's message (the reference's guard messages, lcpp_shim.cu:690-791).
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgguf_mi355x.so")

GGUF_OK, GGUF_EINVAL, GGUF_EHIP = 0, 1, 2
DT_F32, DT_F16, DT_BF16, DT_U8, DT_OTHER = 0, 1, 2, 3, 4
_DT = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16, torch.uint8: DT_U8}

# op ids (gguf_mi355x.h), by the reference's op names (lcpp_shim.cu:973-983)
OPS = {
    "lcpp_mul_mat_vec_q": 0,
    "lcpp_mul_mat_q": 1,
    "lcpp_mul_mat_vec_iq3": 2,
    "lcpp_mul_mat_vec_iq3_mma": 3,
    "lcpp_mul_mat_vec_own": 4,
    "lcpp_mul_mat_mma_k": 5,
    "lcpp_mul_mat_vec_iq3_mma_packed": 6,
    "lcpp_mul_mat_iq3_packed": 7,
}

# every symbol include/gguf_mi355x.h declares
EXPORTS = (
    "gguf_last_error", "gguf_version", "gguf_check_op", "gguf_op_workspace_bytes", "gguf_mul_mat",
    "gguf_lcpp_mul_mat_vec_q", "gguf_lcpp_mul_mat_q", "gguf_lcpp_mul_mat_vec_iq3",
    "gguf_lcpp_mul_mat_vec_iq3_mma", "gguf_lcpp_mul_mat_vec_own", "gguf_lcpp_mul_mat_mma_k",
    "gguf_lcpp_mul_mat_vec_iq3_mma_packed", "gguf_lcpp_mul_mat_iq3_packed", "gguf_q8_1_bytes",
    "gguf_lcpp_quantize_q8_1", "gguf_iq3_pack_scratch_bytes", "gguf_iq3_pack", "gguf_scratch_bytes",
    "gguf_mul_mat_noalloc", "gguf_dense_mul_mat", "gguf_mul_mat_alloc",
)


class View(ctypes.Structure):
    """struct gguf_view: a strided 1-D/2-D tensor as the guards see it."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("size", ctypes.c_int64 * 2),
        ("stride", ctypes.c_int64 * 2),
        ("device", ctypes.c_int32),
    ]


# gguf_alloc_fn: void* (*)(void* ctx, int what, size_t bytes)
ALLOC_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t)
ALLOC_OUTPUT, ALLOC_WORKSPACE = 0, 1

_lib = None


def load():
    """The loaded library (ctypes.CDLL), loaded once. Raises ImportError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run vllm-gsqrco-exl3_amd/build.py "
                          "(or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    P, I64, I32, SZ, VP = ctypes.POINTER(View), ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
    lib.gguf_last_error.restype = ctypes.c_char_p
    lib.gguf_version.restype = ctypes.c_char_p
    lib.gguf_check_op.argtypes = [I32, P, P, I64, I64, P]
    lib.gguf_op_workspace_bytes.argtypes = [I32, I64, I64, I64, I64, I32]
    lib.gguf_op_workspace_bytes.restype = SZ
    lib.gguf_mul_mat.argtypes = [I32, P, P, I64, I64, P, VP, SZ, VP, SZ, VP]
    lib.gguf_q8_1_bytes.argtypes = [I64, I64, I32]
    lib.gguf_q8_1_bytes.restype = SZ
    lib.gguf_lcpp_quantize_q8_1.argtypes = [P, I64, I32, I32, VP, SZ, VP]
    lib.gguf_iq3_pack_scratch_bytes.argtypes = [I64, I64]
    lib.gguf_iq3_pack_scratch_bytes.restype = SZ
    lib.gguf_iq3_pack.argtypes = [VP, I64, I64, I64, I32, VP, SZ, VP]
    lib.gguf_scratch_bytes.restype = SZ
    lib.gguf_mul_mat_noalloc.argtypes = [I32, P, P, I64, I64, P, VP, SZ, VP]
    lib.gguf_dense_mul_mat.argtypes = [P, P, VP, SZ, VP]
    lib.gguf_mul_mat_alloc.argtypes = [I32, P, P, I64, I64, P, ALLOC_FN, VP, VP]
    _lib = lib
    return lib


def view(t: torch.Tensor | None):
    """gguf_view of a tensor (None -> NULL pointer). Host tensors get device -1."""
    if t is None:
        return None
    v = View()
    v.data = t.data_ptr() if t.numel() else (t.data_ptr() or None)
    v.dtype = _DT.get(t.dtype, DT_OTHER)
    v.ndim = t.dim()
    for i in range(min(2, t.dim())):
        v.size[i] = t.shape[i]
        v.stride[i] = t.stride(i)
    v.device = t.device.index if t.is_cuda else -1
    if t.is_cuda and v.device is None:
        v.device = torch.cuda.current_device()
    return v


def ref(v):
    return ctypes.byref(v) if v is not None else None


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def error(lib) -> str:
    return (lib.gguf_last_error() or b"").decode()


def check(lib, rc: int) -> None:
    if rc != GGUF_OK:
        raise RuntimeError(error(lib))
