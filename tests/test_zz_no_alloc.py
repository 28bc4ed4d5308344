"""gguf_mul_mat_noalloc (the entry point that allocates nothing: its workspace is the library's
static per-GPU scratch) against gguf_mul_mat with a caller workspace, through the C ABI: bit-exact
outputs on two calls in a row, the second on a smaller input (the scratch keeps the first call's
bytes), for the decode GEMV, the int8-MFMA small GEMMs, the fp16 small GEMM and a caller's x_q8;
and a product whose workspace exceeds the scratch is rejected with a clear error. Needs an MI355X.
"""

import ctypes

import numpy as np
import pytest
import torch

import gguf_oracle as o
from _gpu import dev, w_rand, x_rand

pytestmark = pytest.mark.gpu

PACKED_VEC, PACKED_TILED, MUL_MAT_Q, MMA_K, VEC_Q = 6, 7, 1, 5, 0


@pytest.fixture(scope="module")
def lib():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from vllm_gguf_plugin import _capi, ops  # noqa: F401

    return _capi.load()


def _run(lib, entry, op, w, x, qt, rows, x_q8=None):
    """One product through the C ABI: entry 'workspace' (gguf_mul_mat with a fresh workspace of
    the size the library asks for) or 'noalloc' (gguf_mul_mat_noalloc)."""
    from vllm_gguf_plugin import _capi

    n, k = x.shape
    y = torch.full((n, rows), float("nan"), dtype=x.dtype, device="cuda")
    wv, xv, qv = _capi.view(w), _capi.view(x), _capi.view(x_q8)
    stream = torch.cuda.current_stream().cuda_stream
    if entry == "noalloc":
        rc = lib.gguf_mul_mat_noalloc(op, _capi.ref(wv), _capi.ref(xv), qt, rows, _capi.ref(qv), y.data_ptr(),
                                      y.numel() * y.element_size(), stream)
    else:
        nb = lib.gguf_op_workspace_bytes(op, qt, rows, k, n, int(x_q8 is not None))
        ws = torch.full((max(nb, 1),), 0xFF, dtype=torch.uint8, device="cuda")
        rc = lib.gguf_mul_mat(op, _capi.ref(wv), _capi.ref(xv), qt, rows, _capi.ref(qv), y.data_ptr(),
                              y.numel() * y.element_size(), ws.data_ptr(), nb, stream)
    assert rc == 0, _capi.error(lib)
    torch.cuda.synchronize()
    return y


CASES = [
    # (op, type, rows, k, first n, second n)
    (PACKED_VEC, o.IQ3_S, 17408, 5120, 4, 1),      # quantise + packed GEMV (q8_1 copy in scratch)
    (PACKED_VEC, o.IQ3_S, 6144, 5120, 16, 8),      # decode op on the int8 GEMM (xq in scratch)
    (PACKED_TILED, o.IQ3_S, 5120, 17408, 64, 33),  # product op, int8 small GEMM at K = 17408
    (PACKED_TILED, o.IQ3_S, 6144, 5120, 128, 64),  # fp16 small GEMM (xh in scratch)
    (MMA_K, o.Q4_K, 17408, 5120, 32, 9),
    (MUL_MAT_Q, o.Q6_K, 5120, 6144, 48, 17),
    (VEC_Q, o.IQ4_XS, 4096, 4096, 8, 3),
]


@pytest.mark.parametrize("op,qt,rows,k,n1,n2", CASES)
def test_noalloc_equals_workspace_entry(lib, op, qt, rows, k, n1, n2):
    from vllm_gguf_plugin.quantization import iq3_pack

    w = dev(w_rand(qt, rows, k, seed=op * 10 + qt))
    if op in (PACKED_VEC, PACKED_TILED):
        w = iq3_pack.pack(w, qt)
    for call, n in enumerate((n1, n2)):
        x = x_rand(n, k, seed=100 * call + n, dtype=torch.bfloat16).cuda()
        a = _run(lib, "noalloc", op, w, x, qt, rows)
        b = _run(lib, "workspace", op, w, x, qt, rows)
        assert torch.equal(a, b), (call, n)
        assert not torch.isnan(a.float()).any()


def test_noalloc_with_caller_x_q8(lib):
    """A caller's x_q8 through the no-allocation entry: the decode GEMV reads it directly, the
    GEMM converts it into its layout in the scratch (8 rows); both equal the workspace entry."""
    w = dev(w_rand(o.Q4_K, 4096, 5120, seed=5))
    for n in (8, 2):
        x = x_rand(n, 5120, seed=n, dtype=torch.bfloat16).cuda()
        q8 = torch.ops._C_gguf.lcpp_quantize_q8_1(x, o.Q4_K, False, False)
        a = _run(lib, "noalloc", VEC_Q, w, x, o.Q4_K, 4096, q8)
        b = _run(lib, "workspace", VEC_Q, w, x, o.Q4_K, 4096, q8)
        assert torch.equal(a, b), n


def test_noalloc_rejects_workspace_beyond_scratch(lib):
    from vllm_gguf_plugin import _capi

    rows, k, n = 5120, 5120, 2048  # a prefill: its fp16 activation copy is 2048/16 * 20 * 9216 B
    need = lib.gguf_op_workspace_bytes(MUL_MAT_Q, o.Q4_K, rows, k, n, 0)
    assert need > lib.gguf_scratch_bytes()
    w = dev(w_rand(o.Q4_K, rows, k, seed=6))
    x = torch.zeros(n, k, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(n, rows, dtype=torch.bfloat16, device="cuda")
    rc = lib.gguf_mul_mat_noalloc(MUL_MAT_Q, _capi.ref(_capi.view(w)), _capi.ref(_capi.view(x)), o.Q4_K, rows,
                                  None, y.data_ptr(), y.numel() * 2, torch.cuda.current_stream().cuda_stream)
    assert rc == _capi.GGUF_EINVAL
    msg = _capi.error(lib)
    assert "static scratch" in msg and str(need) in msg, msg
