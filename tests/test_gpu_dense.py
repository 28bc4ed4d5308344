"""The small dense product of the GGUF file's F32/F16/BF16 tensors (torch.ops._C_gguf.dense_mul_mat,
gguf_dense_mul_mat) and the linear method's route to it (_unquantized_gemm), against a float64
reference of the same product. The reference routes these shapes to a batched GEMV
(quantization/linear.py:281-291) and tests the linear method's unquantized path the same way.
Needs an MI355X.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

BAR = {torch.float32: 1e-5, torch.float16: 2.5e-3, torch.bfloat16: 5e-3}  # Y rounded to X's dtype


@pytest.fixture(scope="module", autouse=True)
def _ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from vllm_gguf_plugin import ops  # noqa: F401


def _rel(y, ref):
    return float(((y.double() - ref).norm(dim=-1) / ref.norm(dim=-1).clamp_min(1e-30)).max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("n", [1, 3, 8])
@pytest.mark.parametrize("rows,k", [(96, 5120), (128, 6144), (1, 512), (300, 2048)])
def test_dense_mul_mat(dtype, n, rows, k):
    g = torch.Generator().manual_seed(rows + n)
    w = torch.randn(rows, k, generator=g).to(dtype).cuda()
    x = torch.randn(n, k, generator=g).to(dtype).cuda()
    y = torch.ops._C_gguf.dense_mul_mat(w, x)
    assert y.shape == (n, rows) and y.dtype == dtype
    ref = x.double() @ w.double().T
    assert _rel(y, ref) <= BAR[dtype]


def test_dense_strided_rows_and_guards():
    w = torch.randn(64, 1024 + 32, dtype=torch.bfloat16, device="cuda")[:, :1024]
    x = torch.randn(4, 1024 + 64, dtype=torch.bfloat16, device="cuda")[:, :1024]
    y = torch.ops._C_gguf.dense_mul_mat(w, x)
    assert _rel(y, x.double() @ w.double().T) <= BAR[torch.bfloat16]
    with pytest.raises(RuntimeError, match="at most 8 rows"):
        torch.ops._C_gguf.dense_mul_mat(w, torch.zeros(9, 1024, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(RuntimeError, match="one float dtype"):
        torch.ops._C_gguf.dense_mul_mat(w, x.float())
    with pytest.raises(RuntimeError, match="multiple of 32"):
        torch.ops._C_gguf.dense_mul_mat(w[:, :1000], x[:, :1000])
    assert torch.ops._C_gguf.dense_mul_mat(w, x[:0]).shape == (0, 64)


@pytest.mark.parametrize("n,rows,bias", [(4, 96, False), (8, 128, False), (9, 96, False), (2, 129, False),
                                         (2, 96, True)])
def test_unquantized_gemm_route(n, rows, bias):
    """_unquantized_gemm takes the dense kernel at <= 8 rows on <= 128-row weights without bias,
    torch's linear otherwise; both within the bf16 bar of the float64 product."""
    from vllm_gguf_plugin.quantization import linear

    w = torch.randn(rows, 2048, dtype=torch.bfloat16, device="cuda")
    x = torch.randn(n, 2048, dtype=torch.bfloat16, device="cuda")
    b = torch.randn(rows, dtype=torch.bfloat16, device="cuda") if bias else None
    assert linear._dense_ok(x, w, b) == (n <= 8 and rows <= 128 and not bias)
    y = linear._unquantized_gemm(x, w, b)
    ref = x.double() @ w.double().T + (b.double() if bias else 0)
    assert y.shape == (n, rows) and _rel(y, ref) <= 1e-2
    if linear._dense_ok(x, w, b):
        assert torch.equal(y, torch.ops._C_gguf.dense_mul_mat(w, x))
