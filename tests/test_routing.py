"""The Route L op choice per (activation rows n, type, weight rows[, K]) at every boundary of the
reference's routing table (golden cases of tests/cpu/test_lcpp_routing.py:14-67), and the shared
q8_1 quantisation decision of apply() (:70-127), on this build's linear.py."""

import pytest
import torch

from vllm_gguf_plugin.quantization import linear
from vllm_gguf_plugin.quantization.utils import WeightType as T

IQ3, MMA, OWN = "lcpp_mul_mat_vec_iq3", "lcpp_mul_mat_vec_iq3_mma", "lcpp_mul_mat_vec_own"
MMVQ, MMQ, MMA_K = "lcpp_mul_mat_vec_q", "lcpp_mul_mat_q", "lcpp_mul_mat_mma_k"
PACKED_VEC, PACKED_TILED = "lcpp_mul_mat_vec_iq3_mma_packed", "lcpp_mul_mat_iq3_packed"
BIG = 17408
K = 5120

CASES = [
    *[(t, n, rows, want) for t in (T.IQ3_S, T.IQ3_XXS) for rows in (1024, BIG)
      for n, want in ((1, IQ3), (5, IQ3), (6, MMA), (8, MMA), (9, MMQ))],
    (T.Q4_K, 1, BIG, MMVQ), (T.Q4_K, 2, BIG, MMVQ), (T.Q4_K, 3, BIG, OWN), (T.Q4_K, 8, BIG, OWN),
    (T.Q4_K, 9, BIG, MMA_K), (T.Q4_K, 32, BIG, MMA_K), (T.Q4_K, 33, BIG, MMQ),
    (T.Q4_K, 3, 2049, OWN), (T.Q4_K, 9, 2049, MMA_K),
    (T.IQ2_S, 1, BIG, OWN), (T.IQ2_S, 8, BIG, OWN), (T.IQ2_S, 9, BIG, MMA_K), (T.IQ2_S, 32, BIG, MMA_K),
    (T.IQ2_S, 33, BIG, MMQ), (T.IQ2_S, 1, 2049, OWN), (T.IQ2_S, 32, 2049, MMA_K),
    (T.IQ4_XS, 7, BIG, MMVQ), (T.IQ4_XS, 8, BIG, MMQ), (T.IQ4_XS, 9, 2049, MMA_K),
    (T.IQ4_XS, 16, 2049, MMA_K), (T.IQ4_XS, 17, 2049, MMQ), (T.IQ4_XS, 17, BIG, MMA_K),
    (T.IQ4_XS, 32, BIG, MMA_K), (T.IQ4_XS, 33, BIG, MMQ),
    (T.IQ4_XS, 17, 12288, MMA_K), (T.IQ4_XS, 17, 12032, MMQ), (T.IQ4_XS, 17, (6144, 2 * K), MMA_K),
    (T.Q4_K, 4, 2048, MMVQ), (T.Q4_K, 8, 2048, MMQ), (T.IQ2_S, 1, 2048, MMVQ), (T.IQ2_S, 8, 2048, MMQ),
    (T.Q4_K, 9, 2048, MMQ), (T.IQ2_S, 32, 2048, MMQ), (T.IQ4_XS, 9, 2048, MMQ),
    *[(t, n, BIG, want) for t in (T.Q2_K, T.Q6_K, T.IQ2_XXS, T.IQ2_XS)
      for n, want in ((1, MMVQ), (7, MMVQ), (8, MMQ), (9, MMQ), (32, MMQ))],
    *[(T.IQ1_M, n, rows, want) for rows in (1024, BIG)
      for n, want in ((1, MMVQ), (8, MMVQ), (9, MMVQ), (32, MMVQ), (33, None))],
]


@pytest.mark.parametrize("qt,n,rows,want", CASES, ids=lambda v: getattr(v, "name", str(v)))
def test_lcpp_op(qt, n, rows, want):
    rows, k = rows if isinstance(rows, tuple) else (rows, K)
    assert linear._lcpp_op(n, int(qt), rows, k) == want
    assert linear._lcpp_op(n, int(qt), rows, k, False) == want


PACKED_CASES = [
    *[(t, n, rows, want) for t in (T.IQ3_S, T.IQ3_XXS) for rows in (1024, BIG)
      for n, want in ((1, PACKED_VEC), (5, PACKED_VEC), (6, PACKED_VEC), (8, PACKED_VEC),
                      (9, PACKED_TILED), (32, PACKED_TILED), (128, PACKED_TILED), (2048, PACKED_TILED))],
    (T.Q4_K, 3, BIG, OWN), (T.Q4_K, 9, BIG, MMA_K), (T.IQ4_XS, 8, BIG, MMQ), (T.IQ1_M, 9, BIG, MMVQ),
]


@pytest.mark.parametrize("qt,n,rows,want", PACKED_CASES, ids=lambda v: getattr(v, "name", str(v)))
def test_lcpp_op_packed(qt, n, rows, want):
    assert linear._lcpp_op(n, int(qt), rows, K, True) == want


def test_case_count():
    # the reference's 84 unpacked and 36 packed (type, n, rows) cases, all kept
    assert (len(CASES), len(PACKED_CASES)) == (84, 36)


class _Quantizer:
    """Stands in for torch.ops._C_gguf: records which type the shared quantize runs with."""

    def __init__(self):
        self.calls = []

    def lcpp_quantize_q8_1(self, x, qt, mmq, vendored):
        self.calls.append((qt, mmq, vendored))
        return "filled"


# The reference's cases (tests/cpu/test_lcpp_routing.py:81-92), restricted to runs of the types
# this build serves (Route L here serves Q4_K, Q6_K, IQ3_S and IQ4_XS): runs of IQ2_XS / IQ1_M
# route to no op in this build, so they never ask for the shared q8_1.
@pytest.mark.parametrize("n,types,rows,want", [
    (4, [T.Q4_K, T.IQ4_XS], [2048, BIG], T.Q4_K),      # first run that reads q8_1
    (8, [T.Q4_K], [BIG], T.Q4_K),                      # the Q4_K decode op reads it at 8 rows
    (8, [T.Q4_K], [2048], None),                       # MMQ quantizes for itself
    (8, [T.IQ4_XS, T.Q4_K], [BIG, BIG], T.Q4_K),       # MMQ beside the Q4_K decode op
    (8, [T.Q4_K, T.IQ3_S], [2048, BIG], T.IQ3_S),      # MMQ beside the IQ3 decode op
    (9, [T.IQ3_S, T.Q4_K], [BIG, BIG], None),          # MMQ and mma_k quantize for themselves
    (4, [T.Q6_K], [BIG], T.Q6_K),                      # Q6_K on the decode op
    (0, [T.IQ3_S], [BIG], None),                       # no rows: nothing to quantize
    (4, [T.IQ2_XS, T.Q4_K], [BIG, BIG], T.Q4_K),       # a type with no op here is skipped
], ids=lambda v: str(v) if not isinstance(v, list) else "+".join(getattr(t, "name", str(t)) for t in v))
def test_quantize_x_q8_1_fills(monkeypatch, n, types, rows, want, packed=False):
    q = _Quantizer()
    monkeypatch.setattr(torch.ops, "_C_gguf", q, raising=False)
    x = torch.zeros(n, 512, dtype=torch.bfloat16)
    out = linear._quantize_x_q8_1(x, [int(t) for t in types], rows, packed)
    if want is None:
        assert q.calls == [] and out.dtype == torch.uint8 and out.numel() == n * 512 // 32 * 36
    else:
        assert q.calls == [(int(want), False, False)] and out == "filled"


@pytest.mark.parametrize("n,types,rows,want", [
    (4, [T.IQ3_S, T.Q4_K], [BIG, BIG], T.IQ3_S),       # the packed decode op reads it
    (9, [T.IQ3_S, T.Q4_K], [BIG, BIG], None),          # tiled + mma_k
], ids=lambda v: str(v) if not isinstance(v, list) else "+".join(getattr(t, "name", str(t)) for t in v))
def test_quantize_x_q8_1_fills_packed(monkeypatch, n, types, rows, want):
    test_quantize_x_q8_1_fills(monkeypatch, n, types, rows, want, packed=True)


def test_fused_mul_mat_gguf_zero_rows():
    """0 activation rows return an empty [0, rows] result before any routing or launch."""
    y = linear._fused_mul_mat_gguf(torch.zeros(0, 512, dtype=torch.bfloat16),
                                   torch.zeros(BIG, 512 // 256 * 110, dtype=torch.uint8), int(T.IQ3_S))
    assert y.shape == (0, BIG) and y.dtype == torch.bfloat16


def test_unserved_type_raises():
    with pytest.raises(NotImplementedError):
        linear._fused_mul_mat_gguf(torch.zeros(2, 512, dtype=torch.bfloat16),
                                   torch.zeros(64, 512 // 256 * 82, dtype=torch.uint8), int(T.IQ2_S))


def test_chunk_rule_matches_reference_budget():
    """Products whose fp32 dst would pass 256 MiB run in 128-row multiples (linear.py:117-130)."""
    rows = 151936
    step = max(1, linear._FP32_DST_BUDGET // (rows * 4))
    assert step == 441 and step - step % 128 == 384
