"""The routing decisions of the linear method, driven by the case table
tests/golden/routing_cases.json (the reference's routing cases, cited in the file):
  * op_cases: the Route L op name _lcpp_op gives per (type, activation rows, weight rows, K,
    packed), at every boundary of the table;
  * shared_q8_1_cases: which run's type apply()'s single q8_1 quantisation of X is made for, or
    none when every run's op quantises X itself.
Plus the rules around them: the empty product, an unserved type, and the fp32-dst chunk size.
"""

import json
import os

import pytest
import torch
from conftest import GOLDEN

from vllm_gguf_plugin.quantization import linear
from vllm_gguf_plugin.quantization.utils import WeightType

with open(os.path.join(GOLDEN, "routing_cases.json")) as _f:
    _DOC = json.load(_f)
OP_CASES = _DOC["op_cases"]
SHARED = _DOC["shared_q8_1_cases"]


def _tid(c):
    return f"{c['type']}-n{c['n']}-r{c['rows']}-k{c['k']}{'-packed' if c['packed'] else ''}"


@pytest.mark.parametrize("case", OP_CASES, ids=_tid)
def test_op_case(case):
    t = int(WeightType[case["type"]])
    got = linear._lcpp_op(case["n"], t, case["rows"], case["k"], case["packed"])
    assert got == case["op"]
    if not case["packed"]:  # the default argument is the unpacked table
        assert linear._lcpp_op(case["n"], t, case["rows"], case["k"]) == got


def test_op_table_size_and_reach():
    """84 unpacked and 36 packed cases, and every op name of the table appears in them."""
    packed = [c for c in OP_CASES if c["packed"]]
    assert (len(OP_CASES) - len(packed), len(packed)) == (84, 36)
    assert {c["op"] for c in OP_CASES} == {
        "lcpp_mul_mat_vec_q", "lcpp_mul_mat_q", "lcpp_mul_mat_vec_iq3", "lcpp_mul_mat_vec_iq3_mma",
        "lcpp_mul_mat_vec_own", "lcpp_mul_mat_mma_k", "lcpp_mul_mat_vec_iq3_mma_packed", "lcpp_mul_mat_iq3_packed",
        None}


@pytest.mark.parametrize("case", SHARED, ids=lambda c: f"n{c['n']}-{'+'.join(c['types'])}-{c['packed']}")
def test_shared_q8_1_type(case):
    from vllm_gguf_plugin import ops

    types = [int(WeightType[t]) for t in case["types"]]
    assert all(t in ops.LCPP_QUANT_TYPES for t in types)
    want = case["quantize_as"]
    got = linear._q8_1_type(case["n"], 512, types, case["rows"], case["packed"])
    assert got == (None if want is None else int(WeightType[want]))


def test_unquantized_shared_buffer_has_q8_1_size():
    """When no run's op reads q8_1, _quantize_x_q8_1 returns an unfilled buffer of the q8_1 size
    (n * K / 32 blocks of 36 bytes) and launches nothing (host x: no kernel can run)."""
    for n, types, rows in ((9, ["IQ3_S", "Q4_K"], [17408, 17408]), (0, ["IQ3_S"], [17408])):
        x = torch.zeros(n, 1024, dtype=torch.bfloat16)
        out = linear._quantize_x_q8_1(x, [int(WeightType[t]) for t in types], rows)
        assert out.dtype == torch.uint8 and out.shape == (n * 1024 // 32 * 36,)


def test_empty_product_launches_nothing():
    """No activation rows: an empty [0, weight rows] result in X's dtype before any routing (host
    tensors, so any launch would fail)."""
    w = torch.zeros(17408, 2 * 110, dtype=torch.uint8)
    for packed in (False, True):
        y = linear._fused_mul_mat_gguf(torch.zeros(0, 512, dtype=torch.float16), w, int(WeightType.IQ3_S), None,
                                       packed)
        assert y.shape == (0, 17408) and y.dtype == torch.float16


def test_served_types_are_the_route_l_set():
    """Every Route L type of the reference (ops.py:96-110) is served."""
    from vllm_gguf_plugin import ops

    names = {"Q2_K", "Q4_K", "Q6_K", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S", "IQ4_XS", "IQ1_M"}
    assert {WeightType(t).name for t in ops.LCPP_QUANT_TYPES} == names


def test_unserved_type_is_refused():
    """A quantized type outside the Route L set raises NotImplementedError naming it."""
    x = torch.zeros(2, 512, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="IQ1_S"):
        linear._fused_mul_mat_gguf(x, torch.zeros(64, 2 * 50, dtype=torch.uint8), int(WeightType.IQ1_S))


def test_fp32_dst_chunk_rows():
    """A product whose fp32 dst would pass _FP32_DST_BUDGET (256 MiB) runs in activation-row chunks
    of the largest multiple of 128 that fits (reference linear.py:117-130): 384 for a 151936-row
    vocab head, and whole below 442 rows."""
    rows = 151936
    assert linear._FP32_DST_BUDGET == 256 << 20
    fits = linear._FP32_DST_BUDGET // (rows * 4)
    assert fits == 441 and fits - fits % 128 == 384
    assert 441 * rows * 4 <= linear._FP32_DST_BUDGET < 442 * rows * 4
