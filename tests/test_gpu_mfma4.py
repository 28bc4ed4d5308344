"""The MFMA decode GEMV (csrc/gemv_mfma4.hip, gemv_mfma4_kernel): Q4_K, IQ4_XS and Q6_K decode
ops at 2-4 activation rows (Q4_K / IQ4_XS also at one row on K > 8192) on weights of at least one
4-row unit per CU, through the C ABI (torch.ops._C_gguf -> libgguf_mi355x.so); the one-row cases
at K <= 8192 and of Q6_K exercise the row-chunk GEMV. Needs an MI355X.

  * exact-integer mode (block scales 1, Q6_K sub-scales within +-31, X integers with every q8_1
    d = 1): every output equals the oracle's int64 sum of the slice terms (Q4_K
    sc * sumi - m * sum(q8), IQ4_XS ls * sumi, Q6_K sc_a * sumi_a + sc_b * sumi_b), at the configs' shapes
    17408 x 5120 and 5120 x 17408 (K blocks 20 and 68: 10 and 34 block pairs, 17 and 5 units per
    CU) and on smaller weights (one unit per CU, K = 1024 with two block pairs, K = 9216 at one
    row);
  * the q81 model (MMVQ form) at the full shapes with bf16 (5e-3: the output is rounded to bf16)
    and fp32 (1e-3) activations;
  * the caller's x_q8 (lcpp_mul_mat_vec_q with x_q8) gives the same bytes as X quantised by the op;
  * graph replays equal the eager call bit for bit.
"""

import numpy as np
import pytest
import torch

import gguf_oracle as o
from _gpu import TIGHT, C, dev, exact_ref, exact_weights, exact_x, graph_replays_equal, w_rand, x_rand

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from vllm_gguf_plugin import ops  # noqa: F401

    return torch.ops._C_gguf


TYPES = (o.Q4_K, o.IQ4_XS, o.Q6_K)
TN = {t: o.TYPE_NAMES[t] for t in TYPES}
# the decode ops each type is accepted by (lcpp_mul_mat_vec_own takes Q4_K and IQ2_S only)
OPS = {o.Q4_K: ("lcpp_mul_mat_vec_q", "lcpp_mul_mat_vec_own"), o.IQ4_XS: ("lcpp_mul_mat_vec_q",),
       o.Q6_K: ("lcpp_mul_mat_vec_q",)}


def _routed(qt):
    """The op the routing table (quantization/linear.py:_lcpp_op) picks at 3-4 rows."""
    return OPS[qt][-1]


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("rows,k", [(17408, 5120), (5120, 17408), (1024, 4096), (1024, 1024), (2064, 2560),
                                    (1024, 9216)])
@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_mfma4_exact_integer(qt, rows, k, n):
    raw = exact_weights(qt, rows, k, seed=300 + n + qt)
    w = dev(raw)
    x = exact_x(n, k, seed=301 + n, dtype=torch.float32)
    want = exact_ref(raw, qt, x)
    for op in OPS[qt]:
        y = getattr(C(), op)(w, x.cuda(), qt, rows).cpu().numpy()
        np.testing.assert_array_equal(y.astype(np.int64), want, err_msg=f"{op} n={n}")


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("rows,k", [(17408, 5120), (5120, 17408)])
@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_mfma4_full_size_q81(qt, rows, k, n):
    raw = w_rand(qt, rows, k, seed=310 + n + qt)
    w = dev(raw)
    x = x_rand(n, k, seed=311 + n)
    for dt in (torch.bfloat16, torch.float32):
        xd = x.to(dt)
        y = getattr(C(), _routed(qt))(w, xd.cuda(), qt, rows)
        assert y.dtype == dt and y.shape == (n, rows)
        err = o.rel_l2(y.float().cpu().numpy(), o.q81_model(raw, qt, xd, layout="mmvq"))
        assert err <= TIGHT[dt], (str(dt), err)


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [2, 4])
def test_mfma4_shared_x_q8(qt, n):
    rows, k = 17408, 5120
    w = dev(w_rand(qt, rows, k, seed=320 + n))
    x = x_rand(n, k, seed=321 + n, dtype=torch.bfloat16).cuda()
    xq = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)  # apply()'s shared q8_1, made for another type
    a = C().lcpp_mul_mat_vec_q(w, x, qt, rows)
    b = C().lcpp_mul_mat_vec_q(w, x, qt, rows, xq)
    assert torch.equal(a, b)


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("rows,k", [(17408, 5120), (5120, 17408)])
def test_mfma4_graph_replay(qt, rows, k):
    w = dev(w_rand(qt, rows, k, seed=330))
    xs = {n: x_rand(n, k, seed=331 + n, dtype=torch.bfloat16).cuda() for n in (2, 3, 4)}
    op = getattr(C(), _routed(qt))
    eager = torch.cat([op(w, xs[n], qt, rows).flatten() for n in xs])
    torch.cuda.synchronize()
    graph_replays_equal(lambda: torch.cat([op(w, xs[n], qt, rows).flatten() for n in xs]), eager)
