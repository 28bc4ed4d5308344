"""Every cell of the benchmark configs that the other GPU tests cover only in part, through the
routing table's op (quantization/linear.py:_lcpp_op, the reference's linear.py:85-114), against
the oracle's q81 model in the op's activation layout. Needs an MI355X.

  * configs[2], the MTP verify small GEMM: IQ3_S (packed), IQ4_XS and Q6_K on q_proj 6144 x 5120,
    k/v_proj 1024 x 5120 and o_proj 5120 x 6144 at M = 4, 8, 16, 32, 48, with the config's bf16
    activations (5e-3 relative L2: the output is rounded to bf16) and with fp32 activations at the
    north star's 1e-3; every output row of the 1024-row weights, 384 sampled rows of the others;
    one graph-replay equality check per type and shape (the K-split and range plans depend on
    both).
  * configs[1], the decode GEMV: IQ3_S gate 17408 x 5120 and down 5120 x 17408 at M = 1 and 4
    with fp32 activations at 1e-3 (the bf16 runs are in test_gpu_parity.py and
    test_gpu_shapes.py).
  * configs[0], the CPU-path case: Q4_K 4096 x 4096 with the config's scale recipe
    (d, dmin ~ |N(0, 1e-3)|), fp32 X, through its routed op.
The decode ops (`lcpp_mul_mat_vec_*`) quantise X to block_q8_1 (the 'mmvq' model), the product
ops to block_q8_1_mmq (the 'mmq' model; Q4_K's min term in the MMQ form).
"""

import numpy as np
import pytest
import torch

import gguf_oracle as o
from _gpu import TIGHT, C, dev, graph_replays_equal

pytestmark = pytest.mark.gpu

MTP_TYPES = (o.IQ3_S, o.IQ4_XS, o.Q6_K)
MTP_SHAPES = ((6144, 5120), (1024, 5120), (5120, 6144))
MTP_ROWS = (4, 8, 16, 32, 48)


@pytest.fixture(scope="module", autouse=True)
def _ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from vllm_gguf_plugin import ops  # noqa: F401

    return torch.ops._C_gguf


_WEIGHTS = {}


def _weight(qt, rows, k, seed, scale_sigma=2e-3):
    """(GGUF rows on the host, the device weight in the layout the linear method stores: IQ3_S
    packed), cached per module (the configs reuse one weight over all M)."""
    key = (qt, rows, k, seed, scale_sigma)
    if key not in _WEIGHTS:
        from vllm_gguf_plugin.quantization import iq3_pack

        raw = o.random_blocks(np.random.default_rng(seed), qt, rows, k, scale_sigma=scale_sigma)
        w = dev(raw)
        if qt == o.IQ3_S:
            w = iq3_pack.pack(w, qt)
        _WEIGHTS[key] = (raw, w)
    return _WEIGHTS[key]


def _rows_checked(rows, seed):
    if rows <= 1024:
        return np.arange(rows)
    rng = np.random.default_rng(seed)
    pick = set(rng.choice(rows, size=382, replace=False).tolist()) | {0, rows - 1}
    return np.array(sorted(pick))


def _routed(n, qt, rows, k):
    from vllm_gguf_plugin.quantization import linear

    name = linear._lcpp_op(n, qt, rows, k, qt == o.IQ3_S)
    return name, getattr(C(), name), ("mmvq" if "_vec_" in name else "mmq")


@pytest.mark.parametrize("n", MTP_ROWS)
@pytest.mark.parametrize("rows,k", MTP_SHAPES)
@pytest.mark.parametrize("qt", MTP_TYPES)
def test_mtp_small_gemm_cell(qt, rows, k, n):
    raw, w = _weight(qt, rows, k, seed=2000 + qt)
    name, op, layout = _routed(n, qt, rows, k)
    rs = _rows_checked(rows, seed=n)
    g = torch.Generator().manual_seed(10 * n + qt)
    x = torch.randn(n, k, generator=g)
    for dt in (torch.bfloat16, torch.float32):
        xd = x.to(dt)
        y = op(w, xd.cuda(), qt, rows)
        assert y.dtype == dt and y.shape == (n, rows)
        err = o.rel_l2(y.float().cpu().numpy()[:, rs], o.q81_model(raw[rs], qt, xd, layout=layout))
        assert err <= TIGHT[dt], (name, str(dt), err)


@pytest.mark.parametrize("rows,k", MTP_SHAPES)
@pytest.mark.parametrize("qt", MTP_TYPES)
def test_mtp_small_gemm_graph_replay(qt, rows, k):
    """M = 8 (the decode/product boundary), 16 and 48 captured in one graph: every replay equals
    the eager calls bit for bit."""
    raw, w = _weight(qt, rows, k, seed=2000 + qt)
    xs = {n: torch.randn(n, k, generator=torch.Generator().manual_seed(n)).to(torch.bfloat16).cuda()
          for n in (8, 16, 48)}
    ops = {n: _routed(n, qt, rows, k)[1] for n in xs}
    eager = [ops[n](w, xs[n], qt, rows) for n in xs]
    torch.cuda.synchronize()
    graph_replays_equal(lambda: torch.cat([ops[n](w, xs[n], qt, rows).flatten() for n in xs]),
                        torch.cat([e.flatten() for e in eager]))


@pytest.mark.parametrize("n", [1, 4])
@pytest.mark.parametrize("rows,k", [(17408, 5120), (5120, 17408)])
def test_decode_gemv_fp32_activations(rows, k, n):
    """configs[1] with fp32 X: every output row within 1e-3 of the q81 model."""
    raw, w = _weight(o.IQ3_S, rows, k, seed=7 + rows)
    name, op, layout = _routed(n, o.IQ3_S, rows, k)
    assert name == "lcpp_mul_mat_vec_iq3_mma_packed"
    x = torch.randn(n, k, generator=torch.Generator().manual_seed(rows + n))
    y = op(w, x.cuda(), o.IQ3_S, rows).cpu().numpy()
    assert o.rel_l2(y, o.q81_model(raw, o.IQ3_S, x, layout=layout)) <= 1e-3


def test_cpu_path_config_q4k():
    """Q4_K 4096 x 4096, d and dmin ~ |N(0, 1e-3)|, X 1 x 4096 fp32 N(0,1), seed 0,
    through the routed decode op."""
    rows = k = 4096
    raw, w = _weight(o.Q4_K, rows, k, seed=0, scale_sigma=1e-3)
    name, op, layout = _routed(1, o.Q4_K, rows, k)
    x = torch.from_numpy(np.random.default_rng(0).standard_normal((1, k)).astype(np.float32))
    y = op(w, x.cuda(), o.Q4_K, rows).cpu().numpy()
    assert o.rel_l2(y, o.q81_model(raw, o.Q4_K, x, layout=layout)) <= 1e-3
