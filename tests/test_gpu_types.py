"""The GGUF types served by the generic kernels: Q2_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ1_M.
Each goes through every op the reference routes it to (linear.py:85-114 and the op type checks
of lcpp_shim.cu:767-773), through the C ABI. Needs an MI355X.

Bars (as tests/test_gpu_parity.py):
  * q8_1 bytes of the MMQ layouts (Q2_K's D2S6): bit-exact with the oracle;
  * exact mode (every block scale 1, integer X with one 127 per slice): the fp32 output equals
    the oracle's exact sum of slice values, the decode ops' truncating MMVQ values
    (oracle.mmvq_slice_units) for decode ops, the product ops' dot / den for product ops;
  * random weights and X with outliers: within 1e-3 relative L2 of the q81 model (fp32 X), the
    reference's tight bars for 16-bit X, and 3e-2 of the full-precision product;
  * the reference's real GGUF rows (tests/golden/dequant) of each type;
  * bit-identical outputs across hipGraph replays.
"""

import glob
import os

import numpy as np
import pytest
import torch

import gguf_oracle as o
from _gpu import TIGHT, C, dev, exact_ref, exact_weights, exact_x, graph_replays_equal, poison_allocator, w_rand, x_rand
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

GENERIC = [o.Q2_K, o.IQ2_XXS, o.IQ2_XS, o.IQ2_S, o.IQ3_XXS, o.IQ1_M]
TN = {t: o.TYPE_NAMES[t] for t in GENERIC}

# the decode ops each type is routed to or accepted by (1..8 rows; the packed op to 32)
DECODE_OPS = {
    o.Q2_K: ["lcpp_mul_mat_vec_q"],
    o.IQ2_XXS: ["lcpp_mul_mat_vec_q"],
    o.IQ2_XS: ["lcpp_mul_mat_vec_q"],
    o.IQ2_S: ["lcpp_mul_mat_vec_q", "lcpp_mul_mat_vec_own"],
    o.IQ3_XXS: ["lcpp_mul_mat_vec_q", "lcpp_mul_mat_vec_iq3", "lcpp_mul_mat_vec_iq3_mma",
                "lcpp_mul_mat_vec_iq3_mma_packed"],
    o.IQ1_M: ["lcpp_mul_mat_vec_q"],
}
# the product ops (IQ1_M has none: "no MMQ for IQ1_M")
PRODUCT_OPS = {
    o.Q2_K: ["lcpp_mul_mat_q"],
    o.IQ2_XXS: ["lcpp_mul_mat_q"],
    o.IQ2_XS: ["lcpp_mul_mat_q"],
    o.IQ2_S: ["lcpp_mul_mat_q", "lcpp_mul_mat_mma_k"],
    o.IQ3_XXS: ["lcpp_mul_mat_q", "lcpp_mul_mat_iq3_packed"],
}
MAX_ROWS = {"lcpp_mul_mat_vec_iq3_mma_packed": 32, "lcpp_mul_mat_mma_k": 64}

DECODE_CASES = [(qt, op) for qt in GENERIC for op in DECODE_OPS[qt]]
PRODUCT_CASES = [(qt, op) for qt in PRODUCT_OPS for op in PRODUCT_OPS[qt]]


def _id(case):
    qt, op = case
    return f"{TN[qt]}-{op.replace('lcpp_mul_mat_', '')}"


@pytest.fixture(scope="module", autouse=True)
def _ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from vllm_gguf_plugin import ops  # noqa: F401

    return torch.ops._C_gguf


def _weights(raw, op, qt):
    """W as the op reads it: the packed ops take iq3_pack's layout (IQ3_XXS: its unit layout)."""
    w = dev(raw)
    if op.endswith("_packed"):
        from vllm_gguf_plugin.quantization import iq3_pack

        import _tile

        w = iq3_pack.pack(w, qt)
        np.testing.assert_array_equal(w.cpu().numpy(), _tile.pack_xxs(raw) if qt == o.IQ3_XXS else _tile.pack(raw))
    return w


def _call(op, w, x, qt, rows, x_q8=None):
    f = getattr(C(), op)
    return f(w, x, qt, rows) if x_q8 is None or op in ("lcpp_mul_mat_q", "lcpp_mul_mat_mma_k",
                                                        "lcpp_mul_mat_iq3_packed") else f(w, x, qt, rows, x_q8)


# ------------------------------------------------------------------------------------ q8_1
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("n,k", [(1, 512), (9, 5120), (64, 2048)])
def test_quantize_q8_1_mmq_d2s6_bit_exact(dtype, n, k):
    """Q2_K's D2S6 block_q8_1_mmq: fp16 d per 64 values, fp16 sums of the first six 16-value
    groups of each 128, with an all-zero 64-value group."""
    x = x_rand(n, k, seed=7 * n + k, dtype=dtype)
    x[-1, 128:192] = 0
    got = C().lcpp_quantize_q8_1(x.cuda(), o.Q2_K, True, False).cpu().numpy()
    np.testing.assert_array_equal(got, o.quantize_q8_1_mmq(x, o.Q2_K))


@pytest.mark.parametrize("qt", [o.IQ2_XXS, o.IQ3_XXS, o.IQ1_M], ids=lambda t: TN[t])
def test_quantize_q8_1_generic_types(qt):
    x = x_rand(3, 1024, seed=qt)
    got = C().lcpp_quantize_q8_1(x.cuda(), qt, False, False).cpu().numpy()
    np.testing.assert_array_equal(got, o.quantize_q8_1(x))
    if qt != o.IQ1_M:
        got = C().lcpp_quantize_q8_1(x.cuda(), qt, True, False).cpu().numpy()
        np.testing.assert_array_equal(got, o.quantize_q8_1_mmq(x, qt))


def test_iq1m_has_no_mmq_quantiser():
    x = torch.zeros(2, 512, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="bad arguments"):
        C().lcpp_quantize_q8_1(x, o.IQ1_M, True, False)


# ------------------------------------------------------------------------------------ exact mode
# (weight rows, K): the one-lane-per-slice GEMV (K / 256 below 8 blocks, or X past the LDS
# budget of the slices GEMV) and the slices GEMV with X in LDS (rows not a multiple of its 8-row
# tile; K = 17408 at 1-2 rows)
DECODE_SHAPES = [(80, 1024), (100, 2048), (96, 17408)]


@pytest.mark.parametrize("case", DECODE_CASES, ids=_id)
@pytest.mark.parametrize("n", [1, 2, 5, 8, 13, 32])
@pytest.mark.parametrize("rows,k", DECODE_SHAPES)
def test_decode_exact(case, n, rows, k):
    qt, op = case
    if n > MAX_ROWS.get(op, 8):
        pytest.skip(f"{op} takes at most {MAX_ROWS.get(op, 8)} rows")
    if op.endswith("_packed") and rows % 16:
        rows = 96
    raw = exact_weights(qt, rows, k, seed=10 * n + qt)
    x = exact_x(n, k, seed=20 * n + qt, dtype=torch.float32)
    y = _call(op, _weights(raw, op, qt), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.float64), exact_ref(raw, qt, x, "mmvq"))


@pytest.mark.parametrize("case", PRODUCT_CASES, ids=_id)
@pytest.mark.parametrize("n", [1, 9, 16, 33, 64, 100])
def test_product_exact(case, n):
    qt, op = case
    if n > MAX_ROWS.get(op, 1 << 30):
        pytest.skip(f"{op} takes at most {MAX_ROWS[op]} rows")
    rows, k = 48, 1024
    raw = exact_weights(qt, rows, k, seed=30 * n + qt)
    x = exact_x(n, k, seed=40 * n + qt, dtype=torch.float32)
    y = _call(op, _weights(raw, op, qt), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.float64), exact_ref(raw, qt, x, "mmq"))


# ------------------------------------------------------------------------------------ q81 model
@pytest.mark.parametrize("case", DECODE_CASES, ids=_id)
@pytest.mark.parametrize("n", [1, 3, 8])
def test_decode_vs_q81(case, n):
    qt, op = case
    rows, k = 96, 2048
    raw = w_rand(qt, rows + 16, k, seed=n * 7 + qt)    # W has more rows than the product uses
    x = x_rand(n, k, seed=n + 100 + qt)
    y = _call(op, _weights(raw, op, qt)[:rows + 16], x.cuda(), qt, rows).cpu().numpy()
    ref = o.q81_model(raw[:rows], qt, x)
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)
    assert o.rel_l2(y, o.full_model(raw[:rows], qt, x)) <= 3e-2


@pytest.mark.parametrize("case", PRODUCT_CASES, ids=_id)
@pytest.mark.parametrize("n", [9, 17, 48, 130, 300])
def test_product_vs_q81(case, n):
    qt, op = case
    if n > MAX_ROWS.get(op, 1 << 30):
        pytest.skip(f"{op} takes at most {MAX_ROWS[op]} rows")
    rows, k = 80, 1024
    raw = w_rand(qt, rows, k, seed=n * 11 + qt)
    x = x_rand(n, k, seed=n + 200 + qt)
    y = _call(op, _weights(raw, op, qt), x.cuda(), qt, rows).cpu().numpy()
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)
    # Q2_K's D2S6 layout quantises X with one scale per 64 values, so a 64-value group holding
    # one of X's 20x outliers keeps fewer bits of the rest: the q8_1 error alone is larger
    loose = 6e-2 if qt == o.Q2_K else 3e-2
    assert o.rel_l2(y, o.full_model(raw, qt, x)) <= loose


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("qt", GENERIC, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 4, 16])
def test_16bit_x(qt, n, dtype):
    if qt == o.IQ1_M and n > 8:
        n = 8
    rows, k = 64, 1024
    raw = w_rand(qt, rows, k, seed=n * 13 + qt)
    x = x_rand(n, k, seed=n + 300 + qt, dtype=dtype)
    op = "lcpp_mul_mat_vec_q" if n <= 8 else "lcpp_mul_mat_q"
    y = getattr(C(), op)(dev(raw), x.cuda(), qt, rows)
    assert y.dtype == dtype and y.shape == (n, rows)
    ref = o.q81_model(raw, qt, x, layout="mmvq" if n <= 8 else "mmq")
    assert o.rel_l2(y.float().cpu().numpy(), ref) <= TIGHT[dtype]


def _golden(qt):
    """The reference's real GGUF rows of type qt, grouped by row size."""
    rows = {}
    for f in sorted(glob.glob(os.path.join(GOLDEN, "dequant", f"{TN[qt]}__*.npz"))):
        raw = np.load(f, allow_pickle=False)["raw"]
        rows.setdefault(raw.size, []).append(raw)
    return rows


@pytest.mark.parametrize("qt", GENERIC, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 4, 16, 48])
def test_golden_rows(qt, n):
    """Real GGUF rows of the reference's fixtures, 32 rows cycled per K."""
    if qt == o.IQ1_M and n > 8:
        pytest.skip("IQ1_M has no product op")
    golden = _golden(qt)
    assert golden, TN[qt]
    for same_k in golden.values():
        raw = np.stack([same_k[i % len(same_k)] for i in range(32)])
        k = raw.shape[1] // o.BLOCK_BYTES[qt] * 256
        x = x_rand(n, k, seed=n + 400)
        op = "lcpp_mul_mat_vec_q" if n <= 8 else "lcpp_mul_mat_q"
        y = getattr(C(), op)(dev(raw), x.cuda(), qt, 32).cpu().numpy()
        ref = o.q81_model(raw, qt, x, layout="mmvq" if n <= 8 else "mmq")
        assert o.rel_l2(y, ref) <= 1e-3, (k, o.rel_l2(y, ref))


# ------------------------------------------------------------------------------------ shapes
@pytest.mark.parametrize("qt", GENERIC, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 4])
def test_full_size_decode(qt, n):
    """The 27B gate/up shape 17408 x 5120 (more row groups than the GEMV's 2048-workgroup grid,
    so workgroups loop), sampled rows against the q81 model."""
    rows, k = 17408, 5120
    raw = w_rand(qt, rows, k, seed=500 + qt)
    x = x_rand(n, k, seed=501 + n)
    y = C().lcpp_mul_mat_vec_q(dev(raw), x.cuda(), qt, rows).cpu().numpy()
    rs = np.unique(np.concatenate([[0, rows - 1], np.random.default_rng(qt).choice(rows, 96, replace=False)]))
    ref = o.q81_model(raw[rs], qt, x)
    assert o.rel_l2(y[:, rs], ref) <= 1e-3
    assert np.isfinite(y).all()


# the stream GEMV (gemv_generic_stream_kernel: 1-4 rows, rows % 4 == 0, a 4-row unit per CU or
# more): one unit per CU at 256 CUs with two block pairs; 516 units (2 or 3 per CU); K = 17408
# (34 block pairs per unit)
STREAM_SHAPES = [(1024, 1024), (2064, 2560), (1024, 17408)]


@pytest.mark.parametrize("qt", GENERIC, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 2, 3, 4])
@pytest.mark.parametrize("rows,k", STREAM_SHAPES)
def test_stream_decode_exact(qt, n, rows, k):
    raw = exact_weights(qt, rows, k, seed=900 + 10 * n + qt)
    x = exact_x(n, k, seed=901 + n, dtype=torch.float32)
    y = C().lcpp_mul_mat_vec_q(dev(raw), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.float64), exact_ref(raw, qt, x, "mmvq"))


@pytest.mark.parametrize("qt", GENERIC, ids=lambda t: TN[t])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("n", [1, 2])
def test_stream_fused_quantisation(qt, dtype, n):
    """At 1-2 rows and K <= 8192 the stream GEMV quantises X itself: bit-identical to the q8_1
    quantiser followed by the GEMV (the op given x_q8), for each X dtype, on X as rows of a wider
    tensor (row stride above K) with an all-zero slice (d = 0)."""
    rows, k = 2064, 5120
    w = dev(w_rand(qt, rows, k, seed=960 + qt))
    wide = x_rand(n, k + 512, seed=961 + n, dtype=dtype).cuda()
    x = wide[:, 256:256 + k]
    x[:, 64:96] = 0
    q8 = C().lcpp_quantize_q8_1(x, qt, False, False)
    a = C().lcpp_mul_mat_vec_q(w, x, qt, rows)
    b = C().lcpp_mul_mat_vec_q(w, x, qt, rows, q8)
    assert torch.equal(a, b)


@pytest.mark.parametrize("qt", GENERIC, ids=lambda t: TN[t])
def test_stream_down_shape(qt):
    """5120 x 17408 (5 units per CU, 34 block pairs) at 2 rows, bf16 X: sampled rows against the
    q81 model; one graph replay equals the eager call."""
    rows, k, n = 5120, 17408, 2
    raw = w_rand(qt, rows, k, seed=950 + qt)
    w = dev(raw)
    x = x_rand(n, k, seed=951, dtype=torch.bfloat16).cuda()
    y = C().lcpp_mul_mat_vec_q(w, x, qt, rows)
    rs = np.unique(np.concatenate([[0, rows - 1], np.random.default_rng(qt).choice(rows, 254, replace=False)]))
    assert o.rel_l2(y.float().cpu().numpy()[:, rs], o.q81_model(raw[rs], qt, x.cpu())) <= TIGHT[torch.bfloat16]
    torch.cuda.synchronize()
    graph_replays_equal(lambda: C().lcpp_mul_mat_vec_q(w, x, qt, rows), y)


@pytest.mark.parametrize("qt", [o.Q2_K, o.IQ2_S, o.IQ3_XXS], ids=lambda t: TN[t])
def test_down_shape_product(qt):
    """5120 x 17408 at 48 activation rows: sampled rows against the q81 model."""
    rows, k, n = 5120, 17408, 48
    raw = w_rand(qt, rows, k, seed=600 + qt)
    x = x_rand(n, k, seed=601)
    y = C().lcpp_mul_mat_q(dev(raw), x.cuda(), qt, rows).cpu().numpy()
    rs = np.unique(np.concatenate([[0, rows - 1], np.random.default_rng(qt).choice(rows, 32, replace=False)]))
    ref = o.q81_model(raw[rs], qt, x, layout="mmq")
    assert o.rel_l2(y[:, rs], ref) <= 1e-3


@pytest.mark.parametrize("qt", GENERIC, ids=lambda t: TN[t])
def test_shared_x_q8_equals_own_quantize(qt):
    """A decode op given apply()'s shared q8_1 (made for another type) equals quantising itself."""
    rows, k, n = 64, 2048, 5
    raw = w_rand(qt, rows, k, seed=700 + qt)
    x = x_rand(n, k, seed=701).cuda()
    q8 = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)
    a = C().lcpp_mul_mat_vec_q(dev(raw), x, qt, rows)
    b = C().lcpp_mul_mat_vec_q(dev(raw), x, qt, rows, q8)
    assert torch.equal(a, b)


@pytest.mark.parametrize("case", [(o.IQ2_S, "lcpp_mul_mat_vec_own"), (o.Q2_K, "lcpp_mul_mat_q"),
                                  (o.IQ3_XXS, "lcpp_mul_mat_vec_iq3_mma_packed"), (o.IQ1_M, "lcpp_mul_mat_vec_q")],
                         ids=_id)
def test_graph_replay_bit_exact(case):
    qt, op = case
    rows, k, n = 256, 2048, 4 if "vec" in op else 24
    raw = w_rand(qt, rows, k, seed=800 + qt)
    w = _weights(raw, op, qt)
    x = x_rand(n, k, seed=801).cuda()
    eager = getattr(torch.ops._C_gguf, op)(w, x, qt, rows)
    torch.cuda.synchronize()
    graph_replays_equal(lambda: getattr(torch.ops._C_gguf, op)(w, x, qt, rows), eager)


# ------------------------------------------------------------------------------------ routing
@pytest.mark.parametrize("n", [1, 8, 9, 17, 32, 33])
def test_iq1m_routing(n):
    """IQ1_M: one MMVQ call up to 8 rows, 8-row calls up to 32 (linear.py's split), none above."""
    from vllm_gguf_plugin.quantization import linear

    rows, k = 256, 2048
    raw = w_rand(o.IQ1_M, rows, k, seed=900)
    x = x_rand(n, k, seed=901 + n).cuda()
    if n > 32:
        with pytest.raises(NotImplementedError, match="IQ1_M"):
            linear._fused_mul_mat_gguf(x, dev(raw), o.IQ1_M)
        return
    poison_allocator()
    y = linear._fused_mul_mat_gguf(x, dev(raw), o.IQ1_M)
    want = torch.cat([C().lcpp_mul_mat_vec_q(dev(raw), x[i:i + 8], o.IQ1_M, rows) for i in range(0, n, 8)])
    assert torch.equal(y, want)
    assert o.rel_l2(y.cpu().numpy(), o.q81_model(raw, o.IQ1_M, x.cpu())) <= 1e-3


@pytest.mark.parametrize("n", [1, 6, 9, 40])
def test_iq3xxs_packed_layer(n):
    """A qkv layer of IQ3_XXS q with IQ3_S k, v: the layer packs both (each into its unit layout) and
    apply() equals each run's packed op on its own bytes."""
    from test_gpu_layers import build_layer, routed

    k = 2048
    q, kw, vw = w_rand(o.IQ3_XXS, 512, k, 1), w_rand(o.IQ3_S, 256, k, 2), w_rand(o.IQ3_S, 256, k, 3)
    layer, method = build_layer([(q, o.IQ3_XXS), (kw, o.IQ3_S), (vw, o.IQ3_S)], k, ["q", "k", "v"])
    assert layer.weight.iq3_packed
    x = x_rand(n, k, seed=950 + n).to(torch.bfloat16).cuda()
    poison_allocator()
    y = method.apply(layer, x)
    ref = torch.cat([routed(q, x, o.IQ3_XXS, True), routed(np.concatenate([kw, vw]), x, o.IQ3_S, True)], dim=1)
    assert torch.equal(y, ref)
    layout = "mmvq" if n <= 8 else "mmq"
    assert o.rel_l2(y[:, :512].float().cpu().numpy(), o.q81_model(q, o.IQ3_XXS, x.cpu(), layout)) <= TIGHT[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("qt", [o.Q2_K, o.IQ3_XXS, o.IQ1_M], ids=lambda t: TN[t])
@pytest.mark.parametrize("n,k", [(1, 2048), (3, 5120), (8, 2048), (2, 17408)])
def test_own_quantisation_equals_x_q8(qt, dtype, n, k):
    """The decode op quantising X itself (no x_q8; X in any dtype, rows strided) gives the same
    bytes as on X quantised by lcpp_quantize_q8_1 (itself bit-exact with the oracle)."""
    rows = 64
    raw = w_rand(qt, rows, k, seed=1100 + qt)
    x = x_rand(n, k + 64, seed=1101 + n, dtype=dtype)[:, :k].cuda()  # row stride k + 64
    q8 = C().lcpp_quantize_q8_1(x, qt, False, False)
    a = C().lcpp_mul_mat_vec_q(dev(raw), x, qt, rows)
    b = C().lcpp_mul_mat_vec_q(dev(raw), x, qt, rows, q8)
    assert torch.equal(a, b)
    assert o.rel_l2(a.float().cpu().numpy(), o.q81_model(raw, qt, x.cpu())) <= TIGHT[dtype] if dtype != torch.float32 else 1e-3
