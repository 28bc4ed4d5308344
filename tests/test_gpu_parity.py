"""Parity of the gfx950 kernels with the CPU oracle, through the C ABI (torch.ops._C_gguf ->
libgguf_mi355x.so). Needs an MI355X.

Bars:
  * q8_1 bytes (both layouts): bit-exact with the oracle;
  * int32 slice dots: bit-exact, checked through the real product kernels in an exact-integer
    mode (block scales d = dmin = 1, X integer-valued with one 127 per slice so every q8_1 scale
    is 1): every partial sum is then an integer below 2^24, so the fp32 output must equal the
    oracle's int64 sum of slice dots exactly;
  * fp32 outputs (fp32 X): within 1e-3 relative L2 (max over activation rows) of the q81 model
    dequant(W) @ dequant(q8_1(X)) in float64; 16-bit X/Y: within the reference's tight bars
    (5e-3 bf16, 2.5e-3 fp16, tests/gpu/test_kernel_parity.py:40) since Y is rounded to X's dtype;
  * bit-identical outputs across hipGraph replays.
Every op call first poisons torch's caching allocator (tests/_gpu.py).
"""

import glob
import os

import numpy as np
import pytest
import torch
from conftest import GOLDEN

import _tile
import gguf_oracle as o
from _gpu import TIGHT, C
from _gpu import dev as _dev
from _gpu import exact_ref as _exact_ref
from _gpu import exact_weights as _exact_weights
from _gpu import exact_x as _exact_x
from _gpu import w_rand as _w
from _gpu import x_rand as _x

pytestmark = pytest.mark.gpu

TYPES = [o.IQ3_S, o.Q4_K, o.IQ4_XS, o.Q6_K]
TN = {t: o.TYPE_NAMES[t] for t in TYPES}
VEC_OP = {o.IQ3_S: "lcpp_mul_mat_vec_iq3", o.Q4_K: "lcpp_mul_mat_vec_own", o.IQ4_XS: "lcpp_mul_mat_vec_q",
          o.Q6_K: "lcpp_mul_mat_vec_q"}
GEMM_OP = {o.IQ3_S: "lcpp_mul_mat_q", o.Q4_K: "lcpp_mul_mat_mma_k", o.IQ4_XS: "lcpp_mul_mat_mma_k",
           o.Q6_K: "lcpp_mul_mat_q"}


@pytest.fixture(scope="module", autouse=True)
def _ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from vllm_gguf_plugin import ops  # noqa: F401  registers torch.ops._C_gguf (fails if not built)

    return torch.ops._C_gguf


# ------------------------------------------------------------------------------------ q8_1
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("n,k", [(1, 512), (3, 5120), (8, 17408), (48, 5120)])
def test_quantize_q8_1_bit_exact(dtype, n, k):
    x = _x(n, k, seed=n + k, dtype=dtype)
    x[0, 64:96] = 0                                   # an all-zero block
    got = C().lcpp_quantize_q8_1(x.cuda(), o.IQ3_S, False, False).cpu().numpy()
    np.testing.assert_array_equal(got, o.quantize_q8_1(x))


@pytest.mark.parametrize("qt", [o.IQ3_S, o.Q4_K], ids=lambda t: TN[t])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("n,k", [(1, 512), (9, 5120), (64, 2048)])
def test_quantize_q8_1_mmq_bit_exact(qt, dtype, n, k):
    x = _x(n, k, seed=3 * n + k, dtype=dtype)
    x[-1, 128:160] = 0
    got = C().lcpp_quantize_q8_1(x.cuda(), qt, True, False).cpu().numpy()
    np.testing.assert_array_equal(got, o.quantize_q8_1_mmq(x, qt))


def test_quantize_strided_rows():
    x = _x(4, 1024 + 64, seed=5)[:, :1024]           # row stride > K
    got = C().lcpp_quantize_q8_1(x.cuda(), o.IQ3_S, False, False).cpu().numpy()
    np.testing.assert_array_equal(got, o.quantize_q8_1(x.contiguous()))


# ------------------------------------------------------------------------------------ exact ints
@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 2, 4, 5, 8])
def test_gemv_exact_integer_dots(qt, n):
    rows, k = 64, 512
    raw = _exact_weights(qt, rows, k, seed=10 + n)
    x = _exact_x(n, k, seed=20 + n, dtype=torch.float32)
    y = getattr(C(), VEC_OP[qt])(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x))
    assert (y == y.astype(np.int64)).all()


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
def test_gemv_exact_integer_bf16_output_is_rounded_exact(qt):
    """bf16 X: the fp32 result is the exact integer, stored with round-to-nearest-even."""
    rows, k, n = 64, 512, 3
    raw = _exact_weights(qt, rows, k, seed=15)
    x = _exact_x(n, k, seed=25)
    y = getattr(C(), VEC_OP[qt])(_dev(raw), x.cuda(), qt, rows).cpu()
    want = torch.from_numpy(_exact_ref(raw, qt, x).astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [9, 16, 33, 64])
def test_gemm_exact_integer_dots(qt, n):
    rows, k = 48, 512
    raw = _exact_weights(qt, rows, k, seed=30 + n)
    x = _exact_x(n, k, seed=40 + n, dtype=torch.float32)
    op = GEMM_OP[qt] if n <= 64 else "lcpp_mul_mat_q"
    y = getattr(C(), op)(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x))
    assert (y == y.astype(np.int64)).all()


def test_packed_exact_integer_dots():
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k = 64, 512
    raw = _exact_weights(o.IQ3_S, rows, k, seed=50)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    for n, op in ((1, "lcpp_mul_mat_vec_iq3_mma_packed"), (8, "lcpp_mul_mat_vec_iq3_mma_packed"),
                  (24, "lcpp_mul_mat_vec_iq3_mma_packed"), (40, "lcpp_mul_mat_iq3_packed")):
        x = _exact_x(n, k, seed=60 + n, dtype=torch.float32)
        y = getattr(C(), op)(w, x.cuda(), o.IQ3_S, rows).cpu().numpy()
        np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, o.IQ3_S, x), err_msg=f"{op} n={n}")


# ------------------------------------------------------------------------------------ q81 model
@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 3, 4, 8])
@pytest.mark.parametrize("rows,k", [(96, 2048), (100, 512)])
def test_gemv_vs_q81(qt, n, rows, k):
    raw = _w(qt, rows + 4, k, seed=n * 7 + rows)    # W has more rows than the product uses
    x = _x(n, k, seed=n + 100)
    y = getattr(C(), VEC_OP[qt])(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    ref = o.q81_model(raw[:rows], qt, x)
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)
    assert o.rel_l2(y, o.full_model(raw[:rows], qt, x)) <= 3e-2


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [9, 17, 32, 48, 130])
def test_gemm_vs_q81(qt, n):
    rows, k = 80, 1024
    raw = _w(qt, rows, k, seed=n * 11)
    x = _x(n, k, seed=n + 200)
    op = GEMM_OP[qt] if n <= 64 else "lcpp_mul_mat_q"
    y = getattr(C(), op)(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)


# the int8 raw GEMM with K split over workgroups (grids of fewer than two workgroups per CU):
# (rows, k, n); 48 x 5120 splits 4 ways, 1000 x 2048 (ragged last tile, 3 column tiles) and
# 5120 x 6144 2 ways, 64 x 17408 4 ways
SPLIT_SHAPES = [(48, 5120, 16), (1000, 2048, 33), (5120, 6144, 9), (64, 17408, 48)]
RAW_TYPES = [o.Q4_K, o.IQ4_XS, o.Q6_K]


def _split_ws(lib, op, qt, rows, k, n, has_q8=0):
    """Asserts that the op's plan splits K: its workspace holds more than the xq copy of X. Q4_K
    at 33-48 rows on these weights (fewer than two tiles per CU) is planned unsplit instead, in
    groups of two column tiles: there the workspace is exactly the xq copy."""
    xq = -(-n // 16) * (k // 256) * 4608
    ws = lib.gguf_op_workspace_bytes(op, qt, rows, k, n, has_q8)
    if qt == o.Q4_K and 33 <= n <= 48:
        assert ws == xq, (ws, xq)
    else:
        assert ws > xq, (ws, xq)


@pytest.mark.parametrize("qt", RAW_TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("rows,k,n", SPLIT_SHAPES, ids=lambda v: str(v))
def test_split_k_exact_integer_dots(lib, qt, rows, k, n):
    """Exact-integer mode through the K-split raw GEMM: each split's partial sums and their
    fixed-order total are integers, so the output equals the oracle's int64 sum exactly."""
    op = GEMM_OP[qt]
    _split_ws(lib, _capi_op(op), qt, rows, k, n)
    raw = _exact_weights(qt, rows, k, seed=300 + rows + n)
    x = _exact_x(n, k, seed=310 + n, dtype=torch.float32)
    y = getattr(C(), op)(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x))


@pytest.mark.parametrize("qt", RAW_TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("with_q8", [False, True], ids=["x", "x_q8"])
def test_split_k_decode_op(lib, qt, with_q8):
    """A decode op at 8 rows on the split GEMM, with X or the caller's q8_1 (converted by the
    kernel that also clears the split counters): exact-integer output."""
    rows, k, n = 48, 5120, 8
    op = "lcpp_mul_mat_vec_q"
    _split_ws(lib, 0, qt, rows, k, n, int(with_q8))
    raw = _exact_weights(qt, rows, k, seed=320 + qt)
    x = _exact_x(n, k, seed=330, dtype=torch.float32).cuda()
    q8 = C().lcpp_quantize_q8_1(x, qt, False, False) if with_q8 else None
    y = getattr(C(), op)(_dev(raw), x, qt, rows, q8).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x.cpu()))


@pytest.mark.parametrize("qt", RAW_TYPES, ids=lambda t: TN[t])
def test_split_k_vs_q81_deterministic_and_graph_replays(lib, qt):
    """The split GEMM on random weights with zero-d blocks against the q81 model (bf16 bar);
    repeated calls and graph replays are bit-identical: the counters are cleared on every call
    and the partial sums are added in split order."""
    rows, k, n = 1000, 2048, 40
    op = GEMM_OP[qt]
    _split_ws(lib, _capi_op(op), qt, rows, k, n)
    raw = _w(qt, rows, k, seed=340 + qt)
    b = raw.reshape(rows, k // 256, o.BLOCK_BYTES[qt])
    zero = np.random.default_rng(341).random((rows, k // 256)) < 0.2
    for off in o.SCALE_OFFSETS[qt]:
        b[zero, off:off + 2] = 0
    x = _x(n, k, seed=342, dtype=torch.bfloat16)
    w, xc = _dev(raw), x.cuda()
    f = lambda: getattr(C(), op)(w, xc, qt, rows)
    y = f()
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y.float().cpu().numpy(), ref) <= TIGHT[torch.bfloat16]
    for _ in range(3):
        assert torch.equal(f(), y)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y)
        assert torch.equal(f(), y)  # eager work between the replays


# the packed IQ3_S tile GEMM with K split over workgroups: (rows, k, n, op); 64 x 17408 splits
# 4 ways at 2+ column tiles, 256 x 12288 2 ways at one, 1024 x 5120 (64 tiles) 2 ways
PACKED_SPLIT = [(64, 17408, 48, "lcpp_mul_mat_iq3_packed"), (1024, 5120, 16, "lcpp_mul_mat_iq3_packed"),
                (256, 12288, 8, "lcpp_mul_mat_vec_iq3_mma_packed"), (64, 17408, 24, "lcpp_mul_mat_vec_iq3_mma_packed")]


@pytest.mark.parametrize("rows,k,n,op", PACKED_SPLIT, ids=lambda v: str(v))
@pytest.mark.parametrize("with_q8", [False, True], ids=["x", "x_q8"])
def test_packed_split_k_exact_integer_dots(lib, rows, k, n, op, with_q8):
    """Exact-integer mode through the K-split tile GEMM on the unit layout, from X or (decode op)
    from the caller's q8_1: the output equals the oracle's int64 sum exactly."""
    from vllm_gguf_plugin.quantization import iq3_pack

    if with_q8 and op != "lcpp_mul_mat_vec_iq3_mma_packed":
        pytest.skip("x_q8 is an argument of the decode ops only")
    _split_ws(lib, _capi_op(op), o.IQ3_S, rows, k, n, int(with_q8))
    raw = _exact_weights(o.IQ3_S, rows, k, seed=350 + rows + n)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    x = _exact_x(n, k, seed=360 + n, dtype=torch.float32).cuda()
    args = (C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False),) if with_q8 else ()
    y = getattr(C(), op)(w, x, o.IQ3_S, rows, *args).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, o.IQ3_S, x.cpu()))


def test_packed_split_k_vs_q81_deterministic_and_graph_replays(lib):
    """The split tile GEMM (1024 rows: 64 tiles, 2 ways, 3 column tiles) on random weights against
    the q81 model (bf16 bar); repeated calls and graph replays are bit-identical."""
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k, n = 1024, 5120, 40
    _split_ws(lib, _capi_op("lcpp_mul_mat_iq3_packed"), o.IQ3_S, rows, k, n)
    raw = _w(o.IQ3_S, rows, k, seed=370)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    xc = _x(n, k, seed=371, dtype=torch.bfloat16).cuda()
    f = lambda: C().lcpp_mul_mat_iq3_packed(w, xc, o.IQ3_S, rows)
    y = f()
    ref = o.q81_model(raw, o.IQ3_S, xc.cpu(), layout="mmq")
    assert o.rel_l2(y.float().cpu().numpy(), ref) <= TIGHT[torch.bfloat16]
    for _ in range(3):
        assert torch.equal(f(), y)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y)
        assert torch.equal(f(), y)


def _capi_op(name):
    from vllm_gguf_plugin import _capi

    return _capi.OPS[name]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 4, 16])
def test_16bit_x(qt, n, dtype):
    rows, k = 64, 1024
    raw = _w(qt, rows, k, seed=n * 13)
    x = _x(n, k, seed=n + 300, dtype=dtype)
    op = VEC_OP[qt] if n <= 8 else GEMM_OP[qt]
    y = getattr(C(), op)(_dev(raw), x.cuda(), qt, rows)
    assert y.dtype == dtype and y.shape == (n, rows)
    ref = o.q81_model(raw, qt, x, layout="mmvq" if n <= 8 else "mmq")
    assert o.rel_l2(y.float().cpu().numpy(), ref) <= TIGHT[dtype]


def _golden(qt):
    files = sorted(glob.glob(os.path.join(GOLDEN, "dequant", f"{TN[qt]}__*.npz")))
    rows = {}
    for f in files:
        raw = np.load(f, allow_pickle=False)["raw"]
        rows.setdefault(raw.size, []).append(raw)
    return rows


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 4, 16, 48])
def test_golden_rows(qt, n):
    """Real GGUF rows of the reference's fixtures, 32 rows cycled per K."""
    for same_k in _golden(qt).values():
        raw = np.stack([same_k[i % len(same_k)] for i in range(32)])
        k = raw.shape[1] // o.BLOCK_BYTES[qt] * 256
        x = _x(n, k, seed=n + 400)
        op = VEC_OP[qt] if n <= 8 else GEMM_OP[qt]
        y = getattr(C(), op)(_dev(raw), x.cuda(), qt, 32).cpu().numpy()
        ref = o.q81_model(raw, qt, x, layout="mmvq" if n <= 8 else "mmq")
        assert o.rel_l2(y, ref) <= 1e-3, (k, o.rel_l2(y, ref))


# ------------------------------------------------------------------------------------ fp16 small GEMM
# Product ops of 64..255 activation rows with K <= 8192 on packed IQ3_S and Q4_K run the fp16
# small GEMM: one 16-row tile per workgroup below 1024 tiles, two from 1024 tiles on.
SMALL_H_ROWS = {o.IQ3_S: (64, 16 * 1025), o.Q4_K: (100, 16 * 1024 + 9)}


def _small_h_op(qt, raw, rows):
    from vllm_gguf_plugin.quantization import iq3_pack

    if qt == o.IQ3_S:
        return lambda x: C().lcpp_mul_mat_iq3_packed(iq3_pack.pack(_dev(raw), qt), x, qt, rows)
    return lambda x: C().lcpp_mul_mat_q(_dev(raw), x, qt, rows)


@pytest.mark.parametrize("qt", [o.IQ3_S, o.Q4_K], ids=lambda t: TN[t])
@pytest.mark.parametrize("tiles", [0, 1], ids=["one_tile", "two_tiles"])
@pytest.mark.parametrize("n", [64, 100, 255])
def test_small_fp16_exact_integer_dots(qt, tiles, n):
    """Exact-integer mode through the fp16 small GEMM: weight x sub-scale and the q8 values are exact
    fp16 integers, so every output is the oracle's int64 sum of slice dots (rows past the last full
    tile or tile pair, activation rows past the last column tile)."""
    rows, k = SMALL_H_ROWS[qt][tiles], 512
    raw = _exact_weights(qt, rows, k, seed=160 + n)
    x = _exact_x(n, k, seed=170 + n, dtype=torch.float32)
    y = _small_h_op(qt, raw, rows)(x.cuda()).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x))


@pytest.mark.parametrize("qt", [o.IQ3_S, o.Q4_K], ids=lambda t: TN[t])
@pytest.mark.parametrize("tiles", [0, 1], ids=["one_tile", "two_tiles"])
@pytest.mark.parametrize("n", [64, 200])
def test_small_fp16_vs_q81_with_zero_blocks(qt, tiles, n):
    """The running block scale: blocks with d = 0 (a row's first block, blocks inside a row, and a
    row with every block zero; Q4_K keeps its dmin term) against the q81 model."""
    rows, k = SMALL_H_ROWS[qt][tiles], 2048
    raw = _w(qt, rows, k, seed=180 + n + tiles)
    b = raw.reshape(rows, k // 256, o.BLOCK_BYTES[qt])
    rng = np.random.default_rng(190 + n)
    zero = rng.random((rows, k // 256)) < 0.2
    zero[:, 0] |= rng.random(rows) < 0.5
    zero[3] = True
    b[zero, 0:2] = 0
    x = _x(n, k, seed=n + 800)
    y = _small_h_op(qt, raw, rows)(x.cuda()).cpu().numpy()
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)
    if qt == o.IQ3_S:
        assert (y[:, 3] == 0).all()


# Product ops of up to 48 activation rows (IQ3_S from 33, Q4_K from 17) on weights of 1..5 row tiles
# per CU run the fp16 small GEMM's range plan: one workgroup per CU over its run of row tiles (300
# tiles: runs of 1 or 2; 1100: 4 or 5; 1280: 5), all column tiles in the workgroup.
RANGE_ROWS = {o.IQ3_S: (16 * 1030, 16 * 1100, 16 * 1280), o.Q4_K: (16 * 1030 + 9, 16 * 1100, 16 * 1280)}
RANGE_N = {o.IQ3_S: [33, 40, 48], o.Q4_K: [17, 32, 33, 48]}


@pytest.mark.parametrize("qt,n", [(qt, n) for qt in (o.IQ3_S, o.Q4_K) for n in RANGE_N[qt]],
                         ids=[f"{TN[qt]}-{n}" for qt in (o.IQ3_S, o.Q4_K) for n in RANGE_N[qt]])
@pytest.mark.parametrize("ri", [0, 1, 2], ids=["runs4-5a", "runs4-5b", "runs5"])
def test_small_fp16_range_exact_integer_dots(lib, qt, ri, n):
    """Exact-integer mode through the range plan (asserted from the op's workspace: the fp16
    activation layout): every output is the oracle's int64 sum of slice dots."""
    rows, k = RANGE_ROWS[qt][ri], 512
    op = 7 if qt == o.IQ3_S else 1
    assert lib.gguf_op_workspace_bytes(op, qt, rows, k, n, 0) == -(-n // 16) * (k // 256) * 9216
    raw = _exact_weights(qt, rows, k, seed=240 + n + ri)
    x = _exact_x(n, k, seed=250 + n, dtype=torch.float32)
    y = _small_h_op(qt, raw, rows)(x.cuda()).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x))


@pytest.mark.parametrize("qt,n", [(o.IQ3_S, 33), (o.IQ3_S, 48), (o.Q4_K, 17), (o.Q4_K, 48)])
def test_small_fp16_range_vs_q81_with_zero_blocks(qt, n):
    """The range plan against the q81 model with zero-d blocks (running block scale), bf16 output,
    and graph replays bit-identical."""
    rows, k = RANGE_ROWS[qt][1], 2048
    raw = _w(qt, rows, k, seed=260 + n)
    b = raw.reshape(rows, k // 256, o.BLOCK_BYTES[qt])
    rng = np.random.default_rng(270 + n)
    zero = rng.random((rows, k // 256)) < 0.2
    zero[:, 0] |= rng.random(rows) < 0.5
    b[zero, 0:2] = 0
    from vllm_gguf_plugin.quantization import iq3_pack

    x = _x(n, k, seed=n + 280, dtype=torch.bfloat16)
    if qt == o.IQ3_S:
        w = iq3_pack.pack(_dev(raw), qt)
        f = lambda xx: C().lcpp_mul_mat_iq3_packed(w, xx, qt, rows)
    else:
        w = _dev(raw)
        f = lambda xx: C().lcpp_mul_mat_q(w, xx, qt, rows)
    xc = x.cuda()
    y = f(xc)
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y.float().cpu().numpy(), ref) <= TIGHT[torch.bfloat16]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f(xc)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y)


@pytest.mark.parametrize("qt", [o.IQ3_S, o.Q4_K], ids=lambda t: TN[t])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_small_fp16_16bit_x(qt, dtype):
    rows, k, n = SMALL_H_ROWS[qt][0], 5120, 96
    raw = _w(qt, rows, k, seed=210)
    x = _x(n, k, seed=211, dtype=dtype)
    y = _small_h_op(qt, raw, rows)(x.cuda())
    assert y.dtype == dtype and y.shape == (n, rows)
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y.float().cpu().numpy(), ref) <= TIGHT[dtype]


# ------------------------------------------------------------------------------------ packed
def test_pack_is_the_tile_layout_and_roundtrips():
    from vllm_gguf_plugin.quantization import iq3_pack

    raw = _w(o.IQ3_S, 272, 1024, seed=70)
    w = _dev(raw)
    p = iq3_pack.pack(w, o.IQ3_S)
    np.testing.assert_array_equal(p.cpu().numpy(), _tile.pack(raw))
    np.testing.assert_array_equal(iq3_pack.unpack(p, o.IQ3_S).cpu().numpy(), raw)


@pytest.mark.parametrize("rows,k", [(272, 1024), (32, 1536)])
def test_pack_is_the_xxs_unit_layout_and_roundtrips(rows, k):
    """IQ3_XXS: the GPU repack equals the numpy statement of the unit layout (a ragged last
    unit-block at K = 1536) and unpacks back to the GGUF rows."""
    from vllm_gguf_plugin.quantization import iq3_pack

    raw = _w(o.IQ3_XXS, rows, k, seed=72)
    p = iq3_pack.pack(_dev(raw), o.IQ3_XXS)
    np.testing.assert_array_equal(p.cpu().numpy(), _tile.pack_xxs(raw))
    np.testing.assert_array_equal(iq3_pack.unpack(p, o.IQ3_XXS).cpu().numpy(), raw)


# Packed IQ3_XXS through both packed ops: the stream GEMV at 1..32 rows (q8_1 in groups of at most
# 4 activation rows, fused at 1-2 rows for K <= 8192; 65536 x 5120 at 4 rows runs in two row
# ranges, 61440 rows filling the partial-sum slots of LDS on 256 CUs) and the generic GEMM staging
# the unit layout, against the q81 model of each op's arithmetic.
@pytest.mark.parametrize("rows,k,n", [(64, 512, 1), (64, 1536, 3), (1024, 5120, 1), (1024, 5120, 2),
                                      (4096, 5120, 4), (256, 17408, 1), (256, 17408, 5), (64, 5120, 32),
                                      (17408, 5120, 2), (17408, 5120, 4), (65536, 5120, 4), (64, 1536, 33),
                                      (1024, 5120, 300)])
def test_packed_xxs_ops_vs_q81(rows, k, n):
    from vllm_gguf_plugin.quantization import iq3_pack

    raw = _w(o.IQ3_XXS, rows, k, seed=rows + k + n)
    w = iq3_pack.pack(_dev(raw), o.IQ3_XXS)
    x = _x(n, k, seed=n + 510)
    gemm = n > 32
    op = "lcpp_mul_mat_iq3_packed" if gemm else "lcpp_mul_mat_vec_iq3_mma_packed"
    mid = min(61440, rows // 2)  # 65536 rows: where the second row range starts
    sel = slice(None) if rows <= 4096 else np.r_[0:256, mid - 128:mid + 128, rows - 256:rows]
    y = getattr(C(), op)(w, x.cuda(), o.IQ3_XXS, rows).cpu().numpy()
    ref = o.q81_model(raw[sel], o.IQ3_XXS, x, layout="mmq" if gemm else "mmvq")
    assert o.rel_l2(y[:, sel], ref) <= 1e-3


def test_packed_xxs_decode_with_shared_q8_1_and_replays():
    """The packed IQ3_XXS GEMV on the caller's x_q8 equals the op quantising X itself, and graph
    replays of the fused op with new X equal eager calls."""
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k = 4096, 5120
    raw = _w(o.IQ3_XXS, rows, k, seed=73)
    w = iq3_pack.pack(_dev(raw), o.IQ3_XXS)
    for n in (1, 2, 4):
        x = _x(n, k, seed=520 + n).cuda()
        q8 = C().lcpp_quantize_q8_1(x, o.IQ3_XXS, False, False)
        a = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_XXS, rows)
        b = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_XXS, rows, q8)
        assert torch.equal(a, b)
    xs = _x(1, k, seed=530).cuda()
    C().lcpp_mul_mat_vec_iq3_mma_packed(w, xs, o.IQ3_XXS, rows)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ys = C().lcpp_mul_mat_vec_iq3_mma_packed(w, xs, o.IQ3_XXS, rows)
    for i in range(3):
        xs.copy_(_x(1, k, seed=540 + i).cuda())
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys, C().lcpp_mul_mat_vec_iq3_mma_packed(w, xs, o.IQ3_XXS, rows))


def test_pack_inplace_inside_padded_buffer():
    from vllm_gguf_plugin.quantization import iq3_pack

    raw = _w(o.IQ3_S, 48, 512, seed=71)
    buf = torch.full((80, raw.shape[1] + 64), 7, dtype=torch.uint8, device="cuda")
    run = buf[16:16 + 48].view(-1)[: raw.size].view(48, raw.shape[1])
    run.copy_(_dev(raw))
    before = buf.clone()
    iq3_pack.pack_(run, o.IQ3_S)
    np.testing.assert_array_equal(run.cpu().numpy(), _tile.pack(raw))
    outside = torch.ones_like(buf, dtype=torch.bool)
    outside.view(-1)[16 * buf.shape[1]:16 * buf.shape[1] + raw.size] = False
    assert torch.equal(buf[outside], before[outside])


@pytest.mark.parametrize("n", [1, 2, 4, 8, 12, 32, 33, 130])
@pytest.mark.parametrize("k", [512, 5120])
def test_packed_ops_vs_q81(n, k):
    from vllm_gguf_plugin.quantization import iq3_pack

    rows = 64
    raw = _w(o.IQ3_S, rows, k, seed=n + k)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    x = _x(n, k, seed=n + 500)
    op = "lcpp_mul_mat_vec_iq3_mma_packed" if n <= 32 else "lcpp_mul_mat_iq3_packed"
    y = getattr(C(), op)(w, x.cuda(), o.IQ3_S, rows).cpu().numpy()
    # the decode op quantises X as block_q8_1 at every row count (lcpp_shim.cu:883-888)
    ref = o.q81_model(raw, o.IQ3_S, x, layout="mmvq" if n <= 32 else "mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)


# ------------------------------------------------------------------------------------ prefill
# Product ops from 256 activation rows on run the 128 x 128-tile prefill GEMM.
PREFILL_N = [256, 300, 600]


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [256, 330])
def test_prefill_exact_integer_dots(qt, n):
    """Rows past the last full 128-row group and activation rows past the last 16-column tile."""
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k = 144 if qt == o.IQ3_S else 150, 512
    raw = _exact_weights(qt, rows, k, seed=130 + n)
    x = _exact_x(n, k, seed=140 + n, dtype=torch.float32)
    want = _exact_ref(raw, qt, x)
    if qt == o.IQ3_S:
        w = iq3_pack.pack(_dev(raw), qt)
        y = C().lcpp_mul_mat_iq3_packed(w, x.cuda(), qt, rows).cpu().numpy()
    else:
        y = C().lcpp_mul_mat_q(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), want)
    assert (y == y.astype(np.int64)).all()


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
def test_prefill_wide_exact_integer_dots(qt):
    """A grid of 256 workgroup tiles (the prefill GEMM's wide-workgroup plan for IQ3_S / Q4_K),
    in the exact-integer mode; with every scale 1 the float64 q81 model is the exact integer."""
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k, n = 4096, 512, 2048
    raw = _exact_weights(qt, rows, k, seed=150)
    x = _exact_x(n, k, seed=151, dtype=torch.float32)
    want = o.q81_model(raw, qt, x, layout="mmq")
    assert np.abs(want).max() < 2 ** 24 and (want == np.round(want)).all()
    if qt == o.IQ3_S:
        y = C().lcpp_mul_mat_iq3_packed(iq3_pack.pack(_dev(raw), qt), x.cuda(), qt, rows)
    else:
        y = C().lcpp_mul_mat_q(_dev(raw), x.cuda(), qt, rows)
    np.testing.assert_array_equal(y.cpu().numpy().astype(np.float64), want)


@pytest.mark.parametrize("qt", [o.Q4_K, o.IQ4_XS, o.Q6_K], ids=lambda t: TN[t])
@pytest.mark.parametrize("n", PREFILL_N)
def test_prefill_vs_q81(qt, n):
    rows, k = 272, 1024
    raw = _w(qt, rows, k, seed=n * 17 + qt)
    x = _x(n, k, seed=n + 600)
    x[-1, 256:288] = 0  # an all-zero slice
    y = C().lcpp_mul_mat_q(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)


def test_prefill_q6k_largest_subscales():
    """Q6_K on the fp16 prefill GEMM folds each 16-value sub-scale into the decoded operand;
    (q - 32) * sc is exact in fp16 up to 2048 and rounds beyond. Every sub-scale at +-127 (each
    product of magnitude 2048..4064 then rounds): the output still meets the fp32 bar of the
    float64 model, and an exact-integer run with sub-scales in [-64, 64] (odd products up to
    2047 in magnitude, all exact) matches the integer sum."""
    rows, k, n = 144, 1024, 300
    raw = _w(o.Q6_K, rows, k, seed=611)
    b = raw.reshape(-1, o.BLOCK_BYTES[o.Q6_K])
    sign = np.random.default_rng(612).choice([-1, 1], size=(b.shape[0], 16))
    b[:, 192:208] = (127 * sign).astype(np.int8).view(np.uint8)
    x = _x(n, k, seed=613)
    y = C().lcpp_mul_mat_q(_dev(raw), x.cuda(), o.Q6_K, rows).cpu().numpy()
    ref = o.q81_model(raw, o.Q6_K, x, layout="mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)
    raw = _exact_weights(o.Q6_K, rows, k, seed=614)
    b = raw.reshape(-1, o.BLOCK_BYTES[o.Q6_K])
    b[:, 192:208] = np.random.default_rng(615).integers(-64, 65, size=(b.shape[0], 16)).astype(np.int8).view(np.uint8)
    x = _exact_x(n, k, seed=616, dtype=torch.float32)
    y = C().lcpp_mul_mat_q(_dev(raw), x.cuda(), o.Q6_K, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, o.Q6_K, x))


@pytest.mark.parametrize("n", PREFILL_N)
@pytest.mark.parametrize("k", [512, 1536])
def test_prefill_packed_xxs_exact(n, k):
    """IQ3_XXS in its unit layout on the fp16 prefill GEMM (operand w * ls, row scale d / 4), in
    the exact mode: the product ops' slice values dot / 4 summed, multiples of 1/4 exact in fp32;
    144 rows (a partial last 128-row group) and K = 1536 (a ragged last unit-block)."""
    from vllm_gguf_plugin.quantization import iq3_pack

    rows = 144
    raw = _exact_weights(o.IQ3_XXS, rows, k, seed=160 + n + k)
    x = _exact_x(n, k, seed=170 + n, dtype=torch.float32)
    want = _exact_ref(raw, o.IQ3_XXS, x, form="mmq")
    w = iq3_pack.pack(_dev(raw), o.IQ3_XXS)
    y = C().lcpp_mul_mat_iq3_packed(w, x.cuda(), o.IQ3_XXS, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.float64), want)


@pytest.mark.parametrize("rows,k,n", [(272, 5120, 256), (272, 5120, 600), (2048, 5120, 2048)])
def test_prefill_packed_xxs_vs_q81(rows, k, n):
    """IQ3_XXS prefill (the 4-wave and the 8-wave plans) against the q81 model of the product ops."""
    from vllm_gguf_plugin.quantization import iq3_pack

    raw = _w(o.IQ3_XXS, rows, k, seed=rows + n + 9)
    x = _x(n, k, seed=n + 710)
    x[-1, 256:288] = 0  # an all-zero slice
    y = C().lcpp_mul_mat_iq3_packed(iq3_pack.pack(_dev(raw), o.IQ3_XXS), x.cuda(), o.IQ3_XXS, rows).cpu().numpy()
    ref = o.q81_model(raw, o.IQ3_XXS, x, layout="mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)


@pytest.mark.parametrize("n", PREFILL_N)
@pytest.mark.parametrize("k", [512, 5120])
def test_prefill_packed_vs_q81(n, k):
    from vllm_gguf_plugin.quantization import iq3_pack

    rows = 272
    raw = _w(o.IQ3_S, rows, k, seed=n + k + 7)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    x = _x(n, k, seed=n + 700)
    y = C().lcpp_mul_mat_iq3_packed(w, x.cuda(), o.IQ3_S, rows).cpu().numpy()
    ref = o.q81_model(raw, o.IQ3_S, x, layout="mmq")
    assert o.rel_l2(y, ref) <= 1e-3, o.rel_l2(y, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
def test_prefill_16bit_x(qt, dtype):
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k, n = 128, 1024, 260
    raw = _w(qt, rows, k, seed=qt + 800)
    x = _x(n, k, seed=801, dtype=dtype)
    if qt == o.IQ3_S:
        y = C().lcpp_mul_mat_iq3_packed(iq3_pack.pack(_dev(raw), qt), x.cuda(), qt, rows)
    else:
        y = C().lcpp_mul_mat_q(_dev(raw), x.cuda(), qt, rows)
    assert y.dtype == dtype and y.shape == (n, rows)
    ref = o.q81_model(raw, qt, x, layout="mmq")
    assert o.rel_l2(y.float().cpu().numpy(), ref) <= TIGHT[dtype]


@pytest.mark.parametrize("n,rows,k", [(1, 16 * 700, 2048), (2, 16 * 700, 2048), (3, 16 * 700, 2048),
                                      (4, 16 * 700, 2048), (2, 16 * 200, 21504)])
def test_packed_gemv_many_tiles(n, rows, k):
    """The persistent GEMV on q8_1 input: 11200 rows have more 16-row tiles than its grid (two
    workgroups per CU), so each workgroup loops over several tiles (1-4 activation rows; K = 2048
    is 8 blocks, one per wave); 3200 x 21504 at two rows is a large weight with fewer tiles than
    the grid. X given as q8_1 (x_q8), which keeps n = 1 off the fused path: exact-integer dots,
    the q81 model, and bit-identical CUDA-graph replays."""
    from vllm_gguf_plugin.quantization import iq3_pack

    op = C().lcpp_mul_mat_vec_iq3_mma_packed
    raw = _exact_weights(o.IQ3_S, rows, k, seed=160 + n)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    x = _exact_x(n, k, seed=161 + n, dtype=torch.float32).cuda()
    q8 = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)
    y = op(w, x, o.IQ3_S, rows, q8).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, o.IQ3_S, x.cpu()))
    raw = _w(o.IQ3_S, rows, k, seed=170 + n)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    x = _x(n, k, seed=171 + n, dtype=torch.bfloat16).cuda()
    q8 = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)
    eager = op(w, x, o.IQ3_S, rows, q8)
    assert o.rel_l2(eager.float().cpu().numpy(), o.q81_model(raw, o.IQ3_S, x.cpu())) <= TIGHT[torch.bfloat16]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = op(w, x, o.IQ3_S, rows, q8)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# ------------------------------------------------------------------------------------ x_q8, graphs
@pytest.mark.parametrize("qt", TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [2, 4, 8])
def test_shared_x_q8_equals_own_quantize(qt, n):
    """A caller's x_q8 gives the same bits as the op's own quantisation, on the GEMV and (from a
    per-type row count on) on the MFMA GEMM, which converts x_q8 into its operand layout."""
    rows, k = 64, 1024
    raw = _dev(_w(qt, rows, k, seed=80 + n))
    x = _x(n, k, seed=81 + n, dtype=torch.bfloat16).cuda()
    q8 = C().lcpp_quantize_q8_1(x, qt, False, False)
    a = getattr(C(), VEC_OP[qt])(raw, x, qt, rows)
    b = getattr(C(), VEC_OP[qt])(raw, x, qt, rows, q8)
    assert torch.equal(a, b)


@pytest.mark.parametrize("n,dtype", [(1, torch.bfloat16), (1, torch.float16), (1, torch.float32),
                                     (4, torch.bfloat16), (8, torch.bfloat16), (24, torch.bfloat16)])
def test_shared_x_q8_packed(n, dtype):
    """n = 1 on these small weights takes the GEMV that quantises X itself: it must give the
    bits of the q8_1 quantiser followed by the GEMV."""
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k = 64, 1024
    w = iq3_pack.pack(_dev(_w(o.IQ3_S, rows, k, seed=90 + n)), o.IQ3_S)
    x = _x(n, k, seed=91 + n, dtype=dtype).cuda()
    x[:, 64:96] = 0  # an all-zero slice (d = 0, q = 0)
    q8 = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)
    a = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows)
    b = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows, q8)
    assert torch.equal(a, b)


@pytest.mark.parametrize("qt", [o.Q4_K, o.IQ4_XS, o.Q6_K], ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 2])
def test_raw_gemv_tiles(qt, n):
    """The GGUF-row decode GEMV's tile kernel (1-2 rows, K >= 2048): a row count that is not a
    multiple of 16 and more tiles than the persistent grid; exact-integer dots, the q81 model and
    bit-identical CUDA-graph replays."""
    rows, k = 16 * 700 + 5, 2048
    op = getattr(C(), VEC_OP[qt])
    raw = _exact_weights(qt, rows, k, seed=190 + n)
    x = _exact_x(n, k, seed=191 + n, dtype=torch.float32)
    y = op(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x))
    raw = _w(qt, rows, k, seed=192 + n)
    w = _dev(raw)
    x = _x(n, k, seed=193 + n, dtype=torch.bfloat16).cuda()
    eager = op(w, x, qt, rows)
    assert o.rel_l2(eager.float().cpu().numpy(), o.q81_model(raw, qt, x.cpu())) <= TIGHT[torch.bfloat16]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = op(w, x, qt, rows)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("qt", [o.Q4_K, o.IQ4_XS, o.Q6_K], ids=lambda t: TN[t])
@pytest.mark.parametrize("n,k", [(3, 17408), (4, 17408), (1, 40960)])
def test_rows_gemv_k_phases(qt, n, k):
    """The row-chunk GEMV when X's q8_1 exceeds its LDS budget: K runs in two phases of blocks
    with X staged per phase between barriers (21 tiles, the last one partial, one per workgroup):
    exact-integer dots (at K = 17408; at K = 40960 the exact sums pass 2^24), the q81 model and
    bit-identical CUDA-graph replays. (Q4_K at 4 rows over K phases runs the int8 small GEMM.)"""
    rows = 16 * 20 + 5
    op = getattr(C(), VEC_OP[qt])
    if k <= 17408:
        raw = _exact_weights(qt, rows, k, seed=200 + n)
        x = _exact_x(n, k, seed=201 + n, dtype=torch.float32)
        y = op(_dev(raw), x.cuda(), qt, rows).cpu().numpy()
        np.testing.assert_array_equal(y.astype(np.int64), _exact_ref(raw, qt, x))
    raw = _w(qt, rows, k, seed=202 + n)
    w = _dev(raw)
    x = _x(n, k, seed=203 + n, dtype=torch.bfloat16).cuda()
    eager = op(w, x, qt, rows)
    assert o.rel_l2(eager.float().cpu().numpy(), o.q81_model(raw, qt, x.cpu())) <= TIGHT[torch.bfloat16]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = op(w, x, qt, rows)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("rows,k,n,dtype", [
    (16 * 700, 2048, 1, torch.bfloat16), (16 * 700, 2048, 1, torch.float16), (16 * 700, 2048, 1, torch.float32),
    (16 * 700, 2048, 2, torch.bfloat16), (16 * 700, 2048, 2, torch.float32),
    (17408, 5120, 1, torch.bfloat16), (17408, 5120, 2, torch.bfloat16),
    (8192, 5120, 1, torch.bfloat16), (6144, 5120, 1, torch.bfloat16),
    (5120, 6144, 1, torch.bfloat16), (5120, 6144, 1, torch.float16), (5120, 6144, 1, torch.float32),
    (512, 6144, 1, torch.bfloat16), (512, 6144, 1, torch.float32)])
def test_fused_quantisation_large_weights(lib, rows, k, n, dtype):
    """Without x_q8, the packed decode op quantises X itself. The stream kernel (weights of at least
    one 4-row unit per CU, K <= 8192) quantises all of X into LDS first, at one or two rows; the
    one-tile kernel quantises block by block at one row on smaller weights (512 rows). It must give
    the bits of the q8_1 quantiser followed by the GEMV. That these shapes take the fused path is
    asserted from the op's workspace size (none: no q8_1 copy of X)."""
    from vllm_gguf_plugin.quantization import iq3_pack

    assert lib.gguf_op_workspace_bytes(6, o.IQ3_S, rows, k, n, 0) == 0  # the fused GEMV
    assert lib.gguf_op_workspace_bytes(6, o.IQ3_S, rows, k, n, 1) == 0
    w = iq3_pack.pack(_dev(_w(o.IQ3_S, rows, k, seed=180 + n)), o.IQ3_S)
    x = _x(n, k, seed=181 + n, dtype=dtype).cuda()
    x[:, 96:128] = 0  # an all-zero slice (d = 0, q = 0)
    q8 = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)
    a = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows)
    b = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows, q8)
    assert torch.equal(a, b)


def _tie_slices(k, dtype, seed):
    """One activation row whose 32-value slices put x / d exactly on, or one fp32 ulp either side
    of, a half-integer (d = amax / 127), with all-zero, tiny-amax, negative, infinite and NaN
    slices among random ones: the cases where a quantiser that divides differs from one that
    multiplies by a reciprocal."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(k, generator=g, dtype=torch.float64)
    ks = torch.arange(32, dtype=torch.float64)
    halves = (ks * 4 % 127) + 0.5                  # k + 0.5 for k in 0..126
    for sl in range(k // 32):
        v = x[32 * sl: 32 * sl + 32]
        kind = sl % 9
        scale = 2.0 ** float((sl // 9) % 7 - 3)
        if kind == 0:    # exact ties, d = scale
            v[:] = halves * scale
            v[31] = 127 * scale
        elif kind == 1:  # negative ties
            v[:] = -halves * scale
            v[31] = -127 * scale
        elif kind == 2:  # one fp32 ulp above / below the tie
            t = (halves * scale).to(torch.float32)
            v[:] = torch.where(ks % 2 == 0, torch.nextafter(t, t + 1), torch.nextafter(t, t - 1)).double()
            v[31] = 127 * scale
        elif kind == 3:
            v[:] = 0.0
        elif kind == 4:  # tiny amax: fp32 subnormal d (bf16 / fp32 only)
            v[:] = v * 1e-37
        elif kind == 5 and sl % 4 == 1:
            v[7] = float("inf")
        elif kind == 6 and sl % 4 == 2:
            v[3] = float("nan")
    return x.to(dtype)


@pytest.mark.parametrize("n,dtype,rows", [(1, torch.bfloat16, 16 * 700), (1, torch.float16, 16 * 700),
                                          (1, torch.float32, 16 * 700), (2, torch.bfloat16, 16 * 700),
                                          (2, torch.float32, 16 * 700), (1, torch.bfloat16, 512),
                                          (1, torch.float16, 512), (1, torch.float32, 512)])
def test_fused_quantisation_ties(n, dtype, rows):
    """The packed GEMV's in-kernel quantisation (all of X into LDS on the stream kernel, 11200 rows;
    block by block on the one-tile kernel, 512 rows) rounds x / d from a reciprocal product
    and takes the IEEE division for values near a tie, non-finite values and tiny scales: its
    bytes, and so the outputs, must equal those of the q8_1 quantiser bit for bit (NaN included)."""
    from vllm_gguf_plugin.quantization import iq3_pack

    k = 4096  # 11200 x 4096: more than one unit per CU (stream kernel); 512 rows: the one-tile kernel
    w = iq3_pack.pack(_dev(_w(o.IQ3_S, rows, k, seed=190 + n)), o.IQ3_S)
    x = torch.stack([_tie_slices(k, dtype, seed=191 + c) for c in range(n)]).cuda()
    q8 = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)
    a = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows)
    b = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows, q8)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(a.view(bits), b.view(bits))


@pytest.mark.parametrize("n", [1, 2, 3, 4])
@pytest.mark.parametrize("rows,k", [(16 * 70, 5632), (16 * 70, 5120), (4096, 1536)])
def test_stream_gemv_units(n, rows, k):
    """The stream GEMV over 4-row units: 1120 rows give 280 units over the CUs, so workgroups own 1
    or 2 units and waves' runs start and end inside units; K = 5632 (22 blocks) ends every unit in
    a 2-block unit-block, whose other lanes must add nothing; 4096 x 1536 has 6 blocks per row.
    With x_q8 (q8_1 input, 1-4 rows) and without (X quantised in the kernel, 1-2 rows): within 1e-3
    of the q81 model, the two bit-identical, and graph replays bit-identical."""
    from vllm_gguf_plugin.quantization import iq3_pack

    raw = _w(o.IQ3_S, rows, k, seed=230 + n)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    x = _x(n, k, seed=231 + n, dtype=torch.bfloat16).cuda()
    q8 = C().lcpp_quantize_q8_1(x, o.IQ3_S, False, False)
    b = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows, q8)
    ref = o.q81_model(raw, o.IQ3_S, x.cpu())
    assert o.rel_l2(b.float().cpu().numpy(), ref) <= TIGHT[torch.bfloat16]
    a = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows)
    assert torch.equal(a, b)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x, o.IQ3_S, rows, q8)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, b)


ROWS_TYPES = [o.Q4_K, o.IQ4_XS, o.Q6_K]
OP_ID = {"lcpp_mul_mat_vec_q": 0, "lcpp_mul_mat_vec_own": 4}


@pytest.mark.parametrize("qt", ROWS_TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 2])
@pytest.mark.parametrize("rows,k", [(16 * 700 + 5, 2048), (1000, 5120), (333, 6144)])
def test_rows_fused_quantisation(lib, qt, n, rows, k):
    """Without x_q8, a Q4_K / IQ4_XS / Q6_K decode op at one or two rows and K <= 8192 quantises X
    inside the row-chunk GEMV, each wave its own part of X. It must give the bits of the q8_1
    quantiser followed by the GEMV (partial last tile at 333 rows, three groups per lane at two rows
    of K = 6144). The zero workspace shows that the fused path is the one taken."""
    op = VEC_OP[qt]
    assert lib.gguf_op_workspace_bytes(OP_ID[op], qt, rows, k, n, 0) == 0
    w = _dev(_w(qt, rows, k, seed=210 + n))
    x = _x(n, k, seed=211 + n, dtype=torch.bfloat16).cuda()
    x[:, 96:128] = 0  # an all-zero slice (d = 0, q = 0)
    q8 = C().lcpp_quantize_q8_1(x, qt, False, False)
    a = getattr(C(), op)(w, x, qt, rows)
    b = getattr(C(), op)(w, x, qt, rows, q8)
    assert torch.equal(a, b)


@pytest.mark.parametrize("qt", ROWS_TYPES, ids=lambda t: TN[t])
@pytest.mark.parametrize("n", [1, 2])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=str)
def test_rows_fused_quantisation_ties(qt, n, dtype):
    """The row-chunk GEMV's in-kernel quantisation on values on and next to ties, infinities, NaN
    and tiny scales: outputs equal to those of the q8_1 quantiser + GEMV bit for bit (NaN
    included); Q4_K and Q6_K also take the sums of q from the quantised bytes."""
    rows, k = 1000, 4096
    w = _dev(_w(qt, rows, k, seed=220 + n))
    x = torch.stack([_tie_slices(k, dtype, seed=221 + c) for c in range(n)]).cuda()
    q8 = C().lcpp_quantize_q8_1(x, qt, False, False)
    a = getattr(C(), VEC_OP[qt])(w, x, qt, rows)
    b = getattr(C(), VEC_OP[qt])(w, x, qt, rows, q8)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(a.view(bits), b.view(bits))


@pytest.mark.parametrize("op,qt,n,packed", [
    ("lcpp_mul_mat_vec_iq3_mma_packed", o.IQ3_S, 4, True),
    ("lcpp_mul_mat_iq3_packed", o.IQ3_S, 32, True),
    ("lcpp_mul_mat_vec_own", o.Q4_K, 4, False),
    ("lcpp_mul_mat_mma_k", o.Q4_K, 16, False),
    ("lcpp_mul_mat_q", o.Q6_K, 48, False),
    ("lcpp_mul_mat_vec_q", o.IQ4_XS, 1, False),
    ("lcpp_mul_mat_iq3_packed", o.IQ3_S, 300, True),
    ("lcpp_mul_mat_q", o.Q4_K, 260, False),
    ("lcpp_mul_mat_iq3_packed", o.IQ3_S, 64, True),
    ("lcpp_mul_mat_q", o.Q4_K, 100, False),
])
def test_graph_replay_bit_exact(op, qt, n, packed):
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k = 256, 2048
    w = _dev(_w(qt, rows, k, seed=90))
    if packed:
        w = iq3_pack.pack(w, qt)
    fn = getattr(C(), op)
    xs = [_x(n, k, seed=91 + i, dtype=torch.bfloat16).cuda() for i in range(3)]
    eager = [fn(w, x, qt, rows).clone() for x in xs]
    static_x = xs[0].clone()
    fn(w, static_x, qt, rows)  # warm up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = fn(w, static_x, qt, rows)
    for rep in range(2):
        for i, x in enumerate(xs):
            static_x.copy_(x)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager[i]), (op, rep, i)


# ------------------------------------------------------------------------------------ full sizes
@pytest.mark.parametrize("n", [1, 4])
def test_full_size_iq3s_gate_packed(n):
    """The decode benchmark's gate shape at its real size (17408 x 5120), M = 1 and 4, through the packed path."""
    from vllm_gguf_plugin.quantization import iq3_pack

    rows, k = 17408, 5120
    raw = _w(o.IQ3_S, rows, k, seed=2)
    w = iq3_pack.pack(_dev(raw), o.IQ3_S)
    x = _x(n, k, seed=3, dtype=torch.bfloat16)
    y = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x.cuda(), o.IQ3_S, rows).float().cpu().numpy()
    assert o.rel_l2(y, o.q81_model(raw, o.IQ3_S, x)) <= TIGHT[torch.bfloat16]


def test_full_size_q4k_cpu_config():
    """The CPU-path benchmark case: Q4_K 4096 x 4096 with d, dmin ~ |N(0, 1e-3)| (the config's
    recipe), X 1 x 4096 fp32 N(0,1), seed 0."""
    rows = k = 4096
    raw = o.random_blocks(np.random.default_rng(0), o.Q4_K, rows, k, scale_sigma=1e-3)
    x = torch.from_numpy(np.random.default_rng(0).standard_normal((1, k)).astype(np.float32))
    y = C().lcpp_mul_mat_vec_q(_dev(raw), x.cuda(), o.Q4_K, rows).cpu().numpy()
    assert o.rel_l2(y, o.q81_model(raw, o.Q4_K, x)) <= 1e-3
