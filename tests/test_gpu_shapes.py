"""Parity at the benchmark configs' full shapes and on every launch plan they reach, through the
C ABI (torch.ops._C_gguf -> libgguf_mi355x.so). Needs an MI355X.

  * the IQ3_S down shape 5120 x 17408 at M = 1..4 against the oracle's q81 model
    (the gate shape 17408 x 5120 is in test_gpu_parity.py);
  * the packed IQ3_S GEMM's four-wave plan (gemm_iq3s_tile_kernel with one column tile on
    weights of 512 tiles or more: 5..16 activation rows, decode and product ops);
  * a prefill product at M = 8192, K = 5120, N = 17408 with the benchmark's
    activations (1 % outliers of magnitude 20), checked on sampled weight rows;
  * two decoder layers of the GSQ-RCO mix plus the Q6_K 151936 x 5120 head at
    M = 1, 4, 16, 32, every call captured in one CUDA graph, sampled rows of every product
    against the q81 model and two replays byte-equal;
  * the Q4_K min term of the product ops in the reference's MMQ form on residual-heavy
    activations (vecdotq.cuh:549-552), and of the decode ops in the MMVQ form (:525).
Bars as in test_gpu_parity.py: 1e-3 relative L2 with fp32 activations, 5e-3 with bf16 (the output
is rounded to bf16), bit-exact where every scale is 1.
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


def _pack(w, qt=o.IQ3_S):
    from vllm_gguf_plugin.quantization import iq3_pack

    return iq3_pack.pack(w, qt)


def x_bench(n, k, seed):
    """The benchmark configs' activations: bf16 N(0,1) with a seeded 1 % of the entries set to
    +-20; bench.py draws its prefill input with this same recipe."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, k, generator=g)
    m = torch.rand(n, k, generator=g) < 0.01
    x[m] = 20.0 * torch.sign(torch.randn(int(m.sum()), generator=g))
    return x.to(torch.bfloat16)


def _sampled(rows, count, seed):
    """`count` weight rows spread over [0, rows): the first and last of the weight and a seeded
    sample between them."""
    rng = np.random.default_rng(seed)
    pick = set(rng.choice(rows, size=min(rows, count) - 2, replace=False).tolist()) | {0, rows - 1}
    return np.array(sorted(pick))


# ------------------------------------------------------------------------------------ configs[1]
@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_full_size_iq3s_down_packed(n):
    """IQ3_S down projection 5120 x 17408 (320 tiles, 68 K blocks) through the packed decode op:
    quantise + one-tile GEMV at 1-4 rows (its 8- and 4-wave K splits over 68 blocks). Every output
    row against the q81 model at M = 1 and 4, 1024 sampled rows at M = 2 and 3."""
    rows, k = 5120, 17408
    raw = w_rand(o.IQ3_S, rows, k, seed=40 + n)
    w = _pack(dev(raw))
    x = x_rand(n, k, seed=41 + n, dtype=torch.bfloat16)
    y = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x.cuda(), o.IQ3_S, rows).float().cpu().numpy()
    rs = np.arange(rows) if n in (1, 4) else _sampled(rows, 1024, seed=n)
    assert o.rel_l2(y[:, rs], o.q81_model(raw[rs], o.IQ3_S, x)) <= TIGHT[torch.bfloat16]


def test_full_size_iq3s_down_exact_integer():
    """The same shape in the exact-integer mode: every output is the oracle's int64 sum."""
    rows, k = 5120, 17408
    raw = exact_weights(o.IQ3_S, rows, k, seed=45)
    w = _pack(dev(raw))
    for n in (1, 4):
        x = exact_x(n, k, seed=46 + n, dtype=torch.float32)
        y = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x.cuda(), o.IQ3_S, rows).cpu().numpy()
        np.testing.assert_array_equal(y.astype(np.int64), exact_ref(raw, o.IQ3_S, x), err_msg=f"n={n}")


@pytest.mark.parametrize("n", [3, 4])
def test_stream_lds_limit(n):
    """53264 x 5120 (13316 units, 53 per CU at 256 CUs): at 4 rows X's q8_1 and the partial-sum
    slots of 53 units need 131,584 B of dynamic LDS, more than the 131,056 B a workgroup may take
    beside the table, so the decode op takes the one-tile GEMV; at 3 rows (98,688 B) the stream
    GEMV. Sampled rows against the q81 model, bf16 X."""
    rows, k = 53264, 5120
    raw = w_rand(o.IQ3_S, rows, k, seed=90 + n)
    w = _pack(dev(raw))
    x = x_rand(n, k, seed=91 + n, dtype=torch.bfloat16)
    y = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x.cuda(), o.IQ3_S, rows).float().cpu().numpy()
    rs = _sampled(rows, 768, seed=92 + n)
    assert o.rel_l2(y[:, rs], o.q81_model(raw[rs], o.IQ3_S, x)) <= TIGHT[torch.bfloat16]


# ------------------------------------------------------------------------------------ tile GEMM, 4 waves
# The packed IQ3_S GEMM runs one column tile (up to 16 activation rows) with four K-splitting
# waves per 16-row tile on weights of 512 tiles or more (8192 rows), eight waves below.
@pytest.mark.parametrize("n", [5, 8, 9, 16])
def test_tile_gemm_four_waves_exact_integer(n):
    rows, k = 8192, 2048
    raw = exact_weights(o.IQ3_S, rows, k, seed=60 + n)
    w = _pack(dev(raw))
    x = exact_x(n, k, seed=61 + n, dtype=torch.float32)
    want = exact_ref(raw, o.IQ3_S, x)
    ops = ["lcpp_mul_mat_vec_iq3_mma_packed"] + (["lcpp_mul_mat_iq3_packed"] if n > 8 else [])
    for op in ops:
        y = getattr(C(), op)(w, x.cuda(), o.IQ3_S, rows).cpu().numpy()
        np.testing.assert_array_equal(y.astype(np.int64), want, err_msg=op)


@pytest.mark.parametrize("n", [5, 8, 16])
def test_tile_gemm_four_waves_vs_q81(n):
    """17408 x 5120 (the gate shape, 1088 tiles): the decode op's q8_1 arithmetic (block_q8_1)
    and the product op's MMQ arithmetic, each against its q81 model, and graph replays."""
    rows, k = 17408, 5120
    raw = w_rand(o.IQ3_S, rows, k, seed=70 + n)
    w = _pack(dev(raw))
    x = x_rand(n, k, seed=71 + n)
    rs = _sampled(rows, 512, seed=72 + n)
    y = C().lcpp_mul_mat_vec_iq3_mma_packed(w, x.cuda(), o.IQ3_S, rows)
    assert o.rel_l2(y.cpu().numpy()[:, rs], o.q81_model(raw[rs], o.IQ3_S, x)) <= 1e-3
    xd = x.cuda()
    graph_replays_equal(lambda: C().lcpp_mul_mat_vec_iq3_mma_packed(w, xd, o.IQ3_S, rows), y)
    if n > 8:
        y = C().lcpp_mul_mat_iq3_packed(w, xd, o.IQ3_S, rows).cpu().numpy()
        assert o.rel_l2(y[:, rs], o.q81_model(raw[rs], o.IQ3_S, x, layout="mmq")) <= 1e-3


# ------------------------------------------------------------------------------------ configs[3]
@pytest.mark.parametrize("qt", [o.IQ3_S, o.Q4_K, o.Q6_K], ids=lambda t: o.TYPE_NAMES[t])
def test_prefill_full_size_sampled(qt):
    """M = 8192, K = 5120, N = 17408, the benchmark's outlier activations; the whole product on
    the GPU, 256 sampled weight rows (all 8192 activation rows) against the q81 model."""
    rows, k, n = 17408, 5120, 8192
    raw = w_rand(qt, rows, k, seed=80 + qt)
    w = dev(raw)
    if qt == o.IQ3_S:
        w = _pack(w)
    x = x_bench(n, k, seed=81)
    op = C().lcpp_mul_mat_iq3_packed if qt == o.IQ3_S else C().lcpp_mul_mat_q
    y = op(w, x.cuda(), qt, rows)
    assert y.shape == (n, rows) and y.dtype == torch.bfloat16
    rs = _sampled(rows, 256, seed=82)
    got = y[:, torch.from_numpy(rs).cuda()].float().cpu().numpy()
    del y
    assert np.isfinite(got).all()
    assert o.rel_l2(got, o.q81_model(raw[rs], qt, x, layout="mmq")) <= TIGHT[torch.bfloat16]


# ------------------------------------------------------------------------------------ configs[4]
LAYER = [("q", o.IQ3_S, 6144, 5120), ("k", o.IQ3_S, 1024, 5120), ("v", o.IQ3_S, 1024, 5120),
         ("o", o.IQ3_S, 5120, 6144), ("gate", o.IQ3_S, 17408, 5120), ("up", o.IQ3_S, 17408, 5120),
         ("down", o.IQ4_XS, 5120, 17408)]
HEAD = ("head", o.Q6_K, 151936, 5120)


@pytest.fixture(scope="module")
def decoder_weights():
    """Two layers of the GSQ-RCO mix and the Q6_K head: (name, type, rows, k, raw, device)."""
    out = []
    for li in range(2):
        for name, qt, rows, k in LAYER:
            raw = w_rand(qt, rows, k, seed=900 + 10 * li + len(out))
            w = dev(raw)
            out.append((f"{li}.{name}", qt, rows, k, raw, _pack(w) if qt == o.IQ3_S else w))
    name, qt, rows, k = HEAD
    raw = w_rand(qt, rows, k, seed=999)
    out.append((name, qt, rows, k, raw, dev(raw)))
    return out


@pytest.mark.parametrize("m", [1, 4, 16, 32])
def test_decoder_sweep_graph(decoder_weights, m):
    """Every product of two layers and the head at M activation rows, each through the op the
    routing table picks, captured in one CUDA graph: two replays give identical bytes, equal to
    the eager calls, and 64 sampled rows of each product are within the bf16 bar of the q81 model
    in the layout the op quantises with."""
    from vllm_gguf_plugin.quantization import linear

    xs = {k: x_bench(m, k, seed=1000 + k + m) for k in (5120, 6144, 17408)}
    xd = {k: v.cuda() for k, v in xs.items()}
    calls = []
    for name, qt, rows, k, raw, w in decoder_weights:
        op = linear._lcpp_op(m, qt, rows, k, qt == o.IQ3_S)
        calls.append((name, qt, rows, k, raw, w, op))
    fns = [lambda w=w, op=op, x=xd[k], qt=qt, rows=rows: getattr(C(), op)(w, x, qt, rows)
           for _, qt, rows, k, _, w, op in calls]
    eager = [f() for f in fns]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    ys = []
    with torch.cuda.graph(g):
        for f in fns:
            ys.append(f())
    g.replay()
    torch.cuda.synchronize()
    first = [y.clone() for y in ys]
    g.replay()
    torch.cuda.synchronize()
    for (name, *_rest), a, b, e in zip(calls, first, ys, eager):
        assert torch.equal(a, b), f"{name}: replays differ"
        assert torch.equal(a, e), f"{name}: graph differs from eager"
    for (name, qt, rows, k, raw, _, op), y in zip(calls, first):
        rs = _sampled(rows, 64, seed=rows + m)
        layout = "mmq" if op in linear._OWN_QUANTIZE_OPS else "mmvq"
        got = y[:, torch.from_numpy(rs).cuda()].float().cpu().numpy()
        e = o.rel_l2(got, o.q81_model(raw[rs], qt, xs[k], layout=layout))
        assert e <= TIGHT[torch.bfloat16], (name, op, e)


# ------------------------------------------------------------------------------------ Q4_K min term
def _residual_heavy_x(n, k, seed):
    """Per 32-value slice one value of magnitude a and 31 of magnitude 0.49 * a / 127, of one
    sign: every small value rounds to q = 0, so sum(x) exceeds d * sum(q) by about 15 d."""
    rng = np.random.default_rng(seed)
    a = np.exp2(rng.uniform(-2, 2, (n, k // 32, 1))).astype(np.float32)
    sign = rng.choice([-1.0, 1.0], size=(n, k // 32, 1)).astype(np.float32)
    x = np.broadcast_to(a * np.float32(0.49 / 127), (n, k // 32, 32)).copy()
    x[..., rng.integers(0, 32)] = a[..., 0]
    return torch.from_numpy((x * sign).reshape(n, k).astype(np.float32))


@pytest.mark.parametrize("op,n", [("lcpp_mul_mat_mma_k", 9), ("lcpp_mul_mat_mma_k", 32), ("lcpp_mul_mat_q", 48),
                                  ("lcpp_mul_mat_q", 100), ("lcpp_mul_mat_q", 300),
                                  ("lcpp_mul_mat_vec_own", 3), ("lcpp_mul_mat_vec_own", 8),
                                  ("lcpp_mul_mat_vec_q", 1)])
def test_q4k_min_term_form(op, n):
    """Q4_K on activations whose slice sums differ from d * sum(q) by about 10 %: the product ops
    (int8 small GEMM, fp16 small GEMM at 64-255 rows, prefill from 256 rows) follow the MMQ form
    dmin * m * half(sum x), the decode ops (GEMV, and the int8 GEMM they take from 3 rows) the
    MMVQ form dmin * m * d8 * sum(q8); the two forms are more than 1e-2 apart here."""
    rows, k = 2304 if op == "lcpp_mul_mat_vec_own" else 272, 2048
    raw = w_rand(o.Q4_K, rows, k, seed=110 + n)
    x = _residual_heavy_x(n, k, seed=111 + n)
    y = getattr(C(), op)(dev(raw), x.cuda(), o.Q4_K, rows).cpu().numpy()
    mmq, mmvq = o.q81_model(raw, o.Q4_K, x, "mmq"), o.q81_model(raw, o.Q4_K, x, "mmvq")
    assert o.rel_l2(mmq, mmvq) > 1e-2
    want, other = (mmq, mmvq) if op in ("lcpp_mul_mat_mma_k", "lcpp_mul_mat_q") else (mmvq, mmq)
    assert o.rel_l2(y, want) <= 1e-3, (o.rel_l2(y, want), o.rel_l2(y, other))
