"""The GGUF linear method end to end on the GPU: layers built through create_weights, the shard
weight loaders, process_weights_after_loading (the padded run-contiguous weight and the IQ3_S
repack hook) and apply(), against the ops called on each same-type run's own bytes (bit-exact)
and against the CPU oracle (the bf16 bar on sampled rows). The reference tests the same surface
in tests/gpu/test_kernel_parity.py:770-876 (mixed-shard and same-type-run layers),
:1041-1100 (routing on a whole packed tensor), :1103-1151 (the packed layer, all or nothing) and
:216-264 (the vocab head at prompt row counts, fp32-dst chunking and peak memory). Needs an
MI355X.
"""

import numpy as np
import pytest
import torch

import gguf_oracle as o
from _gpu import TIGHT, C, dev, poison_allocator, w_rand

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _ops():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from vllm_gguf_plugin import ops  # noqa: F401

    return torch.ops._C_gguf


def x_bf16(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=g).to(torch.bfloat16)


def build_layer(shards, k, shard_ids=None):
    """A linear layer of the method, loaded shard by shard as vLLM's loader does: create_weights
    under the target device (vLLM's loader builds the model inside `with torch.device(...)`),
    each shard's bytes and type through the parameters' weight loaders, then
    process_weights_after_loading. shards: [(raw uint8 [rows, row_bytes], ggml type)]."""
    from vllm_gguf_plugin.quantization.linear import GGUFLinearMethod

    layer = torch.nn.Module()
    method = GGUFLinearMethod()
    sizes = [r.shape[0] for r, _ in shards]
    with torch.device("cuda"):
        method.create_weights(layer, input_size_per_partition=k, output_partition_sizes=sizes, input_size=k,
                              output_size=sum(sizes), params_dtype=torch.bfloat16)
    if shard_ids is None:
        shard_ids = list(range(len(shards))) if len(shards) > 1 else [None]
    for sid, (raw, qt) in zip(shard_ids, shards):
        layer.weight.weight_loader(layer.weight, dev(raw), sid)
        layer.weight_type.weight_loader(layer.weight_type, torch.tensor(qt), sid)
    method.process_weights_after_loading(layer)
    return layer, method


def routed(raw, x, qt, packed):
    """What the routing table gives for one run on its own bytes (packed: in the tile layout)."""
    from vllm_gguf_plugin.quantization import iq3_pack, linear

    w = dev(raw)
    if packed:
        w = iq3_pack.pack(w, qt)
    return linear._fused_mul_mat_gguf(x, w, qt, None, packed)


def check_oracle(y, runs, x, nsample=48, seed=0):
    """Sampled output columns of each run against the q81 model of the run's op."""
    from vllm_gguf_plugin.quantization import linear

    n, k = x.shape
    col = 0
    for raw, qt, packed in runs:
        rows = raw.shape[0]
        op = linear._lcpp_op(n, qt, rows, k, packed)
        layout = "mmq" if op in linear._OWN_QUANTIZE_OPS else "mmvq"
        rng = np.random.default_rng(seed + rows)
        rs = np.unique(np.concatenate([[0, rows - 1], rng.choice(rows, size=min(rows, nsample), replace=False)]))
        got = y[:, col + torch.from_numpy(rs).cuda()].float().cpu().numpy()
        e = o.rel_l2(got, o.q81_model(raw[rs], qt, x.cpu(), layout=layout))
        assert e <= TIGHT[torch.bfloat16], (qt, rows, op, e)
        col += rows


NS = [1, 2, 4, 8, 9, 16, 32, 128, 300]


@pytest.mark.parametrize("n", NS)
def test_mixed_type_qkv_layer(n):
    """q IQ3_S (6144 rows) with k, v Q4_K (1024 rows each): two runs, the Q4_K run one 2048-row
    product on a view into the padded weight; the IQ3_S run is packed in place; the runs share one
    q8_1 of X where their ops read it. Bit-exact with each run's op on its own bytes."""
    k = 5120
    q, kw, vw = w_rand(o.IQ3_S, 6144, k, 1), w_rand(o.Q4_K, 1024, k, 2), w_rand(o.Q4_K, 1024, k, 3)
    layer, method = build_layer([(q, o.IQ3_S), (kw, o.Q4_K), (vw, o.Q4_K)], k, ["q", "k", "v"])
    w = layer.weight
    assert w.iq3_packed and w.shape == (8192, 144 * 20)
    from vllm_gguf_plugin.quantization.linear import _shard_weight

    lo, hi = w.data_ptr(), w.data_ptr() + w.numel()
    kv = _shard_weight(w, w.shard_offset_map["k"][0], w.shard_offset_map["v"][1], w.shard_offset_map["k"][2])
    assert lo <= kv.data_ptr() < hi and torch.equal(kv, dev(np.concatenate([kw, vw])))  # a view
    x = x_bf16(n, k, seed=10 + n).cuda()
    poison_allocator()
    y = method.apply(layer, x)
    kvraw = np.concatenate([kw, vw])
    ref = torch.cat([routed(q, x, o.IQ3_S, True), routed(kvraw, x, o.Q4_K, False)], dim=1)
    assert torch.equal(y, ref)
    check_oracle(y, [(q, o.IQ3_S, True), (kvraw, o.Q4_K, False)], x)


@pytest.mark.parametrize("n", NS)
def test_same_type_gate_up_layer(n):
    """gate | up, both IQ3_S 17408 x 5120: one product over the 34816-row packed weight."""
    k = 5120
    g, u = w_rand(o.IQ3_S, 17408, k, 4), w_rand(o.IQ3_S, 17408, k, 5)
    layer, method = build_layer([(g, o.IQ3_S), (u, o.IQ3_S)], k)
    assert layer.weight.iq3_packed
    x = x_bf16(n, k, seed=20 + n).cuda()
    poison_allocator()
    y = method.apply(layer, x)
    both = np.concatenate([g, u])
    assert torch.equal(y, routed(both, x, o.IQ3_S, True))
    check_oracle(y, [(g, o.IQ3_S, True), (u, o.IQ3_S, True)], x)


@pytest.mark.parametrize("n", [1, 4, 9, 32])
def test_unpackable_layer_stays_gguf(n):
    """An IQ3_S run of 200 rows (not a multiple of 16) with a Q4_K run: the layer is not packed
    (all or nothing), the bytes stay GGUF blocks, apply() routes the unpacked IQ3_S ops."""
    k = 2048
    a, b = w_rand(o.IQ3_S, 200, k, 6), w_rand(o.Q4_K, 2304, k, 7)
    layer, method = build_layer([(a, o.IQ3_S), (b, o.Q4_K)], k)
    assert not getattr(layer.weight, "iq3_packed", False)
    from vllm_gguf_plugin.quantization.linear import _shard_weight

    assert torch.equal(_shard_weight(layer.weight, *layer.weight.shard_offset_map[0]), dev(a))
    x = x_bf16(n, k, seed=30 + n).cuda()
    poison_allocator()
    y = method.apply(layer, x)
    assert torch.equal(y, torch.cat([routed(a, x, o.IQ3_S, False), routed(b, x, o.Q4_K, False)], dim=1))
    check_oracle(y, [(a, o.IQ3_S, False), (b, o.Q4_K, False)], x)


def test_single_tensor_layer_packed():
    """One IQ3_S tensor, no shards: packed in place by the hook, apply() on the packed ops."""
    k = 5120
    a = w_rand(o.IQ3_S, 5120, k, 8)
    layer, method = build_layer([(a, o.IQ3_S)], k)
    assert layer.weight.iq3_packed and not layer.weight.shard_id
    for n in (1, 8, 33):
        x = x_bf16(n, k, seed=40 + n).cuda()
        y = method.apply(layer, x)
        assert torch.equal(y, routed(a, x, o.IQ3_S, True))
        check_oracle(y, [(a, o.IQ3_S, True)], x)


@pytest.mark.parametrize("n", [1, 4, 8, 9, 16, 32, 33, 128, 2048])
def test_routing_on_whole_packed_tensor(n):
    """_fused_mul_mat_gguf(packed=True) on a packed 17408 x 5120 tensor: the packed decode op
    up to 8 rows, the tiled op above, bit-exact with the op called directly."""
    from vllm_gguf_plugin.quantization import iq3_pack, linear

    k, rows = 5120, 17408
    raw = w_rand(o.IQ3_S, rows, k, 9)
    p = iq3_pack.pack(dev(raw), o.IQ3_S)
    x = x_bf16(n, k, seed=50 + n).cuda()
    poison_allocator()
    y = linear._fused_mul_mat_gguf(x, p, o.IQ3_S, None, True)
    op = "lcpp_mul_mat_vec_iq3_mma_packed" if n <= linear.PACKED_VEC_MAX_ROWS else "lcpp_mul_mat_iq3_packed"
    assert torch.equal(y, getattr(C(), op)(p, x, o.IQ3_S, rows))
    check_oracle(y, [(raw, o.IQ3_S, True)], x)


@pytest.fixture(scope="module")
def head():
    """The benchmark's Q6_K output head, 151936 x 5120 (638 MB): (raw, device copy)."""
    raw = w_rand(o.Q6_K, 151936, 5120, 11)
    return raw, dev(raw)


@pytest.mark.parametrize("n", [1, 5, 300, 512, 1000])
def test_vocab_head_prompt_rows(head, n):
    """The Q6_K output head 151936 x 5120 at prompt-logprob row counts: from n * rows * 4 >
    256 MiB (442 rows) the product runs in activation-row chunks of 384 (_FP32_DST_BUDGET), each
    routed for its own row count into one bf16 output; bit-exact with the chunks' own ops, the
    oracle on sampled rows, and peak memory within the output, one chunk's output and 64 MiB
    (workspace and allocator rounding)."""
    from vllm_gguf_plugin.quantization import linear

    k, rows = 5120, 151936
    raw, w = head
    x = x_bf16(n, k, seed=60 + n).cuda()
    torch.cuda.synchronize()
    poison_allocator()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    y = linear._fused_mul_mat_gguf(x, w, o.Q6_K)
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated() - base
    assert y.shape == (n, rows) and y.dtype == torch.bfloat16
    assert torch.isfinite(y).all()
    step = n if n * rows * 4 <= linear._FP32_DST_BUDGET else 384
    chunks = [(i, min(n, i + step)) for i in range(0, n, step)]
    assert len(chunks) == (1 if n <= 441 else -(-n // 384))
    for a, b in chunks:
        op = linear._lcpp_op(b - a, o.Q6_K, rows, k)
        assert torch.equal(y[a:b], getattr(C(), op)(w, x[a:b], o.Q6_K, rows)), (a, b, op)
    check_oracle(y, [(raw, o.Q6_K, False)], x, nsample=32)
    chunk_out = step * rows * 2 if len(chunks) > 1 else 0
    assert extra <= n * rows * 2 + chunk_out + (64 << 20), extra


def test_headcheck_log(tmp_path, monkeypatch):
    """VLLM_GGUF_HEADCHECK (reference linear.py:67-70,143-163): a product on a > 50,000-row weight
    at more than 8 activation rows appends one JSON record comparing the routed op with the decode
    op in 8-row calls; smaller products and 8-row products write nothing."""
    import json

    from vllm_gguf_plugin.quantization import linear

    log = tmp_path / "head.jsonl"
    monkeypatch.setattr(linear, "_HEADCHECK", str(log))
    k, rows = 512, 50048
    w = dev(w_rand(o.Q4_K, rows, k, 12))
    for n in (8, 24):
        linear._fused_mul_mat_gguf(x_bf16(n, k, seed=70 + n).cuda(), w, o.Q4_K)
    linear._fused_mul_mat_gguf(x_bf16(24, k, seed=71).cuda(), w[:1000], o.Q4_K)
    recs = [json.loads(line) for line in log.read_text().splitlines()]
    assert len(recs) == 1
    r = recs[0]
    assert (r["n"], r["rows"], r["route"]) == (24, rows, linear._lcpp_op(24, o.Q4_K, rows, k))
    assert r["max_rel"] < 0.05 and not r["bad_rows"] and r["x_finite"] and r["y_finite"]
