"""Helpers shared by the GPU test modules: seeded inputs, the exact-integer mode, and the op
namespace with allocator poisoning.

Every op called through C() first fills the free blocks of torch's caching allocator with 0xFF
(NaN as fp32 / fp16 / bf16, -1 as int8), unless a CUDA graph is being captured: an output element
or workspace byte that a kernel reads before writing, or never writes, then holds garbage rather
than a stale copy of an earlier, identical result.
"""

import numpy as np
import torch

import gguf_oracle as o

TIGHT = {torch.float32: 1e-3, torch.bfloat16: 5e-3, torch.float16: 2.5e-3}

# sizes of the poisoned blocks: two of each power of two from 512 B to 256 MiB
_POISON_SIZES = [1 << p for p in range(9, 29) for _ in range(2)]


def poison_allocator() -> None:
    """Fill the caching allocator's free memory with 0xFF: allocate blocks of every size class,
    fill them, free them (they stay cached and are handed out to the next allocations)."""
    if torch.cuda.is_current_stream_capturing():
        return
    blocks = [torch.empty(n, dtype=torch.uint8, device="cuda") for n in _POISON_SIZES]
    for b in blocks:
        b.fill_(0xFF)
    del blocks


class _PoisonedOps:
    """torch.ops._C_gguf with poison_allocator() before every call."""

    def __getattr__(self, name):
        op = getattr(torch.ops._C_gguf, name)

        def call(*args, **kwargs):
            poison_allocator()
            return op(*args, **kwargs)

        call.__name__ = name
        return call


_OPS = _PoisonedOps()


def C():
    return _OPS


def x_rand(n, k, seed, dtype=torch.float32):
    """N(0,1) activations with about 1/256 of the columns scaled by 20 (outliers)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, k, generator=g)
    x[:, torch.randperm(k, generator=g)[: max(1, k // 256)]] *= 20
    return x.to(dtype)


def w_rand(qt, rows, k, seed):
    return o.random_blocks(np.random.default_rng(seed), qt, rows, k)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def exact_weights(qt, rows, k, seed):
    """Random codes with every block scale (d, and dmin where the type has one) 1.0 (Q6_K
    sub-scales kept within +-31)."""
    w = w_rand(qt, rows, k, seed)
    b = w.reshape(-1, o.BLOCK_BYTES[qt])
    one = np.array([0x00, 0x3C], dtype=np.uint8)  # fp16 1.0
    if qt == o.Q6_K:
        sc = np.random.default_rng(seed + 1).integers(-31, 32, size=(b.shape[0], 16)).astype(np.int8)
        b[:, 192:208] = sc.view(np.uint8)
    for off in o.SCALE_OFFSETS[qt]:
        b[:, off:off + 2] = one
    if qt == o.IQ1_M:
        o.set_iq1m_d(b, np.ones(b.shape[0], dtype=np.float16))
    return w


def exact_x(n, k, seed, dtype=torch.bfloat16):
    """Integers in [-2, 2] with one +-127 per 32-slice: every q8_1 scale is exactly 1."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-2, 3, size=(n, k)).astype(np.float32)
    pos = rng.integers(0, 32, size=(n, k // 32)) + 32 * np.arange(k // 32)
    x[np.arange(n)[:, None], pos] = 127 * rng.choice([-1.0, 1.0], size=(n, k // 32))
    return torch.from_numpy(x).to(dtype)


def exact_ref(raw, qt, x, form="mmvq"):
    """The exact output with every scale 1: the int64 sum of the oracle's slice dots, or for the
    single-scale IQ types the sum of their slice values (a multiple of 1/8): the decode ops'
    truncating MMVQ values (form 'mmvq') or the product ops' dot / den (form 'mmq')."""
    q, d, _ = o.dequant_q8_1(o.quantize_q8_1(x), x.shape[0], x.shape[1])
    assert (d == 1).all()
    if qt in o.UNIT_TYPES:
        if form == "mmvq":  # integers, IQ1_M multiples of 1/8
            y, den = o.mmvq_slice_units(raw, qt, q).sum(-1), 8 if qt == o.IQ1_M else 1
        else:               # multiples of 1/den
            dots = o.slice_dots(raw, qt, q)
            y, den = dots["dot"].sum(-1) / dots["den"], dots["den"]
        assert np.abs(y).max() * den < 2 ** 23  # every partial sum stays exact in fp32
        return y
    dots = o.slice_dots(raw, qt, q)
    y = dots["dot"].sum(-1)
    if qt in (o.Q4_K, o.Q2_K):
        y = y - dots["m"].sum(-1)
    assert np.abs(y).max() < 2 ** 24
    return y


def graph_replays_equal(fn, eager, reps=3):
    """Capture fn() in a CUDA graph and check that every replay equals `eager` bit for bit."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    for _ in range(reps):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
