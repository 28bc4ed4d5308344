"""The build's IQ3_S unit layout (tests/_tile.py restates csrc/iq3_tile.h) on the CPU: a bijection
on every bit pattern (not only what a quantizer writes) and on the reference's golden rows, local
to each 4-row unit, for K of any number of blocks (a last unit-block of 1-3 blocks), and
decodable: the signed-grid words a kernel reads through it equal the oracle's decode of the GGUF
bytes. The GPU repack is checked against it in test_gpu_parity.py."""

import glob
import os

import numpy as np
import pytest
from conftest import GOLDEN

import _tile
import gguf_oracle as o


def _random(rows, blocks, seed=0):
    return np.random.default_rng(seed).integers(0, 256, size=(rows, blocks * 110), dtype=np.uint8)


@pytest.mark.parametrize("rows,blocks", [(4, 1), (16, 2), (8, 3), (32, 4), (16, 5), (272, 20), (48, 68), (12, 22)])
def test_roundtrip_random_bytes(rows, blocks):
    w = _random(rows, blocks, seed=rows + blocks)
    p = _tile.pack(w)
    assert p.shape == w.shape and not np.array_equal(p, w)
    np.testing.assert_array_equal(_tile.unpack(p), w)
    for u in range(rows // 4):  # unit u depends only on rows 4u..4u+3
        np.testing.assert_array_equal(p[4 * u:4 * u + 4], _tile.pack(w[4 * u:4 * u + 4]))


def test_roundtrip_golden_rows():
    files = sorted(glob.glob(os.path.join(GOLDEN, "dequant", "IQ3_S__*.npz")))
    rows = [np.load(f, allow_pickle=False)["raw"] for f in files]
    w = np.stack([rows[i % len(rows)] for i in range(32)])
    np.testing.assert_array_equal(_tile.unpack(_tile.pack(w)), w)


def test_unit_block_offsets():
    """Unit-blocks tile the unit's bytes: full ones at 1760 kb, a ragged last one of 440 r bytes."""
    for nb in range(1, 24):
        ub = _tile.unit_blocks(nb)
        assert sum(440 * r for _, r, _ in ub) == 4 * nb * 110
        for kb, r, off in ub:
            assert off == 1760 * kb and r == min(4, nb - 4 * kb)


def _signed_table():
    """Entry (qs | ex << 8): grid[qs | (ex >> 4) << 8] with the bytes flagged in ex & 0xF negated."""
    idx = np.arange(8192)
    g = o.IQ3S_GRID[(idx & 0xFF) | ((idx >> 12) << 8)].astype(np.int32)       # [8192, 4]
    sign = ((idx[:, None] >> (8 + np.arange(4))) & 1).astype(np.int32)
    return (g * (1 - 2 * sign)).astype(np.int8)


@pytest.mark.parametrize("blocks", [4, 6])
def test_kernel_view_decodes_to_oracle_values(blocks):
    """Reading a packed unit-block the way the decode GEMV does (lane L = 8p + s, p = 2 bi + rp;
    perm of qs and ex bytes into table indices) gives the oracle's signed int8 weights for every
    (row, block, slice, group), the ragged last unit-block included."""
    w = _random(4, blocks, seed=9)
    p = _tile.pack(w).reshape(-1)
    tbl = _signed_table()
    ref = o.decode_int(w.reshape(-1), o.IQ3_S)["w"].reshape(4, blocks, 8, 32)  # [row, block, slice, value]
    seen = np.zeros((4, blocks, 8), dtype=bool)
    for kb, r, base in _tile.unit_blocks(blocks):
        t = p[base:base + 440 * r].astype(np.uint32)
        for L in range(16 * r):
            bi, rp, s = L // 16, (L // 8) % 2, L % 8
            l2 = t[_tile.L2 * r + 2 * L] | t[_tile.L2 * r + 2 * L + 1] << 8
            for rr in range(2):
                e8 = [t[_tile.E8 * r + 8 * L + 4 * rr + j] for j in range(4)]
                lo = [e & 0x1F for e in e8]
                hi = [(e8[j] >> 5) | (((l2 >> (8 * rr + 2 * j)) & 3) << 3) for j in range(4)]
                ex = lo + hi
                qs = t[_tile.QS * r + 16 * L + 8 * rr:_tile.QS * r + 16 * L + 8 * rr + 8]
                got = np.concatenate([tbl[int(qs[e]) | (int(ex[e]) << 8)] for e in range(8)])
                np.testing.assert_array_equal(got, ref[2 * rp + rr, 4 * kb + bi, s])
                seen[2 * rp + rr, 4 * kb + bi, s] = True
    assert seen.all()
