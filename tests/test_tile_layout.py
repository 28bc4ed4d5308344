"""The build's IQ3_S tile layout (tests/_tile.py restates csrc/iq3_tile.h) on the CPU: a bijection
on every bit pattern (not only what a quantizer writes) and on the reference's golden rows, local
to each 16-row tile, and decodable: the signed-grid words a kernel reads through it equal the
oracle's decode of the GGUF bytes. The GPU repack is checked against it in test_gpu_parity.py."""

import glob
import os

import numpy as np
import pytest
from conftest import GOLDEN

import _tile
import gguf_oracle as o


def _random(rows, blocks, seed=0):
    return np.random.default_rng(seed).integers(0, 256, size=(rows, blocks * 110), dtype=np.uint8)


@pytest.mark.parametrize("rows,blocks", [(16, 1), (32, 2), (272, 20), (48, 68)])
def test_roundtrip_random_bytes(rows, blocks):
    w = _random(rows, blocks, seed=rows + blocks)
    p = _tile.pack(w)
    assert p.shape == w.shape and not np.array_equal(p, w)
    np.testing.assert_array_equal(_tile.unpack(p), w)
    for t in range(rows // 16):  # tile t depends only on rows 16t..16t+15
        np.testing.assert_array_equal(p[16 * t:16 * t + 16], _tile.pack(w[16 * t:16 * t + 16]))


def test_roundtrip_golden_rows():
    files = sorted(glob.glob(os.path.join(GOLDEN, "dequant", "IQ3_S__*.npz")))
    rows = [np.load(f, allow_pickle=False)["raw"] for f in files]
    w = np.stack([rows[i % len(rows)] for i in range(32)])
    np.testing.assert_array_equal(_tile.unpack(_tile.pack(w)), w)


def _signed_table():
    """Entry (qs | ex << 8): grid[qs | (ex >> 4) << 8] with the bytes flagged in ex & 0xF negated."""
    idx = np.arange(8192)
    g = o.IQ3S_GRID[(idx & 0xFF) | ((idx >> 12) << 8)].astype(np.int32)       # [8192, 4]
    sign = ((idx[:, None] >> (8 + np.arange(4))) & 1).astype(np.int32)
    return (g * (1 - 2 * sign)).astype(np.int8)


def test_kernel_view_decodes_to_oracle_values():
    """Reading a packed tile-block the way the decode GEMV does (perm of qs and ex bytes into table
    indices) gives the oracle's signed int8 weights for every (row, slice, group)."""
    w = _random(16, 3, seed=9)
    p = _tile.pack(w).reshape(1, 3, 1760)[0]
    tbl = _signed_table()
    ref = o.decode_int(w.reshape(-1), o.IQ3_S)["w"].reshape(16, 3, 8, 32)     # [row, block, slice, value]
    for b in range(3):
        t = p[b].astype(np.uint32)
        for L in range(64):
            pp, s = L // 8, L % 8
            l2 = t[_tile.L2 + 2 * L] | t[_tile.L2 + 2 * L + 1] << 8
            for r in range(2):
                e8 = [t[_tile.E8 + 8 * L + 4 * r + j] for j in range(4)]
                lo = [e & 0x1F for e in e8]
                hi = [(e8[j] >> 5) | (((l2 >> (8 * r + 2 * j)) & 3) << 3) for j in range(4)]
                ex = lo + hi
                qs = t[_tile.QS + 16 * L + 8 * r:_tile.QS + 16 * L + 8 * r + 8]
                got = np.concatenate([tbl[int(qs[e]) | (int(ex[e]) << 8)] for e in range(8)])
                np.testing.assert_array_equal(got, ref[2 * pp + r, b, s])
