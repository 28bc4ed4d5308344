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


# ------------------------------------------------------------------------------------- IQ3_XXS
def _random_xxs(rows, blocks, seed=0):
    return np.random.default_rng(seed).integers(0, 256, size=(rows, blocks * 98), dtype=np.uint8)


@pytest.mark.parametrize("rows,blocks", [(4, 1), (16, 2), (8, 3), (32, 4), (16, 5), (272, 20), (48, 68), (12, 22)])
def test_xxs_roundtrip_random_bytes(rows, blocks):
    w = _random_xxs(rows, blocks, seed=rows + blocks)
    p = _tile.pack_xxs(w)
    assert p.shape == w.shape and not np.array_equal(p, w)
    np.testing.assert_array_equal(_tile.unpack_xxs(p), w)
    for u in range(rows // 4):  # unit u depends only on rows 4u..4u+3
        np.testing.assert_array_equal(p[4 * u:4 * u + 4], _tile.pack_xxs(w[4 * u:4 * u + 4]))


def test_xxs_roundtrip_golden_rows():
    files = sorted(glob.glob(os.path.join(GOLDEN, "dequant", "IQ3_XXS__*.npz")))
    assert files
    rows = [np.load(f, allow_pickle=False)["raw"] for f in files]
    w = np.stack([rows[i % len(rows)] for i in range(32)])
    np.testing.assert_array_equal(_tile.unpack_xxs(_tile.pack_xxs(w)), w)


def test_xxs_unit_block_offsets():
    for nb in range(1, 24):
        ub = _tile.xxs_unit_blocks(nb)
        assert sum(392 * r for _, r, _ in ub) == 4 * nb * 98
        for kb, r, off in ub:
            assert off == 1568 * kb and r == min(4, nb - 4 * kb)


def _xxs_signed_table():
    """Entry (q | n << 8): grid[q] with the bytes flagged in the nibble n negated."""
    idx = np.arange(4096)
    g = o.IQ3XXS_GRID[idx & 0xFF].astype(np.int32)                       # [4096, 4]
    sign = ((idx[:, None] >> (8 + np.arange(4))) & 1).astype(np.int32)
    return (g * (1 - 2 * sign)).astype(np.int8)


@pytest.mark.parametrize("blocks", [4, 6])
def test_xxs_kernel_view_decodes_to_oracle_values(blocks):
    """Reading a packed IQ3_XXS unit-block the way the stream GEMV does (lane L = 8p + s: QS 16 B
    at 16L, AUX 8 B at 8L, D 4 B at 4p; the second word's nibble from bits 4..6 of the 7-bit sign
    index and the index's parity, formed by the kernel's two three-way xors) gives the oracle's
    signed weights, scales and d for every (row, block, slice), the ragged last unit-block
    included."""
    w = _random_xxs(4, blocks, seed=11)
    p = _tile.pack_xxs(w).reshape(-1)
    tbl = _xxs_signed_table()
    dec = o.decode_int(w.reshape(-1), o.IQ3_XXS)
    ref = dec["w"].reshape(4, blocks, 8, 32)
    seen = np.zeros((4, blocks, 8), dtype=bool)
    for kb, r, base in _tile.xxs_unit_blocks(blocks):
        t = p[base:base + 392 * r]
        for L in range(16 * r):
            bi, rp, s = L // 16, (L // 8) % 2, L % 8
            p_ = L // 8
            for rr in range(2):
                qs = t[16 * L + 8 * rr:16 * L + 8 * rr + 8]
                a = int.from_bytes(t[256 * r + 8 * L + 4 * rr:256 * r + 8 * L + 4 * rr + 4].tobytes(), "little")
                x = a ^ (a >> 1) ^ (a >> 2)
                par = x ^ (x >> 3) ^ (a >> 6)
                hi = ((par << 3) & 0x01020408) | ((a >> 4) & ~0x01020408 & 0xFFFFFFFF)
                words = []
                for g in range(4):
                    words.append(tbl[int(qs[2 * g]) | (((a >> (7 * g)) & 0xF) << 8)])
                    words.append(tbl[int(qs[2 * g + 1]) | (((hi >> (7 * g)) & 0xF) << 8)])
                row, blk = 2 * rp + rr, 4 * kb + bi
                np.testing.assert_array_equal(np.concatenate(words), ref[row, blk, s])
                d = t[384 * r + 4 * p_ + 2 * rr:384 * r + 4 * p_ + 2 * rr + 2].view(np.float16)[0]
                np.testing.assert_array_equal(d, w[row, 98 * blk:98 * blk + 2].view(np.float16)[0])
                assert (a >> 28) == (int.from_bytes(w[row, 98 * blk + 66 + 4 * s:98 * blk + 70 + 4 * s].tobytes(),
                                                    "little") >> 28)
                seen[row, blk, s] = True
    assert seen.all()
