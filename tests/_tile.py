"""numpy statement of this build's IQ3_S tile layout (csrc/iq3_tile.h), for checking the GPU
repack. The layout is the build's own (not a reference format). Rows are grouped in tiles of 16;
each 256-value block of a tile is one 1760-byte tile-block. Lane L = 8p + s owns rows 2p, 2p+1
(r = 0, 1) of slice s; for group e (0..7) of row r,
  ex(r, e) = sign nibble e of the slice's sign bytes | (bit e of qh[s]) << 4.
  [   0, 1024) QS 16 B at 16L: qs[8s:8s+8] of row 2p, then of row 2p+1
  [1024, 1536) E8  8 B at 8L : byte 4r+j = ex(r, j) | (ex(r, 4+j) & 7) << 5
  [1536, 1664) L2  2 B at 2L : bits 8r+2j.. = ex(r, 4+j) >> 3
  [1664, 1728) SC  2 B at 2(4p+j): scales[j] of row 2p, then of row 2p+1
  [1728, 1760) D   4 B at 4p : d of row 2p, then of row 2p+1
"""

import numpy as np

QS, E8, L2, SC, D = 0, 1024, 1536, 1664, 1728


def _tileblocks(w):
    rows, rb = w.shape
    nb = rb // 110
    return w.reshape(rows // 16, 16, nb, 110), nb


def pack(w: np.ndarray) -> np.ndarray:
    """[rows, row_bytes] GGUF IQ3_S rows (rows % 16 == 0) -> the tile layout."""
    rows, rb = w.shape
    t, nb = _tileblocks(w.astype(np.uint32))
    nt = rows // 16
    out = np.zeros((nt, nb, 1760), dtype=np.uint8)
    for L in range(64):
        p, s = L // 8, L % 8
        l2 = np.zeros((nt, nb), dtype=np.uint32)
        for r in range(2):
            blk = t[:, 2 * p + r]                                   # [nt, nb, 110]
            out[:, :, QS + 16 * L + 8 * r:QS + 16 * L + 8 * r + 8] = blk[..., 2 + 8 * s:10 + 8 * s]
            sg = (blk[..., 74 + 4 * s] | blk[..., 75 + 4 * s] << 8 | blk[..., 76 + 4 * s] << 16
                  | blk[..., 77 + 4 * s] << 24)
            qh = blk[..., 66 + s]
            ex = [((sg >> (4 * e)) & 0xF) | (((qh >> e) & 1) << 4) for e in range(8)]
            for j in range(4):
                out[:, :, E8 + 8 * L + 4 * r + j] = ex[j] | ((ex[4 + j] & 7) << 5)
                l2 |= (ex[4 + j] >> 3) << (8 * r + 2 * j)
        out[:, :, L2 + 2 * L] = l2 & 0xFF
        out[:, :, L2 + 2 * L + 1] = l2 >> 8
    for p in range(8):
        for j in range(4):
            for r in range(2):
                out[:, :, SC + 2 * (4 * p + j) + r] = t[:, 2 * p + r, :, 106 + j]
        for r in range(2):
            out[:, :, D + 4 * p + 2 * r:D + 4 * p + 2 * r + 2] = t[:, 2 * p + r, :, 0:2]
    return out.reshape(rows, rb)


def unpack(pk: np.ndarray) -> np.ndarray:
    rows, rb = pk.shape
    nb = rb // 110
    nt = rows // 16
    tb = pk.reshape(nt, nb, 1760).astype(np.uint32)
    out = np.zeros((nt, 16, nb, 110), dtype=np.uint32)
    for L in range(64):
        p, s = L // 8, L % 8
        l2 = tb[..., L2 + 2 * L] | tb[..., L2 + 2 * L + 1] << 8
        for r in range(2):
            row = out[:, 2 * p + r]
            row[..., 2 + 8 * s:10 + 8 * s] = tb[..., QS + 16 * L + 8 * r:QS + 16 * L + 8 * r + 8]
            sg = np.zeros((nt, nb), dtype=np.uint32)
            qh = np.zeros((nt, nb), dtype=np.uint32)
            for e in range(8):
                j = e % 4
                byte = tb[..., E8 + 8 * L + 4 * r + j]
                ex = (byte & 0x1F) if e < 4 else ((byte >> 5) | (((l2 >> (8 * r + 2 * j)) & 3) << 3))
                sg |= (ex & 0xF) << (4 * e)
                qh |= ((ex >> 4) & 1) << e
            for i in range(4):
                row[..., 74 + 4 * s + i] = (sg >> (8 * i)) & 0xFF
            row[..., 66 + s] = qh
    for p in range(8):
        for j in range(4):
            for r in range(2):
                out[:, 2 * p + r, :, 106 + j] = tb[..., SC + 2 * (4 * p + j) + r]
        for r in range(2):
            out[:, 2 * p + r, :, 0:2] = tb[..., D + 4 * p + 2 * r:D + 4 * p + 2 * r + 2]
    return out.astype(np.uint8).reshape(rows, rb)
