"""numpy statement of this build's IQ3_S tile layout (csrc/iq3_tile.h), for checking the GPU
repack. The layout is the build's own (not a reference format): 16-row tiles, each 256-value
block of a tile stored as one 1760-byte tile-block:
  [   0, 1024) lane L = 8p + s: qs[8s:8s+8] of row 2p, then of row 2p+1
  [1024, 1536) lane L: signs[4s:4s+4] of row 2p, then of row 2p+1
  [1536, 1664) lane L: qh[s] of row 2p, then of row 2p+1
  [1664, 1728) (p, j): scales[j] of row 2p, then of row 2p+1
  [1728, 1760) p: d (2 bytes) of row 2p, then of row 2p+1
"""

import numpy as np


def tile_source_map() -> tuple[np.ndarray, np.ndarray]:
    """(row, byte in the row's block) for each of the 1760 tile-block bytes."""
    r = np.zeros(1760, dtype=np.int64)
    o = np.zeros(1760, dtype=np.int64)
    j = 0
    for L in range(64):                      # qs
        p, s = L // 8, L % 8
        for i in range(16):
            r[j], o[j] = 2 * p + i // 8, 2 + 8 * s + i % 8
            j += 1
    for L in range(64):                      # signs
        p, s = L // 8, L % 8
        for i in range(8):
            r[j], o[j] = 2 * p + i // 4, 74 + 4 * s + i % 4
            j += 1
    for L in range(64):                      # qh
        p, s = L // 8, L % 8
        for i in range(2):
            r[j], o[j] = 2 * p + i, 66 + s
            j += 1
    for p in range(8):                       # scales
        for jj in range(4):
            for i in range(2):
                r[j], o[j] = 2 * p + i, 106 + jj
                j += 1
    for p in range(8):                       # d
        for i in range(2):
            for byte in range(2):
                r[j], o[j] = 2 * p + i, byte
                j += 1
    assert j == 1760
    return r, o


def pack(w: np.ndarray) -> np.ndarray:
    """[rows, row_bytes] GGUF IQ3_S rows (rows % 16 == 0) -> the tile layout."""
    rows, rb = w.shape
    nb = rb // 110
    r, o = tile_source_map()
    t = w.reshape(rows // 16, 16, nb, 110)                      # tile, row, block, byte
    out = t[:, r, :, o]                                         # [1760, tiles, nb] (advanced idx first)
    return np.ascontiguousarray(out.transpose(1, 2, 0)).reshape(rows, rb)


def unpack(p: np.ndarray) -> np.ndarray:
    rows, rb = p.shape
    nb = rb // 110
    r, o = tile_source_map()
    t = p.reshape(rows // 16, nb, 1760)
    out = np.zeros((rows // 16, 16, nb, 110), dtype=p.dtype)
    out[:, r, :, o] = t.transpose(2, 0, 1)
    return out.reshape(rows, rb)
