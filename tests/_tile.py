"""numpy statement of this build's IQ3_S unit layout (csrc/iq3_tile.h), for checking the GPU
repack. The layout is the build's own (not a reference format). Rows are grouped in units of 4;
the K blocks of a unit are taken four at a time, blocks 4kb..4kb+3 forming the 1760-byte
unit-block kb at byte 1760 kb of the unit (a last unit-block of r = nb % 4 blocks takes 440 r
bytes, its fields scaled by r/4). Lane L = 8p + s, p = 2 bi + rp, owns rows 2rp, 2rp+1 (r = 0, 1)
of the unit in slice s of block 4kb + bi; for group e (0..7) of row r,
  ex(r, e) = sign nibble e of the slice's sign bytes | (bit e of qh[s]) << 4.
  [    0, 256 r) QS 16 B at 16L: qs[8s:8s+8] of row 2rp, then of row 2rp+1
  [256 r, 384 r) E8  8 B at 8L : byte 4r+j = ex(r, j) | (ex(r, 4+j) & 7) << 5
  [384 r, 416 r) L2  2 B at 2L : bits 8r+2j.. = ex(r, 4+j) >> 3
  [416 r, 432 r) SC  2 B at 2(4p+j): scales[j] of row 2rp, then of row 2rp+1
  [432 r, 440 r) D   4 B at 4p : d of row 2rp, then of row 2rp+1
"""

import numpy as np

QS, E8, L2, SC, D = 0, 256, 384, 416, 432   # field bases per block of the unit-block (times r)


def unit_blocks(nb):
    """(kb, r, byte offset in the unit) of each unit-block of a unit of nb blocks."""
    out, off = [], 0
    for kb in range((nb + 3) // 4):
        r = min(4, nb - 4 * kb)
        out.append((kb, r, off))
        off += 440 * r
    return out


def _lane_ex(blk, s):
    """ex(r, e) of slice s for a [..., 110] array of GGUF blocks (uint32)."""
    sg = blk[..., 74 + 4 * s] | blk[..., 75 + 4 * s] << 8 | blk[..., 76 + 4 * s] << 16 | blk[..., 77 + 4 * s] << 24
    qh = blk[..., 66 + s]
    return [((sg >> (4 * e)) & 0xF) | (((qh >> e) & 1) << 4) for e in range(8)]


def pack(w: np.ndarray) -> np.ndarray:
    """[rows, row_bytes] GGUF IQ3_S rows (rows % 4 == 0) -> the unit layout."""
    rows, rb = w.shape
    nb = rb // 110
    nu = rows // 4
    g = w.astype(np.uint32).reshape(nu, 4, nb, 110)
    out = np.zeros((nu, 4 * rb), dtype=np.uint8)
    for kb, r, base in unit_blocks(nb):
        for L in range(16 * r):
            bi, rp, s = L // 16, (L // 8) % 2, L % 8
            b = 4 * kb + bi
            l2 = np.zeros(nu, dtype=np.uint32)
            for rr in range(2):
                blk = g[:, 2 * rp + rr, b]                          # [nu, 110]
                o = base + QS * r + 16 * L + 8 * rr
                out[:, o:o + 8] = blk[:, 2 + 8 * s:10 + 8 * s]
                ex = _lane_ex(blk, s)
                for j in range(4):
                    out[:, base + E8 * r + 8 * L + 4 * rr + j] = ex[j] | ((ex[4 + j] & 7) << 5)
                    l2 |= (ex[4 + j] >> 3) << (8 * rr + 2 * j)
            out[:, base + L2 * r + 2 * L] = l2 & 0xFF
            out[:, base + L2 * r + 2 * L + 1] = l2 >> 8
        for p in range(2 * r):
            bi, rp = p // 2, p % 2
            b = 4 * kb + bi
            for rr in range(2):
                for j in range(4):
                    out[:, base + SC * r + 2 * (4 * p + j) + rr] = g[:, 2 * rp + rr, b, 106 + j]
                o = base + D * r + 4 * p + 2 * rr
                out[:, o:o + 2] = g[:, 2 * rp + rr, b, 0:2]
    return out.reshape(rows, rb)  # a unit's bytes occupy its 4 rows in order


def unpack(pk: np.ndarray) -> np.ndarray:
    rows, rb = pk.shape
    nb = rb // 110
    nu = rows // 4
    t = pk.reshape(nu, 4 * rb).astype(np.uint32)
    out = np.zeros((nu, 4, nb, 110), dtype=np.uint32)
    for kb, r, base in unit_blocks(nb):
        for L in range(16 * r):
            bi, rp, s = L // 16, (L // 8) % 2, L % 8
            b = 4 * kb + bi
            l2 = t[:, base + L2 * r + 2 * L] | t[:, base + L2 * r + 2 * L + 1] << 8
            for rr in range(2):
                row = out[:, 2 * rp + rr, b]
                o = base + QS * r + 16 * L + 8 * rr
                row[:, 2 + 8 * s:10 + 8 * s] = t[:, o:o + 8]
                sg = np.zeros(nu, dtype=np.uint32)
                qh = np.zeros(nu, dtype=np.uint32)
                for e in range(8):
                    j = e % 4
                    byte = t[:, base + E8 * r + 8 * L + 4 * rr + j]
                    ex = (byte & 0x1F) if e < 4 else ((byte >> 5) | (((l2 >> (8 * rr + 2 * j)) & 3) << 3))
                    sg |= (ex & 0xF) << (4 * e)
                    qh |= ((ex >> 4) & 1) << e
                for i in range(4):
                    row[:, 74 + 4 * s + i] = (sg >> (8 * i)) & 0xFF
                row[:, 66 + s] = qh
        for p in range(2 * r):
            bi, rp = p // 2, p % 2
            b = 4 * kb + bi
            for rr in range(2):
                for j in range(4):
                    out[:, 2 * rp + rr, b, 106 + j] = t[:, base + SC * r + 2 * (4 * p + j) + rr]
                o = base + D * r + 4 * p + 2 * rr
                out[:, 2 * rp + rr, b, 0:2] = t[:, o:o + 2]
    return out.astype(np.uint8).reshape(rows, rb)


# ---------------------------------------------------------------------------------------------
# The IQ3_XXS unit layout (csrc/iq3_tile.h): the same units, unit-blocks and lanes, 1568-byte
# unit-blocks (392 r for a last one of r blocks). block_iq3_xxs: d[0:2], qs[2:66] (one grid index
# per 4 values), per slice s a dword at 66 + 4s (four 7-bit sign indices, the scale in bits 28..31).
#   [    0, 256 r) QS  16 B at 16L: qs[8s:8s+8] of row 2rp, then of row 2rp+1
#   [256 r, 384 r) AUX  8 B at 8L : the slice's dword of row 2rp, then of row 2rp+1
#   [384 r, 392 r) D    4 B at 4p : d of row 2rp, then of row 2rp+1

XQS, XAUX, XD = 0, 256, 384   # field bases per block of the unit-block (times r)


def xxs_unit_blocks(nb):
    """(kb, r, byte offset in the unit) of each IQ3_XXS unit-block of a unit of nb blocks."""
    out, off = [], 0
    for kb in range((nb + 3) // 4):
        r = min(4, nb - 4 * kb)
        out.append((kb, r, off))
        off += 392 * r
    return out


def _xxs_sources(nb):
    """For every byte of a unit in the layout, (row in the unit, byte of that GGUF row)."""
    src = []
    for kb, r, base in xxs_unit_blocks(nb):
        ub = [None] * (392 * r)
        for L in range(16 * r):
            bi, rp, s = L // 16, (L // 8) % 2, L % 8
            b = 4 * kb + bi
            for rr in range(2):
                for i in range(8):
                    ub[XQS * r + 16 * L + 8 * rr + i] = (2 * rp + rr, 98 * b + 2 + 8 * s + i)
                for i in range(4):
                    ub[XAUX * r + 8 * L + 4 * rr + i] = (2 * rp + rr, 98 * b + 66 + 4 * s + i)
        for p in range(2 * r):
            bi, rp = p // 2, p % 2
            for rr in range(2):
                for i in range(2):
                    ub[XD * r + 4 * p + 2 * rr + i] = (2 * rp + rr, 98 * (4 * kb + bi) + i)
        src += ub
    return src


def pack_xxs(w: np.ndarray) -> np.ndarray:
    """[rows, row_bytes] GGUF IQ3_XXS rows (rows % 4 == 0) -> the unit layout."""
    rows, rb = w.shape
    nb, nu = rb // 98, rows // 4
    src = _xxs_sources(nb)
    ridx = np.array([r for r, _ in src]) * rb + np.array([c for _, c in src])
    return w.reshape(nu, 4 * rb)[:, ridx].reshape(rows, rb)


def unpack_xxs(pk: np.ndarray) -> np.ndarray:
    rows, rb = pk.shape
    nb, nu = rb // 98, rows // 4
    src = _xxs_sources(nb)
    ridx = np.array([r for r, _ in src]) * rb + np.array([c for _, c in src])
    out = np.zeros((nu, 4 * rb), dtype=pk.dtype)
    out[:, ridx] = pk.reshape(nu, 4 * rb)
    return out.reshape(rows, rb)
