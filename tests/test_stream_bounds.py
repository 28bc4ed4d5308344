"""A host model of the IQ3_S and IQ3_XXS stream GEMV's weight loads (csrc/gemv_iq3.hip,
gemv_iq3s_stream_kernel), checked on the CPU.

The kernel reads W through one buffer descriptor per workgroup, with the unit-block's field bases
as scalar offsets and the lane's part as the lane offset. The hardware range check sees only the
lane offset, so a load is safe only if the whole access stays inside the workgroup's bytes. This
test enumerates, for a set of shapes and compute-unit counts, every load the kernel issues: the
workgroup's run of units, each wave's run of (unit, unit-block) items, the two loads each wave
issues past its run (which must use the empty descriptor), and per lane the five fields (QS 16 B,
E8 8 B, L2 2 B, SC 2 B, D 4 B). It checks that every in-run access lies inside the unit-block it
belongs to, on full unit-blocks and on a ragged last one of two blocks (K % 1024 == 512), where the
lanes of the absent blocks take the offsets of lane L - 32; and that the items of all waves cover
each (unit, unit-block) of the weight exactly once. The IQ3_XXS unit layout takes the same lane
offsets for its three fields (QS 16 B at 16L, AUX 8 B at 8L, D 4 B at 4p) in unit-blocks of
392 r bytes.
"""

import numpy as np
import pytest

UNIT_ROWS, WAVES = 4, 8
FIELD_SIZE = {"qs": 16, "e8": 8, "l2": 2, "sc": 2, "d": 4}


def unit_blocks(nb, kb):
    """Blocks in unit-block kb (iq3_tile.h: iq3_unit_blocks)."""
    return 4 if kb < nb >> 2 else nb & 3


def unitblock_bases(r):
    """Field bases of a unit-block of r blocks, from its first byte (iq3_unitblock_fields)."""
    return {"qs": 0, "e8": 256 * r, "l2": 384 * r, "sc": 416 * r, "d": 432 * r}


def lane_offsets(lane):
    """unit_lane_offsets(lane, p, s) of the kernel, vectorised over lanes."""
    p, s = lane >> 3, lane & 7
    return {"qs": 16 * lane, "e8": 8 * lane, "l2": 2 * lane, "sc": 2 * (4 * p + (s >> 1)), "d": 4 * p}


LANES = np.arange(64)
OFF = lane_offsets(LANES)
OFF_RAGGED = lane_offsets(LANES & 31)  # lane L - 32 for the lanes of absent blocks


def check_unitblock(nb, kb):
    r = unit_blocks(nb, kb)
    assert r in (2, 4)
    bases = unitblock_bases(r)
    ragged = (nb & 3) != 0 and kb == (nb + 3) // 4 - 1
    offs = OFF_RAGGED if ragged else OFF
    for f, size in FIELD_SIZE.items():
        lo = bases[f] + offs[f]
        assert lo.min() >= 0 and (lo + size).max() <= 440 * r, (nb, kb, f)
    if not ragged:  # full unit-blocks: the 64 lanes' QS and E8 parts tile their fields exactly
        assert sorted((bases["qs"] + OFF["qs"]).tolist()) == list(range(0, 256 * r, 16))
        assert sorted((bases["e8"] + OFF["e8"]).tolist()) == list(range(256 * r, 384 * r, 8))


def enumerate_loads(nrows, k, cus):
    """(per-unit-block hit counts, number of past-the-run loads) of one launch."""
    nb = k // 256
    nkb = (nb + 3) // 4
    nunits = nrows // UNIT_ROWS
    grid = min(nunits, cus)
    hits = np.zeros((nunits, nkb), dtype=np.int64)
    past = 0
    for g in range(grid):
        u0, u1 = g * nunits // grid, (g + 1) * nunits // grid
        items = (u1 - u0) * nkb
        for w in range(WAVES):
            j0, j1 = w * items // WAVES, (w + 1) * items // WAVES
            # load_next is called twice before the loop and once per computed item
            for lj in range(j0, j0 + (j1 - j0) + 2):
                if lj < j1:
                    hits[u0 + lj // nkb, lj % nkb] += 1
                else:
                    past += 1
    return hits, past, grid


@pytest.mark.parametrize("blocks", [2, 4, 6, 10, 18, 20, 22, 24, 68, 70])
def test_every_field_access_stays_in_its_unit_block(blocks):
    for kb in range((blocks + 3) // 4):
        check_unitblock(blocks, kb)


@pytest.mark.parametrize("nrows,k,cus", [(17408, 5120, 256), (5120, 17408, 256), (1024, 4608, 256),
                                         (4096, 2560, 256), (17408, 5120, 304), (5200, 1536, 80),
                                         (2064, 17920, 256)])
def test_items_cover_each_unit_block_once(nrows, k, cus):
    hits, past, grid = enumerate_loads(nrows, k, cus)
    assert (hits == 1).all()
    assert past == 2 * WAVES * grid  # each wave's two trailing loads use the empty range


XXS_FIELD_SIZE = {"qs": 16, "e8": 8, "d": 4}  # the kernel loads AUX with the E8 lane offset


def xxs_unitblock_bases(r):
    """Field bases of an IQ3_XXS unit-block of r blocks (xxs_unitblock_fields)."""
    return {"qs": 0, "e8": 256 * r, "d": 384 * r}


@pytest.mark.parametrize("blocks", [2, 4, 6, 10, 18, 20, 22, 24, 68, 70])
def test_xxs_every_field_access_stays_in_its_unit_block(blocks):
    for kb in range((blocks + 3) // 4):
        r = unit_blocks(blocks, kb)
        bases = xxs_unitblock_bases(r)
        ragged = (blocks & 3) != 0 and kb == (blocks + 3) // 4 - 1
        offs = OFF_RAGGED if ragged else OFF
        for f, size in XXS_FIELD_SIZE.items():
            lo = bases[f] + offs[f]
            assert lo.min() >= 0 and (lo + size).max() <= 392 * r, (blocks, kb, f)
        if not ragged:  # the 64 lanes' QS and AUX parts tile their fields exactly
            assert sorted((bases["qs"] + OFF["qs"]).tolist()) == list(range(0, 256 * r, 16))
            assert sorted((bases["e8"] + OFF["e8"]).tolist()) == list(range(256 * r, 384 * r, 8))
            assert sorted(set((bases["d"] + OFF["d"]).tolist())) == list(range(384 * r, 392 * r, 4))
