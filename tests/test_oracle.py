"""Pins the CPU oracle (oracle/gguf_oracle.py) before anything is checked against it.

dequant   bit-exact against the reference's golden rows (fp32 gguf-py b11211 output on real
          GGUF rows, tests/fixtures/dequant of the reference, copied to tests/golden/dequant).
tables    against the reference header itself (oracle/_ref/ref_tables, built by oracle/Makefile
          from ggml-common.h where it lies) when that is built, and against invariants always.
q8_1      closed-form properties plus independent scalar restatements on small inputs; planted
          mistakes (x*(1/d) rounding, sequential sum order, half-even rounding) must be told
          apart from the real arithmetic.
dots      brute-force int64 loops on tiny inputs; the dequant identity on real rows.
"""

import glob
import json
import os
import subprocess

import numpy as np
import pytest
from conftest import GOLDEN, ORACLE

import gguf_oracle as o

FILES = sorted(glob.glob(os.path.join(GOLDEN, "dequant", "*.npz")))
IDS = [os.path.basename(f)[:-4] for f in FILES]
TYPES = [o.IQ3_S, o.Q4_K, o.IQ4_XS, o.Q6_K, o.Q2_K, o.IQ2_XXS, o.IQ2_XS, o.IQ2_S, o.IQ3_XXS, o.IQ1_M]


def _load(path):
    z = np.load(path, allow_pickle=False)
    return z["raw"], z["ref"], int(z["ggml_type"])


def test_manifest_matches_files():
    m = json.load(open(os.path.join(GOLDEN, "dequant", "manifest.json")))
    assert {f["file"] for f in m["fixtures"]} == {os.path.basename(f) for f in FILES}
    assert set(m["types"]) == {o.TYPE_NAMES[t] for t in TYPES}
    assert len(FILES) == 84  # 9 rows per type, 3 for IQ1_M


@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_dequant_bit_exact_vs_golden(path):
    raw, ref, qt = _load(path)
    y = o.dequantize(raw, qt)
    np.testing.assert_array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_golden_rows_reach_every_iq3s_grid_entry():
    """Every one of the 512 grid entries is used by the golden rows, so the bit-exact dequant
    above pins the whole grid (a blocks' d is never 0 on these rows)."""
    seen = set()
    for f in FILES:
        raw, _, qt = _load(f)
        if qt != o.IQ3_S:
            continue
        b = raw.reshape(-1, 110).astype(np.int64)
        assert (b[:, 0] | b[:, 1]).all()
        g = np.arange(64)
        seen |= set((b[:, 2:66] | (((b[:, 66:74][:, g // 8] >> (g % 8)) & 1) << 8)).ravel().tolist())
    assert seen == set(range(512))


def test_tables_invariants():
    g = o.IQ3S_GRID
    assert g.shape == (512, 4)
    assert set(np.unique(g).tolist()) <= {1, 3, 5, 7, 9, 11, 13, 15}
    u = o.IQ3S_GRID_U32.astype(np.int64)
    assert (np.diff(u) > 0).all()                    # ascending, hence distinct
    assert u[0] == 0x01010101 and u[-1] == 0x0F0F0101
    kv = o.KVALUES_IQ4NL.astype(int)
    assert (np.diff(kv) > 0).all() and kv[0] == -127 and kv[-1] == 113


def _ref_tables():
    exe = os.path.join(ORACLE, "_ref", "ref_tables")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref not built (needs the reference tree; `make -C oracle`)")
    out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    tables = {}
    for l in out:
        p = l.split()
        if len(p) == 3 and p[0] != "sizeof":
            tables.setdefault(p[0], []).append(int(p[2]))
    sizes = [l for l in out if l.startswith("sizeof")][0].split()
    return tables, dict(zip(sizes[1::2], map(int, sizes[2::2])))


def test_tables_equal_reference_header():
    tables, sizes = _ref_tables()
    kv = tables["kvalues_iq4nl"]
    assert o.IQ3S_GRID_U32.astype(np.int64).tolist() == tables["iq3s_grid"]
    names = {o.IQ3_S: "block_iq3_s", o.Q4_K: "block_q4_K", o.Q6_K: "block_q6_K", o.IQ4_XS: "block_iq4_xs",
             o.Q2_K: "block_q2_K", o.IQ2_XXS: "block_iq2_xxs", o.IQ2_XS: "block_iq2_xs", o.IQ2_S: "block_iq2_s",
             o.IQ3_XXS: "block_iq3_xxs", o.IQ1_M: "block_iq1_m"}
    assert sizes["block_q8_1"] == 36
    assert {t: sizes[nm] for t, nm in names.items()} == o.BLOCK_BYTES
    for name, grid in (("iq2xxs_grid", o.IQ2XXS_GRID), ("iq2xs_grid", o.IQ2XS_GRID), ("iq2s_grid", o.IQ2S_GRID),
                       ("iq3xxs_grid", o.IQ3XXS_GRID), ("iq1s_grid", o.IQ1S_GRID)):
        assert o.grid_words(grid).tolist() == tables[name], name
    assert o.KVALUES_IQ4NL.astype(int).tolist() == kv
    assert o.KSIGNS_IQ2XS.astype(int).tolist() == tables["ksigns_iq2xs"]


# ------------------------------------------------------------------------------------ q8_1
def _x(n, k, seed=0, dtype="float32"):
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, k, generator=g)
    x[:, torch.randperm(k, generator=g)[: max(1, k // 256)]] *= 20
    return x.to(getattr(torch, dtype))


def _ties(n, k, seed):
    """Tie-heavy float32 blocks: values at (j + 1/2) * amax/127, where x/d lands on or next to
    a rounding tie (random inputs almost never do)."""
    rng = np.random.default_rng(seed)
    amax = np.exp2(rng.uniform(-4, 4, (n, k // 32))).astype(np.float32)
    j = rng.integers(-126, 126, (n, k // 32, 32)).astype(np.float32)
    x = ((j + np.float32(0.5)) * (amax / np.float32(127))[..., None]).astype(np.float32)
    x[..., 0] = amax
    return x.reshape(n, k)


def _q8_scalar(xrow):
    """Independent scalar restatement of one block_q8_1 (lcpp_shim.cu:274-294), float32 ops
    through numpy scalars, the butterfly spelled out lane by lane."""
    f = np.float32
    x = [f(v) for v in xrow]
    amax = f(0)
    for v in x:
        amax = max(amax, f(abs(v)))
    lanes = list(x)
    for off in (16, 8, 4, 2, 1):
        lanes = [f(lanes[i] + lanes[i ^ off]) for i in range(32)]
    d = f(amax / f(127))
    q = []
    for v in x:
        if amax == 0:
            q.append(0)
            continue
        t = f(v / d)
        r = int(np.trunc(t))
        if abs(float(t) - r) >= 0.5:
            r += 1 if t > 0 else -1
        q.append(r)
    return d, lanes[0], q


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_q8_1_matches_scalar_restatement(dtype):
    x = _x(2, 512, seed=3, dtype=dtype)
    q8 = o.quantize_q8_1(x)
    q, d, s = o.dequant_q8_1(q8, 2, 512)
    xf = x.float().numpy()
    for r in range(2):
        for b in range(16):
            dd, ss, qq = _q8_scalar(xf[r, 32 * b:32 * b + 32])
            assert d[r, b] == np.float32(np.float16(dd))
            assert s[r, b] == np.float32(np.float16(ss))
            assert q[r, 32 * b:32 * b + 32].tolist() == qq


def test_q8_1_properties():
    x = _x(4, 4096, seed=1).numpy()
    x[1, :32] = 0                                    # an all-zero block
    q8 = o.quantize_q8_1(x)
    assert q8.size == 4 * 4096 // 32 * 36
    q, d, s = o.dequant_q8_1(q8, 4, 4096)
    assert (np.abs(q.astype(int)) <= 127).all()
    assert d[1, 0] == 0 and s[1, 0] == 0 and (q[1, :32] == 0).all()
    # d = half(amax/127): every block with amax > 0 reaches |q| = 127 at its amax element
    b = np.abs(q.reshape(4, -1, 32).astype(int)).max(-1)
    nz = np.abs(x.reshape(4, -1, 32)).max(-1) > 0
    assert (b[nz] == 127).all()
    # dequant within half a step (fp32 d, before the half rounding of the stored scale)
    d32 = np.abs(x.reshape(4, -1, 32)).max(-1) / np.float32(127)
    err = np.abs(q.reshape(4, -1, 32) * d32[..., None] - x.reshape(4, -1, 32))
    assert (err <= d32[..., None] * 0.5000001 + 1e-30).all()


def test_q8_1_planted_mistakes_are_visible():
    """The tests above would notice each of these plausible mistakes on ordinary inputs."""
    xr = _x(8, 4096, seed=2).numpy()
    n, k = xr.shape
    x = _ties(n, k, seed=11)
    good = o.dequant_q8_1(o.quantize_q8_1(x), n, k)
    b = x.reshape(n, -1, 32)
    amax = np.abs(b).max(-1)
    d = (amax / np.float32(127)).astype(np.float32)
    # (1) x * (1/d) instead of x / d
    q_mul = o._roundf((b * (np.float32(1) / d)[..., None]).astype(np.float32)).astype(np.int8)
    # (2) half-to-even instead of roundf
    q_even = np.rint((b / d[..., None]).astype(np.float32)).astype(np.int8)
    # (3) sequential sum instead of the butterfly (random inputs)
    br = xr.reshape(n, -1, 32)
    seq = br[..., 0].copy()
    for i in range(1, 32):
        seq = (seq + br[..., i]).astype(np.float32)
    good_r = o.dequant_q8_1(o.quantize_q8_1(xr), n, k)
    diffs = [
        (q_mul.reshape(n, k) != good[0]).any(),
        (q_even.reshape(n, k) != good[0]).any(),
        (seq.astype(np.float16) != good_r[2].astype(np.float16)).any(),
    ]
    assert all(diffs), diffs


def test_q8_1_mmq_layout_and_rounding():
    x = _x(3, 1024, seed=4).numpy()
    x[2, 128:160] = 0
    for qt in (o.IQ3_S, o.Q4_K):
        q8 = o.quantize_q8_1_mmq(x, qt)
        assert q8.size == 3 * 1024 // 128 * 144
        q, d = o.dequant_q8_1_mmq(q8, 3, 1024, qt)
        blk = q8.reshape(1024 // 128, 3, 144)
        # block (k/128)*n + row holds row's values k..k+127
        assert np.array_equal(blk[1, 2, 16:].view(np.int8), q[2, 128:256])
        assert (q[2, 128:160] == 0).all() and d[2, 4] == 0
        # scalar restatement: q = roundf(x * (127/amax)), d = 1/(127/amax)
        for r, b in ((0, 0), (1, 17), (2, 31)):
            xb = x[r, 32 * b:32 * b + 32].astype(np.float32)
            dinv = np.float32(127) / np.float32(np.abs(xb).max())
            qq = o._roundf((xb * dinv).astype(np.float32))
            assert np.array_equal(q[r, 32 * b:32 * b + 32], qq.astype(np.int8))
            dd = np.float32(1) / dinv
            want = np.float32(np.float16(dd)) if qt == o.Q4_K else dd
            assert d[r, b] == want
    # the two layouts round differently somewhere (x/d vs x*(127/amax))
    qa, _, _ = o.dequant_q8_1(o.quantize_q8_1(x), 3, 1024)
    qb, _ = o.dequant_q8_1_mmq(o.quantize_q8_1_mmq(x, o.IQ3_S), 3, 1024, o.IQ3_S)
    big = _ties(16, 4096, seed=9)
    qa2, _, _ = o.dequant_q8_1(o.quantize_q8_1(big), 16, 4096)
    qb2, _ = o.dequant_q8_1_mmq(o.quantize_q8_1_mmq(big, o.IQ3_S), 16, 4096, o.IQ3_S)
    assert (qa2 != qb2).any() and np.abs(qa2.astype(int) - qb2.astype(int)).max() == 1



def _ds4_absorbing_slices(nslices, seed):
    """Slices whose DS4 sum depends on the summation order: value 0 is 2^26 and value 16 is
    -2^26; values 1-3 are 1, 2, 3 and values 17-19 are -1 (each below half an fp32 ulp of the
    +-2^26 they meet, 8, so added to it first they vanish); the other 24 values are small
    integers (exact in any order)."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-9, 10, size=(nslices, 32)).astype(np.float32)
    x[:, 0], x[:, 16] = 2.0 ** 26, -(2.0 ** 26)
    x[:, 1:4] = [1.0, 2.0, 3.0]
    x[:, 17:20] = -1.0
    return x


def test_q8_1_mmq_ds4_sum_pinned():
    """The DS4 sum field (lcpp_shim.cu:320-326): the sum of the 32 raw x values, lane sums
    ((x0 + x1) + x2) + x3 over 8 lanes of 4, then an xor butterfly with offsets 4, 2, 1, as
    half. Pinned by (a) integer inputs, where every order is exact, against the exact sum (a sum
    of q, or of q * d, fails); (b) absorbing inputs, where the 4-value lanes 0 and 4 each reduce
    to +-2^26 before they meet, so exactly the other six lanes survive: the 32-lane butterfly of
    the block_q8_1 quantiser (x0 + x16 first, then the rest exactly) keeps the 1 + 2 + 3 - 3 of
    lanes 0 and 4, and a serial sum drops other values, so both fail."""
    # (a) exact
    rng = np.random.default_rng(21)
    xi = rng.integers(-20, 21, size=(3, 1024)).astype(np.float32)
    s = o.mmq_ds4_sums(o.quantize_q8_1_mmq(xi, o.Q4_K), 3, 1024)
    np.testing.assert_array_equal(s, xi.reshape(3, -1, 32).sum(-1))
    q, d = o.dequant_q8_1_mmq(o.quantize_q8_1_mmq(xi, o.Q4_K), 3, 1024, o.Q4_K)
    qsum = q.astype(np.float64).reshape(3, -1, 32).sum(-1)
    assert (qsum != s).mean() > 0.9 and (np.abs(qsum * d - s) > 0.01).mean() > 0.5
    # (b) order
    xa = _ds4_absorbing_slices(16, seed=22)
    s = o.mmq_ds4_sums(o.quantize_q8_1_mmq(xa.reshape(1, -1), o.Q4_K), 1, 512)[0]
    lanes = xa.reshape(16, 8, 4)
    want = lanes[:, [1, 2, 3, 5, 6, 7]].sum((1, 2))
    np.testing.assert_array_equal(s, want)
    np.testing.assert_array_equal(xa.astype(np.float64).sum(-1) - want, 3.0)  # the exact sum
    bf32 = xa.copy()                                  # block_q8_1's 32-lane order
    for off in (16, 8, 4, 2, 1):
        bf32 = (bf32 + bf32[:, np.arange(32) ^ off]).astype(np.float32)
    np.testing.assert_array_equal(bf32[:, 0] - want, 3.0)
    serial = xa[:, 0].copy()
    for i in range(1, 32):
        serial = (serial + xa[:, i]).astype(np.float32)
    assert (serial != want).any()



def test_q8_1_mmq_d2s6_pinned():
    """Q2_K's MMQ layout D2S6 (mmq.cuh:60-100, lcpp_shim.cu:298-355 with 64 values per scale and 16
    per sum): one half d per 64 values (d_inv = 127 / amax over the 64, q = roundf(x * d_inv)),
    half sums of the 16-value groups 0..5 of every 128 values, none for groups 6, 7. Integer inputs
    pin the sums (exact in every order) and the per-64 scale (a per-32 scale gives other q); the
    absorbing lanes of the DS4 test, placed in one 16-value group, pin the order ((s0 + s2) +
    (s1 + s3)) of its four 4-value lanes."""
    rng = np.random.default_rng(31)
    x = rng.integers(-20, 21, size=(2, 512)).astype(np.float32)
    x[1, 64:128] = 0                                   # an all-zero 64-value half
    x[0, 0:32] *= 0.25                                 # a 32-value half with a smaller amax
    q8 = o.quantize_q8_1_mmq(x, o.Q2_K)
    q, d = o.dequant_q8_1_mmq(q8, 2, 512, o.Q2_K)
    sums = o.mmq_d2s6_sums(q8, 2, 512).reshape(2, 4, 8)
    g16 = x.reshape(2, 4, 8, 16).sum(-1)
    np.testing.assert_array_equal(sums[..., :6], g16[..., :6])
    assert np.isnan(sums[..., 6:]).all()
    for r in range(2):
        for h in range(8):
            xb = x[r, 64 * h:64 * h + 64]
            amax = np.float32(np.abs(xb).max())
            if amax == 0:
                assert (q[r, 64 * h:64 * h + 64] == 0).all() and d[r, 2 * h] == 0
                continue
            dinv = np.float32(127) / amax
            np.testing.assert_array_equal(q[r, 64 * h:64 * h + 64], o._roundf((xb * dinv).astype(np.float32)))
            assert d[r, 2 * h] == d[r, 2 * h + 1] == np.float32(np.float16(np.float32(1) / dinv))
    assert (np.abs(q[0, 0:32]).max() < 127)            # scaled by the 64-value amax, not its own
    # order: lanes 0 and 2 of group 0 reduce to +-2^26 and cancel, the others survive exactly
    xa = rng.integers(-9, 10, size=(1, 128)).astype(np.float32)
    xa[0, 0], xa[0, 1:4], xa[0, 8], xa[0, 9:12] = 2.0 ** 26, [1, 2, 3], -(2.0 ** 26), [-1, -1, -1]
    s0 = o.mmq_d2s6_sums(o.quantize_q8_1_mmq(xa, o.Q2_K), 1, 128)[0, 0]
    assert s0 == xa[0, 4:8].sum() + xa[0, 12:16].sum()
    assert xa[0, :16].astype(np.float64).sum() - s0 == 3.0

def _residual_heavy_x(n, k, seed):
    """Per 32-value slice one value of magnitude a and 31 of magnitude 0.49 * a / 127, all of one
    sign: every small value rounds to q = 0, so sum(x) exceeds d * sum(q) by about 15 d."""
    rng = np.random.default_rng(seed)
    a = np.exp2(rng.uniform(-2, 2, (n, k // 32, 1))).astype(np.float32)
    sign = rng.choice([-1.0, 1.0], size=(n, k // 32, 1)).astype(np.float32)
    x = np.broadcast_to(a * np.float32(0.49 / 127), (n, k // 32, 32)).copy()
    x[..., rng.integers(0, 32)] = a[..., 0]
    return (x * sign).reshape(n, k).astype(np.float32)


def test_q81_model_q4k_min_term_forms():
    """Q4_K's two min-term forms: equal (and equal to the full model) where q * d8 == x exactly;
    apart on residual-heavy inputs, where the 'mmq' form's min term is dmin * m * half(sum x)
    and the 'mmvq' form's dmin * m * d8 * sum(q) (vecdotq.cuh:533-557 against :508-530)."""
    rng = np.random.default_rng(23)
    raw = o.random_blocks(rng, o.Q4_K, 24, 1024)
    xi = rng.integers(-2, 3, size=(3, 1024)).astype(np.float32)
    xi.reshape(3, -1, 32)[..., 5] = 127.0                  # d8 = 1 in both layouts
    a, b, f = (o.q81_model(raw, o.Q4_K, xi, "mmq"), o.q81_model(raw, o.Q4_K, xi, "mmvq"),
               o.full_model(raw, o.Q4_K, xi))
    # equal up to the fp32 rounding of gguf-py's dequantised weight (d*sc*q - dmin*m)
    np.testing.assert_allclose(a, f, rtol=1e-8)
    np.testing.assert_allclose(b, f, rtol=1e-8)
    xr = _residual_heavy_x(3, 1024, seed=24)
    a, b = o.q81_model(raw, o.Q4_K, xr, "mmq"), o.q81_model(raw, o.Q4_K, xr, "mmvq")
    assert o.rel_l2(a, b) > 1e-2                      # ten times the kernels' 1e-3 bar
    # the 'mmq' form keeps the exact slice sums (up to half rounding): it is closer to x . W
    f = o.full_model(raw, o.Q4_K, xr)
    assert o.rel_l2(a, f) < o.rel_l2(b, f)

# ------------------------------------------------------------------------------------ dots
def _brute_dots(raw, qt, q):
    """Pure-Python loops over a tiny case: decode every value from the block bytes directly
    (struct-free bit arithmetic on Python ints), multiply by q8, sum per slice."""
    rows = raw.shape[0]
    n, k = q.shape
    bs = o.BLOCK_BYTES[qt]
    grid = [int(v) for v in o.IQ3S_GRID_U32]
    kv = [int(v) for v in o.KVALUES_IQ4NL]
    out = {}
    for xr in range(n):
        for wr in range(rows):
            for s in range(k // 32):
                blk = [int(v) for v in raw[wr, (s // 8) * bs:(s // 8 + 1) * bs]]
                u = s % 8
                acc, acc_m = 0, 0
                for j in range(32):
                    i = 32 * u + j
                    qx = int(q[xr, 32 * s + j])
                    if qt == o.IQ3_S:
                        gidx = blk[2 + i // 4] | (((blk[66 + i // 32] >> ((i // 4) % 8)) & 1) << 8)
                        gv = (grid[gidx] >> (8 * (i % 4))) & 0xFF
                        sign = -1 if (blk[74 + i // 8] >> (i % 8)) & 1 else 1
                        acc += sign * gv * qx
                    elif qt == o.IQ4_XS:
                        byte = blk[8 + 16 * u + (j % 16)]
                        acc += kv[(byte >> (4 * (j // 16))) & 0xF] * qx
                    elif qt == o.Q4_K:
                        byte = blk[16 + 32 * (u // 2) + j]
                        acc += ((byte >> (4 * (u % 2))) & 0xF) * qx
                        acc_m += qx
                    elif qt == o.Q6_K:
                        h, v = i // 128, i % 128
                        lo = (blk[64 * h + (v % 64)] >> (4 * (v // 64))) & 0xF
                        hi = (blk[128 + 32 * h + (v % 32)] >> (2 * (v // 32))) & 3
                        sc = blk[192 + i // 16]
                        sc = sc - 256 if sc > 127 else sc
                        acc += sc * ((lo | (hi << 4)) - 32) * qx
                    else:
                        wv, scale, mv = _brute_value(blk, qt, i)
                        acc += scale * wv * qx
                        acc_m += mv * qx
                if qt == o.IQ3_S:
                    ls = (blk[106 + u // 2] >> (4 * (u % 2))) & 0xF
                    acc *= 1 + 2 * ls
                elif qt == o.IQ4_XS:
                    sh = blk[2] | (blk[3] << 8)
                    ls = ((blk[4 + u // 2] >> (4 * (u % 2))) & 0xF) | (((sh >> (2 * u)) & 3) << 4)
                    acc *= ls - 32
                elif qt == o.Q4_K:
                    sc12 = blk[4:16]
                    if u < 4:
                        scv, mv = sc12[u] & 63, sc12[u + 4] & 63
                    else:
                        scv = (sc12[u + 4] & 0xF) | ((sc12[u - 4] >> 6) << 4)
                        mv = (sc12[u + 4] >> 4) | ((sc12[u] >> 6) << 4)
                    acc *= scv
                    acc_m *= mv
                out[(xr, wr, s)] = (acc, acc_m)
    return out


def _u16(blk, o2):
    return blk[o2] | (blk[o2 + 1] << 8)


def _u32(blk, o4):
    return _u16(blk, o4) | (_u16(blk, o4 + 2) << 16)


def _brute_value(blk, qt, i):
    """(integer value, integer sub-scale, min factor) of value i of a block of the newer formats,
    from the bytes with plain integer arithmetic (ggml-common.h layouts, dequantize.cuh formulas);
    the value is d * scale * w / den (den 8 for the IQ2 / IQ1 formats, 4 for IQ3_XXS), and Q2_K's
    is d * scale * w - dmin * min."""
    s32, g8, j = i // 32, (i % 32) // 8, i % 8
    if qt == o.Q2_K:
        n, r = i // 128, i % 128
        q = (blk[16 + 32 * n + r % 32] >> (2 * (r // 32))) & 3
        sc = blk[i // 16]
        return q, sc & 0xF, sc >> 4
    if qt in (o.IQ2_XXS, o.IQ3_XXS):
        aux = _u32(blk, 2 + 8 * s32 + 4) if qt == o.IQ2_XXS else _u32(blk, 66 + 4 * s32)
        sign_idx = (aux >> (7 * g8)) & 127
        signs = sign_idx | ((bin(sign_idx).count("1") & 1) << 7)
        if qt == o.IQ2_XXS:
            mag = int(o.IQ2XXS_GRID[blk[2 + 8 * s32 + g8]][j])
        else:
            mag = int(o.IQ3XXS_GRID[blk[2 + 8 * s32 + 2 * g8 + j // 4]][j % 4])
        return (-mag if signs >> j & 1 else mag), 2 * (aux >> 28) + 1, 0
    if qt == o.IQ2_XS:
        v = _u16(blk, 2 + 2 * (4 * s32 + g8))
        signs = (v >> 9) | ((bin(v >> 9).count("1") & 1) << 7)
        mag = int(o.IQ2XS_GRID[v & 511][j])
        sc = (blk[66 + s32] >> (4 * (g8 // 2))) & 0xF
        return (-mag if signs >> j & 1 else mag), 2 * sc + 1, 0
    if qt == o.IQ2_S:
        idx = blk[2 + 4 * s32 + g8] | (((blk[66 + s32] >> (2 * g8)) & 3) << 8)
        signs = blk[34 + 4 * s32 + g8]
        mag = int(o.IQ2S_GRID[idx][j])
        sc = (blk[74 + s32] >> (4 * (g8 // 2))) & 0xF
        return (-mag if signs >> j & 1 else mag), 2 * sc + 1, 0
    if qt == o.IQ1_M:
        grp = i // 8
        nib = (blk[32 + grp // 2] >> (4 * (grp % 2))) & 0xF
        idx = blk[grp] | ((nib & 7) << 8)
        g = int(o.IQ1S_GRID[idx][j])
        delta = -1 if nib & 8 else 1
        sc16 = i // 16
        sc = (_u16(blk, 48 + 2 * (sc16 // 4)) >> (3 * (sc16 % 4))) & 7
        return 8 * g + delta, 2 * sc + 1, 0
    raise ValueError(qt)


@pytest.mark.parametrize("qt", TYPES, ids=lambda t: o.TYPE_NAMES[t])
def test_slice_dots_brute_force(qt):
    rng = np.random.default_rng(5)
    raw = o.random_blocks(rng, qt, 3, 512)
    q = rng.integers(-127, 128, size=(2, 512)).astype(np.int8)
    dots = o.slice_dots(raw, qt, q)
    brute = _brute_dots(raw, qt, q)
    for (xr, wr, s), (a, m) in brute.items():
        assert dots["dot"][xr, wr, s] == a
        if qt in (o.Q4_K, o.Q2_K):
            assert dots["m"][xr, wr, s] == m


@pytest.mark.parametrize("path", [f for f in FILES if "__r0" in f], ids=lambda p: os.path.basename(p)[:-4])
def test_slice_dots_scale_identity_on_golden_rows(path):
    """d_w * (integer slice dot) * d8 summed over slices == dequant(W) . (q * d8), both in
    float64, to 1e-12 relative: the integer dots carry every sub-scale of the format."""
    raw, ref, qt = _load(path)
    k = ref.size
    x = _x(2, k, seed=6).numpy()
    q, d8, _ = o.dequant_q8_1(o.quantize_q8_1(x), 2, k)
    dots = o.slice_dots(raw.reshape(1, -1), qt, q)
    t = o.decode_int(raw, qt)
    dw = np.repeat(t["d"].astype(np.float64), 8)
    y = (dots["dot"][:, 0, :] * dw[None] * d8).sum(-1) / dots.get("den", 1)
    if "m" in dots:
        y -= (dots["m"][:, 0, :] * np.repeat(t["dmin"].astype(np.float64), 8)[None] * d8).sum(-1)
    want = (q.astype(np.float64).reshape(2, -1, 32) * d8[..., None]).reshape(2, k) @ ref.astype(np.float64)
    np.testing.assert_allclose(y, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())


def test_q81_model_close_to_full_and_not_equal():
    rng = np.random.default_rng(7)
    raw = o.random_blocks(rng, o.IQ3_S, 64, 2048)
    x = _x(4, 2048, seed=8)
    y81 = o.q81_model(raw, o.IQ3_S, x)
    yf = o.full_model(raw, o.IQ3_S, x)
    e = o.rel_l2(y81, yf)
    assert 1e-4 < e < 2e-2, e


# ------------------------------------------------------------------------------------ MMVQ forms
def _units_inputs(qt, seed):
    rng = np.random.default_rng(seed)
    raw = o.random_blocks(rng, qt, 16, 1024)
    q = rng.integers(-127, 128, size=(3, 1024)).astype(np.int8)
    return raw, q, o.slice_dots(raw, qt, q)


@pytest.mark.parametrize("qt", o.UNIT_TYPES, ids=lambda t: o.TYPE_NAMES[t])
def test_mmvq_slice_units_pinned(qt):
    """The decode ops' truncated slice values against what fixes them without the C expression:
      * within 1.125 of the exact dot / den (truncations lose less than 1 plus 1/8);
      * IQ2_XXS: the truncation of dot / 8; IQ1_M: dot / 8 itself (no division);
      * IQ3_XXS: the truncation of dot / 4, the identity the reference's owned kernel states for
        the vendored (s * sumi + sumi / 2) / 2 (lcpp_owned_iq3_mma.cu:31);
      * IQ2_XS, IQ2_S: the truncation of dot / 8 wherever sumi_a + sumi_b is even (the inner
        halving is then exact), and a different value somewhere it is odd with a negative total
        (the inner truncation then rounds toward zero from the other side)."""
    raw, q, dots = _units_inputs(qt, 9)
    units = o.mmvq_slice_units(raw, qt, q)
    exact = dots["dot"] / dots["den"]
    assert np.abs(units - exact).max() < 1.125
    assert (units == np.round(units)).all() or qt == o.IQ1_M
    trunc = np.trunc(exact)
    if qt == o.IQ2_XXS:
        np.testing.assert_array_equal(units, np.trunc(dots["dot"] / 8))
    elif qt == o.IQ1_M:
        np.testing.assert_array_equal(units, dots["dot"] / 8)
    elif qt == o.IQ3_XXS:
        np.testing.assert_array_equal(units, np.trunc(dots["dot"] / 4))
    else:
        t = o.decode_int(raw.reshape(-1), qt)
        w = t["w"].astype(np.int64).reshape(16, 32, 2, 16)
        qq = q.astype(np.int64).reshape(3, 32, 2, 16)
        tot = np.einsum("rsth,nsth->nrs", w, qq)
        even = tot % 2 == 0
        np.testing.assert_array_equal(units[even], trunc[even])
        assert (units[~even] != trunc[~even]).any()


def test_mmvq_planted_floor_division_is_visible():
    """Floor division in place of C's truncation changes the IQ3_XXS values on these inputs."""
    raw, q, dots = _units_inputs(o.IQ3_XXS, 10)
    units = o.mmvq_slice_units(raw, o.IQ3_XXS, q)
    assert (units != np.floor(dots["dot"] / 4)).any()
    assert (dots["dot"] < 0).any()
