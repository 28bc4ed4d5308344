"""CPU oracle for the GGUF quantized-matmul path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker (or, in bench.py, as the timed CPU baseline). The
product path (vllm-gsqrco-exl3_amd/) never imports it and has no CPU fallback.

A numpy restatement of the reference's arithmetic, each function citing the reference
file:line it follows (paths relative to the reference repository root):

  formats     plugin/vllm_gguf_plugin/csrc/lcpp/ggml/src/ggml-common.h:259-268 (block_q8_1),
              :327-338 (block_q4_K), :362-368 (block_q6_K), :415-422 (block_iq3_s),
              :454-460 (block_iq4_xs), :1052 (iq3s_grid), :1120 (kvalues_iq4nl)
  dequant     gguf-py b11211 gguf.quants.<T>.dequantize_blocks (a third-party dependency of
              the reference, absent here; called from tests/gpu/_refs.py:33-37 and pinned by
              the golden rows tests/fixtures/dequant/*.npz); the same formulas as
              plugin/vllm_gguf_plugin/csrc/gguf/dequantize.cuh:156-197,233-256,335-353,421-434
  q8_1        plugin/vllm_gguf_plugin/csrc/lcpp_shim.cu:274-294 (MMVQ layout) and :298-355
              (MMQ layout, block_q8_1_mmq of ggml-cuda/mmq.cuh:27-56, ds layout :60-100);
              warp reductions ggml-cuda/common.cuh:468-474,528-534
  slice dots  ggml-cuda/vecdotq.cuh:508-530 (Q4_K MMVQ), :627-648 (Q6_K MMVQ),
              :1211-1248 (IQ3_S), :1357-1380 (IQ4_XS)
  q81 model   tests/gpu/_refs.py:40-54,78-91 (y = dequant(q8_1(x)) @ dequant(W).T, float64)

How each part is pinned (tests/test_oracle.py):
  dequant     bit-exact against the reference's golden rows (tests/golden/dequant, fp32 gguf-py
              output on real GGUF rows) for IQ3_S, Q4_K, IQ4_XS and Q6_K.
  tables      IQ3S_GRID against the reference header itself when oracle/_ref is built (the
              recipe in oracle/Makefile compiles ggml-common.h's tables), else against the
              golden rows (every entry the rows reach) and the grid's invariants.
  q8_1        closed form: d = amax/127 exactly as IEEE fp32 division, roundf ties away from
              zero, |q| <= 127, all-zero block -> (0, 0, 0), the xor-butterfly sum order
              checked against brute-force float32 trees, dequant(q8_1(x)) within d/2 of x.
  slice dots  brute force: int64 sum of decoded int8 weight x q8 per slice, and the identity
              d_w*scale*sumi*d8 == sum(dequant(w) * q*d8) up to fp32 rounding.
The reference's q8_1 bytes have no golden vectors in the reference repository (its checks
are GPU-vs-GPU), so the q8_1 bytes are pinned by the closed form only.
"""

from __future__ import annotations

import numpy as np

QK_K = 256
QK8_1 = 32

# ggml type ids (gguf-py GGMLQuantizationType, restated from tests/cpu/test_lcpp_guards.py:22)
Q4_K, Q6_K, IQ3_S, IQ4_XS = 12, 14, 21, 23
TYPE_NAMES = {Q4_K: "Q4_K", Q6_K: "Q6_K", IQ3_S: "IQ3_S", IQ4_XS: "IQ4_XS"}
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}
# bytes per 256-value block (ggml-common.h static_asserts)
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, IQ3_S: 110, IQ4_XS: 136}

# --------------------------------------------------------------------------- tables
# iq3s_grid (ggml-common.h:1052) is the ascending list of the 512 points of {1,3,..,15}^4
# that IQ3_S uses. Encoded here as a 4096-bit membership set over codes
# c = sum_i ((byte_i - 1) / 2) << 3i; enumerating members in ascending c gives the table in
# its ascending uint32 order (byte 3 is the most significant in both).
_IQ3S_MEMBERS = (
    0x92050aa5082357a7, 0x0422001022892317, 0x09000aa4112249a3, 0x228005104a052208,
    0x0100020904128801, 0x084000a208450014, 0x0200040002000a40, 0x0000110008450015,
    0x040250005205ab17, 0x410005020902114b, 0x040120090411a401, 0x0104000211820992,
    0x000011440a001428, 0x0000020005020902, 0x0000005000910000, 0x010400022002050a,
    0x2980052a058a55ab, 0x0000020412248905, 0x12008802810a0092, 0x004001040a140225,
    0x2400000224090082, 0x0100080180040210, 0x0002200000020085, 0x0000010801400220,
    0x020802942a04aa04, 0x44010001000a102a, 0x0000010014010401, 0x0800208a018a1102,
    0x0011040002044208, 0x0800401004200502, 0x0000000200004000, 0x000000002005000a,
    0x0100010204910411, 0x0000220821040a84, 0x010480010802210a, 0x0000000022050a10,
    0x0200000180100005, 0x00040000000200a0, 0x0001000010000800, 0x0000020801002100,
    0x1040049100041104, 0x040000000402042a, 0x0000080041080201, 0x0820021000800184,
    0x0000004004010012, 0x00000a0000400400, 0x0000000400000000, 0x0000000000040014,
    0x000100000a002a00, 0x0010000000810001, 0x0104200410000400, 0x0000000100021001,
    0x0004000800200000, 0x0001000010000009, 0x0000000100000020, 0x0000000000000a00,
    0x0004100140050091, 0x0000002800100204, 0x0000020001024112, 0x0000080024000004,
    0x0000010000010822, 0x0000000400040000, 0x0000000002000004, 0x0000000000000001,
)


def _iq3s_grid() -> np.ndarray:
    codes = [w * 64 + j for w, bits in enumerate(_IQ3S_MEMBERS) for j in range(64) if bits >> j & 1]
    out = np.zeros((len(codes), 4), dtype=np.uint8)
    for i, c in enumerate(codes):
        for b in range(4):
            out[i, b] = 2 * ((c >> (3 * b)) & 7) + 1
    return out


IQ3S_GRID = _iq3s_grid()                     # [512, 4] uint8, byte b of entry i
IQ3S_GRID_U32 = IQ3S_GRID.astype(np.uint32) @ (1 << (8 * np.arange(4, dtype=np.uint32)))
# kvalues_iq4nl (ggml-common.h:1120): the IQ4_NL / IQ4_XS non-linear codebook
KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                         dtype=np.int8)


# --------------------------------------------------------------------------- helpers
def _blocks(raw: np.ndarray, qt: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    bs = BLOCK_BYTES[qt]
    assert raw.size % bs == 0, (raw.shape, qt)
    return raw.reshape(-1, bs)


def _f16(b: np.ndarray) -> np.ndarray:
    """[..., 2] uint8 little-endian -> float32 (fp16 widened, exact)."""
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)[..., 0]


def _q4k_scale_min(sc12: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """get_scale_min_k4 (csrc/gguf/dequantize.cuh:156-163) for j = 0..7: 6-bit scale and min."""
    s = sc12.astype(np.int32)
    j = np.arange(8)
    lo = j < 4
    sc = np.where(lo, s[:, np.minimum(j, 3)] & 63,
                  (s[:, np.minimum(j + 4, 11)] & 0xF) | ((s[:, np.maximum(j - 4, 0)] >> 6) << 4))
    mn = np.where(lo, s[:, np.minimum(j + 4, 11)] & 63,
                  (s[:, np.minimum(j + 4, 11)] >> 4) | ((s[:, np.minimum(j, 7)] >> 6) << 4))
    return sc, mn


# --------------------------------------------------------------------------- integer decode
def decode_int(raw: np.ndarray, qt: int) -> dict:
    """Blocks -> integer codes and scales, the form the kernels' integer dots use.

    Returns (per block b, value i in 0..255):
      IQ3_S : w[b,i] = sign * grid (odd, |w| <= 15); ls[b,s] = 1 + 2*scale nibble (per 32); d[b]
      IQ4_XS: w = kvalues_iq4nl[q]; ls[b,s] = scale - 32 (per 32); d[b]
      Q4_K  : w = 4-bit quant (0..15); sc[b,s], m[b,s] (6-bit, per 32); d[b], dmin[b]
      Q6_K  : w = q - 32 (in [-32, 31]); sc[b,t] int8 per 16; d[b]
    """
    b = _blocks(raw, qt)
    nb = b.shape[0]
    if qt == IQ3_S:
        # block_iq3_s: d[0:2] qs[2:66] qh[66:74] signs[74:106] scales[106:110]
        d = _f16(b[:, 0:2])
        qs = b[:, 2:66].astype(np.int32)                   # [nb, 64] one per 4-value group
        qh = b[:, 66:74].astype(np.int32)                  # [nb, 8] bit e of qh[s] -> group 8s+e
        g = np.arange(64)
        idx = qs | (((qh[:, g // 8] >> (g % 8)) & 1) << 8)
        vals = IQ3S_GRID[idx].astype(np.int32)             # [nb, 64, 4]
        sg = b[:, 74:106].astype(np.int32)                 # [nb, 32]: byte t -> values 8t..8t+7
        v = np.arange(256)
        sbit = (sg[:, v // 8] >> (v % 8)) & 1
        w = vals.reshape(nb, 256) * (1 - 2 * sbit)
        sc = b[:, 106:110].astype(np.int32)
        s = np.arange(8)
        ls = 1 + 2 * ((sc[:, s // 2] >> (4 * (s % 2))) & 0xF)
        return {"w": w.astype(np.int8), "ls": ls, "d": d}
    if qt == IQ4_XS:
        # block_iq4_xs: d[0:2] scales_h[2:4] scales_l[4:8] qs[8:136]
        d = _f16(b[:, 0:2])
        sh = b[:, 2].astype(np.int32) | (b[:, 3].astype(np.int32) << 8)
        sl = b[:, 4:8].astype(np.int32)
        s = np.arange(8)
        ls = ((sl[:, s // 2] >> (4 * (s % 2))) & 0xF) | (((sh[:, None] >> (2 * s)) & 3) << 4)
        qs = b[:, 8:136].astype(np.int32).reshape(nb, 8, 16)   # slice s: 16 bytes
        q = np.concatenate([qs & 0xF, qs >> 4], axis=2)          # values 0..15 low, 16..31 high
        w = KVALUES_IQ4NL[q.reshape(nb, 256)]
        return {"w": w, "ls": ls - 32, "d": d}
    if qt == Q4_K:
        # block_q4_K: d[0:2] dmin[2:4] scales[4:16] qs[16:144]
        d = _f16(b[:, 0:2])
        dmin = _f16(b[:, 2:4])
        sc, m = _q4k_scale_min(b[:, 4:16])
        qs = b[:, 16:144].astype(np.int32).reshape(nb, 4, 32)  # qs[32j+l]: values 64j+l, 64j+32+l
        q = np.concatenate([qs & 0xF, qs >> 4], axis=2)         # [nb, 4, 64]
        return {"w": q.reshape(nb, 256).astype(np.int8), "sc": sc, "m": m, "d": d, "dmin": dmin}
    if qt == Q6_K:
        # block_q6_K: ql[0:128] qh[128:192] scales[192:208] (int8) d[208:210]
        ql = b[:, 0:128].astype(np.int32).reshape(nb, 2, 64)
        qh = b[:, 128:192].astype(np.int32).reshape(nb, 2, 32)
        sc = b[:, 192:208].view(np.int8).astype(np.int32)
        d = _f16(b[:, 208:210])
        l = np.arange(32)
        q = np.empty((nb, 2, 128), dtype=np.int32)
        q[:, :, l] = (ql[:, :, l] & 0xF) | ((qh[:, :, l] & 3) << 4)
        q[:, :, l + 32] = (ql[:, :, l + 32] & 0xF) | (((qh[:, :, l] >> 2) & 3) << 4)
        q[:, :, l + 64] = (ql[:, :, l] >> 4) | (((qh[:, :, l] >> 4) & 3) << 4)
        q[:, :, l + 96] = (ql[:, :, l + 32] >> 4) | (((qh[:, :, l] >> 6) & 3) << 4)
        return {"w": (q.reshape(nb, 256) - 32).astype(np.int8), "sc": sc, "d": d}
    raise ValueError(f"decode_int: type {qt} not served")


# --------------------------------------------------------------------------- dequant (gguf-py)
def dequantize(raw: np.ndarray, qt: int) -> np.ndarray:
    """GGUF blocks -> float32 values, the gguf-py b11211 arithmetic (products in float32, the
    same order; every product below is exact in float32 except Q6_K's d*sc*q and Q4_K's
    difference, each a single rounding of the exact value)."""
    t = decode_int(raw, qt)
    nb = t["w"].shape[0]
    w = t["w"].astype(np.float32)
    if qt == IQ3_S:
        db = (t["d"][:, None] * t["ls"].astype(np.float32))          # [nb, 8]
        return (np.repeat(db, 32, axis=1) * w).reshape(-1)
    if qt == IQ4_XS:
        dl = (t["d"][:, None] * t["ls"].astype(np.float32))
        return (np.repeat(dl, 32, axis=1) * w).reshape(-1)
    if qt == Q4_K:
        dd = t["d"][:, None] * t["sc"].astype(np.float32)
        dm = t["dmin"][:, None] * t["m"].astype(np.float32)
        return (np.repeat(dd, 32, axis=1) * w - np.repeat(dm, 32, axis=1)).reshape(-1)
    if qt == Q6_K:
        dd = t["d"][:, None] * t["sc"].astype(np.float32)            # [nb, 16]
        return (np.repeat(dd, 16, axis=1) * w).reshape(nb * 256)
    raise ValueError(qt)


# --------------------------------------------------------------------------- q8_1
def _roundf(t: np.ndarray) -> np.ndarray:
    """C roundf on float32: nearest integer, ties away from zero (t - trunc(t) is exact)."""
    r = np.trunc(t)
    frac = np.abs(t - r)
    return r + np.where(frac >= 0.5, np.sign(t), 0).astype(np.float32)


def _xor_tree_sum(v: np.ndarray, offsets) -> np.ndarray:
    """Lane 0 of a float32 xor-butterfly sum over the last axis (x += shfl_xor(x, off))."""
    n = v.shape[-1]
    lanes = np.arange(n)
    for off in offsets:
        v = (v + v[..., lanes ^ off]).astype(np.float32)
    return v[..., 0]


def _as_f32(x) -> np.ndarray:
    if hasattr(x, "detach"):  # torch tensor of any float dtype: widening to fp32 is exact
        x = x.detach().cpu().float().numpy()
    return np.ascontiguousarray(x, dtype=np.float32)


def quantize_q8_1(x) -> np.ndarray:
    """X [n, K] -> block_q8_1 bytes (n*K/32 blocks of 36 B, row-major by (row, block)):
    half d, half sum, 32 x int8. lcpp_shim.cu:274-294: d = amax/127.0f, q = amax == 0 ? 0 :
    roundf(x/d), sum by a 32-lane xor butterfly (offsets 16..1), ds = make_half2(d, sum)."""
    xf = _as_f32(x)
    n, k = xf.shape
    assert k % QK8_1 == 0
    b = xf.reshape(n, k // QK8_1, QK8_1)
    amax = np.abs(b).max(-1)
    s = _xor_tree_sum(b, (16, 8, 4, 2, 1))
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (b / d[..., None]).astype(np.float32)
    q = np.where(amax[..., None] == 0, 0, _roundf(t)).astype(np.int8)
    out = np.zeros((n, k // QK8_1, 36), dtype=np.uint8)
    with np.errstate(over="ignore"):
        out[..., 0:2] = d.astype(np.float16)[..., None].view(np.uint8)
        out[..., 2:4] = s.astype(np.float16)[..., None].view(np.uint8)
    out[..., 4:36] = q.view(np.uint8)
    return out.reshape(-1)


def dequant_q8_1(q8: np.ndarray, n: int, k: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """block_q8_1 bytes -> (q int8 [n, K], d float32 [n, K/32] (from half), sum float32)."""
    blk = np.ascontiguousarray(q8, dtype=np.uint8).reshape(n, k // QK8_1, 36)
    d = blk[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    s = blk[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float32)
    q = blk[..., 4:36].copy().view(np.int8).reshape(n, k)
    return q, d, s


# ds layouts of block_q8_1_mmq (mmq.cuh:60-100) for the served types
MMQ_DS4_TYPES = (Q4_K,)


def quantize_q8_1_mmq(x, qt: int) -> np.ndarray:
    """X [n, K] -> block_q8_1_mmq bytes: 144-B blocks of 128 values, block index
    (k/128)*n + row; bytes 0..15 = 4 x fp32 d (D4) or 4 x half2(d, sum) (DS4, Q4_K), bytes
    16..143 = 128 x int8. lcpp_shim.cu:298-355: per 32 values d_inv = 127/amax,
    q = roundf(x*d_inv), d = 1/d_inv; sum = ((x0+x1)+x2)+x3 per lane, then xor offsets 4,2,1.
    amax == 0 gives q = 0 and d = 0 (the reference's NaN -> 0 int8 conversion and 1/inf)."""
    xf = _as_f32(x)
    n, k = xf.shape
    assert k % 128 == 0
    b = xf.reshape(n, k // 32, 32)
    amax = np.abs(b).max(-1)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        d_inv = (np.float32(127.0) / amax).astype(np.float32)
        t = (b * d_inv[..., None]).astype(np.float32)
        d = (np.float32(1.0) / d_inv).astype(np.float32)
    q = np.where(amax[..., None] == 0, 0, _roundf(np.nan_to_num(t))).astype(np.int8)
    d = np.where(amax == 0, np.float32(0), d).astype(np.float32)
    lane = b.reshape(n, k // 32, 8, 4)
    ls = (((lane[..., 0] + lane[..., 1]).astype(np.float32) + lane[..., 2]).astype(np.float32)
          + lane[..., 3]).astype(np.float32)
    s = _xor_tree_sum(ls, (4, 2, 1))
    out = np.zeros((k // 128, n, 144), dtype=np.uint8)
    d4 = d.reshape(n, k // 128, 4).transpose(1, 0, 2)
    q4 = q.reshape(n, k // 128, 128).transpose(1, 0, 2)
    s4 = s.reshape(n, k // 128, 4).transpose(1, 0, 2)
    if qt in MMQ_DS4_TYPES:
        with np.errstate(over="ignore"):
            ds = np.stack([d4.astype(np.float16), s4.astype(np.float16)], -1)  # [.., 4, 2]
        out[..., 0:16] = np.ascontiguousarray(ds).view(np.uint8).reshape(k // 128, n, 16)
    else:
        out[..., 0:16] = np.ascontiguousarray(d4).view(np.uint8).reshape(k // 128, n, 16)
    out[..., 16:144] = q4.view(np.uint8)
    return out.reshape(-1)


def mmq_ds4_sums(q8: np.ndarray, n: int, k: int) -> np.ndarray:
    """The half2 sum field of DS4 block_q8_1_mmq bytes (Q4_K), widened: float32 [n, K/32]."""
    blk = np.ascontiguousarray(q8, dtype=np.uint8).reshape(k // 128, n, 144)
    s = blk[..., :16].copy().view(np.float16).reshape(k // 128, n, 4, 2)[..., 1].astype(np.float32)
    return np.ascontiguousarray(s.transpose(1, 0, 2).reshape(n, k // 32))


def dequant_q8_1_mmq(q8: np.ndarray, n: int, k: int, qt: int) -> tuple[np.ndarray, np.ndarray]:
    """block_q8_1_mmq bytes -> (q int8 [n, K], d float32 [n, K/32]) (d from half for DS4)."""
    blk = np.ascontiguousarray(q8, dtype=np.uint8).reshape(k // 128, n, 144)
    q = blk[..., 16:].copy().view(np.int8).transpose(1, 0, 2).reshape(n, k)
    hdr = blk[..., :16].copy()
    if qt in MMQ_DS4_TYPES:
        d = hdr.view(np.float16).reshape(k // 128, n, 4, 2)[..., 0].astype(np.float32)
    else:
        d = hdr.view(np.float32).reshape(k // 128, n, 4)
    return q, np.ascontiguousarray(d.transpose(1, 0, 2).reshape(n, k // 32))


# --------------------------------------------------------------------------- integer slice dots
def slice_dots(raw: np.ndarray, qt: int, q: np.ndarray) -> dict:
    """Per (activation row, weight row, 32-value slice) integer dot products, int64, exactly as
    the reference's vec_dot functions form them before any float scale:
      IQ3_S : sumi * (1 + 2*ls)                        (vecdotq.cuh:1211-1248)
      IQ4_XS: sumi * (ls - 32)                         (vecdotq.cuh:1357-1380)
      Q6_K  : sc_a * sumi_a + sc_b * sumi_b, 16 each   (vecdotq.cuh:627-648)
      Q4_K  : 'd' = sc * sum(nib * q8), 'm' = m * sum(q8)  (vecdotq.cuh:508-530)
    raw: [rows, row_bytes]; q: int8 [n, K]. Returns dict of int64 [n, rows, K/32]."""
    rows = raw.shape[0]
    t = decode_int(raw.reshape(-1), qt)
    n, k = q.shape
    ns = k // 32
    w = t["w"].astype(np.int64).reshape(rows, ns, 32)
    qq = q.astype(np.int64).reshape(n, ns, 32)
    if qt == Q6_K:
        w16 = w.reshape(rows, ns, 2, 16)
        q16 = qq.reshape(n, ns, 2, 16)
        sumi = np.einsum("rstv,nstv->nrst", w16, q16)                   # [n, rows, ns, 2]
        sc = t["sc"].reshape(rows, ns, 2).astype(np.int64)
        return {"dot": (sumi * sc[None]).sum(-1)}
    sumi = np.einsum("rsv,nsv->nrs", w, qq)
    if qt == IQ3_S or qt == IQ4_XS:
        return {"dot": sumi * t["ls"].reshape(rows, ns).astype(np.int64)[None]}
    if qt == Q4_K:
        sq = qq.sum(-1)                                                 # [n, ns]
        return {"dot": sumi * t["sc"].reshape(rows, ns).astype(np.int64)[None],
                "m": sq[:, None, :] * t["m"].reshape(rows, ns).astype(np.int64)[None]}
    raise ValueError(qt)


# --------------------------------------------------------------------------- reference models
def q81_model(raw: np.ndarray, qt: int, x, layout: str = "mmvq") -> np.ndarray:
    """float64 y[n, rows] = dequant(q8_1(x)) @ dequant(W).T (tests/gpu/_refs.py:40-54,83).
    layout 'mmvq': x' = q * half(d) (block_q8_1, lcpp_shim.cu:274-294); 'mmq': x' = q * d
    with the MMQ layout's rounding and fp32 d (half d for DS4 types, lcpp_shim.cu:298-355).
    Q4_K's min term follows the layout's vec_dot: with 'mmvq' it is dmin * m * d8 * sum(q8) per
    slice (vec_dot_q4_K_q8_1_impl_vmmq, vecdotq.cuh:508-530), which is what dequant(q8_1(x)) .
    dequant(W) gives; with 'mmq' it is dmin * m * half(sum(x)) per slice, the DS4 sum of the
    block_q8_1_mmq bytes (vec_dot_q4_K_q8_1_impl_mmq, vecdotq.cuh:533-557)."""
    xf = _as_f32(x)
    n, k = xf.shape
    rows = raw.shape[0]
    if layout == "mmvq":
        q, d, _ = dequant_q8_1(quantize_q8_1(xf), n, k)
    else:
        q8 = quantize_q8_1_mmq(xf, qt)
        q, d = dequant_q8_1_mmq(q8, n, k, qt)
    xq = (q.astype(np.float64).reshape(n, k // 32, 32) * d.astype(np.float64)[..., None]).reshape(n, k)
    if qt == Q4_K and layout == "mmq":
        t = decode_int(raw.reshape(-1), qt)
        dd = (t["d"][:, None] * t["sc"].astype(np.float32)).astype(np.float64)        # [nb, 8]
        main = (np.repeat(dd, 32, axis=1) * t["w"].astype(np.float64)).reshape(rows, k)
        mins = (t["dmin"][:, None] * t["m"].astype(np.float32)).astype(np.float64).reshape(rows, k // 32)
        return xq @ main.T - mmq_ds4_sums(q8, n, k).astype(np.float64) @ mins.T
    W = dequantize(raw.reshape(-1), qt).astype(np.float64).reshape(rows, k)
    return xq @ W.T


def full_model(raw: np.ndarray, qt: int, x) -> np.ndarray:
    """float64 x @ dequant(W).T (no activation quantization)."""
    xf = _as_f32(x).astype(np.float64)
    rows = raw.shape[0]
    W = dequantize(raw.reshape(-1), qt).astype(np.float64).reshape(rows, xf.shape[1])
    return xf @ W.T


def rel_l2(y, ref) -> float:
    """max over activation rows of ||y - ref|| / ||ref|| (tests/gpu/_refs.py:94-99)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    num = np.linalg.norm(y - ref, axis=-1)
    den = np.maximum(np.linalg.norm(ref, axis=-1), 1e-30)
    return float((num / den).max())


# --------------------------------------------------------------------------- synthetic weights
def random_blocks(rng: np.random.Generator, qt: int, rows: int, k: int,
                  scale_sigma: float = 2e-3) -> np.ndarray:
    """Seeded synthetic GGUF rows [rows, k/256*bytes]: uniform random code bytes with every fp16
    scale replaced by |N(0, scale_sigma)| (the benchmark configs; the reference's recipe is
    kit/synth.py:70-87, uniform bytes with valid fp16 scales)."""
    bs = BLOCK_BYTES[qt]
    nb = rows * (k // QK_K)
    b = rng.integers(0, 256, size=(nb, bs), dtype=np.uint8)
    offs = {IQ3_S: (0,), IQ4_XS: (0,), Q4_K: (0, 2), Q6_K: (208,)}[qt]
    for off in offs:
        s = np.abs(rng.normal(0.0, scale_sigma, nb)).astype(np.float16)
        b[:, off:off + 2] = s.view(np.uint8).reshape(nb, 2)
    return b.reshape(rows, -1)
