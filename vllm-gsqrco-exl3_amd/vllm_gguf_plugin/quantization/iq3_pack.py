"""Load-time repack of IQ3 weight rows into this build's layout, in place.

Replaces the reference's quantization/iq3_pack.py (ROWS 36, pack_ 121-131, pack 134-138,
unpack 141-181) with the same interface over layouts of this build's own:
  * IQ3_S: 4-row units whose 1760-byte unit-blocks (4 rows x 4 K blocks) are ordered for the
    gfx950 decode GEMV's coalesced 16-byte loads (csrc/iq3_tile.h documents the byte map).
  * IQ3_XXS: the same units, 1568-byte unit-blocks with the grid indices, the sign / scale words
    and the d values of a unit-block's 16 blocks each in one field (csrc/iq3_tile.h).
The permutations run on the GPU (gguf_iq3_pack in libgguf_mi355x.so); each is a bijection
(unpack(pack(w)) == w) that keeps every 4-row unit inside its own rows' bytes.
"""

import torch

from .. import _capi
from .utils import WeightType

ROWS = 16  # rows per tile


_BLOCK_BYTES = {WeightType.IQ3_S: 110, WeightType.IQ3_XXS: 98}


def _run(w: torch.Tensor, weight_type: int, unpack: bool) -> None:
    weight_type = WeightType(weight_type)
    assert weight_type in _BLOCK_BYTES, weight_type
    assert w.dim() == 2 and w.dtype == torch.uint8, (w.dim(), w.dtype)
    rows, rb = w.shape
    assert rows % ROWS == 0 and rb % _BLOCK_BYTES[weight_type] == 0, w.shape
    assert rows == 1 or w.stride(0) == rb, "rows must be contiguous"
    if not w.is_cuda:
        raise RuntimeError("iq3_pack: W must be a CUDA tensor (the repack runs on the GPU)")
    lib = _capi.load()
    sb = lib.gguf_iq3_pack_scratch_bytes(rows, rb)
    scratch = torch.empty(sb, dtype=torch.uint8, device=w.device)
    with torch.cuda.device(w.device):
        _capi.check(lib, lib.gguf_iq3_pack(w.data_ptr(), int(weight_type), rows, rb, int(unpack), scratch.data_ptr(),
                                           sb, _capi.stream_of(w)))


def pack_(w: torch.Tensor, weight_type: int) -> None:
    """GGUF IQ3 rows [rows, row_bytes] (rows % 16 == 0) -> this build's layout, in place."""
    _run(w, weight_type, unpack=False)


def pack(w: torch.Tensor, weight_type: int) -> torch.Tensor:
    """This build's layout of w, as a new tensor of the same shape."""
    p = w.clone()
    pack_(p, weight_type)
    return p


def unpack(p: torch.Tensor, weight_type: int) -> torch.Tensor:
    """Inverse of pack: the GGUF block bytes."""
    u = p.clone()
    _run(u, weight_type, unpack=True)
    return u
