"""The C-ABI library loads without a GPU and exports every symbol include/gguf_mi355x.h declares;
its host-side helpers answer without touching the GPU."""

import ctypes
import os
import re

from conftest import ROOT

from vllm_gguf_plugin import _capi

HEADER = os.path.join(ROOT, "include", "gguf_mi355x.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"GGUF_API\s+[\w\s\*]+?\b(gguf_\w+)\s*\(", src)))


def test_header_declares_the_op_surface():
    names = _declared()
    assert len(names) == 21
    for op in _capi.OPS:
        assert "gguf_" + op in names
    assert "gguf_lcpp_quantize_q8_1" in names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)
    assert set(_declared()) == set(_capi.EXPORTS)


def test_no_other_exports():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", _capi.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == set(_declared())


def test_host_helpers(lib):
    assert lib.gguf_version().startswith(b"gguf_mi355x")
    assert lib.gguf_q8_1_bytes(4, 5120, 0) == 4 * 5120 // 32 * 36
    assert lib.gguf_q8_1_bytes(512, 5120, 1) == 2949120
    # decode ops need the q8_1 copy of X unless x_q8 is given; GEMM ops always the MMQ copy
    assert lib.gguf_op_workspace_bytes(0, 21, 17408, 5120, 4, 0) >= 4 * 5120 // 32 * 36
    assert lib.gguf_op_workspace_bytes(0, 21, 17408, 5120, 4, 1) == 0
    assert lib.gguf_op_workspace_bytes(1, 21, 17408, 5120, 48, 1) >= 48 * 5120 // 128 * 144
    # whole 16-row tiles, at most 64 MiB (or the whole tensor if smaller)
    assert lib.gguf_iq3_pack_scratch_bytes(17408, 2200) == 17408 * 2200
    assert lib.gguf_iq3_pack_scratch_bytes(65536, 2200) == (64 << 20) // (16 * 2200) * 16 * 2200


def test_workspace_follows_the_product_plan(lib):
    """Product ops size their workspace for the activation layout of the GEMM they run: the int8
    layout (4,608 B per 16 rows x 256 values) below 64 rows, the fp16 one (9,216 B) for packed
    IQ3_S and Q4_K from 64 rows at K <= 8192, below that where the fp16 GEMM's range plan takes
    the weight (1..5 row tiles per CU, 256 CUs assumed without a GPU; IQ3_S from 33 rows, Q4_K
    from 17), and for the prefill from 256 rows; IQ4_XS and K = 17408 stay on the int8 layout below the prefill
    (plus a K split's slots and counters on grids of few tiles)."""
    xq = lambda n, k: -(-n // 16) * (k // 256) * 4608
    xh = lambda n, k: -(-n // 16) * (k // 256) * 9216
    packed, mmq = 7, 1
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 48, 0) == xh(48, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 33, 0) == xh(33, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 32, 0) == xq(32, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 8, 0) == xq(8, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 49, 0) == xq(49, 5120)
    # 64 tiles: the tile GEMM splits K 2 ways (slots and counters after the xq copy)
    assert lib.gguf_op_workspace_bytes(packed, 21, 1024, 5120, 48, 0) == xq(48, 5120) + 64 * 2 * 3072 + 256
    assert lib.gguf_op_workspace_bytes(packed, 21, 6144, 5120, 48, 0) == xq(48, 5120)  # 1.5 tiles per CU
    assert lib.gguf_op_workspace_bytes(mmq, 12, 17408, 5120, 32, 0) == xh(32, 5120)
    assert lib.gguf_op_workspace_bytes(mmq, 12, 17408, 5120, 16, 0) == xq(16, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 64, 0) == xh(64, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 255, 0) == xh(255, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 256, 0) == xh(256, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 5120, 17408, 64, 0) == xq(64, 17408) + 320 * 4 * 4096 + 1280
    assert lib.gguf_op_workspace_bytes(mmq, 12, 17408, 5120, 64, 0) == xh(64, 5120)
    assert lib.gguf_op_workspace_bytes(mmq, 23, 17408, 5120, 64, 0) == xq(64, 5120)


def test_workspace_of_the_split_raw_gemm(lib):
    """Q4_K / IQ4_XS / Q6_K on the int8 GEMM with fewer than two (16-row tile, column group)
    workgroups per CU split K over 2 or 4 workgroups where that cuts the rounds of workgroups per
    CU: the workspace adds a 1 KiB slot per column tile, tile and split, then one counter per tile
    and column group (256-B aligned). 256 CUs assumed without a GPU."""
    xq = lambda n, k: -(-n // 16) * (k // 256) * 4608
    a256 = lambda b: -(-b // 256) * 256
    mmq, vec = 1, 0
    # 320 tiles, one column tile, 68 blocks: 4 ways
    assert lib.gguf_op_workspace_bytes(mmq, 23, 5120, 17408, 16, 0) == xq(16, 17408) + 320 * 4 * 1024 + a256(320 * 4)
    # 320 tiles, 2 column tiles, 24 blocks: 2 ways
    assert lib.gguf_op_workspace_bytes(mmq, 14, 5120, 6144, 32, 0) == xq(32, 6144) + 320 * 2 * 2048 + a256(320 * 4)
    # 64 tiles (under half a workgroup per CU): 4 ways; a decode op at 8 rows likewise
    assert lib.gguf_op_workspace_bytes(mmq, 14, 1024, 5120, 16, 0) == xq(16, 5120) + 64 * 4 * 1024 + a256(64 * 4)
    assert lib.gguf_op_workspace_bytes(vec, 14, 1024, 5120, 8, 1) == xq(8, 5120) + 64 * 4 * 1024 + a256(64 * 4)
    # unsplit: K = 512 (2 blocks); 512+ tiles; 256 workgroups (one round either way); 20 blocks
    # at 320 or 384 tiles (under 3 blocks per wave for a 2-way split)
    assert lib.gguf_op_workspace_bytes(mmq, 14, 1024, 512, 16, 0) == xq(16, 512)
    assert lib.gguf_op_workspace_bytes(mmq, 23, 8192, 5120, 16, 0) == xq(16, 5120)
    assert lib.gguf_op_workspace_bytes(vec, 23, 4096, 4096, 8, 0) == xq(8, 4096)
    assert lib.gguf_op_workspace_bytes(mmq, 12, 5120, 5120, 48, 0) == xq(48, 5120)
    assert lib.gguf_op_workspace_bytes(mmq, 23, 6144, 5120, 32, 0) == xq(32, 5120)
    # 3 column tiles keep 4 blocks per wave: 24 blocks do not split 2 ways
    assert lib.gguf_op_workspace_bytes(mmq, 14, 5120, 6144, 48, 0) == xq(48, 6144)


def test_workspace_of_the_split_tile_gemm(lib):
    """Packed IQ3_S on the int8 tile GEMM splits K on 48+ blocks (4 ways from 2 column tiles, 2 at
    one) and 2 ways where the grid fills under half the CUs; same workspace layout as the raw GEMM."""
    xq = lambda n, k: -(-n // 16) * (k // 256) * 4608
    a256 = lambda b: -(-b // 256) * 256
    packed_vec, packed = 6, 7
    assert lib.gguf_op_workspace_bytes(packed, 21, 5120, 17408, 48, 0) == xq(48, 17408) + 320 * 4 * 3072 + a256(320 * 4)
    assert lib.gguf_op_workspace_bytes(packed_vec, 21, 5120, 17408, 8, 0) == xq(8, 17408) + 320 * 2 * 1024 + a256(320 * 4)
    assert lib.gguf_op_workspace_bytes(packed, 21, 1024, 5120, 16, 0) == xq(16, 5120) + 64 * 2 * 1024 + a256(64 * 4)
    # unsplit: 20 blocks on 384 tiles; 1088 tiles
    assert lib.gguf_op_workspace_bytes(packed, 21, 6144, 5120, 16, 0) == xq(16, 5120)
    assert lib.gguf_op_workspace_bytes(packed, 21, 17408, 5120, 16, 0) == xq(16, 5120)


def test_guard_call_does_not_need_a_gpu(lib):
    import torch

    W = torch.zeros(32, 2200, dtype=torch.uint8)
    X = torch.zeros(2, 5120, dtype=torch.bfloat16)
    rc = lib.gguf_check_op(0, _capi.ref(_capi.view(W)), _capi.ref(_capi.view(X)), 21, 32, None)
    assert rc == _capi.GGUF_EINVAL
    assert _capi.error(lib).endswith("W and X must be CUDA tensors")


def test_noalloc_entry_guards_without_a_gpu(lib):
    """The no-allocation entry point states its scratch size and runs the same guards first: host
    views are rejected before any device or scratch lookup."""
    import torch

    assert lib.gguf_scratch_bytes() == 8 << 20
    W = torch.zeros(32, 2200, dtype=torch.uint8)
    X = torch.zeros(2, 5120, dtype=torch.bfloat16)
    Y = torch.empty(2, 32, dtype=torch.bfloat16)
    rc = lib.gguf_mul_mat_noalloc(6, _capi.ref(_capi.view(W)), _capi.ref(_capi.view(X)), 21, 32, None,
                                  Y.data_ptr(), Y.numel() * 2, None)
    assert rc == _capi.GGUF_EINVAL
    assert _capi.error(lib) == "lcpp_mul_mat_vec_iq3_mma_packed: W and X must be CUDA tensors"


def test_alloc_entry_guards_before_allocating(lib):
    """gguf_mul_mat_alloc runs the guards once, before it asks the caller's allocator for anything:
    a rejected call (bad row, then host views) never reaches the allocator."""
    import torch

    asked = []

    @_capi.ALLOC_FN
    def alloc(ctx, what, nbytes):
        asked.append((what, nbytes))
        return None

    W = torch.zeros(32, 2200, dtype=torch.uint8)
    X = torch.zeros(2, 5120, dtype=torch.bfloat16)
    wv, xv = _capi.view(W), _capi.view(X)
    rc = lib.gguf_mul_mat_alloc(6, _capi.ref(wv), _capi.ref(xv), 21, 24, None, alloc, None, None)
    assert rc == _capi.GGUF_EINVAL
    assert "must be a multiple of 16" in _capi.error(lib)
    rc = lib.gguf_mul_mat_alloc(6, _capi.ref(wv), _capi.ref(xv), 21, 32, None, alloc, None, None)
    assert rc == _capi.GGUF_EINVAL
    assert _capi.error(lib) == "lcpp_mul_mat_vec_iq3_mma_packed: W and X must be CUDA tensors"
    assert asked == []
