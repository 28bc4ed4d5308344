"""The ops' input guards, driven by the case table tests/golden/guard_cases.json (the reference's
guard cases and messages, cited in the file).

Each case builds its W and X views (shape, row stride, byte offset from a 16-byte aligned base,
dtype, transposed or flat) and is checked two ways that must agree:
  * through the registered torch op (torch.ops._C_gguf.<op>) on host tensors: every op has a CPU
    registration whose only work is the library's guards, so a call either names the first guard
    that fails or ends with "must be CUDA tensors" once every layout guard has passed;
  * through the C ABI alone (gguf_check_op with the same views, or the quantiser's entry point),
    which must report the same message: the torch layer adds no guard of its own.
The GPU variant (marked gpu) runs the same table on device tensors: bad layouts must be rejected
with the same message before any launch, and valid ones must run and return zeros (all-zero
weights and activations); it adds the device checks (host X beside a device W, an x_q8 that is
not on X's device, too short or misaligned).
"""

import ctypes
import json
import os
import subprocess
import sys

import pytest
import torch
from conftest import GOLDEN, PKG_ROOT

PASSED_LAYOUT = "must be CUDA tensors"
with open(os.path.join(GOLDEN, "guard_cases.json")) as _f:
    TABLE = json.load(_f)["cases"]
BY_ID = {c["id"]: c for c in TABLE}


def _aligned_bytes(nbytes, device):
    """A uint8 buffer whose first byte is 16-byte aligned, with room for nbytes."""
    raw = torch.zeros(nbytes + 32, dtype=torch.uint8, device=device)
    skip = (-raw.data_ptr()) % 16
    return raw[skip:skip + nbytes]


def build_w(spec, device="cpu"):
    dtype = getattr(torch, spec.get("dtype", "uint8"))
    es = torch.empty(0, dtype=dtype).element_size()
    rows, rb = spec["rows"], spec["row_bytes"]
    stride = spec.get("row_stride", rb)
    off = spec.get("byte_offset", 0)
    assert off % es == 0
    flat = _aligned_bytes((rows * stride + 64) * es + off, device)[off:]
    w = flat[:rows * stride * es].view(dtype).as_strided((rows, rb), (stride, 1))
    view = spec.get("view", "2d")
    if view == "transposed":
        w = w.t()
    elif view == "flat":
        w = w.reshape(-1)
    return w


def build_x(spec, device="cpu"):
    dtype = getattr(torch, spec.get("dtype", "bfloat16"))
    n, k = spec["n"], spec["k"]
    if spec.get("view") == "transposed":
        return torch.zeros(k, n, dtype=dtype, device=device).t()
    return torch.zeros(n, k, dtype=dtype, device=device)


def _first_line(e):
    return str(e).splitlines()[0]


def run_op(case, device="cpu"):
    """The op's result on views built for `case`: ("ok", output) or ("error", message)."""
    from vllm_gguf_plugin import ops  # noqa: F401

    C = torch.ops._C_gguf
    w, x = build_w(case["w"], device), build_x(case["x"], device)
    try:
        if case["op"] == "lcpp_quantize_q8_1":
            return "ok", C.lcpp_quantize_q8_1(x, case["type"], False, False)
        return "ok", getattr(C, case["op"])(w, x, case["type"], case["row"])
    except RuntimeError as e:
        return "error", _first_line(e)


def abi_message(case):
    """The C ABI's verdict on the same host views (gguf_check_op, or the quantiser's entry)."""
    from vllm_gguf_plugin import _capi

    lib = _capi.load()
    w, x = build_w(case["w"]), build_x(case["x"])
    xv = _capi.view(x)
    if case["op"] == "lcpp_quantize_q8_1":
        rc = lib.gguf_lcpp_quantize_q8_1(ctypes.byref(xv), case["type"], 0, 0, None, 0, None)
    else:
        wv = _capi.view(w)
        rc = lib.gguf_check_op(_capi.OPS[case["op"]], ctypes.byref(wv), ctypes.byref(xv), case["type"],
                               case["row"], None)
    assert rc != 0, "host views never pass every guard"
    return _capi.error(lib)


@pytest.mark.parametrize("cid", list(BY_ID))
def test_guard_case(cid):
    case = BY_ID[cid]
    kind, msg = run_op(case)
    assert kind == "error", "a host call must be rejected"
    assert case["expect"] in msg, msg
    assert msg.startswith(case["op"]), msg
    assert abi_message(case) == msg


def test_table_covers_every_op_and_outcome():
    ops = {c["op"] for c in TABLE}
    assert ops == {"lcpp_mul_mat_vec_q", "lcpp_mul_mat_q", "lcpp_mul_mat_vec_iq3", "lcpp_mul_mat_vec_iq3_mma",
                   "lcpp_mul_mat_vec_iq3_mma_packed", "lcpp_mul_mat_iq3_packed", "lcpp_mul_mat_vec_own",
                   "lcpp_mul_mat_mma_k", "lcpp_quantize_q8_1"}
    for op in ops - {"lcpp_quantize_q8_1"}:
        outcomes = {c["expect"] for c in TABLE if c["op"] == op}
        assert PASSED_LAYOUT in outcomes and len(outcomes) >= 5, (op, outcomes)


_NO_GPU_INIT = """
import sys, torch
sys.path.insert(0, sys.argv[1])
from vllm_gguf_plugin import ops
C = torch.ops._C_gguf
w = torch.zeros(16, 220, dtype=torch.uint8)
x = torch.zeros(2, 512, dtype=torch.bfloat16)
for op in ("lcpp_mul_mat_vec_q", "lcpp_mul_mat_q", "lcpp_mul_mat_vec_iq3", "lcpp_mul_mat_vec_iq3_mma",
           "lcpp_mul_mat_vec_iq3_mma_packed", "lcpp_mul_mat_iq3_packed"):
    try:
        getattr(C, op)(w, x, 21, 16)
    except RuntimeError:
        pass
print("initialised" if torch.cuda.is_initialized() else "not initialised")
"""


def test_registration_and_host_guards_do_not_touch_the_gpu():
    """Importing the plugin registers the ops, and host calls run the guards, without
    initialising the GPU runtime (checked in a child with the GPU hidden)."""
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="", ROCR_VISIBLE_DEVICES="")
    p = subprocess.run([sys.executable, "-c", _NO_GPU_INIT, PKG_ROOT], capture_output=True, text=True,
                       timeout=300, env=env)
    assert p.returncode == 0, p.stderr[-2000:]
    assert p.stdout.strip().splitlines()[-1] == "not initialised"


# ------------------------------------------------------------------------------------ device tensors
@pytest.mark.gpu
def test_guard_table_on_device_tensors():
    """Every case again with W and X on the GPU: a layout the host call rejects before the device
    check is rejected with the same message; one that passed every layout guard now runs (or is
    rejected for its type, as on the host) and returns zeros of the right shape and dtype."""
    assert torch.cuda.is_available()
    for case in TABLE:
        kind, host_msg = run_op(case)
        kind_d, got = run_op(case, "cuda")
        if host_msg.endswith(PASSED_LAYOUT) or "bad arguments" in host_msg:
            if case["op"] == "lcpp_quantize_q8_1":
                assert kind_d == "ok", got
                continue
            assert kind_d == "ok", (case["id"], got)
            n = case["x"]["n"]
            assert got.shape == (n, case["row"]) and got.dtype == getattr(torch, case["x"].get("dtype", "bfloat16"))
            assert not got.any(), case["id"]
        else:
            assert kind_d == "error" and got == host_msg, (case["id"], got, host_msg)
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_device_placement_guards():
    from vllm_gguf_plugin import ops  # noqa: F401

    C = torch.ops._C_gguf
    w = torch.zeros(64, 220, dtype=torch.uint8, device="cuda")
    x = torch.zeros(2, 512, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="W and X must be CUDA tensors"):
        C.lcpp_mul_mat_vec_q(w, x.cpu(), 21, 64)
    with pytest.raises(RuntimeError, match="W and X must be CUDA tensors"):
        C.lcpp_mul_mat_q(w.cpu(), x, 21, 64)
    q8 = C.lcpp_quantize_q8_1(x, 21, False, False)
    assert q8.numel() == 2 * 512 // 32 * 36 and q8.is_cuda
    with pytest.raises(RuntimeError, match="x_q8 must be on X's device"):
        C.lcpp_mul_mat_vec_iq3(w, x, 21, 64, q8.cpu())
    with pytest.raises(RuntimeError, match="at least 576 bytes"):  # one row: 16 blocks of 36 bytes
        C.lcpp_mul_mat_vec_iq3(w, x[:1], 21, 64, q8[:575])
    with pytest.raises(RuntimeError, match="x_q8 must be 16-byte aligned"):
        C.lcpp_mul_mat_vec_iq3(w, x, 21, 64, torch.cat([q8, q8])[4:4 + q8.numel()])
    y = C.lcpp_mul_mat_vec_iq3(w, x, 21, 64, q8)
    assert y.shape == (2, 64) and not y.any()
    torch.cuda.synchronize()
