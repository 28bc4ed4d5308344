"""Builds libgguf_mi355x.so (the C-ABI library of include/gguf_mi355x.h) for gfx950 with hipcc,
and the torch op registration over it.

    python vllm-gsqrco-exl3_amd/build.py [--jobs N]

Each csrc/*.hip is compiled to an object in _build/ (in parallel), then linked into
vllm_gguf_plugin/libgguf_mi355x.so, in-tree, where vllm_gguf_plugin._capi loads it.
csrc/torch_ops.cpp (host C++ against PyTorch-ROCm's headers) is compiled alongside into
vllm_gguf_plugin/_C_gguf_ops.so, which links libgguf_mi355x.so next to it and registers
torch.ops._C_gguf when vllm_gguf_plugin._C_gguf loads it. csrc/bench/peaks.hip (bench.py's
measurement kernels, outside the C ABI) is built into vllm_gguf_plugin/libgguf_peaks.so.
"""

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "vllm_gguf_plugin", "libgguf_mi355x.so")
OPS_OUT = os.path.join(HERE, "vllm_gguf_plugin", "_C_gguf_ops.so")
# bench.py's measurement kernels (streaming-read floor, MFMA peak): not part of the C ABI
PEAKS_SRC = os.path.join(CSRC, "bench", "peaks.hip")
PEAKS_OUT = os.path.join(HERE, "vllm_gguf_plugin", "libgguf_peaks.so")
CXX = os.environ.get("CXX", "g++")
ARCH = os.environ.get("GGUF_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no packed fp32 instructions in device code (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature: not an error
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (p.stderr or "").splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def _torch_flags():
    """Include / library directories and ABI flag of the installed PyTorch (ROCm build)."""
    import torch

    tdir = os.path.dirname(torch.__file__)
    inc = [os.path.join(tdir, "include"), os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
           "/opt/rocm/include"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, os.path.join(tdir, "lib"), abi


def _compile_ops():
    """csrc/torch_ops.cpp -> _build/torch_ops.o (host C++ only)."""
    inc, _, abi = _torch_flags()
    obj = os.path.join(BUILD, "torch_ops.o")
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-c", os.path.join(CSRC, "torch_ops.cpp"), "-o", obj,
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-Wall", "-Wno-unused-function", *[f"-I{d}" for d in inc]]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"{CXX} failed on torch_ops.cpp:\n{p.stderr}")
    return obj, p.stderr


def _link_ops(obj):
    _, libdir, _ = _torch_flags()
    tmp = OPS_OUT + ".tmp"
    cmd = [CXX, "-shared", "-fPIC", "-o", tmp, obj, f"-L{os.path.dirname(OUT)}", "-lgguf_mi355x",
           f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link of _C_gguf_ops.so failed:\n{p.stderr}")
    os.replace(tmp, OPS_OUT)


def _build_peaks():
    """csrc/bench/peaks.hip -> libgguf_peaks.so (one step: compile and link)."""
    tmp = PEAKS_OUT + ".tmp"
    cmd = [HIPCC, *FLAGS, "-shared", PEAKS_SRC, "-o", tmp]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed on {PEAKS_SRC}:\n{p.stderr}")
    os.replace(tmp, PEAKS_OUT)


def build(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs) + 2))) as ex:
        ops = ex.submit(_compile_ops)
        peaks = ex.submit(_build_peaks)
        results = list(ex.map(_compile, srcs))
        ops_obj, ops_err = ops.result()
        peaks.result()
    for _, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr}")
    os.replace(tmp, OUT)
    if ops_err.strip() and verbose:
        print(ops_err, file=sys.stderr)
    _link_ops(ops_obj)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
