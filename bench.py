#!/usr/bin/env python3
"""Benchmark of the GGUF quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-points] [--no-cpu] [--kernel-only]

Workload: IQ3_S decode GEMV at M = 1 and 4 on the two 27B-layer
shapes, gate/up 17408 x 5120 and down 5120 x 17408, bf16 activations N(0,1) quantised to q8_1,
weights in IQ3_S super-blocks with uniform random codes and d ~ |N(0, 2e-3)|, in the build's
packed tile layout (the route the linear method takes for IQ3_S). A step is one op call
(quantise + GEMV, torch.ops._C_gguf.lcpp_mul_mat_vec_iq3_mma_packed) per (shape, M) on each of
8 distinct weight copies per shape (>= 306 MB per shape, beyond the 256 MB Infinity Cache), all
captured in CUDA graphs; K steps are timed with HIP events on torch's current stream between a
synchronize on each side. `value` is the whole-job algorithmic throughput (weights + X + Y bytes
per call) in GB/s.

Also reported: the dominant kernel's roofline (the packed decode GEMV kernel at 17408 x 5120,
M = 1, timed alone with the q8_1 input precomputed), the metric's other points (IQ3_S and Q4_K at
M = 1, 4, 16, 32, 48 on 17408 x 5120, each through the routing table's op), and the CPU oracle
(numpy dequantise + torch fp32 matmul) timed on the host cores on a bounded sample.

`traffic` (HBM bytes per launch of the dominant kernel) is read from the committed PMC summary
profiles/gemv_iq3s_tile_17408x5120_m1.traffic.json when present (null otherwise). That summary
comes from `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` runs of `bench.py --kernel-only`,
which times only the dominant kernel and then runs a plain elementwise copy of 256 MiB (read
256 MiB, write 256 MiB) whose counter readings calibrate the counters' byte scale.
"""

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vllm-gsqrco-exl3_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
NBUF = 8                       # distinct weight copies per shape (defeats the 256 MB MALL)
COPY_BYTES = 256 << 20         # calibration copy: bytes read (and written) per launch
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_iq3s_tile_17408x5120_m1.traffic.json")
IQ3_S, Q4_K = 21, 12
BLOCK = {IQ3_S: 110, Q4_K: 144}
SCALE_OFFSETS = {IQ3_S: (0,), Q4_K: (0, 2)}


def make_weights(torch, qt, rows, k, seed):
    """Uniform random code bytes, every fp16 block scale |N(0, 2e-3)|."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    nb = rows * k // 256
    w = torch.randint(0, 256, (nb, BLOCK[qt]), dtype=torch.uint8, device="cuda", generator=g)
    for off in SCALE_OFFSETS[qt]:
        s = (torch.randn(nb, device="cuda", generator=g) * 2e-3).abs().half()
        w[:, off:off + 2] = s.view(torch.uint8).view(nb, 2)
    return w.view(rows, -1)


def graph(torch, calls):
    """One CUDA graph replaying `calls` (zero-arg launchers) back to back."""
    for c in calls[:2]:
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    g.replay()
    torch.cuda.synchronize()
    return g


def time_graphs(torch, graphs, reps):
    """Milliseconds per replay of the graph list, HIP events on the current stream."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        for g in graphs:
            g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def cpu_baseline(torch):
    """The oracle's CPU path (numpy dequantise, q8_1 round trip of X, torch fp32 matmul) on the
    host cores: IQ3_S 17408 x 5120 at M = 1 (config 2's gate shape); median of 3 runs."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import gguf_oracle as o

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    rows, k = 17408, 5120
    raw = o.random_blocks(np.random.default_rng(0), o.IQ3_S, rows, k)
    x = np.random.default_rng(1).standard_normal((1, k)).astype(np.float32)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        W = torch.from_numpy(o.dequantize(raw.reshape(-1), o.IQ3_S).reshape(rows, k))
        q, d, _ = o.dequant_q8_1(o.quantize_q8_1(x), 1, k)
        xq = torch.from_numpy((q.astype(np.float32).reshape(1, -1, 32) * d[..., None]).reshape(1, k))
        (xq @ W.T).sum().item()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(raw.nbytes / t / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"IQ3_S 17408x5120 M=1 (config 2 gate), numpy dequant + q8_1 + torch fp32 matmul, "
                      f"median of 3: {t * 1e6:.0f} us/call"}


def load_traffic():
    """HBM bytes per launch of the dominant kernel from the committed PMC summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def dominant_kernel(torch, C, ws, steps):
    """The packed decode GEMV kernel alone (17408 x 5120, M = 1, q8_1 input precomputed): one graph
    of one launch per weight copy, timed with HIP events on the stream the op launches on."""
    rows, k, m = 17408, 5120, 1
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    q8 = C.lcpp_quantize_q8_1(x, IQ3_S, False, False)
    kg = graph(torch, [lambda w=w: C.lcpp_mul_mat_vec_iq3_mma_packed(w, x, IQ3_S, rows, q8) for w in ws])
    kernel_us = time_graphs(torch, [kg], max(5, steps)) * 1e3 / len(ws)
    alg_bytes = ws[0].numel() + q8.numel() + m * rows * 2
    achieved = alg_bytes / (kernel_us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic(),
            "kernel": "gemv_iq3s_tile_kernel<1,1,8> (17408x5120, M=1, q8_1 precomputed)",
            "us_per_launch": round(kernel_us, 3), "alg_bytes_per_launch": alg_bytes}


def copy_calibration(torch):
    """A plain elementwise map over COPY_BYTES (torch.neg, float32 in, float32 out: COPY_BYTES read,
    COPY_BYTES written), three launches, so that a PMC run can read what FETCH_SIZE / WRITE_SIZE
    report for a known byte count."""
    src = torch.randn(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def kernel_only(torch, C, iq3_pack, steps):
    """--kernel-only: the dominant kernel (as in the full run) and the calibration copy; prints one
    JSON line with the roofline object."""
    ws = [iq3_pack.pack(make_weights(torch, IQ3_S, 17408, 5120, i), IQ3_S) for i in range(NBUF)]
    roofline = dominant_kernel(torch, C, ws, steps)
    del ws
    torch.cuda.empty_cache()
    copy_calibration(torch)
    print(json.dumps({"mode": "kernel-only", "roofline": roofline, "copy_bytes": COPY_BYTES}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-points", action="store_true", help="skip the metric's other (type, M) points")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--kernel-only", action="store_true",
                    help="time only the dominant kernel, then run the counter-calibration copy (for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the path "
              "would shard along the weight rows, one slice of rows per GPU", file=sys.stderr)
        sys.exit(2)

    import torch

    from vllm_gguf_plugin import ops  # noqa: F401  registers torch.ops._C_gguf
    from vllm_gguf_plugin.quantization import iq3_pack, linear

    C = torch.ops._C_gguf
    torch.cuda.set_device(0)
    if args.kernel_only:
        kernel_only(torch, C, iq3_pack, args.steps)
        return

    # ------------------------------------------------------------------ headline workload
    cases = [(17408, 5120, 1), (17408, 5120, 4), (5120, 17408, 1), (5120, 17408, 4)]
    shapes = sorted({(r, k) for r, k, _ in cases})
    weights = {}
    for si, (rows, k) in enumerate(shapes):
        weights[(rows, k)] = [iq3_pack.pack(make_weights(torch, IQ3_S, rows, k, 100 * si + i), IQ3_S)
                              for i in range(NBUF)]
    step_graphs, per_case, step_bytes = [], [], 0
    for rows, k, m in cases:
        x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        ws = weights[(rows, k)]
        calls = [lambda w=w, x=x, rows=rows: C.lcpp_mul_mat_vec_iq3_mma_packed(w, x, IQ3_S, rows) for w in ws]
        g = graph(torch, calls)
        step_graphs.append(g)
        call_bytes = ws[0].numel() + m * k * 2 + m * rows * 2
        step_bytes += call_bytes * len(calls)
        per_case.append((rows, k, m, g, call_bytes, len(calls), x))

    for _ in range(args.warmup):
        for g in step_graphs:
            g.replay()
    torch.cuda.synchronize()
    ms_per_step = time_graphs(torch, step_graphs, args.steps)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    detail = []
    for rows, k, m, g, cb, ncalls, x in per_case:
        us = time_graphs(torch, [g], max(3, args.steps)) * 1e3 / ncalls
        detail.append({"shape": f"{rows}x{k}", "m": m, "us_per_call": round(us, 2),
                       "gbps": round(cb / (us * 1e-6) / 1e9, 1), "frac_hbm": round(cb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3)})

    roofline = dominant_kernel(torch, C, weights[(17408, 5120)], args.steps)
    del weights
    torch.cuda.empty_cache()

    # ------------------------------------------------------------------ the metric's other points
    points = []
    if not args.no_points:
        rows, k = 17408, 5120
        for qt, name in ((IQ3_S, "IQ3_S"), (Q4_K, "Q4_K")):
            ws = [make_weights(torch, qt, rows, k, 1000 + i) for i in range(NBUF)]
            packed = qt == IQ3_S
            if packed:
                ws = [iq3_pack.pack(w, qt) for w in ws]
            for m in (1, 4, 16, 32, 48):
                op = linear._lcpp_op(m, qt, rows, k, packed)
                fn = getattr(C, op)
                x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
                g = graph(torch, [lambda w=w, x=x, fn=fn: fn(w, x, qt, rows) for w in ws])
                us = time_graphs(torch, [g], 5) * 1e3 / len(ws)
                cb = ws[0].numel() + m * k * 2 + m * rows * 2
                points.append({"type": name, "shape": f"{rows}x{k}", "m": m, "op": op, "us_per_call": round(us, 2),
                               "gbps": round(cb / (us * 1e-6) / 1e9, 1),
                               "frac_hbm": round(cb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3),
                               "weight_us_per_MB": round(us / (ws[0].numel() / 1e6), 4)})
            del ws
            torch.cuda.empty_cache()

    cpu = None if args.no_cpu else cpu_baseline(torch)

    line = {
        "metric": "µs/call + achieved HBM GB/s (% of peak), IQ3_S/Q4_K matmul at M=1,4,16,32,48",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (uniform random IQ3_S codes, d ~ |N(0,2e-3)|; X bf16 N(0,1))",
        "config": {"workload": "IQ3_S decode GEMV (packed tile layout) at M=1,4 on 17408x5120 and 5120x17408, "
                               "BASELINE configs[1]; 8 weight copies per shape per step",
                   "calls_per_step": sum(n for *_, n, _ in per_case), "bytes_per_step": step_bytes},
        "detail": detail,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "points": points,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
