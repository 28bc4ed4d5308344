#!/usr/bin/env python3
"""Benchmark of the GGUF quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-points] [--no-configs] [--no-cpu]
                    [--kernel-only | --section {mtp,prefill,layers}]

Workload: IQ3_S decode GEMV at M = 1 and 4 on the two 27B-layer
shapes, gate/up 17408 x 5120 and down 5120 x 17408, bf16 activations N(0,1) quantised to q8_1,
weights in IQ3_S super-blocks with uniform random codes and d ~ |N(0, 2e-3)|, in the build's
packed unit layout (the route the linear method takes for IQ3_S). A step is one op call
(quantise + GEMV, torch.ops._C_gguf.lcpp_mul_mat_vec_iq3_mma_packed) per (shape, M) on each of
8 distinct weight copies per shape (>= 306 MB per shape, beyond the 256 MB Infinity Cache), all
captured in CUDA graphs; K steps are timed with HIP events on torch's current stream between a
synchronize on each side. `value` is the whole-job algorithmic throughput (weights + X + Y bytes
per call) in GB/s.

Also reported: the dominant kernel's roofline (the packed decode GEMV kernel at 17408 x 5120,
M = 1, which quantises X itself, timed alone, with the per-launch floor of as many graph-replayed
launches of a 512 KB fill beside it), the metric's other points (IQ3_S and Q4_K at
M = 1, 4, 16, 32, 48 on 17408 x 5120, each through the routing table's op), and the CPU oracle
(numpy dequantise + torch fp32 matmul) timed on the host cores on a bounded sample; and the other
benchmark configs under "configs": the CPU-path Q4_K 4096x4096 case next to its GPU op, the MTP
small GEMM (IQ3_S / IQ4_XS / Q6_K at M = 4..48 on the attention shapes), the prefill GEMM
(M = 512..8192, with MFMA utilisation), the six types served by the generic kernels at the gate/up
shape, and the 64-layer decoder sweep under one CUDA graph with a replay bit-exactness check.
Under "eager": the headline op called eagerly (no graph) at M = 1 and a 512-row prefill chunk, with
the host's time per call.

Also measured on the GPU (--no-peaks skips them): the read floor, one streaming launch over a
headline weight's bytes (38.3 MB) and a gate|up pair's (76.6 MB) with the decode GEMV's access
pattern, and the dense MFMA rate (v_mfma_i32_16x16x64_i8, v_mfma_f32_16x16x32_f16), so that the
roofline carries a measured peak beside the published one.

Output: each detail section on a line of its own ({"bench_detail": name, "result": ...}), then
the headline, a compact JSON object, as the last line of stdout.

`traffic` (HBM bytes per launch of the dominant kernel) is read from the committed PMC summary
profiles/gemv_iq3s_stream_17408x5120_m1.traffic.json when present (null otherwise). That summary
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
NBUF = 8                       # the fewest distinct weight copies a timed graph rotates through
ROTATE_BYTES = 512 << 20       # ... and at least this many weight bytes: twice the 256 MB MALL,
                               # so that no copy is still cached when its turn comes again
COPY_BYTES = 256 << 20         # calibration copy: bytes read (and written) per launch
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_iq3s_stream_17408x5120_m1.traffic.json")
IQ3_S, Q4_K, Q6_K, IQ4_XS = 21, 12, 14, 23
Q2_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ2_S, IQ1_M = 10, 16, 17, 18, 22, 29
TYPE_NAME = {IQ3_S: "IQ3_S", Q4_K: "Q4_K", Q6_K: "Q6_K", IQ4_XS: "IQ4_XS", Q2_K: "Q2_K", IQ2_XXS: "IQ2_XXS",
             IQ2_XS: "IQ2_XS", IQ3_XXS: "IQ3_XXS", IQ2_S: "IQ2_S", IQ1_M: "IQ1_M"}
BLOCK = {IQ3_S: 110, Q4_K: 144, Q6_K: 210, IQ4_XS: 136, Q2_K: 84, IQ2_XXS: 66, IQ2_XS: 74, IQ3_XXS: 98,
         IQ2_S: 82, IQ1_M: 56}
SCALE_OFFSETS = {IQ3_S: (0,), Q4_K: (0, 2), Q6_K: (208,), IQ4_XS: (0,), Q2_K: (80, 82), IQ2_XXS: (0,),
                 IQ2_XS: (0,), IQ3_XXS: (0,), IQ2_S: (0,), IQ1_M: ()}
PACKED_TYPES = (IQ3_S, IQ3_XXS)  # the types the linear method's repack hook stores packed
MFMA_I8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


def rotation_copies(weight_bytes):
    """Weight copies for a timed graph: NBUF, or more where NBUF copies fit twice in the MALL."""
    return max(NBUF, -(-ROTATE_BYTES // weight_bytes))


def make_weights(torch, qt, rows, k, seed):
    """Uniform random code bytes, every fp16 block scale |N(0, 2e-3)| (benchmark configs)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    nb = rows * k // 256
    w = torch.randint(0, 256, (nb, BLOCK[qt]), dtype=torch.uint8, device="cuda", generator=g)
    for off in SCALE_OFFSETS[qt]:
        s = (torch.randn(nb, device="cuda", generator=g) * 2e-3).abs().half()
        w[:, off:off + 2] = s.view(torch.uint8).view(nb, 2)
    if qt == IQ1_M:  # fp16 d in the top nibbles of the four scale words (bytes 49, 51, 53, 55)
        bits = (torch.randn(nb, device="cuda", generator=g) * 2e-3).abs().half().view(torch.int16).int() & 0xFFFF
        for j in range(4):
            hi = ((bits >> (4 * j)) & 0xF).to(torch.uint8) << 4
            w[:, 49 + 2 * j] = (w[:, 49 + 2 * j] & 0x0F) | hi
    return w.view(rows, -1)


def graph(torch, calls, outputs=None):
    """One CUDA graph replaying `calls` (zero-arg launchers) back to back. `outputs`, a list, receives
    the tensors the captured calls return: they live in the graph's pool and every replay rewrites
    them in place."""
    for c in calls[:2]:
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            r = c()
            if outputs is not None:
                outputs.append(r)
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


def x_outliers(torch, m, k, seed):
    """BASELINE configs[3]'s activations: bf16 N(0,1) with a seeded 1 % of the entries set to +-20
    (the same recipe as the tests' x_bench), drawn on the device."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g)
    mask = torch.rand(m, k, device="cuda", generator=g) < 0.01
    x = torch.where(mask, 20.0 * torch.sign(torch.randn(m, k, device="cuda", generator=g)), x)
    return x.to(torch.bfloat16)


def op_points(torch, C, iq3_pack, linear, qt, rows, k, ms, ncopies=None, reps=5, seed=0, outliers=False):
    """us/call of the routing table's op for a qt weight [rows, k] at each M in ms (bf16 X N(0,1),
    with outliers: x_outliers), over ncopies weight copies (default: rotation_copies) captured in
    one graph per M. IQ3_S and IQ3_XXS in their packed unit layouts."""
    if ncopies is None:
        ncopies = rotation_copies(rows * (k // 256) * BLOCK[qt])
    ws = [make_weights(torch, qt, rows, k, seed + i) for i in range(ncopies)]
    packed = qt in PACKED_TYPES
    if packed:
        ws = [iq3_pack.pack(w, qt) for w in ws]
    out = []
    for m in ms:
        op = linear._lcpp_op(m, qt, rows, k, packed)
        fn = getattr(C, op)
        x = x_outliers(torch, m, k, seed + m) if outliers else torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        g = graph(torch, [lambda w=w, x=x, fn=fn: fn(w, x, qt, rows) for w in ws])
        us = time_graphs(torch, [g], reps) * 1e3 / len(ws)
        wb = ws[0].numel()
        cb = wb + m * k * 2 + m * rows * 2
        out.append({"type": TYPE_NAME[qt], "shape": f"{rows}x{k}", "m": m, "op": op, "us_per_call": round(us, 2),
                    "gbps": round(cb / (us * 1e-6) / 1e9, 1), "frac_hbm": round(cb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3),
                    "weight_us_per_MB": round(us / (wb / 1e6), 4),
                    "int8_tops": round(2.0 * m * rows * k / (us * 1e-6) / 1e12, 2)})
        del g
    del ws
    torch.cuda.empty_cache()
    return out


def config_mtp(torch, C, iq3_pack, linear):
    """benchmark configs[2]: MTP verify small GEMM at M = 4, 8, 16, 32, 48 on q_proj 6144x5120,
    k/v_proj 1024x5120 and o_proj 5120x6144 for IQ3_S (packed), IQ4_XS and Q6_K."""
    out = []
    for qt in (IQ3_S, IQ4_XS, Q6_K):
        for rows, k in ((6144, 5120), (1024, 5120), (5120, 6144)):
            out += op_points(torch, C, iq3_pack, linear, qt, rows, k, (4, 8, 16, 32, 48), seed=2000)
    return out


def config_prefill(torch, C, iq3_pack, linear):
    """benchmark configs[3]: prefill GEMM at M = 512, 2048, 8192 over K = 5120, N = 17408 and 5120,
    IQ3_S (packed), Q4_K, Q6_K; int8 TOP/s against the dense int8 MFMA peak; X bf16 N(0,1) with 1 %
    outliers of magnitude 20 (the config's recipe)."""
    out = []
    for qt in (IQ3_S, Q4_K, Q6_K):
        for rows in (17408, 5120):
            pts = op_points(torch, C, iq3_pack, linear, qt, rows, 5120, (512, 2048, 8192), ncopies=2, reps=2,
                            seed=3000, outliers=True)
            for p in pts:
                # IQ3_S and Q4_K run on fp16 MFMAs (exact sub-scaled integer operands), Q6_K on int8
                p["mfma"] = "f16" if qt in (IQ3_S, Q4_K) else "i8"
                p["frac_mfma_i8"] = round(p["int8_tops"] / MFMA_I8_PEAK_TOPS, 4)
                p["frac_mfma_f16"] = round(p["int8_tops"] / MFMA_F16_PEAK_TFLOPS, 4)
            out += pts
    return out


def config_types(torch, C, iq3_pack, linear):
    """The types served by the generic kernels (Q2_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS packed as the
    repack hook stores it, IQ1_M) at the gate/up shape 17408 x 5120, M = 1, 4 (decode ops) and 16, 48
    (product ops; IQ1_M's 8-row MMVQ calls), each through the routing table's op."""
    out = []
    for qt in (Q2_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ1_M):
        out += op_points(torch, C, iq3_pack, linear, qt, 17408, 5120, (1, 4) if qt == IQ1_M else (1, 4, 16, 48),
                         seed=4000)
    return out


def config_decode(torch, C, iq3_pack, linear):
    """The decode ops of every type with a dedicated decode GEMV at M = 1..4 on the FFN shapes
    17408 x 5120 and 5120 x 17408: IQ3_S (packed: the stream GEMV), Q4_K, IQ4_XS and Q6_K (the
    row-chunk GEMV at one row, the 4 x 4 x 4 MFMA GEMV at 2-4 rows), through the routing table's
    op."""
    out = []
    for qt in (IQ3_S, Q4_K, IQ4_XS, Q6_K):
        for rows, k in ((17408, 5120), (5120, 17408)):
            out += op_points(torch, C, iq3_pack, linear, qt, rows, k, (1, 2, 3, 4), seed=5000)
    return out


def config_layers(torch, C, iq3_pack, linear, steps, ms=(1, 4, 16, 32), nlayers=64, merged=False):
    """benchmark configs[4]: a 64-layer synthetic 27B-style decoder's linear layers (hidden 5120,
    intermediate 17408, 48 query / 8 KV heads of dim 128) in the GSQ-RCO mix -- IQ3_S (packed)
    q/k/v/o/gate/up, IQ4_XS down -- plus the Q6_K output head 151936x5120, every call of a step
    captured in one CUDA graph. Per M: ms/step, weight GB streamed per step, and whether two
    replays give bit-identical outputs. merged: one product per same-type run of a fused layer,
    as the reference's glue issues them (linear.py:166-218: the q/k/v shards as one 8192-row
    weight, gate/up as one 34816-row weight; the same bytes in 4 calls per layer instead of 7)."""
    if merged:
        shapes = [("qkv", IQ3_S, 8192, 5120), ("o", IQ3_S, 5120, 6144), ("gate_up", IQ3_S, 34816, 5120),
                  ("down", IQ4_XS, 5120, 17408)]
    else:
        shapes = [("q", IQ3_S, 6144, 5120), ("k", IQ3_S, 1024, 5120), ("v", IQ3_S, 1024, 5120),
                  ("o", IQ3_S, 5120, 6144), ("gate", IQ3_S, 17408, 5120), ("up", IQ3_S, 17408, 5120),
                  ("down", IQ4_XS, 5120, 17408)]
    layers = []
    for li in range(nlayers):
        lw = []
        for name, qt, rows, k in shapes:
            w = make_weights(torch, qt, rows, k, 10000 + 16 * li + len(lw))
            lw.append((qt, rows, k, iq3_pack.pack(w, qt) if qt == IQ3_S else w))
        layers.append(lw)
    head = (Q6_K, 151936, 5120, make_weights(torch, Q6_K, 151936, 5120, 99999))
    calls = [c for lw in layers for c in lw] + [head]
    weight_bytes = sum(w.numel() for *_, w in calls)
    out = []
    for m in ms:
        xs = {k: torch.randn(m, k, device="cuda", dtype=torch.bfloat16) for k in (5120, 6144, 17408)}
        ys = []  # the captured calls' outputs (graph-owned, rewritten by every replay)
        fns = []
        for qt, rows, k, w in calls:
            op = getattr(C, linear._lcpp_op(m, qt, rows, k, qt == IQ3_S))
            fns.append(lambda op=op, w=w, x=xs[k], qt=qt, rows=rows: op(w, x, qt, rows))
        g = graph(torch, fns, ys)
        g.replay()
        torch.cuda.synchronize()
        first = [y.clone() for y in ys]
        ms_step = time_graphs(torch, [g], max(3, steps // 4))
        g.replay()
        torch.cuda.synchronize()
        exact = all(torch.equal(a, b) for a, b in zip(first, ys))
        out.append({"m": m, "ms_per_step": round(ms_step, 3), "weight_gb_per_step": round(weight_bytes / 1e9, 3),
                    "weight_gbps": round(weight_bytes / (ms_step * 1e-3) / 1e9, 1), "calls_per_step": len(fns),
                    "replay_bit_exact": bool(exact)})
        del g, first, ys, fns, xs
        torch.cuda.empty_cache()
    del layers, calls, head
    torch.cuda.empty_cache()
    return out


def _cpu_model():
    """The host CPU's model name (lscpu's 'Model name', from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_s(fn, runs=5):
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def _cpu_path_times(torch, o, raw, qt, rows, k, ms, threads):
    """The CPU reference path on GGUF rows raw [rows, ...]: numpy dequantise (median of 5), then
    per M and thread count the q8_1 round trip of X plus the torch fp32 matmul (median of 5).
    Returns (dequant seconds, {(m, threads): matmul seconds})."""
    import numpy as np

    holder = {}
    t_deq = _median_s(lambda: holder.__setitem__("W", o.dequantize(raw.reshape(-1), qt).reshape(rows, k)))
    W = torch.from_numpy(holder["W"])
    mm = {}
    for m in ms:
        x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)

        def run():
            q, d, _ = o.dequant_q8_1(o.quantize_q8_1(x), m, k)
            xq = torch.from_numpy((q.astype(np.float32).reshape(m, -1, 32) * d[..., None]).reshape(m, k))
            (xq @ W.T).sum().item()

        for th in threads:
            torch.set_num_threads(th)
            mm[(m, th)] = _median_s(run)
    return t_deq, mm


def config_cpu_q4k(torch, C):
    """benchmark configs[0]: Q4_K 4096x4096 at M = 1, fp32 X N(0,1): the GPU op (the routing
    table's, lcpp_mul_mat_vec_q at one row) next to the CPU
    reference path (numpy dequantise + q8_1 round trip + torch fp32 matmul), seed 0; dequantise and
    matmul each the median of 5, the matmul on all threads and on one."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import gguf_oracle as o

    rows = k = 4096
    raw = o.random_blocks(np.random.default_rng(0), o.Q4_K, rows, k, scale_sigma=1e-3)
    threads = torch.get_num_threads()
    t_deq, mm = _cpu_path_times(torch, o, raw, o.Q4_K, rows, k, (1,), (threads, 1))
    torch.set_num_threads(threads)
    x = np.random.default_rng(0).standard_normal((1, k)).astype(np.float32)
    wd = torch.from_numpy(raw).cuda()
    xd = torch.from_numpy(x).cuda()
    from vllm_gguf_plugin.quantization import linear

    op = linear._lcpp_op(1, Q4_K, rows, k, False)
    fn = getattr(C, op)
    g = graph(torch, [lambda: fn(wd, xd, Q4_K, rows)] * 8)
    us = time_graphs(torch, [g], 10) * 1e3 / 8
    return {"shape": "4096x4096", "m": 1, "op": op, "gpu_us_per_call": round(us, 2),
            "cpu_us_per_call": round((t_deq + mm[(1, threads)]) * 1e6, 1),
            "cpu_us_per_call_1_thread": round((t_deq + mm[(1, 1)]) * 1e6, 1),
            "cpu_dequant_us": round(t_deq * 1e6, 1), "cpu_matmul_us": round(mm[(1, threads)] * 1e6, 1),
            "cpu_matmul_us_1_thread": round(mm[(1, 1)] * 1e6, 1), "cpu_threads": threads,
            "nproc": os.cpu_count() or 1, "cpu_model": _cpu_model()}


CPU_SAMPLE_ROWS = 2048  # rows of each config-2 shape the CPU path dequantises and multiplies


def cpu_baseline(torch):
    """The oracle's CPU path (numpy dequantise, q8_1 round trip of X, torch fp32 matmul) on the
    host cores, on the headline workload (configs[1]: IQ3_S at M = 1 and 4 on 17408 x 5120 and
    5120 x 17408), bounded: CPU_SAMPLE_ROWS weight rows of each shape, each part the median of 5,
    per-call times scaled to the full row count (both parts are linear in the rows). `value`: the
    four calls' weight bytes over their summed CPU time on all threads (torch's thread count; the
    dequantise is numpy, one thread); also on one thread, per case, and dequantise / matmul apart."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import gguf_oracle as o

    threads = torch.get_num_threads()
    cases, tot_bytes, tot_s, tot_s1 = [], 0, 0.0, 0.0
    for rows, k in ((17408, 5120), (5120, 17408)):
        rs = min(rows, CPU_SAMPLE_ROWS)
        raw = o.random_blocks(np.random.default_rng(rows), o.IQ3_S, rs, k)
        t_deq, mm = _cpu_path_times(torch, o, raw, o.IQ3_S, rs, k, (1, 4), (threads, 1))
        scale = rows / rs
        wbytes = rows * (k // 256) * BLOCK[IQ3_S]
        for m in (1, 4):
            t_all = (t_deq + mm[(m, threads)]) * scale
            t_one = (t_deq + mm[(m, 1)]) * scale
            tot_bytes += wbytes
            tot_s += t_all
            tot_s1 += t_one
            cases.append({"shape": f"{rows}x{k}", "m": m, "us_per_call": round(t_all * 1e6, 1),
                          "us_per_call_1_thread": round(t_one * 1e6, 1),
                          "dequant_us": round(t_deq * scale * 1e6, 1),
                          "matmul_us": round(mm[(m, threads)] * scale * 1e6, 1),
                          "matmul_us_1_thread": round(mm[(m, 1)] * scale * 1e6, 1),
                          "gbps": round(wbytes / t_all / 1e9, 4)})
    torch.set_num_threads(threads)
    return {"value": round(tot_bytes / tot_s / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "value_1_thread": round(tot_bytes / tot_s1 / 1e9, 4), "nproc": os.cpu_count() or 1,
            "cpu_model": _cpu_model(),
            "sample": f"IQ3_S configs[1] (17408x5120 and 5120x17408, M = 1 and 4): the first "
                      f"{CPU_SAMPLE_ROWS} rows of each shape, numpy dequantise + q8_1 round trip + torch "
                      f"fp32 matmul, each part the median of 5, scaled to the full rows",
            "cases": cases}


PEAKS_LIB = os.path.join(ROOT, "vllm-gsqrco-exl3_amd", "vllm_gguf_plugin", "libgguf_peaks.so")
FLOOR_SIZES = (38297600, 76595200)  # one 17408 x 5120 IQ3_S weight; a gate|up pair
GEMV_LAUNCH = (256, 512)  # the stream GEMV's launch: one workgroup of 8 waves per CU


def measured_peaks(torch, reps=5):
    """The two denominators measured on this GPU (libgguf_peaks.so, csrc/bench/peaks.hip):
    * read floor: one launch streaming FLOOR_SIZES bytes (a headline weight, and a gate|up pair),
      each workgroup over a contiguous equal share with 16-byte buffer loads, as the decode GEMV
      reads; graph replays of one launch per buffer over rotation_copies buffers (beyond the
      MALL), HIP events; the fastest of a sweep of launch shapes (workgroups x threads x loads in
      flight x cache policy), with the shape that gave it, and the fastest at the stream GEMV's
      own launch shape (GEMV_LAUNCH);
    * MFMA peak: 2048 workgroups of 4 waves, each wave 8 MFMAs per iteration in independent
      chains with register operands, one kernel per shape: v_mfma_i32_16x16x64_i8,
      v_mfma_f32_16x16x32_f16 (the shapes the GEMMs use), the 32 x 32 shapes
      v_mfma_i32_32x32x32_i8 and v_mfma_f32_32x32x16_f16, v_mfma_i32_16x16x32_i8,
      v_mfma_i32_4x4x4_16b_i8, and v_dot4_i32_i8 on the VALU (TOP/s or TFLOP/s)."""
    import ctypes

    lib = ctypes.CDLL(PEAKS_LIB)
    lib.gguf_peak_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    lib.gguf_peak_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_void_p]
    key = 0x9E3779B9  # a sum the data never gives: the kernels' guard store stays unexecuted
    sink = torch.zeros(2048 * 1024, dtype=torch.int32, device="cuda")
    out = {"read_floor": [], "mfma": {}}
    for nbytes in FLOOR_SIZES:
        nbuf = rotation_copies(nbytes)
        stride = (nbytes + 255) // 256 * 256
        pool = torch.randint(0, 256, (nbuf * stride,), dtype=torch.uint8, device="cuda")
        best, at_gemv = None, None
        for grid in (256, 512, 1024, 2048):
            for threads in (256, 512, 1024):
                for unroll in (1, 2, 4, 8):
                    for nt in (0, 1):
                        def call(i, grid=grid, threads=threads, unroll=unroll, nt=nt):
                            rc = lib.gguf_peak_read(pool.data_ptr() + i * stride, nbytes, grid, threads, unroll, nt,
                                                    key, sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
                            assert rc == 0, rc
                        g = graph(torch, [lambda i=i: call(i) for i in range(nbuf)])
                        us = time_graphs(torch, [g], reps) * 1e3 / nbuf
                        if best is None or us < best[0]:
                            best = (us, grid, threads, unroll, nt)
                        if (grid, threads) == GEMV_LAUNCH and (at_gemv is None or us < at_gemv[0]):
                            at_gemv = (us, grid, threads, unroll, nt)
                        del g
        for key_name, (us, grid, threads, unroll, nt) in (("best", best), ("at_gemv_launch", at_gemv)):
            out["read_floor"].append({"bytes": nbytes, "of": key_name, "us": round(us, 3),
                                      "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                                      "shape": f"{grid}x{threads} u{unroll}{' nt' if nt else ''}"})
        del pool
    grid, iters = 2048, 2000
    for kind, name, per in ((0, "i8_16x16x64_tops", 32768), (1, "f16_16x16x32_tflops", 16384),
                            (2, "i8_32x32x32_tops", 65536), (3, "f16_32x32x16_tflops", 32768),
                            (4, "i8_16x16x32_tops", 16384), (5, "i8_4x4x4_16b_tops", 2048),
                            (6, "valu_dot4_i8_tops", 512)):
        def mcall(kind=kind):
            rc = lib.gguf_peak_mfma(kind, grid, iters, key, sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
            assert rc == 0, rc
        g = graph(torch, [mcall] * 3)
        ms = time_graphs(torch, [g], 3) / 3
        out["mfma"][name] = round(grid * 4 * 8 * iters * per / (ms * 1e-3) / 1e12, 1)
        del g
    del sink
    torch.cuda.empty_cache()
    return out


def load_traffic():
    """HBM bytes per launch of the dominant kernel from the committed PMC summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def dominant_kernel(torch, C, ws, steps):
    """The headline's dominant kernel alone: the packed decode op at 17408 x 5120, M = 1, bf16 X,
    which is one launch of the stream GEMV that quantises X itself
    (gemv_iq3s_stream_kernel<IQ3_S, 1, bf16, 2, false, 8>); one graph of one launch per weight copy,
    timed with HIP events on the stream the op launches on."""
    rows, k, m = 17408, 5120, 1
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    kg = graph(torch, [lambda w=w: C.lcpp_mul_mat_vec_iq3_mma_packed(w, x, IQ3_S, rows) for w in ws])
    kernel_us = time_graphs(torch, [kg], max(5, steps)) * 1e3 / len(ws)
    alg_bytes = ws[0].numel() + m * k * 2 + m * rows * 2
    achieved = alg_bytes / (kernel_us * 1e-6) / 1e9
    # the per-launch floor of back-to-back graph launches: as many launches of a 512 KB fill
    t = torch.empty(131072, device="cuda", dtype=torch.float32)
    fg = graph(torch, [lambda: t.fill_(0.0) for _ in ws])
    floor_us = time_graphs(torch, [fg], max(5, steps)) * 1e3 / len(ws)
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic(),
            "kernel": "gemv_iq3s_stream_kernel<IQ3_S,1,bf16,2,false,8> (17408x5120, M=1, X quantised in the kernel)",
            "us_per_launch": round(kernel_us, 3), "alg_bytes_per_launch": alg_bytes,
            "launch_floor_us": round(floor_us, 3)}


def eager_calls(torch, C, ws, rows, k, ms=(1, 512), calls=200, reps=5):
    """The op called eagerly (no graph), as under enforce_eager or in prefill chunks, cycling through
    the weight copies ws as the timed graphs do:
    `us_per_call` is the time per call of a run of calls issued back to back (one synchronize at
    the end), `host_issue_us` the host's time to issue one call of that run (torch dispatch, the
    op's views and guards, the caching-allocator allocations, the launches), `call_sync_us` one call
    followed by a synchronize. With host_issue_us below the graph-replayed kernel time, eager calls
    keep the GPU busy."""
    out = []
    for m in ms:
        op = C.lcpp_mul_mat_vec_iq3_mma_packed if m <= 32 else C.lcpp_mul_mat_iq3_packed
        x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        for i in range(20):
            op(ws[i % len(ws)], x, IQ3_S, rows)
        runs, issue, sync = [], [], []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(calls):
                op(ws[i % len(ws)], x, IQ3_S, rows)
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            issue.append((t1 - t0) / calls)
            runs.append((t2 - t0) / calls)
        for i in range(10 * reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            op(ws[i % len(ws)], x, IQ3_S, rows)
            torch.cuda.synchronize()
            sync.append(time.perf_counter() - t0)
        out.append({"shape": f"{rows}x{k}", "m": m, "op": "lcpp_mul_mat_vec_iq3_mma_packed" if m <= 32
                    else "lcpp_mul_mat_iq3_packed", "us_per_call": round(statistics.median(runs) * 1e6, 2),
                    "host_issue_us": round(statistics.median(issue) * 1e6, 2),
                    "call_sync_us": round(statistics.median(sync) * 1e6, 2)})
    return out


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
    ws = [iq3_pack.pack(make_weights(torch, IQ3_S, 17408, 5120, i), IQ3_S)
          for i in range(rotation_copies(17408 * 20 * BLOCK[IQ3_S]))]
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
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other benchmark configs (CPU Q4_K, MTP small GEMM, prefill, 64-layer sweep)")
    ap.add_argument("--section", choices=["mtp", "prefill", "layers", "types", "peaks", "decode"],
                    help="run only this benchmark config and print its JSON (for rocprofv3 counter runs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured read floor and MFMA peak")
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
    if args.section:
        fn = {"mtp": lambda: config_mtp(torch, C, iq3_pack, linear),
              "prefill": lambda: config_prefill(torch, C, iq3_pack, linear),
              "types": lambda: config_types(torch, C, iq3_pack, linear),
              "decode": lambda: config_decode(torch, C, iq3_pack, linear),
              "peaks": lambda: measured_peaks(torch),
              "layers": lambda: {"layer_sweep_64": config_layers(torch, C, iq3_pack, linear, args.steps),
                                 "layer_sweep_64_runs": config_layers(torch, C, iq3_pack, linear, args.steps,
                                                                      merged=True)}}[args.section]
        print(json.dumps({"mode": "section", "section": args.section, "result": fn()}), flush=True)
        return

    # ------------------------------------------------------------------ headline workload
    cases = [(17408, 5120, 1), (17408, 5120, 4), (5120, 17408, 1), (5120, 17408, 4)]
    shapes = sorted({(r, k) for r, k, _ in cases})
    weights = {}
    for si, (rows, k) in enumerate(shapes):
        weights[(rows, k)] = [iq3_pack.pack(make_weights(torch, IQ3_S, rows, k, 100 * si + i), IQ3_S)
                              for i in range(rotation_copies(rows * (k // 256) * BLOCK[IQ3_S]))]
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
    eager = eager_calls(torch, C, weights[(17408, 5120)], 17408, 5120)
    del weights
    torch.cuda.empty_cache()
    emit("headline_cases", detail)
    emit("eager", eager)

    # ------------------------------------------------------------------ measured denominators
    peaks = None
    if not args.no_peaks:
        peaks = measured_peaks(torch)
        emit("measured_peaks", peaks)
        floor = peaks["read_floor"][0]  # one launch over the headline weight's bytes
        roofline["peak_measured"] = floor["gbps"]
        roofline["frac_measured"] = round(roofline["achieved"] / floor["gbps"], 4)
        roofline["read_floor_us"] = floor["us"]

    # ------------------------------------------------------------------ the metric's other points
    points = []
    if not args.no_points:
        for qt in (IQ3_S, Q4_K):
            points += op_points(torch, C, iq3_pack, linear, qt, 17408, 5120, (1, 4, 16, 32, 48), seed=1000)
        emit("points", points)

    if not args.no_configs:
        for name, fn in (("cpu_q4k_4096", lambda: config_cpu_q4k(torch, C)),
                         ("mtp_small_gemm", lambda: config_mtp(torch, C, iq3_pack, linear)),
                         ("prefill", lambda: config_prefill(torch, C, iq3_pack, linear)),
                         ("generic_types", lambda: config_types(torch, C, iq3_pack, linear)),
                         ("layer_sweep_64", lambda: config_layers(torch, C, iq3_pack, linear, args.steps)),
                         ("layer_sweep_64_runs",
                          lambda: config_layers(torch, C, iq3_pack, linear, args.steps, merged=True))):
            emit(name, fn())

    cpu = None if args.no_cpu else cpu_baseline(torch)
    if cpu is not None:
        emit("cpu_baseline_cases", cpu.pop("cases"))

    # the headline: one compact JSON object, the last line of stdout (the details are above)
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
        "config": {"workload": "IQ3_S decode GEMV (packed unit layout) at M=1,4 on 17408x5120 and 5120x17408, "
                               "benchmark configs[1]; per shape, weight copies of at least 512 MiB in all",
                   "calls_per_step": sum(n for *_, n, _ in per_case), "bytes_per_step": step_bytes},
        "us_per_call": {f"{c['shape']} M={c['m']}": c["us_per_call"] for c in detail},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if points:
        line["points_us"] = {TYPE_NAME[qt]: {str(p["m"]): p["us_per_call"] for p in points
                                             if p["type"] == TYPE_NAME[qt]} for qt in (IQ3_S, Q4_K)}
    if peaks is not None:
        line["measured_peaks"] = {"read_floor_gbps": [f["gbps"] for f in peaks["read_floor"] if f["of"] == "best"],
                                  "read_floor_gemv_launch_gbps": [f["gbps"] for f in peaks["read_floor"]
                                                                  if f["of"] == "at_gemv_launch"],
                                  **{k: v for k, v in peaks["mfma"].items()
                                     if k in ("i8_16x16x64_tops", "f16_16x16x32_tflops", "i8_32x32x32_tops",
                                              "f16_32x32x16_tflops")}}
    print(json.dumps(line, separators=(",", ":")), flush=True)


def emit(name, result):
    """One detail section of the full run, on its own stdout line before the headline."""
    print(json.dumps({"bench_detail": name, "result": result}, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
