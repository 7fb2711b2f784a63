#!/usr/bin/env python3
"""Benchmark of the INT4 superblock dequant-GEMM on one MI355X.

Workload (default): the FFN projection K=3072 x M=8192, weights ~N(0, 0.02)
(seed 1003) quantized to 144-byte superblocks (3072*8192/256 = 98,304
records, 14.16 MB) and stored in strip order (the loader's layout for such
shapes; --row-order: the reference's row-order stream), fp16 activations
~N(0, 1), swept over N = 1, 2, 4, 8, 16, 32 parallel traces.  One "step" is
one sweep: six projections, one per N, each on a different copy of the
weight stream (copies rotate so that the 256 MB Infinity Cache cannot serve
repeats: >= 300 MB of distinct records); steps are replayed as HIP graphs of
consecutive sweeps, as a decode loop is captured.  Beside it, the largest single-GPU
projection, K=8192 x M=28672 (132 MB of records, 0.1 % outliers at 8 sigma),
at N = 1, 8, 32 in strip, tile and row order.

Printed: one JSON line with the whole-job throughput (tokens/s over the
sweep), per-N microseconds per call (HIP-graph replay of back-to-back calls,
HIP events on the launch stream), HBM GB/s and roofline fraction on that
time, the same bytes read by a plain streaming-read kernel (the floor), the
roofline of the dominant call (with the HBM traffic that rocprofv3 counted
for it, when profiles/ holds it) and the CPU baseline (the numpy oracle of
the reference CPU path on the host cores, with matmul-only, torch and
one-thread variants).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
CONFIGS = {
    # name: (K, M, weight std, weight seed, outlier fraction, default Ns)
    "k2048_m2048": (2048, 2048, 0.02, 1001, 0.0, [8]),
    "k2048_m5504": (2048, 5504, 0.02, 1002, 0.0, [1, 2, 4, 8, 16, 32]),
    "k3072_m8192": (3072, 8192, 0.02, 1003, 0.0, [1, 2, 4, 8, 16, 32]),
    "k8192_m28672": (8192, 28672, 0.01, 1005, 0.001, [1, 32]),
    "k2048_m32000": (2048, 32000, 0.02, 1006, 0.0, [1, 2, 4, 8, 16, 32]),
    "k4096_m14336": (4096, 14336, 0.02, 1007, 0.0, [1, 2, 4, 8, 16, 32]),
    "k2048_m6144": (2048, 6144, 0.02, 1008, 0.0, [16]),
    "k2048_m11264": (2048, 11264, 0.02, 1009, 0.0, [16]),
    "k5632_m2048": (5632, 2048, 0.02, 1010, 0.0, [16]),
}
WORKLOAD_NAMES = {
    "k2048_m2048": "int4 superblock projection 2048x2048",
    "k2048_m5504": "int4 superblock FFN gate/up projection K=2048 M=5504, N sweep 1..32",
    "k3072_m8192": "int4 superblock FFN projection K=3072 M=8192, N sweep 1..32",
    "k8192_m28672": "int4 superblock projection K=8192 M=28672 (70B-class FFN, 0.1% 8-sigma outliers)",
    "k2048_m32000": "int4 superblock LM head K=2048 (hidden) x M=32000 (vocabulary), N sweep 1..32",
    "k4096_m14336": "int4 superblock FFN projection K=4096 M=14336 (8B-class), N sweep 1..32",
    "k2048_m6144": "int4 superblock Q|K|V projection of a hidden-2048 layer (K=2048, M=3x2048)",
    "k2048_m11264": "int4 superblock gate|up projection of a hidden-2048 layer (K=2048, M=2x5632)",
    "k5632_m2048": "int4 superblock down projection of a hidden-2048 layer (K=5632, M=2048)",
}
ROTATE_BYTES = 300 * 1024 * 1024
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak (information: the path is HBM-bound)
DEFAULT_CONFIG = "k3072_m8192"
# measured beside the default workload: the largest single-GPU projection
SIDE_CONFIG = ("k8192_m28672", [1, 8, 32])
# One decoder layer's projections at hidden 2048 (Q, K, V, O 2048x2048; gate
# and up 2048x5632; down 5632 -> 2048), run back to back at N = 16 traces.
LAYER = [("q", 2048, 2048), ("k", 2048, 2048), ("v", 2048, 2048), ("o", 2048, 2048),
         ("gate", 2048, 5632), ("up", 2048, 5632), ("down", 5632, 2048)]
LAYER_N = 16
LAYER_SEED = 1004


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algo_bytes(N: int, K: int, M: int) -> int:
    """Algorithmic HBM bytes of one call: records (0.5625 B/weight) + fp16 X + fp32 Y."""
    return 144 * K * M // 256 + 2 * N * K + 4 * N * M


def _thread_info() -> dict:
    import torch
    info = {"os_cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "torch_threads": torch.get_num_threads()}
    try:
        from threadpoolctl import threadpool_info
        pools = threadpool_info()
        info["blas_threads"] = max((p.get("num_threads") or 1) for p in pools) if pools else None
        info["blas"] = sorted({p.get("internal_api", "?") for p in pools})
    except Exception:  # threadpoolctl missing
        info["blas_threads"] = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return info


def cpu_baseline(K, M, ns, blob, budget_s: float):
    """The reference CPU path on the host (the oracle: decode the records,
    then a float32 matmul), per N, median of 3-10 repetitions, and beside it:
    the matmul alone on weights decoded beforehand, torch.matmul in fp32 on
    the CPU, and decode + matmul on one thread (BLAS and torch limited to 1).
    `value` is decode + matmul on all threads over the N sweep."""
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import superblock_oracle as O

    info = _thread_info()
    w32 = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    w32_t = torch.from_numpy(w32)
    xs = {N: O.synthetic_activations(N, K, 2200 + N) for N in ns}
    per_variant_budget = budget_s / 4

    def timed(fn, budget):
        fn()  # warm
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < budget and len(times) < 10):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times)

    def sweep(make_fn, nlist, budget):
        out, tt, tok = {}, 0.0, 0
        for N in nlist:
            med, reps = timed(make_fn(N), budget / len(nlist))
            out[N] = {"ms_per_call": round(med * 1e3, 3), "tok_s": round(N / med, 2), "reps": reps}
            tt += med
            tok += N
        return out, tok / tt

    full, value = sweep(lambda N: (lambda: O.gemm_ref(xs[N], blob, K, M)), ns, per_variant_budget)
    mm, mm_v = sweep(lambda N: (lambda: xs[N].astype(np.float32) @ w32), ns, per_variant_budget)
    tm, tm_v = sweep(lambda N: (lambda: torch.from_numpy(xs[N].astype(np.float32)) @ w32_t), ns, per_variant_budget)
    prev_torch = torch.get_num_threads()
    try:
        from threadpoolctl import threadpool_limits
        limiter = threadpool_limits(limits=1)
    except Exception:
        limiter = None
    torch.set_num_threads(1)
    try:
        one, one_v = sweep(lambda N: (lambda: O.gemm_ref(xs[N], blob, K, M)), ns, per_variant_budget)
    finally:
        torch.set_num_threads(prev_torch)
        if limiter is not None:
            limiter.restore_original_limits()
    return {
        "value": round(value, 2),
        "unit": "tok/s",
        "cores": int(info.get("blas_threads") or 1),
        "kind": "port",
        "sample": (f"numpy oracle of the reference CPU path (decode the {K}x{M} records to fp16, then a float32 "
                   f"BLAS matmul), per N in {ns}, median of 3-10 reps each (~{budget_s:.0f} s for all variants); "
                   f"decode is single-threaded numpy, the matmul uses {info.get('blas_threads')} BLAS threads"),
        "threads": info,
        "per_n": full,
        "variants": {
            "matmul_only_predecoded_f32": {"tok_s": round(mm_v, 2), "per_n": mm},
            "torch_matmul_f32_cpu": {"tok_s": round(tm_v, 2), "per_n": tm, "torch_threads": info["torch_threads"]},
            "decode_plus_matmul_1_thread": {"tok_s": round(one_v, 2), "per_n": one},
        },
    }


def traffic_from_counters(fetch_csv: str, write_csv: str, config: str, n: int) -> dict:
    """HBM bytes per call of the GEMM from two rocprofv3 --pmc runs of this
    script (FETCH_SIZE, then WRITE_SIZE, CSV output, ``--ns n``), counting
    every kernel of the call (the main kernel and, when the plan has one, the
    fix-up kernel).  Each counter is scaled by what it reads for the largest
    plain copy of the same run: the clones of the weight stream, whose size is
    known (every clone reads and writes exactly the record bytes).  Returns
    the entry written to profiles/traffic_<config>_<layout>.json."""
    import csv
    K, M = CONFIGS[config][:2]
    sb_bytes = 144 * K * M // 256

    def per_kernel(path, counter):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        copies = [float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]]
        scale = sb_bytes / (max(copies) * 1024.0)  # counter reads KiB
        out = {}
        for r in rows:
            name = r["Kernel_Name"]
            if "gemm" in name or "fixup" in name or "splitk_sum" in name:
                key = name.split("(")[0].replace("void ", "")
                out.setdefault(key, []).append(float(r["Counter_Value"]) * 1024.0 * scale)
        med = {k: float(np.median(v)) for k, v in out.items()}
        return med, scale

    fetch, fs = per_kernel(fetch_csv, "FETCH_SIZE")
    write, ws = per_kernel(write_csv, "WRITE_SIZE")
    kernels = {k: {"read_bytes": round(fetch.get(k, 0.0)), "written_bytes": round(write.get(k, 0.0))}
               for k in sorted(set(fetch) | set(write))}
    main_k = max(kernels, key=lambda k: kernels[k]["read_bytes"])
    total = sum(v["read_bytes"] + v["written_bytes"] for v in kernels.values())
    return {"n": n, "traffic": total, "kernel": main_k, "algorithmic_bytes": algo_bytes(n, K, M),
            "traffic_over_algorithmic": round(total / algo_bytes(n, K, M), 3),
            "kernels": kernels, "scale": {"FETCH_SIZE": round(fs, 4), "WRITE_SIZE": round(ws, 4)},
            "calibration": f"largest __amd_rocclr_copyBuffer of the run = one clone of the {sb_bytes}-byte record stream"}


class Timer:
    """Timing on one capture stream: per-call time from HIP-graph replays of
    back-to-back calls, HIP events on the launch stream around the replays.
    (rocprofv3's kernel durations for the same calls agree with it within a
    few per cent: the dispatch gap between graph kernels is small.  HIP
    events inside a graph, which would bracket single kernels, are not
    available on ROCm, and events around eager launches add the launch path's
    own time.)"""

    def __init__(self, torch):
        self.torch = torch
        self.cap = torch.cuda.Stream()
        self.cap.wait_stream(torch.cuda.current_stream())
        self.events_in_graph = True

    def capture(self, fn, calls):
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.cap):
            for c in range(calls):
                fn(c)
        torch.cuda.synchronize()
        return g

    def replay_us(self, graphs, reps):
        """Elapsed microseconds of `reps` replays (cycling through `graphs`)."""
        torch = self.torch
        with torch.cuda.stream(self.cap):
            for g in graphs[:2]:
                g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(self.cap)
            for r in range(reps):
                graphs[r % len(graphs)].replay()
            e1.record(self.cap)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3

    def run_us(self, graphs):
        """Elapsed microseconds of one replay of each graph in `graphs`, in order."""
        torch = self.torch
        with torch.cuda.stream(self.cap):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(self.cap)
            for g in graphs:
                g.replay()
            e1.record(self.cap)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3

    def per_call_us(self, fn, calls, total_calls=200):
        g = self.capture(fn, calls)
        warm = self.replay_us([g], 1)
        self.replay_us([g], max(1, int(20000 / max(warm, 1.0))))  # ~20 ms: the GPU leaves its idle clocks
        reps = max(1, total_calls // calls)
        return self.replay_us([g], reps) / (reps * calls)


def build_projection(torch, dev, config, layout):
    """Weights of `config` quantized on the GPU (row, tile or strip order),
    and enough copies of the records that the rotated set exceeds the 256 MB
    Infinity Cache."""
    from moat_amd.dequant import quantize_to_superblocks, records_to_strips, records_to_tiles
    K, M, std, seed, outl, _ = CONFIGS[config]
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((K, M), dtype=np.float32) * np.float32(std)
    if outl:
        n_out = int(round(outl * K * M))
        pos = rng.choice(K * M, size=n_out, replace=False)
        w.reshape(-1)[pos] = rng.choice(np.array([-1.0, 1.0], np.float32), size=n_out) * np.float32(8 * std)
    blob0 = quantize_to_superblocks(torch.from_numpy(w).to(dev))  # (S, 144) uint8 on the GPU
    del w
    row_blob = blob0
    if layout == "tile":
        blob0 = records_to_tiles(blob0, K, M)
    elif layout == "strip":
        blob0 = records_to_strips(blob0, K, M)
    copies = max(2, -(-ROTATE_BYTES // blob0.numel()))
    blobs = [blob0] + [blob0.clone() for _ in range(copies - 1)]
    return blobs, row_blob


def measure_projection(torch, timer, lib, config, ns, layout, args, with_floor=True):
    """Per-N figures of one projection shape: per-call time (graph replay),
    kernel time (events around each call), the streaming-read floor of the
    same record bytes, GB/s and roofline fraction on the kernel time."""
    from moat_amd.dequant import _gemm_into
    dev = torch.device("cuda", 0)
    K, M = CONFIGS[config][:2]
    blobs, row_blob = build_projection(torch, dev, config, layout)
    copies = len(blobs)
    sb_bytes = blobs[0].numel()
    order = layout
    log(f"[bench] {config} ({order} order): K={K} M={M}, {copies} copies of {sb_bytes / 1e6:.2f} MB records")
    xs = {N: torch.from_numpy(np.random.default_rng(2000 + 100 * 2 + N).standard_normal((N, K), dtype=np.float32)
                              .astype(np.float16)).to(dev) for N in ns}
    ys = {N: torch.empty((N, M), dtype=torch.float32, device=dev) for N in ns}

    def call(N, i):
        _gemm_into(xs[N], blobs[i % copies], ys[N], K, M, args.algo, args.splits, args.batch, args.finish,
                   args.front, group=args.group, waves=args.waves, tile_order=layout == "tile",
                   strip_order=layout == "strip")

    with torch.cuda.stream(timer.cap):
        for N in ns:  # creates this stream's workspace before any capture
            for i in range(3):
                call(N, i)
    torch.cuda.synchronize()
    floor = None
    if with_floor:
        sink = torch.zeros(1, dtype=torch.int32, device=dev)

        def read(i):
            _lib_check(lib.moat_int4_stream_read(blobs[i % copies].data_ptr(), sb_bytes, 0, sink.data_ptr(),
                                                 timer.cap.cuda_stream))
        f_call = timer.per_call_us(read, copies, args.calls)
        floor = {"bytes": sb_bytes, "us_per_call": round(f_call, 3), "gbs": round(sb_bytes / f_call / 1e3, 1),
                 "kernel": "stream_read_kernel (16-byte loads, up to 2048 workgroups of 256 threads)"}
        log(f"[bench]   read floor: {f_call:7.2f} us per call ({sb_bytes / f_call / 1e3:6.0f} GB/s)")
    per_n = {}
    for N in ns:
        us = timer.per_call_us(lambda c: call(N, c), copies, args.calls)
        b = algo_bytes(N, K, M)
        tflops = 2.0 * N * K * M / us / 1e6
        per_n[N] = {"us_per_call": round(us, 3), "gbs": round(b / us / 1e3, 1),
                    "roofline_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "tok_s": round(N / us * 1e6, 1),
                    "algo_bytes": b, "tflops": round(tflops, 2),
                    "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 5)}
        if floor:
            per_n[N]["over_read_floor"] = round(us / floor["us_per_call"], 3)
        log(f"[bench]   N={N:2d}: {us:8.2f} us/call  {b / us / 1e3:7.0f} GB/s  "
            f"{100 * b / us / 1e3 / HBM_PEAK_GBS:5.1f}% of 8 TB/s"
            + (f"  | {us / floor['us_per_call']:.2f}x read floor" if floor else ""))
    t1 = per_n[ns[0]]["us_per_call"] / ns[0]
    for N in ns:
        per_n[N]["per_token_speedup_vs_first"] = round(t1 / (per_n[N]["us_per_call"] / N), 3)
    return {"K": K, "M": M, "order": order, "copies": copies, "per_n": per_n, "read_floor": floor,
            "call": call, "row_blob": row_blob}


# The reference's native benchmark (antigravity-engine/src/metal_runner.cpp:
# 120-157): the dense fp16 GEMM at N = 8, K = M = 2048, 0.2638 ms per call on
# an Apple M1 (30,327.6 tok/s).
DENSE_CONFIG = ("dense_k2048_m2048", 2048, 2048, [1, 8, 32])
DENSE_REFERENCE_TOK_S = 30327.6


def dense_bytes(N: int, K: int, M: int) -> int:
    """Algorithmic HBM bytes of one dense call: fp16 W + fp16 X + fp16 Y."""
    return 2 * K * M + 2 * N * K + 2 * N * M


def measure_dense(torch, timer, lib, K, M, ns, args):
    """The dense fp16 product (``moat_dense_gemm``) per N: graph replay of
    back-to-back calls over rotated weight copies (> 256 MB), the
    streaming-read floor of the same weight bytes beside it."""
    from moat_amd.dense import dense_gemm
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(1010)
    w0 = torch.from_numpy((0.02 * rng.standard_normal((K, M), dtype=np.float32)).astype(np.float16)).to(dev)
    copies = max(2, -(-ROTATE_BYTES // (2 * K * M)))
    ws = [w0] + [w0.clone() for _ in range(copies - 1)]
    xs = {N: torch.from_numpy(rng.standard_normal((N, K), dtype=np.float32).astype(np.float16)).to(dev) for N in ns}
    ys = {N: torch.empty((N, M), dtype=torch.float16, device=dev) for N in ns}

    def call(N, i):
        dense_gemm(xs[N], ws[i % copies], ys[N], splits=args.splits)

    with torch.cuda.stream(timer.cap):
        for N in ns:  # the capture stream's workspace exists before any capture
            call(N, 0)
    torch.cuda.synchronize()
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    wb = 2 * K * M

    def read(i):
        _lib_check(lib.moat_int4_stream_read(ws[i % copies].data_ptr(), wb, 0, sink.data_ptr(),
                                             timer.cap.cuda_stream))
    f_call = timer.per_call_us(read, copies, args.calls)
    log(f"[bench] dense fp16 K={K} M={M}: {copies} copies of {wb / 1e6:.2f} MB; read floor {f_call:7.2f} us")
    per_n = {}
    for N in ns:
        us = timer.per_call_us(lambda c: call(N, c), copies, args.calls)
        b = dense_bytes(N, K, M)
        per_n[str(N)] = {"us_per_call": round(us, 3), "gbs": round(b / us / 1e3, 1),
                         "roofline_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "tok_s": round(N / us * 1e6, 1),
                         "algo_bytes": b, "over_read_floor": round(us / f_call, 3)}
        log(f"[bench]   dense N={N:2d}: {us:8.2f} us/call  {b / us / 1e3:7.0f} GB/s  {us / f_call:.2f}x read floor")
    del ws
    return {"workload": f"dense fp16 decode product K={K} M={M} (fp16 weights, fp32 sums, fp16 out)", "K": K,
            "M": M, "copies": copies, "per_n": per_n,
            "read_floor": {"bytes": wb, "us_per_call": round(f_call, 3), "gbs": round(wb / f_call / 1e3, 1)}}


def run_dense(args) -> int:
    """The reference's native benchmark shape on the dense fp16 path: value =
    tokens/s at N = 8 (the shape it times), vs_baseline against its M1
    figure; the other N and the read floor beside it."""
    import torch
    from moat_amd import _lib

    lib = _lib.load()
    torch.cuda.set_device(0)
    _, K, M, ns0 = DENSE_CONFIG
    if args.dense_shape:
        K, M = (int(v) for v in args.dense_shape.lower().split("x"))
    ns = [int(v) for v in args.ns.split(",")] if args.ns else ns0
    timer = Timer(torch)
    d = measure_dense(torch, timer, lib, K, M, ns, args)
    dom = "8" if "8" in d["per_n"] else str(ns[0])
    r = d["per_n"][dom]
    cpu = None
    if not args.no_cpu_baseline:
        # the reference's CPU product (test_batched_speed.py:31-42): fp16(f32(X) @ f32(W)), the
        # oracle's dense_gemm_ref, on the host's BLAS threads; median of 3-10 calls per N
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import dense_oracle as DO
        info = _thread_info()
        rng = np.random.default_rng(1011)
        w_h = (0.02 * rng.standard_normal((K, M))).astype(np.float16)
        per = {}
        for N in ns:
            x_h = rng.standard_normal((N, K)).astype(np.float16)
            DO.dense_gemm_ref(x_h, w_h)
            times, t_start = [], time.perf_counter()
            while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_budget / len(ns) and len(times) < 10):
                t0 = time.perf_counter()
                DO.dense_gemm_ref(x_h, w_h)
                times.append(time.perf_counter() - t0)
            med = float(np.median(times))
            per[str(N)] = {"ms_per_call": round(med * 1e3, 3), "tok_s": round(N / med, 1), "reps": len(times)}
        c = per.get(dom, per[str(ns[0])])
        cpu = {"value": c["tok_s"], "unit": "tok/s", "cores": info.get("blas_threads"), "kind": "port",
               "sample": f"fp16(f32(X) @ f32(W)) (oracle dense_gemm_ref, the reference's CPU product) at "
                         f"N = {dom}, K = {K}, M = {M}; every N timed, median of 3-10 calls",
               "per_n": per, "threads": info}
        log(f"[bench] CPU baseline: {c['tok_s']:.1f} tok/s at N={dom} ({info.get('blas_threads')} BLAS threads)")
    out = {
        "metric": "dense fp16 GEMM µs/call and tok/s (the reference's native benchmark shape)",
        "value": r["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.calls, "warmup": 1,
        "ms_per_step": round(r["us_per_call"] / 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": (round(r["tok_s"] / DENSE_REFERENCE_TOK_S, 2)
                        if dom == "8" and (K, M) == DENSE_CONFIG[1:3] else None),
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": d["workload"], "K": K, "M": M, "n": int(dom), "ns": ns,
                   "weight_copies_rotated": d["copies"]},
        "per_n": d["per_n"], "read_floor": d["read_floor"],
        "roofline": {"bound": "hbm", "achieved": r["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": r["roofline_frac"], "traffic": None,
                     "kernel": f"dense_gemm_kernel N={dom}: {r['algo_bytes']} algorithmic B per call / "
                               f"{r['us_per_call']} us per call (HIP-graph replay of back-to-back calls)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def _lib_check(st):
    if st != 0:
        raise RuntimeError(f"libmoat_int4 call failed with status {st}")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default=DEFAULT_CONFIG,
                    choices=sorted(CONFIGS) + ["layer_h2048", "quantize_load", DENSE_CONFIG[0]]
                    + sorted(SAMPLE_CONFIGS),
                    help="projection shape (default: K=3072 x M=8192, N = 1..32, with K=8192 x M=28672 "
                         "measured beside it); layer_h2048: one decoder layer's 7 projections at N=16; "
                         "quantize_load: fp16 weights of one layer to INT4 records on the GPU; "
                         "sample_v32000 / sample_v128256: token sampling from V=32000 (K=2048 LM head) or "
                         "V=128256 (K=4096) logits, alone and after the INT4 LM head; dense_k2048_m2048: the "
                         "dense fp16 product at the reference's native benchmark shape")
    ap.add_argument("--dense-shape", default=None, metavar="KxM",
                    help="dense_k2048_m2048: another K x M for the dense fp16 product (fp16 weights)")
    ap.add_argument("--ns", default=None, help="comma-separated N values (default: the config's)")
    ap.add_argument("--algo", type=int, default=0, help="0 auto, 1 dot2, 2 mfma")
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--calls", type=int, default=200, help="timed launches per N for the per-N table")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-side", action="store_true",
                    help="skip the K=8192 x M=28672 block measured beside the default workload")
    ap.add_argument("--batch", type=int, default=0, help="rounds of loads issued together (0 auto)")
    ap.add_argument("--finish", type=int, default=0, help="split-K hand-off (0 auto, 1 atomics, 2 fences, 3 kernel)")
    ap.add_argument("--waves", type=int, default=0, help="waves per workgroup, 4 or 8 (0 auto)")
    ap.add_argument("--group", type=int, default=0,
                    help="row order: tile groups (0 auto); strip order: 0 auto, 1 the strip-group kernel (N > 8), "
                         "2 the strip kernel 8 rows a launch, 3 the wide strip kernel")
    ap.add_argument("--front", type=int, default=0,
                    help="load front end (0 auto, 1 LDS-staged, 2 direct, 3 LDS DMA, 4 record stream)")
    ap.add_argument("--tile-order", action="store_true",
                    help="GEMM configs: weights stored in tile order (each 256-column tile's rows contiguous; "
                         "moat_int4_records_to_tiles), read by moat_int4_gemm_tiles; needs M %% 256 == 0")
    ap.add_argument("--strip-order", action="store_true",
                    help="GEMM configs: weights in strip order (moat_int4_records_to_strips), read by "
                         "moat_int4_gemm_strips -- the default wherever the loader stores it (K >= 2048, "
                         "K %% 32 == 0, M %% 32 == 0)")
    ap.add_argument("--row-order", action="store_true",
                    help="GEMM configs: weights in the reference's row order, read by moat_int4_gemm_ex")
    ap.add_argument("--fused", action="store_true",
                    help="layer_h2048: Q, K, V in one launch and gate/up fused with SwiGLU (h feeds down)")
    ap.add_argument("--driver", action="store_true",
                    help="layer_h2048: through moat_amd.layer.LayerProjections (strip order, Q|K|V and gate|up "
                         "each one launch, SwiGLU kernel, one graph over consecutive layers)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"), default=None,
                    help="no GPU run: turn two rocprofv3 --pmc counter CSVs (FETCH_SIZE, WRITE_SIZE) of "
                         "`bench.py --ns N` into profiles/traffic_<config>_<layout>.json")
    args = ap.parse_args()

    if args.traffic_from:
        n = int(args.ns.split(",")[0]) if args.ns else max(CONFIGS[args.config][5])
        K, M = CONFIGS[args.config][:2]
        layout = "tile" if args.tile_order else ("row" if args.row_order or not (K >= 2048 and K % 32 == 0
                                                                                   and M % 32 == 0) else "strip")
        entry = traffic_from_counters(args.traffic_from[0], args.traffic_from[1], args.config, n)
        entry["layout"] = layout
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            f"traffic_{args.config}_{layout}.json")
        data = json.load(open(path)) if os.path.exists(path) else {}
        data[str(n)] = entry
        with open(path, "w") as f:
            json.dump(data, f, indent=1)
        print(json.dumps(entry))
        return 0

    if args.gpus != 1:
        print(f"bench.py measures one GPU: moat_amd has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2

    if args.config == "layer_h2048":
        return run_layer(args)
    if args.config == "quantize_load":
        return run_quantize_load(args)
    if args.config in SAMPLE_CONFIGS:
        return run_sample(args)
    if args.config == DENSE_CONFIG[0]:
        return run_dense(args)

    import torch
    from moat_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    K, M = CONFIGS[args.config][:2]
    if args.tile_order and M % 256 != 0:
        print(f"--tile-order needs M % 256 == 0 (M = {M})", file=sys.stderr)
        return 2
    ns = [int(v) for v in args.ns.split(",")] if args.ns else CONFIGS[args.config][5]
    timer = Timer(torch)
    strip_ok = K >= 2048 and K % 32 == 0 and M % 32 == 0  # the loader's strip_layout_ok
    if args.tile_order:
        layout = "tile"
    elif args.row_order or not strip_ok:
        if args.strip_order:
            print(f"--strip-order needs K >= 2048, K %% 32 == 0 and M %% 32 == 0 (K = {K}, M = {M})", file=sys.stderr)
            return 2
        layout = "row"
    else:
        layout = "strip"
    main_res = measure_projection(torch, timer, lib, args.config, ns, layout, args)
    per_n, call = main_res["per_n"], main_res["call"]
    copies = main_res["copies"]

    # steps: one sweep over ns per step, `copies` steps to a graph (a decode
    # loop is captured whole, so one graph launch serves many steps; with
    # one step a graph, the launch's own 2-4 us would fall on every step),
    # call c of a graph on weight copy c % copies; exactly args.steps steps
    # are timed (whole graphs, then one graph of the remaining steps)
    per_graph = copies
    full = timer.capture(lambda c: call(ns[c % len(ns)], c), per_graph * len(ns))
    rest = args.steps % per_graph
    tail = timer.capture(lambda c: call(ns[c % len(ns)], c), rest * len(ns)) if rest else None
    with torch.cuda.stream(timer.cap):
        for _ in range(-(-args.warmup // per_graph)):
            full.replay()
    torch.cuda.synchronize()
    sequence = [full] * (args.steps // per_graph) + ([tail] if tail is not None else [])
    us_total = timer.run_us(sequence)
    ms_step = us_total / args.steps / 1e3
    tokens = sum(ns)
    value = tokens / (ms_step / 1e3)
    log(f"[bench] sweep: {ms_step * 1e3:.1f} us/step, {value:.0f} tok/s")

    side = None
    if args.config == DEFAULT_CONFIG and not args.no_side and not args.ns:
        side_cfg, side_ns = SIDE_CONFIG
        side = {}
        for lay in ("strip", "tile", "row"):
            r = measure_projection(torch, timer, lib, side_cfg, side_ns, lay, args, with_floor=lay == "strip")
            side[lay + "_order"] = {
                "per_n": {str(k): v for k, v in r["per_n"].items()}, "read_floor": r["read_floor"],
                "copies": r["copies"]}
            del r
            torch.cuda.empty_cache()
        side = {"workload": WORKLOAD_NAMES[side_cfg], "K": CONFIGS[side_cfg][0], "M": CONFIGS[side_cfg][1],
                "ns": side_ns, **side}

    layer_driver = None
    if args.config == DEFAULT_CONFIG and not args.no_side and not args.ns:
        torch.cuda.empty_cache()
        d = measure_layer_driver(args, with_cpu=False)
        layer_driver = {"workload": d["config"]["workload"], "n": d["config"]["n"],
                        "us_per_layer": round(d["ms_per_step"] * 1e3, 3), "tok_s": d["value"],
                        "layers_in_graph": d["config"]["layers_in_graph"], "layouts": d["config"]["layouts"],
                        "per_launch": d["per_launch"], "roofline": d["roofline"]}
        del d
        torch.cuda.empty_cache()

    dense = None
    if args.config == DEFAULT_CONFIG and not args.no_side and not args.ns:
        torch.cuda.empty_cache()
        dense = measure_dense(torch, timer, lib, DENSE_CONFIG[1], DENSE_CONFIG[2], DENSE_CONFIG[3], args)
        dense["reference"] = {"n": 8, "tok_s": DENSE_REFERENCE_TOK_S, "hardware": "Apple M1",
                              "source": "metal_hardware_proof.md:37-42"}
        torch.cuda.empty_cache()

    dom = max(ns, key=lambda n: per_n[n]["us_per_call"])
    roof = {
        "bound": "hbm",
        "achieved": per_n[dom]["gbs"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": per_n[dom]["roofline_frac"],
        "traffic": None,
        "kernel": (f"int4 gemm N={dom} (the sweep's longest call): {per_n[dom]['algo_bytes']} algorithmic B per "
                   f"call / {per_n[dom]['us_per_call']} us per call (HIP-graph replay of back-to-back calls; the "
                   f"main kernel plus the fix-up kernel when the plan has one)"),
    }
    traffic_name = f"traffic_{args.config}_{layout}.json"
    traffic_file = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", traffic_name)
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            tr = json.load(f).get(str(dom))
        if tr is not None:
            roof["traffic"] = tr["traffic"]
            roof["traffic_over_algorithmic"] = tr["traffic_over_algorithmic"]
            roof["traffic_source"] = f"profiles/{traffic_name} (rocprofv3 FETCH_SIZE + WRITE_SIZE, all kernels of the call)"

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (numpy oracle) ...")
        cpu = cpu_baseline(K, M, ns, main_res["row_blob"].cpu().numpy(), args.cpu_budget)
        log(f"[bench] CPU baseline: {cpu['value']:.1f} tok/s (decode + matmul, {cpu['cores']} BLAS threads); "
            f"matmul alone {cpu['variants']['matmul_only_predecoded_f32']['tok_s']:.1f}, torch fp32 "
            f"{cpu['variants']['torch_matmul_f32_cpu']['tok_s']:.1f}, one thread "
            f"{cpu['variants']['decode_plus_matmul_1_thread']['tok_s']:.1f} tok/s")

    out = {
        "metric": "INT4 dequant-GEMM µs/call, HBM GB/s (% roofline), tok/s at N=1..32",
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",  # dequantized weights and activations in fp16, products summed in fp32
        "data": "synthetic",
        "config": {"workload": WORKLOAD_NAMES[args.config], "K": K, "M": M, "ns": ns,
                   "weight_copies_rotated": copies,
                   "timing": "steps: HIP graphs of consecutive N sweeps (one weight copy per call), exactly "
                             "`steps` sweeps timed; per N: HIP graph replay of back-to-back calls; HIP events on the "
                             "launch stream",
                   "algo": args.algo, "splits": args.splits, "batch": args.batch, "finish": args.finish,
                   "front": args.front, "weights": "int4 superblocks (144 B per 256 weights)"
                   + f", {layout} order",
                   "activations": "fp16", "output": "fp32"},
        "per_n": {str(k): v for k, v in per_n.items()},
        "read_floor": main_res["read_floor"],
        "largest_projection": side,
        "layer_driver": layer_driver,
        "dense_fp16": dense,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


# name -> (LM head K, vocabulary V): a 32000-token vocabulary after a hidden
# size of 2048, and Llama-3's 128256 tokens after 4096
SAMPLE_CONFIGS = {"sample_v32000": (2048, 32000), "sample_v128256": (4096, 128256)}
SAMPLE_T = 0.7  # the coordinator's default temperature (batch_generator.py:190)


def run_sample(args) -> int:
    """Token sampling from LM-head logits, N = 1..32 rows: the sampler alone
    (greedy and T = 0.7, logits already on the GPU), and one decode step's
    tail -- the INT4 LM head K x V (weight copies rotated) followed by the
    T = 0.7 sampler.  value = tokens/s of the LM head + sampler over the N
    sweep; the CPU baseline is the numpy oracle of the reference's sampler on
    the same logits."""
    import torch
    from moat_amd import _lib
    from moat_amd.dequant import _gemm_into, quantize_to_superblocks, records_to_strips
    from moat_amd.sampling import TokenSampler

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    ns = [int(v) for v in args.ns.split(",")] if args.ns else [1, 2, 4, 8, 16, 32]
    K, V = SAMPLE_CONFIGS[args.config]
    sampler = TokenSampler()
    table = sampler.exp_lut.table()
    step = sampler.exp_lut.step_f32
    rng = np.random.default_rng(1007)
    w = torch.from_numpy(rng.standard_normal((K, V), dtype=np.float32) * np.float32(0.02)).to(dev)
    blob0 = records_to_strips(quantize_to_superblocks(w), K, V)  # the loader's layout for this shape
    del w
    copies = max(2, -(-ROTATE_BYTES // blob0.numel()))
    blobs = [blob0] + [blob0.clone() for _ in range(copies - 1)]
    xs = {N: torch.from_numpy(np.random.default_rng(2100 + N).standard_normal((N, K), dtype=np.float32)
                              .astype(np.float16)).to(dev) for N in ns}
    logits = {N: torch.empty((N, V), dtype=torch.float32, device=dev) for N in ns}
    toks = {N: torch.empty(N, dtype=torch.int32, device=dev) for N in ns}
    lps = {N: torch.empty(N, dtype=torch.float32, device=dev) for N in ns}
    ws_bytes = int(lib.moat_sample_workspace_size(max(ns), V))
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)  # row counters start at zero
    log(f"[bench] {args.config}: LM head {K}x{V} ({blob0.numel() / 1e6:.2f} MB records, {copies} copies), "
        f"table {sampler.exp_lut.size} entries")
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())

    def sample(N, temp, seed):
        _lib.check(lib.moat_sample_tokens(logits[N].data_ptr(), _lib.DTYPE_F32, N, V, temp, sampler.top_k, seed,
                                          table.data_ptr(), sampler.exp_lut.size, step, toks[N].data_ptr(),
                                          lps[N].data_ptr(), ws.data_ptr(), ws_bytes, cap.cuda_stream), "sample")

    def head(N, i):
        _gemm_into(xs[N], blobs[i % copies], logits[N], K, V, strip_order=True)

    with torch.cuda.stream(cap):
        for N in ns:
            for i in range(2):
                head(N, i)
                sample(N, SAMPLE_T, i)
                sample(N, 0.0, i)
    torch.cuda.synchronize()

    def capture(fn, calls):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            for c in range(calls):
                fn(c)
        torch.cuda.synchronize()
        return g

    def timed(g, reps):
        with torch.cuda.stream(cap):
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cap)
            for _ in range(reps):
                g.replay()
            e1.record(cap)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps  # us per replay

    per_n = {}
    calls = max(copies, 20)
    for N in ns:
        greedy = timed(capture(lambda c: sample(N, 0.0, c), calls), max(2, args.steps // 10)) / calls
        samp = timed(capture(lambda c: sample(N, SAMPLE_T, c), calls), max(2, args.steps // 10)) / calls
        pipe = timed(capture(lambda c: (head(N, c), sample(N, SAMPLE_T, c)), copies),
                     max(2, args.steps // 10)) / copies
        sbytes = N * V * 4 + 2 * sampler.exp_lut.size + 8 * N  # logits, the table, tokens and logs
        per_n[N] = {"sample_us": round(samp, 3), "greedy_us": round(greedy, 3), "lm_head_plus_sample_us": round(pipe, 3),
                    "tok_s": round(N / pipe * 1e6, 1), "sample_bytes": sbytes,
                    "sample_gbs": round(sbytes / samp / 1e3, 1)}
        log(f"[bench] N={N:2d}: sample {samp:7.2f} us  greedy {greedy:7.2f} us  LM head + sample {pipe:7.2f} us  "
            f"({N / pipe * 1e6:9.0f} tok/s)")
    total_us = sum(per_n[N]["lm_head_plus_sample_us"] for N in ns)
    value = sum(ns) / (total_us / 1e6)
    log(f"[bench] sweep: {total_us:.1f} us, {value:.0f} tok/s (LM head + sampler)")
    dom = max(ns)
    roof = {"bound": "hbm", "achieved": per_n[dom]["sample_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(per_n[dom]["sample_gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": (f"sampler (chunk stats, sums, select + draw: 3 launches) N={dom}: "
                       f"{per_n[dom]['sample_bytes']} B per call (fp32 logits, the 64 KB table, tokens and logs) / "
                       f"{per_n[dom]['sample_us']} us")}
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import sampling_oracle as S
        host = logits[16 if 16 in ns else dom].cpu().numpy()
        t0 = time.perf_counter()
        rows = 0
        while time.perf_counter() - t0 < min(args.cpu_budget, 10.0):
            S.sample_tokens(host, temperature=SAMPLE_T, seed=rows)
            rows += host.shape[0]
        dt = time.perf_counter() - t0
        cpu = {"value": rows / dt, "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"numpy oracle of the reference's sampler (table softmax, top-50, one draw) on "
                         f"{host.shape[0]}x{V} fp32 logits, repeated for ~10 s; sampling only, no LM head"}
        log(f"[bench] CPU baseline: {cpu['value']:.1f} tok/s sampled")
    out = {
        "metric": "token sampling from LM-head logits: us/call and tok/s of INT4 LM head + sampler at N=1..32",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": 1,
        "ms_per_step": round(total_us / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"LM head K={K} x V={V} (INT4 records) then table-softmax top-50 sampling at "
                               f"T={SAMPLE_T}, N sweep {ns}", "copies": copies,
                   "timing": "HIP graph replay, HIP events on the launch stream"},
        "per_n": {str(k): v for k, v in per_n.items()},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def run_quantize_load(args) -> int:
    """Quantize-on-load of one decoder layer's weights (the 7 projections at
    hidden 2048, fp16, 57.8 MB): the loader's rule (fp16 scale first) and the
    144-byte records written in one kernel per tensor.  Throughput in weights/s
    and GB/s of fp16 read + records written; the CPU baseline is the oracle
    (quantize, then serialize) on the host."""
    import torch
    from moat_amd import _lib
    from moat_amd.dequant import _float_dtype_code

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    rng = np.random.default_rng(LAYER_SEED)
    host = [(rng.standard_normal((K, M), dtype=np.float32) * np.float32(0.02)).astype(np.float16) for _, K, M in LAYER]
    layer_w = sum(K * M for _, K, M in LAYER)
    copies = max(2, -(-ROTATE_BYTES // (2 * layer_w)))
    ws = [[torch.from_numpy(h).to(dev) for h in host] for _ in range(copies)]
    outs = [torch.empty((K * M // 256, 144), dtype=torch.uint8, device=dev) for _, K, M in LAYER]
    log(f"[bench] quantize_load: 7 tensors, {layer_w / 1e6:.1f} M weights per layer, {copies} copies")
    cap = torch.cuda.Stream()

    def one_layer(c):
        for t, o in zip(ws[c], outs):
            w, code = _float_dtype_code(t)
            _lib.check(lib.moat_int4_quantize_pack(w.data_ptr(), code, w.numel(), _lib.SCALE_F16, o.data_ptr(),
                                                   cap.cuda_stream), "quantize_load")

    with torch.cuda.stream(cap):
        one_layer(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for c in range(copies):
            one_layer(c)
    torch.cuda.synchronize()
    with torch.cuda.stream(cap):
        graph.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cap)
        reps = max(1, args.steps // copies)
        for _ in range(reps):
            graph.replay()
        e1.record(cap)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
    bytes_layer = layer_w * 2 + layer_w * 144 // 256
    value = layer_w / (us / 1e6)
    log(f"[bench] quantize_load: {us:.2f} us/layer, {value / 1e9:.2f} G weights/s, {bytes_layer / us / 1e3:.0f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import superblock_oracle as O
        t0 = time.perf_counter()
        n_done = 0
        for h in host:
            q, s = O.quantize_b(h.reshape(-1))
            O.serialize_superblocks(q, s)
            n_done += h.size
            if time.perf_counter() - t0 > args.cpu_budget:
                break
        dt = time.perf_counter() - t0
        cpu = {"value": n_done / dt, "unit": "weights/s", "cores": 1, "kind": "port",
               "sample": f"numpy oracle: surface-B quantize + serialize of {n_done} weights of the same layer "
                         f"(single-threaded numpy elementwise work)"}
        log(f"[bench] CPU baseline: {cpu['value'] / 1e6:.1f} M weights/s")
    out = {
        "metric": "INT4 quantize-on-load weights/s (fp16 weights to 144-byte records)",
        "value": round(value, 1), "unit": "weights/s", "n_gpus": 1, "steps": reps * copies, "warmup": 1,
        "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "quantize-on-load of one decoder layer at hidden 2048 (7 fp16 tensors, "
                               f"{layer_w} weights), fp16-scale rule, records written", "copies": copies},
        "roofline": {"bound": "hbm", "achieved": round(bytes_layer / us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(bytes_layer / us / 1e3 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"quantize_pack_kernel: {bytes_layer} B per layer (fp16 in, records out) / {us:.2f} us"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def measure_layer_driver(args, with_cpu: bool = True) -> dict:
    """One decoder layer's projections through moat_amd.layer.LayerProjections
    at N = 16: Q|K|V in one strip-order launch, O, gate|up with the SwiGLU
    epilogue in one launch (fp16 h) and down(h), captured in one HIP graph that
    holds `copies` distinct layers (>= 300 MB of records, so no layer is served
    from the Infinity Cache), like consecutive layers of a model.  A step is
    one layer.  Returns the JSON object of the measurement."""
    import torch
    from moat_amd.dequant import quantize_to_superblocks
    from moat_amd.layer import LayerProjections

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    N = int(args.ns.split(",")[0]) if args.ns else LAYER_N
    names = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "o": "o_proj", "gate": "gate_proj", "up": "up_proj",
             "down": "down_proj"}
    rng = np.random.default_rng(LAYER_SEED)
    first = {}
    for name, K, M in LAYER:
        w = rng.standard_normal((K, M), dtype=np.float32) * np.float32(0.02)
        first[names[name]] = (quantize_to_superblocks(torch.from_numpy(w).to(dev)), K, M)
    layer_bytes = sum(144 * K * M // 256 for _, K, M in LAYER)
    copies = max(2, -(-ROTATE_BYTES // layer_bytes))
    log(f"[bench] layer driver: {layer_bytes / 1e6:.2f} MB of records per layer, {copies} layers, N={N}")
    layers = [LayerProjections(first, max_batch=N)]
    for c in range(1, copies):  # distinct weight memory per layer (same values)
        layers.append(LayerProjections({k: (r.clone(), K, M) for k, (r, K, M) in first.items()}, max_batch=N))
    log(f"[bench] layouts: {layers[0].layouts}")
    xr = np.random.default_rng(2400)
    for lay in layers:
        for buf in (lay.x, lay.attn, lay.x_mlp):
            buf.copy_(torch.from_numpy(xr.standard_normal(tuple(buf.shape), dtype=np.float32).astype(np.float16)))
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())

    def graph_of(fn):
        with torch.cuda.stream(cap):
            for lay in layers[:2]:
                fn(lay)
        cap.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            for lay in layers:
                fn(lay)
        torch.cuda.synchronize()
        return g

    def timed(g, replays):
        with torch.cuda.stream(cap):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cap)
            for _ in range(replays):
                g.replay()
            e1.record(cap)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3  # us

    graph = graph_of(lambda lay: lay.run(N))
    warm_us = timed(graph, 1)
    timed(graph, max(1, int(20000 / max(warm_us, 1.0))))
    replays = max(1, -(-args.steps // copies))
    us = timed(graph, replays) / (replays * copies)
    value = N / (us / 1e6)
    H, I = 2048, 5632
    qkv_m = layers[0].q_dim + 2 * layers[0].kv_dim
    parts = {
        "qkv": (lambda lay: lay.attention_inputs(N), algo_bytes(N, H, qkv_m)),
        "o": (lambda lay: lay.output_projection(N), algo_bytes(N, layers[0].q_dim, H)),
        # fused (strip order): weights + X + fp16 h; else the fp32 gate|up output
        # is written, read back by the SwiGLU kernel, and h written
        "gate_up+swiglu": (lambda lay: lay.mlp_front(N),
                           algo_bytes(N, H, 2 * I) - 8 * N * I + 2 * N * I if layers[0].gate_up_w.fused
                           else algo_bytes(N, H, 2 * I) + 8 * N * I + 2 * N * I),
        "down": (lambda lay: lay.down_projection(N), algo_bytes(N, I, H)),
    }
    bytes_layer = sum(b for _, b in parts.values())
    log(f"[bench] layer driver: {us:.2f} us/layer, {value:.0f} tok/s, {bytes_layer / us / 1e3:.0f} GB/s")
    per_part = {}
    for pname, (fn, b) in parts.items():
        g = graph_of(fn)
        timed(g, 2)
        reps = max(2, args.calls // copies)
        pus = timed(g, reps) / (reps * copies)
        per_part[pname] = {"us_per_call": round(pus, 3), "algorithmic_bytes": b, "gbs": round(b / pus / 1e3, 1),
                           "roofline_frac": round(b / pus / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"[bench] {pname:15s}: {pus:7.2f} us  {b / pus / 1e3:6.0f} GB/s")
        del g
    for lay in layers:
        lay.check()

    cpu = None
    if with_cpu and not args.no_cpu_baseline:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import superblock_oracle as O
        hosts = {k: r.cpu().numpy() for k, (r, K, M) in first.items()}
        x_h, a_h, m_h = (t[:N].cpu().numpy() for t in (layers[0].x, layers[0].attn, layers[0].x_mlp))
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_budget and len(times) < 10):
            t0 = time.perf_counter()
            for k in ("q_proj", "k_proj", "v_proj"):
                O.gemm_ref(x_h, hosts[k], H, H)
            O.gemm_ref(a_h, hosts["o_proj"], H, H)
            h = O.swiglu_ref(m_h, hosts["gate_proj"], hosts["up_proj"], H, I).astype(np.float16)
            O.gemm_ref(h, hosts["down_proj"], I, H)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        cpu = {"value": N / med, "unit": "tok/s", "cores": os.cpu_count(), "kind": "port",
               "sample": (f"numpy oracle: one layer's projections (Q, K, V, O, SwiGLU of gate/up, down of fp16 h; "
                          f"decode records, float32 matmul) at N={N}, median of {len(times)} layers; "
                          f"host os.cpu_count()={os.cpu_count()}")}
        log(f"[bench] CPU baseline: {cpu['value']:.1f} tok/s")

    out = {
        "metric": "INT4 dequant-GEMM µs/call, HBM GB/s (% roofline), tok/s at N=1..32",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": replays * copies, "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "decoder layer projections at hidden 2048 (Q,K,V,O 2048x2048, gate/up 2048x5632, "
                               f"down 5632x2048), N={N}, through the layer driver: Q|K|V one launch, O, gate|up "
                               "with SwiGLU one launch (fp16 h), down(h), one graph over consecutive layers",
                   "n": N, "layouts": layers[0].layouts, "layers_in_graph": copies,
                   "timing": "HIP graph replay, HIP events on the launch stream",
                   "weights": "int4 superblocks (144 B per 256 weights)", "activations": "fp16", "output": "fp32"},
        "per_launch": per_part,
        "roofline": {"bound": "hbm", "achieved": round(bytes_layer / us / 1e3, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(bytes_layer / us / 1e3 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"layer: {bytes_layer} algorithmic B per layer / {us:.2f} us per layer"},
        "cpu_baseline": cpu,
    }
    return out


def run_layer_driver(args) -> int:
    print(json.dumps(measure_layer_driver(args)), flush=True)
    return 0


def run_layer(args) -> int:
    """One decoder layer's projections (Q, K, V, O, gate, up, down) at N = 16,
    back to back on one stream, each on its own weights; the layer's weights
    rotate over enough copies (>= 300 MB) that no projection is served from
    the Infinity Cache.  A step is one layer."""
    import torch
    if args.driver:
        return run_layer_driver(args)
    from moat_amd import _lib
    from moat_amd.dequant import _gemm_into, _multi_into, _swiglu_into, quantize_to_superblocks

    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    N = int(args.ns.split(",")[0]) if args.ns else LAYER_N
    rng = np.random.default_rng(LAYER_SEED)
    layer_bytes = sum(144 * K * M // 256 for _, K, M in LAYER)
    copies = max(2, -(-ROTATE_BYTES // layer_bytes))
    log(f"[bench] building layer_h2048: 7 projections, {layer_bytes / 1e6:.2f} MB of records, {copies} copies")
    blobs = []  # blobs[c][p]
    first = []
    for name, K, M in LAYER:
        w = rng.standard_normal((K, M), dtype=np.float32) * np.float32(0.02)
        first.append(quantize_to_superblocks(torch.from_numpy(w).to(dev)))
    blobs.append(first)
    for c in range(1, copies):
        blobs.append([b.clone() for b in first])
    xs = [torch.from_numpy(np.random.default_rng(2400 + i).standard_normal((N, K), dtype=np.float32)
                           .astype(np.float16)).to(dev) for i, (_, K, M) in enumerate(LAYER)]
    ys = [torch.empty((N, M), dtype=torch.float32, device=dev) for _, K, M in LAYER]

    h = torch.empty((N, 5632), dtype=torch.float16, device=dev)

    def layer(c):
        b = blobs[c % copies]
        if args.fused:
            # Q, K, V: one launch on the shared input; O; gate/up + SwiGLU -> h; down(h)
            _multi_into(xs[0], b[0:3], ys[0:3], 2048, 2048)
            _gemm_into(xs[3], b[3], ys[3], 2048, 2048)
            _swiglu_into(xs[4], b[4], b[5], h, 2048, 5632)
            _gemm_into(h, b[6], ys[6], 5632, 2048)
            return
        for p, (_, K, M) in enumerate(LAYER):
            _gemm_into(xs[p], b[p], ys[p], K, M, args.algo, args.splits, args.batch, args.finish, args.front)

    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        for c in range(2):
            layer(c)
    torch.cuda.synchronize()
    # one graph holds one layer on every weight copy (`copies` layers)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for c in range(copies):
            layer(c)
    torch.cuda.synchronize()

    def timed(replays):
        with torch.cuda.stream(cap):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cap)
            for r in range(replays):
                graph.replay()
            e1.record(cap)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3  # us

    warm_us = timed(1)
    timed(max(1, int(20000 / max(warm_us, 1.0))))  # about 20 ms at full clocks
    replays = max(1, -(-args.steps // copies))
    us = timed(replays) / (replays * copies)
    value = N / (us / 1e6)
    bytes_layer = sum(algo_bytes(N, K, M) for _, K, M in LAYER)
    if args.fused:  # X read once by Q/K/V and by gate/up; h (fp16) written once instead of gate and up
        bytes_layer -= 2 * (2 * N * 2048) + 2 * 4 * N * 5632 - 2 * N * 5632
    log(f"[bench] layer{' (fused)' if args.fused else ''}: {us:.2f} us/layer, {value:.0f} tok/s, "
        f"{bytes_layer / us / 1e3:.0f} GB/s")

    # per projection: one graph of that projection on every weight copy
    per_proj = {}
    for p, (name, K, M) in enumerate(LAYER):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            for c in range(copies):
                _gemm_into(xs[p], blobs[c][p], ys[p], K, M, args.algo, args.splits, args.batch, args.finish,
                           args.front)
        torch.cuda.synchronize()
        reps = max(2, args.calls // copies)
        with torch.cuda.stream(cap):
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(cap)
            for r in range(reps):
                g.replay()
            e1.record(cap)
        e1.synchronize()
        pus = e0.elapsed_time(e1) * 1e3 / (reps * copies)
        b = algo_bytes(N, K, M)
        per_proj[name] = {"K": K, "M": M, "us_per_call": round(pus, 3), "gbs": round(b / pus / 1e3, 1),
                          "roofline_frac": round(b / pus / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"[bench] {name:4s} {K}x{M}: {pus:7.2f} us/call  {b / pus / 1e3:6.0f} GB/s")
        del g

    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import superblock_oracle as O
        hosts = [(first[p].cpu().numpy(), xs[p].cpu().numpy(), K, M) for p, (_, K, M) in enumerate(LAYER)]
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < args.cpu_budget and len(times) < 10):
            t0 = time.perf_counter()
            for blob_h, x_h, K, M in hosts:
                O.gemm_ref(x_h, blob_h, K, M)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        cpu = {"value": N / med, "unit": "tok/s", "cores": os.cpu_count(), "kind": "port",
               "sample": (f"numpy oracle: the 7 projections of one layer (decode records, float32 matmul) at "
                          f"N={N}, median of {len(times)} layers; host os.cpu_count()={os.cpu_count()}")}
        log(f"[bench] CPU baseline: {cpu['value']:.1f} tok/s")

    out = {
        "metric": "INT4 dequant-GEMM µs/call, HBM GB/s (% roofline), tok/s at N=1..32",
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "decoder layer projections at hidden 2048 (Q,K,V,O 2048x2048, gate/up 2048x5632, "
                               f"down 5632x2048), N={N}, back to back"
                               + (", Q/K/V in one launch, gate/up fused with SwiGLU" if args.fused else ""),
                   "n": N, "fused": bool(args.fused),
                   "weight_copies_rotated": copies, "timing": "HIP graph replay, HIP events on the launch stream",
                   "weights": "int4 superblocks (144 B per 256 weights)", "activations": "fp16", "output": "fp32"},
        "per_projection": per_proj,
        "roofline": {"bound": "hbm", "achieved": round(bytes_layer / us / 1e3, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(bytes_layer / us / 1e3 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"7 projections: {bytes_layer} algorithmic B per layer / {us:.2f} us per layer"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
