#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-linear hot path (one GPU).

Headline (BASELINE.json metric, config 2): W4A16 decode-regime GEMMs at Qwen3-8B
shapes (qkv 4096->6144, o 4096->4096, gate_up 4096->24576, down 12288->4096),
int4 g128 symmetric with fp16 scales, bf16 N(0,1) activations, M in {1, 4, 16}.
A step is one pass over those 12 GEMMs. ``value`` is whole-step algorithmic
GB/s (weights + scales + x + y bytes / time); inputs are resident in HBM and
weights rotate over copies totalling > 512 MB so the 256 MB MALL cannot serve
them. Steps are captured once in a HIP graph and replayed, so host launch cost
is not measured. Extra fields report the prefill regime (config 3, TFLOP/s vs
bf16 dense MFMA peak) and config 1.

``roofline`` covers the dominant kernel (the decode kernel): achieved =
algorithmic bytes per launch / average launch time from HIP events around the
graph replays on the launch stream. ``cpu_baseline`` times the oracle's
dequantize-then-matmul (numpy, all host cores) on config 1.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0

SHAPES = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 24576), ("down", 12288, 4096)]
DECODE_M = [1, 4, 16]
PREFILL_M = [256, 1024, 4096]
GROUP = 128


def w4a16_bytes(m, n, k, g=GROUP):
    return n * k // 2 + n * (k // g) * 2 + m * k * 2 + m * n * 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--quick", action="store_true", help="skip the prefill sweep and the CPU baseline")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


class Layer:
    """One repacked int4 weight (several rotating copies) for a K->N shape."""

    def __init__(self, torch, ops, k, n, copies, seed):
        from oracle import oracle as O  # seeded synthetic inputs only
        _, packed, scale = O.make_w4a16(1, n, k, GROUP, seed=seed)
        pk = torch.from_numpy(packed).cuda()
        sc = torch.from_numpy(scale).cuda()
        w, s = ops.repack_int4_marlin_cuda(pk, sc, 1, GROUP)
        # Enough copies that rotating over them alone exceeds 512 MB (the MALL is 256 MB).
        copies = max(copies, -(-600_000_000 // (w.numel() * 4 + s.numel() * 2)))
        self.copies = [(w, s)] + [(w.clone(), s.clone()) for _ in range(copies - 1)]
        self.k, self.n = k, n
        del pk, sc


def cpu_baseline(budget_s=15.0):
    """Oracle dequantize-then-matmul on the host cores, config 1 (M=16, K=N=4096)."""
    from oracle import oracle as O
    cores = len(os.sched_getaffinity(0))
    x, packed, scale = O.make_w4a16(16, 4096, 4096, GROUP, seed=1)
    times, tdq, tmm = [], [], []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        w = O.dequant_int4(packed, scale, 1, GROUP)
        t1 = time.perf_counter()
        y = x @ w.T  # float32 BLAS, fp32 accumulation (test_marlin.cpp:108-111)
        O.bf16_round(y)
        t2 = time.perf_counter()
        times.append(t2 - t0)
        tdq.append(t1 - t0)
        tmm.append(t2 - t1)
        if len(times) >= 5 and time.perf_counter() > t_end:
            break
    med = float(np.median(times))
    return {
        "value": w4a16_bytes(16, 4096, 4096) / med / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"config 1 (M=16, K=N=4096, int4 g128) x{len(times)} runs, median "
                  f"{med * 1e3:.1f} ms (dequant {np.median(tdq) * 1e3:.1f} ms, matmul {np.median(tmm) * 1e3:.1f} ms), "
                  f"numpy oracle",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(no multi-GPU path: the north star is single-GPU)", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from pulsarlm_amd import _lib, ops

    torch.cuda.init()
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    lib = _lib.load()

    # Rotating weight copies: 99.4 MB per layer set -> 6 copies ~ 600 MB > 512 MB.
    copies = 6
    layers = [Layer(torch, ops, k, n, copies, seed=i) for i, (_, k, n) in enumerate(SHAPES)]
    xs = {m: {k: torch.randn(m, k, device=dev).to(torch.bfloat16) for k in (4096, 12288)}
          for m in DECODE_M + PREFILL_M}
    ys = {(m, n): torch.empty(m, n, device=dev, dtype=torch.bfloat16) for m in DECODE_M + PREFILL_M
          for n in (4096, 6144, 24576)}
    ws_bytes = max(lib.plm_gemm_workspace_bytes(_lib.PLM_INT4, m, n, k)
                   for m in DECODE_M + PREFILL_M for (_, k, n) in SHAPES)
    ws = torch.zeros(max(ws_bytes, 1 << 16), dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream()

    def launch(m, layer, copy):
        w, s = layer.copies[copy]
        x = xs[m][layer.k]
        y = ys[(m, layer.n)]
        rc = lib.plm_gemm(_lib.PLM_INT4, x.data_ptr(), _lib.PLM_BF16, w.data_ptr(), s.data_ptr(), _lib.PLM_FP16,
                          m, layer.n, layer.k, 1, GROUP, y.data_ptr(), ws.data_ptr(), ws.numel(),
                          stream.cuda_stream)
        _lib.check(rc)

    def capture(ms):
        """One graph = every copy x every layer x every M in ms (rotation inside the graph)."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            for c in range(copies):  # eager warm-up of every launch
                for L in layers:
                    for m in ms:
                        launch(m, L, c)
            stream.synchronize()
            with torch.cuda.graph(g, stream=stream):
                for c in range(copies):
                    for L in layers:
                        for m in ms:
                            launch(m, L, c)
        return g

    def time_graph(g, reps, warm):
        # Replays run on `stream` (the stream the kernels were captured on), and the
        # events bracketing them are recorded on the same stream.
        with torch.cuda.stream(stream):
            for _ in range(warm):
                g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3  # seconds

    # ---------------- decode regime (headline) ----------------
    g_dec = capture(DECODE_M)
    # A step = the 12 GEMMs; one graph replay = `copies` steps.
    reps = max(1, -(-args.steps // copies))
    warm = max(1, -(-args.warmup // copies))
    t = time_graph(g_dec, reps, warm)
    steps = reps * copies
    step_bytes = sum(w4a16_bytes(m, n, k) for (_, k, n) in SHAPES for m in DECODE_M)
    ms_per_step = t / steps * 1e3
    value = step_bytes * steps / t / 1e9
    launches = steps * len(SHAPES) * len(DECODE_M)
    per_launch_bytes = step_bytes / (len(SHAPES) * len(DECODE_M))
    avg_launch_s = t / launches

    # Per-shape / per-M breakdown (each its own graph, same rotation).
    detail = {}
    for name, k, n in SHAPES:
        L = layers[[s[0] for s in SHAPES].index(name)]
        for m in DECODE_M:
            g = torch.cuda.CUDAGraph()
            nc = len(L.copies)
            with torch.cuda.stream(stream):
                for c in range(nc):
                    launch(m, L, c)
                stream.synchronize()
                with torch.cuda.graph(g, stream=stream):
                    for c in range(nc):
                        launch(m, L, c)
            tt = time_graph(g, 10, 1) / (10 * nc)
            detail[f"{name}_m{m}"] = {"us": round(tt * 1e6, 2),
                                      "GB/s": round(w4a16_bytes(m, n, k) / tt / 1e9, 1),
                                      "frac_hbm": round(w4a16_bytes(m, n, k) / tt / 1e9 / HBM_PEAK_GBS, 3)}

    # ---------------- prefill regime (config 3) ----------------
    prefill = {}
    if not args.quick:
        for name, k, n in SHAPES:
            L = layers[[s[0] for s in SHAPES].index(name)]
            for m in PREFILL_M:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.stream(stream):
                    launch(m, L, 0)
                    stream.synchronize()
                    with torch.cuda.graph(g, stream=stream):
                        for c in range(copies):
                            launch(m, L, c)
                reps_p = 3 if m == 4096 else 5
                tt = time_graph(g, reps_p, 1) / (reps_p * copies)
                tf = 2 * m * n * k / tt / 1e12
                prefill[f"{name}_m{m}"] = {"us": round(tt * 1e6, 1), "TFLOP/s": round(tf, 1),
                                           "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 3)}
        tot_flop = sum(2 * m * n * k for (_, k, n) in SHAPES for m in PREFILL_M)
        tot_t = sum(v["us"] for v in prefill.values()) * 1e-6
        prefill["aggregate_TFLOP/s"] = round(tot_flop / tot_t / 1e12, 1)

    result = {
        "metric": "W4A16 GEMM GB/s & TFLOP/s (% roofline) at M=1..4096, Qwen3-8B shapes",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm * copies,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded: x ~ N(0,1) bf16, q ~ U[-8,7], fp16 scales |N(0,.02)|+1e-3)",
        "config": {
            "workload": "BASELINE config 2: Qwen3-8B decode layer set (qkv, o, gate_up, down) x M in {1,4,16}, "
                        "int4 g128, one step = 12 GEMMs, weights rotated over 6 copies (~600 MB)",
            "shapes_KxN": [[k, n] for (_, k, n) in SHAPES],
            "M": DECODE_M,
            "group_size": GROUP,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(per_launch_bytes / avg_launch_s / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(per_launch_bytes / avg_launch_s / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "decode_kernel (plm_gemm, M<=16)",
            "algorithmic_bytes_per_launch": int(per_launch_bytes),
            "avg_launch_us": round(avg_launch_s * 1e6, 3),
        },
        "decode_detail": detail,
        "prefill_config3": prefill,
    }
    if not args.quick and not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
