#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-linear hot path (one GPU).

Headline (headline metric, config 2): W4A16 decode-regime GEMMs at Qwen3-8B
shapes (qkv 4096->6144, o 4096->4096, gate_up 4096->24576, down 12288->4096),
int4 g128 symmetric with fp16 scales, bf16 N(0,1) activations, M in {1, 4, 16}.
A step is one pass over those 12 GEMMs. ``value`` is whole-step algorithmic
GB/s (weights + scales + x + y bytes / time) with inputs resident in HBM;
weights rotate over copies totalling > 512 MB so the 256 MB MALL cannot serve
them. Launches are captured once in a HIP graph and replayed, so host launch
cost is not measured (each graph node still costs its dispatch).

Extra objects: the prefill regime (config 3, TFLOP/s vs bf16 dense MFMA peak),
fp8 block-scaled W8A16 / W8A8 at Qwen3-27B-like shapes (config 4), and the int4
MoE block at T = 256 / 4096 (config 5).

``roofline`` covers the dominant kernel (the decode kernel): achieved =
algorithmic bytes per launch / average launch time from HIP events around the
graph replays on the launch stream; ``traffic`` comes from the committed
rocprofv3 FETCH_SIZE/WRITE_SIZE measurement (profiles/decode_traffic.json) when
present. ``cpu_baseline`` times the oracle's dequantize-then-matmul (its C dequant with
OpenMP, then a numpy float32 BLAS matmul, on the box's CPU share) on config 1.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
       [--only decode|prefill|fp8|moe|copy|crossover [--m 1,2,...]] [--eager] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
MALL_BYTES = 600_000_000  # rotate over more than this (the Infinity Cache is 256 MB)

SHAPES = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 24576), ("down", 12288, 4096)]
FP8_SHAPES = [("qkv", 5120, 7168), ("o", 5120, 5120), ("gate_up", 5120, 34816), ("down", 17408, 5120)]
DECODE_M = [1, 4, 16]
PREFILL_M = [256, 1024, 4096]
FP8_M = [1, 16, 2048]
GROUP = 128


def w4a16_bytes(m, n, k, g=GROUP):
    return n * k // 2 + n * (k // g) * 2 + m * k * 2 + m * n * 2


def fp8_bytes(m, n, k, a8=False):
    return n * k + (n // 128) * (k // 128) * 4 + m * k * (1 if a8 else 2) + m * n * 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # About 25 ms timed after about 20 ms of warm-up: with 6 warm-up steps (0.6 ms) the
    # headline read ~2 % lower and varied more (the GPU clock is still rising).
    p.add_argument("--steps", type=int, default=240)
    p.add_argument("--warmup", type=int, default=200)
    # Exactly these counts are run and reported (a partial last pass over the copies is fine).
    p.add_argument("--quick", action="store_true", help="decode headline only")
    p.add_argument("--only", choices=["decode", "prefill", "fp8", "moe", "copy", "crossover"], default=None)
    p.add_argument("--m", default="1,2,4,8,12,16,24,32,48,64", help="M values of --only crossover")
    p.add_argument("--eager", action="store_true", help="no graphs (for profiler attribution)")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-detail", action="store_true", help="headline step only (profiler runs)")
    p.add_argument("--traffic", metavar="DIR", default=None,
                   help="write profiles/decode_traffic.json from the four rocprofv3 --pmc runs under DIR "
                        "(d_FETCH_SIZE, d_WRITE_SIZE: the headline step; c_FETCH_SIZE, c_WRITE_SIZE: --only copy)")
    return p.parse_args()


def cpu_baseline(budget_s=15.0):
    """Oracle dequantize-then-matmul on the host cores, config 1 (M=16, K=N=4096): the C
    restatement of the dequant (OpenMP) and a float32 BLAS matmul, both on `threads` threads
    (the box's CPU share, OMP_NUM_THREADS, else the cores this process may run on)."""
    from oracle import oracle as O
    from oracle import oracle_c as C
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    x, packed, scale = O.make_w4a16(16, 4096, 4096, GROUP, seed=1)
    times, tdq, tmm = [], [], []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        w = C.dequant_int4(packed, scale, 1, GROUP, threads=threads)
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
        "value": round(w4a16_bytes(16, 4096, 4096) / med / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"config 1 (M=16, K=N=4096, int4 g128) x{len(times)} runs, median "
                  f"{med * 1e3:.2f} ms (dequant {np.median(tdq) * 1e3:.2f} ms: the oracle's C restatement, "
                  f"OpenMP; matmul {np.median(tmm) * 1e3:.2f} ms: numpy float32 BLAS), {threads} threads",
    }


class Bench:
    def __init__(self, eager: bool):
        import torch

        from pulsarlm_amd import _lib, ops

        self.torch, self.lib, self.ops, self._lib = torch, _lib.load(), ops, _lib
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.Stream()
        self.ws = torch.zeros(256 << 20, dtype=torch.uint8, device=self.dev)
        self.eager = eager

    def time(self, launches, reps=5, warm=1):
        """Seconds per pass over `launches` (callables enqueuing on self.stream)."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for f in launches:  # eager warm-up (first-call setup happens here)
                f()
            self.stream.synchronize()
            if self.eager:
                run = lambda: [f() for f in launches]  # noqa: E731
            else:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.stream):
                    for f in launches:
                        f()
                run = g.replay
            for _ in range(warm):
                run()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(self.stream)
            for _ in range(reps):
                run()
            e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / reps

    def int4_layer(self, k, n, seed, min_copies=1):
        from oracle import oracle as O  # seeded synthetic inputs only
        torch = self.torch
        _, packed, scale = O.make_w4a16(1, n, k, GROUP, seed=seed)
        w, s = self.ops.repack_int4_marlin_cuda(torch.from_numpy(packed).to(self.dev),
                                                torch.from_numpy(scale).to(self.dev), 1, GROUP)
        nc = max(min_copies, -(-MALL_BYTES // (w.numel() * 4 + s.numel() * 2)))
        return [(w, s)] + [(w.clone(), s.clone()) for _ in range(nc - 1)]

    def gemm_launch(self, fmt, x, w, s, sdt, m, n, k, bn, y, a8=False):
        lib, L, st = self.lib, self._lib, self.stream.cuda_stream
        ws, wsn = self.ws.data_ptr(), self.ws.numel()
        xd = L.PLM_BF16
        if a8:
            return lambda: L.check(lib.plm_gemm_w8a8(x.data_ptr(), xd, w.data_ptr(), s.data_ptr(), sdt, m, n, k, bn,
                                                     GROUP, y.data_ptr(), ws, wsn, st))
        return lambda: L.check(lib.plm_gemm(fmt, x.data_ptr(), xd, w.data_ptr(), s.data_ptr(), sdt, m, n, k, bn,
                                            GROUP, y.data_ptr(), ws, wsn, st))


def time_steps(b: Bench, launches_for_copies, copies, steps, warmup):
    """Seconds per step over exactly `steps` timed steps after exactly `warmup` untimed
    ones. launches_for_copies(r) gives the launches of the first r steps of a pass over
    the weight copies (step i reads copy i % copies); the step count wraps the pass."""
    torch = b.torch
    graphs = {}

    def runner(r):
        if r not in graphs:
            launches = launches_for_copies(r)
            if b.eager:
                graphs[r] = lambda: [f() for f in launches]
            else:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=b.stream):
                    for f in launches:
                        f()
                graphs[r] = g.replay
        return graphs[r]

    def run(n):
        for _ in range(n // copies):
            runner(copies)()
        if n % copies:
            runner(n % copies)()

    with torch.cuda.stream(b.stream):
        for f in launches_for_copies(copies):  # eager first calls (per-stream set-up), not counted
            f()
        b.stream.synchronize()
        runner(copies)
        if steps % copies:
            runner(steps % copies)
        if warmup % copies:
            runner(warmup % copies)
        run(warmup)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(b.stream)
        run(steps)
        e1.record(b.stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / max(steps, 1)


def section_decode(b: Bench, steps, warmup, detail_shapes=True):
    torch, L = b.torch, b._lib
    layers = {name: b.int4_layer(k, n, i, min_copies=6) for i, (name, k, n) in enumerate(SHAPES)}
    xs = {(m, k): torch.randn(m, k, device=b.dev).to(torch.bfloat16) for m in DECODE_M for k in (4096, 12288)}
    ys = {(m, n): torch.empty(m, n, device=b.dev, dtype=torch.bfloat16) for m in DECODE_M for (_, _, n) in SHAPES}

    def launches_for(names, ms, copies):
        # Every launch reads a weight copy that no launch of the last ~500 MB touched, so
        # neither L2 nor the MALL serves weights (no layer is re-read for the next M).
        out = []
        for c in range(copies):
            for mi, m in enumerate(ms):
                for name, k, n in SHAPES:
                    if name not in names:
                        continue
                    w, s = layers[name][(c * len(ms) + mi) % len(layers[name])]
                    out.append(b.gemm_launch(L.PLM_INT4, xs[(m, k)], w, s, L.PLM_FP16, m, n, k, 1, ys[(m, n)]))
        return out

    # Headline: the 12-GEMM step, rotated over 6 copies of the layer set (~600 MB). Exactly
    # `warmup` untimed steps, then exactly `steps` timed ones: whole passes over the copies
    # replay one graph, and a last partial pass replays a graph of its first r steps.
    copies = 6
    t_step = time_steps(b, lambda r: launches_for({s[0] for s in SHAPES}, DECODE_M, r),
                        copies, steps, warmup)
    step_bytes = sum(w4a16_bytes(m, n, k) for (_, k, n) in SHAPES for m in DECODE_M)
    detail = {}
    for name, k, n in (SHAPES if detail_shapes else []):
        for m in DECODE_M:
            nc = len(layers[name])
            tt = b.time(launches_for({name}, [m], nc), reps=5) / nc
            gbs = w4a16_bytes(m, n, k) / tt / 1e9
            detail[f"{name}_m{m}"] = {"us": round(tt * 1e6, 2), "GB/s": round(gbs, 1),
                                      "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
    launches_per_step = len(SHAPES) * len(DECODE_M)
    return {
        "value": step_bytes / t_step / 1e9,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": t_step * 1e3,
        "per_launch_bytes": step_bytes / launches_per_step,
        "avg_launch_s": t_step / launches_per_step,
        "detail": detail,
    }


def mfma_plan(b: Bench, m, n, k, fmt=None, a8=False):
    """The MFMA kernel's decomposition of a plain GEMM (an internal hook of the library)."""
    import ctypes
    fn = b.lib.plm_internal_mfma_plan
    fn.restype, fn.argtypes = None, [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int32)]
    out = (ctypes.c_int32 * 8)()
    fn(b._lib.PLM_INT4 if fmt is None else fmt, m, n, k, int(a8), out)
    return {"tile": f"{out[0]}x{out[1]}", "tiles": out[2], "k_splits": out[3], "tail_tiles": out[4],
            "tail": "128-row halves" if out[6] else (f"K split {out[5]} ways" if out[4] else None),
            "skip_reduction_build": bool(out[7])}


def section_prefill(b: Bench):
    """Config 3. Cases whose plan splits K across workgroups or runs a tail launch (the
    split-K / stream-K-style decomposition) are also timed under PLM_MFMA_UNSPLIT, which takes
    the best plan with whole-K tiles and no tail launch (`no_split_us`, its plan in
    `no_split_plan`), so what the decomposition buys is measured live; the reduction's own
    cost is measured with a PLM_MEASURE_SKIP_REDUCTION build."""
    torch, L = b.torch, b._lib
    out = {}
    tot_flop = tot_t = 0.0
    for i, (name, k, n) in enumerate(SHAPES):
        copies = b.int4_layer(k, n, i, min_copies=2)
        for m in PREFILL_M:
            x = torch.randn(m, k, device=b.dev).to(torch.bfloat16)
            y = torch.empty(m, n, device=b.dev, dtype=torch.bfloat16)
            launches = [b.gemm_launch(L.PLM_INT4, x, w, s, L.PLM_FP16, m, n, k, 1, y) for (w, s) in copies]
            tt = b.time(launches, reps=2 if m == 4096 else 4) / len(copies)
            tf = 2 * m * n * k / tt / 1e12
            tot_flop += 2 * m * n * k
            tot_t += tt
            plan = mfma_plan(b, m, n, k)
            rec = {"us": round(tt * 1e6, 1), "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 3),
                   "plan": {key: v for key, v in plan.items() if key != "skip_reduction_build"}}
            if plan["k_splits"] > 1 or plan["tail_tiles"]:
                saved = os.environ.get("PLM_MFMA_UNSPLIT")
                os.environ["PLM_MFMA_UNSPLIT"] = "1"
                L.reload_tuning()
                try:
                    tu = b.time(launches, reps=2 if m == 4096 else 4) / len(copies)
                    up = mfma_plan(b, m, n, k)
                finally:
                    if saved is None:
                        del os.environ["PLM_MFMA_UNSPLIT"]
                    else:
                        os.environ["PLM_MFMA_UNSPLIT"] = saved
                    L.reload_tuning()
                rec["no_split_us"] = round(tu * 1e6, 1)
                rec["no_split_plan"] = f"{up['tile']} x{up['tiles']}"
            out[f"{name}_m{m}"] = rec
        del copies
    if mfma_plan(b, 256, 4096, 4096)["skip_reduction_build"]:
        out["measurement_build"] = "PLM_MEASURE_SKIP_REDUCTION: split-K reductions skipped, results invalid"
    out["aggregate_TFLOP/s"] = round(tot_flop / tot_t / 1e12, 1)
    out["vendor_bf16_reference"] = vendor_bf16_reference(b)
    return out


def vendor_bf16_reference(b: Bench):
    """A reference point, not this library: torch.matmul (the ROCm BLAS) on dense bf16
    weights of the same shapes at M=4096 -- no quantization, no dequant, 4x the weight
    bytes. Fractions of the same bf16 dense peak."""
    torch = b.torch
    out = {}
    for name, k, n in SHAPES:
        x = torch.randn(4096, k, device=b.dev).to(torch.bfloat16)
        w = torch.randn(n, k, device=b.dev).to(torch.bfloat16)
        y = torch.empty(4096, n, device=b.dev, dtype=torch.bfloat16)
        tt = b.time([lambda: torch.matmul(x, w.t(), out=y)], reps=4)
        out[f"{name}_m4096"] = {"us": round(tt * 1e6, 1), "frac_mfma": round(2 * 4096 * n * k / tt / 1e12 / BF16_PEAK_TFLOPS, 3)}
        del x, w, y
    return out


def section_fp8(b: Bench):
    from oracle import oracle as O
    torch, L, ops = b.torch, b._lib, b.ops
    out = {}
    for i, (name, k, n) in enumerate(FP8_SHAPES):
        rng = np.random.default_rng(40 + i)
        w = O.bf16_round(rng.standard_normal((n, k), dtype=np.float32) * 0.02)
        codes, scale = O.fp8_block_quantize(w, 128, 128)
        wt, st = ops.repack_fp8_marlin_cuda(torch.from_numpy(codes).to(b.dev).view(torch.float8_e4m3fn),
                                            torch.from_numpy(scale).to(b.dev), 128, 128)
        nc = max(2, -(-MALL_BYTES // (wt.numel() * 4)))
        copies = [(wt, st)] + [(wt.clone(), st.clone()) for _ in range(nc - 1)]
        for m in FP8_M:
            x = torch.randn(m, k, device=b.dev).to(torch.bfloat16)
            y = torch.empty(m, n, device=b.dev, dtype=torch.bfloat16)
            for a8 in (False, True):
                launches = [b.gemm_launch(L.PLM_FP8, x, w_, s_, L.PLM_FP32, m, n, k, 128, y, a8=a8)
                            for (w_, s_) in copies]
                tt = b.time(launches, reps=3) / len(copies)
                key = f"{name}_m{m}_{'w8a8' if a8 else 'w8a16'}"
                gbs = fp8_bytes(m, n, k, a8) / tt / 1e9
                tf = 2 * m * n * k / tt / 1e12
                peak = FP8_PEAK_TFLOPS if a8 else BF16_PEAK_TFLOPS
                out[key] = {"us": round(tt * 1e6, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3),
                            "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / peak, 3)}
        del copies
    return out


def section_moe(b: Bench):
    from oracle import oracle as O
    torch, ops = b.torch, b.ops
    e, hidden, inter, top_k = 128, 2048, 768, 8
    rng = np.random.default_rng(5)

    def experts(n, k):
        packed = rng.integers(-2**31, 2**31, size=(e, n, k // 8), dtype=np.int64).astype(np.int32)
        scale = (np.abs(rng.standard_normal((e, n, k // GROUP)) * 0.02) + 1e-3).astype(np.float16)
        return ops.repack_int4_experts(torch.from_numpy(packed).to(b.dev), torch.from_numpy(scale).to(b.dev), GROUP)

    gu, dn = experts(2 * inter, hidden), experts(hidden, inter)
    out = {}
    for t in (256, 4096):
        ex, wts = O.zipf_routing(t, e, top_k, seed=t)
        h = torch.randn(t, hidden, device=b.dev).to(torch.bfloat16)
        te = torch.from_numpy(ex.astype(np.int32)).to(b.dev)
        tw = torch.from_numpy(wts).to(b.dev)
        hit = len(np.unique(ex))
        tt = b.time([lambda: ops.routed_experts_int4_cuda(h, te, tw, gu, dn, inter, GROUP)], reps=5)
        rows = t * top_k
        flop = 2 * rows * (hidden * 2 * inter + inter * hidden)
        wbytes = hit * (2 * inter * hidden // 2 + 2 * inter * (hidden // GROUP) * 2 + hidden * inter // 2 +
                        hidden * (inter // GROUP) * 2)
        act_bytes = rows * hidden * 2 + rows * 2 * inter * 2 * 2 + rows * inter * 2 * 2 + rows * hidden * 2 * 2
        out[f"T{t}"] = {"us": round(tt * 1e6, 1), "experts_hit": hit,
                        "GB/s": round((wbytes + act_bytes) / tt / 1e9, 1),
                        "frac_hbm": round((wbytes + act_bytes) / tt / 1e9 / HBM_PEAK_GBS, 3),
                        "TFLOP/s": round(flop / tt / 1e12, 1),
                        "frac_mfma": round(flop / tt / 1e12 / BF16_PEAK_TFLOPS, 3)}
    return out


def section_crossover(b: Bench, ms):
    """The decode kernel against the MFMA kernel around M = 16 (the Qwen3-8B layers, int4
    g128): run with PLM_DECODE_MAX_M=0 (every M on the MFMA kernel) and with it at 16 or 32."""
    torch, L = b.torch, b._lib
    env = os.environ.get("PLM_DECODE_MAX_M")
    limit = int(env) if env is not None else None  # None: the library's own rule
    out = {"decode_max_m": limit if limit is not None else "rule"}
    for i, (name, k, n) in enumerate(SHAPES):
        copies = b.int4_layer(k, n, i, min_copies=2)
        for m in ms:
            x = torch.randn(m, k, device=b.dev).to(torch.bfloat16)
            y = torch.empty(m, n, device=b.dev, dtype=torch.bfloat16)
            launches = [b.gemm_launch(L.PLM_INT4, x, w, s, L.PLM_FP16, m, n, k, 1, y) for (w, s) in copies]
            tt = b.time(launches, reps=5) / len(copies)
            gbs = w4a16_bytes(m, n, k) / tt / 1e9
            tf = 2 * m * n * k / tt / 1e12
            kernel = "rule" if limit is None else ("decode" if m <= limit else "mfma")
            out[f"{name}_m{m}"] = {"kernel": kernel, "us": round(tt * 1e6, 2),
                                   "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3),
                                   "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}
        del copies
    return out


def section_copy(b: Bench):
    """A plain device copy of known size: the calibration run for the FETCH_SIZE /
    WRITE_SIZE counters (their reading for 256 MiB read + 256 MiB written)."""
    torch = b.torch
    nbytes = 256 << 20
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=b.dev)
    dst = torch.empty_like(src)
    tt = b.time([lambda: dst.copy_(src)], reps=5)
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": round(tt * 1e6, 1),
            "GB/s": round(2 * nbytes / tt / 1e9, 1)}


def _pmc_rows(path):
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"bench.py --traffic: no counter_collection.csv under {path}")
    rows = []
    for f in files:
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    return rows


def write_traffic(pmc_dir):
    """Per-launch HBM bytes of the decode kernels from rocprofv3 FETCH_SIZE / WRITE_SIZE
    (KiB per dispatch), each scaled by what the same counter reads for a plain 256 MiB device
    copy (bench.py --only copy): bytes = counter KiB x 1024 x (copy bytes / copy counter)."""
    def mean(name, pick):
        vals = [float(r["Counter_Value"]) for r in _pmc_rows(os.path.join(pmc_dir, name)) if pick(r["Kernel_Name"])]
        return sum(vals) / len(vals), len(vals)

    copy = lambda k: "copyBuffer" in k  # noqa: E731
    dec = lambda k: "decode_rr_kernel" in k or "decode_kernel" in k  # noqa: E731
    cf, _ = mean("c_FETCH_SIZE", copy)
    cw, _ = mean("c_WRITE_SIZE", copy)
    fetch_factor, write_factor = 262144.0 / cf, 262144.0 / cw
    df, nd = mean("d_FETCH_SIZE", dec)
    dw, _ = mean("d_WRITE_SIZE", dec)
    fetch_b = df * 1024 * fetch_factor
    write_b = dw * 1024 * write_factor
    algo = sum(w4a16_bytes(m, n, k) for (_, k, n) in SHAPES for m in DECODE_M) / (len(SHAPES) * len(DECODE_M))
    out = {
        "kernel": "decode kernels of plm_gemm at M <= 16 (decode_rr_kernel, decode_kernel), Qwen3-8B decode layer "
                  "set, M in {1,4,16}",
        "hbm_bytes_per_launch": int(round(fetch_b + write_b)),
        "algorithmic_bytes_per_launch": int(algo),
        "ratio": round((fetch_b + write_b) / algo, 4),
        "fetch_bytes_per_launch": int(round(fetch_b)),
        "write_bytes_per_launch": int(round(write_b)),
        "dispatches": nd,
        "fetch_factor": round(fetch_factor, 4),
        "write_factor": round(write_factor, 4),
        "calibration": f"__amd_rocclr_copyBuffer of 256 MiB (python3 bench.py --only copy): FETCH_SIZE {cf:.1f} KiB, "
                       f"WRITE_SIZE {cw:.1f} KiB per dispatch",
        "commands": [
            f"cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc {c} -f csv -d "
            f"/root/repo/{pmc_dir.rstrip('/')}/{p}_{c} -- python3 /root/repo/bench.py {a}"
            for c in ("FETCH_SIZE", "WRITE_SIZE")
            for p, a in (("d", "--quick --eager --no-cpu --no-detail"), ("c", "--only copy"))
        ] + [f"python3 bench.py --traffic {pmc_dir}"],
        "note": "means over every decode-kernel dispatch of the headline step (12 GEMMs per step, eager, so each "
                "dispatch is attributed)",
    }
    with open(os.path.join(ROOT, "profiles", "decode_traffic.json"), "w") as f:
        json.dump(out, f, indent=2)
        f.write("\n")
    print(json.dumps(out))


def main():
    args = parse()
    if args.traffic:
        write_traffic(args.traffic)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the hot path is single-GPU)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, ROOT)
    import torch

    torch.cuda.init()
    torch.manual_seed(0)
    b = Bench(args.eager)
    if args.only and args.only != "decode":
        ms = [int(v) for v in args.m.split(",")]
        fn = {"prefill": section_prefill, "fp8": section_fp8, "moe": section_moe, "copy": section_copy,
              "crossover": lambda b_: section_crossover(b_, ms)}[args.only]
        print(json.dumps({args.only: fn(b)}))
        return

    if mfma_plan(b, 256, 4096, 4096)["skip_reduction_build"]:
        print("bench.py: this library is a PLM_MEASURE_SKIP_REDUCTION measurement build (invalid results); "
              "only --only prefill runs on it", file=sys.stderr)
        sys.exit(2)
    d = section_decode(b, args.steps, args.warmup, detail_shapes=not args.no_detail)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    achieved = d["per_launch_bytes"] / d["avg_launch_s"] / 1e9
    result = {
        "metric": "W4A16 GEMM GB/s & TFLOP/s (% roofline) at M=1..4096, Qwen3-8B shapes",
        "value": round(d["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": d["steps"],
        "warmup": d["warmup"],
        "ms_per_step": round(d["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded: x ~ N(0,1) bf16, q ~ U[-8,7], fp16 scales |N(0,.02)|+1e-3)",
        "config": {
            "workload": "benchmark config 2: Qwen3-8B decode layer set (qkv 4096->6144, o 4096->4096, gate_up "
                        "4096->24576, down 12288->4096) x M in {1,4,16}, int4 g128; one step = 12 GEMMs; weights "
                        "rotated over 6 copies (~600 MB) so the 256 MB MALL cannot serve them",
            "M": DECODE_M,
            "group_size": GROUP,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "decode_rr_kernel / decode_kernel (plm_gemm, M <= 16)",
            "algorithmic_bytes_per_launch": int(d["per_launch_bytes"]),
            "avg_launch_us": round(d["avg_launch_s"] * 1e6, 3),
        },
        "decode_detail": d["detail"],
    }
    if not args.quick and args.only is None:
        result["prefill_config3"] = section_prefill(b)
        result["fp8_config4"] = section_fp8(b)
        result["moe_config5"] = section_moe(b)
    if not args.quick and not args.no_cpu and args.only is None:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
