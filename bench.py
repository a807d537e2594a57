#!/usr/bin/env python3
"""Benchmark of the quantized hot path on one MI355X.

Headline (BASELINE.json metric "Q4_0 GEMV GB/s (% HBM peak); Q8_0 GEMM int8 TOPS
(% MFMA peak)"): one step = one Q4_0 x Q8_0 decode GEMV, W 4096 x 4096
(configs[3]), through the C-ABI entry tcrv_hip_gemv_q4_0_q8_0.  The weight
matrix rotates over enough distinct copies (> 256 MB) that every launch reads
W from HBM, not from the 256 MB Infinity Cache.  The second half of the metric,
the Q8_0 x Q8_0 GEMM 4096^3 in int8 TOPS, and the other configs
are reported in the same JSON line.

Inputs are synthetic (tianchen-rv_amd/synth.py, seeds 1001-1009) and already
resident in HBM when a timed region starts.  Timed regions are bracketed by
torch.cuda.synchronize() and HIP events recorded on the launch stream.
The cpu_baseline leg times the scalar C oracle (oracle/) on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tianchen-rv_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
N = 4096


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--gemm-steps", type=int, default=50)
    ap.add_argument("--mode", choices=["graph", "eager"], default="graph",
                    help="launch the timed steps from a captured HIP graph or eagerly")
    ap.add_argument("--copies", type=int, default=40,
                    help="distinct weight copies rotated by the GEMV (>256 MB total)")
    ap.add_argument("--cpu-seconds", type=float, default=4.0,
                    help="wall time per CPU-baseline leg")
    ap.add_argument("--only", choices=["all", "gemv", "gemm"], default="all")
    return ap.parse_args()


class Timer:
    """Events on the launch stream around a region of `count` launches."""

    def __init__(self, torch, stream):
        self.torch = torch
        self.stream = stream
        self.start = torch.cuda.Event(enable_timing=True)
        self.stop = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.torch.cuda.synchronize()
        self.start.record(self.stream)
        return self

    def __exit__(self, *exc):
        self.stop.record(self.stream)
        self.torch.cuda.synchronize()
        self.ms = self.start.elapsed_time(self.stop)


def run_region(torch, stream, launch, steps, mode):
    """Runs `steps` launches (launch(i) issues step i) and returns elapsed ms."""
    if mode == "graph":
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(steps):
                launch(i)
        torch.cuda.synchronize()
        g.replay()  # untimed first replay
        with Timer(torch, stream) as t:
            g.replay()
        return t.ms
    with Timer(torch, stream) as t:
        for i in range(steps):
            launch(i)
    return t.ms


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the sharding design is described in DESIGN.md); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import synth
    import tcrv_hip

    tcrv_hip.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    sptr = stream.cuda_stream
    result = {}

    # ------------------------------------------------------------ GEMV ---
    if args.only in ("all", "gemv"):
        log("building GEMV inputs (W 4096x4096 Q4_0 seed 1006, x Q8_0 seed 1007)")
        w = synth.q4_0_matrix(N, N, synth.SEEDS["gemv_w"], 0.02)
        x = synth.q8_0_matrix(1, N, synth.SEEDS["gemv_x"], 1.0).reshape(-1)
        bx = w.shape[1]
        wbytes = w.size
        w_dev = torch.from_numpy(w).to(dev).reshape(-1)
        copies = torch.empty((args.copies, wbytes), dtype=torch.uint8, device=dev)
        copies[:] = w_dev
        del w_dev
        x_dev = torch.from_numpy(x).to(dev)
        y_dev = torch.empty((args.copies, N), dtype=torch.float32, device=dev)
        lib = tcrv_hip.load()
        fn = lib.tcrv_hip_gemv_q4_0_q8_0
        wp = [copies[i].data_ptr() for i in range(args.copies)]
        yp = [y_dev[i].data_ptr() for i in range(args.copies)]
        xp = x_dev.data_ptr()

        def gemv(i):
            k = i % args.copies
            st = fn(N, yp[k], wp[k], bx, xp, N, sptr)
            if st != 0:
                raise RuntimeError(tcrv_hip.status_string(st))

        with torch.cuda.stream(stream):
            log(f"GEMV warmup {args.warmup} ({args.mode})")
            run_region(torch, stream, gemv, args.warmup, args.mode)
            log(f"GEMV timed {args.steps} steps over {args.copies} weight copies")
            ms = run_region(torch, stream, gemv, args.steps, args.mode)
        ms_step = ms / args.steps
        gemv_bytes = wbytes + x.size + N * 4  # 9 457 920 B at 4096 x 4096
        gbs = gemv_bytes / (ms_step * 1e-3) / 1e9
        result["gemv"] = {"ms_per_step": ms_step, "bytes": gemv_bytes, "gbs": gbs}
        log(f"GEMV {ms_step * 1e3:.2f} us/step, {gbs:.0f} GB/s "
            f"({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")
        del copies, y_dev

    # ------------------------------------------------------------ GEMM ---
    if args.only in ("all", "gemm"):
        log("building GEMM inputs (A 4096 tokens Q8_0 seed 1008, B 4096x4096 Q8_0 seed 1009)")
        a = synth.q8_0_matrix(N, N, synth.SEEDS["gemm_a"], 1.0)
        b = synth.q8_0_matrix(N, N, synth.SEEDS["gemm_b"], 0.02)
        a_dev = torch.from_numpy(a).to(dev)
        b_dev = torch.from_numpy(b).to(dev)
        c_dev = torch.empty(N * N, dtype=torch.float32, device=dev)
        lib = tcrv_hip.load()
        gfn = lib.tcrv_hip_q8_0_q8_0_gemm
        ap_, bp_, cp_ = a_dev.data_ptr(), b_dev.data_ptr(), c_dev.data_ptr()
        rb = a.shape[1]

        def gemm(i):
            st = gfn(N, cp_, bp_, ap_, rb, N, N, rb, N, sptr)
            if st != 0:
                raise RuntimeError(tcrv_hip.status_string(st))

        with torch.cuda.stream(stream):
            run_region(torch, stream, gemm, 5, "eager")
            ms = run_region(torch, stream, gemm, args.gemm_steps, "eager")
        ms_step = ms / args.gemm_steps
        ops = 2.0 * N * N * N
        tops = ops / (ms_step * 1e-3) / 1e12
        result["gemm"] = {"ms_per_step": ms_step, "ops": ops, "tops": tops}
        log(f"GEMM {ms_step * 1e3:.1f} us/step, {tops:.1f} TOPS "
            f"({100 * tops / INT8_PEAK_TOPS:.1f}% of int8 peak)")
        del a_dev, b_dev, c_dev

    # ---------------------------------------------------- CPU baseline ---
    cpu = cpu_baseline(args, result)

    # --------------------------------------------------------- report ---
    traffic = load_traffic()
    line = {
        "metric": "Q4_0 GEMV GB/s (% HBM peak); Q8_0 GEMM int8 TOPS (% MFMA peak)",
        "higher_is_better": True,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0/q8_0 blocks, int32 block sums, f32 fold",
        "data": "synthetic: splitmix64 Box-Muller seeds 1006/1007 (GEMV), 1008/1009 (GEMM)",
        "config": {"workload": "gemv_q4_0_q8_0 4096x4096 (configs[3])", "rows": N, "cols": N,
                   "launch": args.mode, "weight_copies": args.copies},
    }
    if "gemv" in result:
        g = result["gemv"]
        line.update({
            "value": round(g["gbs"], 2), "unit": "GB/s",
            "ms_per_step": g["ms_per_step"],
            "roofline": {"bound": "hbm", "achieved": round(g["gbs"], 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": traffic.get("gemv_q4_0_q8_0")},
        })
    if "gemm" in result:
        m = result["gemm"]
        line["gemm"] = {
            "workload": "q8_0_q8_0_gemm 4096x4096x4096 (configs[4])",
            "value": round(m["tops"], 2), "unit": "TOPS", "ms_per_step": m["ms_per_step"],
            "steps": args.gemm_steps,
            "roofline": {"bound": "mfma", "achieved": round(m["tops"], 2),
                         "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                         "frac": round(m["tops"] / INT8_PEAK_TOPS, 4),
                         "traffic": traffic.get("q8_0_q8_0_gemm")},
        }
        if "gemv" not in result:
            line.update({"value": line["gemm"]["value"], "unit": "TOPS",
                         "ms_per_step": m["ms_per_step"]})
    line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return {}


def cpu_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        return max(1, int(env))
    return max(1, min(os.cpu_count() or 1, 16))


def cpu_baseline(args, result):
    """Times the scalar C oracle on the host on a bounded sample of the same
    workload.  The GEMV leg runs whole 4096x4096 GEMVs; the GEMM leg runs a
    64-row slice of the 4096^3 GEMM and scales by rows."""
    if args.cpu_seconds <= 0:
        return None
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_binding
    import synth

    ora = oracle_binding.load()
    threads = cpu_threads()
    out = {}
    if "gemv" in result:
        w = synth.q4_0_matrix(N, N, synth.SEEDS["gemv_w"], 0.02)
        x = synth.q8_0_matrix(1, N, synth.SEEDS["gemv_x"], 1.0).reshape(-1)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            ora.gemm_q4_0(N, w, x, 0, N, 1, w.shape[1], 1, threads)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        out["gemv_gbs"] = result["gemv"]["bytes"] / dt / 1e9
        out["gemv_reps"] = reps
        log(f"CPU GEMV oracle: {dt * 1e3:.2f} ms per 4096x4096 GEMV on {threads} threads")
    if "gemm" in result:
        rows = 64
        b = synth.q8_0_matrix(rows, N, synth.SEEDS["gemm_b"], 0.02)
        a = synth.q8_0_matrix(N, N, synth.SEEDS["gemm_a"], 1.0)
        t0 = time.perf_counter()
        ora.gemm_q8_0(N, b, a, a.shape[1], rows, N, b.shape[1], N, threads)
        dt = (time.perf_counter() - t0) * (N / rows)
        out["gemm_tops"] = 2.0 * N * N * N / dt / 1e12
        log(f"CPU GEMM oracle: 64-row slice -> {out['gemm_tops']:.4f} TOPS scaled to 4096 rows")
    primary = "gemv_gbs" if "gemv_gbs" in out else "gemm_tops"
    return {
        "value": round(out[primary], 4),
        "unit": "GB/s" if primary == "gemv_gbs" else "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": (f"scalar C oracle (gcc -O3, OpenMP over rows, fold serial per row) on "
                   f"{threads} host threads: whole 4096x4096 GEMVs repeated for "
                   f"{args.cpu_seconds:.0f} s; GEMM = 64-row slice of 4096^3 scaled x64"),
        "gemm_tops": round(out.get("gemm_tops", 0.0), 4) if "gemm_tops" in out else None,
    }


if __name__ == "__main__":
    main()
