#!/usr/bin/env python3
"""Benchmark of the quantized hot path on one MI355X.

BASELINE.json metric: "Q4_0 GEMV GB/s (% HBM peak); Q8_0 GEMM int8 TOPS (% MFMA
peak)".  `value` is the first half: the Q4_0 x Q8_0 decode GEMV, W 4096 x 4096
(configs[3]), through the C-ABI entry tcrv_hip_gemv_q4_0_q8_0.  One step is one
decode pass over a stack of LAYERS distinct 4096 x 4096 Q4_0 weight matrices
(the configs[3] matrix, copied): LAYERS GEMV launches, each reading its own
matrix, 605 MB per step -- more than the 256 MB Infinity Cache, so every launch
reads its weights from HBM whatever --steps is; the steps run in HIP graphs of
at most 32 steps, and the median of GEMV_REGIONS timed regions of --steps steps
is reported with its min and max.  The second half, the Q8_0 x Q8_0 GEMM 4096^3
(configs[4]) in the reference ABI through the workspace entry
tcrv_hip_q8_0_q8_0_gemm_ws, is timed in the same run and reported under "gemm"
beside the plain entry, pre-packed weights and the tiled kernel alone;
configs[0..2] (add, dequant, block dot) and the other kernels are reported
under "configs".

Timing: inputs are synthetic (tianchen-rv_amd/synth.py seeds) and resident in
HBM before a timed region starts.  A region is a HIP graph of launches,
replayed once untimed and then once between HIP events recorded on the launch
stream, bracketed by torch.cuda.synchronize(); per-launch time = region /
launches.  Every bandwidth-bound config rotates through enough distinct input
sets (> 256 MB, the Infinity Cache size) that each launch reads its inputs
from HBM, and times at least as many launches as it has sets.

cpu_baseline: the scalar C oracle (oracle/, the CPU restatement of the
reference emitters) timed on the host cores over a bounded sample of the same
GEMV workload, on all host threads and on one, with the host recorded.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tianchen-rv_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, published
N = 4096
MALL_BYTES = 256 << 20       # Infinity Cache
LAYERS = 64                  # GEMV launches (distinct weight matrices) per step: 605 MB
GEMV_REGIONS = 3             # timed regions of --steps steps each; the median is reported
HOST_COPIES = 48             # CPU-baseline GEMV weight copies (453 MB > host last-level cache)

METRIC = "Q4_0 GEMV GB/s (% HBM peak); Q8_0 GEMM int8 TOPS (% MFMA peak)"

# Algorithmic bytes per launch (the roofline's `achieved` numerators).
GEMV_BYTES = N * (N // 32) * 18 + (N // 32) * 34 + N * 4        # 9 457 920
ADD_BYTES = 12 * (1 << 24)                                      # 201 326 592
DEQ_BYTES = (N * N // 32) * (34 + 128)                          # 84 934 656
DEQ4_BYTES = (N * N // 32) * (18 + 128)                         # 76 546 048
DOT_ROWS = 16384
DOT_BYTES = DOT_ROWS * (2 * (N // 32) * 34 + 4)                 # 142 671 872
GEMM_OPS = 2.0 * N * N * N                                      # 137 438 953 472
PACK_BYTES = 2 * N * (N // 32) * 18                             # 18 874 368
REPACK8_BYTES = N * (N // 32) * 34 + (N // 32) * 34 + N * 4     # 17 846 528
BATCH_TOKENS = 4  # the batched-decode GEMM entries of `configs`
PREFILL_TOKENS = 128  # the short-prompt GEMM entries of `configs`
PREFILL_OPS = 2.0 * N * PREFILL_TOKENS * N                      # 4 294 967 296
QUANT_BYTES = N * N * 4 + (N * N // 32) * 34                    # 84 934 656


_INPUTS = {}


def inputs(name: str):
    """The synthetic host arrays, built once per process: the same bytes feed
    the GPU runs and the CPU baselines."""
    if name not in _INPUTS:
        import synth
        seeds = synth.SEEDS
        make = {
            "gemv_w": lambda: synth.q4_0_matrix(N, N, seeds["gemv_w"], 0.02),
            "gemv_x": lambda: synth.q8_0_matrix(1, N, seeds["gemv_x"], 1.0).reshape(-1),
            "gemm_a": lambda: synth.q8_0_matrix(N, N, seeds["gemm_a"], 1.0),
            "gemm_a_f32": lambda: synth.normal_f32(seeds["gemm_a"], N * N, 0.0, 1.0),
            "gemm_b": lambda: synth.q8_0_matrix(N, N, seeds["gemm_b"], 0.02),
            "add_a": lambda: synth.uniform_f32(seeds["add_a"], 1 << 24),
            "add_b": lambda: synth.uniform_f32(seeds["add_b"], 1 << 24),
            "dequant_q": lambda: synth.quantize_q8_0(
                synth.normal_f32(seeds["dequant_w"], N * N, 0.0, 0.02)),
            "dequant_q4": lambda: synth.quantize_q4_0(
                synth.normal_f32(seeds["dequant_w"], N * N, 0.0, 0.02)),
            "dot_x": lambda: synth.q8_0_matrix(DOT_ROWS, N, seeds["dot_x"], 1.0),
            "dot_y": lambda: synth.q8_0_matrix(DOT_ROWS, N, seeds["dot_y"], 1.0),
        }[name]
        _INPUTS[name] = make()
    return _INPUTS[name]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32,
                    help=f"timed GEMV steps (each {LAYERS} launches over distinct weights)")
    ap.add_argument("--warmup", type=int, default=4, help="untimed GEMV steps")
    ap.add_argument("--gemm-steps", type=int, default=20, help="GEMM launches per timed region")
    ap.add_argument("--gemm-regions", type=int, default=5,
                    help="timed GEMM regions; the median region is reported")
    ap.add_argument("--config-steps", type=int, default=50,
                    help="timed launches for each of add / dequant / block dot")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall time of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--only", choices=["all", "gemv", "gemv_rows", "gemm", "configs", "schedules",
                                       "calib"],
                    default="all",
                    help="calib: 10 launches of add_f32 over n = 2^24 (reads 128 MiB, writes "
                         "64 MiB each), the known-size kernel the HBM byte counters are "
                         "scaled against")
    return ap.parse_args()


class Region:
    """HIP events on the launch stream around one replay of a captured graph
    of `steps` launches; ms = region time."""

    def __init__(self, torch, stream, launch, steps):
        self.torch, self.stream = torch, stream
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(self.graph, stream=stream):
                for i in range(steps):
                    launch(i)
        torch.cuda.synchronize()

    def timed(self) -> float:
        """One untimed replay (first-replay costs stay out of the figure), then
        the timed one."""
        self.run()
        return self.run()

    def run(self) -> float:
        torch = self.torch
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        # replay() launches on torch's current stream: make it the launch stream
        # so the graph runs between the two events.
        with torch.cuda.stream(self.stream):
            e0.record(self.stream)
            self.graph.replay()
            e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)


def checked(fn, name):
    import tcrv_hip

    def call(*args):
        st = fn(*args)
        if st != 0:
            raise tcrv_hip.TcrvHipError(st, f"{name}: {tcrv_hip.status_string(st)}")
    return call


def same_as_eager(torch, stream, graph_out, eager_launch, what):
    """Guards the timing: the output a graph replay left behind must equal the
    output of one eager launch of the same step (so the graph really ran)."""
    ref = torch.empty_like(graph_out)
    with torch.cuda.stream(stream):
        eager_launch(ref.data_ptr())
    torch.cuda.synchronize()
    if not torch.equal(ref.view(torch.int32), graph_out.view(torch.int32)):
        raise RuntimeError(f"{what}: graph replay output differs from an eager launch")


def copies_for(nbytes: int, minimum: int = 2) -> int:
    """Rotating input sets for a kernel that moves nbytes per launch: at least
    2.5 x the Infinity Cache.  A rotation only 1.6 x it still hits: add_f32
    over 2 sets (403 MB) ran 27.8 us, over 3-8 sets (604 MB-1.6 GB) 34.5-34.7 us."""
    return max(minimum, -(-(MALL_BYTES * 5 // 2) // nbytes))


def bench_gemv(torch, lib, stream, args):
    """K steps of LAYERS GEMVs each, every launch over its own weight matrix;
    the graphs hold at most 32 steps (2048 launches) and are replayed back to
    back between one pair of events."""
    log("GEMV inputs: W 4096x4096 Q4_0 (seed 1006, N(0,0.02)), x Q8_0 (seed 1007, N(0,1))")
    w = inputs("gemv_w")
    x = inputs("gemv_x")
    dev = torch.device("cuda:0")
    copies = LAYERS
    assert copies * w.size > MALL_BYTES
    wd = torch.empty((copies, w.size), dtype=torch.uint8, device=dev)
    wd[:] = torch.from_numpy(w.reshape(-1)).to(dev)
    xd = torch.from_numpy(x).to(dev)
    yd = torch.empty((copies, N), dtype=torch.float32, device=dev)
    fn = checked(lib.tcrv_hip_gemv_q4_0_q8_0, "gemv")
    wp = [wd[i].data_ptr() for i in range(copies)]
    yp = [yd[i].data_ptr() for i in range(copies)]
    sp = stream.cuda_stream
    bx = w.shape[1]

    def launch(i):
        k = i % copies
        fn(N, yp[k], wp[k], bx, xd.data_ptr(), N, sp)

    if args.warmup > 0:
        Region(torch, stream, launch, args.warmup * LAYERS).run()
    steps = max(args.steps, 1)
    per_graph = min(steps, 32)
    full, rest = divmod(steps, per_graph)
    graphs = [(Region(torch, stream, launch, per_graph * LAYERS), full)]
    if rest:
        graphs.append((Region(torch, stream, launch, rest * LAYERS), 1))
    for g, _ in graphs:  # one untimed replay of each graph
        g.run()
    yd.zero_()
    region_ms = []
    for _ in range(GEMV_REGIONS):  # each region replays every graph once
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            e0.record(stream)
            for g, reps in graphs:
                for _ in range(reps):
                    g.graph.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        region_ms.append(e0.elapsed_time(e1))
    same_as_eager(torch, stream, yd[0], lambda out: fn(N, out, wp[0], bx, xd.data_ptr(), N, sp),
                  "GEMV")
    region_ms.sort()
    ms = region_ms[len(region_ms) // 2]
    launches = steps * LAYERS
    us = ms * 1e3 / launches
    gbs = GEMV_BYTES / (us * 1e-6) / 1e9
    log(f"GEMV {us:.3f} us/launch over {launches} launches ({steps} steps of {LAYERS} "
        f"weight matrices; median of {GEMV_REGIONS} regions, min "
        f"{region_ms[0] * 1e3 / launches:.3f}, max {region_ms[-1] * 1e3 / launches:.3f}): "
        f"{gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")
    return {"us": us, "gbs": gbs, "copies": copies, "ms_region": ms, "launches": launches,
            "steps": steps, "ms_per_step": ms / steps, "regions": GEMV_REGIONS,
            "us_min": region_ms[0] * 1e3 / launches, "us_max": region_ms[-1] * 1e3 / launches,
            "bytes_touched_per_step": copies * (w.size + N * 4) + x.size}


def bench_gemv_rows(torch, lib, stream, args):
    """The same GEMV kernel at more weight rows (K = 4096): the weight matrix
    is the 4096-row configs[3] matrix repeated, one launch per rotating copy.
    Past a few tens of MB the fixed cost of a launch (the launch itself and one
    short read) is amortised and the kernel's own streaming rate shows."""
    w = inputs("gemv_w")
    x = inputs("gemv_x")
    dev = torch.device("cuda:0")
    wt = torch.from_numpy(w).to(dev)
    xd = torch.from_numpy(x).to(dev)
    fn = checked(lib.tcrv_hip_gemv_q4_0_q8_0, "gemv")
    sp, bx = stream.cuda_stream, w.shape[1]
    out = {}
    for nr, steps in ((16384, 200), (65536, 100), (262144, 40)):
        rows_bytes = nr * bx
        copies = copies_for(rows_bytes, 2)
        wd = wt.repeat(copies * (nr // N), 1).view(copies, rows_bytes)
        yd = torch.empty((copies, nr), dtype=torch.float32, device=dev)
        wp = [wd[i].data_ptr() for i in range(copies)]
        yp = [yd[i].data_ptr() for i in range(copies)]

        def launch(i, nr=nr, wp=wp, yp=yp, copies=copies):
            k = i % copies
            fn(N, yp[k], wp[k], bx, xd.data_ptr(), nr, sp)

        Region(torch, stream, launch, max(steps // 4, 4)).run()
        ms = Region(torch, stream, launch, max(steps, copies)).timed()
        same_as_eager(torch, stream, yd[(steps - 1) % copies],
                      lambda o, nr=nr, k=(steps - 1) % copies, wp=wp:
                      fn(N, o, wp[k], bx, xd.data_ptr(), nr, sp), f"GEMV {nr} rows")
        us = ms * 1e3 / steps
        nbytes = rows_bytes + (N // 32) * 34 + nr * 4
        gbs = nbytes / (us * 1e-6) / 1e9
        log(f"GEMV {nr}x{N}: {us:.2f} us/launch, {gbs:.0f} GB/s "
            f"({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak), {copies} copies")
        out[str(nr)] = {"us": round(us, 3), "GB/s": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes, "copies": copies}
        del wd, yd
        torch.cuda.empty_cache()
    return out


SCHEDULE_SHAPES = ((4096, N), (2048, N))  # (weight rows, K) for the decode GEMV's knob


def bench_schedules(torch, lib, stream, args):
    """Every candidate of the schedule registry that an entry takes at run time
    (tcrv_hip_route_schedule rows with an entry: the decode GEMV's
    rows_per_wave through tcrv_hip_gemv_q4_0_q8_0_shaped), timed at the
    registry's reference shapes over rotating weight copies past the Infinity
    Cache, each candidate's output checked bit for bit against the plain
    entry's.  The route tests compare the registry's defaults with a recorded
    run of this (profiles/schedules.json)."""
    import tcrv_hip
    dev = torch.device("cuda:0")
    w = inputs("gemv_w")
    x = inputs("gemv_x")
    wt = torch.from_numpy(w).to(dev)
    xd = torch.from_numpy(x).to(dev)
    bx, sp = w.shape[1], stream.cuda_stream
    shaped = checked(lib.tcrv_hip_gemv_q4_0_q8_0_shaped, "gemv_shaped")
    plain = checked(lib.tcrv_hip_gemv_q4_0_q8_0, "gemv")
    out = []
    sched = [r for r in tcrv_hip.route_schedules() if r["entry"]]
    for nr, k in SCHEDULE_SHAPES:
        copies = copies_for(nr * bx, 2)
        wd = wt[:nr].reshape(1, -1).repeat(copies, 1)
        yd = torch.empty((copies, nr), dtype=torch.float32, device=dev)
        ref = torch.empty(nr, dtype=torch.float32, device=dev)
        with torch.cuda.stream(stream):
            plain(k, ref.data_ptr(), wd[0].data_ptr(), bx, xd.data_ptr(), nr, sp)
        torch.cuda.synchronize()
        for r in sched:
            v = int(r["value"])

            def launch(i, v=v):
                j = i % copies
                shaped(k, yd[j].data_ptr(), wd[j].data_ptr(), bx, xd.data_ptr(), nr, v, sp)

            steps = max(256, copies)
            Region(torch, stream, launch, steps).run()
            reg = Region(torch, stream, launch, steps)
            per = sorted(reg.run() * 1e3 / steps for _ in range(5))
            if not torch.equal(yd[0].view(torch.int32), ref.view(torch.int32)):
                raise RuntimeError(f"{r['knob']}={v}: output differs from the plain entry")
            out.append({"op": r["op"], "m_regime": r["m_regime"], "knob": r["knob"], "value": v,
                        "entry": r["entry"], "rows": nr, "k": k, "us": round(per[2], 4),
                        "us_min": round(per[0], 4), "us_max": round(per[-1], 4)})
            log(f"schedule {r['knob']}={v} at {nr}x{k}: {per[2]:.3f} us (min {per[0]:.3f})")
        del wd, yd
        torch.cuda.empty_cache()
    return out


def bench_gemm(torch, lib, stream, args):
    """The 4096^3 Q8_0 GEMM in the reference ABI through the workspace entry
    (both operands packed into the GEMM-tile layout, then the DMA-staged tiled
    kernel), beside the plain entry, the path with weights packed once (only
    the activations packed per call) and the tiled kernel alone (the roofline
    kernel).  Median of --gemm-regions regions of --gemm-steps launches each."""
    log("GEMM inputs: A 4096 tokens x 4096 Q8_0 (seed 1008, N(0,1)), "
        "B 4096x4096 Q8_0 (seed 1009, N(0,0.02))")
    a = inputs("gemm_a")
    b = inputs("gemm_b")
    dev = torch.device("cuda:0")
    ad = torch.from_numpy(a).to(dev)
    bd = torch.from_numpy(b).to(dev)
    cd = torch.empty(N * N, dtype=torch.float32, device=dev)
    rb, sp = a.shape[1], stream.cuda_stream
    nb = N // 32
    plain = checked(lib.tcrv_hip_q8_0_q8_0_gemm, "gemm")
    ws_fn = checked(lib.tcrv_hip_q8_0_q8_0_gemm_ws, "gemm_ws")
    pack = checked(lib.tcrv_hip_pack_q8_0_to_gemm_tiles, "pack_q8_0_to_gemm_tiles")
    tiles = checked(lib.tcrv_hip_q8_0_q8_0_gemm_tiles, "gemm_tiles")
    wsb = lib.tcrv_hip_q8_0_q8_0_gemm_workspace_bytes(N, N, N)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    txb = lib.tcrv_hip_gemm_tiles_bytes(N, nb)
    tx = torch.empty(txb, dtype=torch.uint8, device=dev)       # weights, packed once
    ty = torch.empty(wsb - txb, dtype=torch.uint8, device=dev)  # activations, per call
    with torch.cuda.stream(stream):
        pack(N, nb, bd.data_ptr(), rb, tx.data_ptr(), sp)
        pack(N, nb, ad.data_ptr(), rb, ty.data_ptr(), sp)
    torch.cuda.synchronize()

    # s[ir*bs + col]: ir = weight row (B), col = token (A)
    paths = {
        "gemm_ws": lambda out: ws_fn(N, out, bd.data_ptr(), ad.data_ptr(), rb, N, N, rb, N,
                                     ws.data_ptr(), wsb, sp),
        "plain": lambda out: plain(N, out, bd.data_ptr(), ad.data_ptr(), rb, N, N, rb, N, sp),
        "prepacked_weights": lambda out: (pack(N, nb, ad.data_ptr(), rb, ty.data_ptr(), sp),
                                          tiles(N, out, tx.data_ptr(), ty.data_ptr(), N, N, N,
                                                sp)),
        "tiles_kernel": lambda out: tiles(N, out, tx.data_ptr(), ty.data_ptr(), N, N, N, sp),
    }
    # ~50 launches (~10 ms of dense MFMA work) bring the clocks to their loaded
    # state before anything is timed
    Region(torch, stream, lambda i: paths["gemm_ws"](cd.data_ptr()), 50).run()
    res = {}
    for name, fn in paths.items():
        cd.zero_()
        timed = Region(torch, stream, lambda i, fn=fn: fn(cd.data_ptr()), args.gemm_steps)
        timed.run()  # untimed first replay
        per = sorted(timed.run() * 1e3 / args.gemm_steps for _ in range(args.gemm_regions))
        # the graph really ran, and every path writes what the plain entry writes
        same_as_eager(torch, stream, cd, paths["plain"], f"GEMM {name}")
        us = per[len(per) // 2]
        res[name] = {"us": us, "tops": GEMM_OPS / (us * 1e-6) / 1e12, "us_min": per[0],
                     "us_max": per[-1]}
        log(f"GEMM {name}: {us:.1f} us/launch (median of {len(per)} regions of "
            f"{args.gemm_steps}; min {per[0]:.1f}, max {per[-1]:.1f}): "
            f"{res[name]['tops']:.0f} TOPS ({100 * res[name]['tops'] / INT8_PEAK_TOPS:.1f}% of "
            f"dense int8 peak)")
    m = res["gemm_ws"]
    return {"us": m["us"], "tops": m["tops"], "us_min": m["us_min"], "us_max": m["us_max"],
            "regions": args.gemm_regions, "paths": res}


def bench_configs(torch, lib, stream, args):
    """configs[0..2]: add f32 2^24, Q8_0 dequant 4096x4096, Q8_0.Q8_0 block dot
    16384 x 4096 -- each over rotating input sets larger than the MALL -- plus
    the x16-repacked Q4_0 GEMV and the Q4_0 x Q8_0 prefill GEMM."""
    dev = torch.device("cuda:0")
    sp = stream.cuda_stream
    out = {}
    steps = args.config_steps

    # add
    n = 1 << 24
    sets = copies_for(12 * n, 2)
    a = torch.from_numpy(inputs("add_a")).to(dev)
    b = torch.from_numpy(inputs("add_b")).to(dev)
    A = torch.empty((sets, n), device=dev); A[:] = a
    B = torch.empty((sets, n), device=dev); B[:] = b
    C = torch.empty((sets, n), device=dev)
    fn = checked(lib.tcrv_hip_add_f32, "add")
    ptrs = [(A[i].data_ptr(), B[i].data_ptr(), C[i].data_ptr()) for i in range(sets)]
    reg = Region(torch, stream, lambda i: fn(*ptrs[i % sets], n, sp), steps)
    reg.run()
    us = reg.run() * 1e3 / steps
    out["add_f32"] = {"workload": "configs[0] add f32 n=2^24", "us": round(us, 3),
                      "GB/s": round(ADD_BYTES / us / 1e3, 1), "sets": sets}
    del A, B, C, a, b, reg

    # dequant
    nb = N * N // 32
    q = inputs("dequant_q")
    sets = copies_for(DEQ_BYTES, 2)
    Q = torch.empty((sets, q.size), dtype=torch.uint8, device=dev)
    Q[:] = torch.from_numpy(q).to(dev)
    Y = torch.empty((sets, nb * 32), device=dev)
    fn = checked(lib.tcrv_hip_dequantize_row_q8_0, "dequant")
    ptrs = [(Q[i].data_ptr(), Y[i].data_ptr()) for i in range(sets)]
    reg = Region(torch, stream, lambda i: fn(*ptrs[i % sets], N * N, sp), steps)
    reg.run()
    us = reg.run() * 1e3 / steps
    out["dequant_q8_0"] = {"workload": "configs[1] Q8_0 dequant 4096x4096", "us": round(us, 3),
                           "GB/s": round(DEQ_BYTES / us / 1e3, 1), "sets": sets}
    del Q, Y, reg

    # the Q4_0 block dequant of the same N(0, 0.02) values quantized to Q4_0
    # (d = max / -8): 18 B in and 128 B out per block
    q4 = inputs("dequant_q4")
    sets = copies_for(DEQ4_BYTES, 2)
    Q = torch.empty((sets, q4.size), dtype=torch.uint8, device=dev)
    Q[:] = torch.from_numpy(q4).to(dev)
    Y = torch.empty((sets, nb * 32), device=dev)
    fn = checked(lib.tcrv_hip_dequantize_row_q4_0, "dequant_q4")
    ptrs = [(Q[i].data_ptr(), Y[i].data_ptr()) for i in range(sets)]
    reg = Region(torch, stream, lambda i: fn(*ptrs[i % sets], N * N, sp), steps)
    reg.run()
    us = reg.run() * 1e3 / steps
    same_as_eager(torch, stream, Y[(steps - 1) % sets],
                  lambda o: fn(Q[(steps - 1) % sets].data_ptr(), o, N * N, sp), "dequant_q4")
    out["dequant_q4_0"] = {"workload": "a3b Q4_0 dequant 4096x4096 (the configs[1] values "
                                       "quantized to Q4_0)", "us": round(us, 3),
                           "GB/s": round(DEQ4_BYTES / us / 1e3, 1), "sets": sets,
                           "bytes_per_launch": DEQ4_BYTES}
    del Q, Y, reg

    # block dot
    xq = inputs("dot_x")
    yq = inputs("dot_y")
    sets = copies_for(DOT_BYTES, 2)
    X = torch.empty((sets, xq.size), dtype=torch.uint8, device=dev)
    X[:] = torch.from_numpy(xq.reshape(-1)).to(dev)
    Yd = torch.empty((sets, yq.size), dtype=torch.uint8, device=dev)
    Yd[:] = torch.from_numpy(yq.reshape(-1)).to(dev)
    S = torch.empty((sets, DOT_ROWS), device=dev)
    fn = checked(lib.tcrv_hip_q8_0_q8_0_block_dot_rows, "block_dot_rows")
    rb = xq.shape[1]
    ptrs = [(S[i].data_ptr(), X[i].data_ptr(), Yd[i].data_ptr()) for i in range(sets)]

    def dot(i):
        s_, x_, y_ = ptrs[i % sets]
        fn(N, s_, x_, rb, y_, rb, DOT_ROWS, sp)

    reg = Region(torch, stream, dot, max(steps // 2, 1))
    reg.run()
    us = reg.run() * 1e3 / max(steps // 2, 1)
    out["vec_dot_q8_0_q8_0"] = {"workload": "configs[2] Q8_0.Q8_0 block dot 16384 x 4096",
                                "us": round(us, 3), "GB/s": round(DOT_BYTES / us / 1e3, 1),
                                "sets": sets}
    del X, Yd, S, reg

    # x16 repacked decode GEMV (the reference's selected decode path at VLEN128)
    w = inputs("gemv_w")
    x = inputs("gemv_x")
    nb = N // 32
    src = torch.from_numpy(w.reshape(N // 16, 16, nb, 18).transpose(0, 2, 1, 3).copy()).to(dev)
    packed = torch.empty(N // 16 * nb * 288, dtype=torch.uint8, device=dev)
    checked(lib.tcrv_hip_pack_q4_0_to_q4_0x16, "pack")(N // 16 * nb, src.data_ptr(),
                                                        packed.data_ptr(), sp)
    sets = copies_for(packed.numel(), 2)
    P = torch.empty((sets, packed.numel()), dtype=torch.uint8, device=dev)
    P[:] = packed
    xd = torch.from_numpy(x).to(dev)
    Yv = torch.empty((sets, N), device=dev)
    fn = checked(lib.tcrv_hip_repack_gemv_q4_0_q8_0, "repack_gemv")
    ptrs = [(Yv[i].data_ptr(), P[i].data_ptr()) for i in range(sets)]
    reg = Region(torch, stream, lambda i: fn(N, ptrs[i % sets][0], ptrs[i % sets][1],
                                             xd.data_ptr(), N, sp), 500)
    reg.run()
    us = reg.run() * 1e3 / 500
    out["repack_gemv_q4_0_q8_0"] = {"workload": "a8 x16-repacked Q4_0 GEMV 4096x4096",
                                    "us": round(us, 3), "GB/s": round(GEMV_BYTES / us / 1e3, 1),
                                    "sets": sets}
    # the Q8_0 x16 GEMV (tcrv_rvv.repack_gemv_q8_0_q8_0) over the configs[4] weights
    w8 = inputs("gemm_b")
    src8 = torch.from_numpy(w8.reshape(N // 16, 16, nb, 34).transpose(0, 2, 1, 3).copy()).to(dev)
    packed8 = torch.empty(N // 16 * nb * 544, dtype=torch.uint8, device=dev)
    checked(lib.tcrv_hip_pack_q8_0_to_q8_0x16, "pack8")(N // 16 * nb, src8.data_ptr(),
                                                         packed8.data_ptr(), sp)
    sets8 = copies_for(packed8.numel(), 2)
    P8 = torch.empty((sets8, packed8.numel()), dtype=torch.uint8, device=dev)
    P8[:] = packed8
    fn8 = checked(lib.tcrv_hip_repack_gemv_q8_0_q8_0, "repack_gemv_q8")
    ptrs8 = [(Yv[i % sets].data_ptr(), P8[i].data_ptr()) for i in range(sets8)]
    reg = Region(torch, stream, lambda i: fn8(N, ptrs8[i % sets8][0], ptrs8[i % sets8][1],
                                              xd.data_ptr(), N, sp), 500)
    reg.run()
    us = reg.run() * 1e3 / 500
    out["repack_gemv_q8_0_q8_0"] = {"workload": "a8 x16-repacked Q8_0 GEMV 4096x4096 "
                                                "(configs[4] weights)",
                                    "us": round(us, 3),
                                    "GB/s": round(REPACK8_BYTES / us / 1e3, 1), "sets": sets8}
    del P8, src8, packed8, reg
    # the x16 pack of the same weights (read 9.4 MB, write 9.4 MB)
    src_all = torch.empty((sets, packed.numel()), dtype=torch.uint8, device=dev)
    src_all[:] = src.view(-1)
    fn = checked(lib.tcrv_hip_pack_q4_0_to_q4_0x16, "pack")
    ptrs = [(src_all[i].data_ptr(), P[i].data_ptr()) for i in range(sets)]
    reg = Region(torch, stream, lambda i: fn(N // 16 * nb, ptrs[i % sets][0], ptrs[i % sets][1],
                                             sp), 200)
    reg.run()
    us = reg.run() * 1e3 / 200
    same_as_eager(torch, stream, P[199 % sets],
                  lambda o: fn(N // 16 * nb, src_all[199 % sets].data_ptr(), o, sp), "pack")
    out["pack_q4_0_to_q4_0x16"] = {"workload": "a8 pack_q4_0_to_q4_0x16, 4096x4096 Q4_0 weights",
                                   "us": round(us, 3), "GB/s": round(PACK_BYTES / us / 1e3, 1),
                                   "sets": sets}
    del P, Yv, reg, src, packed, src_all

    # the decode GEMV over the split (SoA) layout of the same weights
    wd = torch.from_numpy(inputs("gemv_w")).to(dev)
    soa = torch.empty(N * nb * 18, dtype=torch.uint8, device=dev)
    checked(lib.tcrv_hip_pack_q4_0_to_soa, "pack_soa")(N, nb, wd.data_ptr(), nb * 18,
                                                      soa.data_ptr(), sp)
    sets = max(LAYERS, copies_for(soa.numel(), 2))
    S = torch.empty((sets, soa.numel()), dtype=torch.uint8, device=dev)
    S[:] = soa
    Yv = torch.empty((sets, N), device=dev)
    fn = checked(lib.tcrv_hip_gemv_q4_0_soa_q8_0, "gemv_soa")
    ptrs = [(Yv[i].data_ptr(), S[i].data_ptr()) for i in range(sets)]
    reg = Region(torch, stream, lambda i: fn(N, ptrs[i % sets][0], ptrs[i % sets][1],
                                             xd.data_ptr(), N, sp), 2000)
    reg.run()
    us = reg.run() * 1e3 / 2000
    same_as_eager(torch, stream, Yv[1999 % sets],
                  lambda o: fn(N, o, S[1999 % sets].data_ptr(), xd.data_ptr(), N, sp), "gemv_soa")
    out["gemv_q4_0_soa_q8_0"] = {"workload": "decode GEMV 4096x4096 over the split (SoA) Q4_0 layout",
                                 "us": round(us, 3), "GB/s": round(GEMV_BYTES / us / 1e3, 1),
                                 "sets": sets}
    del S, Yv, soa, wd, reg

    # batched decode: the a7 and a9 GEMMs with BATCH_TOKENS tokens (the
    # multi-column GEMVs), and the a9 GEMM with one token (the Q8_0 decode
    # GEMV), every launch over its own copy of the weights; bytes are the
    # weights, the tokens' rows and the outputs
    act = inputs("gemm_a")[:BATCH_TOKENS].copy()
    actd = torch.from_numpy(act).to(dev)
    for name, wsrc, entry_fn, nt, what in (
            ("q4_0_q8_0_gemm_4_tokens", inputs("gemv_w"), lib.tcrv_hip_q4_0_q8_0_gemm,
             BATCH_TOKENS,
             "a7 Q4_0 x Q8_0 GEMM 4096 weight rows x 4 tokens x 4096 (batched decode)"),
            ("q8_0_q8_0_gemm_4_tokens", inputs("gemm_b"), lib.tcrv_hip_q8_0_q8_0_gemm,
             BATCH_TOKENS,
             "a9 Q8_0 x Q8_0 GEMM 4096 weight rows x 4 tokens x 4096 (batched decode)"),
            ("q8_0_q8_0_gemv", inputs("gemm_b"), lib.tcrv_hip_q8_0_q8_0_gemm, 1,
             "a9 Q8_0 x Q8_0 GEMM 4096 weight rows x 1 token x 4096 (the Q8_0 decode GEMV)")):
        sets = copies_for(wsrc.size, 2)
        Wc = torch.empty((sets, wsrc.size), dtype=torch.uint8, device=dev)
        Wc[:] = torch.from_numpy(wsrc.reshape(-1)).to(dev)
        Cb = torch.empty((sets, N * nt), device=dev)
        fn = checked(entry_fn, name)
        bx = wsrc.shape[1]
        ptrs = [(Cb[i].data_ptr(), Wc[i].data_ptr()) for i in range(sets)]
        reg = Region(torch, stream,
                     lambda i, fn=fn, ptrs=ptrs, sets=sets, bx=bx, nt=nt: fn(
                         N, ptrs[i % sets][0], ptrs[i % sets][1], actd.data_ptr(), act.shape[1],
                         N, nt, bx, nt, sp), 400)
        reg.run()
        us = reg.run() * 1e3 / 400
        same_as_eager(torch, stream, Cb[399 % sets],
                      lambda o, fn=fn, bx=bx, k=399 % sets, nt=nt: fn(
                          N, o, Wc[k].data_ptr(), actd.data_ptr(), act.shape[1], N,
                          nt, bx, nt, sp), name)
        nbytes = wsrc.size + act.shape[1] * nt + N * nt * 4
        out[name] = {"workload": what, "us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                     "sets": sets}
        del Wc, Cb, reg

    # a short prompt: the a7 and a9 GEMMs with PREFILL_TOKENS tokens through the
    # plain entries (few output tiles: packed in LDS per work-group, one 32 x 32
    # tile a wave) and the workspace entries (packed per call, the same tile per
    # wave straight from the records), every launch over its own weight copy
    act = inputs("gemm_a")[:PREFILL_TOKENS].copy()
    actd = torch.from_numpy(act).to(dev)
    for quant, wsrc in (("q4_0", inputs("gemv_w")), ("q8_0", inputs("gemm_b"))):
        sets = copies_for(wsrc.size, 2)
        Wc = torch.empty((sets, wsrc.size), dtype=torch.uint8, device=dev)
        Wc[:] = torch.from_numpy(wsrc.reshape(-1)).to(dev)
        Cb = torch.empty((sets, N * PREFILL_TOKENS), device=dev)
        bx = wsrc.shape[1]
        plain = checked(getattr(lib, f"tcrv_hip_{quant}_q8_0_gemm"), f"{quant} prefill")
        ws_fn = checked(getattr(lib, f"tcrv_hip_{quant}_q8_0_gemm_ws"), f"{quant} prefill ws")
        wsb = getattr(lib, f"tcrv_hip_{quant}_q8_0_gemm_workspace_bytes")(N, N, PREFILL_TOKENS)
        wsp = torch.empty(wsb, dtype=torch.uint8, device=dev)
        ptrs = [(Cb[i].data_ptr(), Wc[i].data_ptr()) for i in range(sets)]
        calls = {
            f"{quant}_q8_0_gemm_128_tokens": lambda i: plain(
                N, ptrs[i % sets][0], ptrs[i % sets][1], actd.data_ptr(), act.shape[1], N,
                PREFILL_TOKENS, bx, PREFILL_TOKENS, sp),
            f"{quant}_q8_0_gemm_ws_128_tokens": lambda i: ws_fn(
                N, ptrs[i % sets][0], ptrs[i % sets][1], actd.data_ptr(), act.shape[1], N,
                PREFILL_TOKENS, bx, PREFILL_TOKENS, wsp.data_ptr(), wsb, sp)}
        for name, step in calls.items():
            reg = Region(torch, stream, step, 100)
            reg.run()
            us = sorted(reg.run() * 1e3 / 100 for _ in range(3))[1]
            same_as_eager(torch, stream, Cb[99 % sets],
                          lambda o, k=99 % sets: plain(N, o, Wc[k].data_ptr(), actd.data_ptr(),
                                                       act.shape[1], N, PREFILL_TOKENS, bx,
                                                       PREFILL_TOKENS, sp), name)
            out[name] = {"workload": f"{'a7 Q4_0' if quant == 'q4_0' else 'a9 Q8_0'} x Q8_0 GEMM "
                                     f"4096 weight rows x {PREFILL_TOKENS} tokens x 4096 "
                                     f"({'workspace entry' if '_ws_' in name else 'plain entry'})",
                         "us": round(us, 2), "TOPS": round(PREFILL_OPS / us / 1e6, 1),
                         "sets": sets}
        del Wc, Cb, wsp

    # a10 quantize_row_q8_0: 4096 activation rows x 4096 f32 -> Q8_0 (the prefill
    # GEMM's activation operand; read 64 MiB, write 17.8 MB)
    xf = torch.from_numpy(inputs("gemm_a_f32")).to(dev)
    sets = copies_for(QUANT_BYTES, 2)
    XF = torch.empty((sets, N * N), device=dev)
    XF[:] = xf
    QO = torch.empty((sets, N * N // 32 * 34), dtype=torch.uint8, device=dev)
    fn = checked(lib.tcrv_hip_quantize_row_q8_0, "quantize")
    ptrs = [(XF[i].data_ptr(), QO[i].data_ptr()) for i in range(sets)]
    reg = Region(torch, stream, lambda i: fn(N * N, ptrs[i % sets][0], ptrs[i % sets][1], sp),
                 steps)
    reg.run()
    us = reg.run() * 1e3 / steps
    out["quantize_row_q8_0"] = {"workload": "a10 quantize_row_q8_0, 4096 x 4096 f32 -> Q8_0",
                                "us": round(us, 3), "GB/s": round(QUANT_BYTES / us / 1e3, 1),
                                "sets": sets}
    del XF, QO, xf, reg

    # Q4_0 x Q8_0 prefill GEMM 4096^3 (MFMA)
    a = inputs("gemm_a")
    ad = torch.from_numpy(a).to(dev)
    wd = torch.from_numpy(w).to(dev)
    cd = torch.empty(N * N, device=dev)
    fn = checked(lib.tcrv_hip_q4_0_q8_0_gemm, "q4_gemm")
    def q4_gemm(i):
        fn(N, cd.data_ptr(), wd.data_ptr(), ad.data_ptr(), a.shape[1], N, N, w.shape[1], N, sp)

    Region(torch, stream, q4_gemm, 50).run()  # loaded clocks, as for the Q8_0 GEMM
    reg = Region(torch, stream, q4_gemm, 10)
    reg.run()
    per = sorted(reg.run() * 1e3 / 10 for _ in range(3))
    us = per[1]
    out["q4_0_q8_0_gemm"] = {"workload": "a7 Q4_0 x Q8_0 GEMM 4096 rows x 4096 tokens x 4096",
                             "us": round(us, 1), "TOPS": round(GEMM_OPS / us / 1e6, 1),
                             "regions": 3}
    # the same GEMM over the GEMM-tile layout: the reference ABI with a workspace
    # (both operands packed per call), Q4_0 weights packed once (outside the
    # timed region) with the activations packed per call, and the tiled kernel
    # alone; each checked against one eager launch of the plain entry
    nb = N // 32
    tx4 = torch.empty(lib.tcrv_hip_gemm_tiles_bytes(N, nb), dtype=torch.uint8, device=dev)
    ty4 = torch.empty(lib.tcrv_hip_gemm_tiles_bytes(N, nb), dtype=torch.uint8, device=dev)
    wsb4 = lib.tcrv_hip_q4_0_q8_0_gemm_workspace_bytes(N, N, N)
    ws4 = torch.empty(wsb4, dtype=torch.uint8, device=dev)
    pack_w = checked(lib.tcrv_hip_pack_q4_0_to_gemm_tiles, "pack_q4_0_to_gemm_tiles")
    pack_a = checked(lib.tcrv_hip_pack_q8_0_to_gemm_tiles, "pack_q8_0_to_gemm_tiles")
    tiles4 = checked(lib.tcrv_hip_q4_0_q8_0_gemm_tiles, "q4_0_q8_0_gemm_tiles")
    ws_fn4 = checked(lib.tcrv_hip_q4_0_q8_0_gemm_ws, "q4_0_q8_0_gemm_ws")
    with torch.cuda.stream(stream):
        pack_w(N, nb, wd.data_ptr(), w.shape[1], tx4.data_ptr(), sp)
        pack_a(N, nb, ad.data_ptr(), a.shape[1], ty4.data_ptr(), sp)
    torch.cuda.synchronize()
    q4_paths = {
        "q4_0_q8_0_gemm_ws": (
            "a7 Q4_0 x Q8_0 GEMM 4096^3 through tcrv_hip_q4_0_q8_0_gemm_ws (the reference ABI): "
            "per call both operands packed into the workspace (one launch) + the tiled kernel",
            lambda i: ws_fn4(N, cd.data_ptr(), wd.data_ptr(), ad.data_ptr(), a.shape[1], N, N,
                             w.shape[1], N, ws4.data_ptr(), wsb4, sp)),
        "q4_0_q8_0_gemm_prepacked_weights": (
            "a7 Q4_0 x Q8_0 GEMM 4096^3, Q4_0 weights pre-packed into the GEMM-tile layout; "
            "per call: pack the Q8_0 activations + the tiled kernel",
            lambda i: (pack_a(N, nb, ad.data_ptr(), a.shape[1], ty4.data_ptr(), sp),
                       tiles4(N, cd.data_ptr(), tx4.data_ptr(), ty4.data_ptr(), N, N, N, sp))),
        "q4_0_q8_0_gemm_tiles_kernel": (
            "a7 Q4_0 x Q8_0 GEMM 4096^3, the tiled kernel alone (both operands pre-packed)",
            lambda i: tiles4(N, cd.data_ptr(), tx4.data_ptr(), ty4.data_ptr(), N, N, N, sp)),
    }
    for name, (what, step) in q4_paths.items():
        cd.zero_()
        reg = Region(torch, stream, step, 10)
        reg.run()
        per = sorted(reg.run() * 1e3 / 10 for _ in range(3))
        same_as_eager(torch, stream, cd, lambda o: fn(N, o, wd.data_ptr(), ad.data_ptr(),
                                                      a.shape[1], N, N, w.shape[1], N, sp),
                      name)
        out[name] = {"workload": what, "us": round(per[1], 1),
                     "TOPS": round(GEMM_OPS / per[1] / 1e6, 1), "regions": 3}
    del tx4, ty4, ws4
    # the repack GEMM over the same weights (x16) and activations (x4), 4096^3
    nb = N // 32
    srcw = torch.from_numpy(w.reshape(N // 16, 16, nb, 18).transpose(0, 2, 1, 3).copy()).to(dev)
    wx16 = torch.empty(N // 16 * nb * 288, dtype=torch.uint8, device=dev)
    checked(lib.tcrv_hip_pack_q4_0_to_q4_0x16, "pack")(N // 16 * nb, srcw.data_ptr(),
                                                        wx16.data_ptr(), sp)
    ax4 = torch.empty(N // 4 * nb * 136, dtype=torch.uint8, device=dev)
    checked(lib.tcrv_hip_pack_q8_0_to_q8_0x4, "pack_x4")(N, nb, ad.data_ptr(), a.shape[1],
                                                          ax4.data_ptr(), sp)
    del srcw
    fn = checked(lib.tcrv_hip_repack_gemm_q4_0_q8_0, "repack_gemm")

    def rp_gemm(i):
        fn(N, cd.data_ptr(), wx16.data_ptr(), ax4.data_ptr(), N, N, N, sp)

    Region(torch, stream, rp_gemm, 50).run()
    reg = Region(torch, stream, rp_gemm, 10)
    reg.run()
    per = sorted(reg.run() * 1e3 / 10 for _ in range(3))
    us = per[1]
    out["repack_gemm_q4_0_q8_0"] = {"workload": "a8 repack GEMM: x16 Q4_0 weights 4096 x x4 "
                                                "Q8_0 activations 4096 x K 4096",
                                    "us": round(us, 1), "TOPS": round(GEMM_OPS / us / 1e6, 1),
                                    "regions": 3}
    for k, v in out.items():
        if "GB/s" in v:
            v["roofline"] = {"bound": "hbm", "achieved": v["GB/s"], "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(v["GB/s"] / HBM_PEAK_GBS, 4)}
            log(f"{k}: {v['us']:.1f} us, {v['GB/s']:.0f} GB/s "
                f"({100 * v['GB/s'] / HBM_PEAK_GBS:.1f}% of HBM peak)")
        else:
            v["roofline"] = {"bound": "mfma", "achieved": v["TOPS"], "peak": INT8_PEAK_TOPS,
                             "unit": "TOPS", "frac": round(v["TOPS"] / INT8_PEAK_TOPS, 4)}
            log(f"{k}: {v['us']:.1f} us, {v['TOPS']:.0f} TOPS "
                f"({100 * v['TOPS'] / INT8_PEAK_TOPS:.1f}% of dense int8 peak)")
    return out


ORACLE_BUILD = ("gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp, every fold an explicit "
                "fmaf in the reference order (the bits -ffp-contract=on gives for the "
                "reference's one-expression folds)")


def host_cpu():
    """The host's CPU facts and the thread count the baselines use:
    OMP_NUM_THREADS when set (the GPU box sets it to the host-CPU share of one
    GPU, 16), else every CPU this process may run on."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = int(omp) if omp and omp.isdigit() and int(omp) > 0 else aff
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"threads": threads, "nproc": os.cpu_count(), "affinity_cpus": aff,
            "omp_num_threads": omp, "cpu_model": model, "build": ORACLE_BUILD}


def cpu_threads() -> int:
    return host_cpu()["threads"]


def split_run(pool, calls):
    """Runs the calls (oracle slices: ctypes releases the GIL) on the pool and
    waits for all of them."""
    for f in [pool.submit(c) for c in calls]:
        f.result()


def slices(total: int, parts: int):
    step = -(-total // parts)
    return [(i, min(i + step, total)) for i in range(0, total, step)]


def cpu_baseline(seconds: float):
    """The scalar C oracle (the CPU restatement of the reference's emitters) on
    the host: whole 4096x4096 Q4_0 x Q8_0 GEMVs repeated for `seconds`, OpenMP
    over rows (each row's fold stays serial, so results equal the 1-thread
    run), plus a 1-thread figure over a quarter of the time."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_binding

    import numpy as np

    ora = oracle_binding.load()
    threads = cpu_threads()
    w = inputs("gemv_w")
    x = inputs("gemv_x")
    # rotating weight copies, 453 MB in all: more than the host's last-level
    # cache, as the GPU's copies exceed its Infinity Cache
    ws = np.ascontiguousarray(np.broadcast_to(w, (HOST_COPIES,) + w.shape))

    def rate(nt, budget):
        reps, t0 = 0, time.perf_counter()
        while True:
            ora.gemm_q4_0(N, ws[reps % HOST_COPIES], x, 0, N, 1, w.shape[1], 1, nt)
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= budget:
                return GEMV_BYTES * reps / dt / 1e9, reps

    one, reps1 = rate(1, seconds / 4)
    many, reps = rate(threads, seconds)
    cpu = host_cpu()
    log(f"CPU oracle GEMV: {many:.1f} GB/s on {threads} threads, {one:.2f} GB/s on 1 "
        f"({cpu['cpu_model']}, nproc {cpu['nproc']}, affinity {cpu['affinity_cpus']})")
    return {
        "value": round(many, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"oracle/ scalar C, OpenMP over rows with a serial fmaf fold per row: {reps} "
                   f"whole 4096x4096 Q4_0xQ8_0 GEMVs over {HOST_COPIES} rotating weight copies "
                   f"in {seconds:.0f} s on {threads} threads of {cpu['cpu_model']}; "
                   f"1 thread: {one:.3f} GB/s ({reps1} GEMVs)"),
        "value_1thread": round(one, 4), "host": cpu,
    }


def cpu_baseline_gemm(seconds: float):
    """The oracle's Q8_0 x Q8_0 GEMM on the host, for the GEMM object: slices
    of 16 weight rows x all 4096 tokens x K 4096 (1/256 of the GEMM each),
    repeated for `seconds` on all threads (OpenMP over rows, serial fold)."""
    import synth
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_binding

    ora = oracle_binding.load()
    threads = cpu_threads()
    rows = 16
    a = inputs("gemm_a")
    b = synth.q8_0_matrix(rows, N, synth.SEEDS["gemm_b"], 0.02)
    reps, t0 = 0, time.perf_counter()
    while True:
        ora.gemm_q8_0(N, b, a, a.shape[1], rows, N, b.shape[1], N, threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    tops = 2.0 * rows * N * N * reps / dt / 1e12
    log(f"CPU oracle GEMM: {tops * 1e3:.1f} GOPS on {threads} threads")
    return {"value": round(tops, 5), "unit": "TOPS", "cores": threads, "kind": "port",
            "host": host_cpu(),
            "sample": (f"oracle/ scalar C, OpenMP over rows: {reps} slices of {rows} weight rows "
                       f"x 4096 tokens x 4096 (1/256 of the GEMM each) in {dt:.1f} s")}


def cpu_baseline_configs(seconds: float):
    """The oracle on the host beside each of configs[0..2] and the other
    kernels, each timed for `seconds` on a bounded sample of its workload, on
    one thread and on all the baseline's threads (row-parallel oracles use
    OpenMP over rows with every row's fold serial; element-wise ones run one
    contiguous slice per thread)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_binding

    ora = oracle_binding.load()
    threads = cpu_threads()
    pool = ThreadPoolExecutor(max_workers=threads)

    def timed(call):
        reps, t0 = 0, time.perf_counter()
        while True:
            call()
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= seconds:
                return reps, dt

    def entry(work, unit, sample, one, many):
        """one/many: callables doing one whole sample on 1 / all threads."""
        r1, d1 = timed(one)
        rn, dn = timed(many)
        return {"value": round(work * rn / dn / (1e9 if unit == "GB/s" else 1e12), 4),
                "unit": unit, "cores": threads, "kind": "port",
                "value_1thread": round(work * r1 / d1 / (1e9 if unit == "GB/s" else 1e12), 4),
                "sample": f"{sample}; {rn} on {threads} threads in {dn:.1f} s, {r1} on 1 "
                          f"thread in {d1:.1f} s"}

    out = {}
    a = inputs("add_a")
    b = inputs("add_b")
    n = a.size
    out["add_f32"] = entry(
        ADD_BYTES, "GB/s", "whole adds of n = 2^24", lambda: ora.add_f32(a, b),
        lambda: split_run(pool, [lambda i=i, j=j: ora.add_f32(a[i:j], b[i:j])
                                 for i, j in slices(n, threads)]))
    q = inputs("dequant_q")
    nbq = N * N // 32
    out["dequant_q8_0"] = entry(
        DEQ_BYTES, "GB/s", "whole 4096x4096 dequants", lambda: ora.dequantize_row_q8_0(q, N * N),
        lambda: split_run(pool, [lambda i=i, j=j: ora.dequantize_row_q8_0(q[34 * i:34 * j],
                                                                         32 * (j - i))
                                 for i, j in slices(nbq, threads)]))
    q4 = inputs("dequant_q4")
    out["dequant_q4_0"] = entry(
        DEQ4_BYTES, "GB/s", "whole 4096x4096 Q4_0 dequants",
        lambda: ora.dequantize_row_q4_0(q4, N * N),
        lambda: split_run(pool, [lambda i=i, j=j: ora.dequantize_row_q4_0(q4[18 * i:18 * j],
                                                                         32 * (j - i))
                                 for i, j in slices(nbq, threads)]))
    xq = inputs("dot_x")
    yq = inputs("dot_y")
    rb = xq.shape[1]
    out["vec_dot_q8_0_q8_0"] = entry(
        DOT_BYTES, "GB/s", "whole 16384 x 4096 block dots (143 MB each), OpenMP over rows",
        lambda: ora.vec_dot_q8_0_rows(N, xq, rb, yq, rb, DOT_ROWS, 1),
        lambda: ora.vec_dot_q8_0_rows(N, xq, rb, yq, rb, DOT_ROWS, threads))
    w = inputs("gemv_w")
    x = inputs("gemv_x")
    nb = N // 32
    src = w.reshape(N // 16, 16, nb, 18).transpose(0, 2, 1, 3).copy().reshape(-1)
    packed = ora.pack_q4_0x16(src, N // 16 * nb)
    ps = np.ascontiguousarray(np.broadcast_to(packed, (HOST_COPIES,) + packed.shape))
    k = [0]
    gb = nb * 288  # bytes per 16-row group

    def repack_one():
        ora.repack_gemv_q4_0(N, ps[k[0] % HOST_COPIES], x, N)
        k[0] += 1

    def repack_many():
        p = ps[k[0] % HOST_COPIES]
        split_run(pool, [lambda i=i, j=j: ora.repack_gemv_q4_0(N, p[gb * i:gb * j], x, 16 * (j - i))
                         for i, j in slices(N // 16, threads)])
        k[0] += 1
    out["repack_gemv_q4_0_q8_0"] = entry(
        GEMV_BYTES, "GB/s", f"whole 4096x4096 x16 GEMVs over {HOST_COPIES} rotating weight "
        "copies (threads split the 16-row groups)", repack_one, repack_many)
    del ps
    w8 = inputs("gemm_b")
    packed8 = ora.pack_q8_0x16(
        w8.reshape(N // 16, 16, nb, 34).transpose(0, 2, 1, 3).copy().reshape(-1), N // 16 * nb)
    copies8 = HOST_COPIES // 2
    ps8 = np.ascontiguousarray(np.broadcast_to(packed8, (copies8,) + packed8.shape))
    k8 = [0]
    gb8 = nb * 544

    def repack8_one():
        ora.repack_gemv_q8_0(N, ps8[k8[0] % copies8], x, N)
        k8[0] += 1

    def repack8_many():
        p = ps8[k8[0] % copies8]
        split_run(pool, [lambda i=i, j=j: ora.repack_gemv_q8_0(N, p[gb8 * i:gb8 * j], x,
                                                               16 * (j - i))
                         for i, j in slices(N // 16, threads)])
        k8[0] += 1
    out["repack_gemv_q8_0_q8_0"] = entry(
        REPACK8_BYTES, "GB/s", f"whole 4096x4096 Q8_0 x16 GEMVs over {copies8} rotating weight "
        "copies", repack8_one, repack8_many)
    del ps8
    nx16 = N // 16 * nb
    out["pack_q4_0_to_q4_0x16"] = entry(
        PACK_BYTES, "GB/s", "packs of the 4096x4096 Q4_0 weights",
        lambda: ora.pack_q4_0x16(src, nx16),
        lambda: split_run(pool, [lambda i=i, j=j: ora.pack_q4_0x16(src[288 * i:288 * j], j - i)
                                 for i, j in slices(nx16, threads)]))
    xf = inputs("gemm_a_f32")
    out["quantize_row_q8_0"] = entry(
        QUANT_BYTES, "GB/s", "quantizations of 4096 x 4096 f32", lambda: ora.quantize_q8_0(xf),
        lambda: split_run(pool, [lambda i=i, j=j: ora.quantize_q8_0(xf[32 * i:32 * j])
                                 for i, j in slices(N * N // 32, threads)]))
    a8 = inputs("gemm_a")
    w16 = w[:16].copy()
    out["q4_0_q8_0_gemm"] = entry(
        2.0 * 16 * N * N, "TOPS", "slices of 16 weight rows x 4096 tokens x 4096 (1/256 of the "
        "GEMM each), OpenMP over the 16 weight rows",
        lambda: ora.gemm_q4_0(N, w16, a8, a8.shape[1], 16, N, w16.shape[1], N, 1),
        lambda: ora.gemm_q4_0(N, w16, a8, a8.shape[1], 16, N, w16.shape[1], N, threads))
    # batched decode: the whole 4096-row GEMMs with BATCH_TOKENS tokens, OpenMP
    # over the weight rows (each output's fold serial)
    act = a8[:BATCH_TOKENS].copy()
    w8 = inputs("gemm_b")
    for name, wsrc, gemm, nt in (("q4_0_q8_0_gemm_4_tokens", w, ora.gemm_q4_0, BATCH_TOKENS),
                                 ("q8_0_q8_0_gemm_4_tokens", w8, ora.gemm_q8_0, BATCH_TOKENS),
                                 ("q8_0_q8_0_gemv", w8, ora.gemm_q8_0, 1)):
        nbytes = wsrc.size + act.shape[1] * nt + N * nt * 4
        out[name] = entry(
            nbytes, "GB/s", f"whole 4096 x {nt} x 4096 GEMMs over one weight copy (the "
            "host's caches hold it), OpenMP over weight rows",
            lambda wsrc=wsrc, gemm=gemm, nt=nt: gemm(N, wsrc, act[:nt].copy(), act.shape[1], N,
                                                     nt, wsrc.shape[1], nt, 1),
            lambda wsrc=wsrc, gemm=gemm, nt=nt: gemm(N, wsrc, act[:nt].copy(), act.shape[1], N,
                                                     nt, wsrc.shape[1], nt, threads))
    # a short prompt: slices of 64 weight rows x 128 tokens (1/64 of the GEMM),
    # OpenMP over the 64 rows
    act128 = a8[:PREFILL_TOKENS].copy()
    for name, wsrc, gemm in (("q4_0_q8_0_gemm_128_tokens", w, ora.gemm_q4_0),
                             ("q8_0_q8_0_gemm_128_tokens", w8, ora.gemm_q8_0)):
        w64 = wsrc[:64].copy()
        out[name] = entry(
            2.0 * 64 * PREFILL_TOKENS * N, "TOPS", "slices of 64 weight rows x 128 tokens x "
            "4096 (1/64 of the GEMM each), OpenMP over the 64 weight rows",
            lambda w64=w64, gemm=gemm: gemm(N, w64, act128, act128.shape[1], 64, PREFILL_TOKENS,
                                            w64.shape[1], PREFILL_TOKENS, 1),
            lambda w64=w64, gemm=gemm: gemm(N, w64, act128, act128.shape[1], 64, PREFILL_TOKENS,
                                            w64.shape[1], PREFILL_TOKENS, threads))
    wx16 = ora.pack_q4_0x16(src, nx16)
    ax4s = [ora.pack_q8_0x4(a8[16 * t:16 * t + 16].copy(), 16, nb, a8.shape[1])
            for t in range(threads)]
    out["repack_gemm_q4_0_q8_0"] = entry(
        2.0 * 16 * N * N, "TOPS", "slices of 16 activation rows x 4096 weight rows x 4096 "
        "(1/256 of the GEMM), one slice per thread",
        lambda: ora.repack_gemm_q4_0(N, wx16, ax4s[0], 16, N, N),
        lambda: split_run(pool, [lambda t=t: ora.repack_gemm_q4_0(N, wx16, ax4s[t], 16, N, N)
                                 for t in range(threads)]))
    # the all-thread repack GEMM sample does `threads` slices per call
    out["repack_gemm_q4_0_q8_0"]["value"] = round(out["repack_gemm_q4_0_q8_0"]["value"] * threads,
                                                  4)
    pool.shutdown()
    host = host_cpu()
    for v in out.values():
        v["host"] = host
    log("CPU oracle configs: " + ", ".join(f"{k} {v['value']} {v['unit']} "
                                           f"({v['value_1thread']} on 1 thread)"
                                           for k, v in out.items()))
    return out


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return {}


def device_peaks(torch):
    """The GPU's CU count and top shader clock (rocminfo, run as a child
    process) and the int8 MFMA peak they imply at 8192 int8 ops per clock and
    CU, next to the published figure used for `frac`."""
    props = torch.cuda.get_device_properties(0)
    out = {"name": props.name, "arch": props.gcnArchName, "cus": props.multi_processor_count,
           "max_sclk_mhz": None, "int8_tops_derived": None, "int8_tops_published": INT8_PEAK_TOPS,
           "hbm_gbs_published": HBM_PEAK_GBS}
    try:
        import subprocess
        text = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        return out
    for agent in text.split("Agent ")[1:]:
        fields = {}
        for ln in agent.splitlines():
            if ":" in ln:
                k, v = ln.split(":", 1)
                fields.setdefault(k.strip(), v.strip())
        if fields.get("Device Type") == "GPU":
            try:
                mhz, cus = int(fields["Max Clock Freq. (MHz)"]), int(fields["Compute Unit"])
            except (KeyError, ValueError):
                break
            out.update({"max_sclk_mhz": mhz, "cus_rocminfo": cus,
                        "int8_tops_derived": round(cus * mhz * 1e6 * 8192 / 1e12, 1)})
            break
    return out


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each config "
              "would shard by output rows, with no exchange but an all-gather of the "
              "output).  Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import tcrv_hip

    lib = tcrv_hip.load()
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    if args.only == "calib":
        n = 1 << 24
        a = torch.rand(n, device="cuda:0")
        b = torch.rand(n, device="cuda:0")
        c = torch.empty(n, device="cuda:0")
        fn = checked(lib.tcrv_hip_add_f32, "add")
        for _ in range(10):
            fn(a.data_ptr(), b.data_ptr(), c.data_ptr(), n, stream.cuda_stream)
        torch.cuda.synchronize()
        print(json.dumps({"calib": "add_f32", "n": n, "read_bytes": 8 * n, "write_bytes": 4 * n}))
        return
    res = {}
    if args.only in ("all", "gemv"):
        res["gemv"] = bench_gemv(torch, lib, stream, args)
    if args.only in ("all", "gemv_rows"):
        res["gemv_rows"] = bench_gemv_rows(torch, lib, stream, args)
    if args.only in ("all", "gemm"):
        res["gemm"] = bench_gemm(torch, lib, stream, args)
    if args.only in ("all", "configs"):
        res["configs"] = bench_configs(torch, lib, stream, args)
    if args.only in ("all", "schedules"):
        res["schedules"] = bench_schedules(torch, lib, stream, args)
    cpu = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 else None
    cpu_gemm = (cpu_baseline_gemm(args.cpu_seconds / 2)
                if args.cpu_seconds > 0 and "gemm" in res else None)
    traffic = load_traffic()

    g = res.get("gemv", {})
    line = {
        "metric": METRIC,
        "higher_is_better": True,
        "n_gpus": 1,
        "steps": g.get("steps", args.steps),
        "warmup": args.warmup,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "arith": "int8 block quants (q4_0 / q8_0) -> exact int32 block sums -> fp32 fold in the "
                 "reference order",
        "data": "synthetic: splitmix64 Box-Muller, seeds 1001-1009 (tianchen-rv_amd/synth.py)",
        "config": {"workload": f"gemv_q4_0_q8_0 W 4096x4096 Q4_0 x Q8_0 vector (configs[3]); "
                               f"one step = {LAYERS} GEMVs over {LAYERS} distinct weight "
                               f"matrices (a decode pass), 605 MB > the 256 MB Infinity Cache",
                   "rows": N, "cols": N, "launches_per_step": LAYERS,
                   "launches_timed": g.get("launches"),
                   "launch": "HIP graphs of up to 32 steps, each replayed once untimed first; "
                             "the median of 3 timed regions, each replaying every graph once",
                   "us_min": round(g["us_min"], 4) if "us_min" in g else None,
                   "us_max": round(g["us_max"], 4) if "us_max" in g else None,
                   "bytes_touched_per_step": g.get("bytes_touched_per_step")},
    }
    traffic_src = ("stored figure from profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE and "
                   "WRITE_SIZE per dispatch, scaled by the add_f32 calibration); not measured "
                   "in this run")
    if "gemv" in res:
        line.update({
            "value": round(g["gbs"], 2), "unit": "GB/s", "ms_per_step": g["ms_per_step"],
            "roofline": {"bound": "hbm", "achieved": round(g["gbs"], 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": traffic.get("gemv_q4_0_q8_0", {}).get("bytes"),
                         "traffic_source": traffic_src,
                         "kernel": "gemv_q4_0_q8_0_direct",
                         "bytes_per_launch": GEMV_BYTES,
                         "us_per_launch": round(g["us"], 4)},
        })
    if "gemm" in res:
        m = res["gemm"]
        k = m["paths"]["tiles_kernel"]
        line["gemm"] = {
            "workload": "q8_0_q8_0_gemm 4096 weight rows x 4096 tokens x 4096 (configs[4]) in "
                        "the reference ABI through tcrv_hip_q8_0_q8_0_gemm_ws: both operands "
                        "packed into the GEMM-tile layout, then the tiled kernel, every launch",
            "value": round(m["tops"], 2), "unit": "TOPS", "ms_per_step": m["us"] / 1e3,
            "steps": args.gemm_steps, "regions": m["regions"], "cpu_baseline": cpu_gemm,
            "us_min": round(m["us_min"], 2), "us_max": round(m["us_max"], 2),
            "paths": {name: {"us": round(v["us"], 2), "TOPS": round(v["tops"], 2),
                             "us_min": round(v["us_min"], 2), "us_max": round(v["us_max"], 2)}
                      for name, v in m["paths"].items()},
            "paths_note": "gemm_ws = the value; plain = tcrv_hip_q8_0_q8_0_gemm (no workspace); "
                          "prepacked_weights = weights packed once, activations packed per "
                          "call; tiles_kernel = the tiled kernel alone on packed operands",
            "roofline": {"bound": "mfma", "achieved": round(k["tops"], 2),
                         "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                         "frac": round(k["tops"] / INT8_PEAK_TOPS, 4),
                         "traffic": traffic.get("q8_0_q8_0_gemm_tiles", {}).get("bytes"),
                         "traffic_source": traffic_src,
                         "kernel": "tcrv::gemm_tiles256_q8", "ops_per_launch": GEMM_OPS,
                         "us_per_launch": round(k["us"], 2)},
        }
        if "gemv" not in res:
            line.update({"value": line["gemm"]["value"], "unit": "TOPS",
                         "ms_per_step": line["gemm"]["ms_per_step"]})
    if "gemv_rows" in res:
        line["gemv_rows"] = {
            "workload": "gemv_q4_0_q8_0 at more weight rows, K 4096 (the configs[3] matrix "
                        "repeated); same kernel as `value`", "by_rows": res["gemv_rows"]}
    if "configs" in res:
        if args.cpu_seconds > 0:
            for k, v in cpu_baseline_configs(max(0.5, args.cpu_seconds / 10)).items():
                res["configs"][k]["cpu_baseline"] = v
            soa = res["configs"].get("gemv_q4_0_soa_q8_0")
            if soa is not None and cpu is not None:
                # the split layout holds the same blocks: the CPU path for this
                # workload is the oracle's plain GEMV timed for the headline
                soa["cpu_baseline"] = dict(cpu, sample="the headline GEMV's (same workload, "
                                                       "plain layout): " + cpu["sample"])
        line["configs"] = res["configs"]
        if "value" not in line:
            first = next(iter(res["configs"].values()))
            line.update({"value": first["GB/s"], "unit": "GB/s", "ms_per_step": first["us"] / 1e3})
    if "schedules" in res:
        line["schedules"] = res["schedules"]
        if "value" not in line:
            first = res["schedules"][0]
            line.update({"value": first["us"], "unit": "us", "higher_is_better": False,
                         "ms_per_step": first["us"] / 1e3})
    line["cpu_baseline"] = cpu
    if args.only == "all":
        line["device"] = device_peaks(torch)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
