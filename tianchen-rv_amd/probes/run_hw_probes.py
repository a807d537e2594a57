#!/usr/bin/env python3
"""Runs the hardware probes (hw_probes.hip, built by `make -C tianchen-rv_amd probes`)
on cuda:0 and prints one line per measurement."""
import ctypes
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libtcrv_probes.so")


def graph_us(stream, launch, n=1000, reps=5):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for _ in range(n):
                launch()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / n)
    return best


def main():
    if not os.path.exists(LIB):
        sys.exit(f"{LIB} missing: run `make -C tianchen-rv_amd probes`")
    lib = ctypes.CDLL(LIB)
    lib.probe_mix.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                              ctypes.c_int, ctypes.c_void_p]
    lib.probe_empty.argtypes = [ctypes.c_void_p]
    lib.probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                               ctypes.c_void_p]
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    inp = torch.randint(-100, 100, (4096,), dtype=torch.int32, device=dev)
    grid, iters = 256, 4000
    out = torch.empty(grid * 512, device=dev)
    names = ["MFMA only (2 x i8 32x32x32 per iteration)", "VALU only (64 x v_fma_f32)",
             "both in every wave", "waves 0-3 MFMA, waves 4-7 VALU"]
    for mode, name in enumerate(names):
        assert lib.probe_mix(mode, inp.data_ptr(), out.data_ptr(), 10, grid, sp) == 0
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            assert lib.probe_mix(mode, inp.data_ptr(), out.data_ptr(), iters, grid, sp) == 0
            e1.record(stream)
        torch.cuda.synchronize()
        print(f"mix mode {mode} ({name}): {e0.elapsed_time(e1):.3f} ms "
              f"[{grid} x 512 threads, {iters} iterations]", flush=True)
    lib.probe_fold.argtypes = lib.probe_mix.argtypes
    fold_out = torch.empty(256 * 1024, device=dev)
    fold_iters = 2000
    fold_names = ["full GEMM inner loop", "MFMAs only (i8 + 2-block f32)", "i8 MFMA only",
                  "VALU only: xor + cvt + fma per element, 48 per tile-block"]
    for mode, name in enumerate(fold_names):
        assert lib.probe_fold(mode, inp.data_ptr(), fold_out.data_ptr(), 10, 256, sp) == 0
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            assert lib.probe_fold(mode, inp.data_ptr(), fold_out.data_ptr(), fold_iters, 256,
                                  sp) == 0
            e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        tile_blocks = 4 * fold_iters * 8  # per SIMD: 4 waves x iterations x 8 blocks
        print(f"fold mode {mode} ({name}): {ms:.3f} ms = {ms * 1e6 / tile_blocks:.2f} ns per "
              f"32x32 tile and block per SIMD [256 x 1024 threads, {fold_iters} x 8 blocks]",
              flush=True)
    # the shader clock while the GEMM inner loop runs: one wave's clock64 cycles
    # over its wall_clock64 ticks (a constant 100 MHz counter on this part)
    lib.probe_fold_clock.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    clk = torch.zeros(2, dtype=torch.int64, device=dev)
    assert lib.probe_fold_clock(inp.data_ptr(), fold_out.data_ptr(), clk.data_ptr(),
                                fold_iters, 256, sp) == 0
    torch.cuda.synchronize()
    cycles, ticks = (int(v) for v in clk.cpu())
    print(f"shader clock in the GEMM inner loop: {cycles / ticks * 0.1:.2f} GHz ({cycles} cycles "
          f"over {ticks} ticks of the 100 MHz wall clock, wave 0 of work-group 0)", flush=True)
    print(f"empty kernel, graph of 1000: {graph_us(stream, lambda: lib.probe_empty(sp)):.2f} "
          f"us per launch", flush=True)
    nbytes = 9437184
    copies = 40
    bufs = torch.empty((copies, nbytes), dtype=torch.uint8, device=dev)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    for grid in (576, 1024, 2304):
        k = [0]

        def launch():
            lib.probe_read(bufs[k[0] % copies].data_ptr(), nbytes, sink.data_ptr(), grid, sp)
            k[0] += 1
        us = graph_us(stream, launch)
        print(f"read-only {nbytes} B over {copies} rotating buffers, grid {grid} x 256: "
              f"{us:.2f} us per launch ({nbytes / us / 1e3:.0f} GB/s)", flush=True)
    del bufs
    torch.cuda.empty_cache()
    # the streaming-read roofline at the block dot's size (configs[2] reads
    # 142 606 336 B per launch), over 3 rotating buffers (> 256 MB MALL)
    lib.probe_read_wide.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_void_p]
    nbytes, copies = 142606336, 3
    bufs = torch.empty((copies, nbytes), dtype=torch.uint8, device=dev)
    for unroll in (1, 2, 4):
        k = [0]

        def launch():
            assert lib.probe_read_wide(bufs[k[0] % copies].data_ptr(), nbytes, sink.data_ptr(),
                                       unroll, sp) == 0
            k[0] += 1
        us = graph_us(stream, launch, n=60)
        print(f"read-wide {nbytes} B over {copies} rotating buffers, {unroll} x 16 B per thread: "
              f"{us:.2f} us per launch ({nbytes / us / 1e3:.0f} GB/s)", flush=True)


if __name__ == "__main__":
    main()
