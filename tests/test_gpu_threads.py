"""Several host threads, each with its own stream, output buffers and GEMM workspace, calling
the library at the same time.  The entries keep no mutable state between calls (the boundary
is reentrant, and calls on one stream run in order), so every thread's results equal a
single-threaded run's bit for bit.  ctypes releases the GIL for the duration of each call, so
the host side of the calls overlaps as well as the kernels."""
import threading

import numpy as np
import pytest
import torch

import synth
from gpu_util import to_dev

pytestmark = pytest.mark.gpu


def test_threads_on_their_own_streams_match_a_serial_run(hip, dev):
    nthreads, iters = 4, 6
    n = 4096
    nr_v = 4096
    nr, nc = 512, 130  # two tile rows, a partial token tile
    w = synth.q4_0_matrix(nr_v, n, 1021, 0.02)
    x = synth.q8_0_matrix(1, n, 1022, 1.0).reshape(-1)
    gw = synth.q8_0_matrix(nr, n, 1023, 0.02)
    ga = synth.q8_0_matrix(nc, n, 1024, 1.0)
    gw4 = synth.q4_0_matrix(nr, n, 1025, 0.02)
    dw, dx, dgw, dga, dgw4 = (to_dev(a, dev) for a in (w, x, gw, ga, gw4))
    ws8 = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws4 = hip.q4_0_q8_0_gemm_workspace_bytes(n, nr, nc)

    def run(st, ws_a, ws_b):
        v = torch.empty(nr_v, device=dev)
        g8 = torch.empty(nr * nc, device=dev)
        g4 = torch.empty(nr * nc, device=dev)
        hip.gemv_q4_0_q8_0(n, v, dw, w.shape[1], dx, nr_v, stream=st)
        hip.q8_0_q8_0_gemm_ws(n, g8, dgw, dga, ga.shape[1], nr, nc, gw.shape[1], nc, ws_a, ws8,
                              stream=st)
        hip.q4_0_q8_0_gemm_ws(n, g4, dgw4, dga, ga.shape[1], nr, nc, gw4.shape[1], nc, ws_b,
                              ws4, stream=st)
        return v, g8, g4

    ref_stream = torch.cuda.Stream()
    ref = run(ref_stream, torch.empty(ws8, dtype=torch.uint8, device=dev),
              torch.empty(ws4, dtype=torch.uint8, device=dev))
    ref_stream.synchronize()
    ref = [r.view(torch.int32).cpu() for r in ref]

    errors = []
    start = threading.Barrier(nthreads)

    def worker(t):
        try:
            st = torch.cuda.Stream()
            ws_a = torch.empty(ws8, dtype=torch.uint8, device=dev)
            ws_b = torch.empty(ws4, dtype=torch.uint8, device=dev)
            start.wait()
            outs = [run(st, ws_a, ws_b) for _ in range(iters)]
            st.synchronize()
            for i, out in enumerate(outs):
                for k, (got, want) in enumerate(zip(out, ref)):
                    if not torch.equal(got.view(torch.int32).cpu(), want):
                        errors.append(f"thread {t} call {i} output {k} differs")
        except Exception as e:  # reported below, with the thread that raised it
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nthreads)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    assert np.isfinite(ref[0].view(torch.float32).numpy()).all()
