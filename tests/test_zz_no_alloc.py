"""tcrv_hip_q8_0_q8_0_gemm_noalloc: tcrv_hip_q8_0_q8_0_gemm_ws with the
library's fixed device scratch as its workspace.  Checked against the
workspace entry bit for bit (and against the oracle), on two calls in a row,
the second smaller, so the second reads none of the first's leftovers."""
import numpy as np
import pytest
import torch

import synth
from gpu_util import assert_f32_parity, empty_dev, from_dev, to_dev

pytestmark = pytest.mark.gpu


def run_both(hip, dev, nr, nc, nb, xpad, ypad, seed):
    n = nb * 32
    w = np.pad(synth.q8_0_matrix(nr, n, seed, 0.02), ((0, 0), (0, xpad)))
    a = np.pad(synth.q8_0_matrix(nc, n, seed + 1, 1.0), ((0, 0), (0, ypad)))
    bs = nc + 5
    dw, da = to_dev(w, dev), to_dev(a, dev)
    wsb = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(max(wsb, 16), torch.uint8, dev)
    s_ws = to_dev(np.full(nr * bs, -3.0, np.float32), dev)
    s_na = to_dev(np.full(nr * bs, -3.0, np.float32), dev)
    hip.q8_0_q8_0_gemm_ws(n, s_ws, dw, da, a.shape[1], nr, nc, w.shape[1], bs, ws, wsb)
    hip.q8_0_q8_0_gemm_noalloc(n, s_na, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
    got, want = from_dev(s_na), from_dev(s_ws)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"noalloc differs from gemm_ws at {nr}x{nc}x{n}"
    return w, a, got.reshape(nr, bs), bs


def test_noalloc_matches_gemm_ws_on_two_calls_the_second_smaller(hip, oracle, dev):
    print("noalloc: 520 x 200 x K 1280, then 300 x 70 x K 288", flush=True)
    w, a, got, bs = run_both(hip, dev, 520, 200, 40, 6, 2, 1201)
    n = 40 * 32
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], 520, 200, w.shape[1], bs, 8).reshape(520, bs)
    assert_f32_parity(got[:, :200], want[:, :200], what="noalloc 520x200")
    assert np.all(got[:, 200:] == -3.0)
    w, a, got, bs = run_both(hip, dev, 300, 70, 9, 0, 4, 1203)
    n = 9 * 32
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], 300, 70, w.shape[1], bs, 8).reshape(300, bs)
    assert_f32_parity(got[:, :70], want[:, :70], what="noalloc 300x70")


def test_noalloc_shapes_without_workspace(hip, dev):
    """Shapes gemm_ws serves with the plain GEMM (nr < 256, decode) use no scratch."""
    for nr, nc, nb in ((100, 70, 8), (300, 1, 8)):
        print(f"noalloc fallback {nr} x {nc} x K {nb * 32}", flush=True)
        run_both(hip, dev, nr, nc, nb, 0, 0, 1205)


def test_noalloc_refuses_a_workspace_beyond_its_scratch(hip, dev):
    limit = hip.q8_0_q8_0_gemm_noalloc_max_bytes()
    assert limit == 64 << 20
    nr = nc = 4096
    nb = 241  # 2 x 64 groups x 241 blocks x 2176 B = 67.1 MB > 64 MiB
    n = nb * 32
    assert hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc) > limit
    assert hip.q8_0_q8_0_gemm_workspace_bytes(n - 32, nr, nc) <= limit
    # real buffers of the full size, so nothing could read out of bounds
    w = torch.zeros(nr * nb * 34, dtype=torch.uint8, device=dev)
    a = torch.zeros(nc * nb * 34, dtype=torch.uint8, device=dev)
    s = torch.full((nr * nc,), -3.0, dtype=torch.float32, device=dev)
    st = hip.q8_0_q8_0_gemm_noalloc(n, s, w, a, nb * 34, nr, nc, nb * 34, nc, check=False)
    assert st == hip.ERR_SCRATCH_LIMIT
    assert "scratch" in hip.status_string(st)
    torch.cuda.synchronize()
    assert bool(torch.all(s == -3.0))  # nothing was launched


def test_noalloc_under_graph_capture(hip, oracle, dev):
    """The callers it is for: a HIP graph captures the entry (after one eager
    call on the device, which looks up the scratch address); every replay,
    with eager work and synchronizations between replays, equals the eager
    result bit for bit."""
    nr, nc, nb = 300, 70, 9
    n = nb * 32
    w = synth.q8_0_matrix(nr, n, 1207, 0.02)
    a = synth.q8_0_matrix(nc, n, 1208, 1.0)
    dw, da = to_dev(w, dev), to_dev(a, dev)
    eager = empty_dev(nr * nc, torch.float32, dev)
    hip.q8_0_q8_0_gemm_noalloc(n, eager, dw, da, a.shape[1], nr, nc, w.shape[1], nc)
    torch.cuda.synchronize()
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    assert_f32_parity(from_dev(eager), want, what="noalloc eager")
    out = torch.full((nr * nc,), -3.0, dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            hip.q8_0_q8_0_gemm_noalloc(n, out, dw, da, a.shape[1], nr, nc, w.shape[1], nc,
                                       stream=stream)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(-3.0)
        # eager work between replays, on the same device's scratch
        hip.q8_0_q8_0_gemm_noalloc(n, eager, dw, da, a.shape[1], nr, nc, w.shape[1], nc)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32)), f"replay {rep}"
