"""GPU parity at the sizes where 32-bit indexing would break: more than 2^32
elements (add, dequant), more than 2^31 bytes in one operand (block dot rows,
GEMV).  Outputs are checked on sampled indices -- every sample against numpy or
the CPU oracle on the same bytes -- including the last elements, where an
index that wrapped would land."""
import numpy as np
import pytest
import torch

import synth
from gpu_util import assert_f32_parity

pytestmark = pytest.mark.gpu

BIG = (1 << 32) + 1031  # elements: past 2^32, and ragged for the 16-element vector path


def free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def sample_indices(n, k=4096, seed=0):
    rng = np.random.default_rng(seed)
    edges = np.concatenate([np.arange(64), np.arange(n - 2048, n),
                            (1 << 31) + np.arange(-8, 8), (1 << 32) + np.arange(-8, 8)])
    edges = edges[(edges >= 0) & (edges < n)]
    return np.unique(np.concatenate([edges, rng.integers(0, n, k)]))


def test_add_f32_beyond_2_pow_32(hip, dev):
    a = torch.rand(BIG, dtype=torch.float32, device=dev) * 2 - 1
    b = torch.rand(BIG, dtype=torch.float32, device=dev) * 2 - 1
    out = torch.empty(BIG, dtype=torch.float32, device=dev)
    hip.add_f32(a, b, out, BIG)
    idx = torch.from_numpy(sample_indices(BIG)).to(dev)
    av, bv, ov = (t[idx].cpu().numpy() for t in (a, b, out))
    del a, b, out
    free()
    assert np.array_equal(ov.view(np.uint32), (av + bv).view(np.uint32))


def test_dequantize_beyond_2_pow_32(hip, dev):
    nb = BIG // 32 + 1  # 134217761 blocks: 4.56 GB in, 17.2 GB out
    n = nb * 32
    vx = torch.randint(0, 256, (nb, 34), dtype=torch.uint8, device=dev)
    # finite, varied fp16 scales: exponent field 1..30, any mantissa and sign
    sc = torch.randint(0, 1 << 16, (nb,), dtype=torch.int32, device=dev)
    exp = (torch.remainder(sc >> 10, 30) + 1) << 10
    half = ((sc & 0x83FF) | exp).to(torch.int32)
    vx[:, 0] = (half & 0xFF).to(torch.uint8)
    vx[:, 1] = ((half >> 8) & 0xFF).to(torch.uint8)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    hip.dequantize_row_q8_0(vx, y, n)
    blocks = np.unique(np.concatenate([sample_indices(nb, 2048, 1), [nb - 1]]))
    bi = torch.from_numpy(blocks).to(dev)
    raw = vx[bi].cpu().numpy()
    got = y.view(nb, 32)[bi].cpu().numpy()
    del vx, y, sc, exp, half
    free()
    d = raw[:, :2].copy().view(np.float16).astype(np.float32)
    want = raw[:, 2:].view(np.int8).astype(np.float32) * d
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_q4_0_beyond_2_pow_32(hip, dev):
    nb = BIG // 32 + 1  # 134217761 blocks: 2.42 GB in, 17.2 GB out
    n = nb * 32
    vx = torch.randint(0, 256, (nb, 18), dtype=torch.uint8, device=dev)
    sc = torch.randint(0, 1 << 16, (nb,), dtype=torch.int32, device=dev)
    exp = (torch.remainder(sc >> 10, 30) + 1) << 10
    half = ((sc & 0x83FF) | exp).to(torch.int32)
    vx[:, 0] = (half & 0xFF).to(torch.uint8)
    vx[:, 1] = ((half >> 8) & 0xFF).to(torch.uint8)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    hip.dequantize_row_q4_0(vx, y, n)
    blocks = np.unique(np.concatenate([sample_indices(nb, 2048, 2), [nb - 1]]))
    bi = torch.from_numpy(blocks).to(dev)
    raw = vx[bi].cpu().numpy()
    got = y.view(nb, 32)[bi].cpu().numpy()
    del vx, y, sc, exp, half
    free()
    d = raw[:, :2].copy().view(np.float16).astype(np.float32)
    qs = raw[:, 2:].astype(np.int64)
    vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), (vals * d).view(np.uint32))


def test_q8_0_block_dot_rows_operands_over_2_gib(hip, oracle, dev):
    rows, nb = 520000, 128  # 2.26 GB per operand
    n = nb * 32
    rb = nb * 34
    base_x = synth.q8_0_matrix(64, n, 1004, 1.0)
    base_y = synth.q8_0_matrix(64, n, 1005, 1.0)
    # rows repeat a 64-row pattern shifted by the row index, so each sampled
    # row's bytes are known on the host
    dx = torch.from_numpy(base_x).to(dev)
    dy = torch.from_numpy(base_y).to(dev)
    vx = dx.repeat(rows // 64 + 1, 1)[:rows].contiguous()
    vy = dy.roll(7, 0).repeat(rows // 64 + 1, 1)[:rows].contiguous()
    s = torch.empty(rows, dtype=torch.float32, device=dev)
    hip.q8_0_q8_0_block_dot_rows(n, s, vx, rb, vy, rb, rows)
    got = s.cpu().numpy()
    del vx, vy, s
    free()
    pick = np.unique(np.concatenate([sample_indices(rows, 256, 2), [rows - 1]]))
    bx = base_x[pick % 64]
    by = np.roll(base_y, 7, 0)[pick % 64]
    want = oracle.vec_dot_q8_0_rows(n, bx, rb, by, rb, len(pick), 8)
    assert_f32_parity(got[pick], want, what="q8 rows over 2 GiB")


def test_gemv_weights_over_2_gib(hip, oracle, dev):
    nr, nb = 1000000, 128  # Q4_0 weights: 2.3 GB
    n = nb * 32
    rb = nb * 18
    base = synth.q4_0_matrix(96, n, 1006, 0.02)
    x = synth.q8_0_matrix(1, n, 1007, 1.0).reshape(-1)
    w = torch.from_numpy(base).to(dev).repeat(nr // 96 + 1, 1)[:nr].contiguous()
    s = torch.empty(nr, dtype=torch.float32, device=dev)
    hip.gemv_q4_0_q8_0(n, s, w, rb, torch.from_numpy(x).to(dev), nr)
    got = s.cpu().numpy()
    del w, s
    free()
    pick = np.unique(np.concatenate([sample_indices(nr, 256, 3), [nr - 1]]))
    want = oracle.gemm_q4_0(n, base[pick % 96], x, 0, len(pick), 1, rb, 1, 8)
    assert_f32_parity(got[pick], want, what="gemv over 2 GiB")


def test_gemm_output_beyond_2_pow_32(hip, oracle, dev):
    """The GEMM entries with an output of more than 2^32 elements (65600 x 65600 at a padded
    stride, 17.2 GB of fp32): the tiled kernels (through the workspace entries, Q8_0 and
    Q4_0 weights) and the plain Q8_0 entry, every output index formed in 64 bits.  K = 64
    keeps the work small; sampled rows, the last included, against the CPU oracle."""
    nr = nc = 65600
    nb = 2
    n = nb * 32
    bs = nc + 8
    assert (nr - 1) * bs + nc > 1 << 32
    w8 = synth.q8_0_matrix(nr, n, 1011, 0.02)
    w4 = synth.q4_0_matrix(nr, n, 1012, 0.02)
    a = synth.q8_0_matrix(nc, n, 1013, 1.0)
    rng = np.random.default_rng(9)
    pick = np.unique(np.concatenate([[0, 1, nr // 2, nr - 2, nr - 1], rng.integers(0, nr, 59)]))
    s = torch.empty(nr * bs, dtype=torch.float32, device=dev)
    da = torch.from_numpy(a).to(dev)
    rows = torch.from_numpy(pick).to(dev)
    for name, w, entry, ref in (
            ("q8_0 ws", w8, "q8_0_q8_0_gemm_ws", oracle.gemm_q8_0),
            ("q4_0 ws", w4, "q4_0_q8_0_gemm_ws", oracle.gemm_q4_0),
            ("q8_0 plain", w8, "q8_0_q8_0_gemm", oracle.gemm_q8_0)):
        dw = torch.from_numpy(w).to(dev)
        s.fill_(float("nan"))
        if entry.endswith("_ws"):
            wsb = getattr(hip, entry.replace("_ws", "_workspace_bytes"))(n, nr, nc)
            ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
            getattr(hip, entry)(n, s, dw, da, a.shape[1], nr, nc, w.shape[1], bs, ws, wsb)
            del ws
        else:
            getattr(hip, entry)(n, s, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
        got = s.view(nr, bs).index_select(0, rows).cpu().numpy()
        del dw
        want = ref(n, w[pick], a, a.shape[1], len(pick), nc, w.shape[1], bs, 8).reshape(len(pick), bs)
        assert_f32_parity(got[:, :nc], want[:, :nc], what=f"{name} gemm, output past 2^32")
        assert np.all(np.isnan(got[:, nc:])), f"{name}: a store past column nc"
    del s, da, rows
    free()


def test_gemm_tiled_operands_over_2_gib(hip, oracle, dev):
    """The workspace entries (both operands packed into the GEMM-tile layout, then the DMA-
    staged tiled kernel) with a packed weight operand past 2 GiB: 8192 weight rows x K 262144
    (2.28 GB of records), so the DMA sources, record offsets and chunk offsets all need 64
    bits.  Weight rows repeat a 96-row pattern (built on the device), so each sampled row's
    bytes are known on the host."""
    nr, nc, nb = 8192, 128, 8192
    n = nb * 32
    a = synth.q8_0_matrix(nc, n, 1015, 1.0)
    da = torch.from_numpy(a).to(dev)
    rng = np.random.default_rng(11)
    pick = np.unique(np.concatenate([[0, 95, 96, nr // 2, nr - 1], rng.integers(0, nr, 27)]))
    rows = torch.from_numpy(pick).to(dev)
    bs = nc + 4
    for name, base, entry, ref in (
            ("q8_0", synth.q8_0_matrix(96, n, 1016, 0.02), "q8_0_q8_0_gemm_ws", oracle.gemm_q8_0),
            ("q4_0", synth.q4_0_matrix(96, n, 1017, 0.02), "q4_0_q8_0_gemm_ws", oracle.gemm_q4_0)):
        dw = torch.from_numpy(base).to(dev).repeat(nr // 96 + 1, 1)[:nr].contiguous()
        wsb = getattr(hip, entry.replace("_ws", "_workspace_bytes"))(n, nr, nc)
        assert wsb > 1 << 31
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        s = torch.full((nr * bs,), float("nan"), dtype=torch.float32, device=dev)
        getattr(hip, entry)(n, s, dw, da, a.shape[1], nr, nc, base.shape[1], bs, ws, wsb)
        got = s.view(nr, bs).index_select(0, rows).cpu().numpy()
        del dw, ws, s
        free()
        want = ref(n, base[pick % 96], a, a.shape[1], len(pick), nc, base.shape[1], bs,
                   8).reshape(len(pick), bs)
        assert_f32_parity(got[:, :nc], want[:, :nc], what=f"{name} gemm_ws, operand past 2 GiB")
    del da, rows
    free()


@pytest.mark.parametrize("nb", [1973789, 1973790])
def test_q8_0_gemm_ws_at_the_tiled_block_bound(hip, oracle, dev, nb):
    """K at the workspace entry's bound (the 256-row tiled kernels' 32-bit DMA chunk offset):
    n/32 = 1 973 789 blocks (odd: no multi-column GEMV) is packed and runs the tiled kernel of
    this shape -- one 32 x 32 tile a wave, its last block's records 2 KB below 2^32 bytes into
    a group; one block more runs the plain GEMM.  256 weight rows x 2 tokens; every row repeats
    a 2048-block pattern along K (built on the device), so the sampled rows' bytes are known on
    the host."""
    nr, nc, pat = 256, 2, 2048
    n = nb * 32
    rb = nb * 34
    reps = -(-nb // pat)
    base_w = synth.q8_0_matrix(nr, pat * 32, 1031, 0.02)
    base_a = synth.q8_0_matrix(nc, pat * 32, 1032, 1.0)
    dw = torch.from_numpy(base_w).to(dev).repeat(1, reps)[:, :rb].contiguous()
    da = torch.from_numpy(base_a).to(dev).repeat(1, reps)[:, :rb].contiguous()
    wsb = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    s = torch.full((nr * nc,), float("nan"), dtype=torch.float32, device=dev)
    hip.q8_0_q8_0_gemm_ws(n, s, dw, da, rb, nr, nc, rb, nc, ws, wsb)
    got = s.view(nr, nc).cpu().numpy()
    del dw, da, ws, s
    free()
    pick = np.array([0, 1, 137, 255])
    w_rows = np.ascontiguousarray(np.tile(base_w[pick], (1, reps))[:, :rb])
    a_rows = np.ascontiguousarray(np.tile(base_a, (1, reps))[:, :rb])
    want = oracle.gemm_q8_0(n, w_rows, a_rows, rb, len(pick), nc, rb, nc, 8).reshape(len(pick), nc)
    assert_f32_parity(got[pick], want, what=f"q8_0 gemm_ws at nb = {nb}")
