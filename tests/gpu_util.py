"""Small helpers for the GPU parity tests (device copies, bit comparisons)."""
import numpy as np


def to_dev(a: np.ndarray, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def empty_dev(shape, dtype, dev):
    import torch
    return torch.empty(shape, dtype=dtype, device=dev)


def from_dev(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_f32_parity(got: np.ndarray, want: np.ndarray, rtol: float = 1e-5, what: str = ""):
    """The bar: within rtol AND bit-identical, since
    every kernel reproduces the reference fold order with the same fmaf."""
    got = np.asarray(got, dtype=np.float32).reshape(-1)
    want = np.asarray(want, dtype=np.float32).reshape(-1)
    assert got.shape == want.shape, (got.shape, want.shape)
    denom = np.maximum(np.abs(want), np.float32(1e-30))
    rel = np.abs(got.astype(np.float64) - want) / denom
    bad = np.flatnonzero(rel > rtol)
    assert bad.size == 0, (f"{what}: {bad.size} elements beyond rtol {rtol}; first at "
                           f"{bad[0]}: got {got[bad[0]]!r} want {want[bad[0]]!r}")
    diff = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert diff.size == 0, (f"{what}: {diff.size} elements not bit-identical; first at "
                            f"{diff[0]}: got {got[diff[0]]!r} want {want[diff[0]]!r}")


def assert_f32_parity_nan(got: np.ndarray, want: np.ndarray, what: str = ""):
    """Bit-identical outside NaNs; NaN exactly where the oracle has NaN.  The
    payload of a NaN is not part of the contract: a RISC-V FPU returns the
    canonical NaN where x86 and the GPU propagate an input's payload."""
    got = np.asarray(got, dtype=np.float32).reshape(-1)
    want = np.asarray(want, dtype=np.float32).reshape(-1)
    assert got.shape == want.shape, (got.shape, want.shape)
    gn, wn = np.isnan(got), np.isnan(want)
    bad = np.flatnonzero(gn != wn)
    assert bad.size == 0, (f"{what}: NaN pattern differs at {bad.size} elements; first at "
                           f"{bad[0]}: got {got[bad[0]]!r} want {want[bad[0]]!r}")
    ok = ~wn
    diff = np.flatnonzero(got[ok].view(np.uint32) != want[ok].view(np.uint32))
    assert diff.size == 0, (f"{what}: {diff.size} elements not bit-identical; first: got "
                            f"{got[ok][diff[0]]!r} want {want[ok][diff[0]]!r}")


def q4_tiles_gemm(hip, dev, n, w, a, nr, nc, bs, s):
    """The Q4_0 x Q8_0 GEMM through the GEMM-tile layout: both operands packed
    (tcrv_hip_pack_q4_0_to_gemm_tiles, tcrv_hip_pack_q8_0_to_gemm_tiles), then
    tcrv_hip_q4_0_q8_0_gemm_tiles into the device buffer s."""
    import torch
    nb = n // 32
    tx = empty_dev(hip.gemm_tiles_bytes(nr, nb), torch.uint8, dev)
    ty = empty_dev(hip.gemm_tiles_bytes(nc, nb), torch.uint8, dev)
    hip.pack_q4_0_to_gemm_tiles(nr, nb, to_dev(w, dev), w.shape[1], tx)
    hip.pack_q8_0_to_gemm_tiles(nc, nb, to_dev(a, dev), a.shape[1], ty)
    hip.q4_0_q8_0_gemm_tiles(n, s, tx, ty, nr, nc, bs)
    return s
