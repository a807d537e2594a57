"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): the CPU oracle must still reproduce them, their
integer block sums must match a numpy brute force, and (-m gpu) every kernel
must reproduce them byte for byte through the C-ABI."""
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ["add", "quant", "dequant_q4", "dot_q8", "dot_q4", "gemm_q8", "gemm_q4", "repack", "repack_gemm"]


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def same_f32_nan_as_nan(got, want):
    """Bit-equal, except that a NaN matches any NaN (a NaN's sign and payload
    are the arithmetic unit's, e.g. 0 * inf gives x86's negative default NaN)."""
    nan = np.isnan(want)
    return (np.array_equal(np.isnan(got), nan)
            and np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)))


def test_fixtures_present():
    for name in NAMES:
        assert os.path.exists(os.path.join(HERE, f"{name}.npz")), name


def test_oracle_reproduces_fixtures(oracle):
    g = load("add")
    assert np.array_equal(bits(oracle.add_f32(g["a"], g["b"])), bits(g["out"]))
    assert np.array_equal(oracle.add_i32(g["ai"], g["bi"]), g["outi"])
    g = load("quant")
    assert np.array_equal(oracle.quantize_q8_0(g["x"]), g["q"])
    assert np.array_equal(bits(oracle.dequantize_row_q8_0(g["q"], g["x"].size)), bits(g["deq"]))
    g = load("dequant_q4")
    assert np.array_equal(bits(oracle.dequantize_row_q4_0(g["q"], int(g["n"]))), bits(g["deq"]))
    for name, f in (("dot_q8", oracle.vec_dot_q8_0_rows), ("dot_q4", oracle.vec_dot_q4_0_rows)):
        g = load(name)
        n, vx, vy = int(g["n"]), g["vx"], g["vy"]
        got = f(n, vx, vx.shape[1], vy, vy.shape[1], vx.shape[0])
        assert np.array_equal(bits(got), bits(g["s"])), name
    g = load("gemm_q8")
    n, w, a = int(g["n"]), g["w"], g["a"]
    got = oracle.gemm_q8_0(n, w, a, a.shape[1], w.shape[0], a.shape[0], w.shape[1], a.shape[0])
    assert np.array_equal(bits(got), bits(g["s"]))
    g = load("gemm_q4")
    n, w, a = int(g["n"]), g["w"], g["a"]
    got = oracle.gemm_q4_0(n, w, a, a.shape[1], w.shape[0], a.shape[0], w.shape[1], a.shape[0])
    assert np.array_equal(bits(got), bits(g["s"]))
    g = load("repack")
    n = int(g["n"])
    nblk = g["p4"].size // 288
    assert np.array_equal(oracle.pack_q4_0x16(g["src4"], nblk), g["p4"])
    assert np.array_equal(oracle.pack_q8_0x16(g["src8"], nblk), g["p8"])
    assert np.array_equal(bits(oracle.repack_gemv_q4_0(n, g["p4"], g["act"], 32)), bits(g["s4"]))
    assert np.array_equal(bits(oracle.repack_gemv_q8_0(n, g["p8"], g["act"], 32)), bits(g["s8"]))
    g = load("repack_gemm")
    n = int(g["n"])
    a = g["act"]
    assert np.array_equal(oracle.pack_q8_0x4(a, 8, n // 32, a.shape[1]), g["ax4"])
    assert np.array_equal(bits(oracle.repack_gemm_q4_0(n, g["p4"], g["ax4"], 8, 32, 32)),
                          bits(g["s"]))


def test_fixture_dequant_q4_closed_form():
    # (nibble - 8) * d by numpy, element j the low nibble of byte j and
    # element 16 + j its high nibble; the trailing partial block is dropped
    g = load("dequant_q4")
    b = g["q"].reshape(-1, 18)
    assert g["deq"].size == (int(g["n"]) // 32) * 32 == b.shape[0] * 32
    d = b[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    qs = b[:, 2:].astype(np.int64)
    vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1).astype(np.float32)
    with np.errstate(invalid="ignore"):
        want = (vals * d[:, None]).reshape(-1)
    assert same_f32_nan_as_nan(g["deq"], want)
    assert np.isnan(g["deq"]).any() and np.isinf(g["deq"]).any()


def test_fixture_block_sums_brute_force():
    g = load("dot_q8")
    vx = g["vx"].reshape(4, -1, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    vy = g["vy"].reshape(4, -1, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    assert np.array_equal((vx * vy).sum(axis=2), g["sumi"])
    assert g["sumi"][0, 0] == 32 * 128 * 128
    g = load("dot_q4")
    qs = g["vx"].reshape(8, -1, 18)[:, :, 2:].astype(np.int64)
    w = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=2)
    y = g["vy"].reshape(8, -1, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    assert np.array_equal((w * y).sum(axis=2), g["sumi"])


@pytest.mark.gpu
def test_kernels_reproduce_fixtures(hip, dev):
    import torch
    from gpu_util import empty_dev, from_dev, to_dev

    g = load("add")
    out = empty_dev(g["a"].size, torch.float32, dev)
    hip.add_f32(to_dev(g["a"], dev), to_dev(g["b"], dev), out, g["a"].size)
    assert np.array_equal(bits(from_dev(out)), bits(g["out"]))
    outi = empty_dev(g["ai"].size, torch.int32, dev)
    hip.add_i32(to_dev(g["ai"], dev), to_dev(g["bi"], dev), outi, g["ai"].size)
    assert np.array_equal(from_dev(outi), g["outi"])

    g = load("quant")
    q = empty_dev(g["q"].size, torch.uint8, dev)
    hip.quantize_row_q8_0(g["x"].size, to_dev(g["x"], dev), q)
    assert np.array_equal(from_dev(q), g["q"])
    y = empty_dev(g["x"].size, torch.float32, dev)
    hip.dequantize_row_q8_0(to_dev(g["q"], dev), y, g["x"].size)
    assert np.array_equal(bits(from_dev(y)), bits(g["deq"]))

    g = load("dequant_q4")
    y = empty_dev(g["deq"].size, torch.float32, dev)
    hip.dequantize_row_q4_0(to_dev(g["q"], dev), y, int(g["n"]))
    assert same_f32_nan_as_nan(from_dev(y), g["deq"])

    for name, f in (("dot_q8", hip.q8_0_q8_0_block_dot_rows),
                    ("dot_q4", hip.q4_0_q8_0_block_dot_rows)):
        g = load(name)
        n, vx, vy = int(g["n"]), g["vx"], g["vy"]
        s = empty_dev(vx.shape[0], torch.float32, dev)
        f(n, s, to_dev(vx, dev), vx.shape[1], to_dev(vy, dev), vy.shape[1], vx.shape[0])
        assert np.array_equal(bits(from_dev(s)), bits(g["s"])), name
        sums = empty_dev(g["sumi"].size, torch.int32, dev)
        sf = hip.q8_0_q8_0_block_sums if name == "dot_q8" else hip.q4_0_q8_0_block_sums
        sf(n, sums, to_dev(vx, dev), vx.shape[1], to_dev(vy, dev), vy.shape[1], vx.shape[0])
        assert np.array_equal(from_dev(sums).reshape(g["sumi"].shape), g["sumi"]), name

    for name, f in (("gemm_q8", hip.q8_0_q8_0_gemm), ("gemm_q4", hip.q4_0_q8_0_gemm)):
        g = load(name)
        n, w, a = int(g["n"]), g["w"], g["a"]
        nr, nc = w.shape[0], a.shape[0]
        s = empty_dev(nr * nc, torch.float32, dev)
        f(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], nc)
        assert np.array_equal(bits(from_dev(s)), bits(g["s"])), name
    g = load("gemm_q4")
    s = empty_dev(g["w"].shape[0], torch.float32, dev)
    hip.gemv_q4_0_q8_0(int(g["n"]), s, to_dev(g["w"], dev), g["w"].shape[1],
                       to_dev(g["a"][0], dev), g["w"].shape[0])
    assert np.array_equal(bits(from_dev(s)), bits(g["gemv"]))

    g = load("repack")
    n = int(g["n"])
    nblk = g["p4"].size // 288
    p4 = empty_dev(g["p4"].size, torch.uint8, dev)
    hip.pack_q4_0_to_q4_0x16(nblk, to_dev(g["src4"], dev), p4)
    assert np.array_equal(from_dev(p4), g["p4"])
    p8 = empty_dev(g["p8"].size, torch.uint8, dev)
    hip.pack_q8_0_to_q8_0x16(nblk, to_dev(g["src8"], dev), p8)
    assert np.array_equal(from_dev(p8), g["p8"])
    s = empty_dev(32, torch.float32, dev)
    hip.repack_gemv_q4_0_q8_0(n, s, p4, to_dev(g["act"], dev), 32)
    assert np.array_equal(bits(from_dev(s)), bits(g["s4"]))
    hip.repack_gemv_q8_0_q8_0(n, s, p8, to_dev(g["act"], dev), 32)
    assert np.array_equal(bits(from_dev(s)), bits(g["s8"]))

    g = load("repack_gemm")
    n = int(g["n"])
    a = g["act"]
    ax4 = empty_dev(g["ax4"].size, torch.uint8, dev)
    hip.pack_q8_0_to_q8_0x4(8, n // 32, to_dev(a, dev), a.shape[1], ax4)
    assert np.array_equal(from_dev(ax4), g["ax4"])
    s = empty_dev(8 * 32, torch.float32, dev)
    hip.repack_gemm_q4_0_q8_0(n, s, to_dev(g["p4"], dev), ax4, 8, 32, 32)
    assert np.array_equal(bits(from_dev(s)), bits(g["s"]))
