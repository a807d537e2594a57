"""GPU parity: every libtcrv_hip entry point, called through the C-ABI, against
the CPU oracle on the same seeded inputs.  Integer sums must be bit-exact;
fp32 outputs within 1e-5 relative and, by construction, bit-identical."""
import numpy as np
import pytest
import torch

import synth
from gpu_util import assert_f32_parity, assert_f32_parity_nan, empty_dev, from_dev, q4_tiles_gemm, to_dev

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------- a1 add ---

@pytest.mark.parametrize("n", [1, 3, 1031, 4096 + 5, (1 << 20) + 3])
def test_add_f32_sizes(hip, oracle, dev, n):
    a = synth.uniform_f32(1001, n)
    b = synth.uniform_f32(1002, n)
    da, db = to_dev(a, dev), to_dev(b, dev)
    out = empty_dev(n, torch.float32, dev)
    hip.add_f32(da, db, out, n)
    assert_f32_parity(from_dev(out), oracle.add_f32(a, b), what=f"add n={n}")


def test_add_f32_misaligned_and_inplace(hip, oracle, dev):
    n = 5000
    a = synth.uniform_f32(11, n + 1)
    b = synth.uniform_f32(12, n + 1)
    da, db = to_dev(a, dev), to_dev(b, dev)
    out = empty_dev(n + 1, torch.float32, dev)
    hip.add_f32(da[1:], db[1:], out[1:], n)  # 4-byte aligned only: scalar path
    assert_f32_parity(from_dev(out)[1:], oracle.add_f32(a[1:].copy(), b[1:].copy()))
    hip.add_f32(da, db, da, n + 1)           # out aliases lhs
    assert_f32_parity(from_dev(da), oracle.add_f32(a, b))


def test_add_f32_full_config(hip, oracle, dev):
    n = 1 << 24
    a = synth.uniform_f32(1001, n)
    b = synth.uniform_f32(1002, n)
    out = empty_dev(n, torch.float32, dev)
    hip.add_f32(to_dev(a, dev), to_dev(b, dev), out, n)
    assert_f32_parity(from_dev(out), oracle.add_f32(a, b), what="add 2^24")


def test_add_i32_harness_vector_via_f32_bits(hip, dev):
    # harness_add.cpp:14-21 inputs (3i-17, 41-2i, n=1031) as exactly representable floats
    n = 1031
    i = np.arange(n, dtype=np.float32)
    a, b = 3 * i - 17, 41 - 2 * i
    out = empty_dev(n, torch.float32, dev)
    hip.add_f32(to_dev(a, dev), to_dev(b, dev), out, n)
    assert np.array_equal(from_dev(out), i + 24)


# --------------------------------------------------------------- a3 dequant ---

@pytest.mark.parametrize("nb", [1, 127, 128, 131, 4096 * 4096 // 32])
def test_dequant_q8_0(hip, oracle, dev, nb):
    n = nb * 32
    vx = synth.quantize_q8_0(synth.normal_f32(1003, n, 0.0, 0.02))
    y = empty_dev(n, torch.float32, dev)
    hip.dequantize_row_q8_0(to_dev(vx, dev), y, n)
    assert_f32_parity(from_dev(y), oracle.dequantize_row_q8_0(vx, n), what=f"dequant nb={nb}")


# -------------------------------------------------------------- a3b dequant ---

@pytest.mark.parametrize("nb", [1, 7, 63, 64, 65, 129, 4096 * 4096 // 32])
def test_dequant_q4_0(hip, oracle, dev, nb):
    # 4096^2 is the config-2 shape with Q4_0 weights (N(0, 0.02), d = max / -8)
    n = nb * 32
    vx = synth.quantize_q4_0(synth.normal_f32(1003, n, 0.0, 0.02))
    y = empty_dev(n, torch.float32, dev)
    hip.dequantize_row_q4_0(to_dev(vx, dev), y, n)
    assert_f32_parity(from_dev(y), oracle.dequantize_row_q4_0(vx, n), what=f"dequant q4 nb={nb}")


def test_dequant_q4_0_edges(hip, oracle, dev):
    # every weight byte value, special fp16 scales (+-0, subnormals, 65504,
    # +-inf, quiet and signalling NaN), a trailing partial block (dropped, its
    # outputs untouched), a source 2 bytes past a 16-byte boundary and an output
    # only 4-byte aligned (scalar stores), across work-group edges
    nb = 64 * 3 + 5
    w = synth.quantize_q4_0(synth.normal_f32(41, nb * 32, 0.0, 0.02)).reshape(nb, 18)
    w[:16, 2:] = np.arange(256, dtype=np.uint8).reshape(16, 16)
    special = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03ff, 0x7bff, 0xfbff, 0x7c00, 0xfc00,
                        0x7e00, 0x7d01, 0xfe00], dtype=np.uint16)
    w[:special.size, 0:2] = special.view(np.uint8).reshape(-1, 2)
    w[70:70 + special.size, 0:2] = special.view(np.uint8).reshape(-1, 2)
    w = w.reshape(-1)
    n = nb * 32 + 31  # 31 trailing elements: no 198th block is read
    want = oracle.dequantize_row_q4_0(w, n)
    for src_off, dst_off in ((0, 0), (2, 0), (0, 1), (2, 1), (6, 3)):
        buf = empty_dev(w.size + 16, torch.uint8, dev)
        buf[src_off:src_off + w.size] = to_dev(w, dev)
        y = torch.full((nb * 32 + 64,), 1234.5, dtype=torch.float32, device=dev)
        hip.dequantize_row_q4_0(buf[src_off:src_off + w.size], y[dst_off:], n)
        got = from_dev(y)
        assert_f32_parity_nan(got[dst_off:dst_off + nb * 32], want,
                              what=f"dequant q4 src+{src_off} dst+{4 * dst_off}")
        assert np.all(got[:dst_off] == 1234.5) and np.all(got[dst_off + nb * 32:] == 1234.5)
    # n < 32: nothing to do, nothing written
    y = torch.full((32,), 7.0, dtype=torch.float32, device=dev)
    hip.dequantize_row_q4_0(to_dev(w, dev), y, 31)
    assert np.all(from_dev(y) == 7.0)


# -------------------------------------------------------------- a10 quantize ---

@pytest.mark.parametrize("nb", [1, 31, 32, 33, 63, 64, 65, 100, 4096 * 4096 // 32])
def test_quantize_q8_0(hip, oracle, dev, nb):
    n = nb * 32
    x = synth.normal_f32(1007, n, 0.0, 1.0)
    x[:32] = 0.0
    if nb > 3:
        x[32:64] = np.arange(32) - 15.5
        x[64:96] = 1e-30
    vy = empty_dev(nb * 34, torch.uint8, dev)
    hip.quantize_row_q8_0(n, to_dev(x, dev), vy)
    got = from_dev(vy)
    want = oracle.quantize_q8_0(x)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} bytes differ"


# ------------------------------------------------- a4 standalone integer core ---

@pytest.mark.parametrize("n,off", [(0, 0), (1, 0), (16, 0), (4095, 0), (1 << 20, 0), (1000, 3),
                                   ((1 << 20) + 7, 1)])
def test_int_core_reduce(hip, oracle, dev, n, off):
    """tcrv_hip_packed_i4_offset_binary_x_i8_product_reduce against the oracle:
    16-byte aligned operands take the v_dot4 path, others the byte path; every
    weight byte value appears."""
    rng = np.random.default_rng(n + off)
    w = rng.integers(0, 256, n + off).astype(np.uint8)
    w[off:off + min(n, 256)] = np.arange(min(n, 256))
    qlo = rng.integers(-128, 128, n + off).astype(np.int8)
    qhi = rng.integers(-128, 128, n + off).astype(np.int8)
    acc = np.array([-12345], np.int32)
    want = oracle.int_core_reduce(w[off:].view(np.int8).copy(), qlo[off:].copy(), qhi[off:].copy(),
                                  int(acc[0]))
    dw, dl, dh = to_dev(w, dev), to_dev(qlo, dev), to_dev(qhi, dev)
    out = to_dev(np.array([7], np.int32), dev)
    hip.packed_i4_offset_binary_x_i8_product_reduce(dw[off:], dl[off:], dh[off:],
                                                    to_dev(acc, dev), out, n)
    assert int(from_dev(out)[0]) == want
    # the accumulator cell may be the output cell
    cell = to_dev(acc.copy(), dev)
    hip.packed_i4_offset_binary_x_i8_product_reduce(dw[off:], dl[off:], dh[off:], cell, cell, n)
    assert int(from_dev(cell)[0]) == want


def test_int_core_reduce_wraps_int32(hip, oracle, dev):
    """n large enough that the sum leaves int32: the cell wraps as the RVV
    integer add does."""
    n = 1 << 21
    w = np.zeros(n, np.uint8)            # every nibble 0 -> -8
    qlo = np.full(n, -128, np.int8)       # -8 * -128 = 1024 per element
    qhi = np.full(n, -128, np.int8)
    acc = np.array([2**31 - 5], np.int32)
    want = oracle.int_core_reduce(w.view(np.int8), qlo, qhi, int(acc[0]))
    assert want == ((2**31 - 5 + 2048 * n + 2**31) % 2**32) - 2**31
    out = empty_dev(1, torch.int32, dev)
    hip.packed_i4_offset_binary_x_i8_product_reduce(to_dev(w, dev), to_dev(qlo, dev),
                                                    to_dev(qhi, dev), to_dev(acc, dev), out, n)
    assert int(from_dev(out)[0]) == want


# ------------------------------------------------------------ block sums a4/a5 ---

@pytest.mark.parametrize("nb,rows", [(1, 3), (2, 5), (128, 64), (131, 7), (300, 2)])
def test_block_sums_q8_0(hip, oracle, dev, nb, rows):
    n = nb * 32
    vx = synth.q8_0_matrix(rows, n, 1004, 1.0)
    vy = synth.q8_0_matrix(rows, n, 1005, 1.0)
    vx[0, 2:34] = 0x80  # -128 * -128 bound
    vy[0, 2:34] = 0x80
    rb = vx.shape[1]
    sumi = empty_dev(rows * nb, torch.int32, dev)
    hip.q8_0_q8_0_block_sums(n, sumi, to_dev(vx, dev), rb, to_dev(vy, dev), rb, rows)
    got = from_dev(sumi).reshape(rows, nb)
    for r in range(rows):
        assert np.array_equal(got[r], oracle.block_sums_q8_0(n, vx[r].copy(), vy[r].copy()))
    assert got[0, 0] == 524288


@pytest.mark.parametrize("nb,rows", [(1, 3), (2, 5), (128, 64), (131, 7)])
def test_block_sums_q4_0_all_weight_bytes(hip, oracle, dev, nb, rows):
    n = nb * 32
    rng = np.random.default_rng(nb * 1000 + rows)
    vx = synth.q4_0_matrix(rows, n, 1006, 0.02)
    # every weight byte value 0..255 appears in the quants
    qs = vx.reshape(rows, nb, 18)[:, :, 2:]
    qs[...] = rng.permutation(np.resize(np.arange(256, dtype=np.uint8), qs.size)).reshape(qs.shape)
    vy = synth.q8_0_matrix(rows, n, 1007, 1.0)
    sumi = empty_dev(rows * nb, torch.int32, dev)
    hip.q4_0_q8_0_block_sums(n, sumi, to_dev(vx, dev), vx.shape[1], to_dev(vy, dev),
                             vy.shape[1], rows)
    got = from_dev(sumi).reshape(rows, nb)
    for r in range(rows):
        assert np.array_equal(got[r], oracle.block_sums_q4_0(n, vx[r].copy(), vy[r].copy()))


# ------------------------------------------------------------ a5/a6 block dots ---

def test_q8_0_block_dot_single(hip, oracle, dev):
    for nb in (0, 1, 2, 7, 128, 129):
        n = nb * 32 + (5 if nb == 7 else 0)  # trailing partial block is ignored
        vx = synth.q8_0_matrix(1, max(nb, 1) * 32, 50 + nb, 1.0).reshape(-1)
        vy = synth.q8_0_matrix(1, max(nb, 1) * 32, 60 + nb, 1.0).reshape(-1)
        s = to_dev(np.full(1, 7.0, np.float32), dev)
        hip.q8_0_q8_0_block_dot(n, s, to_dev(vx, dev), to_dev(vy, dev))
        assert_f32_parity(from_dev(s), [oracle.vec_dot_q8_0(n, vx, vy)], what=f"nb={nb}")


def test_q4_0_block_dot_single_ggml_abi(hip, oracle, dev):
    for nb in (0, 1, 3, 128, 130):
        n = nb * 32
        vx = synth.q4_0_matrix(1, max(nb, 1) * 32, 70 + nb, 0.02).reshape(-1)
        vy = synth.q8_0_matrix(1, max(nb, 1) * 32, 80 + nb, 1.0).reshape(-1)
        s = to_dev(np.full(1, 7.0, np.float32), dev)
        # bs, bx, by, nrc are not read (as in the reference); pass junk
        hip.q4_0_q8_0_block_dot(n, s, 999, to_dev(vx, dev), 12345, to_dev(vy, dev), 777, 2)
        assert_f32_parity(from_dev(s), [oracle.vec_dot_q4_0(n, vx, vy)], what=f"nb={nb}")


# even nb with 4-byte aligned rows take the register-direct kernel (partial
# chunks, two chunks with a carried sum, pair counts that are not a multiple of
# the 16 pairs per work-group); odd nb or 2-byte aligned rows the LDS one
@pytest.mark.parametrize("rows,nb,pad", [(16384, 128, 0), (33, 131, 16), (5, 1, 0), (9, 256, 32),
                                         (21, 6, 0), (7, 130, 4), (3, 4, 2), (4101, 64, 4),
                                         (4103, 32, 8)])
def test_q8_0_block_dot_rows(hip, oracle, dev, rows, nb, pad):
    n = nb * 32
    vx = synth.q8_0_matrix(rows, n, 1004, 1.0)
    vy = synth.q8_0_matrix(rows, n, 1005, 1.0)
    if pad:
        vx = np.pad(vx, ((0, 0), (0, pad)))
        vy = np.pad(vy, ((0, 0), (0, pad)))
    bx = vx.shape[1]
    s = empty_dev(rows, torch.float32, dev)
    hip.q8_0_q8_0_block_dot_rows(n, s, to_dev(vx, dev), bx, to_dev(vy, dev), bx, rows)
    want = oracle.vec_dot_q8_0_rows(n, vx, bx, vy, bx, rows, 8)
    assert_f32_parity(from_dev(s), want, what=f"q8 rows={rows} nb={nb}")


@pytest.mark.parametrize("rows,nb,pad", [(16384, 128, 0), (33, 131, 16), (5, 1, 0), (9, 256, 32),
                                         (21, 6, 0), (7, 130, 4), (7, 130, 2), (4101, 64, 4),
                                         (4103, 32, 8)])
def test_q4_0_block_dot_rows(hip, oracle, dev, rows, nb, pad):
    n = nb * 32
    vx = synth.q4_0_matrix(rows, n, 1006, 0.02)
    vy = synth.q8_0_matrix(rows, n, 1007, 1.0)
    if pad:
        vx = np.pad(vx, ((0, 0), (0, pad)))
        vy = np.pad(vy, ((0, 0), (0, pad)))
    s = empty_dev(rows, torch.float32, dev)
    hip.q4_0_q8_0_block_dot_rows(n, s, to_dev(vx, dev), vx.shape[1], to_dev(vy, dev),
                                 vy.shape[1], rows)
    want = oracle.vec_dot_q4_0_rows(n, vx, vx.shape[1], vy, vy.shape[1], rows, 8)
    assert_f32_parity(from_dev(s), want, what=f"q4 rows={rows} nb={nb}")


# ------------------------------------------------------------ a7 GEMV / GEMM ---

@pytest.mark.parametrize("nr,nb", [(4096, 128), (1, 128), (13, 5), (1000, 131), (64, 256),
                                   (2048, 258),   # 2 rows per wave, chunk prefetch, a 2-block tail
                                   (2049, 128),   # 4 rows per wave from 2049 rows, ragged last wave
                                   (2500, 260),   # 4 rows per wave with the chunk prefetch
                                   (4096, 64),    # n = 2048: the half-wave kernel, 4 rows a wave
                                   (8200, 64),    # the half-wave kernel, 8 rows a wave, ragged
                                   (4100, 32)])   # n = 1024: a quarter-wave group per 2 rows
def test_gemv_q4_0_q8_0(hip, oracle, dev, nr, nb):
    n = nb * 32
    w = synth.q4_0_matrix(nr, n, 1006, 0.02)
    x = synth.q8_0_matrix(1, n, 1007, 1.0).reshape(-1)
    s = empty_dev(nr, torch.float32, dev)
    hip.gemv_q4_0_q8_0(n, s, to_dev(w, dev), w.shape[1], to_dev(x, dev), nr)
    want = oracle.gemm_q4_0(n, w, x, 0, nr, 1, w.shape[1], 1, 8)[:nr]
    assert_f32_parity(from_dev(s), want, what=f"gemv nr={nr} nb={nb}")


# the lane-group kernels for rows of 2048 and 1024 quants with padded rows (bx
# past the row bytes)
@pytest.mark.parametrize("nr,nb,pad", [(4096, 64, 4), (8200, 64, 16), (4100, 32, 4),
                                       (14336, 32, 16), (2048, 64, 4), (1024, 32, 16)])
def test_gemv_q4_0_q8_0_padded_short_rows(hip, oracle, dev, nr, nb, pad):
    n = nb * 32
    w = np.pad(synth.q4_0_matrix(nr, n, 1016, 0.02), ((0, 0), (0, pad)))
    x = synth.q8_0_matrix(1, n, 1017, 1.0).reshape(-1)
    s = empty_dev(nr, torch.float32, dev)
    dw = to_dev(w, dev)
    hip.gemv_q4_0_q8_0(n, s, dw, w.shape[1], to_dev(x, dev), nr)
    want = oracle.gemm_q4_0(n, w, x, 0, nr, 1, w.shape[1], 1, 8)[:nr]
    assert_f32_parity(from_dev(s), want, what=f"gemv nr={nr} nb={nb} pad={pad}")
    for rpw in (2, 4, 8):
        hip.gemv_q4_0_q8_0_shaped(n, s, dw, w.shape[1], to_dev(x, dev), nr, rpw)
        assert_f32_parity(from_dev(s), want, what=f"gemv rows_per_wave={rpw} pad={pad}")


@pytest.mark.parametrize("nr,nb", [(1000, 128), (333, 40), (129, 200), (70, 9), (8200, 64),
                                   (1000, 32)])
def test_gemv_shapes_are_bit_identical(hip, oracle, dev, nr, nb):
    """The decode GEMV's schedule knob (rows per wave 2, 4, 8) changes how it
    runs, never what it computes: every shape equals the oracle and the plain
    entry bit for bit (one 128-block chunk, one partial chunk, two chunks, and
    odd nb, which the LDS-staged kernel serves whatever the knob)."""
    n = nb * 32
    w = synth.q4_0_matrix(nr, n, 2201, 0.02)
    x = synth.q8_0_matrix(1, n, 2202, 1.0)[0]
    want = oracle.gemm_q4_0(n, w, x, 0, nr, 1, w.shape[1], 1, 8)[:nr]
    dw, dx = to_dev(w, dev), to_dev(x, dev)
    plain = empty_dev(nr, torch.float32, dev)
    hip.gemv_q4_0_q8_0(n, plain, dw, w.shape[1], dx, nr)
    assert_f32_parity(from_dev(plain), want, what="plain")
    for rpw in (2, 4, 8):
        s = empty_dev(nr, torch.float32, dev)
        hip.gemv_q4_0_q8_0_shaped(n, s, dw, w.shape[1], dx, nr, rpw)
        assert_f32_parity(from_dev(s), want, what=f"rows_per_wave {rpw}")
    s = empty_dev(nr, torch.float32, dev)
    for bad in (0, 1, 3, 16):
        assert hip.gemv_q4_0_q8_0_shaped(n, s, dw, w.shape[1], dx, nr, bad,
                                         check=False) == hip.ERR_BAD_SIZE
    torch.cuda.synchronize()


def test_q4_0_gemm_entry_nc1_strided_output(hip, oracle, dev):
    n, nr, bs = 32 * 40, 77, 3
    w = np.pad(synth.q4_0_matrix(nr, n, 5, 0.02), ((0, 0), (0, 48)))
    x = synth.q8_0_matrix(1, n, 6, 1.0).reshape(-1)
    s = to_dev(np.full(nr * bs, -1.0, np.float32), dev)
    hip.q4_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(x, dev), 0, nr, 1, w.shape[1], bs)
    got = from_dev(s)
    want = oracle.gemm_q4_0(n, w, x, 0, nr, 1, w.shape[1], bs)
    assert_f32_parity(got[::bs], want[:nr * bs:bs])
    assert np.all(got.reshape(nr, bs)[:, 1:] == -1.0)  # untouched between rows


@pytest.mark.parametrize("m,nb,pad", [(4, 128, 0), (6, 5, 0), (1, 2, 0), (33, 64, 8), (4, 130, 2)])
def test_q4_0_gemm_tile(hip, oracle, dev, m, nb, pad):
    """tcrv_rvv.q4_0_q8_0_gemm_tile: one weight row x m activation columns."""
    n = nb * 32
    w = synth.q4_0_matrix(1, n, 1006, 0.02)
    a = np.pad(synth.q8_0_matrix(m, n, 1007, 1.0), ((0, 0), (0, pad)))
    s = empty_dev(m, torch.float32, dev)
    hip.q4_0_q8_0_gemm_tile(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], m)
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], 1, m, w.shape[1], m, 8)
    assert_f32_parity(from_dev(s), want, what=f"gemm tile m={m} nb={nb}")


@pytest.mark.parametrize("nr,nc,nb", [(37, 5, 8), (16, 64, 128), (3, 2, 1), (1, 70, 128)])
def test_q4_0_gemm_multi_column(hip, oracle, dev, nr, nc, nb):
    n = nb * 32
    w = synth.q4_0_matrix(nr, n, 7, 0.02)
    a = np.pad(synth.q8_0_matrix(nc, n, 8, 1.0), ((0, 0), (0, 16)))
    bs = nc + 3
    s = to_dev(np.zeros(nr * bs, np.float32), dev)
    hip.q4_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], bs)
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], bs, 8)
    got = from_dev(s).reshape(nr, bs)
    assert_f32_parity(got[:, :nc], want.reshape(nr, bs)[:, :nc], what="q4 gemm")


@pytest.mark.parametrize("nr,nc,nb,ypad", [
    (4096, 2, 128, 0),   # one chunk, two columns
    (4096, 3, 128, 0),   # a four-column group with three present
    (100, 7, 130, 16),   # partial work-group, two chunks (the second of 2 blocks), 4 + 3
    (300, 6, 258, 4),    # three chunks, 4 + 2 columns
    (64, 9, 64, 0),      # nb < 128, 4 + 4 + 1 (the last column through the GEMV)
    (48, 64, 8, 0),      # the largest token count of the multi-column path
    (40, 5, 7, 0),       # odd nb: the MFMA GEMM instead
])
def test_q4_0_gemm_few_tokens(hip, oracle, dev, nr, nc, nb, ypad):
    """The a7 GEMM with a few tokens (batched decode) runs as GEMVs over groups
    of up to four activation columns, the weights read once per group: every
    output equals the oracle's, and the output row padding stays untouched."""
    n = nb * 32
    w = synth.q4_0_matrix(nr, n, 1017, 0.02)
    a = np.pad(synth.q8_0_matrix(nc, n, 1016, 1.0), ((0, 0), (0, ypad)))
    a[0, 2:34] = 0x80
    bs = nc + 5
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    hip.q4_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], bs)
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], bs, 8).reshape(nr, bs)
    got = from_dev(s).reshape(nr, bs)
    assert_f32_parity(got[:, :nc], want[:, :nc], what=f"q4 gemm {nr}x{nc}x{n}")
    assert np.all(got[:, nc:] == -7.0)


# ------------------------------------------------------------------ a9 GEMM ---

@pytest.mark.parametrize("nr,nc,nb,ypad", [
    (4096, 2, 128, 0),   # one chunk, two columns
    (4096, 5, 128, 0),   # an eight-column group with five present
    (100, 7, 130, 16),   # partial work-group, two chunks, seven columns
    (300, 11, 258, 4),   # three chunks, 8 + 3 columns
    (64, 13, 64, 0),     # nb < 128, 8 + 4 + 1 (the last column through the block dots)
    (48, 64, 8, 0),      # the largest token count of the multi-column path
    (40, 3, 7, 0),       # odd nb: the MFMA GEMM instead
])
def test_q8_0_gemm_few_tokens(hip, oracle, dev, nr, nc, nb, ypad):
    """The a9 GEMM with a few tokens runs as GEMVs over groups of up to eight
    activation columns: every output equals the oracle's (the a5 fold with the
    exact d_x*d_y), and the output row padding stays untouched."""
    n = nb * 32
    w = synth.q8_0_matrix(nr, n, 1015, 0.02)
    a = np.pad(synth.q8_0_matrix(nc, n, 1014, 1.0), ((0, 0), (0, ypad)))
    w[0, 2:34] = 0x80
    a[0, 2:34] = 0x80  # -128 x -128 block sums
    bs = nc + 5
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    hip.q8_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], bs)
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], nr, nc, w.shape[1], bs, 8).reshape(nr, bs)
    got = from_dev(s).reshape(nr, bs)
    assert_f32_parity(got[:, :nc], want[:, :nc], what=f"q8 gemm {nr}x{nc}x{n}")
    assert np.all(got[:, nc:] == -7.0)


@pytest.mark.parametrize("nr,nc,nb,xpad,ypad", [
    (128, 128, 8, 0, 0),      # one tile, one K chunk
    (256, 128, 128, 0, 0),    # full K, two tiles
    (100, 70, 9, 16, 32),     # partial tiles, partial K chunk, padded strides
    (33, 1, 3, 0, 0),         # single column (decode-shaped), odd nb: the MFMA path
    (4096, 1, 128, 0, 0),     # decode: the register-direct GEMV
    (1023, 1, 260, 0, 0),     # decode, one pair per wave: 2 chunks + 4 blocks, ragged rows
    (1001, 1, 64, 0, 0),      # decode, n = 2048: two pairs per wave, one per half-wave
    (1003, 1, 32, 0, 0),      # decode, n = 1024: four pairs per wave, one per lane group
    (77, 1, 6, 4, 0),         # decode, padded rows, output stride bs = 6
    (1, 1, 2, 0, 0),          # one output
    (1, 45, 1, 0, 0),         # single weight row, one block
    (1, 300, 64, 0, 8),       # single weight row: register-direct block dots
    (1, 33, 260, 0, 0),       # single weight row, 2 chunks + 4 blocks
    (512, 512, 128, 0, 0),
    # 256+ weight rows take the wide 256x128 tile with 4-block K chunks
    (300, 130, 7, 16, 32),    # partial wide tiles both ways, 4 + 3 blocks, padded strides
    (256, 2, 1, 0, 0),        # one block: only the partial chunk
    (520, 257, 13, 0, 4),     # three tile rows, 3 full chunks + 1 block
    (300, 130, 8, 0, 0),      # two full chunks, partial tiles both ways
    (520, 257, 16, 16, 32),   # four full chunks, padded strides, three tile rows
    (256, 64, 8, 4, 0),       # one full tile row, a stride of 276 bytes
])
def test_q8_0_gemm(hip, oracle, dev, nr, nc, nb, xpad, ypad):
    n = nb * 32
    w = np.pad(synth.q8_0_matrix(nr, n, 1009, 0.02), ((0, 0), (0, xpad)))
    a = np.pad(synth.q8_0_matrix(nc, n, 1008, 1.0), ((0, 0), (0, ypad)))
    bs = nc + (5 if xpad else 0)
    s = to_dev(np.zeros(nr * bs, np.float32), dev)
    hip.q8_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], bs)
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], nr, nc, w.shape[1], bs, 8)
    got = from_dev(s).reshape(nr, bs)
    assert_f32_parity(got[:, :nc], want.reshape(nr, bs)[:, :nc], what=f"gemm {nr}x{nc}x{n}")


def test_q8_0_gemm_full_config_sampled_rows(hip, oracle, dev):
    """4096 x 4096 x 4096 on the GPU; 96 output rows (every column) checked
    against the oracle, plus 96 sampled columns of every row."""
    n = nr = nc = 4096
    w = synth.q8_0_matrix(nr, n, 1009, 0.02)
    a = synth.q8_0_matrix(nc, n, 1008, 1.0)
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q8_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], nc)
    got = from_dev(s).reshape(nr, nc)
    rng = np.random.default_rng(99)
    rows = np.sort(rng.choice(nr, 96, replace=False))
    for r in rows:
        want = oracle.gemm_q8_0(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r], want, what=f"row {r}")
    cols = np.sort(rng.choice(nc, 96, replace=False))
    sub = np.ascontiguousarray(a[cols])
    want = oracle.gemm_q8_0(n, w, sub, sub.shape[1], nr, len(cols), w.shape[1], len(cols), 8)
    assert_f32_parity(got[:, cols], want.reshape(nr, len(cols)), what="sampled cols")


# --------------------------------------------------------------- error paths ---

def test_argument_errors_launch_nothing(hip, dev):
    t = empty_dev(4096, torch.uint8, dev)
    f = empty_dev(1024, torch.float32, dev)
    st = hip.call
    assert st("tcrv_hip_q8_0_q8_0_gemm", 64, f, t[1:], t, 34 * 2, 2, 2, 34 * 2, 2,
              0, check=False) == hip.ERR_MISALIGNED
    assert st("tcrv_hip_q8_0_q8_0_gemm", 64, f, t, t, 66, 2, 2, 68, 2,
              0, check=False) == hip.ERR_BAD_SIZE    # by < row bytes (68)
    assert st("tcrv_hip_q8_0_q8_0_gemm", 64, f, t, t, 69, 2, 2, 68, 2,
              0, check=False) == hip.ERR_MISALIGNED  # odd stride
    assert st("tcrv_hip_q8_0_q8_0_gemm", 64, f, t, t, 68, 3, 2, 68, 1,
              0, check=False) == hip.ERR_BAD_SIZE    # bs < nc
    assert st("tcrv_hip_gemv_q4_0_q8_0", 64, 0, t, 48, t, 2, 0,
              check=False) == hip.ERR_NULL_POINTER
    torch.cuda.synchronize()


# ------------------------------------------ 2-byte aligned (non-16) layouts ---

def test_unaligned_rows_all_entries(hip, oracle, dev):
    """Rows that start 2 bytes past a 16-byte boundary and odd-block strides
    (34*nb, 18*nb with nb odd) take the narrow-load staging path; results must
    be identical to the oracle."""
    nb, rows = 37, 11
    n = nb * 32
    x8 = synth.q8_0_matrix(rows, n, 21, 1.0)
    y8 = synth.q8_0_matrix(rows, n, 22, 1.0)
    x4 = synth.q4_0_matrix(rows, n, 23, 0.02)
    rb8, rb4 = x8.shape[1], x4.shape[1]

    def shifted(a):  # device copy whose first byte sits 2 bytes past a 16-byte boundary
        buf = empty_dev(a.size + 16, torch.uint8, dev)
        buf[2:2 + a.size] = to_dev(a.reshape(-1), dev)
        return buf[2:2 + a.size]

    dx8, dy8, dx4 = shifted(x8), shifted(y8), shifted(x4)
    s = empty_dev(rows, torch.float32, dev)
    hip.q8_0_q8_0_block_dot_rows(n, s, dx8, rb8, dy8, rb8, rows)
    assert_f32_parity(from_dev(s), oracle.vec_dot_q8_0_rows(n, x8, rb8, y8, rb8, rows))
    hip.q4_0_q8_0_block_dot_rows(n, s, dx4, rb4, dy8, rb8, rows)
    assert_f32_parity(from_dev(s), oracle.vec_dot_q4_0_rows(n, x4, rb4, y8, rb8, rows))
    hip.gemv_q4_0_q8_0(n, s, dx4, rb4, dy8, rows)
    assert_f32_parity(from_dev(s), oracle.gemm_q4_0(n, x4, y8[0].copy(), 0, rows, 1, rb4, 1))
    g = empty_dev(rows * rows, torch.float32, dev)
    hip.q8_0_q8_0_gemm(n, g, dx8, dy8, rb8, rows, rows, rb8, rows)
    assert_f32_parity(from_dev(g), oracle.gemm_q8_0(n, x8, y8, rb8, rows, rows, rb8, rows))
    y = empty_dev(n + 1, torch.float32, dev)
    hip.dequantize_row_q8_0(dx8, y[1:], n)  # 4-byte aligned output: scalar stores
    assert_f32_parity(from_dev(y)[1:], oracle.dequantize_row_q8_0(x8[0].copy(), n))
    xf = synth.normal_f32(24, n + 1)
    dq = empty_dev(nb * 34 + 16, torch.uint8, dev)
    hip.quantize_row_q8_0(n, to_dev(xf, dev)[1:], dq[2:])
    assert np.array_equal(from_dev(dq)[2:2 + nb * 34], oracle.quantize_q8_0(xf[1:].copy()))


# ------------------------------------------------------- a8 x16 repack layout ---

def x16_source(w, nb, k):
    """Plain rows (nc x nb blocks of k bytes) in pack order: group x, block b
    takes block b of rows 16x .. 16x+15."""
    nc = w.shape[0]
    return np.ascontiguousarray(np.concatenate(
        [w[16 * x:16 * x + 16, k * b:k * b + k] for x in range(nc // 16) for b in range(nb)]
    ).reshape(-1))


@pytest.mark.parametrize("nblocks", [1, 7, 64, 65, 100, 4096 * 128 // 16])
def test_pack_q4_0x16(hip, oracle, dev, nblocks):
    src = synth.q4_0_matrix(1, 16 * nblocks * 32, 61, 0.02).reshape(-1)
    dst = empty_dev(nblocks * 288, torch.uint8, dev)
    hip.pack_q4_0_to_q4_0x16(nblocks, to_dev(src, dev), dst)
    assert np.array_equal(from_dev(dst), oracle.pack_q4_0x16(src, nblocks))


@pytest.mark.parametrize("nblocks", [1, 9, 32, 33, 70, 4096 * 128 // 16])
def test_pack_q8_0x16(hip, oracle, dev, nblocks):
    src = synth.q8_0_matrix(1, 16 * nblocks * 32, 62, 1.0).reshape(-1)
    dst = empty_dev(nblocks * 544, torch.uint8, dev)
    hip.pack_q8_0_to_q8_0x16(nblocks, to_dev(src, dev), dst)
    assert np.array_equal(from_dev(dst), oracle.pack_q8_0x16(src, nblocks))


@pytest.mark.parametrize("quant,nblocks", [("q4_0", 33), ("q8_0", 17)])
def test_pack_x16_two_byte_aligned_source(hip, oracle, dev, quant, nblocks):
    """16-byte aligned spans take the LDS-staged quad-transpose pack; a source
    only 2-byte aligned takes the per-dword gather: both give the oracle's
    bytes."""
    q4 = quant == "q4_0"
    mat = synth.q4_0_matrix if q4 else synth.q8_0_matrix
    src = mat(1, 16 * nblocks * 32, 63, 0.02).reshape(-1)
    xb = 288 if q4 else 544
    pack = hip.pack_q4_0_to_q4_0x16 if q4 else hip.pack_q8_0_to_q8_0x16
    want = (oracle.pack_q4_0x16 if q4 else oracle.pack_q8_0x16)(src, nblocks)
    buf = empty_dev(src.size + 16, torch.uint8, dev)
    buf[2:2 + src.size] = to_dev(src, dev)
    for what, s_dev in (("aligned", to_dev(src, dev)), ("2-byte", buf[2:2 + src.size])):
        dst = empty_dev(nblocks * xb, torch.uint8, dev)
        pack(nblocks, s_dev, dst)
        assert np.array_equal(from_dev(dst), want), f"{quant} {what} source"


@pytest.mark.parametrize("nc,nb", [(4096, 128), (48, 131), (40, 3), (16, 1), (32, 256)])
def test_repack_gemv_q4_0(hip, oracle, dev, nc, nb):
    n = nb * 32
    w = synth.q4_0_matrix(nc, n, 1006, 0.02)
    x = synth.q8_0_matrix(1, n, 1007, 1.0).reshape(-1)
    groups = nc // 16
    packed = oracle.pack_q4_0x16(x16_source(w[:16 * groups], nb, 18), groups * nb)
    s = to_dev(np.full(nc, -7.0, np.float32), dev)
    hip.repack_gemv_q4_0_q8_0(n, s, to_dev(packed, dev), to_dev(x, dev), nc)
    got = from_dev(s)
    assert_f32_parity(got[:16 * groups], oracle.repack_gemv_q4_0(n, packed, x, nc)[:16 * groups],
                      what=f"repack q4 nc={nc} nb={nb}")
    assert np.all(got[16 * groups:] == -7.0)  # trailing partial group untouched


@pytest.mark.parametrize("nc,nb", [(4096, 128), (48, 131), (16, 1), (32, 256)])
def test_repack_gemv_q8_0_equals_plain_gemv(hip, oracle, dev, nc, nb):
    n = nb * 32
    w = synth.q8_0_matrix(nc, n, 1009, 0.02)
    x = synth.q8_0_matrix(1, n, 1008, 1.0).reshape(-1)
    w[0, 2:34] = 0x80
    x[2:34] = 0x80
    dsrc = to_dev(x16_source(w, nb, 34), dev)
    packed = empty_dev(nc // 16 * nb * 544, torch.uint8, dev)
    hip.pack_q8_0_to_q8_0x16(nc // 16 * nb, dsrc, packed)
    s = empty_dev(nc, torch.float32, dev)
    hip.repack_gemv_q8_0_q8_0(n, s, packed, to_dev(x, dev), nc)
    got = from_dev(s)
    host_packed = from_dev(packed)
    assert_f32_parity(got, oracle.repack_gemv_q8_0(n, host_packed, x, nc), what="repack q8")
    assert_f32_parity(got, oracle.gemm_q8_0(n, w, x, 0, nc, 1, w.shape[1], 1, 8)[:nc],
                      what="repack q8 vs plain")



@pytest.mark.parametrize("quant,nc,nb", [("q4_0", 48, 131), ("q8_0", 32, 37), ("q4_0", 16, 1),
                                         ("q8_0", 16, 256)])
def test_repack_gemv_unaligned_operands(hip, oracle, dev, quant, nc, nb):
    """The kernel stages a wave's share with 128-bit loads only when weights
    and activation are 16-byte aligned; a 2-byte aligned activation (one that
    follows an odd number of 34-byte blocks) and 4-byte aligned weights take
    the narrower copies: every combination gives the oracle's bits."""
    n = nb * 32
    q4 = quant == "q4_0"
    w = (synth.q4_0_matrix if q4 else synth.q8_0_matrix)(nc, n, 1010, 0.02)
    x = synth.q8_0_matrix(1, n, 1011, 1.0).reshape(-1)
    groups = nc // 16
    pack = oracle.pack_q4_0x16 if q4 else oracle.pack_q8_0x16
    packed = pack(x16_source(w, nb, w.shape[1] // nb), groups * nb)
    ref = (oracle.repack_gemv_q4_0 if q4 else oracle.repack_gemv_q8_0)(n, packed, x, nc)
    run = hip.repack_gemv_q4_0_q8_0 if q4 else hip.repack_gemv_q8_0_q8_0
    wbuf = empty_dev(packed.size + 16, torch.uint8, dev)
    wbuf[4:4 + packed.size] = to_dev(packed, dev)
    buf = empty_dev(x.size + 16, torch.uint8, dev)
    buf[2:2 + x.size] = to_dev(x, dev)
    for wwhat, wdev in (("16-byte", to_dev(packed, dev)), ("4-byte", wbuf[4:4 + packed.size])):
        for what, act in (("16-byte", to_dev(x, dev)), ("2-byte", buf[2:2 + x.size])):
            s = empty_dev(nc, torch.float32, dev)
            run(n, s, wdev, act, nc)
            assert_f32_parity(from_dev(s), ref,
                              what=f"repack {quant} {wwhat} weights, {what} activation")

# ------------------------------------------------------ a8 repack GEMM (x16 x x4) ---

@pytest.mark.parametrize("nr,nb,pad", [(4, 1, 0), (12, 5, 6), (130, 9, 0)])
def test_pack_q8_0x4(hip, oracle, dev, nr, nb, pad):
    a = np.pad(synth.q8_0_matrix(nr, nb * 32, 70, 1.0), ((0, 0), (0, pad)))
    dst = to_dev(np.full(nr // 4 * nb * 136, 0xEE, np.uint8), dev)
    hip.pack_q8_0_to_q8_0x4(nr, nb, to_dev(a, dev), a.shape[1], dst)
    assert np.array_equal(from_dev(dst), oracle.pack_q8_0x4(a, nr, nb, a.shape[1]))


@pytest.mark.parametrize("nr,nc,nb,bpad", [
    (4, 16, 1, 0),        # one group each way, one block
    (128, 256, 128, 0),   # one full 256 x 128 tile, full K
    (38, 40, 7, 3),       # partial chunk (4 + 3 blocks); trailing rows and columns unwritten
    (520, 300, 13, 5),    # five token tiles, two weight tiles (the second partial)
])
def test_repack_gemm_q4_0(hip, oracle, dev, nr, nc, nb, bpad):
    n = nb * 32
    w = synth.q4_0_matrix(nc, n, 71, 0.02)
    a = synth.q8_0_matrix(nr, n, 72, 1.0)
    a[0, 2:34] = 0x80  # -128 activations: the i16 lo/hi bound against -8 weights
    groups = nc // 16
    packed = oracle.pack_q4_0x16(x16_source(w[:16 * groups], nb, 18), groups * nb)
    ax4 = to_dev(np.zeros(nr // 4 * nb * 136, np.uint8), dev)
    hip.pack_q8_0_to_q8_0x4(nr, nb, to_dev(a, dev), a.shape[1], ax4)
    bs = nc + bpad
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    hip.repack_gemm_q4_0_q8_0(n, s, to_dev(packed, dev), ax4, nr, nc, bs)
    got = from_dev(s).reshape(nr, bs)
    want = oracle.repack_gemm_q4_0(n, packed, from_dev(ax4), nr, nc, bs).reshape(nr, bs)
    rows, cols = nr // 4 * 4, 16 * groups
    assert_f32_parity(got[:rows, :cols], want[:rows, :cols], what=f"repack gemm {nr}x{nc}x{n}")
    assert np.all(got[rows:] == -7.0) and np.all(got[:, cols:] == -7.0)  # unwritten


def test_pack_q8_0x4_two_byte_aligned_source(hip, oracle, dev):
    nr, nb = 8, 3
    a = synth.q8_0_matrix(nr, nb * 32, 73, 1.0)
    buf = empty_dev(a.size + 16, torch.uint8, dev)
    buf[2:2 + a.size] = to_dev(a.reshape(-1), dev)
    dst = empty_dev(nr // 4 * nb * 136, torch.uint8, dev)
    hip.pack_q8_0_to_q8_0x4(nr, nb, buf[2:2 + a.size], a.shape[1], dst)
    assert np.array_equal(from_dev(dst), oracle.pack_q8_0x4(a, nr, nb, a.shape[1]))


def test_repack_gemm_full_size_sampled_tokens(hip, oracle, dev):
    """4096 weight rows x 4096 tokens x K 4096 on the GPU; the oracle checks three
    4-token groups (first, middle, last) against all 4096 weight rows."""
    n = 4096
    nb = n // 32
    w = synth.q4_0_matrix(4096, n, 1006, 0.02)
    a = synth.q8_0_matrix(4096, n, 1008, 1.0)
    packed = oracle.pack_q4_0x16(x16_source(w, nb, 18), 256 * nb)
    ax4 = empty_dev(1024 * nb * 136, torch.uint8, dev)
    hip.pack_q8_0_to_q8_0x4(4096, nb, to_dev(a, dev), a.shape[1], ax4)
    s = empty_dev(4096 * 4096, torch.float32, dev)
    hip.repack_gemm_q4_0_q8_0(n, s, to_dev(packed, dev), ax4, 4096, 4096, 4096)
    got = from_dev(s).reshape(4096, 4096)
    hx4 = from_dev(ax4).reshape(1024, nb * 136)
    for y in (0, 517, 1023):
        want = oracle.repack_gemm_q4_0(n, packed, np.ascontiguousarray(hx4[y]), 4, 4096, 4096)
        assert_f32_parity(got[4 * y:4 * y + 4], want.reshape(4, 4096), what=f"group {y}")


# ------------------------------------------------ a7 Q4_0 GEMM on MFMA (nc > 1) ---

@pytest.mark.parametrize("nr,nc,nb,pad", [(512, 512, 128, 0), (130, 70, 9, 16), (64, 2, 3, 0),
                                          (300, 130, 7, 16), (256, 3, 1, 0)])
def test_q4_0_gemm_mfma_shapes(hip, oracle, dev, nr, nc, nb, pad):
    n = nb * 32
    w = np.pad(synth.q4_0_matrix(nr, n, 71, 0.02), ((0, 0), (0, pad)))
    a = np.pad(synth.q8_0_matrix(nc, n, 72, 1.0), ((0, 0), (0, pad)))
    bs = nc + 1
    s = to_dev(np.zeros(nr * bs, np.float32), dev)
    hip.q4_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], bs)
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], bs, 8)
    got = from_dev(s).reshape(nr, bs)
    assert_f32_parity(got[:, :nc], want.reshape(nr, bs)[:, :nc], what=f"q4 gemm {nr}x{nc}x{n}")


def test_q4_0_gemm_full_size_sampled(hip, oracle, dev):
    """4096 weight rows x 4096 tokens x K 4096 on the GPU; 64 rows and 64
    columns checked against the oracle."""
    n = nr = nc = 4096
    w = synth.q4_0_matrix(nr, n, 1006, 0.02)
    a = synth.q8_0_matrix(nc, n, 1008, 1.0)
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q4_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], nc)
    got = from_dev(s).reshape(nr, nc)
    rng = np.random.default_rng(7)
    for r in np.sort(rng.choice(nr, 64, replace=False)):
        want = oracle.gemm_q4_0(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r], want, what=f"row {r}")
    cols = np.sort(rng.choice(nc, 64, replace=False))
    sub = np.ascontiguousarray(a[cols])
    want = oracle.gemm_q4_0(n, w, sub, sub.shape[1], nr, len(cols), w.shape[1], len(cols), 8)
    assert_f32_parity(got[:, cols], want.reshape(nr, len(cols)), what="sampled cols")


# ---------------------------------------------------- typed tcrv_rvv.binary ---

BINARY_ELEMS = [("i8", np.int8), ("u8", np.uint8), ("i16", np.int16), ("u16", np.uint16),
                ("i32", np.int32), ("u32", np.uint32), ("i64", np.int64), ("f32", np.float32),
                ("f64", np.float64)]


def _binary_inputs(dtype, n, seed):
    rng = np.random.default_rng(seed)
    if np.issubdtype(dtype, np.integer):
        info = np.iinfo(dtype)
        a = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
        b = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
        a[:4] = [info.min, info.max, info.max, -1 if info.min < 0 else info.max]
        b[:4] = [info.min, 1, info.max, -1 if info.min < 0 else info.max]  # all-ones x all-ones
    else:
        a = (rng.standard_normal(n) * 1e3).astype(dtype)
        b = rng.standard_normal(n).astype(dtype)
        tiny = np.finfo(dtype).smallest_subnormal
        a[:3] = [tiny, np.finfo(dtype).max, -0.0]
        b[:3] = [tiny, np.finfo(dtype).max, 0.0]
    return a, b


@pytest.mark.parametrize("elem,dtype", BINARY_ELEMS)
@pytest.mark.parametrize("kind", [0, 1, 2])
def test_binary_all_types(hip, oracle, dev, kind, elem, dtype):
    for n, off in ((1031, 0), ((1 << 20) + 5, 0), (777, 1)):  # off 1: unaligned -> scalar path
        a, b = _binary_inputs(dtype, n + off, 100 * kind + n % 97)
        da, db = to_dev(a.view(np.uint8), dev), to_dev(b.view(np.uint8), dev)
        out = empty_dev((n + off) * a.itemsize, torch.uint8, dev)
        k = a.itemsize * off
        hip.binary(kind, elem, da[k:], db[k:], out[k:], n)
        want = oracle.binary(kind, hip.ELEM[elem], a[off:].copy(), b[off:].copy())
        got = from_dev(out)[k:].view(dtype)
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (elem, kind, n)


def test_add_i32_harness_vector(hip, dev):
    n = 1031
    i = np.arange(n, dtype=np.int64)
    a = (3 * i - 17).astype(np.int32)
    b = (41 - 2 * i).astype(np.int32)
    out = empty_dev(n, torch.int32, dev)
    hip.add_i32(to_dev(a, dev), to_dev(b, dev), out, n)
    assert np.array_equal(from_dev(out), (i + 24).astype(np.int32))


# ------------------------------------------- several host threads, own streams ---

def test_concurrent_host_threads_on_own_streams(hip, oracle, dev):
    """The library keeps no global state: four host threads, each launching on
    its own stream, interleave decode GEMVs and Q8_0 GEMMs on their own inputs;
    every output must still be the oracle's, bit for bit."""
    import threading

    n, nr, nc, nw = 1024, 256, 64, 96
    jobs = []
    for t in range(4):
        w4 = synth.q4_0_matrix(nr, n, 2000 + t, 0.02)
        x = synth.q8_0_matrix(1, n, 2100 + t, 1.0).reshape(-1)
        a8 = synth.q8_0_matrix(nc, n, 2200 + t, 1.0)
        b8 = synth.q8_0_matrix(nw, n, 2300 + t, 0.02)
        jobs.append({
            "w4": to_dev(w4, dev), "x": to_dev(x, dev), "a8": to_dev(a8, dev),
            "b8": to_dev(b8, dev), "y": empty_dev(nr, torch.float32, dev),
            "c": empty_dev(nw * nc, torch.float32, dev),
            "want_y": oracle.gemm_q4_0(n, w4, x, 0, nr, 1, w4.shape[1], 1, 8)[:nr],
            "want_c": oracle.gemm_q8_0(n, b8, a8, a8.shape[1], nw, nc, b8.shape[1], nc, 8),
            "bx4": w4.shape[1], "rb8": a8.shape[1]})
    torch.cuda.synchronize()
    errors = []

    def worker(j):
        try:
            st = torch.cuda.Stream(device=dev)
            for _ in range(25):
                hip.gemv_q4_0_q8_0(n, j["y"], j["w4"], j["bx4"], j["x"], nr, stream=st)
                hip.q8_0_q8_0_gemm(n, j["c"], j["b8"], j["a8"], j["rb8"], nw, nc, j["rb8"], nc,
                                   stream=st)
            st.synchronize()
        except Exception as e:  # reported below, on the test's thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(j,)) for j in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a launching thread did not finish"
    assert not errors, errors
    for t, j in enumerate(jobs):
        assert_f32_parity(from_dev(j["y"]), j["want_y"], what=f"thread {t} gemv")
        assert_f32_parity(from_dev(j["c"]), j["want_c"], what=f"thread {t} gemm")


# ------------------------------------------------ split (SoA) Q4_0 layout ---

@pytest.mark.parametrize("nr,nb,pad", [(4096, 128, 0), (33, 6, 14), (1, 2, 0), (1000, 256, 0)])
def test_soa_pack_and_gemv(hip, oracle, dev, nr, nb, pad):
    """The GPU pack writes the oracle's split layout byte for byte, and the
    GEMV over it gives the same bits as the plain-row GEMV and the oracle."""
    n = nb * 32
    w = np.pad(synth.q4_0_matrix(nr, n, 1012, 0.02), ((0, 0), (0, pad)))
    x = synth.q8_0_matrix(1, n, 1013, 1.0).reshape(-1)
    bx = w.shape[1]
    soa = empty_dev(nr * nb * 18, torch.uint8, dev)
    hip.pack_q4_0_to_soa(nr, nb, to_dev(w, dev), bx, soa)
    want_soa = oracle.pack_q4_0_soa(np.ascontiguousarray(w).reshape(-1), nr, nb, bx)
    assert np.array_equal(from_dev(soa), want_soa)
    s = empty_dev(nr, torch.float32, dev)
    hip.gemv_q4_0_soa_q8_0(n, s, soa, to_dev(x, dev), nr)
    plain = empty_dev(nr, torch.float32, dev)
    hip.gemv_q4_0_q8_0(n, plain, to_dev(w, dev), bx, to_dev(x, dev), nr)
    want = oracle.gemm_q4_0(n, w, x, 0, nr, 1, bx, 1, 8)[:nr]
    assert_f32_parity(from_dev(s), want, what=f"soa gemv {nr}x{n}")
    assert np.array_equal(from_dev(s).view(np.uint32), from_dev(plain).view(np.uint32))


def test_soa_gemv_rejects_what_it_does_not_cover(hip, dev):
    soa = empty_dev(4 * 3 * 18 + 16, torch.uint8, dev)
    x = empty_dev(3 * 34, torch.uint8, dev)
    s = empty_dev(4, torch.float32, dev)
    st = hip.call("tcrv_hip_gemv_q4_0_soa_q8_0", 96, s, soa, x, 4, 0, check=False)
    assert st == hip.ERR_UNSUPPORTED  # odd block count
    st = hip.call("tcrv_hip_gemv_q4_0_soa_q8_0", 64, s, soa[2:], x, 4, 0, check=False)
    assert st == hip.ERR_MISALIGNED   # not 16-byte aligned


# ------------------------------------------------------------ HIP graph replay ---

def test_graph_replays_match_the_oracle(hip, oracle, dev):
    """Launches captured into a HIP graph (as the bench times them) replay to
    the oracle's bits every time: five replays with eager work, output
    clearing and synchronizations between them.  The captured set includes a
    zero-block call, whose outputs come from a small fill kernel (no
    hipMemsetAsync is ever recorded)."""
    n, nr = 1024, 512
    w4 = synth.q4_0_matrix(nr, n, 3000, 0.02)
    x = synth.q8_0_matrix(1, n, 3001, 1.0).reshape(-1)
    b8 = synth.q8_0_matrix(160, 512, 3002, 0.02)
    a8 = synth.q8_0_matrix(96, 512, 3003, 1.0)
    xf = synth.normal_f32(3004, 4096 + 32, 0.0, 1.0)
    nbr = 16
    wr = synth.q4_0_matrix(32, nbr * 32, 3005, 0.02)
    packed = oracle.pack_q4_0x16(x16_source(wr, nbr, 18), 2 * nbr)
    xr = synth.q8_0_matrix(1, nbr * 32, 3006, 1.0).reshape(-1)
    want = {
        "gemv": oracle.gemm_q4_0(n, w4, x, 0, nr, 1, w4.shape[1], 1, 8)[:nr],
        "gemm": oracle.gemm_q8_0(512, b8, a8, a8.shape[1], 160, 96, b8.shape[1], 96, 8),
        "quant": oracle.quantize_q8_0(xf),
        "repack": oracle.repack_gemv_q4_0(nbr * 32, packed, xr, 32),
        "zero": np.zeros(7, np.float32),
    }
    d = {"w4": to_dev(w4, dev), "x": to_dev(x, dev), "b8": to_dev(b8, dev), "a8": to_dev(a8, dev),
         "xf": to_dev(xf, dev), "packed": to_dev(packed, dev), "xr": to_dev(xr, dev)}
    out = {"gemv": empty_dev(nr, torch.float32, dev), "gemm": empty_dev(160 * 96, torch.float32, dev),
           "quant": empty_dev(want["quant"].size, torch.uint8, dev),
           "repack": empty_dev(32, torch.float32, dev), "zero": empty_dev(7, torch.float32, dev)}
    st = torch.cuda.Stream(device=dev)

    def launch_all():
        hip.gemv_q4_0_q8_0(n, out["gemv"], d["w4"], w4.shape[1], d["x"], nr, stream=st)
        hip.q8_0_q8_0_gemm(512, out["gemm"], d["b8"], d["a8"], a8.shape[1], 160, 96,
                           b8.shape[1], 96, stream=st)
        hip.quantize_row_q8_0(xf.size, d["xf"], out["quant"], stream=st)
        hip.repack_gemv_q4_0_q8_0(nbr * 32, out["repack"], d["packed"], d["xr"], 32, stream=st)
        hip.gemv_q4_0_q8_0(16, out["zero"], d["w4"], w4.shape[1], d["x"], 7, stream=st)

    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            launch_all()
    torch.cuda.synchronize()
    side = empty_dev(nr, torch.float32, dev)
    for rep in range(5):
        for k, t in out.items():
            t.fill_(0xAB if t.dtype == torch.uint8 else float("nan"))
        hip.gemv_q4_0_q8_0(n, side, d["w4"], w4.shape[1], d["x"], nr)  # eager work between
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            graph.replay()
        torch.cuda.synchronize()
        for k in ("gemv", "gemm", "repack", "zero"):
            assert_f32_parity(from_dev(out[k]), want[k], what=f"graph replay {rep} {k}")
        assert np.array_equal(from_dev(out["quant"]), want["quant"]), f"graph replay {rep} quant"
    assert_f32_parity(from_dev(side), want["gemv"], what="eager GEMV between replays")


# ------------------------------------ a9 over the GEMM-tile layout (DMA staged) ---

def tiles_reference(a, nrows, nb):
    """The documented GEMM-tile layout, built independently in numpy from plain
    Q8_0 rows: per 64-row group and block, 64 x 16 quant bytes (elements 0-15),
    64 x 16 (elements 16-31), 64 fp16 scales; rows past nrows zero."""
    ng = -(-nrows // 64)
    blocks = np.zeros((ng * 64, nb, 34), np.uint8)
    blocks[:nrows] = a[:nrows, :nb * 34].reshape(nrows, nb, 34)
    blocks = blocks.reshape(ng, 64, nb, 34).transpose(0, 2, 1, 3)  # g, b, row, byte
    rec = np.concatenate([blocks[..., 2:18].reshape(ng, nb, 1024),
                          blocks[..., 18:34].reshape(ng, nb, 1024),
                          blocks[..., 0:2].reshape(ng, nb, 128)], axis=2)
    return rec.reshape(-1)


@pytest.mark.parametrize("nrows,nb,pad,off", [
    (64, 1, 0, 0), (100, 9, 16, 0), (130, 7, 0, 2), (5, 4, 2, 2),  # the per-record kernel
    (128, 16, 0, 0),   # 16-byte aligned rows: the 8-block span kernel only
    (70, 11, 10, 0),   # spans for blocks 0-7, the per-record kernel for 8-10, partial group
    (200, 24, 16, 0),  # padded 16-byte stride, 3 spans, partial last group
    (1, 8, 0, 0),      # one row
])
def test_pack_q8_0_to_gemm_tiles(hip, dev, nrows, nb, pad, off):
    a = np.pad(synth.q8_0_matrix(nrows, nb * 32, 80, 1.0), ((0, 0), (0, pad)))
    want = tiles_reference(a, nrows, nb)
    assert hip.gemm_tiles_bytes(nrows, nb) == want.size
    buf = empty_dev(a.size + 16, torch.uint8, dev)
    buf[off:off + a.size] = to_dev(a.reshape(-1), dev)  # off 2: 2-byte aligned rows
    dst = to_dev(np.full(want.size, 0xEE, np.uint8), dev)
    hip.pack_q8_0_to_gemm_tiles(nrows, nb, buf[off:off + a.size], a.shape[1], dst)
    assert np.array_equal(from_dev(dst), want)


@pytest.mark.parametrize("nr,nc,nb,xpad,ypad", [
    (256, 128, 4, 0, 0),      # one tile, only a partial chunk (6-block chunks)
    (256, 128, 6, 0, 0),      # exactly one full chunk: no DMA issued inside the fold
    (256, 128, 8, 0, 0),      # one chunk + 2 blocks
    (256, 64, 11, 0, 0),      # one chunk + 5: the tail's DMA, issued slot by slot in chunk
                              # 0's fold, skips the slots of the block it does not have
    (300, 130, 9, 16, 32),    # partial tiles both ways, 1 chunk + 3 blocks, padded strides
    (520, 257, 13, 0, 4),     # three tile rows, 2 chunks + 1 block
    (256, 2, 1, 0, 0),        # one block: only the partial chunk
    (640, 384, 130, 0, 0),    # 21 chunks + 4 blocks, groups past the last one re-read
    (512, 200, 128, 0, 0),    # 16-byte aligned rows: both operands packed by 8-block spans
])
def test_q8_0_gemm_tiles_and_ws(hip, oracle, dev, nr, nc, nb, xpad, ypad):
    n = nb * 32
    w = np.pad(synth.q8_0_matrix(nr, n, 1009, 0.02), ((0, 0), (0, xpad)))
    a = np.pad(synth.q8_0_matrix(nc, n, 1008, 1.0), ((0, 0), (0, ypad)))
    w[0, 2:34] = 0x80
    a[0, 2:34] = 0x80  # -128 x -128 block sums
    bs = nc + 3
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], nr, nc, w.shape[1], bs, 8).reshape(nr, bs)
    dw, da = to_dev(w, dev), to_dev(a, dev)
    # pre-packed operands
    tx = empty_dev(hip.gemm_tiles_bytes(nr, nb), torch.uint8, dev)
    ty = empty_dev(hip.gemm_tiles_bytes(nc, nb), torch.uint8, dev)
    hip.pack_q8_0_to_gemm_tiles(nr, nb, dw, w.shape[1], tx)
    hip.pack_q8_0_to_gemm_tiles(nc, nb, da, a.shape[1], ty)
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    hip.q8_0_q8_0_gemm_tiles(n, s, tx, ty, nr, nc, bs)
    got = from_dev(s).reshape(nr, bs)
    assert_f32_parity(got[:, :nc], want[:, :nc], what=f"tiles gemm {nr}x{nc}x{n}")
    assert np.all(got[:, nc:] == -7.0)
    # the reference ABI with a workspace
    wsb = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s2 = empty_dev(nr * bs, torch.float32, dev)
    hip.q8_0_q8_0_gemm_ws(n, s2, dw, da, a.shape[1], nr, nc, w.shape[1], bs, ws, wsb)
    assert_f32_parity(from_dev(s2).reshape(nr, bs)[:, :nc], want[:, :nc], what="gemm_ws")


@pytest.mark.parametrize("nb", [12, 13, 5])
def test_q8_0_gemm_tiles_more_tiles_than_cus(hip, oracle, dev, nb):
    """17 x 17 = 289 work-group tiles of the tiled kernel, partial ones on both
    edges: more tiles than the part has CUs, so a second round of work-groups
    runs.  K with no partial chunk (12 blocks), with one (13) and with only one
    (5).  The whole output equals the plain entry's bit for bit; sampled rows
    match the oracle."""
    nr, nc, n = 16 * 256 + 100, 16 * 128 + 70, nb * 32
    w = synth.q8_0_matrix(nr, n, 1031, 0.02)
    a = synth.q8_0_matrix(nc, n, 1032, 1.0)
    dw, da = to_dev(w, dev), to_dev(a, dev)
    bs = nc + 1
    wsb = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    hip.q8_0_q8_0_gemm_ws(n, s, dw, da, a.shape[1], nr, nc, w.shape[1], bs, ws, wsb)
    ref = empty_dev(nr * bs, torch.float32, dev)
    hip.q8_0_q8_0_gemm(n, ref, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
    got, want = from_dev(s).reshape(nr, bs), from_dev(ref).reshape(nr, bs)
    assert np.array_equal(got[:, :nc].view(np.uint32), want[:, :nc].view(np.uint32))
    assert np.all(got[:, nc:] == -7.0)
    rng = np.random.default_rng(17)
    for r in np.sort(rng.choice(nr, 16, replace=False)).tolist() + [nr - 1]:
        row = oracle.gemm_q8_0(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r, :nc], row, what=f"row {r}")


def _rounds(nr, nc, bm, bn, cus=256):
    return -(-(-(-nr // bm) * -(-nc // bn)) // cus)


@pytest.mark.parametrize("nr,nc,nb,xpad,ypad", [
    (4096, 4096, 4, 0, 0),     # exactly one 4-block chunk: no DMA issued inside the fold
    (4096, 4096, 5, 0, 0),     # one chunk + 1: chunk 0's fold issues only block 0's slots
    (4096, 4096, 3, 0, 0),     # no full chunk: the tail alone
    (4000, 4050, 13, 16, 4),   # partial tiles both ways, 3 chunks + 1, 2-byte aligned tokens
    (65536, 256, 9, 0, 0),     # one token tile, 256 weight tiles
    (256, 65536, 6, 2, 0),     # one weight tile, 256 token tiles, 2-byte aligned weights
    (8192, 4096, 7, 0, 0),     # two rounds of work-groups
])
def test_q8_0_gemm_tiles_256x256(hip, oracle, dev, nr, nc, nb, xpad, ypad):
    """Shapes that run the 256 x 256 work-group tile of the tiled Q8_0 GEMM (8 waves of
    2 x 4 32 x 32 tiles, 4-block K chunks): the pre-packed entry and the workspace entry
    equal the plain entry (another kernel, the same fold order) bit for bit over the whole
    output, the padding columns stay untouched, and sampled rows, the last included, match
    the oracle."""
    assert _rounds(nr, nc, 256, 256) * 15 <= _rounds(nr, nc, 256, 128) * 8
    n = nb * 32
    w = np.pad(synth.q8_0_matrix(nr, n, 1041, 0.02), ((0, 0), (0, xpad)))
    a = np.pad(synth.q8_0_matrix(nc, n, 1042, 1.0), ((0, 0), (0, ypad)))
    w[0, 2:34] = 0x80
    a[0, 2:34] = 0x80  # -128 x -128 block sums
    dw, da = to_dev(w, dev), to_dev(a, dev)
    bs = nc + 5
    ref = empty_dev(nr * bs, torch.float32, dev)
    hip.q8_0_q8_0_gemm(n, ref, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
    want = from_dev(ref).reshape(nr, bs)[:, :nc]
    del ref
    tx = empty_dev(hip.gemm_tiles_bytes(nr, nb), torch.uint8, dev)
    ty = empty_dev(hip.gemm_tiles_bytes(nc, nb), torch.uint8, dev)
    hip.pack_q8_0_to_gemm_tiles(nr, nb, dw, w.shape[1], tx)
    hip.pack_q8_0_to_gemm_tiles(nc, nb, da, a.shape[1], ty)
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    hip.q8_0_q8_0_gemm_tiles(n, s, tx, ty, nr, nc, bs)
    got = from_dev(s).reshape(nr, bs)
    assert np.array_equal(got[:, :nc].view(np.uint32), want.view(np.uint32)), "tiles != plain"
    assert np.all(got[:, nc:] == -7.0)
    del tx, ty
    wsb = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s.fill_(-7.0)
    hip.q8_0_q8_0_gemm_ws(n, s, dw, da, a.shape[1], nr, nc, w.shape[1], bs, ws, wsb)
    got = from_dev(s).reshape(nr, bs)
    assert np.array_equal(got[:, :nc].view(np.uint32), want.view(np.uint32)), "ws != plain"
    assert np.all(got[:, nc:] == -7.0)
    rng = np.random.default_rng(nr ^ nc)
    rows = np.unique(np.concatenate([[0, nr - 1], rng.choice(nr, 14, replace=False)]))
    sub = np.ascontiguousarray(w[rows])
    ora = oracle.gemm_q8_0(n, sub, a, a.shape[1], len(rows), nc, w.shape[1], nc, 8)
    assert_f32_parity(got[rows, :nc], ora.reshape(len(rows), nc), what=f"{nr}x{nc}x{n} rows")


@pytest.mark.parametrize("nr,nc,nb,xpad,ypad", [
    (4096, 4096, 4, 0, 0),     # exactly one 4-block chunk
    (4096, 4096, 5, 0, 0),     # one chunk + 1
    (4096, 4096, 3, 0, 0),     # the tail alone
    (4000, 4050, 13, 16, 4),   # partial tiles both ways, 3 chunks + 1, 2-byte aligned tokens
    (65536, 256, 9, 0, 0),     # one token tile
    (256, 65536, 6, 2, 0),     # one weight tile
    (8192, 4096, 7, 0, 0),     # two rounds of work-groups
])
def test_q4_0_gemm_tiles_256x256(hip, oracle, dev, nr, nc, nb, xpad, ypad):
    """The tiled Q4_0 GEMM at the shapes that run its 256 x 256 work-group tile (8 waves of
    2 x 4 transposed 32 x 32 tiles, fp32 token scales widened per chunk, stores through
    LDS): the pre-packed entry and the workspace entry equal the plain Q4_0 entry (another
    kernel, the same fold) bit for bit over the whole output, padding columns untouched,
    sampled rows, the last included, against the oracle."""
    assert _rounds(nr, nc, 256, 256) * 15 <= _rounds(nr, nc, 256, 128) * 8
    n = nb * 32
    w = np.pad(synth.q4_0_matrix(nr, n, 1043, 0.02), ((0, 0), (0, xpad)))
    a = np.pad(synth.q8_0_matrix(nc, n, 1044, 1.0), ((0, 0), (0, ypad)))
    a[0, 2:34] = 0x80
    dw, da = to_dev(w, dev), to_dev(a, dev)
    bs = nc + 5
    ref = empty_dev(nr * bs, torch.float32, dev)
    hip.q4_0_q8_0_gemm(n, ref, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
    want = from_dev(ref).reshape(nr, bs)[:, :nc]
    del ref
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    q4_tiles_gemm(hip, dev, n, w, a, nr, nc, bs, s)
    got = from_dev(s).reshape(nr, bs)
    assert np.array_equal(got[:, :nc].view(np.uint32), want.view(np.uint32)), "tiles != plain"
    assert np.all(got[:, nc:] == -7.0)
    wsb = hip.q4_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s.fill_(-7.0)
    hip.q4_0_q8_0_gemm_ws(n, s, dw, da, a.shape[1], nr, nc, w.shape[1], bs, ws, wsb)
    got = from_dev(s).reshape(nr, bs)
    assert np.array_equal(got[:, :nc].view(np.uint32), want.view(np.uint32)), "ws != plain"
    assert np.all(got[:, nc:] == -7.0)
    rng = np.random.default_rng(nr ^ nc ^ 1)
    rows = np.unique(np.concatenate([[0, nr - 1], rng.choice(nr, 14, replace=False)]))
    sub = np.ascontiguousarray(w[rows])
    ora = oracle.gemm_q4_0(n, sub, a, a.shape[1], len(rows), nc, w.shape[1], nc, 8)
    assert_f32_parity(got[rows, :nc], ora.reshape(len(rows), nc), what=f"{nr}x{nc}x{n} rows")


def test_q8_0_gemm_ws_fallbacks_and_checks(hip, oracle, dev):
    """Shapes the tiled kernels do not serve, and a few tokens with 4-byte aligned rows (the
    plain entry's multi-column GEMVs), run the plain entry and leave the workspace alone; a
    workspace that is too small or misaligned is refused."""
    n, nb = 256, 8
    for nr, nc in ((100, 70), (300, 1), (1, 40), (256, 16), (512, 24)):
        w = synth.q8_0_matrix(nr, n, 81, 0.02)
        a = synth.q8_0_matrix(nc, n, 82, 1.0)
        ws = to_dev(np.full(64, 0x5A, np.uint8), dev)
        s = empty_dev(nr * nc, torch.float32, dev)
        hip.q8_0_q8_0_gemm_ws(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc,
                              w.shape[1], nc, ws, 64)
        assert_f32_parity(from_dev(s), oracle.gemm_q8_0(n, w, a, a.shape[1], nr, nc, w.shape[1],
                                                        nc, 8))
        assert np.all(from_dev(ws) == 0x5A)
    w = synth.q8_0_matrix(256, n, 83, 0.02)
    a = synth.q8_0_matrix(72, n, 84, 1.0)  # past the multi-column GEMVs' 24 tokens
    need = hip.q8_0_q8_0_gemm_workspace_bytes(n, 256, 72)
    ws = empty_dev(need + 16, torch.uint8, dev)
    s = empty_dev(256 * 72, torch.float32, dev)
    call = lambda *args: hip.call("tcrv_hip_q8_0_q8_0_gemm_ws", n, s, to_dev(w, dev),
                                  to_dev(a, dev), a.shape[1], 256, 72, w.shape[1], 72, *args, 0,
                                  check=False)
    assert call(ws, need - 1) == hip.ERR_BAD_SIZE
    assert call(ws[8:], need) == hip.ERR_MISALIGNED
    torch.cuda.synchronize()


@pytest.mark.parametrize("quant", ["q8_0", "q4_0"])
@pytest.mark.parametrize("nr,nc,nb", [
    (4096, 130, 13),  # 32 tiles of 256 x 128; tokens end 2 rows into a record group; 7 + 6 blocks
    (300, 70, 7),     # 16 x 16 tiles: 7 blocks (less than one round of the 12 in flight)
    (1000, 600, 1),   # one block: only the clamped prologue loads
    (4100, 960, 20),  # 136 tiles of 256 x 128, 975 work-groups; two rounds and a 6-block rest
    (256, 2, 14),     # two tokens, 16 x 16 tiles: one round of 12 blocks and a 2-block rest
    (4096, 64, 29),   # 16 x 16 tiles, 256 work-groups (the bound): two rounds and a 5-block rest
])
def test_gemm_tiles_one_tile_a_wave(hip, oracle, dev, quant, nr, nc, nb):
    """Pre-packed operands where the 256-row tiles would not fill one round of the CUs: the
    kernels with one 32 x 32 or one 16 x 16 tile a wave; whole outputs against the plain entry
    bit for bit and sampled rows against the oracle, with -128 block sums and a padded output
    stride."""
    n = nb * 32
    q4 = quant == "q4_0"
    w = (synth.q4_0_matrix if q4 else synth.q8_0_matrix)(nr, n, 1030 + nb, 0.02)
    a = synth.q8_0_matrix(nc, n, 1031 + nb, 1.0)
    a[0, 2:34] = 0x80  # -128 quants: -8 x -128 (Q4_0) or -128 x -128 (Q8_0) block sums
    if q4:
        w[nr - 1, 2:18] = 0x00
    else:
        w[nr - 1, 2:34] = 0x80
    bs = nc + 5
    dw, da = to_dev(w, dev), to_dev(a, dev)
    ref = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    getattr(hip, f"{quant}_q8_0_gemm")(n, ref, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
    want = from_dev(ref).reshape(nr, bs)
    tx = empty_dev(hip.gemm_tiles_bytes(nr, nb), torch.uint8, dev)
    ty = empty_dev(hip.gemm_tiles_bytes(nc, nb), torch.uint8, dev)
    getattr(hip, f"pack_{quant}_to_gemm_tiles")(nr, nb, dw, w.shape[1], tx)
    hip.pack_q8_0_to_gemm_tiles(nc, nb, da, a.shape[1], ty)
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    getattr(hip, f"{quant}_q8_0_gemm_tiles")(n, s, tx, ty, nr, nc, bs)
    got = from_dev(s).reshape(nr, bs)
    what = f"{quant} tiles {nr}x{nc}x{n}"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), what
    ora = oracle.gemm_q4_0 if q4 else oracle.gemm_q8_0
    for r in sorted({0, nr // 2, nr - 1}):
        row = ora(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r, :nc], row, what=f"{what}, row {r}")


@pytest.mark.parametrize("quant", ["q8_0", "q4_0"])
@pytest.mark.parametrize("nr,nc,nb", [
    (4096, 130, 16),  # 192 work-groups; tokens end 2 rows into a record group; two chunks
    (300, 70, 8),     # one 8-block chunk; partial row and token groups
    (1000, 600, 40),  # five chunks
    (2100, 333, 24),
    (1000, 600, 48),  # six chunks
    (4096, 128, 128),  # the bench shape: sixteen chunks
    (4100, 300, 32),  # 325 work-groups
])
def test_gemm_plain_rows_few_tiles(hip, oracle, dev, quant, nr, nc, nb):
    """The plain entries at shapes of few output tiles with 16-byte aligned rows and whole
    8-block chunks: each work-group packs its 64 weight rows and 64 tokens into LDS records
    chunk by chunk and folds one 32 x 32 tile a wave.  Whole outputs against the pre-packed
    entry (the one-tile-a-wave kernels over the records) bit for bit, sampled rows against the
    oracle, with -128 block sums and a padded output stride."""
    n = nb * 32
    q4 = quant == "q4_0"
    w = (synth.q4_0_matrix if q4 else synth.q8_0_matrix)(nr, n, 1040 + nb, 0.02)
    a = synth.q8_0_matrix(nc, n, 1041 + nb, 1.0)
    a[nc - 1, 2:34] = 0x80
    if q4:
        w[0, 2:18] = 0x00
    else:
        w[0, 2:34] = 0x80
    bs = nc + 5
    dw, da = to_dev(w, dev), to_dev(a, dev)
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    getattr(hip, f"{quant}_q8_0_gemm")(n, s, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
    got = from_dev(s).reshape(nr, bs)
    tx = empty_dev(hip.gemm_tiles_bytes(nr, nb), torch.uint8, dev)
    ty = empty_dev(hip.gemm_tiles_bytes(nc, nb), torch.uint8, dev)
    getattr(hip, f"pack_{quant}_to_gemm_tiles")(nr, nb, dw, w.shape[1], tx)
    hip.pack_q8_0_to_gemm_tiles(nc, nb, da, a.shape[1], ty)
    s2 = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    getattr(hip, f"{quant}_q8_0_gemm_tiles")(n, s2, tx, ty, nr, nc, bs)
    want = from_dev(s2).reshape(nr, bs)
    what = f"{quant} plain {nr}x{nc}x{n}"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), what
    ora = oracle.gemm_q4_0 if q4 else oracle.gemm_q8_0
    for r in sorted({0, 1, nr // 2, nr - 1}):
        row = ora(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r, :nc], row, what=f"{what}, row {r}")


def _ws_route(nr, nc, nb, bx, by):
    """Which kernel the workspace entries run (the host's rules, restated): the plain entry's
    multi-column GEMVs for a few tokens, one tile a wave below one round of 256 x 128 tiles (and
    at most 1024 of its 64 x 64 work-groups) -- 16 x 16 while those waves fit one a SIMD, the
    plain entry's (packed in LDS) for 16-byte rows up to 448 work-groups and K 4096, else
    32 x 32 -- else the 256 x 256 or 256 x 128 tiles by the rounds rule."""
    if nc <= 24 and nb % 2 == 0 and bx % 4 == 0 and by % 4 == 0:
        return "cols"
    t64 = -(-nr // 64) * -(-nc // 64)
    if -(-nr // 256) * -(-nc // 128) < 256 and t64 <= 1024:
        if -(-nr // 32) * -(-nc // 32) <= 256:
            return "16x16"
        if nb % 8 == 0 and nb <= 128 and bx % 16 == 0 and by % 16 == 0 and t64 <= 448:
            return "plain few tiles"
        return "32x32"
    return "256x256" if _rounds(nr, nc, 256, 256) * 15 <= _rounds(nr, nc, 256, 128) * 8 \
        else "256x128"


@pytest.mark.parametrize("quant", ["q8_0", "q4_0"])
def test_gemm_ws_random_shapes(hip, oracle, dev, quant):
    """28 seeded random shapes through the workspace entry -- a few tokens, a few hundred,
    thousands, and large outputs, so every route runs (the multi-column GEMVs, the one-tile-a-wave
    kernel, both work-group tiles by the rounds rule) with every chunk and tail split -- against
    the plain entry, whole outputs bit for bit, with padded row strides and output strides; one
    sampled row of each against the oracle."""
    rng = np.random.default_rng(2026 if quant == "q8_0" else 2027)
    make = synth.q8_0_matrix if quant == "q8_0" else synth.q4_0_matrix
    wb = 34 if quant == "q8_0" else 18
    seen = set()
    for case in range(28):
        kind = case % 4
        if kind == 3:
            nr, nc = int(rng.integers(4096, 8500)), int(rng.integers(2000, 4700))
        else:
            nr = int(rng.integers(256, 4700))
            nc = int(rng.integers(*((2, 40), (40, 600), (600, 4700))[kind]))
        nb = int(rng.integers(1, 19))
        n = nb * 32
        xpad, ypad = 2 * int(rng.integers(0, 9)), 2 * int(rng.integers(0, 9))
        bs = nc + int(rng.integers(0, 5))
        seen.add(_ws_route(nr, nc, nb, nb * wb + xpad, nb * 34 + ypad))
        w = np.pad(make(nr, n, 3000 + case, 0.02), ((0, 0), (0, xpad)))
        a = np.pad(synth.q8_0_matrix(nc, n, 4000 + case, 1.0), ((0, 0), (0, ypad)))
        dw, da = to_dev(w, dev), to_dev(a, dev)
        plain = getattr(hip, f"{quant}_q8_0_gemm")
        ws_fn = getattr(hip, f"{quant}_q8_0_gemm_ws")
        wsb = getattr(hip, f"{quant}_q8_0_gemm_workspace_bytes")(n, nr, nc)
        ref = empty_dev(nr * bs, torch.float32, dev)
        plain(n, ref, dw, da, a.shape[1], nr, nc, w.shape[1], bs)
        want = from_dev(ref).reshape(nr, bs)[:, :nc]
        ws = empty_dev(wsb, torch.uint8, dev)
        s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
        ws_fn(n, s, dw, da, a.shape[1], nr, nc, w.shape[1], bs, ws, wsb)
        got = from_dev(s).reshape(nr, bs)
        what = f"{quant} case {case}: {nr}x{nc}x{n} pads {xpad},{ypad} bs {bs}"
        assert np.array_equal(got[:, :nc].view(np.uint32), want.view(np.uint32)), what
        assert np.all(got[:, nc:] == -7.0), what
        r = int(rng.integers(0, nr))
        ora = (oracle.gemm_q8_0 if quant == "q8_0" else oracle.gemm_q4_0)
        row = ora(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r, :nc], row, what=f"{what}, row {r}")
        del dw, da, ref, ws, s
    assert seen >= {"cols", "16x16", "32x32", "256x256", "256x128"}  # every route ran


def test_q8_0_gemm_ws_full_size_sampled(hip, oracle, dev):
    """4096 x 4096 x 4096 through the workspace entry; 64 rows and 64 columns
    checked against the oracle."""
    n = nr = nc = 4096
    w = synth.q8_0_matrix(nr, n, 1009, 0.02)
    a = synth.q8_0_matrix(nc, n, 1008, 1.0)
    wsb = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q8_0_q8_0_gemm_ws(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1],
                          nc, ws, wsb)
    got = from_dev(s).reshape(nr, nc)
    rng = np.random.default_rng(11)
    for r in np.sort(rng.choice(nr, 64, replace=False)):
        want = oracle.gemm_q8_0(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r], want, what=f"row {r}")
    cols = np.sort(rng.choice(nc, 64, replace=False))
    sub = np.ascontiguousarray(a[cols])
    want = oracle.gemm_q8_0(n, w, sub, sub.shape[1], nr, len(cols), w.shape[1], len(cols), 8)
    assert_f32_parity(got[:, cols], want.reshape(nr, len(cols)), what="sampled cols")


# ------------------------------------ a7 Q4_0 x Q8_0 over the GEMM-tile layout ---

def q4_tiles_reference(w, nrows, nb):
    """The Q4_0 records of the GEMM-tile layout built in numpy from plain Q4_0
    rows: each nibble decoded to (q - 8) as an int8 byte, element j < 16 from the
    low nibble of quant byte j, element 16 + j from its high nibble; the fp16
    scale bytes copied; rows past nrows zero."""
    blocks = w[:nrows, :nb * 18].reshape(nrows, nb, 18)
    q = blocks[..., 2:18].astype(np.int16)
    q8 = np.zeros((nrows, nb, 34), np.uint8)
    q8[..., 0:2] = blocks[..., 0:2]
    q8[..., 2:18] = ((q & 0x0F) - 8).astype(np.int8).view(np.uint8)
    q8[..., 18:34] = ((q >> 4) - 8).astype(np.int8).view(np.uint8)
    return tiles_reference(q8.reshape(nrows, nb * 34), nrows, nb)


@pytest.mark.parametrize("nrows,nb,pad,off", [
    (64, 1, 0, 0), (100, 9, 14, 0), (130, 7, 0, 2), (5, 4, 2, 2),
    (128, 16, 0, 0),   # 4096-wide-style rows: 16-byte aligned every 8 blocks
    (70, 11, 10, 0), (200, 24, 16, 0), (1, 8, 0, 0),
])
def test_pack_q4_0_to_gemm_tiles(hip, dev, nrows, nb, pad, off):
    w = np.pad(synth.q4_0_matrix(nrows, nb * 32, 90, 1.0), ((0, 0), (0, pad)))
    w[0, 2:18] = np.arange(16, dtype=np.uint8) * 0x11  # every nibble value, both halves
    want = q4_tiles_reference(w, nrows, nb)
    assert hip.gemm_tiles_bytes(nrows, nb) == want.size
    buf = empty_dev(w.size + 16, torch.uint8, dev)
    buf[off:off + w.size] = to_dev(w.reshape(-1), dev)
    dst = to_dev(np.full(want.size, 0xEE, np.uint8), dev)
    hip.pack_q4_0_to_gemm_tiles(nrows, nb, buf[off:off + w.size], w.shape[1], dst)
    assert np.array_equal(from_dev(dst), want)


@pytest.mark.parametrize("nr,nc,nb,xpad,ypad", [
    (256, 128, 6, 0, 0),      # one tile, one chunk
    (256, 128, 12, 0, 0),     # two chunks
    (300, 130, 9, 14, 32),    # partial tiles both ways, 1 chunk + 3 blocks, padded strides
    (520, 257, 13, 0, 4),     # three tile rows, 2 chunks + 1 block
    (256, 2, 1, 0, 0),        # one block: only the partial chunk
    (640, 384, 130, 0, 0),    # 21 chunks + 4 blocks
    (512, 200, 128, 0, 0),    # 16-byte aligned rows: both operands packed by 8-block spans
    (100, 70, 9, 0, 0),       # fewer weight rows and tokens than one work-group tile
    (300, 1, 8, 0, 0),        # one token
    (1, 40, 8, 0, 0),         # one weight row
])
def test_q4_0_gemm_tiles(hip, oracle, dev, nr, nc, nb, xpad, ypad):
    n = nb * 32
    w = np.pad(synth.q4_0_matrix(nr, n, 1019, 0.02), ((0, 0), (0, xpad)))
    a = np.pad(synth.q8_0_matrix(nc, n, 1018, 1.0), ((0, 0), (0, ypad)))
    w[0, 2:18] = 0x00
    a[0, 2:34] = 0x80  # -8 x -128 block sums
    bs = nc + 3
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], bs, 8).reshape(nr, bs)
    s = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    got = from_dev(q4_tiles_gemm(hip, dev, n, w, a, nr, nc, bs, s)).reshape(nr, bs)
    assert_f32_parity(got[:, :nc], want[:, :nc], what=f"q4 tiles gemm {nr}x{nc}x{n}")
    assert np.all(got[:, nc:] == -7.0)
    # the reference ABI with a workspace (shapes below 256 weight rows or with
    # one token run the plain entry)
    wsb = hip.q4_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(max(wsb, 16), torch.uint8, dev)
    s2 = to_dev(np.full(nr * bs, -7.0, np.float32), dev)
    hip.q4_0_q8_0_gemm_ws(n, s2, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1],
                          bs, ws, wsb)
    got2 = from_dev(s2).reshape(nr, bs)
    assert_f32_parity(got2[:, :nc], want[:, :nc], what=f"q4 gemm_ws {nr}x{nc}x{n}")
    assert np.all(got2[:, nc:] == -7.0)


def test_q4_0_gemm_tiles_checks(hip, dev):
    """No blocks: zero outputs; misaligned tiles or a short output stride are
    refused before anything launches."""
    nr, nc, nb = 256, 16, 8
    tx = empty_dev(hip.gemm_tiles_bytes(nr, nb) + 16, torch.uint8, dev)
    ty = empty_dev(hip.gemm_tiles_bytes(nc, nb), torch.uint8, dev)
    s = to_dev(np.full(nr * nc, 3.0, np.float32), dev)
    hip.q4_0_q8_0_gemm_tiles(31, s, tx, ty, nr, nc, nc)  # n < 32: no blocks
    assert np.all(from_dev(s) == 0.0)
    call = lambda *args: hip.call("tcrv_hip_q4_0_q8_0_gemm_tiles", *args, 0, check=False)
    assert call(nb * 32, s, tx[8:], ty, nr, nc, nc) == hip.ERR_MISALIGNED
    assert call(nb * 32, s, tx, ty, nr, nc, nc - 1) == hip.ERR_BAD_SIZE
    torch.cuda.synchronize()


def test_q4_0_gemm_ws_fallbacks_and_checks(hip, oracle, dev):
    """Shapes the tiled kernels do not serve, and a few tokens with 4-byte aligned rows (the
    plain entry's multi-column GEMVs), run the plain entry and leave the workspace alone; a
    workspace that is too small or misaligned is refused."""
    n, nb = 256, 8
    for nr, nc in ((100, 70), (300, 1), (1, 40), (256, 16), (512, 24)):
        w = synth.q4_0_matrix(nr, n, 85, 0.02)
        a = synth.q8_0_matrix(nc, n, 86, 1.0)
        ws = to_dev(np.full(64, 0x5A, np.uint8), dev)
        s = empty_dev(nr * nc, torch.float32, dev)
        hip.q4_0_q8_0_gemm_ws(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc,
                              w.shape[1], nc, ws, 64)
        assert_f32_parity(from_dev(s), oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1],
                                                        nc, 8))
        assert np.all(from_dev(ws) == 0x5A)
    w = synth.q4_0_matrix(256, n, 87, 0.02)
    a = synth.q8_0_matrix(72, n, 88, 1.0)  # past the multi-column GEMVs' 24 tokens
    need = hip.q4_0_q8_0_gemm_workspace_bytes(n, 256, 72)
    assert need == hip.gemm_tiles_bytes(256, nb) + hip.gemm_tiles_bytes(72, nb)
    ws = empty_dev(need + 16, torch.uint8, dev)
    s = empty_dev(256 * 72, torch.float32, dev)
    call = lambda *args: hip.call("tcrv_hip_q4_0_q8_0_gemm_ws", n, s, to_dev(w, dev),
                                  to_dev(a, dev), a.shape[1], 256, 72, w.shape[1], 72, *args, 0,
                                  check=False)
    assert call(ws, need - 1) == hip.ERR_BAD_SIZE
    assert call(ws[8:], need) == hip.ERR_MISALIGNED
    torch.cuda.synchronize()


def test_q4_0_gemm_tiles_full_size_sampled(hip, oracle, dev):
    """4096 x 4096 x 4096 Q4_0 x Q8_0 through the GEMM-tile layout and through
    the workspace entry (the two bit-identical everywhere); 64 rows and 64
    columns checked against the oracle."""
    n = nr = nc = 4096
    w = synth.q4_0_matrix(nr, n, 1006, 0.02)
    a = synth.q8_0_matrix(nc, n, 1008, 1.0)
    s = empty_dev(nr * nc, torch.float32, dev)
    got = from_dev(q4_tiles_gemm(hip, dev, n, w, a, nr, nc, nc, s)).reshape(nr, nc)
    wsb = hip.q4_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s2 = empty_dev(nr * nc, torch.float32, dev)
    hip.q4_0_q8_0_gemm_ws(n, s2, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1],
                          nc, ws, wsb)
    assert np.array_equal(from_dev(s2).reshape(nr, nc).view(np.uint32), got.view(np.uint32))
    rng = np.random.default_rng(13)
    for r in np.sort(rng.choice(nr, 64, replace=False)):
        want = oracle.gemm_q4_0(n, w[r].copy(), a, a.shape[1], 1, nc, w.shape[1], nc, 8)
        assert_f32_parity(got[r], want, what=f"row {r}")
    cols = np.sort(rng.choice(nc, 64, replace=False))
    sub = np.ascontiguousarray(a[cols])
    want = oracle.gemm_q4_0(n, w, sub, sub.shape[1], nr, len(cols), w.shape[1], len(cols), 8)
    assert_f32_parity(got[:, cols], want.reshape(nr, len(cols)), what="sampled cols")
