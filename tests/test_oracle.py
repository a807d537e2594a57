"""Pins the CPU oracle (oracle/libtcrv_oracle.so) before it is trusted.

Each test checks one oracle function against something fixed independently of
it: the reference's own add harness vector, IEEE conversions done by numpy,
exhaustive or brute-force integer sums, exact rational folds (tests/exact.py),
closed forms, and planted mistakes that must be caught.
"""
import numpy as np
import pytest

import exact
import synth

pytestmark = []

RNG = np.random.default_rng(12345)


def rand_q8_blocks(nb, rng=RNG, dmin=-14, dmax=-4):
    """Random block_q8_0 bytes: fp16 d = +-2^k * m, random int8 quants."""
    out = np.zeros((nb, 34), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.0, nb) * 2.0 ** rng.integers(dmin, dmax, nb)).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = rng.integers(0, 256, (nb, 32), dtype=np.uint8)
    return out.reshape(-1)


def rand_q4_blocks(nb, rng=RNG):
    out = np.zeros((nb, 18), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.0, nb) * 2.0 ** rng.integers(-12, -2, nb)).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return out.reshape(-1)


def q8_fields(blocks):
    b = blocks.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.int64)
    return d, q


def q4_fields(blocks):
    b = blocks.reshape(-1, 18)
    d = b[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    qs = b[:, 2:].astype(np.int64)
    vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1)  # element j, j+16
    return d, vals


# ---------------------------------------------------------------- formats ---

def test_block_format_sizes():
    # verifier constants: qk 32, strides 34 / 18 / 288 (RVVDialectWideningOps.cpp:3358-3372,
    # RVVOps.td:3893-3897, :4569-4576)
    assert synth.Q8_0_BLOCK_BYTES == 2 + 32
    assert synth.Q4_0_BLOCK_BYTES == 2 + 16
    assert 16 * 2 + 16 * 16 == 288


def test_fp16_to_f32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_f32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_fp16_round_nearest_even(oracle):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 60000, dtype=np.uint64).astype(np.uint32)
    # concentrate on the fp16 range, subnormals and exact ties
    f = bits.view(np.float32)
    f = np.concatenate([
        f[np.isfinite(f)][:20000],
        rng.normal(0, 1, 20000).astype(np.float32),
        (rng.uniform(-1, 1, 5000) * 2.0 ** -20).astype(np.float32),
        np.array([65504, 65519.996, 65520, 65536, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -25,
                  2.0 ** -26, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -0.0, 0.0,
                  np.inf, -np.inf], dtype=np.float32),
    ])
    ties = (np.arange(-2000, 2000) * 2.0 + 1) * 2.0 ** -11  # halfway between fp16 values
    f = np.concatenate([f, ties.astype(np.float32)])
    with np.errstate(over="ignore"):  # values past 65520 become inf, as intended
        want = f.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_fp16(float(v)) for v in f], dtype=np.uint16)
    assert np.array_equal(got, want)


# -------------------------------------------------------------------- a1 ---

def test_add_i32_harness_vector(oracle):
    # examples/qemu/harness_add.cpp:14-21: lhs = 3i-17, rhs = 41-2i, n = 1031,
    # scalar oracle lhs+rhs.  The closed form is i + 24.
    n = 1031
    i = np.arange(n, dtype=np.int64)
    lhs = (3 * i - 17).astype(np.int32)
    rhs = (41 - 2 * i).astype(np.int32)
    out = oracle.add_i32(lhs, rhs)
    assert np.array_equal(out, (i + 24).astype(np.int32))


def test_add_f32_closed_form(oracle):
    a = synth.uniform_f32(1001, 4099)
    b = synth.uniform_f32(1002, 4099)
    out = oracle.add_f32(a, b)
    assert np.array_equal(out.view(np.uint32), (a + b).view(np.uint32))


# -------------------------------------------------------------------- a3 ---

def test_dequant_closed_form(oracle):
    blocks = rand_q8_blocks(300)
    # special blocks: d = 0, subnormal d, full int8 range
    b = blocks.reshape(-1, 34)
    b[0, 0:2] = 0
    b[1, 0:2] = np.array([1], dtype=np.uint16).view(np.uint8)  # smallest subnormal
    b[2, 2:] = np.arange(-128, 128, 8, dtype=np.int8).view(np.uint8)
    n = 300 * 32
    y = oracle.dequantize_row_q8_0(blocks, n)
    d, q = q8_fields(blocks)
    want = (q.astype(np.float32) * d[:, None]).reshape(-1)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    assert not np.any(y[:32])


# ------------------------------------------------------------------- a3b ---

Q4_SPECIAL_D = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03ff, 0x7bff, 0xfbff, 0x3c00,
                         0xbc00, 0x7c00, 0xfc00, 0x7e00, 0x2e66], dtype=np.uint16)


def q4_dequant_numpy(blocks):
    """Independent statement of ggml's dequantize_row_q4_0: element j is the low
    nibble of byte j minus 8, element j + 16 the high nibble minus 8, times d."""
    d, vals = q4_fields(blocks)
    with np.errstate(invalid="ignore"):  # 0 * inf
        return (vals.astype(np.float32) * d[:, None]).reshape(-1)


def same_bits_or_nan(got, want):
    nan = np.isnan(want)
    return (np.array_equal(np.isnan(got), nan)
            and np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)))


def test_dequant_q4_0_every_byte_and_special_scales(oracle):
    # all 256 weight bytes (16 blocks of 16) under each special fp16 scale:
    # +-0, +-smallest subnormal, largest subnormal, +-65504, +-1, +-inf, NaN, 0.1
    qs = np.arange(256, dtype=np.uint8).reshape(16, 16)
    for h in Q4_SPECIAL_D:
        blocks = np.zeros((16, 18), dtype=np.uint8)
        blocks[:, 0:2] = np.array([h], dtype=np.uint16).view(np.uint8)
        blocks[:, 2:] = qs
        y = oracle.dequantize_row_q4_0(blocks.reshape(-1), 16 * 32)
        d = np.float32(np.array([h], dtype=np.uint16).view(np.float16)[0])
        # closed form per element: (nibble - 8) * d, nibble table from the byte
        lo = (qs.astype(np.int64) & 15) - 8
        hi = (qs.astype(np.int64) >> 4) - 8
        with np.errstate(invalid="ignore"):
            want = np.concatenate([lo, hi], axis=1).astype(np.float32) * d
        assert same_bits_or_nan(y, want.reshape(-1)), hex(h)
        assert same_bits_or_nan(y, q4_dequant_numpy(blocks.reshape(-1))), hex(h)
    # the offset-binary table itself: 0 -> -8, 8 -> 0, 15 -> +7 (RVVOps.td:3837-3838)
    one = np.zeros(18, dtype=np.uint8)
    one[0:2] = np.array([0x3c00], dtype=np.uint16).view(np.uint8)
    one[2:5] = [0x80, 0x08, 0xF0]
    y = oracle.dequantize_row_q4_0(one, 32)
    assert list(y[:3]) == [-8.0, 0.0, -8.0] and list(y[16:19]) == [0.0, -8.0, 7.0]


def test_dequant_q4_0_planted_mistakes_fail(oracle):
    # a plausible mistake in the element order or decode changes the output:
    # interleaved order (lo, hi of byte 0, then byte 1, ...), halves swapped,
    # nibbles without the -8 offset, the Q8_0 two's-complement reading
    blocks = rand_q4_blocks(64)
    y = oracle.dequantize_row_q4_0(blocks, 64 * 32)
    d, vals = q4_fields(blocks)
    interleaved = np.stack([vals[:, :16], vals[:, 16:]], axis=2).reshape(64, 32)
    swapped = np.concatenate([vals[:, 16:], vals[:, :16]], axis=1)
    unbiased = vals + 8
    raw = vals + 8  # the nibbles 0..15
    twos = np.where(raw < 8, raw, raw - 16)  # sign-extended without the 0x88 bias
    for wrong in (interleaved, swapped, unbiased, twos):
        assert not np.array_equal(y, (wrong.astype(np.float32) * d[:, None]).reshape(-1))
    assert np.array_equal(y.view(np.uint32), q4_dequant_numpy(blocks).view(np.uint32))


def test_dequant_q4_0_matches_block_dot_integer_core(oracle):
    # The op pairs the low nibble of byte j with activation quant j and the high
    # nibble with quant 16 + j (RVVOps.td:3841-3842).  With d = 1 the dequant's
    # values are the decoded integers, so their dot with a Q8_0 block's quants
    # must equal the integer core's block sum (pinned separately by brute force).
    rng = np.random.default_rng(31)
    xb = rand_q4_blocks(40, rng)
    x = xb.reshape(-1, 18)
    x[:, 0:2] = np.array([0x3c00], dtype=np.uint16).view(np.uint8)
    yb = rand_q8_blocks(40, rng).reshape(-1, 34)
    vals = oracle.dequantize_row_q4_0(xb, 40 * 32).reshape(40, 32).astype(np.int64)
    for k in range(40):
        want = int(np.dot(vals[k], yb[k, 2:].view(np.int8).astype(np.int64)))
        assert oracle.q4_block_sumi(x[k].copy(), yb[k].copy()) == want


def test_dequant_q4_0_round_trip_and_partial_block(oracle):
    # dequant(quantize_q4_0(x)) stays within |d| (+ the fp16 rounding of d times
    # 8) of x: an element at -8/+7.5..8 steps of d saturates to 15 (7 d) at most
    # one step away, every other element rounds to the nearest step
    x = synth.normal_f32(77, 64 * 32, 0.0, 0.02)
    q = oracle.quantize_q4_0(x)
    y = oracle.dequantize_row_q4_0(q, x.size + 17)  # the trailing 17 elements are dropped
    assert y.size == x.size
    xb = x.reshape(-1, 32)
    amax_idx = np.argmax(np.abs(xb), axis=1)
    d32 = xb[np.arange(xb.shape[0]), amax_idx] / -8.0
    d16 = q.reshape(-1, 18)[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    err = np.abs(y.reshape(-1, 32) - xb)
    bound = np.abs(d32)[:, None] * (1 + 1e-6) + 8 * np.abs(d16 - d32)[:, None]
    assert np.all(err <= bound)


# -------------------------------------------------------------------- a4 ---

def test_q4_integer_core_exhaustive_weight_bytes(oracle):
    rng = np.random.default_rng(3)
    for w in range(256):
        xb = np.zeros(18, dtype=np.uint8)
        xb[2:] = w
        lo, hi = (w & 15) - 8, (w >> 4) - 8
        for _ in range(4):
            yb = rand_q8_blocks(1, rng)
            q = yb[2:].view(np.int8).astype(np.int64)
            want = int(lo * q[:16].sum() + hi * q[16:].sum())
            assert oracle.q4_block_sumi(xb, yb) == want


def test_q4_integer_core_bounds(oracle):
    xb = np.zeros(18, dtype=np.uint8)  # every nibble 0 -> value -8
    yb = np.zeros(34, dtype=np.uint8)
    yb[2:] = np.uint8(0x80)  # -128
    assert oracle.q4_block_sumi(xb, yb) == 32 * 8 * 128


def test_q4_block_sums_bruteforce(oracle):
    nb = 64
    vx, vy = rand_q4_blocks(nb), rand_q8_blocks(nb)
    _, xv = q4_fields(vx)
    _, yq = q8_fields(vy)
    want = (xv * yq).sum(axis=1)
    assert np.array_equal(oracle.block_sums_q4_0(nb * 32, vx, vy), want.astype(np.int32))


# -------------------------------------------------------------------- a5 ---

def test_q8_block_sums_bruteforce_and_bounds(oracle):
    nb = 96
    vx, vy = rand_q8_blocks(nb), rand_q8_blocks(nb)
    vx.reshape(-1, 34)[0, 2:] = 0x80
    vy.reshape(-1, 34)[0, 2:] = 0x80
    _, xq = q8_fields(vx)
    _, yq = q8_fields(vy)
    want = (xq * yq).sum(axis=1)
    got = oracle.block_sums_q8_0(nb * 32, vx, vy)
    assert np.array_equal(got, want.astype(np.int32))
    assert got[0] == 524288


def exact_fold_q8(vx, vy, nb):
    dx, xq = q8_fields(vx)
    dy, yq = q8_fields(vy)
    acc = np.float32(0.0)
    for b in range(nb):
        s = int((xq[b] * yq[b]).sum())
        acc = exact.fma32(np.float32(s), exact.mul32(dx[b], dy[b]), acc)
    return acc


def exact_fold_q4(vx, vy, nb):
    dx, xv = q4_fields(vx)
    dy, yq = q8_fields(vy)
    acc = np.float32(0.0)
    for b in range(nb):
        s = int((xv[b] * yq[b]).sum())
        acc = exact.fma32(exact.mul32(np.float32(s), dx[b]), dy[b], acc)
    return acc


def test_exact_helper_matches_ieee():
    rng = np.random.default_rng(11)
    a = rng.normal(size=500).astype(np.float32)
    b = rng.normal(size=500).astype(np.float32)
    for x, y in zip(a, b):
        assert exact.mul32(x, y) == np.float32(x * y)  # numpy float32 mul is IEEE
        assert exact.fma32(x, np.float32(1.0), y) == np.float32(x + y)


def test_q8_fold_single_block_closed_form(oracle):
    for seed in range(20):
        rng = np.random.default_rng(seed)
        vx, vy = rand_q8_blocks(1, rng), rand_q8_blocks(1, rng)
        dx, xq = q8_fields(vx)
        dy, yq = q8_fields(vy)
        s = int((xq * yq).sum())
        # one block: round(S * (dx*dy)), dx*dy exact in binary32 and S*dx*dy exact in binary64
        want = np.float32(float(s) * (float(dx[0]) * float(dy[0])))
        assert oracle.vec_dot_q8_0(32, vx, vy) == want
    assert oracle.vec_dot_q8_0(0, vx, vy) == 0.0
    assert oracle.vec_dot_q8_0(31, vx, vy) == 0.0  # nb = n/32 drops the remainder


def test_q8_fold_matches_exact_and_catches_mistakes(oracle):
    nb = 8
    mism_rev = mism_q4order = mism_unfused = 0
    for seed in range(40):
        rng = np.random.default_rng(100 + seed)
        vx, vy = rand_q8_blocks(nb, rng, -3, 2), rand_q8_blocks(nb, rng, -3, 2)
        want = exact_fold_q8(vx, vy, nb)
        got = oracle.vec_dot_q8_0(nb * 32, vx, vy)
        assert got.view(np.uint32) == np.float32(want).view(np.uint32)
        # planted mistakes (CPU-only variants of the fold) must change some results
        dx, xq = q8_fields(vx)
        dy, yq = q8_fields(vy)
        sums = [(xq[b] * yq[b]).sum() for b in range(nb)]
        acc = np.float32(0)
        for b in reversed(range(nb)):
            acc = exact.fma32(np.float32(sums[b]), exact.mul32(dx[b], dy[b]), acc)
        mism_rev += acc != want
        acc = np.float32(0)
        for b in range(nb):
            acc = exact.fma32(exact.mul32(np.float32(sums[b]), dx[b]), dy[b], acc)
        mism_q4order += acc != want
        acc = np.float32(0)
        for b in range(nb):
            acc = np.float32(acc + exact.mul32(np.float32(sums[b]), exact.mul32(dx[b], dy[b])))
        mism_unfused += acc != want
    assert mism_rev > 0 and mism_q4order > 0 and mism_unfused > 0


def test_q8_fold_fp64_error_bound(oracle):
    n, rows = 4096, 16
    vx = synth.q8_0_matrix(rows, n, 1004, 1.0)
    vy = synth.q8_0_matrix(rows, n, 1005, 1.0)
    got = oracle.vec_dot_q8_0_rows(n, vx, vx.shape[1], vy, vy.shape[1], rows)
    nb = n // 32
    for r in range(rows):
        dx, xq = q8_fields(vx[r])
        dy, yq = q8_fields(vy[r])
        terms = (xq * yq).sum(axis=1).astype(np.float64) * (dx.astype(np.float64) * dy)
        exact_sum = terms.sum()
        bound = np.abs(terms).sum() * nb * 2.0 ** -24
        assert abs(float(got[r]) - exact_sum) <= bound


# -------------------------------------------------------------------- a6 ---

def test_q4_fold_matches_exact_and_catches_mistakes(oracle):
    nb = 8
    mism_q8order = 0
    for seed in range(40):
        rng = np.random.default_rng(200 + seed)
        vx, vy = rand_q4_blocks(nb, rng), rand_q8_blocks(nb, rng, -3, 2)
        if seed % 2:
            # correlated signs give |sumi| ~ 2^14, so fl(sumi*d_x) really rounds
            _, xv = q4_fields(vx)
            mag = rng.integers(100, 128, xv.shape)
            yb = vy.reshape(nb, 34)
            yb[:, 2:] = (np.where(xv < 0, -mag, mag)).astype(np.int8).view(np.uint8)
        want = exact_fold_q4(vx, vy, nb)
        got = oracle.vec_dot_q4_0(nb * 32, vx, vy)
        assert got.view(np.uint32) == np.float32(want).view(np.uint32)
        dx, xv = q4_fields(vx)
        dy, yq = q8_fields(vy)
        acc = np.float32(0)
        for b in range(nb):
            s = (xv[b] * yq[b]).sum()
            acc = exact.fma32(np.float32(s), exact.mul32(dx[b], dy[b]), acc)
        mism_q8order += acc != want
    assert mism_q8order > 0


def test_q4_fold_single_block(oracle):
    rng = np.random.default_rng(5)
    vx, vy = rand_q4_blocks(1, rng), rand_q8_blocks(1, rng)
    dx, xv = q4_fields(vx)
    dy, yq = q8_fields(vy)
    s = int((xv * yq).sum())
    want = exact.fma32(exact.mul32(np.float32(s), dx[0]), dy[0], np.float32(0))
    assert oracle.vec_dot_q4_0(32, vx, vy) == want


def test_rows_thread_count_invariant(oracle):
    n, rows = 1024, 64
    vx = synth.q4_0_matrix(rows, n, 21, 0.02)
    vy = synth.q8_0_matrix(rows, n, 22, 1.0)
    a = oracle.vec_dot_q4_0_rows(n, vx, vx.shape[1], vy, vy.shape[1], rows, 1)
    b = oracle.vec_dot_q4_0_rows(n, vx, vx.shape[1], vy, vy.shape[1], rows, 4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ----------------------------------------------------------------- a7/a9 ---

@pytest.mark.parametrize("fmt", ["q4", "q8"])
def test_gemm_elements_are_independent_block_dots(oracle, fmt):
    n, nr, nc = 96, 5, 3
    bx_pad, by_pad, bs = 16 if fmt == "q8" else 8, 32, 7
    xbytes = (n // 32) * (18 if fmt == "q4" else 34)
    bx = xbytes + bx_pad
    by = (n // 32) * 34 + by_pad
    rng = np.random.default_rng(9)
    vx = rng.integers(0, 256, nr * bx, dtype=np.uint8)
    vy = rng.integers(0, 256, nc * by, dtype=np.uint8)
    for r in range(nr):  # sane fp16 scales
        for b in range(n // 32):
            o = r * bx + b * (18 if fmt == "q4" else 34)
            vx[o:o + 2] = np.array([rng.uniform(0.01, 0.1)], np.float16).view(np.uint8)
    for c in range(nc):
        for b in range(n // 32):
            o = c * by + b * 34
            vy[o:o + 2] = np.array([rng.uniform(0.01, 0.1)], np.float16).view(np.uint8)
    gemm = oracle.gemm_q4_0 if fmt == "q4" else oracle.gemm_q8_0
    dot = oracle.vec_dot_q4_0 if fmt == "q4" else oracle.vec_dot_q8_0
    s = gemm(n, vx, vy, by, nr, nc, bx, bs)
    for r in range(nr):
        for c in range(nc):
            x = np.ascontiguousarray(vx[r * bx:r * bx + xbytes])
            y = np.ascontiguousarray(vy[c * by:c * by + (n // 32) * 34])
            assert s[r * bs + c] == dot(n, x, y)


def test_gemm_q8_tiny_bruteforce(oracle):
    n, nr, nc = 64, 6, 4
    vx = synth.q8_0_matrix(nr, n, 31, 0.02)
    vy = synth.q8_0_matrix(nc, n, 32, 1.0)
    s = oracle.gemm_q8_0(n, vx, vy, vy.shape[1], nr, nc, vx.shape[1], nc)
    for r in range(nr):
        for c in range(nc):
            assert s[r * nc + c] == np.float32(exact_fold_q8(vx[r], vy[c], n // 32))


# ---------------------------------------------------------------- a10/a11 ---

def test_quantize_q8_0_closed_form_and_special_cases(oracle):
    x = synth.normal_f32(77, 32 * 200, 0.0, 1.0)
    x[:32] = 0.0                      # all-zero block: d = 0, id = 0, q = 0
    x[32:64] = np.arange(32) - 15.5   # halves: x*id ties for some lanes
    x[64:96] = 1e-30                  # tiny: d underflows to fp16 zero, q = 127
    got = oracle.quantize_q8_0(x)
    assert np.array_equal(got, synth.quantize_q8_0(x))
    blocks = got.reshape(-1, 34)
    assert not blocks[0].any()
    amax_lane = np.abs(x.reshape(-1, 32)).argmax(axis=1)
    q = blocks[:, 2:].view(np.int8)
    assert np.all(np.abs(q[np.arange(200), amax_lane][1:]) == 127)
    # round trip: |dequant(quant(x)) - x| <= d/2 + fp16 rounding of d
    d = blocks[:, 0:2].copy().view(np.float16).reshape(-1).astype(np.float32)
    deq = oracle.dequantize_row_q8_0(got, x.size).reshape(-1, 32)
    err = np.abs(deq - x.reshape(-1, 32))[3:]
    assert np.all(err <= d[3:, None] * 0.5 + np.abs(x.reshape(-1, 32)[3:]) * 2e-3)


def test_quantize_q8_0_rne_ties(oracle):
    # amax = 127 -> d = 1, id = 1, so q = rne(x): 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -0.5 -> -0
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5]
    q = oracle.quantize_q8_0(x)[2:].view(np.int8)
    assert list(q[:9]) == [127, 0, 2, 2, 0, -2, -2, 4, 126]


# The reference quantizer converts with vfncvt_x_f_w_i16m4 then vncvt_x_x_w_i8m2
# (RVVOps.td:8376-8377).  RVV 1.0 specifies the first as a narrowing
# float-to-signed-integer conversion under the dynamic rounding mode (frm = RNE),
# with the F extension's invalid-input results (RISC-V unprivileged spec, "Single-
# Precision Floating-Point Conversion": NaN and +inf or any positive value above
# the range give the largest integer, -inf or any negative value below it the
# smallest), and the second as vnsrl.wx with shift 0 (the low SEW bits).  Each row:
# the product x*id the quantizer forms, the i16 the rule gives, the byte stored.
RVV_VFNCVT_RULE = [
    ("NaN", np.nan, 32767, 0xFF),
    ("+inf", np.inf, 32767, 0xFF),
    ("-inf", -np.inf, -32768, 0x00),
    ("RNE tie to even, 2.5", 2.5, 2, 0x02),
    ("RNE tie to even, 3.5", 3.5, 4, 0x04),
    ("RNE tie to even, -2.5", -2.5, -2, 0xFE),
    ("in range, -127", -127.0, -127, 0x81),
]


def test_quantize_conversion_follows_the_rvv_vfncvt_rule(oracle):
    """The oracle's bytes for products that hit each row of the rule table."""
    rows = {name: (i16, byte) for name, _, i16, byte in RVV_VFNCVT_RULE}
    for name, v, i16, byte in RVV_VFNCVT_RULE:  # the table is self-consistent
        assert (i16 & 0xFF) == byte, name
    # amax = 127 -> d = 1, id = 1: the products are the inputs themselves
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:4] = [2.5, 3.5, -2.5]
    x[4] = -127.0
    x[5] = np.nan  # skipped by amax (0.0-seeded max), NaN*1 = NaN
    q = oracle.quantize_q8_0(x)[2:]
    assert q[1] == rows["RNE tie to even, 2.5"][1]
    assert q[2] == rows["RNE tie to even, 3.5"][1]
    assert q[3] == rows["RNE tie to even, -2.5"][1]
    assert q[4] == rows["in range, -127"][1]
    assert q[5] == rows["NaN"][1]
    # subnormal amax: d = amax/127 is so small that id = 1/d overflows to +inf,
    # so a positive input's product is +inf, a negative one's -inf, 0*inf = NaN
    x = np.zeros(32, np.float32)
    x[0] = 1e-40
    x[1] = -1e-40
    q = oracle.quantize_q8_0(x)[2:]
    with np.errstate(over="ignore"):
        assert np.isinf(np.float32(1.0) / (np.float32(1e-40) / np.float32(127.0)))
    assert q[0] == rows["+inf"][1]
    assert q[1] == rows["-inf"][1]
    assert q[2] == rows["NaN"][1]


def test_quantize_q4_0_matches_host_quantizer(oracle):
    x = synth.normal_f32(1006, 32 * 500, 0.0, 0.02)
    x[:32] = 0.0
    got = oracle.quantize_q4_0(x)
    assert np.array_equal(got, synth.quantize_q4_0(x))
    # the element of largest magnitude maps to nibble 0 (value -8): x = max = -8*d
    b = got.reshape(-1, 18)
    idx = np.abs(x.reshape(-1, 32)).argmax(axis=1)
    nib = np.where(idx < 16, b[np.arange(500), 2 + idx % 16] & 15,
                   b[np.arange(500), 2 + idx % 16] >> 4)
    assert np.all(nib[1:] == 0)


# -------------------------------------------------------------------- a8 ---

def unpack_q4_0x16(packed, nblocks):
    out = np.zeros((nblocks * 16, 18), dtype=np.uint8)
    p = packed.reshape(nblocks, 288)
    for o in range(nblocks):
        for i in range(16):
            out[o * 16 + i, 0:2] = p[o, 2 * i:2 * i + 2]
        qs = p[o, 32:] ^ 0x88
        for i in range(256):
            out[o * 16 + i % 16, 2 + i // 16] = qs[i]
    return out.reshape(-1)


def test_pack_q4_0x16_round_trip(oracle):
    src = rand_q4_blocks(64)
    packed = oracle.pack_q4_0x16(src, 4)
    assert np.array_equal(unpack_q4_0x16(packed, 4), src)


def test_repack_gemv_alternate_fold(oracle):
    n, nc = 128, 32
    nb = n // 32
    w = synth.q4_0_matrix(nc, n, 41, 0.02)      # nc rows x nb blocks
    y = synth.q8_0_matrix(1, n, 42, 1.0).reshape(-1)
    # group x, block b gathers block b of rows 16x..16x+15
    src = np.concatenate([w[16 * x + r, 18 * b:18 * b + 18]
                          for x in range(nc // 16) for b in range(nb) for r in range(16)])
    packed = oracle.pack_q4_0x16(src, (nc // 16) * nb)
    got = oracle.repack_gemv_q4_0(n, packed, y, nc)
    dy, yq = q8_fields(y)
    for row in range(nc):
        dx, xv = q4_fields(w[row])
        acc = np.float32(0)
        for b in range(nb):
            s = int((xv[b] * yq[b]).sum())
            acc = exact.fma32(np.float32(s), exact.mul32(dx[b], dy[b]), acc)
        assert got[row] == acc


def unpack_q8_0x16_np(packed, nblocks):
    """Independent numpy inverse of the block_q8_0x16 interleave
    (qs[i*16 + r] = quant i of block r, scales d[r] at 2r)."""
    p = packed.reshape(nblocks, 544)
    out = np.zeros((nblocks, 16, 34), dtype=np.uint8)
    out[:, :, 0:2] = p[:, 0:32].reshape(nblocks, 16, 2)
    out[:, :, 2:] = p[:, 32:].reshape(nblocks, 32, 16).transpose(0, 2, 1)
    return out.reshape(-1)


def test_pack_q8_0x16_round_trip(oracle):
    src = rand_q8_blocks(16 * 5)
    packed = oracle.pack_q8_0x16(src, 5)
    assert np.array_equal(unpack_q8_0x16_np(packed, 5), src)
    assert np.array_equal(oracle.unpack_q8_0x16(packed, 5), src)
    q4 = rand_q4_blocks(16 * 3)
    assert np.array_equal(oracle.unpack_q4_0x16(oracle.pack_q4_0x16(q4, 3), 3), q4)


def x16_gather(w, nb, row_bytes_per_block):
    """Plain rows (nc x nb blocks) -> the source order of the x16 pack: group x,
    block b takes block b of rows 16x .. 16x+15."""
    nc = w.shape[0]
    k = row_bytes_per_block
    return np.concatenate([w[16 * x + r, k * b:k * b + k]
                           for x in range(nc // 16) for b in range(nb) for r in range(16)])


def test_repack_gemv_q8_equals_plain_gemm(oracle):
    """The Q8_0 repacked GEMV folds fma((float)sumi, d_w*d_a, acc) -- the same
    fold as the plain Q8_0 block dot -- so on the same bytes it must equal the
    (separately pinned) plain GEMM bit for bit."""
    n, nc = 4 * 32 * 9, 48
    nb = n // 32
    w = synth.q8_0_matrix(nc, n, 51, 0.02)
    y = synth.q8_0_matrix(1, n, 52, 1.0).reshape(-1)
    w[3, 2:34] = 0x80  # -128 x -128 block
    y[2:34] = 0x80
    packed = oracle.pack_q8_0x16(x16_gather(w, nb, 34), (nc // 16) * nb)
    got = oracle.repack_gemv_q8_0(n, packed, y, nc)
    want = oracle.gemm_q8_0(n, w, y, 0, nc, 1, w.shape[1], 1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_repack_gemv_q8_exact_fold_and_trailing_columns(oracle):
    n, nc = 96, 40           # nc % 16 != 0: the last 8 columns are not written
    nb = n // 32
    w = synth.q8_0_matrix(48, n, 53, 0.02)
    y = synth.q8_0_matrix(1, n, 54, 1.0).reshape(-1)
    packed = oracle.pack_q8_0x16(x16_gather(w[:32], nb, 34), 2 * nb)
    got = oracle.repack_gemv_q8_0(n, packed, y, nc)
    dy, yq = q8_fields(y)
    for row in range(32):
        dx, xq = q8_fields(w[row])
        acc = np.float32(0)
        for b in range(nb):
            s = int((xq[b] * yq[b]).sum())
            acc = exact.fma32(np.float32(s), exact.mul32(dx[b], dy[b]), acc)
        assert got[row] == acc
    assert np.all(got[32:] == 0)


def unpack_q8_0x4_np(packed, ngroups, nb):
    """Independent numpy inverse of block_q8_0x4 (scale of row c at bytes 2c,
    quant e of row c at qs[4e + c]): back to 4 plain rows per group."""
    p = packed.reshape(ngroups, nb, 136)
    out = np.zeros((ngroups, 4, nb, 34), dtype=np.uint8)
    out[:, :, :, 0:2] = p[:, :, 0:8].reshape(ngroups, nb, 4, 2).transpose(0, 2, 1, 3)
    out[:, :, :, 2:] = p[:, :, 8:].reshape(ngroups, nb, 32, 4).transpose(0, 3, 1, 2)
    return out.reshape(ngroups * 4, nb * 34)


def test_pack_q8_0x4_round_trip(oracle):
    nr, nb = 12, 5
    a = synth.q8_0_matrix(nr, nb * 32, 55, 1.0)
    packed = oracle.pack_q8_0x4(a, nr, nb, a.shape[1])
    assert packed.size == nr // 4 * nb * 136
    assert np.array_equal(unpack_q8_0x4_np(packed, nr // 4, nb), a)
    # a padded source stride reads the same rows
    ap = np.pad(a, ((0, 0), (0, 6)))
    assert np.array_equal(oracle.pack_q8_0x4(ap, nr, nb, ap.shape[1]), packed)


def test_repack_gemm_rows_equal_the_repack_gemv(oracle):
    """Every activation row of the repack GEMM is the (separately pinned) x16
    GEMV of that row: same nibble decode, same i16 lo/hi sums, same fold
    fma((float)sumi, d_w*d_a, acc).  Trailing activation rows (nr % 4) and
    weight rows (nc % 16) are not written."""
    nb, nc, nr = 7, 40, 10
    n = nb * 32
    w = synth.q4_0_matrix(nc, n, 56, 0.02)
    a = synth.q8_0_matrix(nr, n, 57, 1.0)
    a[1, 2:34] = 0x80          # -128 activations ...
    w[5, 2:18] = 0x00          # ... against -8 weights: the i16 lo/hi bound (16 * 1024)
    groups = nc // 16
    packed = oracle.pack_q4_0x16(x16_gather(w[:16 * groups], nb, 18), groups * nb)
    ax4 = oracle.pack_q8_0x4(a, nr, nb, a.shape[1])
    bs = nc + 3
    got = oracle.repack_gemm_q4_0(n, packed, ax4, nr, nc, bs).reshape(nr, bs)
    for c in range(nr // 4 * 4):
        want = oracle.repack_gemv_q4_0(n, packed, a[c].copy(), nc)
        assert np.array_equal(got[c, :16 * groups].view(np.uint32),
                              want[:16 * groups].view(np.uint32)), c
    assert np.all(got[:, 16 * groups:] == 0)
    assert np.all(got[nr // 4 * 4:] == 0)


BINARY_ELEMS = [(0, np.int8), (1, np.uint8), (2, np.int16), (3, np.uint16), (4, np.int32),
                (5, np.uint32), (6, np.int64), (7, np.float32), (8, np.float64)]


def binary_inputs(dtype, n, seed):
    rng = np.random.default_rng(seed)
    if np.issubdtype(dtype, np.integer):
        info = np.iinfo(dtype)
        a = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
        b = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
        a[:4] = [info.min, info.max, info.max, 0]  # overflow / wrap cases
        b[:4] = [info.min, 1, info.max, info.min]
    else:
        a = rng.standard_normal(n).astype(dtype) * dtype(1e3)
        b = rng.standard_normal(n).astype(dtype)
        tiny = np.finfo(dtype).smallest_subnormal
        a[:4] = [tiny, np.finfo(dtype).max, -0.0, np.inf]
        b[:4] = [tiny, np.finfo(dtype).max, 0.0, 1.0]
    return a, b


@pytest.mark.parametrize("elem,dtype", BINARY_ELEMS)
@pytest.mark.parametrize("kind", [0, 1, 2])
def test_binary_matches_numpy(oracle, kind, elem, dtype):
    """numpy's fixed-width integer ops wrap and its float ops are single IEEE
    operations -- the semantics of RVV vadd/vsub/vmul and vfadd/vfsub/vfmul."""
    a, b = binary_inputs(dtype, 1031, 10 * kind + elem)
    with np.errstate(over="ignore", invalid="ignore"):
        want = (a + b) if kind == 0 else (a - b) if kind == 1 else (a * b)
    got = oracle.binary(kind, elem, a, b)
    assert np.array_equal(got.view(np.uint8), want.astype(dtype).view(np.uint8))


def test_binary_i32_add_is_the_harness(oracle):
    n = 1031
    i = np.arange(n, dtype=np.int64)
    a = (3 * i - 17).astype(np.int32)
    b = (41 - 2 * i).astype(np.int32)
    assert np.array_equal(oracle.binary(0, 4, a, b), (i + 24).astype(np.int32))


# ------------------------------------------------ split (SoA) Q4_0 layout ---

def test_pack_q4_0_soa_matches_an_independent_gather_and_round_trips(oracle):
    """The split layout is a byte permutation: quants of (row r, block b) at
    (r*nb + b)*16, scales after all quants at (r*nb + b)*2 -- checked with a
    numpy gather written here, on padded rows (bx > the row bytes)."""
    nrows, nb, pad = 5, 7, 6
    plain = synth.q4_0_matrix(nrows, nb * 32, 71, 0.02)
    rows = np.pad(plain, ((0, 0), (0, pad)))
    bx = rows.shape[1]
    soa = oracle.pack_q4_0_soa(np.ascontiguousarray(rows).reshape(-1), nrows, nb, bx)
    blocks = plain.reshape(nrows * nb, 18)
    assert np.array_equal(soa[:nrows * nb * 16].reshape(-1, 16), blocks[:, 2:])
    assert np.array_equal(soa[nrows * nb * 16:].reshape(-1, 2), blocks[:, :2])
    assert np.array_equal(oracle.unpack_q4_0_soa(soa, nrows, nb), plain.reshape(-1))


# ------------------------------------- a4 standalone kernel (integer core) ---

def test_int_core_reduce_equals_block_sums(oracle):
    """The standalone a4 kernel over the 16 weight bytes of a Q4_0 block and the
    two halves of a Q8_0 block is the block's integer core (already pinned by
    brute force above): out = acc + block_sumi, for every block of a matrix."""
    import synth
    rng = np.random.default_rng(41)
    x = synth.q4_0_matrix(4, 32 * 64, 42, 0.02).reshape(-1, 18)
    y = synth.q8_0_matrix(4, 32 * 64, 43, 1.0).reshape(-1, 34)
    for k in range(x.shape[0]):
        w = np.ascontiguousarray(x[k, 2:]).view(np.int8)
        qlo = np.ascontiguousarray(y[k, 2:18]).view(np.int8)
        qhi = np.ascontiguousarray(y[k, 18:]).view(np.int8)
        acc = int(rng.integers(-1000, 1000))
        assert oracle.int_core_reduce(w, qlo, qhi, acc) == \
            acc + oracle.q4_block_sumi(np.ascontiguousarray(x[k]), np.ascontiguousarray(y[k]))


def test_int_core_reduce_brute_force_every_weight_byte(oracle):
    """All 256 weight bytes against the (nibble - 8) definition (RVVOps.td:
    3837-3840) with extreme activations, summed in int64 and wrapped to int32."""
    rng = np.random.default_rng(44)
    w = np.resize(np.arange(256, dtype=np.uint8), 4096)
    qlo = rng.integers(-128, 128, w.size).astype(np.int8)
    qhi = rng.integers(-128, 128, w.size).astype(np.int8)
    qlo[:256] = -128
    qhi[:256] = 127
    lo = (w & 0xF).astype(np.int64) - 8
    hi = (w >> 4).astype(np.int64) - 8
    for acc in (0, -7, 2**31 - 1 - 10):
        want = acc + int(np.sum(lo * qlo.astype(np.int64) + hi * qhi.astype(np.int64)))
        want = (want + 2**31) % 2**32 - 2**31  # the int32 cell wraps
        assert oracle.int_core_reduce(w.view(np.int8), qlo, qhi, acc) == want
    assert oracle.int_core_reduce(w.view(np.int8)[:0], qlo[:0], qhi[:0], 123) == 123
