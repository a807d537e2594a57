"""GPU parity at special values: fp16 block scales of +-0, subnormal, the
largest finite, +-Inf and NaN planted into the operands of every block-dot,
GEMV and GEMM kernel, and quantize_row_q8_0 fed NaN, +-Inf, a subnormal amax
and an amax whose fp16 scale overflows.  Each GPU result is checked against the
oracle on the same bytes: bit-identical everywhere, NaN exactly where the
oracle has NaN (assert_f32_parity_nan).

The scale product d_x*d_y of the Q8_0 GEMMs is computed on the matrix core
(an f16 MFMA), the block dots multiply on the VALU, and the oracle in C: these
cases are where such paths could diverge (a flushed fp16 subnormal, an
Inf * 0, the sign of a zero)."""
import numpy as np
import pytest
import torch

import synth
from gpu_util import assert_f32_parity_nan, empty_dev, from_dev, q4_tiles_gemm, to_dev

pytestmark = pytest.mark.gpu

# fp16 bit patterns
FINITE = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00]
NONFINITE = [0x7C00, 0xFC00, 0x7E00]


def _set_scale(mat, r, b, blk, bits):
    mat[r, blk * b] = bits & 0xFF
    mat[r, blk * b + 1] = bits >> 8


def plant(mat, nb, blk, seed, nonfinite_every=0):
    """Finite special scales at about a fifth of the blocks, every block of
    row 1 subnormal, and (when nonfinite_every > 0) one +-Inf/NaN scale in
    every nonfinite_every-th row."""
    rows = mat.shape[0]
    for r in range(rows):
        for b in range(nb):
            if (3 * r + b + seed) % 5 == 0:
                _set_scale(mat, r, b, blk, FINITE[(r + b + seed) % len(FINITE)])
    if rows > 1:
        for b in range(nb):
            _set_scale(mat, 1, b, blk, 0x0001 + (b * 0x3F) % 0x3FF)
    if nonfinite_every:
        for r in range(nonfinite_every - 1, rows, nonfinite_every):
            _set_scale(mat, r, (r + seed) % nb, blk, NONFINITE[(r // nonfinite_every) % 3])
    return mat


def q8(rows, nb, seed, scale=1.0, nonfinite_every=0):
    return plant(synth.q8_0_matrix(rows, nb * 32, seed, scale), nb, 34, seed, nonfinite_every)


def q4(rows, nb, seed, nonfinite_every=0):
    return plant(synth.q4_0_matrix(rows, nb * 32, seed, 0.02), nb, 18, seed, nonfinite_every)


# ------------------------------------------------------------------ GEMMs ---

@pytest.mark.parametrize("nr,nc,nb,pad", [
    (300, 130, 9, 0),    # wide 256 x 128 tiles: 2 full chunks + 1 block
    (256, 128, 8, 0),    # few tiles, 16-byte rows: packed in LDS, one 32 x 32 tile a wave
    (600, 200, 24, 0),   # the same over three 8-block chunks
    (600, 200, 48, 0),   # the same over six chunks
    (100, 70, 9, 16),    # 128 x 128 tiles (fewer than 256 weight rows)
    (33, 20, 5, 2),      # rows 2-byte aligned only: the raw-block kernel
    (64, 1, 8, 0),       # decode shape: register-direct block dots
    (1, 40, 8, 0),       # one weight row
    (200, 6, 8, 0),      # a few tokens: the multi-column GEMV (8 columns, six present)
    (64, 3, 10, 0),      # a few tokens: 4 columns, three present
])
def test_q8_0_gemm_special_scales(hip, oracle, dev, nr, nc, nb, pad):
    n = nb * 32
    w = np.pad(q8(nr, nb, 11, 0.02, nonfinite_every=16), ((0, 0), (0, pad)))
    a = np.pad(q8(nc, nb, 12, 1.0, nonfinite_every=23), ((0, 0), (0, pad)))
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q8_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], nc)
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    assert_f32_parity_nan(from_dev(s), want, what=f"q8 gemm {nr}x{nc}x{n}")


def test_q8_0_gemm_ws_special_scales(hip, oracle, dev):
    """The workspace entry at a shape of few tiles (its one-tile-a-wave kernel)."""
    nr, nc, nb = 300, 130, 9
    n = nb * 32
    w = q8(nr, nb, 31, 0.02, nonfinite_every=16)
    a = q8(nc, nb, 32, 1.0, nonfinite_every=23)
    wsb = hip.q8_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q8_0_q8_0_gemm_ws(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1],
                          nc, ws, wsb)
    want = oracle.gemm_q8_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    assert_f32_parity_nan(from_dev(s), want, what="q8 gemm_ws")


@pytest.mark.parametrize("nr,nc,nb", [(300, 130, 9), (100, 70, 9), (64, 1, 8), (1, 40, 8),
                                      (600, 200, 24),  # packed in LDS, a 32 x 32 tile a wave
                                      (600, 200, 48),  # the same, six chunks
                                      (200, 4, 8), (64, 3, 10)])  # the last two: multi-column GEMVs
def test_q4_0_gemm_special_scales(hip, oracle, dev, nr, nc, nb):
    n = nb * 32
    w = q4(nr, nb, 13, nonfinite_every=16)
    a = q8(nc, nb, 14, 1.0, nonfinite_every=23)
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q4_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], nc)
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    assert_f32_parity_nan(from_dev(s), want, what=f"q4 gemm {nr}x{nc}x{n}")


def test_q4_0_gemm_tiles_special_scales(hip, oracle, dev):
    """The tiled Q4_0 GEMM over the GEMM-tile layout at a shape of few tiles (one 32 x 32 tile
    a wave)."""
    nr, nc, nb = 300, 130, 9
    n = nb * 32
    w = q4(nr, nb, 33, nonfinite_every=16)
    a = q8(nc, nb, 34, 1.0, nonfinite_every=23)
    s = q4_tiles_gemm(hip, dev, n, w, a, nr, nc, nc, empty_dev(nr * nc, torch.float32, dev))
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    assert_f32_parity_nan(from_dev(s), want, what="q4 gemm tiles")


def test_q4_0_gemm_ws_special_scales(hip, oracle, dev):
    """The workspace entry: both operands packed in one launch (16-byte aligned
    rows, 8-block spans), then the tiled Q4_0 GEMM (one 32 x 32 tile a wave at
    this shape)."""
    nr, nc, nb = 320, 96, 16
    n = nb * 32
    w = q4(nr, nb, 35, nonfinite_every=16)
    a = q8(nc, nb, 36, 1.0, nonfinite_every=23)
    wsb = hip.q4_0_q8_0_gemm_workspace_bytes(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q4_0_q8_0_gemm_ws(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1],
                          nc, ws, wsb)
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    assert_f32_parity_nan(from_dev(s), want, what="q4 gemm_ws")


def test_q4_0_gemm_tiles_nonfinite_dx_mid_k(hip, oracle, dev):
    """The pre-packed Q4_0 GEMM at a shape of few tiles (one 16 x 16 tile a wave,
    folding every block in the exact three-instruction form) with non-finite d_x
    across K: +-Inf planted in the first blocks, in the middle of K and near its
    end, NaN, and an infinite d_x over a zero block sum (0 * Inf = NaN).  The
    256-row tiles' fast-to-exact switch is covered by
    test_gemm_ws_tiles_special_scales."""
    nr, nc, nb = 512, 256, 40  # 6 full chunks + 4 tail blocks
    n = nb * 32
    w = q4(nr, nb, 41)
    a = q8(nc, nb, 42, 1.0, nonfinite_every=37)
    for r, b, bits in ((70, 20, 0x7C00), (130, 0, 0xFC00), (200, 37, 0x7E00),
                       (330, 35, 0x7C00), (400, 10, 0xFC00), (450, 29, 0x7C00)):
        _set_scale(w, r, b, 18, bits)
    w[400, 10 * 18 + 2:10 * 18 + 18] = 0x88  # every quant q - 8 = 0: block sums 0
    s = q4_tiles_gemm(hip, dev, n, w, a, nr, nc, nc, empty_dev(nr * nc, torch.float32, dev))
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    got = from_dev(s)
    assert_f32_parity_nan(got, want, what="q4 tiles, non-finite d_x")
    g = got.reshape(nr, nc)
    assert np.isinf(g[70]).any() and np.isnan(g[400]).all()  # the planted cases took effect


@pytest.mark.parametrize("nb", [40, 42])
def test_q4_0_gemm_nonfinite_dx_mid_k(hip, oracle, dev, nb):
    """The plain Q4_0 entry with non-finite d_x planted across K (nb = 40: the
    plain-row few-tile kernel, one 32 x 32 tile a wave; nb = 42: the 256 x 128
    wide kernel): +-Inf in the first chunk of one wave's rows, in the middle of K,
    in the last block and (nb = 42) in the partial tail, NaN, and an infinite
    d_x over a zero block sum (0 * Inf = NaN)."""
    nr, nc = 512, 256
    n = nb * 32
    w = q4(nr, nb, 43)
    a = q8(nc, nb, 44, 1.0, nonfinite_every=37)
    for r, b, bits in ((70, 20, 0x7C00), (130, 0, 0xFC00), (200, 37, 0x7E00),
                       (330, nb - 1, 0x7C00), (400, 10, 0xFC00), (450, 29, 0x7C00)):
        _set_scale(w, r, b, 18, bits)
    w[400, 10 * 18 + 2:10 * 18 + 18] = 0x88  # every quant q - 8 = 0: block sums 0
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.q4_0_q8_0_gemm(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr, nc, w.shape[1], nc)
    want = oracle.gemm_q4_0(n, w, a, a.shape[1], nr, nc, w.shape[1], nc, 8)
    got = from_dev(s)
    assert_f32_parity_nan(got, want, what=f"q4 gemm, non-finite d_x, nb {nb}")
    g = got.reshape(nr, nc)
    assert np.isinf(g[70]).any() and np.isnan(g[400]).all()  # the planted cases took effect


@pytest.mark.parametrize("nr,nc,kernel", [(4096, 4096, "256x256"), (4196, 4166, "256x128"),
                                          (4096, 130, "32x32"), (4096, 40, "16x16")])
@pytest.mark.parametrize("quant,nonfinite_every", [("q8_0", 16), ("q4_0", 16), ("q4_0", 0)])
def test_gemm_ws_tiles_special_scales(hip, oracle, dev, quant, nonfinite_every, nr, nc, kernel):
    """Each work-group tile of the tiled GEMMs, through the workspace entries (256 x 256: 4096 x
    4096 outputs; 256 x 128: 4196 x 4166, three rounds of it against two of the larger tile; one
    32 x 32 tile a wave: 4096 x 130; one 16 x 16 tile a wave: 4096 x 40): special scales in both
    operands, non-finite d_x in every
    16th weight row (every Q4_0 wave of the 256-row tiles folds exactly from chunk 0) or, with
    none there, +-Inf and NaN planted at chunk 0, in the middle of K, in the last full chunk and
    in the 1-block tail (chunks of 4 and of 6 blocks), and an infinite d_x over a zero block
    sum.  Sampled rows, the planted ones included, against the oracle."""
    print(f"{quant} {kernel} tiles {nr} x {nc}, non-finite every {nonfinite_every}", flush=True)
    nb = 13  # 3 chunks of 4 blocks + 1; 2 chunks of 6 + 1
    n = nb * 32
    if quant == "q8_0":
        w, blk = q8(nr, nb, 51, 0.02, nonfinite_every=nonfinite_every), 34
    else:
        w, blk = q4(nr, nb, 52, nonfinite_every=nonfinite_every), 18
    a = q8(nc, nb, 53, 1.0, nonfinite_every=37)
    planted = ((70, 2, 0x7C00), (130, 0, 0xFC00), (200, 12, 0x7E00), (330, 11, 0x7C00),
               (400, 5, 0xFC00), (450, 9, 0x7C00))
    if not nonfinite_every:
        for r, b, bits in planted:
            _set_scale(w, r, b, blk, bits)
        q0 = 0x88 if quant == "q4_0" else 0x00  # every quant 0: block sums 0
        w[400, 5 * blk + 2:6 * blk] = q0
    wsb = getattr(hip, f"{quant}_q8_0_gemm_workspace_bytes")(n, nr, nc)
    ws = empty_dev(wsb, torch.uint8, dev)
    s = empty_dev(nr * nc, torch.float32, dev)
    getattr(hip, f"{quant}_q8_0_gemm_ws")(n, s, to_dev(w, dev), to_dev(a, dev), a.shape[1], nr,
                                          nc, w.shape[1], nc, ws, wsb)
    got = from_dev(s).reshape(nr, nc)
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([[0, 1, 15, nr - 1], [r for r, _, _ in planted],
                                     rng.choice(nr, 20, replace=False)]))
    sub = np.ascontiguousarray(w[rows])
    ref = oracle.gemm_q8_0 if quant == "q8_0" else oracle.gemm_q4_0
    want = ref(n, sub, a, a.shape[1], len(rows), nc, w.shape[1], nc, 8)
    assert_f32_parity_nan(got[rows].reshape(-1), want, what=f"{quant} {kernel} tiles")
    if not nonfinite_every:
        assert np.isinf(got[70]).any() and np.isnan(got[400]).all()  # the planted cases


def _x16_source(w, nb, k):
    nc = w.shape[0]
    return np.ascontiguousarray(np.concatenate(
        [w[16 * x:16 * x + 16, k * b:k * b + k] for x in range(nc // 16) for b in range(nb)]
    ).reshape(-1))


def test_repack_gemm_special_scales(hip, oracle, dev):
    nr, nc, nb = 136, 272, 9   # tokens, weight rows
    n = nb * 32
    w = q4(nc, nb, 15, nonfinite_every=16)
    a = q8(nr, nb, 16, 1.0, nonfinite_every=23)
    packed = oracle.pack_q4_0x16(_x16_source(w, nb, 18), nc // 16 * nb)
    ax4 = oracle.pack_q8_0x4(a, nr, nb, a.shape[1])
    s = empty_dev(nr * nc, torch.float32, dev)
    hip.repack_gemm_q4_0_q8_0(n, s, to_dev(packed, dev), to_dev(ax4, dev), nr, nc, nc)
    want = oracle.repack_gemm_q4_0(n, packed, ax4, nr, nc, nc)
    assert_f32_parity_nan(from_dev(s), want, what="repack gemm")


# -------------------------------------------------------- GEMVs, block dots ---

# (nr, nb = 64 / 32): the lane-group kernels for rows of 2048 and 1024 quants,
# also with padded rows
@pytest.mark.parametrize("nr,nb,pad", [(512, 128, 0), (33, 7, 2), (520, 64, 0), (8200, 64, 16),
                                       (520, 32, 0), (4100, 32, 4)])
def test_gemv_q4_0_special_scales(hip, oracle, dev, nr, nb, pad):
    n = nb * 32
    w = np.pad(q4(nr, nb, 17, nonfinite_every=16), ((0, 0), (0, pad)))
    x = q8(1, nb, 18, 1.0).reshape(-1)
    s = empty_dev(nr, torch.float32, dev)
    hip.gemv_q4_0_q8_0(n, s, to_dev(w, dev), w.shape[1], to_dev(x, dev), nr)
    want = oracle.gemm_q4_0(n, w, x, 0, nr, 1, w.shape[1], 1, 8)[:nr]
    assert_f32_parity_nan(from_dev(s), want, what="gemv")
    if nb % 2 == 0 and pad == 0:  # the split layout: same blocks, same bits
        soa = empty_dev(nr * nb * 18, torch.uint8, dev)
        hip.pack_q4_0_to_soa(nr, nb, to_dev(w, dev), w.shape[1], soa)
        hip.gemv_q4_0_soa_q8_0(n, s, soa, to_dev(x, dev), nr)
        assert_f32_parity_nan(from_dev(s), want, what="soa gemv")


def test_gemv_q4_0_nonfinite_activation_scale(hip, oracle, dev):
    nr, nb = 256, 64
    n = nb * 32
    w = q4(nr, nb, 19)
    for bits in NONFINITE + [0x0001, 0x8000]:
        x = synth.q8_0_matrix(1, n, 20, 1.0)
        _set_scale(x, 0, 5, 34, bits)
        x = x.reshape(-1)
        s = empty_dev(nr, torch.float32, dev)
        hip.gemv_q4_0_q8_0(n, s, to_dev(w, dev), w.shape[1], to_dev(x, dev), nr)
        want = oracle.gemm_q4_0(n, w, x, 0, nr, 1, w.shape[1], 1, 8)[:nr]
        assert_f32_parity_nan(from_dev(s), want, what=f"gemv activation d={bits:#06x}")


# nb = 64 / 32: the block dots that run two or four row pairs per wave
@pytest.mark.parametrize("rows,nb,pad", [(64, 128, 0), (19, 9, 2), (24, 260, 0), (70, 64, 0),
                                         (70, 64, 4), (132, 32, 0), (132, 32, 16)])
def test_block_dots_special_scales(hip, oracle, dev, rows, nb, pad):
    n = nb * 32
    x8 = np.pad(q8(rows, nb, 21, 1.0, nonfinite_every=8), ((0, 0), (0, pad)))
    y8 = np.pad(q8(rows, nb, 22, 1.0, nonfinite_every=11), ((0, 0), (0, pad)))
    x4 = np.pad(q4(rows, nb, 23, nonfinite_every=8), ((0, 0), (0, pad)))
    s = empty_dev(rows, torch.float32, dev)
    hip.q8_0_q8_0_block_dot_rows(n, s, to_dev(x8, dev), x8.shape[1], to_dev(y8, dev),
                                 y8.shape[1], rows)
    want = oracle.vec_dot_q8_0_rows(n, x8, x8.shape[1], y8, y8.shape[1], rows, 8)
    assert_f32_parity_nan(from_dev(s), want, what="q8 block dot")
    hip.q4_0_q8_0_block_dot_rows(n, s, to_dev(x4, dev), x4.shape[1], to_dev(y8, dev),
                                 y8.shape[1], rows)
    want = oracle.vec_dot_q4_0_rows(n, x4, x4.shape[1], y8, y8.shape[1], rows, 8)
    assert_f32_parity_nan(from_dev(s), want, what="q4 block dot")
    # one activation row shared by every weight row (the Q8_0 decode GEMV)
    hip.q8_0_q8_0_gemm(n, s, to_dev(x8, dev), to_dev(y8[0].copy(), dev), 0, rows, 1,
                       x8.shape[1], 1)
    want = oracle.gemm_q8_0(n, x8, y8[0].copy(), 0, rows, 1, x8.shape[1], 1, 8)
    assert_f32_parity_nan(from_dev(s), want, what="q8 decode gemv")


@pytest.mark.parametrize("quant", ["q4_0", "q8_0"])
def test_repack_gemv_special_scales(hip, oracle, dev, quant):
    nc, nb = 64, 9
    n = nb * 32
    w = q4(nc, nb, 24, nonfinite_every=16) if quant == "q4_0" else \
        q8(nc, nb, 24, 0.02, nonfinite_every=16)
    x = q8(1, nb, 25, 1.0).reshape(-1)
    if quant == "q4_0":
        packed = oracle.pack_q4_0x16(_x16_source(w, nb, 18), nc // 16 * nb)
        want = oracle.repack_gemv_q4_0(n, packed, x, nc)
        run = hip.repack_gemv_q4_0_q8_0
    else:
        packed = oracle.pack_q8_0x16(_x16_source(w, nb, 34), nc // 16 * nb)
        want = oracle.repack_gemv_q8_0(n, packed, x, nc)
        run = hip.repack_gemv_q8_0_q8_0
    s = empty_dev(nc, torch.float32, dev)
    run(n, s, to_dev(packed, dev), to_dev(x, dev), nc)
    assert_f32_parity_nan(from_dev(s), want, what=f"repack gemv {quant}")


# ---------------------------------------------------------------- quantize ---

def special_blocks():
    """f32 blocks of 32 with the cases the RVV quantizer's conversions decide."""
    rng = np.random.default_rng(5)
    blocks = []
    base = lambda: rng.standard_normal(32).astype(np.float32)
    b = base(); b[3] = np.nan; blocks.append(b)                          # quiet NaN
    b = base(); b[7] = np.frombuffer(np.uint32(0x7FA00000).tobytes(), np.float32)[0]
    blocks.append(b)                                                     # signaling NaN
    b = base(); b[0] = np.inf; blocks.append(b)                          # +Inf: d = Inf, id = 0
    b = base(); b[31] = -np.inf; blocks.append(b)                        # -Inf
    b = base(); b[:] = np.inf; blocks.append(b)                          # all +Inf
    b = base(); b[:] = np.nan; blocks.append(b)                          # all NaN: amax = 0
    b = (base() * 1e-40).astype(np.float32); blocks.append(b)            # subnormal amax: 1/d = Inf
    b = np.zeros(32, np.float32); b[4] = 1e-45; blocks.append(b)         # smallest subnormal
    b = base(); b[2] = 1e7; blocks.append(b)                             # d = 78740: fp16 d = Inf
    b = base(); b[9] = 65504.0 * 127.0; blocks.append(b)                 # d = 65504 exactly
    b = base(); b[9] = 65520.0 * 127.0; blocks.append(b)                 # d rounds to fp16 Inf
    b = np.full(32, -0.0, np.float32); blocks.append(b)                  # all -0
    b = base(); b[0] = np.finfo(np.float32).max; blocks.append(b)        # amax = FLT_MAX
    b = np.arange(32, dtype=np.float32) - 15.5; blocks.append(b)         # RNE ties at .5
    return np.concatenate(blocks)


def test_quantize_q8_0_special_inputs(hip, oracle, dev):
    x = special_blocks()
    nb = x.size // 32
    with np.errstate(all="ignore"):
        want = oracle.quantize_q8_0(x)
    vy = empty_dev(nb * 34, torch.uint8, dev)
    hip.quantize_row_q8_0(x.size, to_dev(x, dev), vy)
    got = from_dev(vy)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (f"{bad.size} bytes differ; first in block {bad[0] // 34} at byte "
                           f"{bad[0] % 34}: got {got[bad[0]]:#04x} want {want[bad[0]]:#04x}")
    # the unaligned (4-byte) load path sees the same blocks
    buf = empty_dev(x.size + 1, torch.float32, dev)
    buf[1:] = to_dev(x, dev)
    hip.quantize_row_q8_0(x.size, buf[1:], vy)
    assert np.array_equal(from_dev(vy), want)
