"""Seeded synthetic inputs and host-side ggml quantizers (numpy).

The generator is splitmix64 -> uniform (0,1) -> Box-Muller, written here so
the same seed gives the same bits on any host:

    z   = splitmix64 output i of the stream started at `seed`
    u   = ((z >> 11) + 0.5) * 2**-53                 (float64, never 0 or 1)
    N   : r = sqrt(-2 ln u[2k]), t = 2 pi u[2k+1];  x[2k] = r cos t, x[2k+1] = r sin t
    out = float32(mean + std * x)      or   float32(lo + (hi - lo) * u) for U(lo, hi)

Host quantizers (they produce the input bytes of the benchmark configs):
  - quantize_q8_0: the reference's tcrv_rvv.quantize_row_q8_0 semantics
    (include/TianChenRV/Dialect/RVV/IR/RVVOps.td:8368-8390): d = amax/127,
    id = d ? 1/d : 0, d stored as fp16 (RNE), q = int8(int16 sat rne(x*id)).
  - quantize_q4_0: ggml quantize_row_q4_0_ref: d = max/-8 (max = the signed
    value of largest magnitude, first occurrence), id = d ? 1/d : 0,
    q = min(15, int8(x*id + 8.5)), qs[j] = q[j] | q[j+16] << 4.
All arithmetic is float32 elementwise (numpy does not contract), so the bytes
equal those of a scalar C implementation compiled without contraction.
"""
from __future__ import annotations

import numpy as np

QK = 32
Q8_0_BLOCK_BYTES = 34
Q4_0_BLOCK_BYTES = 18

# Seeds of the five benchmark configurations.
SEEDS = {
    "add_a": 1001, "add_b": 1002,
    "dequant_w": 1003,
    "dot_x": 1004, "dot_y": 1005,
    "gemv_w": 1006, "gemv_x": 1007,
    "gemm_a": 1008, "gemm_b": 1009,
}

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int) -> np.ndarray:
    """The first `count` outputs of splitmix64 started at `seed` (uint64)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, count + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, count: int) -> np.ndarray:
    z = splitmix64(seed, count)
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)


def uniform_f32(seed: int, count: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    u = uniform01(seed, count)
    return (lo + (hi - lo) * u).astype(np.float32)


def normal_f32(seed: int, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    pairs = (count + 1) // 2
    u = uniform01(seed, 2 * pairs)
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    t = 2.0 * np.pi * u[1::2]
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    return (mean + std * z[:count]).astype(np.float32)


def _safe_recip(d: np.ndarray) -> np.ndarray:
    out = np.zeros_like(d)
    nz = d != 0
    out[nz] = np.float32(1.0) / d[nz]
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """float32[n] (n % 32 == 0) -> uint8[n/32 * 34] block_q8_0 bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size % QK:
        raise ValueError("quantize_q8_0 needs a multiple of 32 values")
    xb = x.reshape(-1, QK)
    nb = xb.shape[0]
    amax = np.max(np.abs(xb), axis=1).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = _safe_recip(d)
    v = (xb * inv[:, None]).astype(np.float32)
    r = np.rint(v)
    r = np.where(np.isnan(v), 32767.0, np.clip(r, -32768.0, 32767.0))
    q = (r.astype(np.int32) & 0xFF).astype(np.uint8)
    out = np.empty((nb, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q
    return out.reshape(-1)


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    """float32[n] (n % 32 == 0) -> uint8[n/32 * 18] block_q4_0 bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size % QK:
        raise ValueError("quantize_q4_0 needs a multiple of 32 values")
    xb = x.reshape(-1, QK)
    nb = xb.shape[0]
    idx = np.argmax(np.abs(xb), axis=1)  # first occurrence of the largest |x|
    mx = xb[np.arange(nb), idx]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    inv = _safe_recip(d)
    x0 = (xb[:, :16] * inv[:, None]).astype(np.float32)
    x1 = (xb[:, 16:] * inv[:, None]).astype(np.float32)
    q0 = np.minimum(15, (x0 + np.float32(8.5)).astype(np.int8).astype(np.int32))
    q1 = np.minimum(15, (x1 + np.float32(8.5)).astype(np.int8).astype(np.int32))
    out = np.empty((nb, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = ((q0 & 0xF) | ((q1 & 0xF) << 4)).astype(np.uint8)
    return out.reshape(-1)


def q8_0_matrix(rows: int, n: int, seed: int, std: float) -> np.ndarray:
    """rows x n values ~ N(0, std) quantized to Q8_0, as rows x (n/32*34) bytes."""
    x = normal_f32(seed, rows * n, 0.0, std)
    return quantize_q8_0(x).reshape(rows, (n // QK) * Q8_0_BLOCK_BYTES)


def q4_0_matrix(rows: int, n: int, seed: int, std: float) -> np.ndarray:
    """rows x n values ~ N(0, std) quantized to Q4_0, as rows x (n/32*18) bytes."""
    x = normal_f32(seed, rows * n, 0.0, std)
    return quantize_q4_0(x).reshape(rows, (n // QK) * Q4_0_BLOCK_BYTES)
