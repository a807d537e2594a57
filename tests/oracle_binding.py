"""ctypes binding of oracle/libtcrv_oracle.so (test infrastructure only).

Thin numpy-facing wrappers around the scalar C restatement; used as the
checker by the tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB = os.path.join(ORACLE_DIR, "libtcrv_oracle.so")

_sz = ctypes.c_size_t
_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_int = ctypes.c_int

_SIGS = {
    "tcrv_oracle_fp16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
    "tcrv_oracle_f32_to_fp16": ([ctypes.c_float], ctypes.c_uint16),
    "tcrv_oracle_add_f32": ([_p, _p, _p, _sz], None),
    "tcrv_oracle_add_i32": ([_p, _p, _p, _sz], None),
    "tcrv_oracle_binary": ([_int, _int, _p, _p, _p, _sz], _int),
    "tcrv_oracle_dequantize_row_q8_0": ([_sz, _p, _p], None),
    "tcrv_oracle_dequantize_row_q4_0": ([_sz, _p, _p], None),
    "tcrv_oracle_q4_0_q8_0_block_sumi": ([_p, _p], _i32),
    "tcrv_oracle_q8_0_q8_0_block_sumi": ([_p, _p], _i32),
    "tcrv_oracle_packed_i4_offset_binary_x_i8_product_reduce": ([_p, _p, _p, _p, _p, _sz], None),
    "tcrv_oracle_block_sums_q8_0_q8_0": ([_sz, _p, _p, _p], None),
    "tcrv_oracle_block_sums_q4_0_q8_0": ([_sz, _p, _p, _p], None),
    "tcrv_oracle_vec_dot_q8_0_q8_0": ([_sz, _p, _p, _p], None),
    "tcrv_oracle_vec_dot_q4_0_q8_0": ([_sz, _p, _sz, _p, _sz, _p, _sz, _i32], None),
    "tcrv_oracle_vec_dot_q8_0_q8_0_rows": ([_sz, _p, _p, _sz, _p, _sz, _sz, _int], None),
    "tcrv_oracle_vec_dot_q4_0_q8_0_rows": ([_sz, _p, _p, _sz, _p, _sz, _sz, _int], None),
    "tcrv_oracle_gemm_q4_0_q8_0": ([_sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _int], None),
    "tcrv_oracle_gemm_q8_0_q8_0": ([_sz, _p, _p, _p, _sz, _sz, _sz, _sz, _sz, _int], None),
    "tcrv_oracle_quantize_row_q8_0": ([_sz, _p, _p], None),
    "tcrv_oracle_quantize_row_q4_0": ([_sz, _p, _p], None),
    "tcrv_oracle_pack_q4_0_to_q4_0x16": ([_sz, _p, _p], None),
    "tcrv_oracle_repack_gemv_q4_0_q8_0": ([_sz, _p, _p, _p, _sz], None),
    "tcrv_oracle_pack_q8_0_to_q8_0x16": ([_sz, _p, _p], None),
    "tcrv_oracle_unpack_q4_0x16": ([_sz, _p, _p], None),
    "tcrv_oracle_pack_q4_0_to_soa": ([_sz, _sz, _p, _sz, _p], None),
    "tcrv_oracle_unpack_q4_0_soa": ([_sz, _sz, _p, _p], None),
    "tcrv_oracle_unpack_q8_0x16": ([_sz, _p, _p], None),
    "tcrv_oracle_repack_gemv_q8_0_q8_0": ([_sz, _p, _p, _p, _sz], None),
    "tcrv_oracle_pack_q8_0_to_q8_0x4": ([_sz, _sz, _p, _sz, _p], None),
    "tcrv_oracle_repack_gemm_q4_0_q8_0": ([_sz, _p, _p, _p, _sz, _sz, _sz], None),
}


def _a(x: np.ndarray) -> int:
    assert x.flags["C_CONTIGUOUS"]
    return x.ctypes.data


class Oracle:
    def __init__(self, lib: ctypes.CDLL):
        self.lib = lib
        for name, (argtypes, restype) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype

    # -- scalars -----------------------------------------------------------
    def fp16_to_f32(self, h: int) -> float:
        return self.lib.tcrv_oracle_fp16_to_f32(h)

    def f32_to_fp16(self, f: float) -> int:
        return self.lib.tcrv_oracle_f32_to_fp16(f)

    # -- a1 ----------------------------------------------------------------
    def add_f32(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        out = np.empty_like(a)
        self.lib.tcrv_oracle_add_f32(_a(a), _a(b), _a(out), a.size)
        return out

    def add_i32(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        out = np.empty_like(a)
        self.lib.tcrv_oracle_add_i32(_a(a), _a(b), _a(out), a.size)
        return out

    def binary(self, kind: int, elem: int, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        out = np.empty_like(a)
        assert self.lib.tcrv_oracle_binary(kind, elem, _a(a), _a(b), _a(out), a.size) == 0
        return out

    # -- a3 ----------------------------------------------------------------
    def dequantize_row_q8_0(self, vx: np.ndarray, n: int) -> np.ndarray:
        y = np.zeros((n // 32) * 32, dtype=np.float32)
        self.lib.tcrv_oracle_dequantize_row_q8_0(n, _a(y), _a(vx))
        return y

    def dequantize_row_q4_0(self, vx: np.ndarray, n: int) -> np.ndarray:
        y = np.zeros((n // 32) * 32, dtype=np.float32)
        self.lib.tcrv_oracle_dequantize_row_q4_0(n, _a(y), _a(vx))
        return y

    # -- a4/a5/a6 ----------------------------------------------------------
    def q4_block_sumi(self, xb: np.ndarray, yb: np.ndarray) -> int:
        return self.lib.tcrv_oracle_q4_0_q8_0_block_sumi(_a(xb), _a(yb))

    def int_core_reduce(self, w: np.ndarray, qlo: np.ndarray, qhi: np.ndarray,
                        acc: int) -> int:
        a = np.array([acc], dtype=np.int32)
        out = np.zeros(1, dtype=np.int32)
        self.lib.tcrv_oracle_packed_i4_offset_binary_x_i8_product_reduce(
            _a(w), _a(qlo), _a(qhi), _a(a), _a(out), w.size)
        return int(out[0])

    def q8_block_sumi(self, xb: np.ndarray, yb: np.ndarray) -> int:
        return self.lib.tcrv_oracle_q8_0_q8_0_block_sumi(_a(xb), _a(yb))

    def block_sums_q8_0(self, n: int, vx: np.ndarray, vy: np.ndarray) -> np.ndarray:
        out = np.zeros(n // 32, dtype=np.int32)
        self.lib.tcrv_oracle_block_sums_q8_0_q8_0(n, _a(out), _a(vx), _a(vy))
        return out

    def block_sums_q4_0(self, n: int, vx: np.ndarray, vy: np.ndarray) -> np.ndarray:
        out = np.zeros(n // 32, dtype=np.int32)
        self.lib.tcrv_oracle_block_sums_q4_0_q8_0(n, _a(out), _a(vx), _a(vy))
        return out

    def vec_dot_q8_0(self, n: int, vx: np.ndarray, vy: np.ndarray) -> np.float32:
        s = np.zeros(1, dtype=np.float32)
        self.lib.tcrv_oracle_vec_dot_q8_0_q8_0(n, _a(s), _a(vx), _a(vy))
        return s[0]

    def vec_dot_q4_0(self, n: int, vx: np.ndarray, vy: np.ndarray) -> np.float32:
        s = np.zeros(1, dtype=np.float32)
        self.lib.tcrv_oracle_vec_dot_q4_0_q8_0(n, _a(s), 0, _a(vx), 0, _a(vy), 0, 1)
        return s[0]

    def vec_dot_q8_0_rows(self, n, vx, bx, vy, by, nrows, nthreads=1) -> np.ndarray:
        s = np.zeros(nrows, dtype=np.float32)
        self.lib.tcrv_oracle_vec_dot_q8_0_q8_0_rows(n, _a(s), _a(vx), bx, _a(vy), by, nrows,
                                                    nthreads)
        return s

    def vec_dot_q4_0_rows(self, n, vx, bx, vy, by, nrows, nthreads=1) -> np.ndarray:
        s = np.zeros(nrows, dtype=np.float32)
        self.lib.tcrv_oracle_vec_dot_q4_0_q8_0_rows(n, _a(s), _a(vx), bx, _a(vy), by, nrows,
                                                    nthreads)
        return s

    # -- a7/a9 -------------------------------------------------------------
    def gemm_q4_0(self, n, vx, vy, by, nr, nc, bx, bs, nthreads=1) -> np.ndarray:
        s = np.zeros(max(nr, 1) * max(bs, nc), dtype=np.float32)
        self.lib.tcrv_oracle_gemm_q4_0_q8_0(n, _a(s), _a(vx), _a(vy), by, nr, nc, bx, bs,
                                            nthreads)
        return s

    def gemm_q8_0(self, n, vx, vy, by, nr, nc, bx, bs, nthreads=1) -> np.ndarray:
        s = np.zeros(max(nr, 1) * max(bs, nc), dtype=np.float32)
        self.lib.tcrv_oracle_gemm_q8_0_q8_0(n, _a(s), _a(vx), _a(vy), by, nr, nc, bx, bs,
                                            nthreads)
        return s

    # -- a10/a11 -----------------------------------------------------------
    def quantize_q8_0(self, x: np.ndarray) -> np.ndarray:
        out = np.zeros((x.size // 32) * 34, dtype=np.uint8)
        self.lib.tcrv_oracle_quantize_row_q8_0(x.size, _a(x), _a(out))
        return out

    def quantize_q4_0(self, x: np.ndarray) -> np.ndarray:
        out = np.zeros((x.size // 32) * 18, dtype=np.uint8)
        self.lib.tcrv_oracle_quantize_row_q4_0(x.size, _a(x), _a(out))
        return out

    # -- a8 ----------------------------------------------------------------
    def pack_q4_0x16(self, src: np.ndarray, nblocks: int) -> np.ndarray:
        dst = np.zeros(nblocks * 288, dtype=np.uint8)
        self.lib.tcrv_oracle_pack_q4_0_to_q4_0x16(nblocks, _a(src), _a(dst))
        return dst

    def repack_gemv_q4_0(self, n: int, vx: np.ndarray, vy: np.ndarray, nc: int) -> np.ndarray:
        s = np.zeros(nc, dtype=np.float32)
        self.lib.tcrv_oracle_repack_gemv_q4_0_q8_0(n, _a(s), _a(vx), _a(vy), nc)
        return s

    def pack_q8_0x16(self, src: np.ndarray, nblocks: int) -> np.ndarray:
        dst = np.zeros(nblocks * 544, dtype=np.uint8)
        self.lib.tcrv_oracle_pack_q8_0_to_q8_0x16(nblocks, _a(src), _a(dst))
        return dst

    def pack_q4_0_soa(self, src: np.ndarray, nrows: int, nb: int, bx: int) -> np.ndarray:
        dst = np.zeros(nrows * nb * 18, dtype=np.uint8)
        self.lib.tcrv_oracle_pack_q4_0_to_soa(nrows, nb, _a(src), bx, _a(dst))
        return dst

    def unpack_q4_0_soa(self, src: np.ndarray, nrows: int, nb: int) -> np.ndarray:
        dst = np.zeros(nrows * nb * 18, dtype=np.uint8)
        self.lib.tcrv_oracle_unpack_q4_0_soa(nrows, nb, _a(src), _a(dst))
        return dst

    def unpack_q4_0x16(self, src: np.ndarray, nblocks: int) -> np.ndarray:
        dst = np.zeros(nblocks * 16 * 18, dtype=np.uint8)
        self.lib.tcrv_oracle_unpack_q4_0x16(nblocks, _a(src), _a(dst))
        return dst

    def unpack_q8_0x16(self, src: np.ndarray, nblocks: int) -> np.ndarray:
        dst = np.zeros(nblocks * 16 * 34, dtype=np.uint8)
        self.lib.tcrv_oracle_unpack_q8_0x16(nblocks, _a(src), _a(dst))
        return dst

    def repack_gemv_q8_0(self, n: int, vx: np.ndarray, vy: np.ndarray, nc: int) -> np.ndarray:
        s = np.zeros(nc, dtype=np.float32)
        self.lib.tcrv_oracle_repack_gemv_q8_0_q8_0(n, _a(s), _a(vx), _a(vy), nc)
        return s

    def pack_q8_0x4(self, src: np.ndarray, nrows: int, nb: int, by: int) -> np.ndarray:
        dst = np.zeros(nrows // 4 * nb * 136, dtype=np.uint8)
        self.lib.tcrv_oracle_pack_q8_0_to_q8_0x4(nrows, nb, _a(src), by, _a(dst))
        return dst

    def repack_gemm_q4_0(self, n: int, vx: np.ndarray, vy: np.ndarray, nr: int, nc: int,
                         bs: int) -> np.ndarray:
        s = np.zeros(nr * bs, dtype=np.float32)
        self.lib.tcrv_oracle_repack_gemm_q4_0_q8_0(n, _a(s), _a(vx), _a(vy), nr, nc, bs)
        return s


_oracle = None


def build() -> None:
    subprocess.run(["make", "-C", ORACLE_DIR, "-s"], check=True)


def load() -> Oracle:
    global _oracle
    if _oracle is None:
        if not os.path.exists(LIB):
            build()
        _oracle = Oracle(ctypes.CDLL(LIB))
    return _oracle
