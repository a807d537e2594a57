#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

The reference ships no numeric vectors for its quantized kernels (its lit
fixtures pin emitted structure and fold order only), so these fixtures are
generated here, once, by the oracle (oracle/libtcrv_oracle.so) on seeded
inputs from tianchen-rv_amd/synth.py, and committed.  They are regression
anchors: tests/test_golden.py checks that the oracle still reproduces them and
re-derives their integer sums by brute force; the GPU tests check every kernel
against them byte for byte.

    python3 tests/golden/make_golden.py            (rewrites tests/golden/*.npz)
    python3 tests/golden/make_golden.py NAME ...   (rewrites only those fixtures)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "tianchen-rv_amd"))

import oracle_binding  # noqa: E402
import synth  # noqa: E402


def main():
    ora = oracle_binding.load()
    out = {}

    # a1: add f32 (harness-shaped n = 1031) and i32 (the reference's harness vector)
    n = 1031
    a, b = synth.uniform_f32(11, n), synth.uniform_f32(12, n)
    i = np.arange(n, dtype=np.int64)
    ai, bi = (3 * i - 17).astype(np.int32), (41 - 2 * i).astype(np.int32)
    out["add"] = dict(a=a, b=b, out=ora.add_f32(a, b), ai=ai, bi=bi, outi=ora.add_i32(ai, bi))

    # a3 / a10: quantize 8 blocks (zero block, RNE ties, tiny values) and dequantize
    x = synth.normal_f32(13, 8 * 32, 0.0, 1.0)
    x[:32] = 0.0
    x[32:64] = np.arange(32) - 15.5
    x[64:96] = 1e-30
    q = ora.quantize_q8_0(x)
    out["quant"] = dict(x=x, q=q, deq=ora.dequantize_row_q8_0(q, x.size))

    # a3b: Q4_0 dequantize of 24 blocks: every weight byte value (blocks 0-15),
    # special fp16 scales (+-0, subnormals, 65504, inf, NaN) on blocks 0-11, and
    # 8 blocks quantized from seeded N(0, 0.02) values; n has a trailing partial
    # block of 17 elements, which is dropped
    w = synth.quantize_q4_0(synth.normal_f32(26, 24 * 32, 0.0, 0.02)).reshape(24, 18)
    w[:16, 2:] = np.arange(256, dtype=np.uint8).reshape(16, 16)
    special = np.array([0x0000, 0x8000, 0x0001, 0x83ff, 0x7bff, 0xfbff, 0x7c00, 0xfc00,
                        0x7e00, 0x3c00, 0xbc00, 0x0400], dtype=np.uint16)
    w[:12, 0:2] = special.view(np.uint8).reshape(12, 2)
    w = w.reshape(-1)
    n = 24 * 32 + 17
    out["dequant_q4"] = dict(n=np.int64(n), q=w, deq=ora.dequantize_row_q4_0(w, n))

    # a5: 4 Q8_0 pairs at n = 128, with a -128 x -128 block
    n = 128
    vx, vy = synth.q8_0_matrix(4, n, 14, 1.0), synth.q8_0_matrix(4, n, 15, 1.0)
    vx[0, 2:34] = 0x80
    vy[0, 2:34] = 0x80
    sumi = np.stack([ora.block_sums_q8_0(n, vx[r].copy(), vy[r].copy()) for r in range(4)])
    out["dot_q8"] = dict(n=np.int64(n), vx=vx, vy=vy, sumi=sumi,
                         s=ora.vec_dot_q8_0_rows(n, vx, vx.shape[1], vy, vy.shape[1], 4))

    # a4 / a6: 8 Q4_0 rows at n = 256, every weight byte value present
    n = 256
    wq, yq = synth.q4_0_matrix(8, n, 16, 0.02), synth.q8_0_matrix(8, n, 17, 1.0)
    qs = wq.reshape(8, n // 32, 18)[:, :, 2:]
    qs[...] = np.arange(qs.size, dtype=np.int64).reshape(qs.shape) % 256
    sumi = np.stack([ora.block_sums_q4_0(n, wq[r].copy(), yq[r].copy()) for r in range(8)])
    out["dot_q4"] = dict(n=np.int64(n), vx=wq, vy=yq, sumi=sumi,
                         s=ora.vec_dot_q4_0_rows(n, wq, wq.shape[1], yq, yq.shape[1], 8))

    # a9: Q8_0 GEMM 64 weight rows x 64 tokens x 128
    n = 128
    w8, a8 = synth.q8_0_matrix(64, n, 18, 0.02), synth.q8_0_matrix(64, n, 19, 1.0)
    out["gemm_q8"] = dict(n=np.int64(n), w=w8, a=a8,
                          s=ora.gemm_q8_0(n, w8, a8, a8.shape[1], 64, 64, w8.shape[1], 64))

    # a7: Q4_0 GEMM 32 rows x 48 tokens x 96, and the decode GEMV (one token)
    n = 96
    w4, a4 = synth.q4_0_matrix(32, n, 20, 0.02), synth.q8_0_matrix(48, n, 21, 1.0)
    out["gemm_q4"] = dict(n=np.int64(n), w=w4, a=a4,
                          s=ora.gemm_q4_0(n, w4, a4, a4.shape[1], 32, 48, w4.shape[1], 48),
                          gemv=ora.gemm_q4_0(n, w4, a4[0].copy(), 0, 32, 1, w4.shape[1], 1))

    # a8: x16 pack of 2 groups (32 rows) x 3 blocks and both repacked GEMVs
    n = 96
    nb = n // 32
    wr = synth.q4_0_matrix(32, n, 22, 0.02)
    src4 = np.ascontiguousarray(wr.reshape(2, 16, nb, 18).transpose(0, 2, 1, 3).reshape(-1))
    p4 = ora.pack_q4_0x16(src4, 2 * nb)
    w8r = synth.q8_0_matrix(32, n, 23, 0.02)
    src8 = np.ascontiguousarray(w8r.reshape(2, 16, nb, 34).transpose(0, 2, 1, 3).reshape(-1))
    p8 = ora.pack_q8_0x16(src8, 2 * nb)
    act = synth.q8_0_matrix(1, n, 24, 1.0).reshape(-1)
    out["repack"] = dict(n=np.int64(n), src4=src4, p4=p4, src8=src8, p8=p8, act=act,
                         s4=ora.repack_gemv_q4_0(n, p4, act, 32),
                         s8=ora.repack_gemv_q8_0(n, p8, act, 32))

    # a8: repack GEMM of those x16 Q4_0 weights against 8 activation rows in the
    # 4-row interleave (block_q8_0x4)
    a8r = synth.q8_0_matrix(8, n, 25, 1.0)
    ax4 = ora.pack_q8_0x4(a8r, 8, nb, a8r.shape[1])
    out["repack_gemm"] = dict(n=np.int64(n), p4=p4, act=a8r, ax4=ax4,
                              s=ora.repack_gemm_q4_0(n, p4, ax4, 8, 32, 32))

    only = set(sys.argv[1:])
    for name, arrays in out.items():
        if only and name not in only:
            continue
        path = os.path.join(HERE, f"{name}.npz")
        np.savez(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
