/*
 * tcrv_oracle.h -- scalar CPU restatement of TianChen-RV's quantized hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP library
 * (libtcrv_hip.so).  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it; no product code path calls it, and the product
 * fails loudly when its HIP extension is missing instead of falling back here.
 *
 * Every function restates one emitter of the reference compiler (paths are
 * relative to the TianChen-RV tree) in plain C with the reference's exact
 * per-block fold order, written with explicit fmaf() so that the build's
 * -ffp-contract setting cannot change a rounding.
 *
 * Block formats (ggml, pinned by the reference verifiers):
 *   block_q8_0    34 B : fp16 d @0, int8  qs[32] @2
 *   block_q4_0    18 B : fp16 d @0, uint8 qs[16] @2; element j = (qs[j]&15)-8,
 *                        element j+16 = (qs[j]>>4)-8
 *   block_q4_0x16 288 B: fp16 d[16] @0, uint8 qs[256] @32 (interleaved, ^0x88)
 *   (lib/Dialect/RVV/IR/RVVDialectWideningOps.cpp:3358-3372;
 *    include/TianChenRV/Dialect/RVV/IR/RVVOps.td:3893-3897, :4569-4577)
 */
#ifndef TCRV_ORACLE_H
#define TCRV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TCRV_QK 32
#define TCRV_Q8_0_BLOCK_BYTES 34
#define TCRV_Q4_0_BLOCK_BYTES 18
#define TCRV_Q4_0X16_BLOCK_BYTES 288

/* IEEE binary16 <-> binary32 (the reference reads d as (float)*(const _Float16*),
 * RVVToEmitCBlockQuantLinear.cpp:117,140, and stores it as (_Float16)d, RNE). */
float tcrv_oracle_fp16_to_f32(uint16_t h);
uint16_t tcrv_oracle_f32_to_fp16(float f);

/* a1: tcrv_rvv.binary{kind="add"}; emitBinary RVVToEmitC.cpp:1873-1911. */
void tcrv_oracle_add_f32(const float *lhs, const float *rhs, float *out, size_t n);
void tcrv_oracle_add_i32(const int32_t *lhs, const int32_t *rhs, int32_t *out, size_t n);

/* a1 over the reference's element grid: tcrv_rvv.binary {kind = add|sub|mul}
 * (emitBinary RVVToEmitC.cpp:1873-1911, vadd/vsub/vmul or vfadd/vfsub/vfmul by
 * binaryMnemonic :4976-4993).  kind 0 add, 1 sub, 2 mul; elem 0 i8, 1 u8,
 * 2 i16, 3 u16, 4 i32, 5 u32, 6 i64, 7 f32, 8 f64.  Integers wrap modulo
 * 2^width; floats are single IEEE operations.  Returns 0, or -1 for an unknown
 * kind/elem. */
int tcrv_oracle_binary(int kind, int elem, const void *lhs, const void *rhs, void *out,
                       size_t n);

/* a3: y[32b+j] = qs_b[j] * fp16->f32(d_b) (ggml dequantize_row_q8_0). */
void tcrv_oracle_dequantize_row_q8_0(size_t n, float *y, const uint8_t *vx);

/* a3b: y[32b+j] = (lo nibble of qs_b[j] - 8) * d_b, y[32b+16+j] = (hi nibble
 * of qs_b[j] - 8) * d_b for j < 16 (ggml dequantize_row_q4_0; the op's
 * offset-binary decode, RVVOps.td:3837-3842). */
void tcrv_oracle_dequantize_row_q4_0(size_t n, float *y, const uint8_t *vx);

/* a4: the packed-i4 offset-binary x i8 integer core for one Q4_0 block against
 * one Q8_0 block (RVVToEmitC.cpp:2524-2589). */
int32_t tcrv_oracle_q4_0_q8_0_block_sumi(const uint8_t *xb, const uint8_t *yb);
/* a4 as its standalone kernel: out[0] = acc[0] + sum over i < n of the
 * decoded weight byte w[i]'s low nibble x qlo[i] + high nibble x qhi[i]
 * (int32, wrapping). */
void tcrv_oracle_packed_i4_offset_binary_x_i8_product_reduce(const int8_t *w, const int8_t *qlo,
                                                             const int8_t *qhi,
                                                             const int32_t *acc, int32_t *out,
                                                             size_t n);
/* a5's integer core for one block pair. */
int32_t tcrv_oracle_q8_0_q8_0_block_sumi(const uint8_t *xb, const uint8_t *yb);

/* Per-block integer sums of a whole row pair (nb = n/32 values). */
void tcrv_oracle_block_sums_q8_0_q8_0(size_t n, int32_t *sumi, const uint8_t *vx,
                                      const uint8_t *vy);
void tcrv_oracle_block_sums_q4_0_q8_0(size_t n, int32_t *sumi, const uint8_t *vx,
                                      const uint8_t *vy);

/* a5: ggml_vec_dot_q8_0_q8_0; fold sumf = fma((float)sumi, d_x*d_y, sumf)
 * (RVVToEmitCBlockQuantLinear.cpp:7538-7575). */
void tcrv_oracle_vec_dot_q8_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                   const uint8_t *vy);
/* a6: ggml_vec_dot_q4_0_q8_0 with the ggml vec_dot ABI; fold
 * sumf = fma((float)sumi*d_x, d_y, sumf) (RVVToEmitCBlockQuantLinear.cpp:322-356). */
void tcrv_oracle_vec_dot_q4_0_q8_0(size_t n, float *s, size_t bs, const uint8_t *vx,
                                   size_t bx, const uint8_t *vy, size_t by, int32_t nrc);

/* Batched independent row pairs: s[r] = vec_dot(vx + r*bx, vy + r*by).
 * nthreads <= 1 runs serially; otherwise OpenMP over rows (each row's fold stays
 * serial, so the result is identical for every thread count). */
void tcrv_oracle_vec_dot_q8_0_q8_0_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                        const uint8_t *vy, size_t by, size_t nrows,
                                        int nthreads);
void tcrv_oracle_vec_dot_q4_0_q8_0_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                        const uint8_t *vy, size_t by, size_t nrows,
                                        int nthreads);

/* a7: tcrv_rvv.q4_0_q8_0_gemm, s[ir*bs + col] = a6(vx + ir*bx, vy + col*by)
 * (RVVToEmitCBlockQuantLinear.cpp:1691-2121). nc = 1 is the decode GEMV. */
void tcrv_oracle_gemm_q4_0_q8_0(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                                int nthreads);
/* a9: the Q8_0 x Q8_0 GEMM with the same loop nest and ABI, elements = a5. */
void tcrv_oracle_gemm_q8_0_q8_0(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                                int nthreads);

/* a10: tcrv_rvv.quantize_row_q8_0 (RVVOps.td:8345-8431). */
void tcrv_oracle_quantize_row_q8_0(size_t n, const float *x, uint8_t *vy);
/* a11: ggml quantize_row_q4_0_ref (d = max/-8, q = min(15, (int8)(x*id + 8.5f))). */
void tcrv_oracle_quantize_row_q4_0(size_t n, const float *x, uint8_t *vy);

/* a8: make_block_q4_0x16 (RVVOps.td:4551-4626) over nblocks output blocks, each
 * built from 16 consecutive source blocks. */
void tcrv_oracle_pack_q4_0_to_q4_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst);
/* a8: repack GEMV over x16 weights; fold fma((float)sumi, d_w*d_a, acc)
 * (RVVToEmitCBlockQuantLinear.cpp:3245-3290). s[x*16 + r] for x < nc/16. */
void tcrv_oracle_repack_gemv_q4_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                       const uint8_t *vy, size_t nc);

/* block_q8_0x16 (544 B: fp16 d[16] @0, int8 qs[512] @32, qs[i*16 + r] = quant i
 * of block r; no bias) -- the layout tcrv_rvv.repack_gemv_q8_0_q8_0 reads
 * (RVVOps.td:4846-4867; byte 32 + i*16 + r, RVVToEmitCBlockQuantLinear.cpp:
 * 4204-4215).  The reference has no pack op for it; this is its inverse of the
 * consumer's addressing. */
#define TCRV_Q8_0X16_BLOCK_BYTES 544
void tcrv_oracle_pack_q8_0_to_q8_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst);
/* The split (SoA) Q4_0 layout (a GPU layout; no reference counterpart): for
 * nrows rows of nb blocks read at stride bx, quants of row r block b at
 * dst + (r*nb + b)*16, its fp16 scale at dst + nrows*nb*16 + (r*nb + b)*2. */
void tcrv_oracle_pack_q4_0_to_soa(size_t nrows, size_t nb, const uint8_t *src, size_t bx,
                                  uint8_t *dst);
/* Its inverse (test helper): back to nrows contiguous plain rows. */
void tcrv_oracle_unpack_q4_0_soa(size_t nrows, size_t nb, const uint8_t *src, uint8_t *dst);
/* Inverse of both packs (test helper): x16 blocks back to 16 plain blocks each. */
void tcrv_oracle_unpack_q4_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst);
void tcrv_oracle_unpack_q8_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst);
/* repack GEMV over q8_0x16 weights (emitRepackGemvQ8_0Q8_0,
 * RVVToEmitCBlockQuantLinear.cpp:3930-4379): per row r of group x, sumi =
 * sum_i w[r][i]*a[i] (i16 products widened into i32), fold
 * acc = fma((float)sumi, d_w[r]*d_a, acc) in ascending block order. */
void tcrv_oracle_repack_gemv_q8_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                       const uint8_t *vy, size_t nc);

/* block_q8_0x4 (136 B): fp16 d[4] @0 (row c at byte 2c), int8 qs[128] @8 with
 * quant e of row c at qs[4e + c] -- the layout tcrv_rvv.repack_gemm_q4_0_q8_0
 * reads (RVVOps.td:4228-4338: stride 136, quants at +8, 4-row interleave; the
 * emitter reads al.qs[i*4 + c] and al.qs[64 + i*4 + c] for nibble step i and
 * al.d[c], RVVToEmitCBlockQuantLinear.cpp:2344-2600).  The reference has no
 * producer op for it (ggml repacks the activations); this pack is the inverse
 * of the consumer's addressing: groups of 4 plain Q8_0 rows (stride by), nb
 * blocks each, into nrows/4 groups of nb x4 blocks. */
#define TCRV_Q8_0X4_BLOCK_BYTES 136
void tcrv_oracle_pack_q8_0_to_q8_0x4(size_t nrows, size_t nb, const uint8_t *src, size_t by,
                                     uint8_t *dst);
/* The repack GEMM (emitRepackGemmQ4_0Q8_0, RVVToEmitCBlockQuantLinear.cpp:2122-2600):
 * activation row group y < nr/4 (x4 blocks at vy + y*nb*136), weight group
 * x < nc/16 (x16 blocks at vx + x*nb*288); for activation row c and weight row
 * r, per block: sumi = i16 lo/hi sums of the nibble decode against
 * qs[4i + c] and qs[64 + 4i + c] widened to i32, and the fold
 * acc = fma((float)sumi, d_w[r]*d_a[c], acc) (vfwmul exact, vfmacc fused) in
 * ascending block order; s[(y*4 + c)*bs + x*16 + r] = acc. */
void tcrv_oracle_repack_gemm_q4_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                       const uint8_t *vy, size_t nr, size_t nc, size_t bs);

#ifdef __cplusplus
}
#endif

#endif /* TCRV_ORACLE_H */
