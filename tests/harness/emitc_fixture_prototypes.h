// The exported functions of the reference's emission fixtures, written out
// by hand from each fixture's tcrv_rvv.runtime_abi_value declarations
// (c_type c_name, in declaration order), with the HIP boundary's changes: an
// int status instead of void, and a trailing `void *stream`.  The harness
// includes this after the generated header, so g++ rejects the build if a
// generated prototype differs from the fixture's (two extern "C"
// declarations of one name with different parameters).
#ifndef TCRV_EMITC_FIXTURE_PROTOTYPES_H_
#define TCRV_EMITC_FIXTURE_PROTOTYPES_H_

#include <stddef.h>
#include <stdint.h>

// test/Conversion/RVV/rvv-to-emitc-add-cpp-golden.mlir:15-18,33
extern "C" int tcrv_emitc_explicit_selected_body_add_kernel_explicit_selected_body_rvv_i32_add(
    const int32_t *lhs, const int32_t *rhs, int32_t *out, size_t n, void *stream);
// test/Conversion/RVV/rvv-to-emitc-q8-0-q8-0-block-dot.mlir:17-20
extern "C" int tcrv_emitc_ggml_vec_dot_q8_0_q8_0_kernel_ggml_vec_dot_q8_0_q8_0(
    size_t n, float *s, const uint8_t *vx, const uint8_t *vy, void *stream);
// test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-block-dot-m1.mlir:23-30
extern "C" int tcrv_emitc_ggml_vec_dot_q4_0_q8_0_kernel_ggml_vec_dot_q4_0_q8_0(
    size_t n, float *s, size_t bs, const uint8_t *vx, size_t bx, const uint8_t *vy, size_t by,
    int32_t nrc, void *stream);
// test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-gemm.mlir:23-31
extern "C" int tcrv_emitc_ggml_q4_0_q8_0_gemm_kernel_ggml_q4_0_q8_0_gemm(
    size_t n, float *s, const uint8_t *vx, const uint8_t *vy, size_t by, size_t nr, size_t nc,
    size_t bx, size_t bs, void *stream);
// test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-gemm-tile.mlir:25-29
extern "C" int tcrv_emitc_ggml_q4_0_q8_0_gemm_tile_kernel_ggml_q4_0_q8_0_gemm_tile(
    size_t n, float *s, const uint8_t *vx, const uint8_t *vy, size_t by, void *stream);
// test/Conversion/RVV/rvv-to-emitc-repack-gemv-q4-0-q8-0.mlir:26-30
extern "C" int tcrv_emitc_ggml_repack_gemv_q4_0_q8_0_kernel_ggml_repack_gemv_q4_0_q8_0(
    size_t n, float *s, const uint8_t *vx, const uint8_t *vy, size_t nc, void *stream);
// test/Conversion/RVV/rvv-to-emitc-repack-gemv-q8-0-q8-0.mlir:29-33
extern "C" int tcrv_emitc_ggml_repack_gemv_q8_0_q8_0_kernel_ggml_repack_gemv_q8_0_q8_0(
    size_t n, float *s, const uint8_t *vx, const uint8_t *vy, size_t nc, void *stream);
// test/Conversion/RVV/rvv-to-emitc-repack-gemm-q4-0-q8-0.mlir:22-28
extern "C" int tcrv_emitc_ggml_repack_gemm_q4_0_q8_0_kernel_ggml_repack_gemm_q4_0_q8_0(
    size_t n, float *s, const uint8_t *vx, const uint8_t *vy, size_t nr, size_t nc, size_t bs,
    void *stream);
// test/Conversion/RVV/rvv-to-emitc-pack-q4-0-to-q4-0x16.mlir:20-22
extern "C" int tcrv_emitc_ggml_pack_q4_0_to_q4_0x16_kernel_ggml_pack_q4_0_to_q4_0x16(
    size_t nblocks, const uint8_t *src, uint8_t *dst, void *stream);
// test/Conversion/RVV/rvv-to-emitc-ggml-quantize-row-q8-0.mlir:25-27
extern "C" int tcrv_emitc_quantize_row_q8_0_kernel_quantize_row_q8_0(size_t n, const float *x,
                                                                    uint8_t *vy, void *stream);
// test/Conversion/RVV/rvv-to-emitc-packed-i4-offset-binary-x-i8-product-reduce.mlir:24-29
extern "C" int tcrv_emitc_rvv_q4_0_q8_0_integer_core_kernel_rvv_q4_0_q8_0_integer_core(
    const int8_t *w, const int8_t *qlo, const int8_t *qhi, const int32_t *acc, int32_t *out,
    size_t n, void *stream);

// No fixture (the reference has no block-dequant op): ggml's
// dequantize_row_q8_0 / dequantize_row_q4_0(const block *x, float *y, int64_t k)
// in the boundary's (vx, y, n) form.
extern "C" int tcrv_emitc_ggml_dequantize_row_q8_0_kernel_ggml_dequantize_row_q8_0(
    const uint8_t *vx, float *y, size_t n, void *stream);
extern "C" int tcrv_emitc_ggml_dequantize_row_q4_0_kernel_ggml_dequantize_row_q4_0(
    const uint8_t *vx, float *y, size_t n, void *stream);

#endif  // TCRV_EMITC_FIXTURE_PROTOTYPES_H_
