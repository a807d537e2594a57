/*
 * tcrv_hip.h -- C-ABI of libtcrv_hip.so, the MI355X (gfx950) runtime library
 * for the kernels TianChen-RV compiles: elementwise add, ggml Q8_0/Q4_0 dequant,
 * the Q8_0.Q8_0 and Q4_0.Q8_0 block dots, and the quantized GEMV/GEMM.
 *
 * Every entry point keeps the parameter roles and order of the reference's
 * emitted kernel `extern "C" void tcrv_emitc_<kernel>_<variant>(...)`
 * (lib/Conversion/RVV/RVVToEmitC.cpp:167-172, :258-268: parameters appear in
 * tcrv_rvv.runtime_abi_value declaration order) and appends one `stream`
 * argument.  Differences from the emitted C, all deliberate:
 *   - pointers are DEVICE pointers owned by the caller (the reference's
 *     "target-export-abi-owned" ownership, include/TianChenRV/Support/
 *     RuntimeABI.h:57-60: the library never allocates, frees or retains them);
 *   - the call is asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream) and returns an int status instead of void;
 *   - like the reference, nb = n / 32 and a trailing partial block is ignored
 *     (RVVToEmitCBlockQuantLinear.cpp:7340, RVVOps.td:8395);
 *   - block pointers and row strides need only the 2-byte alignment every
 *     ggml block already has (fp16 d at offset 0); 16-byte aligned rows (every
 *     row of a 4096-wide matrix) take the 128-bit load path.  An odd address or
 *     stride returns TCRV_HIP_ERR_MISALIGNED.
 *
 * Status: 0 = success; negative = an argument error detected before launch
 * (nothing was launched); positive = the hipError_t reported by the launch.
 * Entry points are reentrant and thread-safe; calls on one stream execute in
 * order, calls on different streams may overlap.
 */
#ifndef TCRV_HIP_H
#define TCRV_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define TCRV_HIP_API __attribute__((visibility("default")))
#else
#define TCRV_HIP_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define TCRV_HIP_QK 32
#define TCRV_HIP_Q8_0_BLOCK_BYTES 34
#define TCRV_HIP_Q4_0_BLOCK_BYTES 18
#define TCRV_HIP_Q4_0X16_BLOCK_BYTES 288

enum {
  TCRV_HIP_OK = 0,
  TCRV_HIP_ERR_NULL_POINTER = -1,   /* a required pointer is NULL */
  TCRV_HIP_ERR_BAD_SIZE = -2,       /* a size/stride violates the kernel's contract */
  TCRV_HIP_ERR_MISALIGNED = -3,     /* a pointer/stride is not aligned as documented */
  TCRV_HIP_ERR_TOO_LARGE = -4,      /* a size exceeds the kernel's index range */
  TCRV_HIP_ERR_UNSUPPORTED = -5,    /* argument combination not implemented */
  TCRV_HIP_ERR_SCRATCH_LIMIT = -6   /* the call needs more than the fixed device scratch */
};

/* Human-readable name of a status value (static storage, never NULL). */
TCRV_HIP_API const char *tcrv_hip_status_string(int status);

/* Library version string, e.g. "tcrv_hip 0.1.0 gfx950". */
TCRV_HIP_API const char *tcrv_hip_version(void);

/* Blocks until all work on `stream` is complete; returns a hipError_t. */
TCRV_HIP_API int tcrv_hip_stream_synchronize(void *stream);

/* ---- a1: elementwise add -------------------------------------------------
 * Replaces tcrv_emitc_<kernel>_<variant>(const T *lhs, const T *rhs, T *out,
 * size_t n) for T = float (test/Conversion/RVV/rvv-to-emitc-add-cpp-golden.mlir:
 * 15-18,33; emitBinary lib/Conversion/RVV/RVVToEmitC.cpp:1873-1911).
 * out[i] = lhs[i] + rhs[i], i < n.  Any 4-byte alignment; 16-byte aligned
 * pointers take the 128-bit path.  out may alias lhs or rhs exactly. */
TCRV_HIP_API int tcrv_hip_add_f32(const float *lhs, const float *rhs, float *out, size_t n, void *stream);

/* Typed binary arithmetic: tcrv_rvv.binary {kind = "add" | "sub" | "mul"}
 * (RVVOps.td:3217-3243; verifier RVVDialectArithmeticOps.cpp:38-82; emitBinary
 * RVVToEmitC.cpp:1873-1911 selecting vadd/vsub/vmul or vfadd/vfsub/vfmul by
 * binaryMnemonic :4976-4993) over the element types of the reference's vector
 * type grid (RVVToEmitC.cpp:5040-5075).  out[i] = lhs[i] <kind> rhs[i], i < n.
 * Integer kinds wrap modulo 2^width (RVV vadd/vsub/vmul keep the low bits, so
 * signed and unsigned share one result); float kinds are single IEEE-754
 * round-to-nearest-even operations (never contracted).  A NaN result may carry
 * an input's payload where RISC-V returns its canonical NaN.  Pointers need the
 * element's alignment; 16-byte aligned ones take the 128-bit path.  out may
 * alias lhs or rhs exactly. */
enum {
  TCRV_HIP_BINARY_ADD = 0,
  TCRV_HIP_BINARY_SUB = 1,
  TCRV_HIP_BINARY_MUL = 2
};
enum {
  TCRV_HIP_ELEM_I8 = 0,
  TCRV_HIP_ELEM_U8 = 1,
  TCRV_HIP_ELEM_I16 = 2,
  TCRV_HIP_ELEM_U16 = 3,
  TCRV_HIP_ELEM_I32 = 4,
  TCRV_HIP_ELEM_U32 = 5,
  TCRV_HIP_ELEM_I64 = 6,
  TCRV_HIP_ELEM_F32 = 7,
  TCRV_HIP_ELEM_F64 = 8
};
TCRV_HIP_API int tcrv_hip_binary(int kind, int elem, const void *lhs, const void *rhs, void *out,
                    size_t n, void *stream);

/* The reference's own add slice and golden are i32
 * (test/Conversion/RVV/rvv-to-emitc-add-cpp-golden.mlir:15-18,33;
 * examples/qemu/harness_add.cpp:11-12): (lhs, rhs, out, n). */
TCRV_HIP_API int tcrv_hip_add_i32(const int32_t *lhs, const int32_t *rhs, int32_t *out, size_t n,
                     void *stream);

/* ---- a3: Q8_0 dequantize --------------------------------------------------
 * ggml dequantize_row_q8_0(const block_q8_0 *x, float *y, int64_t k) (no
 * reference op; block layout RVVDialectWideningOps.cpp:3358-3372).
 * y[32b+j] = qs_b[j] * d_b for b < n/32.  y 4-byte aligned. */
TCRV_HIP_API int tcrv_hip_dequantize_row_q8_0(const uint8_t *vx, float *y, size_t n, void *stream);

/* ---- a3b: Q4_0 dequantize -------------------------------------------------
 * ggml dequantize_row_q4_0(const block_q4_0 *x, float *y, int64_t k) (no
 * reference op; block layout RVVOps.td:3893-3897, nibble decode the op's
 * offset-binary (nibble - 8), RVVOps.td:3837-3842).  For b < n/32, j < 16:
 *   y[32b+j]    = ((qs_b[j] & 15) - 8) * d_b
 *   y[32b+16+j] = ((qs_b[j] >> 4) - 8) * d_b
 * Bit-exact (a 4-bit integer times an fp16 value is exact in binary32).
 * vx 2-byte aligned, y 4-byte aligned (16-byte aligned takes 128-bit stores). */
TCRV_HIP_API int tcrv_hip_dequantize_row_q4_0(const uint8_t *vx, float *y, size_t n, void *stream);

/* ---- a10: f32 -> Q8_0 activation quantizer --------------------------------
 * Replaces tcrv_emitc_..._quantize_row_q8_0(size_t n, const float *x,
 * uint8_t *vy) (test/Conversion/RVV/rvv-to-emitc-ggml-quantize-row-q8-0.mlir:
 * 25-27; RVVOps.td:8345-8431).  x 4-byte aligned. */
TCRV_HIP_API int tcrv_hip_quantize_row_q8_0(size_t n, const float *x, uint8_t *vy, void *stream);

/* ---- a4: the packed-i4 offset-binary x i8 integer core --------------------
 * Replaces tcrv_emitc_..._integer_core(const int8_t *w, const int8_t *qlo,
 * const int8_t *qhi, const int32_t *acc, int32_t *out, size_t n)
 * (test/Conversion/RVV/rvv-to-emitc-packed-i4-offset-binary-x-i8-product-
 * reduce.mlir:22-27; op tcrv_rvv.packed_i4_offset_binary_x_i8_product,
 * RVVOps.td:3814-3871):
 *   out[0] = acc[0] + sum_{i<n} (lo(w[i])*qlo[i] + hi(w[i])*qhi[i])
 * where lo/hi are the weight byte's low/high offset-binary nibbles minus 8, in
 * int32 arithmetic that wraps.  acc may alias out; any alignment. */
TCRV_HIP_API int tcrv_hip_packed_i4_offset_binary_x_i8_product_reduce(const int8_t *w,
                                                                      const int8_t *qlo,
                                                                      const int8_t *qhi,
                                                                      const int32_t *acc,
                                                                      int32_t *out, size_t n,
                                                                      void *stream);

/* ---- a5: Q8_0 . Q8_0 block dot ---------------------------------------------
 * Replaces tcrv_emitc_..._q8_0_q8_0_block_dot(size_t n, float *s,
 * const uint8_t *vx, const uint8_t *vy)
 * (test/Conversion/RVV/rvv-to-emitc-q8-0-q8-0-block-dot.mlir:16-19).
 * *s = sum_b fma((float)sumi_b, d_x*d_y, .) in ascending b. */
TCRV_HIP_API int tcrv_hip_q8_0_q8_0_block_dot(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                 void *stream);

/* Batched form: s[r] = block_dot(vx + r*bx, vy + r*by) for r < nrows;
 * bx, by >= the row bytes when nrows > 1. */
TCRV_HIP_API int tcrv_hip_q8_0_q8_0_block_dot_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                      const uint8_t *vy, size_t by, size_t nrows,
                                      void *stream);

/* ---- a6: Q4_0 . Q8_0 block dot ---------------------------------------------
 * Replaces tcrv_emitc_..._q4_0_q8_0_block_dot(size_t n, float *s, size_t bs,
 * const uint8_t *vx, size_t bx, const uint8_t *vy, size_t by, int32_t nrc),
 * the ggml vec_dot ABI (test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-block-dot.
 * mlir:24-31).  As in the reference only n, s, vx, vy are read
 * (RVVToEmitCBlockQuantLinear.cpp:30-46); *s = sum_b fma(fl(sumi_b*d_x), d_y, .). */
TCRV_HIP_API int tcrv_hip_q4_0_q8_0_block_dot(size_t n, float *s, size_t bs, const uint8_t *vx,
                                 size_t bx, const uint8_t *vy, size_t by, int32_t nrc,
                                 void *stream);

/* Batched form: s[r] = block_dot(vx + r*bx, vy + r*by) for r < nrows. */
TCRV_HIP_API int tcrv_hip_q4_0_q8_0_block_dot_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                      const uint8_t *vy, size_t by, size_t nrows,
                                      void *stream);

/* Per-block int32 sums (the integer core of a4/a5/a6, bit-exact) for nrows
 * row pairs: sumi[r*(n/32) + b].  Same alignment rules as the _rows forms. */
TCRV_HIP_API int tcrv_hip_q8_0_q8_0_block_sums(size_t n, int32_t *sumi, const uint8_t *vx, size_t bx,
                                  const uint8_t *vy, size_t by, size_t nrows, void *stream);
TCRV_HIP_API int tcrv_hip_q4_0_q8_0_block_sums(size_t n, int32_t *sumi, const uint8_t *vx, size_t bx,
                                  const uint8_t *vy, size_t by, size_t nrows, void *stream);

/* ---- a7: Q4_0 x Q8_0 GEMM / decode GEMV -----------------------------------
 * Replaces tcrv_emitc_..._q4_0_q8_0_gemm(size_t n, float *s, const uint8_t *vx,
 * const uint8_t *vy, size_t by, size_t nr, size_t nc, size_t bx, size_t bs)
 * (test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-gemm.mlir:23-31;
 * RVVToEmitCBlockQuantLinear.cpp:1691-2121).
 * s[ir*bs + col] = q4_0 block_dot(vx + ir*bx, vy + col*by), ir < nr, col < nc.
 * bx, by >= the row bytes when nr, nc > 1; bs >= nc when nr > 1. */
TCRV_HIP_API int tcrv_hip_q4_0_q8_0_gemm(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                            size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                            void *stream);

/* Replaces tcrv_emitc_..._q4_0_q8_0_gemm_tile(size_t n, float *s,
 * const uint8_t *vx, const uint8_t *vy, size_t by)
 * (test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-gemm-tile.mlir; op RVVOps.td:
 * 4048-4133, emitter RVVToEmitCBlockQuantLinear.cpp:1392-1690): ONE weight row
 * vx times m activation columns vy + j*by, s[j] = q4_0 block_dot(vx, vy + j*by)
 * for j < m.  The reference fixes m as the op's `activation_cols` attribute;
 * here it is an argument.  Same results as the G2 GEMM with nr = 1. */
TCRV_HIP_API int tcrv_hip_q4_0_q8_0_gemm_tile(size_t n, float *s, const uint8_t *vx,
                                              const uint8_t *vy, size_t by, size_t m,
                                              void *stream);

/* The decode GEMV (the q4_0 GEMM with nc = 1): s[ir] for ir < nr. */
TCRV_HIP_API int tcrv_hip_gemv_q4_0_q8_0(size_t n, float *s, const uint8_t *vx, size_t bx,
                            const uint8_t *vy, size_t nr, void *stream);
/* The decode GEMV with its schedule knob set by the caller, as the reference's
 * block-dot ops carry bounded schedule attributes (integer_core_lmul,
 * multi_block_factor, strip_elision: RVVOps.td:3912-3972) that change how the
 * kernel runs and never what it computes.  rows_per_wave (2, 4 or 8; the plain
 * entry uses 2 for nr <= 2048 and 4 above, tcrv_hip_route_schedule lists the
 * candidates) sets how many
 * weight rows one wave of the register-direct kernel owns; the results are
 * bit-identical for every value.  For n = 2048 and 1024, 4 selects the
 * lane-group kernels, whose waves own 4 or 8 rows by n and nr.  Shapes served
 * by the LDS-staged kernel (odd n/32, rows not 4-byte aligned) ignore it.  Any
 * other value returns TCRV_HIP_ERR_BAD_SIZE. */
TCRV_HIP_API int tcrv_hip_gemv_q4_0_q8_0_shaped(size_t n, float *s, const uint8_t *vx, size_t bx,
                                                const uint8_t *vy, size_t nr, int rows_per_wave,
                                                void *stream);

/* ---- a9: Q8_0 x Q8_0 GEMM (prefill) ---------------------------------------
 * Same ABI as the q4_0 GEMM above; elements are the a5 block dot:
 * s[ir*bs + col] = q8_0 block_dot(vx + ir*bx, vy + col*by).
 * Runs on v_mfma_i32_32x32x32_i8 with one MFMA per 32-element block and the
 * per-block fp32 fold in ascending block order; nc = 1 (decode) runs as a
 * bandwidth-bound GEMV instead (same results).
 * bx, by >= the row bytes when nr, nc > 1; bs >= nc when nr > 1. */
TCRV_HIP_API int tcrv_hip_q8_0_q8_0_gemm(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                            size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                            void *stream);

/* ---- a9 over the GEMM-tile layout (no reference counterpart) --------------
 * A GPU layout of the same Q8_0 bytes for the MFMA GEMM: rows in groups of 64;
 * for group g and block b one 2176-byte record at (g*nb + b)*2176 holding, for
 * rows 64g..64g+63, quants 0-15 (16 B a row), then quants 16-31, then the 64
 * fp16 scales.  Rows past nrows in the last group are zero.  The GEMM stages
 * its operands from this layout by DMA, 16-byte aligned, with no realignment.
 * Bytes of the layout for nrows rows of nb blocks: */
TCRV_HIP_API size_t tcrv_hip_gemm_tiles_bytes(size_t nrows, size_t nb);
/* Plain Q8_0 rows (stride bx, 2-byte aligned) -> the layout at dst (16-byte
 * aligned, tcrv_hip_gemm_tiles_bytes(nrows, nb) bytes). */
TCRV_HIP_API int tcrv_hip_pack_q8_0_to_gemm_tiles(size_t nrows, size_t nb, const uint8_t *src,
                                                  size_t bx, uint8_t *dst, void *stream);
/* The Q8_0 x Q8_0 GEMM over operands in that layout (tx: nr weight rows, ty: nc
 * token rows, both 16-byte aligned): s[ir*bs + col] exactly as
 * tcrv_hip_q8_0_q8_0_gemm computes it from the plain rows.  Weights that are
 * packed once serve every later call.  n/32 at most 1 973 789 (a 64-row
 * group's records under 4 GiB), else TCRV_HIP_ERR_TOO_LARGE. */
TCRV_HIP_API int tcrv_hip_q8_0_q8_0_gemm_tiles(size_t n, float *s, const uint8_t *tx,
                                               const uint8_t *ty, size_t nr, size_t nc,
                                               size_t bs, void *stream);
/* tcrv_hip_q8_0_q8_0_gemm (same ABI and results) with a caller-owned device
 * workspace: both operands are packed into it (tx then ty) and the tiled GEMM
 * runs.  Needs tcrv_hip_q8_0_q8_0_gemm_workspace_bytes(n, nr, nc) bytes, 16-byte
 * aligned; shapes the tiled kernel does not serve (nr < 256, nc < 2, n/32 over
 * 1 973 789) run tcrv_hip_q8_0_q8_0_gemm and leave the workspace untouched.
 * Calls that share a workspace must be ordered (one stream). */
TCRV_HIP_API size_t tcrv_hip_q8_0_q8_0_gemm_workspace_bytes(size_t n, size_t nr, size_t nc);
TCRV_HIP_API int tcrv_hip_q8_0_q8_0_gemm_ws(size_t n, float *s, const uint8_t *vx,
                                            const uint8_t *vy, size_t by, size_t nr, size_t nc,
                                            size_t bx, size_t bs, void *workspace,
                                            size_t workspace_bytes, void *stream);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * tcrv_hip_q8_0_q8_0_gemm_ws (same ABI and results) with its workspace in a
 * fixed device array of tcrv_hip_q8_0_q8_0_gemm_noalloc_max_bytes() (64 MiB)
 * per GPU, held until the process ends; calls no allocating routine.  A shape
 * whose workspace exceeds it returns TCRV_HIP_ERR_SCRATCH_LIMIT before
 * launching anything (4096 x 4096 x K 4096 needs 35.7 MB).  Every call on one
 * GPU shares that GPU's array: calls that overlap in time on one GPU race and
 * must be ordered by the caller (one stream).  The first call on a device
 * with a shape that uses the workspace looks up the array's address (not
 * capturable; make it outside a capture); shapes that run the plain GEMM
 * never touch the array. */
TCRV_HIP_API size_t tcrv_hip_q8_0_q8_0_gemm_noalloc_max_bytes(void);
TCRV_HIP_API int tcrv_hip_q8_0_q8_0_gemm_noalloc(size_t n, float *s, const uint8_t *vx,
                                                 const uint8_t *vy, size_t by, size_t nr,
                                                 size_t nc, size_t bx, size_t bs, void *stream);

/* ---- a7 over the GEMM-tile layout (no reference counterpart) --------------
 * Q4_0 weight rows in the same 2176-byte records, their nibbles decoded to the
 * signed quants (q - 8) in element order: quants 0-15 are the low nibbles of a
 * block's 16 bytes, quants 16-31 the high ones; the fp16 scale is copied.
 * tcrv_hip_gemm_tiles_bytes gives the size.  Plain Q4_0 rows (stride bx, 2-byte
 * aligned) -> dst (16-byte aligned): */
TCRV_HIP_API int tcrv_hip_pack_q4_0_to_gemm_tiles(size_t nrows, size_t nb, const uint8_t *src,
                                                  size_t bx, uint8_t *dst, void *stream);
/* The Q4_0 x Q8_0 GEMM over tx (Q4_0 weights packed as above) and ty (Q8_0
 * tokens packed by tcrv_hip_pack_q8_0_to_gemm_tiles): s[ir*bs + col] exactly as
 * tcrv_hip_q4_0_q8_0_gemm computes it from the plain rows.  Weights that are
 * packed once serve every later call. */
TCRV_HIP_API int tcrv_hip_q4_0_q8_0_gemm_tiles(size_t n, float *s, const uint8_t *tx,
                                               const uint8_t *ty, size_t nr, size_t nc,
                                               size_t bs, void *stream);
/* tcrv_hip_q4_0_q8_0_gemm (same ABI and results) with a caller-owned device
 * workspace: the Q4_0 weights and the Q8_0 tokens are packed into it (tx then
 * ty, one launch) and the tiled GEMM runs.  Needs
 * tcrv_hip_q4_0_q8_0_gemm_workspace_bytes(n, nr, nc) bytes, 16-byte aligned;
 * shapes the tiled kernel does not serve (nr < 256, nc < 2, n/32 over
 * 1 973 789) run tcrv_hip_q4_0_q8_0_gemm and leave the workspace untouched.
 * Calls that share a workspace must be ordered (one stream). */
TCRV_HIP_API size_t tcrv_hip_q4_0_q8_0_gemm_workspace_bytes(size_t n, size_t nr, size_t nc);
TCRV_HIP_API int tcrv_hip_q4_0_q8_0_gemm_ws(size_t n, float *s, const uint8_t *vx,
                                            const uint8_t *vy, size_t by, size_t nr, size_t nc,
                                            size_t bx, size_t bs, void *workspace,
                                            size_t workspace_bytes, void *stream);

/* ---- a8: the x16 block-as-lane weight layout ---------------------------
 * Replaces tcrv_emitc_..._pack_q4_0_to_q4_0x16(size_t nblocks, const uint8_t *src,
 * uint8_t *dst) (test/Conversion/RVV/rvv-to-emitc-pack-q4-0-to-q4-0x16.mlir:
 * 19-21; RVVOps.td:4551-4626, make_block_q4_0x16): for each of nblocks output
 * blocks (288 B) built from 16 consecutive source blocks (18 B),
 * d[i] = src[i].d and qs[i] = src[i % 16].qs[i / 16] ^ 0x88.
 * src 2-byte aligned, dst 4-byte aligned. */
TCRV_HIP_API int tcrv_hip_pack_q4_0_to_q4_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst,
                                  void *stream);

/* block_q8_0x16 (544 B: fp16 d[16], then qs[i*16 + r] = quant i of source block
 * r), the layout tcrv_rvv.repack_gemv_q8_0_q8_0 reads (RVVOps.td:4846-4857).
 * The reference has no op that produces it; this entry is the inverse of that
 * consumer's addressing, so the Q8_0 repacked GEMV can be fed from plain rows. */
TCRV_HIP_API int tcrv_hip_pack_q8_0_to_q8_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst,
                                  void *stream);

/* Replace tcrv_emitc_..._repack_gemv_{q4_0,q8_0}_q8_0(size_t n, float *s,
 * const uint8_t *vx, const uint8_t *vy, size_t nc)
 * (test/Conversion/RVV/rvv-to-emitc-repack-gemv-q4-0-q8-0.mlir:24-28 and the
 * q8-0 fixture; emitters RVVToEmitCBlockQuantLinear.cpp:2853-3357, :3930-4379).
 * vx holds nc/16 groups of 16 weight rows in the x16 layout (group x at
 * vx + x*(n/32)*288, or *544 for Q8_0); vy is one plain Q8_0 activation row.
 * s[x*16 + r] = fold_b fma((float)sumi_{r,b}, d_w[r]*d_a, .) in ascending b --
 * for Q4_0 a different rounding from the plain block dot's fold.
 * A trailing partial group (nc % 16) is not written, as in the reference.
 * vx 4-byte aligned, vy 2-byte aligned. */
TCRV_HIP_API int tcrv_hip_repack_gemv_q4_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                   const uint8_t *vy, size_t nc, void *stream);
TCRV_HIP_API int tcrv_hip_repack_gemv_q8_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                   const uint8_t *vy, size_t nc, void *stream);

/* tcrv_rvv.repack_gemm_q4_0_q8_0 (RVVOps.td:4228-4338, emitRepackGemmQ4_0Q8_0
 * RVVToEmitCBlockQuantLinear.cpp:2122-2600; ABI (n, s, vx, vy, nr, nc, bs) as in
 * rvv-to-emitc-repack-gemm-q4-0-q8-0.mlir:22-28): x16 Q4_0 weights (nc/16
 * groups, group x at vx + x*(n/32)*288) times 4-row-interleaved Q8_0
 * activations (block_q8_0x4, 136 B: fp16 d[4] @0, quant e of row c at
 * 8 + 4e + c; nr/4 groups, group y at vy + y*(n/32)*136):
 * s[(4y + c)*bs + 16x + r] = fold_b fma((float)sumi, d_w[r]*d_a[c], .) in
 * ascending b.  Partial groups (nr % 4, nc % 16) are not written, as in the
 * reference.  vx, vy and s 4-byte aligned; bs >= 16*(nc/16). */
TCRV_HIP_API int tcrv_hip_repack_gemm_q4_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                   const uint8_t *vy, size_t nr, size_t nc, size_t bs,
                                   void *stream);
/* No reference counterpart (ggml repacks the activations itself): groups of 4
 * plain Q8_0 rows of nb blocks (row stride by, 2-byte aligned) -> nrows/4
 * groups of nb block_q8_0x4, the layout tcrv_hip_repack_gemm_q4_0_q8_0 reads.
 * dst 4-byte aligned. */
TCRV_HIP_API int tcrv_hip_pack_q8_0_to_q8_0x4(size_t nrows, size_t nb, const uint8_t *src,
                                 size_t by, uint8_t *dst, void *stream);

/* ---- the split (SoA) Q4_0 weight layout: no reference counterpart --------
 * A GPU layout of the same bytes: for nrows rows of nb blocks, the 16 quant
 * bytes of row r block b at dst + (r*nb + b)*16 and its fp16 scale at
 * dst + nrows*nb*16 + (r*nb + b)*2 (nrows*nb*18 bytes in all), so a block
 * pair is two aligned 128-bit loads and one dword.  The pack reads rows at
 * stride bx (2-byte aligned source, dst 16-byte aligned). */
TCRV_HIP_API int tcrv_hip_pack_q4_0_to_soa(size_t nrows, size_t nb, const uint8_t *src, size_t bx,
                              uint8_t *dst, void *stream);

/* The decode GEMV over split-layout weights: s[r] for r < nr is the a6 block
 * dot of weight row r with the plain Q8_0 activation row vy, bit-identical to
 * tcrv_hip_gemv_q4_0_q8_0 over the same rows (same fold, same order).
 * n/32 even; vx 16-byte aligned (as the pack writes it), vy 4-byte aligned. */
TCRV_HIP_API int tcrv_hip_gemv_q4_0_soa_q8_0(size_t n, float *s, const uint8_t *vx,
                                const uint8_t *vy, size_t nr, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TCRV_HIP_H */
