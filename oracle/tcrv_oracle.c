/*
 * tcrv_oracle.c -- scalar CPU restatement of TianChen-RV's quantized hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Each function names the reference emitter it restates (paths relative to the
 * TianChen-RV tree).  Folds use explicit fmaf() in the reference's order, which
 * is what the reference's single-expression C fold contracts to under the
 * default -ffp-contract=on (test/Conversion/RVV/rvv-to-emitc-q4-0-q8-0-block-dot.mlir:77-94).
 * Build with -ffp-contract=off so no other expression is contracted.
 */
#include "tcrv_oracle.h"

#include <math.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* binary16 <-> binary32                                                     */
/* ------------------------------------------------------------------------ */

float tcrv_oracle_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t bits;
  float f;
  if (e == 0) {
    /* zero or subnormal: m * 2^-24, exact in binary32 */
    f = (float)m * 0x1p-24f;
    return sign ? -f : f;
  }
  if (e == 31)
    bits = sign | 0x7f800000u | (m << 13);
  else
    bits = sign | ((e + 112u) << 23) | (m << 13);
  memcpy(&f, &bits, sizeof f);
  return f;
}

uint16_t tcrv_oracle_f32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, sizeof x);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t absx = x & 0x7fffffffu;
  uint32_t e = absx >> 23;
  uint32_t mant = absx & 0x7fffffu;
  if (e == 255) /* inf / nan (quiet the nan, keep the top payload bits) */
    return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
  if (e >= 143) /* >= 2^16: overflows to inf under round-to-nearest */
    return (uint16_t)(sign | 0x7c00u);
  if (e >= 113) { /* normal binary16 range */
    uint32_t h = ((e - 112u) << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
      h += 1u; /* a carry into the exponent is the correct result (incl. inf) */
    return (uint16_t)(sign | h);
  }
  if (e < 102) /* below 2^-25: rounds to (signed) zero */
    return sign;
  { /* binary16 subnormal: round (1.mant * 2^(e-127)) / 2^-24 to an integer */
    uint32_t m = mant | 0x800000u;
    uint32_t shift = 126u - e; /* 14..24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u)))
      q += 1u;
    return (uint16_t)(sign | q);
  }
}

static inline float load_d(const uint8_t *block) {
  uint16_t h;
  memcpy(&h, block, sizeof h);
  return tcrv_oracle_fp16_to_f32(h);
}

static inline void store_d(uint8_t *block, float d) {
  uint16_t h = tcrv_oracle_f32_to_fp16(d);
  memcpy(block, &h, sizeof h);
}

/* ------------------------------------------------------------------------ */
/* a1: elementwise add                                                       */
/* emitScopeForLoop lib/Conversion/RVV/RVVToEmitC.cpp:605 -> emitBinary      */
/* :1873-1911 (vfadd for f32 via binaryMnemonic :4976-4993); harness oracle  */
/* lhs[i]+rhs[i] examples/qemu/harness_add.cpp:16.                            */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_add_f32(const float *lhs, const float *rhs, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i)
    out[i] = lhs[i] + rhs[i];
}

void tcrv_oracle_add_i32(const int32_t *lhs, const int32_t *rhs, int32_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i)
    out[i] = (int32_t)((uint32_t)lhs[i] + (uint32_t)rhs[i]); /* vadd wraps */
}

#define TCRV_ORACLE_BINARY_LOOP(T)                                         \
  do {                                                                     \
    const T *a = (const T *)lhs, *b = (const T *)rhs;                      \
    T *o = (T *)out;                                                       \
    for (size_t i = 0; i < n; ++i)                                         \
      o[i] = kind == 0 ? (T)(a[i] + b[i]) : kind == 1 ? (T)(a[i] - b[i])   \
                                                      : (T)(a[i] * b[i]);  \
  } while (0)

int tcrv_oracle_binary(int kind, int elem, const void *lhs, const void *rhs, void *out,
                       size_t n) {
  if (kind < 0 || kind > 2)
    return -1;
  /* integer elements on unsigned types: the low bits of the result are the
   * RVV vadd/vsub/vmul result for signed and unsigned elements alike
   * (unsigned short promotes to int, so the product is taken in uint32_t) */
  switch (elem) {
  case 0:
  case 1: TCRV_ORACLE_BINARY_LOOP(uint8_t); break;
  case 2:
  case 3: {
    const uint16_t *a = (const uint16_t *)lhs, *b = (const uint16_t *)rhs;
    uint16_t *o = (uint16_t *)out;
    for (size_t i = 0; i < n; ++i) {
      uint32_t x = a[i], y = b[i];
      o[i] = (uint16_t)(kind == 0 ? x + y : kind == 1 ? x - y : x * y);
    }
    break;
  }
  case 4:
  case 5: TCRV_ORACLE_BINARY_LOOP(uint32_t); break;
  case 6: TCRV_ORACLE_BINARY_LOOP(uint64_t); break;
  case 7: TCRV_ORACLE_BINARY_LOOP(float); break;
  case 8: TCRV_ORACLE_BINARY_LOOP(double); break;
  default: return -1;
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* a3: Q8_0 dequantize (ggml dequantize_row_q8_0; block layout pinned by     */
/* RVVDialectWideningOps.cpp:3358-3372, fp16 read RVVToEmitCBlockQuantLinear */
/* .cpp:117,140).  int8 * fp16-valued float is exact in binary32.            */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_dequantize_row_q8_0(size_t n, float *y, const uint8_t *vx) {
  size_t nb = n / TCRV_QK;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t *blk = vx + b * TCRV_Q8_0_BLOCK_BYTES;
    float d = load_d(blk);
    const int8_t *qs = (const int8_t *)(blk + 2);
    for (size_t j = 0; j < TCRV_QK; ++j)
      y[b * TCRV_QK + j] = (float)qs[j] * d;
  }
}

/* ------------------------------------------------------------------------ */
/* a3b: Q4_0 dequantize (ggml dequantize_row_q4_0).  Block layout: fp16 d @0, */
/* 16 packed bytes @2, element j in the low nibble of qs[j] and element j+16 */
/* in the high one (RVVOps.td:3893-3897).  The nibble decode is the op's     */
/* offset-binary one (RVVOps.td:3837-3842; emitOffsetBinaryDecodeValue       */
/* RVVToEmitC.cpp:2524-2561): v = w ^ 0x88, lo = (int8)(v << 4) >> 4,       */
/* hi = (int8)v >> 4, i.e. nibble - 8.  A 4-bit integer times an fp16-valued */
/* float is exact in binary32.                                               */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_dequantize_row_q4_0(size_t n, float *y, const uint8_t *vx) {
  size_t nb = n / TCRV_QK;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t *blk = vx + b * TCRV_Q4_0_BLOCK_BYTES;
    float d = load_d(blk);
    const uint8_t *qs = blk + 2;
    for (size_t j = 0; j < TCRV_QK / 2; ++j) {
      uint8_t v = (uint8_t)(qs[j] ^ 0x88u);
      int8_t lo = (int8_t)((int8_t)(uint8_t)(v << 4) >> 4);
      int8_t hi = (int8_t)((int8_t)v >> 4);
      y[b * TCRV_QK + j] = (float)lo * d;
      y[b * TCRV_QK + TCRV_QK / 2 + j] = (float)hi * d;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* a4: packed-i4 offset-binary x i8 integer core (one Q4_0 block x one Q8_0  */
/* block).  emitOffsetBinaryDecodeValue RVVToEmitC.cpp:2524-2561:            */
/*   v = w ^ 0x88; lo = (int8)(v << 4) >> 4; hi = (int8)v >> 4;             */
/* emitOffsetBinaryProductFromDecodedValue :2563-2589: i16 lanes             */
/*   p = lo*y_lo (vwmul) + hi*y_hi (vwmacc);  then vwredsum to i32           */
/* (RVVToEmitCBlockQuantLinear.cpp:160-220; y_hi at +16, RVVOps.td:3893-3897)*/
/* ------------------------------------------------------------------------ */

/* The same core as the standalone kernel the reference emits for the op      */
/* (rvv-to-emitc-packed-i4-offset-binary-x-i8-product-reduce.mlir:22-27, its  */
/* CHECK lines :48-70): out[0] = acc[0] seeded before the strip loop, then   */
/* each strip's i16 lanes vwredsum'd onto the running int32 cell, which wraps */
/* modulo 2^32 like the RVV integer add.                                       */
void tcrv_oracle_packed_i4_offset_binary_x_i8_product_reduce(const int8_t *w, const int8_t *qlo,
                                                             const int8_t *qhi,
                                                             const int32_t *acc, int32_t *out,
                                                             size_t n) {
  uint32_t cell = (uint32_t)acc[0];
  for (size_t i = 0; i < n; ++i) {
    uint8_t v = (uint8_t)((uint8_t)w[i] ^ 0x88u);
    int8_t lo = (int8_t)((int8_t)(uint8_t)(v << 4) >> 4);
    int8_t hi = (int8_t)((int8_t)v >> 4);
    int16_t lane = (int16_t)((int16_t)lo * (int16_t)qlo[i]);       /* vwmul  */
    lane = (int16_t)(lane + (int16_t)hi * (int16_t)qhi[i]);          /* vwmacc */
    cell += (uint32_t)(int32_t)lane;                                  /* vwredsum */
  }
  out[0] = (int32_t)cell;
}

int32_t tcrv_oracle_q4_0_q8_0_block_sumi(const uint8_t *xb, const uint8_t *yb) {
  const uint8_t *w = xb + 2;
  const int8_t *ylo = (const int8_t *)(yb + 2);
  const int8_t *yhi = (const int8_t *)(yb + 2 + 16);
  int32_t sumi = 0;
  for (int j = 0; j < 16; ++j) {
    uint8_t v = (uint8_t)(w[j] ^ 0x88u);
    int8_t lo = (int8_t)((int8_t)(uint8_t)(v << 4) >> 4);
    int8_t hi = (int8_t)((int8_t)v >> 4);
    int16_t lane = (int16_t)((int16_t)lo * (int16_t)ylo[j]);     /* vwmul  */
    lane = (int16_t)(lane + (int16_t)hi * (int16_t)yhi[j]);        /* vwmacc */
    sumi += lane;                                                   /* vwredsum */
  }
  return sumi;
}

/* a5's integer core: vwmul i8 -> i16, vwredsum i16 -> i32
 * (RVVToEmitCBlockQuantLinear.cpp:7330-7480). */
int32_t tcrv_oracle_q8_0_q8_0_block_sumi(const uint8_t *xb, const uint8_t *yb) {
  const int8_t *qx = (const int8_t *)(xb + 2);
  const int8_t *qy = (const int8_t *)(yb + 2);
  int32_t sumi = 0;
  for (int j = 0; j < TCRV_QK; ++j)
    sumi += (int16_t)((int16_t)qx[j] * (int16_t)qy[j]);
  return sumi;
}

void tcrv_oracle_block_sums_q8_0_q8_0(size_t n, int32_t *sumi, const uint8_t *vx,
                                      const uint8_t *vy) {
  size_t nb = n / TCRV_QK;
  for (size_t b = 0; b < nb; ++b)
    sumi[b] = tcrv_oracle_q8_0_q8_0_block_sumi(vx + b * TCRV_Q8_0_BLOCK_BYTES,
                                               vy + b * TCRV_Q8_0_BLOCK_BYTES);
}

void tcrv_oracle_block_sums_q4_0_q8_0(size_t n, int32_t *sumi, const uint8_t *vx,
                                      const uint8_t *vy) {
  size_t nb = n / TCRV_QK;
  for (size_t b = 0; b < nb; ++b)
    sumi[b] = tcrv_oracle_q4_0_q8_0_block_sumi(vx + b * TCRV_Q4_0_BLOCK_BYTES,
                                               vy + b * TCRV_Q8_0_BLOCK_BYTES);
}

/* ------------------------------------------------------------------------ */
/* a5: tcrv_rvv.q8_0_q8_0_block_dot = ggml_vec_dot_q8_0_q8_0                 */
/* emitQ8_0Q8_0BlockDot RVVToEmitCBlockQuantLinear.cpp:7264-7671.           */
/* nb = n/32 (:7340); ascending block loop; per block sumi reset; fold       */
/*   sumf = sumf + (float)sumi * (d_x * d_y)      (:7538-7575)               */
/* which contracts to fma((float)sumi, d_x*d_y, sumf); *s = sumf (:7655).    */
/* ------------------------------------------------------------------------ */

static float vec_dot_q8_0_q8_0_row(size_t n, const uint8_t *vx, const uint8_t *vy) {
  size_t nb = n / TCRV_QK;
  float sumf = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t *xb = vx + b * TCRV_Q8_0_BLOCK_BYTES;
    const uint8_t *yb = vy + b * TCRV_Q8_0_BLOCK_BYTES;
    float dx = load_d(xb);
    float dy = load_d(yb);
    int32_t sumi = tcrv_oracle_q8_0_q8_0_block_sumi(xb, yb);
    float dxy = dx * dy;
    sumf = fmaf((float)sumi, dxy, sumf);
  }
  return sumf;
}

void tcrv_oracle_vec_dot_q8_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                   const uint8_t *vy) {
  *s = vec_dot_q8_0_q8_0_row(n, vx, vy);
}

/* ------------------------------------------------------------------------ */
/* a6: tcrv_rvv.q4_0_q8_0_block_dot = ggml_vec_dot_q4_0_q8_0                 */
/* emitQ4_0Q8_0BlockDot RVVToEmitCBlockQuantLinear.cpp:29-471; only n, s,    */
/* vx, vy are read (:30-46); fold (:322-356)                                 */
/*   sumf = sumf + ((float)sumi * d_x) * d_y                                 */
/* which contracts to fma(fl((float)sumi*d_x), d_y, sumf).  x = Q4_0 weight, */
/* y = Q8_0 activation.                                                      */
/* ------------------------------------------------------------------------ */

static float vec_dot_q4_0_q8_0_row(size_t n, const uint8_t *vx, const uint8_t *vy) {
  size_t nb = n / TCRV_QK;
  float sumf = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t *xb = vx + b * TCRV_Q4_0_BLOCK_BYTES;
    const uint8_t *yb = vy + b * TCRV_Q8_0_BLOCK_BYTES;
    float dx = load_d(xb);
    float dy = load_d(yb);
    int32_t sumi = tcrv_oracle_q4_0_q8_0_block_sumi(xb, yb);
    float t = (float)sumi * dx;
    sumf = fmaf(t, dy, sumf);
  }
  return sumf;
}

void tcrv_oracle_vec_dot_q4_0_q8_0(size_t n, float *s, size_t bs, const uint8_t *vx,
                                   size_t bx, const uint8_t *vy, size_t by, int32_t nrc) {
  (void)bs;
  (void)bx;
  (void)by;
  (void)nrc;
  *s = vec_dot_q4_0_q8_0_row(n, vx, vy);
}

static int clamp_threads(int nthreads) {
#ifdef _OPENMP
  return nthreads < 1 ? 1 : nthreads;
#else
  (void)nthreads;
  return 1;
#endif
}

void tcrv_oracle_vec_dot_q8_0_q8_0_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                        const uint8_t *vy, size_t by, size_t nrows,
                                        int nthreads) {
  int nt = clamp_threads(nthreads);
  long long nr = (long long)nrows;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
#endif
  for (long long r = 0; r < nr; ++r)
    s[r] = vec_dot_q8_0_q8_0_row(n, vx + (size_t)r * bx, vy + (size_t)r * by);
  (void)nt;
}

void tcrv_oracle_vec_dot_q4_0_q8_0_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                        const uint8_t *vy, size_t by, size_t nrows,
                                        int nthreads) {
  int nt = clamp_threads(nthreads);
  long long nr = (long long)nrows;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
#endif
  for (long long r = 0; r < nr; ++r)
    s[r] = vec_dot_q4_0_q8_0_row(n, vx + (size_t)r * bx, vy + (size_t)r * by);
  (void)nt;
}

/* ------------------------------------------------------------------------ */
/* a7: tcrv_rvv.q4_0_q8_0_gemm (G2), emitQ4_0Q8_0Gemm                        */
/* RVVToEmitCBlockQuantLinear.cpp:1691-2121: row loop ir < nr, weight row    */
/* vx + ir*bx, output row s + ir*bs, every column col < nc reads vy + col*by */
/* and s[ir*bs + col] is the independent a6 block dot (RVVOps.td:4147-4151). */
/* a9: the Q8_0 x Q8_0 GEMM, same nest and ABI, elements = a5.               */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_gemm_q4_0_q8_0(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                                int nthreads) {
  int nt = clamp_threads(nthreads);
  long long nrl = (long long)nr;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
#endif
  for (long long ir = 0; ir < nrl; ++ir)
    for (size_t col = 0; col < nc; ++col)
      s[(size_t)ir * bs + col] =
          vec_dot_q4_0_q8_0_row(n, vx + (size_t)ir * bx, vy + col * by);
  (void)nt;
}

void tcrv_oracle_gemm_q8_0_q8_0(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                                int nthreads) {
  int nt = clamp_threads(nthreads);
  long long nrl = (long long)nr;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt) if (nt > 1)
#endif
  for (long long ir = 0; ir < nrl; ++ir)
    for (size_t col = 0; col < nc; ++col)
      s[(size_t)ir * bs + col] =
          vec_dot_q8_0_q8_0_row(n, vx + (size_t)ir * bx, vy + col * by);
  (void)nt;
}

/* ------------------------------------------------------------------------ */
/* a10: tcrv_rvv.quantize_row_q8_0 (RVVOps.td:8345-8431, ggml riscv/quants.c */
/* RVV path):  amax = max|x| (vfredmax of vfabs seeded with 0.0f);           */
/* d = amax/127.0f; id = d ? 1.0f/d : 0.0f; y.d = (_Float16)d (RNE);         */
/* q = (int8)(int16)sat_rne(x*id)  (vfncvt_x_f_w_i16 then vncvt_x_x_w_i8).   */
/* ------------------------------------------------------------------------ */

static int16_t f32_to_i16_rne_sat(float v) {
  if (v != v)
    return 32767; /* RVV float->int conversion of NaN gives the largest positive */
  float r = rintf(v); /* default rounding mode: nearest-even */
  if (r >= 32767.0f)
    return 32767;
  if (r <= -32768.0f)
    return -32768;
  return (int16_t)r;
}

void tcrv_oracle_quantize_row_q8_0(size_t n, const float *x, uint8_t *vy) {
  size_t nb = n / TCRV_QK;
  for (size_t b = 0; b < nb; ++b) {
    const float *xb = x + b * TCRV_QK;
    uint8_t *yb = vy + b * TCRV_Q8_0_BLOCK_BYTES;
    float amax = 0.0f;
    for (int j = 0; j < TCRV_QK; ++j) {
      float a = fabsf(xb[j]);
      if (a > amax)
        amax = a;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    store_d(yb, d);
    int8_t *qs = (int8_t *)(yb + 2);
    for (int j = 0; j < TCRV_QK; ++j) {
      float v = xb[j] * id;
      int16_t w = f32_to_i16_rne_sat(v);
      qs[j] = (int8_t)(uint8_t)(uint16_t)w; /* vncvt truncates to the low byte */
    }
  }
}

/* ------------------------------------------------------------------------ */
/* a11: Q4_0 quantizer (ggml quantize_row_q4_0_ref; not an op of the         */
/* reference, it only defines the synthetic weight bytes).                   */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_quantize_row_q4_0(size_t n, const float *x, uint8_t *vy) {
  size_t nb = n / TCRV_QK;
  for (size_t b = 0; b < nb; ++b) {
    const float *xb = x + b * TCRV_QK;
    uint8_t *yb = vy + b * TCRV_Q4_0_BLOCK_BYTES;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < TCRV_QK; ++j) {
      float v = xb[j];
      if (amax < fabsf(v)) {
        amax = fabsf(v);
        max = v;
      }
    }
    float d = max / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    store_d(yb, d);
    for (int j = 0; j < 16; ++j) {
      float x0 = xb[j] * id;
      float x1 = xb[16 + j] * id;
      int q0 = (int8_t)(x0 + 8.5f);
      int q1 = (int8_t)(x1 + 8.5f);
      if (q0 > 15)
        q0 = 15;
      if (q1 > 15)
        q1 = 15;
      yb[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

/* ------------------------------------------------------------------------ */
/* a8: make_block_q4_0x16 (RVVOps.td:4551-4626; emitPackQ4_0ToX16            */
/* RVVToEmitCBlockQuantLinear.cpp:2674-2852): out.d[i] = in[i].d;            */
/* out.qs[i] = in[i%16].qs[i/16] ^ 0x88.                                     */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_pack_q4_0_to_q4_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst) {
  for (size_t o = 0; o < nblocks; ++o) {
    const uint8_t *in = src + o * 16 * TCRV_Q4_0_BLOCK_BYTES;
    uint8_t *out = dst + o * TCRV_Q4_0X16_BLOCK_BYTES;
    for (int i = 0; i < 16; ++i)
      memcpy(out + 2 * i, in + i * TCRV_Q4_0_BLOCK_BYTES, 2);
    for (int i = 0; i < 256; ++i)
      out[32 + i] = (uint8_t)(in[(i % 16) * TCRV_Q4_0_BLOCK_BYTES + 2 + i / 16] ^ 0x88u);
  }
}

/* a8: repacked GEMV (emitRepackGemvQ4_0Q8_0 RVVToEmitCBlockQuantLinear.cpp:  */
/* 2853-3357).  Group x of 16 weight rows, block b at vx + (x*nb + b)*288;   */
/* lane r: 16 nibble steps i, byte qs[i*16 + r] (already ^0x88), lo = sext   */
/* low nibble (vsll/vsra), hi = byte >> 4 (vsra); i16 accumulators lo*a.qs[i]*/
/* and hi*a.qs[16+i]; vwadd; fold (:3245-3290)                               */
/*   acc = vfmacc(acc, vfcvt(sumi), vfwmul(d_w[r], d_a))                     */
/* = fma((float)sumi, d_w*d_a, acc) (the f16 x f16 product is exact).        */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_repack_gemv_q4_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                       const uint8_t *vy, size_t nc) {
  size_t nb = n / TCRV_QK;
  size_t ngroups = nc / 16;
  for (size_t x = 0; x < ngroups; ++x) {
    float acc[16];
    for (int r = 0; r < 16; ++r)
      acc[r] = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
      const uint8_t *bl = vx + (x * nb + b) * TCRV_Q4_0X16_BLOCK_BYTES;
      const uint8_t *al = vy + b * TCRV_Q8_0_BLOCK_BYTES;
      const int8_t *aqs = (const int8_t *)(al + 2);
      float da = load_d(al);
      for (int r = 0; r < 16; ++r) {
        int16_t sumi_lo = 0, sumi_hi = 0;
        for (int i = 0; i < 16; ++i) {
          int8_t v = (int8_t)bl[32 + i * 16 + r];
          int8_t lo = (int8_t)((int8_t)(uint8_t)((uint8_t)v << 4) >> 4);
          int8_t hi = (int8_t)(v >> 4);
          sumi_lo = (int16_t)(sumi_lo + (int16_t)lo * (int16_t)aqs[i]);
          sumi_hi = (int16_t)(sumi_hi + (int16_t)hi * (int16_t)aqs[16 + i]);
        }
        int32_t sumi = (int32_t)sumi_lo + (int32_t)sumi_hi;
        float dw = load_d(bl + 2 * r);
        float dc = dw * da;
        acc[r] = fmaf((float)sumi, dc, acc[r]);
      }
    }
    for (int r = 0; r < 16; ++r)
      s[x * 16 + r] = acc[r];
  }
}

/* ------------------------------------------------------------------------ */
/* block_q8_0x16 pack / unpack and the Q8_0 repacked GEMV                    */
/* (emitRepackGemvQ8_0Q8_0 RVVToEmitCBlockQuantLinear.cpp:3930-4379: weight  */
/* group x at vx + x*nb*544, block l at +l*544; position loop i < 32 reads   */
/* byte 32 + i*16 + r of lane r; vwmul i8 x i8 -> i16, vwadd_wv into i32;    */
/* fold vfmacc(acc, vfcvt(sumi), vfwmul(d_w[r], d_a)) (:4258-4330)).         */
/* ------------------------------------------------------------------------ */

void tcrv_oracle_pack_q8_0_to_q8_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst) {
  for (size_t o = 0; o < nblocks; ++o) {
    const uint8_t *in = src + o * 16 * TCRV_Q8_0_BLOCK_BYTES;
    uint8_t *out = dst + o * TCRV_Q8_0X16_BLOCK_BYTES;
    for (int r = 0; r < 16; ++r)
      memcpy(out + 2 * r, in + r * TCRV_Q8_0_BLOCK_BYTES, 2);
    for (int i = 0; i < 32; ++i)
      for (int r = 0; r < 16; ++r)
        out[32 + i * 16 + r] = in[r * TCRV_Q8_0_BLOCK_BYTES + 2 + i];
  }
}

/* The split (SoA) layout: a byte permutation of the plain rows, no arithmetic. */
void tcrv_oracle_pack_q4_0_to_soa(size_t nrows, size_t nb, const uint8_t *src, size_t bx,
                                  uint8_t *dst) {
  uint8_t *scales = dst + nrows * nb * 16;
  for (size_t r = 0; r < nrows; ++r)
    for (size_t b = 0; b < nb; ++b) {
      const uint8_t *blk = src + r * bx + b * TCRV_Q4_0_BLOCK_BYTES;
      memcpy(dst + (r * nb + b) * 16, blk + 2, 16);
      memcpy(scales + (r * nb + b) * 2, blk, 2);
    }
}

void tcrv_oracle_unpack_q4_0_soa(size_t nrows, size_t nb, const uint8_t *src, uint8_t *dst) {
  const uint8_t *scales = src + nrows * nb * 16;
  for (size_t t = 0; t < nrows * nb; ++t) {
    memcpy(dst + t * TCRV_Q4_0_BLOCK_BYTES, scales + t * 2, 2);
    memcpy(dst + t * TCRV_Q4_0_BLOCK_BYTES + 2, src + t * 16, 16);
  }
}

void tcrv_oracle_unpack_q4_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst) {
  for (size_t o = 0; o < nblocks; ++o) {
    const uint8_t *in = src + o * TCRV_Q4_0X16_BLOCK_BYTES;
    uint8_t *out = dst + o * 16 * TCRV_Q4_0_BLOCK_BYTES;
    for (int r = 0; r < 16; ++r)
      memcpy(out + r * TCRV_Q4_0_BLOCK_BYTES, in + 2 * r, 2);
    for (int i = 0; i < 256; ++i)
      out[(i % 16) * TCRV_Q4_0_BLOCK_BYTES + 2 + i / 16] = (uint8_t)(in[32 + i] ^ 0x88u);
  }
}

void tcrv_oracle_unpack_q8_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst) {
  for (size_t o = 0; o < nblocks; ++o) {
    const uint8_t *in = src + o * TCRV_Q8_0X16_BLOCK_BYTES;
    uint8_t *out = dst + o * 16 * TCRV_Q8_0_BLOCK_BYTES;
    for (int r = 0; r < 16; ++r)
      memcpy(out + r * TCRV_Q8_0_BLOCK_BYTES, in + 2 * r, 2);
    for (int i = 0; i < 32; ++i)
      for (int r = 0; r < 16; ++r)
        out[r * TCRV_Q8_0_BLOCK_BYTES + 2 + i] = in[32 + i * 16 + r];
  }
}

void tcrv_oracle_repack_gemv_q8_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                       const uint8_t *vy, size_t nc) {
  size_t nb = n / TCRV_QK;
  size_t ngroups = nc / 16;
  for (size_t x = 0; x < ngroups; ++x) {
    float acc[16];
    for (int r = 0; r < 16; ++r)
      acc[r] = 0.0f;
    for (size_t b = 0; b < nb; ++b) {
      const uint8_t *bl = vx + (x * nb + b) * TCRV_Q8_0X16_BLOCK_BYTES;
      const uint8_t *al = vy + b * TCRV_Q8_0_BLOCK_BYTES;
      const int8_t *aqs = (const int8_t *)(al + 2);
      float da = load_d(al);
      for (int r = 0; r < 16; ++r) {
        int32_t sumi = 0;
        for (int i = 0; i < 32; ++i) {
          int16_t prod = (int16_t)((int16_t)(int8_t)bl[32 + i * 16 + r] * (int16_t)aqs[i]);
          sumi += prod; /* vwadd_wv: i32 += widened i16 */
        }
        float dw = load_d(bl + 2 * r);
        float dc = dw * da; /* vfwmul f16 x f16 -> f32: exact */
        acc[r] = fmaf((float)sumi, dc, acc[r]);
      }
    }
    for (int r = 0; r < 16; ++r)
      s[x * 16 + r] = acc[r];
  }
}

/* Inverse of the repack GEMM's activation addressing (RVVToEmitCBlockQuantLinear.cpp:
 * 2344-2600: al.d[c], al.qs[i*4 + c] low half, al.qs[64 + i*4 + c] high half). */
void tcrv_oracle_pack_q8_0_to_q8_0x4(size_t nrows, size_t nb, const uint8_t *src, size_t by,
                                     uint8_t *dst) {
  for (size_t y = 0; y < nrows / 4; ++y)
    for (size_t b = 0; b < nb; ++b) {
      uint8_t *o = dst + (y * nb + b) * TCRV_Q8_0X4_BLOCK_BYTES;
      for (int c = 0; c < 4; ++c) {
        const uint8_t *blk = src + (y * 4 + c) * by + b * TCRV_Q8_0_BLOCK_BYTES;
        o[2 * c] = blk[0];
        o[2 * c + 1] = blk[1];
        for (int e = 0; e < TCRV_QK; ++e)
          o[8 + 4 * e + c] = blk[2 + e];
      }
    }
}

/* emitRepackGemmQ4_0Q8_0 (RVVToEmitCBlockQuantLinear.cpp:2122-2600), RVV 1.0 form:
 * per (row group y, weight group x, block l) the lane-wise i16 lo/hi sums over
 * the 16 nibble steps, widened and added, then the fp16 x fp16 scale product
 * and one fused multiply-add per (activation row c, weight row r). */
void tcrv_oracle_repack_gemm_q4_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                       const uint8_t *vy, size_t nr, size_t nc, size_t bs) {
  size_t nb = n / TCRV_QK;
  for (size_t y = 0; y < nr / 4; ++y)
    for (size_t x = 0; x < nc / 16; ++x) {
      float acc[4][16];
      for (int c = 0; c < 4; ++c)
        for (int r = 0; r < 16; ++r)
          acc[c][r] = 0.0f;
      for (size_t l = 0; l < nb; ++l) {
        const uint8_t *bl = vx + (x * nb + l) * TCRV_Q4_0X16_BLOCK_BYTES;
        const uint8_t *al = vy + (y * nb + l) * TCRV_Q8_0X4_BLOCK_BYTES;
        for (int c = 0; c < 4; ++c) {
          float da = load_d(al + 2 * c);
          for (int r = 0; r < 16; ++r) {
            int16_t sumi_lo = 0, sumi_hi = 0;
            for (int i = 0; i < 16; ++i) {
              int8_t v = (int8_t)bl[32 + i * 16 + r];
              int8_t lo = (int8_t)((int8_t)(uint8_t)((uint8_t)v << 4) >> 4);
              int8_t hi = (int8_t)(v >> 4);
              sumi_lo = (int16_t)(sumi_lo + (int16_t)lo * (int16_t)(int8_t)al[8 + i * 4 + c]);
              sumi_hi = (int16_t)(sumi_hi + (int16_t)hi * (int16_t)(int8_t)al[8 + 64 + i * 4 + c]);
            }
            int32_t sumi = (int32_t)sumi_lo + (int32_t)sumi_hi;
            float d = load_d(bl + 2 * r) * da;
            acc[c][r] = fmaf((float)sumi, d, acc[c][r]);
          }
        }
      }
      for (int c = 0; c < 4; ++c)
        for (int r = 0; r < 16; ++r)
          s[(y * 4 + c) * bs + x * 16 + r] = acc[c][r];
    }
}
