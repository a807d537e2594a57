// gemm.hip -- a9: Q8_0 x Q8_0 prefill GEMM on MFMA.
//
// Semantics (the reference's GEMM loop nest, RVVToEmitCBlockQuantLinear.cpp:
// 1691-2121, with the Q8_0 block dot of :7264-7671 as the element):
//   s[ir*bs + col] = sum over blocks b ascending of
//                    fma((float)sumi(ir,col,b), d_x(ir,b)*d_y(col,b), .)
// where x = weight rows (vx, stride bx) and y = activation rows (vy, stride by).
//
// K = 32 of v_mfma_i32_32x32x32_i8 is exactly one Q8_0 block, so every MFMA
// yields the int32 block sums of a 32x32 output tile for one block; the fp32
// fold of that block is applied to the tile right away, in ascending block
// order, so every output element sees the reference's sequence of roundings.
//
// Three kernels:
//   gemm_wide<false>       rows 4-byte aligned, at least 256 weight rows: 256 x 128
//                          output tile per work-group (the fast path, below);
//   gemm_occ<false>        rows 4-byte aligned, fewer weight rows: 128 x 128;
//   gemm_q8_0_q8_0_kernel  any 2-byte aligned rows: 4 waves, 2x2 tiles each,
//                          raw block bytes through LDS, scalar scale epilogue.
#include "tcrv_hip_internal.h"
#include "mfma_fold.h"

namespace tcrv {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kGmBM = 128;          // weight rows per work-group
constexpr int kGmBN = 128;          // activation rows per work-group
constexpr int kGmKB = 8;            // blocks per K chunk
constexpr int kGmRow = kGmKB * kQ8Bytes;  // 272 bytes per staged row (16-B multiple)
constexpr int kGmRowChunks = kGmRow / 16; // 17
constexpr int kGmThreads = 256;

// The 16 quant bytes [16h, 16h+16) of block b (b % 2 == kParity) of one staged
// row, as the 4 dwords of an MFMA operand.
template <int kParity>
__device__ __forceinline__ v4i gm_frag(const uint8_t *row, int b, int h) {
  const int off = b * kQ8Bytes + 2 + 16 * h;
  const uint32_t *w = reinterpret_cast<const uint32_t *>(row + (off & ~3));
  v4i f;
  if constexpr (kParity == 0) {  // off % 4 == 2
    const uint32_t r0 = w[0], r1 = w[1], r2 = w[2], r3 = w[3], r4 = w[4];
    f[0] = static_cast<int>(funnel16(r0, r1));
    f[1] = static_cast<int>(funnel16(r1, r2));
    f[2] = static_cast<int>(funnel16(r2, r3));
    f[3] = static_cast<int>(funnel16(r3, r4));
  } else {  // off % 4 == 0
    f[0] = static_cast<int>(w[0]);
    f[1] = static_cast<int>(w[1]);
    f[2] = static_cast<int>(w[2]);
    f[3] = static_cast<int>(w[3]);
  }
  return f;
}

struct GemmTileState {
  float acc[2][2][16];
};

// One block b of the K chunk for this wave's 2x2 tiles.
template <int kParity>
__device__ __forceinline__ void gm_block(GemmTileState &st, const uint8_t *la,
                                         const uint8_t *lb, const float (*da)[kGmBM],
                                         const float (*db)[kGmBN], int b, int wm, int wn,
                                         int li, int h) {
  v4i af[2], bf[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
    af[i] = gm_frag<kParity>(la + (wm * 64 + i * 32 + li) * kGmRow, b, h);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    bf[j] = gm_frag<kParity>(lb + (wn * 64 + j * 32 + li) * kGmRow, b, h);
  const v16i zero = {};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    // rows of this lane's accumulator registers e: 8*(e/4) + 4*h + e%4
    float dx[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v =
          *reinterpret_cast<const float4 *>(&da[b][wm * 64 + i * 32 + 8 * q + 4 * h]);
      dx[4 * q + 0] = v.x;
      dx[4 * q + 1] = v.y;
      dx[4 * q + 2] = v.z;
      dx[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v16i sumi = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], zero, 0, 0, 0);
      const float dy = db[b][wn * 64 + j * 32 + li];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float dxy = dx[e] * dy;
        st.acc[i][j][e] = fmaf(static_cast<float>(sumi[e]), dxy, st.acc[i][j][e]);
      }
    }
  }
}

__global__ __launch_bounds__(kGmThreads) void gemm_q8_0_q8_0_kernel(
    size_t nb, float *s, const uint8_t *vx, const uint8_t *vy, size_t by, size_t nr,
    size_t nc, size_t bx, size_t bs, int rows16) {
  __shared__ __align__(16) uint8_t la[kGmBM * kGmRow + 16];
  __shared__ __align__(16) uint8_t lb[kGmBN * kGmRow + 16];
  __shared__ __align__(16) float da[kGmKB][kGmBM];
  __shared__ __align__(16) float db[kGmKB][kGmBN];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, h = lane >> 5;
  const size_t m0 = static_cast<size_t>(blockIdx.y) * kGmBM;
  const size_t n0 = static_cast<size_t>(blockIdx.x) * kGmBN;

  GemmTileState st;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st.acc[i][j][e] = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kGmKB) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kGmKB), nb - c0));
    const size_t koff = c0 * kQ8Bytes;
    if (nbc == kGmKB && rows16) {  // every staged row segment is 16-byte aligned
      for (int t = tid; t < kGmBM * kGmRowChunks; t += kGmThreads) {
        const int r = t / kGmRowChunks, c = t - r * kGmRowChunks;
        const size_t gr = min(m0 + r, nr - 1);  // rows past nr reuse row nr-1, unstored
        reinterpret_cast<uint4 *>(la + r * kGmRow)[c] =
            reinterpret_cast<const uint4 *>(vx + gr * bx + koff)[c];
      }
      for (int t = tid; t < kGmBN * kGmRowChunks; t += kGmThreads) {
        const int r = t / kGmRowChunks, c = t - r * kGmRowChunks;
        const size_t gc = min(n0 + r, nc - 1);
        reinterpret_cast<uint4 *>(lb + r * kGmRow)[c] =
            reinterpret_cast<const uint4 *>(vy + gc * by + koff)[c];
      }
    } else {
      for (int r = wave; r < kGmBM; r += kGmThreads / 64) {
        const size_t gr = min(m0 + r, nr - 1);
        copy_span_to_lds(la + r * kGmRow, vx + gr * bx + koff, nbc * kQ8Bytes, lane, 64);
      }
      for (int r = wave; r < kGmBN; r += kGmThreads / 64) {
        const size_t gc = min(n0 + r, nc - 1);
        copy_span_to_lds(lb + r * kGmRow, vy + gc * by + koff, nbc * kQ8Bytes, lane, 64);
      }
    }
    __syncthreads();
    for (int t = tid; t < kGmKB * kGmBM; t += kGmThreads) {
      const int b = t / kGmBM, r = t - b * kGmBM;
      if (b < nbc) {
        da[b][r] = fp16_bits_to_f32(
            *reinterpret_cast<const uint16_t *>(la + r * kGmRow + b * kQ8Bytes));
        db[b][r] = fp16_bits_to_f32(
            *reinterpret_cast<const uint16_t *>(lb + r * kGmRow + b * kQ8Bytes));
      }
    }
    __syncthreads();
    for (int b = 0; b < nbc; b += 2) {
      gm_block<0>(st, la, lb, da, db, b, wm, wn, li, h);
      if (b + 1 < nbc)
        gm_block<1>(st, la, lb, da, db, b + 1, wm, wn, li, h);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const size_t col = n0 + wn * 64 + j * 32 + li;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const size_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < nr && col < nc)
          s[row * bs + col] = st.acc[i][j][e];
      }
    }
}


// ---------------------------------------------------------------------------
// Fast path.  Per 32x32 output tile and Q8_0 blocks b, b+1:
//   v_mfma_i32_32x32x32_i8 (x2)  -> sumi(row, col, b) and sumi(row, col, b+1)
//   v_mfma_f32_32x32x1_2b_f32    -> dx(row, b) * dy(col, b) and the same for
//                                   b+1: two rank-1 outer products (K = 1), each
//                                   product of two fp16 values, exact in fp32
//                                   -- no per-element VALU multiply
//   VALU: acc = fma((float)sumi, dxy, acc)   -- the reference fold, in order.
// The matrix core and the VALU overlap while the VALU issue port has room, but
// at four waves per SIMD, the occupancy that issues this fold fastest, the
// MFMAs' issue shares that port and the two add up (placement-controlled
// microbenchmark: two MFMA-only and two VALU-only waves per SIMD take 0.307 ms
// against 0.317 ms for the two alone), so the loop is built to issue the
// fewest VALU instructions: 32 per tile and block, no selects or address
// arithmetic.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kFbBM = 128;                 // weight rows per work-group
constexpr int kFbBN = 128;                 // tokens per work-group
constexpr int kFbKB = 8;                   // blocks per K chunk
constexpr int kFbQRow = kFbKB * kQK + 16;  // 272: quant bytes per staged row (+16 pad: 16-byte
                                           // reads of 32 consecutive rows hit distinct banks)

// Work-group: 16 waves, each owning one 32x32 tile of a 128x128 output tile
// (four waves per SIMD hide LDS and MFMA latency; at most 128 VGPRs).  K chunks
// of 8 blocks are staged split -- each 34-byte block into its 32 quants
// (row-major, 16-byte aligned) and its scale widened to f32 -- and
// double-buffered: each thread loads its one 68-byte block pair of chunk c+1
// into registers before computing chunk c and writes it to the other LDS buffer
// afterwards.
constexpr int kOcThreads = 1024;
constexpr int kOcStage = (kFbBM + kFbBN) * kFbQRow;  // split quants of both panels

struct PairRegs {
  uint32_t r[17];
};

// Loads one staged block pair task (68 bytes, or 34 when only block 2m exists).
__device__ __forceinline__ void load_pair(PairRegs &p, const uint8_t *q, bool two) {
  const uint32_t *g = reinterpret_cast<const uint32_t *>(q);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(g + 4 * k);
    p.r[4 * k + 0] = v.x; p.r[4 * k + 1] = v.y; p.r[4 * k + 2] = v.z; p.r[4 * k + 3] = v.w;
  }
  if (two) {
#pragma unroll
    for (int k = 2; k < 4; ++k) {
      const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(g + 4 * k);
      p.r[4 * k + 0] = v.x; p.r[4 * k + 1] = v.y; p.r[4 * k + 2] = v.z; p.r[4 * k + 3] = v.w;
    }
    p.r[16] = g[16];
  } else {
    p.r[8] = *reinterpret_cast<const uint16_t *>(q + 32);
  }
}

__device__ __forceinline__ void store_pair_quants(const PairRegs &p, bool two, int8_t *qrow) {
  const uint32_t *r = p.r;
  uint4 *dst = reinterpret_cast<uint4 *>(qrow);
  dst[0] = make_uint4(funnel16(r[0], r[1]), funnel16(r[1], r[2]), funnel16(r[2], r[3]),
                      funnel16(r[3], r[4]));
  dst[1] = make_uint4(funnel16(r[4], r[5]), funnel16(r[5], r[6]), funnel16(r[6], r[7]),
                      funnel16(r[7], r[8]));
  if (two) {
    dst[2] = make_uint4(r[9], r[10], r[11], r[12]);
    dst[3] = make_uint4(r[13], r[14], r[15], r[16]);
  }
}

__device__ __forceinline__ void store_pair(const PairRegs &p, bool two, int8_t *qrow,
                                           float *d0, float *d1) {
  store_pair_quants(p, two, qrow);
  *d0 = fp16_bits_to_f32(p.r[0] & 0xffffu);
  if (two)
    *d1 = fp16_bits_to_f32(p.r[8] >> 16);
}

// The same with the scales kept as their fp16 bit patterns (the operands of
// the f16 scale MFMA below).
__device__ __forceinline__ void store_pair_h(const PairRegs &p, bool two, int8_t *qrow,
                                             uint16_t *h0, uint16_t *h1) {
  store_pair_quants(p, two, qrow);
  *h0 = static_cast<uint16_t>(p.r[0] & 0xffffu);
  if (two)
    *h1 = static_cast<uint16_t>(p.r[8] >> 16);
}

// A Q4_0 weight block pair task (36 bytes, or 18 when only block 2m exists),
// decoded into the same staged layout as a Q8_0 pair: 32 int8 quants per
// block (element j < 16 = low nibble of byte j minus 8, element 16+j = its high
// nibble minus 8) and the fp16 scale.
__device__ __forceinline__ void load_pair_q4(PairRegs &p, const uint8_t *q, bool two) {
  const uint32_t *g = reinterpret_cast<const uint32_t *>(q);
  const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(g);
  p.r[0] = v.x; p.r[1] = v.y; p.r[2] = v.z; p.r[3] = v.w;
  if (two) {
    const u32x4a4 u = *reinterpret_cast<const u32x4a4 *>(g + 4);
    p.r[4] = u.x; p.r[5] = u.y; p.r[6] = u.z; p.r[7] = u.w;
    p.r[8] = g[8];
  } else {
    p.r[4] = *reinterpret_cast<const uint16_t *>(q + 16);  // bytes 16-17: last two quant bytes
  }
}

__device__ __forceinline__ void store_q4_block(const uint32_t q[4], int8_t *dst) {
  uint4 *d = reinterpret_cast<uint4 *>(dst);
  d[0] = make_uint4(nibbles_to_i8x4(q[0]), nibbles_to_i8x4(q[1]), nibbles_to_i8x4(q[2]),
                    nibbles_to_i8x4(q[3]));
  d[1] = make_uint4(nibbles_to_i8x4(q[0] >> 4), nibbles_to_i8x4(q[1] >> 4),
                    nibbles_to_i8x4(q[2] >> 4), nibbles_to_i8x4(q[3] >> 4));
}

__device__ __forceinline__ void store_pair_q4(const PairRegs &p, bool two, int8_t *qrow,
                                              float *d0, float *d1) {
  const uint32_t *r = p.r;
  const uint32_t qa[4] = {funnel16(r[0], r[1]), funnel16(r[1], r[2]), funnel16(r[2], r[3]),
                          funnel16(r[3], r[4])};
  store_q4_block(qa, qrow);
  *d0 = fp16_bits_to_f32(r[0] & 0xffffu);
  if (two) {
    const uint32_t qb[4] = {r[5], r[6], r[7], r[8]};
    store_q4_block(qb, qrow + kQK);
    *d1 = fp16_bits_to_f32(r[4] >> 16);
  }
}

// kQ4: the weight rows (vx) are Q4_0 and every output element is the a6 block
// dot -- fold fma(fl((float)sumi * d_x), d_y, acc) (RVVToEmitCBlockQuantLinear.cpp:
// 322-356).  The f16 MFMA then carries d_x against a constant 1.0 (k-slot 0),
// which broadcasts d_x(row) into the accumulator layout exactly; d_y(col) is
// one value per lane.  Otherwise both sides are Q8_0 and the f16 MFMA is the
// outer product d_x*d_y of the a5 fold fma((float)sumi, d_x*d_y, acc).
__device__ __forceinline__ void load_task(PairRegs &p, const uint8_t *q, bool two, bool q4) {
  if (q4)
    load_pair_q4(p, q, two);
  else
    load_pair(p, q, two);
}

__device__ __forceinline__ void store_task(const PairRegs &p, bool two, bool q4, int8_t *qrow,
                                           float *d0, float *d1) {
  if (q4)
    store_pair_q4(p, two, qrow, d0, d1);
  else
    store_pair(p, two, qrow, d0, d1);
}

typedef float v32f __attribute__((ext_vector_type(32)));

// Blocks b and b+1 of the chunk for this wave's 32x32 tile (kTwo = false: block
// b alone).  The scales are staged as f32, [block][row] per panel:
//   sxh = this lane's weight-row scale of block h (h = lane / 32), so one
//         v_mfma_f32_32x32x1_2b_f32 -- lanes 0-31 are its block 0, lanes 32-63
//         its block 1 -- returns d_x*d_y of block b in dxy[0..15] and of block
//         b+1 in dxy[16..31] (each product of two fp16 values, exact in f32);
//   syh = the same for the token scale (Q8_0), or 1.0 (Q4_0: dxy = d_x);
//   syc = this lane's token-column scale of block 0 (Q4_0 fold only).
// qa/qb: this lane's 16 quant bytes of block 0 of the chunk.
template <bool kQ4, bool kTwo, int kSStride = kFbBM>
__device__ __forceinline__ void fold_pair(float (&acc)[16], const int8_t *qa, const int8_t *qb,
                                          const float *sxh, const float *syh, const float *syc,
                                          int b) {
  if constexpr (kQ4) {
    // d_x of this lane's 16 accumulator rows (rows 8g + 4h + 0..3 of the tile,
    // h = lane / 32) read straight from the staged scales: four 128-bit reads
    // per block instead of a broadcasting MFMA (the fold needs no product of
    // scales)
    const int lane = threadIdx.x & 63;
    const float *sxt = sxh - (lane >> 5) * kSStride - (lane & 31) + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < (kTwo ? 2 : 1); ++j) {
      const v4i a = *reinterpret_cast<const v4i *>(qa + (b + j) * kQK);
      const v4i bq = *reinterpret_cast<const v4i *>(qb + (b + j) * kQK);
      float dxe[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 d4 = *reinterpret_cast<const float4 *>(sxt + (b + j) * kSStride + 8 * g);
        dxe[4 * g] = d4.x; dxe[4 * g + 1] = d4.y; dxe[4 * g + 2] = d4.z; dxe[4 * g + 3] = d4.w;
      }
      const float dy = syc[(b + j) * kSStride];
      const v16i sumi = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, v16i{}, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[e] = fmaf(static_cast<float>(sumi[e]) * dxe[e], dy, acc[e]);
    }
  } else {
    const float dx = sxh[b * kSStride];
    const float dy_op = syh[b * kSStride];
    const v32f dxy = __builtin_amdgcn_mfma_f32_32x32x1f32(dx, dy_op, v32f{}, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < (kTwo ? 2 : 1); ++j) {
      const v4i a = *reinterpret_cast<const v4i *>(qa + (b + j) * kQK);
      const v4i bq = *reinterpret_cast<const v4i *>(qb + (b + j) * kQK);
      const v16i sumi = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, v16i{}, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[e] = fmaf(static_cast<float>(sumi[e]), dxy[16 * j + e], acc[e]);
    }
  }
}

template <bool kQ4>
__global__ __launch_bounds__(kOcThreads, 1) void gemm_occ(
    size_t nb, float *s, const uint8_t *vx, const uint8_t *vy, size_t by, size_t nr,
    size_t nc, size_t bx, size_t bs) {
  __shared__ __align__(16) int8_t q[2][kOcStage];
  __shared__ __align__(16) float dsc[2][2][kFbKB][kFbBM];  // [stage][panel][block][row]

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 2, wn = wave & 3;  // 4 x 4 waves, one 32x32 tile each
  const int li = lane & 31, h = lane >> 5;
  const unsigned tiles_m = static_cast<unsigned>((nr + kFbBM - 1) / kFbBM);
  const unsigned tiles_n = static_cast<unsigned>((nc + kFbBN - 1) / kFbBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const size_t m0 = static_cast<size_t>(tm) * kFbBM;
  const size_t n0 = static_cast<size_t>(tn) * kFbBN;

  // staging task of this thread: panel p (0 = weights, 1 = tokens), row r, pair m
  const int sp = tid >> 9;
  const int sr = (tid & 511) >> 2, sm = tid & 3;
  const uint8_t *sbase = sp == 0 ? vx + min(m0 + sr, nr - 1) * bx : vy + min(n0 + sr, nc - 1) * by;
  const bool q4_task = kQ4 && sp == 0;  // wave-uniform: waves 0-7 stage weights
  const int sblk = q4_task ? kQ4Bytes : kQ8Bytes;

  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e)
    acc[e] = 0.0f;

  const size_t nchunks = (nb + kFbKB - 1) / kFbKB;
  PairRegs pr;
  auto chunk_task = [&](size_t c, bool &active, bool &two) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kFbKB), nb - c * kFbKB));
    active = 2 * sm < nbc;
    two = 2 * sm + 1 < nbc;
  };
  bool act, two;
  chunk_task(0, act, two);
  if (act)
    load_task(pr, sbase + 2 * sm * sblk, two, q4_task);
  if (act)
    store_task(pr, two, q4_task, q[0] + (sp * kFbBM + sr) * kFbQRow + 64 * sm,
               &dsc[0][sp][2 * sm][sr], &dsc[0][sp][2 * sm + 1][sr]);
  __syncthreads();

  // this lane's operand addresses in stage 0 (stage 1 is a fixed offset away)
  const int8_t *qa0 = q[0] + (wm * 32 + li) * kFbQRow + 16 * h;
  const int8_t *qb0 = q[0] + (kFbBM + wn * 32 + li) * kFbQRow + 16 * h;
  const float *sxh0 = &dsc[0][0][h][wm * 32 + li];
  const float *syh0 = &dsc[0][1][h][wn * 32 + li];
  const float *syc0 = &dsc[0][1][0][wn * 32 + li];
  constexpr int kDscStage = 2 * kFbKB * kFbBM;

  // Full chunks: the next chunk's loads are in flight while this one is
  // folded; a trailing partial chunk (nb % kFbKB blocks) is folded after the
  // loop, so the loop body has a single path.
  const size_t nfull = nb / kFbKB;
  for (size_t c = 0; c < nfull; ++c) {
    const int st = static_cast<int>(c & 1);
    bool act1 = false, two1 = false;
    if (c + 1 < nchunks) {
      chunk_task(c + 1, act1, two1);
      if (act1)
        load_task(pr, sbase + ((c + 1) * kFbKB + 2 * sm) * sblk, two1, q4_task);
    }
    const int8_t *qa = qa0 + st * kOcStage;
    const int8_t *qb = qb0 + st * kOcStage;
    const float *sxh = sxh0 + st * kDscStage;
    const float *syh = syh0 + st * kDscStage;
    const float *syc = syc0 + st * kDscStage;
#pragma unroll
    for (int b = 0; b < kFbKB; b += 2) {
      fold_pair<kQ4, true>(acc, qa, qb, sxh, syh, syc, b);
      // one block pair at a time (the folded accumulators are pinned here and
      // nothing is scheduled across): keeps the live registers within the 128
      // that four waves per SIMD allow
#pragma unroll
      for (int e = 0; e < 16; ++e)
        asm volatile("" : "+v"(acc[e]));
      __builtin_amdgcn_sched_barrier(0);
    }
    if (act1)
      store_task(pr, two1, q4_task, q[st ^ 1] + (sp * kFbBM + sr) * kFbQRow + 64 * sm,
                 &dsc[st ^ 1][sp][2 * sm][sr], &dsc[st ^ 1][sp][2 * sm + 1][sr]);
    __syncthreads();
  }
  const int nbc = static_cast<int>(nb - nfull * kFbKB);
  if (nbc > 0) {
    const int st = static_cast<int>(nfull & 1);
    const int8_t *qa = qa0 + st * kOcStage;
    const int8_t *qb = qb0 + st * kOcStage;
    const float *sxh = sxh0 + st * kDscStage;
    const float *syh = syh0 + st * kDscStage;
    const float *syc = syc0 + st * kDscStage;
    // nbc < kFbKB, so the 2-block scale read of a last odd block stays inside
    // the stage (its second block is not used)
    int b = 0;
    for (; b + 1 < nbc; b += 2)
      fold_pair<kQ4, true>(acc, qa, qb, sxh, syh, syc, b);
    if (b < nbc)
      fold_pair<kQ4, false>(acc, qa, qb, sxh, syh, syc, b);
  }

  const size_t col = n0 + wn * 32 + li;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const size_t row = m0 + wm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
    if (row < nr && col < nc)
      s[row * bs + col] = acc[e];
  }
}

// Wide tile: 256 weight rows x 128 tokens per work-group, 16 waves, each wave
// two 32x32 tiles stacked in M (64 weight rows x 32 tokens), so every staged
// token row serves twice as many tiles as in gemm_occ; K chunks of 4 blocks,
// double-buffered (384 staged rows of 8 blocks would not fit twice).
constexpr int kWBM = 256, kWBN = 128, kWKB = 4;
constexpr int kWQRow = kWKB * kQK + 16;           // 144: quant bytes per staged row (+16 pad)
constexpr int kWRows = kWBM + kWBN;               // 384 staged rows per chunk
constexpr int kWStage = kWRows * kWQRow;
constexpr int kWTasks = kWRows * (kWKB / 2);      // 768 block-pair tasks per chunk

// ---------------------------------------------------------------------------
// The Q8_0 fold of the wide tile, software-pipelined.  Per 32x32 tile and block:
//   v_mfma_i32_32x32x32_i8  -> sumi(row, col) (exact int32 block sums)
//   v_mfma_f32_32x32x8_f16  -> d_x(row) * d_y(col): k-slot 0 carries the two
//                              fp16 scales, every other k-slot is zero, so each
//                              output is one product of two fp16 values, exact
//                              in fp32 (32 matrix cycles, measured: per block
//                              what the 2-block f32 outer product costs, with
//                              no VALU to build its operands)
//   VALU: acc = fma((float)sumi, dxy, acc) -- the reference fold, in order.
// The MFMAs of step s+1 (tile, block) are issued before the fold of step s, so
// the matrix core works while the VALU folds (on this part one wave issues a
// VALU instruction about every 6 cycles; the matrix core fills the gaps).
// Scales are staged as fp16 bit patterns, [stage][block][row], with 32 zero
// rows after the 384 panel rows: lanes 32-63 (k-slots 4-7 of the f16 MFMA)
// point there, so building an operand costs one 16-bit LDS read and no VALU.
// ---------------------------------------------------------------------------
constexpr int kHRow = kWRows + 32;     // fp16 scales per block row (+32 zero rows)
constexpr int kHStage = kWKB * kHRow;  // per stage
#ifndef TCRV_GEMM_Q8_PIPE
#define TCRV_GEMM_Q8_PIPE 0
#endif
constexpr bool kGemmQ8Pipe = TCRV_GEMM_Q8_PIPE;
// the step after which a wave stores its staged part of the next chunk (a
// sweep over steps 1, 3, 5 and 7 measured within run-to-run noise)
constexpr int kGemmStageStep = 2 * kWKB - 1;

template <bool kQ4>
__global__ __launch_bounds__(kOcThreads, 1) void gemm_wide(
    size_t nb, float *s, const uint8_t *vx, const uint8_t *vy, size_t by, size_t nr,
    size_t nc, size_t bx, size_t bs) {
  __shared__ __align__(16) int8_t q[2][kWStage];
  // scales: f32 [stage][block][row] for the Q4_0 fold, fp16 bit patterns with
  // 32 zero rows for the Q8_0 fold (only the one the instantiation uses is
  // allocated)
  __shared__ __align__(16) float dsc[2][kWKB][kWRows];
  __shared__ __align__(16) uint16_t dsh[2][kWKB][kHRow];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 2, wn = wave & 3;  // 64 weight rows x 32 tokens per wave
  const int li = lane & 31, h = lane >> 5;
  const unsigned tiles_m = static_cast<unsigned>((nr + kWBM - 1) / kWBM);
  const unsigned tiles_n = static_cast<unsigned>((nc + kWBN - 1) / kWBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const size_t m0 = static_cast<size_t>(tm) * kWBM;
  const size_t n0 = static_cast<size_t>(tn) * kWBN;

  // staging task: thread t < 768 stages row t/2 (weights 0..255, tokens
  // 256..383), block pair t%2 of the chunk; waves 12-15 stage nothing
  const bool stager = tid < kWTasks;
  const int sr = min(tid >> 1, kWRows - 1), sm = tid & 1;
  const bool wrow = sr < kWBM;
  const uint8_t *sbase = wrow ? vx + min(m0 + sr, nr - 1) * bx
                              : vy + min(n0 + (sr - kWBM), nc - 1) * by;
  const bool q4_task = kQ4 && wrow;  // wave-uniform: waves 0-7 stage weights
  const int sblk = q4_task ? kQ4Bytes : kQ8Bytes;

  float acc[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[i][e] = 0.0f;

  const size_t nchunks = (nb + kWKB - 1) / kWKB;
  PairRegs pr;
  auto chunk_task = [&](size_t c, bool &active, bool &two) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kWKB), nb - c * kWKB));
    active = stager && 2 * sm < nbc;
    two = 2 * sm + 1 < nbc;
  };
  auto stage = [&](int st, bool two) {
    if constexpr (kQ4)
      store_task(pr, two, q4_task, q[st] + sr * kWQRow + 64 * sm, &dsc[st][2 * sm][sr],
                 &dsc[st][2 * sm + 1][sr]);
    else
      store_pair_h(pr, two, q[st] + sr * kWQRow + 64 * sm, &dsh[st][2 * sm][sr],
                   &dsh[st][2 * sm + 1][sr]);
  };
  if constexpr (!kQ4) {
    if (tid < 2 * kWKB * 32)  // the zero rows of both stages
      dsh[tid >> 7][(tid >> 5) & 3][kWRows + (tid & 31)] = 0;
  }
  bool act, two;
  chunk_task(0, act, two);
  if (act)
    load_task(pr, sbase + 2 * sm * sblk, two, q4_task);
  if (act)
    stage(0, two);
  __syncthreads();

  // this lane's operand addresses in stage 0 for the wave's first tile (the
  // second tile and stage 1 are fixed offsets away)
  const int8_t *qa0 = q[0] + (wm * 64 + li) * kWQRow + 16 * h;
  const int8_t *qb0 = q[0] + (kWBM + wn * 32 + li) * kWQRow + 16 * h;
  const float *sxh0 = &dsc[0][h][wm * 64 + li];
  const float *syh0 = &dsc[0][h][kWBM + wn * 32 + li];
  const float *syc0 = &dsc[0][0][kWBM + wn * 32 + li];
  constexpr int kDscStage = kWKB * kWRows;
  const uint16_t *hx0 = h ? &dsh[0][0][kWRows + li] : &dsh[0][0][wm * 64 + li];
  const uint16_t *hx1 = h ? &dsh[0][0][kWRows + li] : &dsh[0][0][wm * 64 + 32 + li];
  const uint16_t *hy = h ? &dsh[0][0][kWRows + li] : &dsh[0][0][kWBM + wn * 32 + li];

  const size_t nfull = nb / kWKB;
  for (size_t c = 0; c < nfull; ++c) {
    const int st = static_cast<int>(c & 1);
    bool act1 = false, two1 = false;
    if (c + 1 < nchunks) {
      chunk_task(c + 1, act1, two1);
      if (act1)
        load_task(pr, sbase + ((c + 1) * kWKB + 2 * sm) * sblk, two1, q4_task);
    }
    if constexpr (kQ4) {
#pragma unroll
      for (int b = 0; b < kWKB; b += 2) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          fold_pair<kQ4, true, kWRows>(acc[i], qa0 + i * 32 * kWQRow + st * kWStage,
                                       qb0 + st * kWStage, sxh0 + i * 32 + st * kDscStage,
                                       syh0 + st * kDscStage, syc0 + st * kDscStage, b);
#pragma unroll
          for (int e = 0; e < 16; ++e)
            asm volatile("" : "+v"(acc[i][e]));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
      fold_chunk_q8<kGemmQ8Pipe, kWKB, kQK, 32 * kWQRow, kHRow>(
          acc, qa0 + st * kWStage, qb0 + st * kWStage, hx0 + st * kHStage, hx1 + st * kHStage,
          hy + st * kHStage, [&](int step) {
            if (step == kGemmStageStep && act1)
              stage(st ^ 1, two1);
          });
    }
    if constexpr (kQ4) {
      if (act1)
        stage(st ^ 1, two1);
    }
    __syncthreads();
  }
  const int nbc = static_cast<int>(nb - nfull * kWKB);
  if (nbc > 0) {
    const int st = static_cast<int>(nfull & 1);
    if constexpr (kQ4) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int8_t *qa = qa0 + i * 32 * kWQRow + st * kWStage;
        const int8_t *qb = qb0 + st * kWStage;
        const float *sxh = sxh0 + i * 32 + st * kDscStage;
        const float *syh = syh0 + st * kDscStage;
        const float *syc = syc0 + st * kDscStage;
        int b = 0;
        for (; b + 1 < nbc; b += 2)
          fold_pair<kQ4, true, kWRows>(acc[i], qa, qb, sxh, syh, syc, b);
        if (b < nbc)
          fold_pair<kQ4, false, kWRows>(acc[i], qa, qb, sxh, syh, syc, b);
      }
    } else {
      fold_tail_q8<kQK, 32 * kWQRow, kHRow>(acc, qa0 + st * kWStage, qb0 + st * kWStage,
                                            hx0 + st * kHStage, hx1 + st * kHStage,
                                            hy + st * kHStage, nbc);
    }
  }

  const size_t col = n0 + wn * 32 + li;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const size_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
      if (row < nr && col < nc)
        s[row * bs + col] = acc[i][e];
    }
}

// ---------------------------------------------------------------------------
// Repack GEMM (tcrv_rvv.repack_gemm_q4_0_q8_0, RVVOps.td:4228-4338; emitter
// RVVToEmitCBlockQuantLinear.cpp:2122-2600): x16-interleaved Q4_0 weights
// (block_q4_0x16, 288 B: 16 rows per group, nibble bytes biased ^0x88) times
// 4-row-interleaved Q8_0 activations (block_q8_0x4, 136 B: fp16 d[4] @0, quant
// e of row c at 8 + 4e + c), output s[token*bs + weight_row].  Per element and
// block: exact int32 sum, then acc = fma((float)sumi, d_w*d_a, acc) -- the
// x16 fold, the same as the Q8_0 fold -- in ascending block order.
// The kernel is gemm_wide<false>'s pipeline with another staging: each chunk's
// x16 and x4 blocks are turned into the row-major staged layout (int8 quants of
// a row at kWQRow stride, f32 scales [block][row]) with 4x4 byte transposes, so
// the MFMA tiles and the fold are unchanged.  Staging tasks per 4-block chunk:
// 256 weight tasks (x16 group, block, position quad: four 128-bit loads, 16
// rows x 4 positions) on waves 0-3 and 256 activation tasks (x4 group, block,
// half: four 128-bit loads, 4 rows x 16 elements) on waves 4-7.
// ---------------------------------------------------------------------------
constexpr int kQ4x16 = 288, kQ8x4 = 136;

struct RgRegs {
  uint32_t r[18];
};

// A staging task's 64 quant bytes (four 128-bit loads, 4-byte aligned) and 8
// scale bytes.  Weight task (x16 block, position quad q): positions 4q..4q+3,
// 16 rows each, and the scales of rows 4q..4q+3.  Activation task (x4 block,
// half hf): elements 16hf..16hf+15 (dword e: element e of rows 0..3) and the 4
// scales.
__device__ __forceinline__ void rg_load(RgRegs &p, const uint8_t *quant, const uint8_t *scale) {
  const u32x4a4 *src = reinterpret_cast<const u32x4a4 *>(quant);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const u32x4a4 v = src[m];
    p.r[4 * m] = v.x; p.r[4 * m + 1] = v.y; p.r[4 * m + 2] = v.z; p.r[4 * m + 3] = v.w;
  }
  const uint32_t *d = reinterpret_cast<const uint32_t *>(scale);
  p.r[16] = d[0];
  p.r[17] = d[1];
}

// -> rows 16g + 0..15, quants 32j + 4q.. (low nibbles) and 32j + 16 + 4q..
// (high nibbles) as int8, fp16 scales dsh_j[16g + 4q .. +3]
__device__ __forceinline__ void rg_store_w(const RgRegs &p, int8_t *stage, uint16_t *dsh_j, int g,
                                           int j, int q) {
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
    const uint32_t in[4] = {p.r[rq], p.r[4 + rq], p.r[8 + rq], p.r[12 + rq]};
    uint32_t rows[4];
    transpose4x4(in, rows);  // rows[rr]: positions 4q..4q+3 of row 4rq + rr
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const uint32_t raw = rows[rr] ^ 0x88888888u;  // the plain Q4_0 quant bytes
      int8_t *dst = stage + (16 * g + 4 * rq + rr) * kWQRow + kQK * j + 4 * q;
      *reinterpret_cast<uint32_t *>(dst) = nibbles_to_i8x4(raw);
      *reinterpret_cast<uint32_t *>(dst + 16) = nibbles_to_i8x4(raw >> 4);
    }
  }
  *reinterpret_cast<uint2 *>(dsh_j + 16 * g + 4 * q) = make_uint2(p.r[16], p.r[17]);
}

// -> rows kWBM + 4t + 0..3, quants 32j + 16hf + 0..15, fp16 scales dsh_j[kWBM + 4t ..]
__device__ __forceinline__ void rg_store_a(const RgRegs &p, int8_t *stage, uint16_t *dsh_j, int t,
                                           int j, int hf) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    uint32_t rows[4];
    transpose4x4(&p.r[4 * m], rows);  // rows[c]: elements 16hf + 4m .. +3 of row c
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<uint32_t *>(stage + (kWBM + 4 * t + c) * kWQRow + kQK * j + 16 * hf +
                                    4 * m) = rows[c];
  }
  if (hf == 0)
    *reinterpret_cast<uint2 *>(dsh_j + kWBM + 4 * t) = make_uint2(p.r[16], p.r[17]);
}

__global__ __launch_bounds__(kOcThreads, 1) void gemm_repack_q4_0(
    size_t nb, float *s, const uint8_t *vx, const uint8_t *vy, size_t ngw, size_t nga,
    size_t bs, bool vec_out) {
  __shared__ __align__(16) int8_t q[2][kWStage];
  __shared__ __align__(16) uint16_t dsh[2][kWKB][kHRow];  // fp16 scales + 32 zero rows

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 2, wn = wave & 3;  // 64 weight rows x 32 tokens per wave
  const int li = lane & 31, h = lane >> 5;
  const size_t nrw = ngw * 16, ntok = nga * 4;  // rows and tokens written
  const unsigned tiles_m = static_cast<unsigned>((nrw + kWBM - 1) / kWBM);
  const unsigned tiles_n = static_cast<unsigned>((ntok + kWBN - 1) / kWBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const size_t m0 = static_cast<size_t>(tm) * kWBM;
  const size_t n0 = static_cast<size_t>(tn) * kWBN;

  // staging task of this thread: waves 0-3 weights, 4-7 activations, 8-15
  // none (the kind is wave-uniform: taken from the first lane)
  const int swave = __builtin_amdgcn_readfirstlane(wave);
  const bool wtask = swave < 4, atask = swave >= 4 && swave < 8;
  const int k = tid & 255;
  const int sg = wtask ? k >> 4 : k >> 3;              // x16 group / x4 group in the tile
  const int sj = wtask ? (k >> 2) & 3 : (k >> 1) & 3;  // block of the chunk
  const int sq = wtask ? k & 3 : k & 1;                // position quad / half
  const int sblk = wtask ? kQ4x16 : kQ8x4;
  const uint8_t *sblk0 = (wtask ? vx + min(m0 / 16 + sg, ngw - 1) * nb * kQ4x16
                                : vy + min(n0 / 4 + sg, nga - 1) * nb * kQ8x4) + sj * sblk;
  // this task's quant bytes and scale dwords in block sj of chunk 0
  const uint8_t *squant = sblk0 + (wtask ? 32 + 64 * sq : 8 + 64 * sq);
  const uint8_t *sscale = sblk0 + (wtask ? 8 * sq : 0);
  const size_t cstride = static_cast<size_t>(kWKB) * sblk;  // bytes per chunk

  float acc[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[i][e] = 0.0f;

  const size_t nchunks = (nb + kWKB - 1) / kWKB;
  RgRegs pr;
  if (tid < 2 * kWKB * 32)  // the zero rows of both stages
    dsh[tid >> 7][(tid >> 5) & 3][kWRows + (tid & 31)] = 0;
  if ((wtask || atask) && sj < static_cast<int>(min(static_cast<size_t>(kWKB), nb))) {
    rg_load(pr, squant, sscale);
    if (wtask)
      rg_store_w(pr, q[0], dsh[0][sj], sg, sj, sq);
    else
      rg_store_a(pr, q[0], dsh[0][sj], sg, sj, sq);
  }
  __syncthreads();

  const int8_t *qa0 = q[0] + (wm * 64 + li) * kWQRow + 16 * h;
  const int8_t *qb0 = q[0] + (kWBM + wn * 32 + li) * kWQRow + 16 * h;
  const uint16_t *hx0 = h ? &dsh[0][0][kWRows + li] : &dsh[0][0][wm * 64 + li];
  const uint16_t *hx1 = h ? &dsh[0][0][kWRows + li] : &dsh[0][0][wm * 64 + 32 + li];
  const uint16_t *hy = h ? &dsh[0][0][kWRows + li] : &dsh[0][0][kWBM + wn * 32 + li];

  const size_t nfull = nb / kWKB;
  for (size_t c = 0; c < nfull; ++c) {
    const int st = static_cast<int>(c & 1);
    const bool act1 = (wtask || atask) && c + 1 < nchunks &&
                      static_cast<size_t>(sj) < min(static_cast<size_t>(kWKB), nb - (c + 1) * kWKB);
    if (act1)
      rg_load(pr, squant + (c + 1) * cstride, sscale + (c + 1) * cstride);
    fold_chunk_q8<kGemmQ8Pipe, kWKB, kQK, 32 * kWQRow, kHRow>(
        acc, qa0 + st * kWStage, qb0 + st * kWStage, hx0 + st * kHStage, hx1 + st * kHStage,
        hy + st * kHStage, [&](int step) {
          if (step == kGemmStageStep && act1) {
            if (wtask)
              rg_store_w(pr, q[st ^ 1], dsh[st ^ 1][sj], sg, sj, sq);
            else
              rg_store_a(pr, q[st ^ 1], dsh[st ^ 1][sj], sg, sj, sq);
          }
        });
    __syncthreads();
  }
  const int nbc = static_cast<int>(nb - nfull * kWKB);
  if (nbc > 0) {
    const int st = static_cast<int>(nfull & 1);
    fold_tail_q8<kQK, 32 * kWQRow, kHRow>(acc, qa0 + st * kWStage, qb0 + st * kWStage,
                                          hx0 + st * kHStage, hx1 + st * kHStage,
                                          hy + st * kHStage, nbc);
  }

  // a lane holds 4 consecutive weight rows per group of 4 elements: one
  // 128-bit store each when the output allows (nrw is a multiple of 16, so a
  // group is written whole or not at all)
  const size_t tok = n0 + wn * 32 + li;
  if (tok < ntok) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const size_t row = m0 + wm * 64 + i * 32 + 8 * g + 4 * h;
        if (row >= nrw)
          continue;
        float *d = s + tok * bs + row;
        if (vec_out) {
          *reinterpret_cast<float4 *>(d) =
              make_float4(acc[i][4 * g], acc[i][4 * g + 1], acc[i][4 * g + 2], acc[i][4 * g + 3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            d[e] = acc[i][4 * g + e];
        }
      }
  }
}

// Plain Q8_0 rows (stride by), groups of 4, -> block_q8_0x4: thread per output
// dword (2 scale dwords + 32 quant dwords, dword 2 + e = element e of rows 0..3).
__global__ __launch_bounds__(256) void pack_q8_0x4(size_t ngroups, size_t nb, const uint8_t *src,
                                                   size_t by, uint8_t *dst) {
  const size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= ngroups * nb * (kQ8x4 / 4))
    return;
  const size_t o = t / (kQ8x4 / 4);
  const int k = static_cast<int>(t - o * (kQ8x4 / 4));
  const size_t y = o / nb, b = o - y * nb;
  const uint8_t *row0 = src + (y * 4) * by + b * kQ8Bytes;
  uint32_t v;
  if (k < 2) {  // scales of rows 2k, 2k+1
    v = static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(row0 + (2 * k) * by)) |
        (static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(row0 + (2 * k + 1) * by))
         << 16);
  } else {
    const int e = k - 2;
    v = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      v |= static_cast<uint32_t>(row0[c * by + 2 + e]) << (8 * c);
  }
  reinterpret_cast<uint32_t *>(dst + o * kQ8x4)[k] = v;
}
}  // namespace tcrv

namespace tcrv_host {

// Q4_0 x Q8_0 GEMM (nc > 1) on the MFMA kernel; returns TCRV_HIP_ERR_UNSUPPORTED
// when the rows are not 4-byte aligned (the caller then uses the block-dot grid).
int q4_0_gemm_mfma(size_t nb, float *s, const uint8_t *vx, size_t bx, const uint8_t *vy,
                   size_t by, size_t nr, size_t nc, size_t bs, void *stream) {
  if (!(aligned4(vx) && aligned4(vy) && (nr == 1 || bx % 4 == 0) && (nc == 1 || by % 4 == 0)))
    return TCRV_HIP_ERR_UNSUPPORTED;
  const size_t tiles =
      ((nr + tcrv::kFbBM - 1) / tcrv::kFbBM) * ((nc + tcrv::kFbBN - 1) / tcrv::kFbBN);
  if (tiles > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (nr >= static_cast<size_t>(tcrv::kWBM)) {  // at least one full wide tile of weight rows
    const size_t wtiles =
        ((nr + tcrv::kWBM - 1) / tcrv::kWBM) * ((nc + tcrv::kWBN - 1) / tcrv::kWBN);
    tcrv::gemm_wide<true><<<dim3(static_cast<unsigned>(wtiles)), dim3(tcrv::kOcThreads), 0,
                            as_stream(stream)>>>(nb, s, vx, vy, by, nr, nc, bx, bs);
    return launch_status();
  }
  tcrv::gemm_occ<true><<<dim3(static_cast<unsigned>(tiles)), dim3(tcrv::kOcThreads), 0,
                         as_stream(stream)>>>(nb, s, vx, vy, by, nr, nc, bx, bs);
  return launch_status();
}

}  // namespace tcrv_host

extern "C" int tcrv_hip_q8_0_q8_0_gemm(size_t n, float *s, const uint8_t *vx,
                                       const uint8_t *vy, size_t by, size_t nr, size_t nc,
                                       size_t bx, size_t bs, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / tcrv::kQK;
  if (nr == 0 || nc == 0)
    return TCRV_HIP_OK;
  if (nr > 1 && bs < nc)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (nb == 0)
    return zero_outputs(s, nr * nc, bs, nc, stream);
  if (!s || !vx || !vy)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(vx) || !aligned2(vy) || (nr > 1 && (bx & 1u)) || (nc > 1 && (by & 1u)))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t rowbytes = nb * tcrv::kQ8Bytes;
  if ((nr > 1 && bx < rowbytes) || (nc > 1 && by < rowbytes))
    return TCRV_HIP_ERR_BAD_SIZE;
  if (nc == 1 || nr == 1) {  // one operand is a single row: bandwidth-bound block dots
    const int st = nc == 1 ? q8_0_rows_direct(nb, s, nr > 1 ? bs : 0, vx, nr > 1 ? bx : 0, vy,
                                              0, nr, stream)
                           : q8_0_rows_direct(nb, s, 1, vx, 0, vy, by, nc, stream);
    if (st != TCRV_HIP_ERR_UNSUPPORTED)
      return st;
  } else {
    if (!cols_first(nr, nc)) {  // few output tiles: one 32 x 32 tile a wave
      const int st = gemm_rows_few(false, nb, s, vx, bx, vy, by, nr, nc, bs, stream);
      if (st != TCRV_HIP_ERR_UNSUPPORTED)
        return st;
    }
    if (nc <= kGemvColsMax) {  // a few tokens: multi-column GEMVs
      const int st = gemv_cols_q8_0_q8_0(nb, s, bs, vx, bx, vy, by, nr, nc, stream);
      if (st != TCRV_HIP_ERR_UNSUPPORTED)
        return st;
    }
  }
  if (aligned4(vx) && aligned4(vy) && (nr == 1 || bx % 4 == 0) && (nc == 1 || by % 4 == 0)) {
    const size_t tiles =
        ((nr + tcrv::kFbBM - 1) / tcrv::kFbBM) * ((nc + tcrv::kFbBN - 1) / tcrv::kFbBN);
    if (tiles > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    if (nr >= static_cast<size_t>(tcrv::kWBM)) {  // at least one full wide tile of weight rows
      const size_t wtiles =
          ((nr + tcrv::kWBM - 1) / tcrv::kWBM) * ((nc + tcrv::kWBN - 1) / tcrv::kWBN);
      tcrv::gemm_wide<false><<<dim3(static_cast<unsigned>(wtiles)), dim3(tcrv::kOcThreads), 0,
                               as_stream(stream)>>>(nb, s, vx, vy, by, nr, nc, bx, bs);
      return launch_status();
    }
    tcrv::gemm_occ<false><<<dim3(static_cast<unsigned>(tiles)), dim3(tcrv::kOcThreads), 0,
                            as_stream(stream)>>>(nb, s, vx, vy, by, nr, nc, bx, bs);
    return launch_status();
  }
  const int rows16 = aligned16(vx) && aligned16(vy) && (nr == 1 || bx % 16 == 0) &&
                     (nc == 1 || by % 16 == 0);
  const size_t gx = (nc + tcrv::kGmBN - 1) / tcrv::kGmBN;
  const size_t gy = (nr + tcrv::kGmBM - 1) / tcrv::kGmBM;
  if (gx > 0x7fffffffu || gy > 65535u)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::gemm_q8_0_q8_0_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                                dim3(tcrv::kGmThreads), 0, as_stream(stream)>>>(
      nb, s, vx, vy, by, nr, nc, bx, bs, rows16);
  return launch_status();
}

extern "C" int tcrv_hip_repack_gemm_q4_0_q8_0(size_t n, float *s, const uint8_t *vx,
                                              const uint8_t *vy, size_t nr, size_t nc,
                                              size_t bs, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / tcrv::kQK;
  const size_t nga = nr / 4, ngw = nc / 16;  // like the reference, partial groups are not written
  if (nga == 0 || ngw == 0)
    return TCRV_HIP_OK;
  if (bs < ngw * 16)  // every group writes 4 activation rows at stride bs
    return TCRV_HIP_ERR_BAD_SIZE;
  if (nb == 0)
    return zero_outputs(s, nga * 4 * ngw * 16, bs, ngw * 16, stream);
  if (!s || !vx || !vy)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned4(vx) || !aligned4(vy) || !aligned4(s))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t tiles = ((ngw * 16 + tcrv::kWBM - 1) / tcrv::kWBM) *
                       ((nga * 4 + tcrv::kWBN - 1) / tcrv::kWBN);
  if (tiles > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::gemm_repack_q4_0<<<dim3(static_cast<unsigned>(tiles)), dim3(tcrv::kOcThreads), 0,
                           as_stream(stream)>>>(nb, s, vx, vy, ngw, nga, bs,
                                                aligned16(s) && bs % 4 == 0);
  return launch_status();
}

extern "C" int tcrv_hip_pack_q8_0_to_q8_0x4(size_t nrows, size_t nb, const uint8_t *src,
                                            size_t by, uint8_t *dst, void *stream) {
  using namespace tcrv_host;
  const size_t ngroups = nrows / 4;
  if (ngroups == 0 || nb == 0)
    return TCRV_HIP_OK;
  if (!src || !dst)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(src) || (by & 1u) || !aligned4(dst))
    return TCRV_HIP_ERR_MISALIGNED;
  if (by < nb * tcrv::kQ8Bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  const size_t grid = (ngroups * nb * (tcrv::kQ8x4 / 4) + 255) / 256;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::pack_q8_0x4<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, as_stream(stream)>>>(
      ngroups, nb, src, by, dst);
  return launch_status();
}
