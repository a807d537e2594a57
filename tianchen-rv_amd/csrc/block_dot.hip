// block_dot.hip -- the ggml block dots of libtcrv_hip:
//   a4  packed-i4 offset-binary x i8 integer core (Q4_0 . Q8_0 per block)
//   a5  tcrv_rvv.q8_0_q8_0_block_dot  (ggml_vec_dot_q8_0_q8_0)
//   a6  tcrv_rvv.q4_0_q8_0_block_dot  (ggml_vec_dot_q4_0_q8_0)
// as one wavefront per (x row, y row) pair, plus the per-block int32 sums.
//
// Per pair, the wave stages up to 128 blocks of each row through LDS with
// 128-bit loads, lane l computes the integer sums of blocks 2l and 2l+1
// (v_dot4_i32_i8), and the fp32 fold runs serially in ascending block order
// exactly as the reference emits it:
//   Q8_0: sumf = fma((float)sumi, d_x*d_y, sumf)
//         (lib/Conversion/RVV/RVVToEmitCBlockQuantLinear.cpp:7538-7575)
//   Q4_0: sumf = fma(fl((float)sumi*d_x), d_y, sumf)   (same file, :322-356)
// The kernels are built with -ffp-contract=off and use explicit fmaf, so the
// compiler cannot re-associate or re-fuse either fold.
#include "tcrv_hip_internal.h"

namespace tcrv {

enum class DotFmt { kQ8Q8, kQ4Q8 };

constexpr int kChunkBlocks = 128;  // blocks per LDS chunk: 128*34 = 4352 B (16-B multiple)

// One Q8_0 block at block index b of an LDS chunk, read as 9 aligned dwords.
// Even b starts on a dword (34*b % 4 == 0): the quants sit 2 bytes into the
// dword run.  Odd b starts 2 bytes into a dword: the quants are dword aligned.
template <int kParity>
__device__ __forceinline__ void read_q8_block(const uint8_t *chunk, int b, uint32_t q[8],
                                              uint32_t &d_bits) {
  const uint32_t *w = reinterpret_cast<const uint32_t *>(chunk) + ((b * kQ8Bytes) >> 2);
  uint32_t r[9];
#pragma unroll
  for (int k = 0; k < 9; ++k)
    r[k] = w[k];
  if constexpr (kParity == 0) {
    d_bits = r[0] & 0xffffu;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      q[k] = funnel16(r[k], r[k + 1]);
  } else {
    d_bits = r[0] >> 16;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      q[k] = r[k + 1];
  }
}

// One Q4_0 block (18 B) at block index b of an LDS chunk, read as 5 dwords.
template <int kParity>
__device__ __forceinline__ void read_q4_block(const uint8_t *chunk, int b, uint32_t q[4],
                                              uint32_t &d_bits) {
  const uint32_t *w = reinterpret_cast<const uint32_t *>(chunk) + ((b * kQ4Bytes) >> 2);
  uint32_t r[5];
#pragma unroll
  for (int k = 0; k < 5; ++k)
    r[k] = w[k];
  if constexpr (kParity == 0) {
    d_bits = r[0] & 0xffffu;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      q[k] = funnel16(r[k], r[k + 1]);
  } else {
    d_bits = r[0] >> 16;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      q[k] = r[k + 1];
  }
}

// a5 integer core: sum of the 32 int8 products (order-free, exact).
__device__ __forceinline__ int q8_q8_sumi(const uint32_t qx[8], const uint32_t qy[8]) {
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    acc = sdot4(qx[k], qy[k], acc);
  return acc;
}

// a4 integer core: byte j of the Q4_0 quants holds element j (low nibble) and
// element j+16 (high nibble), each offset-binary (value = nibble - 8); they
// pair with Q8_0 quants j and j+16 (RVVToEmitC.cpp:2524-2589).
__device__ __forceinline__ int q4_q8_sumi(const uint32_t qx[4], const uint32_t qy[8]) {
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    acc = sdot4(nibbles_to_i8x4(qx[k]), qy[k], acc);
    acc = sdot4(nibbles_to_i8x4(qx[k] >> 4), qy[k + 4], acc);
  }
  return acc;
}

// Integer sum + fold operands of block b for this lane.  The fold is
// fmaf(t.x, t.y, sumf) for both formats:
//   Q8_0: t = { (float)sumi, d_x*d_y }   (d_x*d_y is exact: two 11-bit significands)
//   Q4_0: t = { fl((float)sumi*d_x), d_y }
template <DotFmt F, int kParity>
__device__ __forceinline__ float2 block_terms(const uint8_t *xc, const uint8_t *yc, int b,
                                              int &sumi) {
  uint32_t qy[8], dy_bits;
  read_q8_block<kParity>(yc, b, qy, dy_bits);
  const float dy = fp16_bits_to_f32(dy_bits);
  if constexpr (F == DotFmt::kQ8Q8) {
    uint32_t qx[8], dx_bits;
    read_q8_block<kParity>(xc, b, qx, dx_bits);
    sumi = q8_q8_sumi(qx, qy);
    const float dx = fp16_bits_to_f32(dx_bits);
    return make_float2(static_cast<float>(sumi), dx * dy);
  } else {
    uint32_t qx[4], dx_bits;
    read_q4_block<kParity>(xc, b, qx, dx_bits);
    sumi = q4_q8_sumi(qx, qy);
    const float dx = fp16_bits_to_f32(dx_bits);
    return make_float2(static_cast<float>(sumi) * dx, dy);
  }
}

// One wave (64 threads) per pair p.  ncols == 0: x row p, y row p, output
// s[p].  ncols > 0: x row p / ncols, y row p % ncols, output
// s[(p / ncols) * bs + p % ncols] (the reference GEMM's loop nest).
// kSums: write sumi[p*nb + b] instead of the fold.
template <DotFmt F, bool kSums>
__global__ __launch_bounds__(64) void block_dot_pairs(size_t nb, float *s, int32_t *sums,
                                                      const uint8_t *vx, size_t bx,
                                                      const uint8_t *vy, size_t by,
                                                      size_t ncols, size_t bs) {
  constexpr int kXBytes = F == DotFmt::kQ8Q8 ? kQ8Bytes : kQ4Bytes;
  // +16: the last even block's 9th dword (or 5th) reads 2 bytes past its end.
  __shared__ __align__(16) uint8_t xl[kChunkBlocks * kXBytes + 16];
  __shared__ __align__(16) uint8_t yl[kChunkBlocks * kQ8Bytes + 16];
  __shared__ float2 terms[kChunkBlocks];

  const size_t p = blockIdx.x;
  size_t xr = p, yr = p, oi = p;
  if (ncols != 0) {
    xr = p / ncols;
    yr = p - xr * ncols;
    oi = xr * bs + yr;
  }
  const uint8_t *xrow = vx + xr * bx;
  const uint8_t *yrow = vy + yr * by;
  const int l = threadIdx.x;
  float sumf = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kChunkBlocks) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kChunkBlocks), nb - c0));
    copy_span_to_lds(xl, xrow + c0 * kXBytes, nbc * kXBytes, l, 64);
    copy_span_to_lds(yl, yrow + c0 * kQ8Bytes, nbc * kQ8Bytes, l, 64);
    __syncthreads();
    {
      int sumi;
      const int b0 = 2 * l;
      if (b0 < nbc) {
        const float2 t = block_terms<F, 0>(xl, yl, b0, sumi);
        if constexpr (kSums)
          sums[p * nb + c0 + b0] = sumi;
        else
          terms[b0] = t;
      }
      const int b1 = 2 * l + 1;
      if (b1 < nbc) {
        const float2 t = block_terms<F, 1>(xl, yl, b1, sumi);
        if constexpr (kSums)
          sums[p * nb + c0 + b1] = sumi;
        else
          terms[b1] = t;
      }
    }
    __syncthreads();
    if constexpr (!kSums) {
      // Serial ascending fold; every lane computes it (LDS broadcast reads).
#pragma unroll 8
      for (int b = 0; b < nbc; ++b) {
        const float2 t = terms[b];
        sumf = fmaf(t.x, t.y, sumf);
      }
      __syncthreads();
    }
  }
  if constexpr (!kSums) {
    if (l == 0)
      s[oi] = sumf;
  }
}

// ---------------------------------------------------------------------------
// Register-direct row pairs (rows 4-byte aligned, even block count): a wave
// owns kPairs row pairs.  For each pair, lane l loads its block pair 2l,
// 2l+1 of both rows straight into registers (68 or 36 bytes, dword aligned --
// across the wave the loads cover the row chunk contiguously), computes the
// two blocks' fold operands and writes them to LDS; then DPP row r folds pair
// r % kPairs with fold_chain, 8 consecutive blocks per lane, so the pairs'
// serial folds run side by side in the same instructions and no LDS access
// sits on the dependency chain (with fewer than four pairs per wave, the
// other DPP rows fold copies, which are not stored).  Pairs per wave:
// two when both operands are distinct rows (16384 Q8_0 pairs of 4096: 24.5
// against 25.5 us with one, 26.8 with four) -- a wave walks its pairs one
// after another, so fewer pairs per wave means more, shorter waves -- and one
// when a stride is 0, one row shared by every pair (the decode GEMV, over 640
// MB of rotating weights: 4096^2 5.34 against 6.01 us, 14336 x 4096 12.2
// against 14.3 us, 1024 x 4096 3.31 against 4.01 us).
// ---------------------------------------------------------------------------
constexpr int kDdWaves = 4;
constexpr int kDdLanes = 16;                          // fold lanes per pair
constexpr int kDdTerms = kChunkBlocks / kDdLanes;     // 8 blocks per fold lane
constexpr int kDdStride = kChunkBlocks + 8;           // float2 per pair row (padded)

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// Blocks 2l, 2l+1 of a Q8_0 row at p (68 bytes, dword aligned): quants as 8
// aligned dwords each, fp16 scale bits.
__device__ __forceinline__ void load_q8_pair(const uint8_t *p, uint32_t q0[8], uint32_t q1[8],
                                             uint32_t &d0, uint32_t &d1) {
  const uint32_t *g = reinterpret_cast<const uint32_t *>(p);
  uint32_t r[17];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(g + 4 * k);
    r[4 * k + 0] = v.x; r[4 * k + 1] = v.y; r[4 * k + 2] = v.z; r[4 * k + 3] = v.w;
  }
  r[16] = g[16];
  d0 = r[0] & 0xffffu;  // block 2l: d at bytes 0-1, quants at 2..33
  d1 = r[8] >> 16;      // block 2l+1: d at 34-35, quants at 36..67
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    q0[k] = funnel16(r[k], r[k + 1]);
    q1[k] = r[k + 9];
  }
}

// Blocks 2l, 2l+1 of a Q4_0 row at p (36 bytes, dword aligned).
__device__ __forceinline__ void load_q4_pair(const uint8_t *p, uint32_t q0[4], uint32_t q1[4],
                                             uint32_t &d0, uint32_t &d1) {
  const uint32_t *g = reinterpret_cast<const uint32_t *>(p);
  const u32x4a4 a = *reinterpret_cast<const u32x4a4 *>(g);
  const u32x4a4 b = *reinterpret_cast<const u32x4a4 *>(g + 4);
  const uint32_t r[9] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, g[8]};
  d0 = r[0] & 0xffffu;  // block 2l: d at bytes 0-1, quants at 2..17
  d1 = r[4] >> 16;      // block 2l+1: d at 18-19, quants at 20..35
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    q0[k] = funnel16(r[k], r[k + 1]);
    q1[k] = r[k + 5];
  }
}

// Fold operands of one block: fmaf(t.x, t.y, sumf) is the reference step.
template <DotFmt F>
__device__ __forceinline__ float2 fold_terms(int sumi, uint32_t dx_bits, uint32_t dy_bits) {
  const float dx = fp16_bits_to_f32(dx_bits), dy = fp16_bits_to_f32(dy_bits);
  if constexpr (F == DotFmt::kQ8Q8)
    return make_float2(static_cast<float>(sumi), dx * dy);  // d_x*d_y exact
  else
    return make_float2(static_cast<float>(sumi) * dx, dy);
}

// Output of pair p: s[p * os].  by = 0 pairs every x row with one y row (the
// GEMM's nc = 1 decode shape).
template <DotFmt F, int kPairs>
__global__ __launch_bounds__(kDdWaves * 64) void block_dot_direct(size_t nb, float *s, size_t os,
                                                                   const uint8_t *vx, size_t bx,
                                                                   const uint8_t *vy, size_t by,
                                                                   size_t npairs) {
  constexpr int kXBytes = F == DotFmt::kQ8Q8 ? kQ8Bytes : kQ4Bytes;
  static_assert(kPairs == 1 || kPairs == 2 || kPairs == 4, "each DPP row folds one pair");
  __shared__ __align__(16) float2 tl[kDdWaves][kPairs][kDdStride];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const size_t p0 = (static_cast<size_t>(blockIdx.x) * kDdWaves + w) * kPairs;
  const int fr = (l >> 4) % kPairs, fp = l & (kDdLanes - 1);  // pair folded, lane in chain
  float sumf = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kChunkBlocks) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kChunkBlocks), nb - c0));
    const int b0 = 2 * l;
#pragma unroll
    for (int r = 0; r < kPairs; ++r) {
      const size_t p = min(p0 + r, npairs - 1);  // pairs past npairs: computed, never stored
      float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);  // absent blocks: fma(0, 0, sumf) == sumf
      if (b0 < nbc) {  // nbc is even: the pair is whole or absent
        uint32_t y0[8], y1[8], dy0, dy1;
        load_q8_pair(vy + p * by + (c0 + b0) * kQ8Bytes, y0, y1, dy0, dy1);
        int s0, s1;
        uint32_t dx0, dx1;
        if constexpr (F == DotFmt::kQ8Q8) {
          uint32_t x0[8], x1[8];
          load_q8_pair(vx + p * bx + (c0 + b0) * kXBytes, x0, x1, dx0, dx1);
          s0 = q8_q8_sumi(x0, y0);
          s1 = q8_q8_sumi(x1, y1);
        } else {
          uint32_t x0[4], x1[4];
          load_q4_pair(vx + p * bx + (c0 + b0) * kXBytes, x0, x1, dx0, dx1);
          s0 = q4_q8_sumi(x0, y0);
          s1 = q4_q8_sumi(x1, y1);
        }
        const float2 t0 = fold_terms<F>(s0, dx0, dy0);
        const float2 t1 = fold_terms<F>(s1, dx1, dy1);
        t = make_float4(t0.x, t0.y, t1.x, t1.y);
      }
      *reinterpret_cast<float4 *>(&tl[w][r][b0]) = t;
    }
    wave_lds_sync();  // the LDS rows are this wave's own
    float ta[kDdTerms], tb[kDdTerms];
#pragma unroll
    for (int k = 0; k < kDdTerms; k += 2) {
      const float4 v = *reinterpret_cast<const float4 *>(&tl[w][fr][fp * kDdTerms + k]);
      ta[k] = v.x; tb[k] = v.y; ta[k + 1] = v.z; tb[k + 1] = v.w;
    }
    // the previous chunk's sum sits in the last lane of the fold row: seed lane 0
    const float carry = __shfl(sumf, (l & ~(kDdLanes - 1)) + kDdLanes - 1);
    sumf = fold_chain<kDdLanes, kDdTerms>(ta, tb, fp == 0 ? carry : 0.0f);
    wave_lds_sync();  // the LDS rows are this wave's own
  }
  if (fp == kDdLanes - 1 && (l >> 4) < kPairs && p0 + fr < npairs)
    s[(p0 + fr) * os] = sumf;
}

// Rows of exactly 128 / kSplit blocks (n = 2048 for kSplit = 2, 1024 for 4):
// kSplit pairs per wave side by side, lane group g = l / (64 / kSplit) on pair
// g, lane l owning blocks 2(l % G), 2(l % G) + 1 (G lanes a group), so no lane
// idles (block_dot_direct would leave all but the first group without a
// block).  DPP row r folds pair r % kSplit (copies past kSplit are not
// stored), 16 lanes: the same chain per pair, bit for bit.
template <DotFmt F, int kSplit = 2>
__global__ __launch_bounds__(kDdWaves * 64) void block_dot_half(float *s, size_t os,
                                                                 const uint8_t *vx, size_t bx,
                                                                 const uint8_t *vy, size_t by,
                                                                 size_t npairs) {
  constexpr int kXBytes = F == DotFmt::kQ8Q8 ? kQ8Bytes : kQ4Bytes;
  constexpr int kNb = kChunkBlocks / kSplit;   // blocks a row
  constexpr int kGroup = 64 / kSplit;          // lanes a group
  constexpr int kTerms = kNb / kDdLanes;       // blocks per fold lane
  static_assert(kSplit == 2 || kSplit == 4, "one DPP row per pair");
  __shared__ __align__(16) float2 tl[kDdWaves][kSplit][kNb + 8];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int hw = l / kGroup, b0 = 2 * (l % kGroup);
  const size_t p0 = (static_cast<size_t>(blockIdx.x) * kDdWaves + w) * kSplit;
  const int fr = (l >> 4) % kSplit, fp = l & (kDdLanes - 1);  // pair folded, lane in chain
  {
    const size_t p = min(p0 + hw, npairs - 1);  // pairs past npairs: computed, never stored
    uint32_t y0[8], y1[8], dy0, dy1;
    load_q8_pair(vy + p * by + b0 * kQ8Bytes, y0, y1, dy0, dy1);
    int s0, s1;
    uint32_t dx0, dx1;
    if constexpr (F == DotFmt::kQ8Q8) {
      uint32_t x0[8], x1[8];
      load_q8_pair(vx + p * bx + b0 * kXBytes, x0, x1, dx0, dx1);
      s0 = q8_q8_sumi(x0, y0);
      s1 = q8_q8_sumi(x1, y1);
    } else {
      uint32_t x0[4], x1[4];
      load_q4_pair(vx + p * bx + b0 * kXBytes, x0, x1, dx0, dx1);
      s0 = q4_q8_sumi(x0, y0);
      s1 = q4_q8_sumi(x1, y1);
    }
    const float2 t0 = fold_terms<F>(s0, dx0, dy0);
    const float2 t1 = fold_terms<F>(s1, dx1, dy1);
    *reinterpret_cast<float4 *>(&tl[w][hw][b0]) = make_float4(t0.x, t0.y, t1.x, t1.y);
  }
  wave_lds_sync();  // the LDS rows are this wave's own
  float ta[kTerms], tb[kTerms];
#pragma unroll
  for (int k = 0; k < kTerms; k += 2) {
    const float4 v = *reinterpret_cast<const float4 *>(&tl[w][fr][fp * kTerms + k]);
    ta[k] = v.x; tb[k] = v.y; ta[k + 1] = v.z; tb[k + 1] = v.w;
  }
  const float sumf = fold_chain<kDdLanes, kTerms>(ta, tb, 0.0f);
  if (fp == kDdLanes - 1 && (l >> 4) < kSplit && p0 + fr < npairs)
    s[(p0 + fr) * os] = sumf;
}

}  // namespace tcrv

namespace tcrv_host {

using tcrv::DotFmt;

// The register-direct row pairs, one pair per wave when a stride is 0 (one row
// shared by every pair), else two; rows of exactly 64 blocks two pairs per
// wave, one per half-wave (the Q8_0 decode GEMV at n = 2048, us, against one
// pair per wave: 4096 rows 3.72/4.83, 11008 rows 6.24/8.27, 2048 rows
// 2.99/3.57; 16384 distinct row pairs 13.8/13.8), rows of 32 blocks four
// (n = 1024: 4096 rows 2.74/4.35, 14336 rows 4.85/8.95; 16384 distinct row
// pairs 7.86/10.05).
template <DotFmt F>
int launch_direct_pairs(size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx,
                        const uint8_t *vy, size_t by, size_t npairs, hipStream_t st) {
  const bool shared = bx == 0 || by == 0;
  const size_t per_group = static_cast<size_t>(tcrv::kDdWaves) * (shared ? 1 : 2);
  const size_t groups = (npairs + per_group - 1) / per_group;
  if (groups > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  const dim3 g(static_cast<unsigned>(groups)), b(tcrv::kDdWaves * 64);
  if (nb == static_cast<size_t>(tcrv::kChunkBlocks / 2)) {
    const size_t per_half = static_cast<size_t>(tcrv::kDdWaves) * 2;
    tcrv::block_dot_half<F><<<dim3(static_cast<unsigned>((npairs + per_half - 1) / per_half)), b, 0,
                              st>>>(s, os, vx, bx, vy, by, npairs);
    return launch_status();
  }
  if (nb == static_cast<size_t>(tcrv::kChunkBlocks / 4)) {
    const size_t per_q = static_cast<size_t>(tcrv::kDdWaves) * 4;
    tcrv::block_dot_half<F, 4><<<dim3(static_cast<unsigned>((npairs + per_q - 1) / per_q)), b, 0,
                                 st>>>(s, os, vx, bx, vy, by, npairs);
    return launch_status();
  }
  if (shared)
    tcrv::block_dot_direct<F, 1><<<g, b, 0, st>>>(nb, s, os, vx, bx, vy, by, npairs);
  else
    tcrv::block_dot_direct<F, 2><<<g, b, 0, st>>>(nb, s, os, vx, bx, vy, by, npairs);
  return launch_status();
}

template <DotFmt F>
int launch_pairs(size_t n, float *s, int32_t *sums, const uint8_t *vx, size_t bx,
                 const uint8_t *vy, size_t by, size_t npairs, size_t ncols, size_t bs,
                 void *stream) {
  const size_t nb = n / tcrv::kQK;
  if (nb == 0 || npairs == 0)
    return TCRV_HIP_OK;  // the reference writes sumf = 0 for nb == 0; see callers
  if (!vx || !vy || (!s && !sums))
    return TCRV_HIP_ERR_NULL_POINTER;
  const size_t xrows = ncols ? npairs / ncols : npairs;
  const size_t yrows = ncols ? ncols : npairs;
  if (!aligned2(vx) || !aligned2(vy) || (xrows > 1 && (bx & 1u)) || (yrows > 1 && (by & 1u)))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t xbytes = nb * (F == DotFmt::kQ8Q8 ? tcrv::kQ8Bytes : tcrv::kQ4Bytes);
  if ((xrows > 1 && bx < xbytes) || (yrows > 1 && by < nb * tcrv::kQ8Bytes))
    return TCRV_HIP_ERR_BAD_SIZE;
  if (npairs > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  hipStream_t st = as_stream(stream);
  const bool direct = !sums && ncols == 0 && nb % 2 == 0 && aligned4(vx) && aligned4(vy) &&
                      (xrows == 1 || bx % 4 == 0) && (yrows == 1 || by % 4 == 0);
  if (direct)
    return launch_direct_pairs<F>(nb, s, 1, vx, bx, vy, by, npairs, st);
  if (sums)
    tcrv::block_dot_pairs<F, true><<<dim3(static_cast<unsigned>(npairs)), dim3(64), 0, st>>>(
        nb, s, sums, vx, bx, vy, by, ncols, bs);
  else
    tcrv::block_dot_pairs<F, false><<<dim3(static_cast<unsigned>(npairs)), dim3(64), 0, st>>>(
        nb, s, sums, vx, bx, vy, by, ncols, bs);
  return launch_status();
}

}  // namespace tcrv_host

// Zero-block calls: the reference still stores sumf = 0.0f (nb = 0 skips the
// loop, then *s = sumf).  A tiny kernel keeps that observable behaviour.
namespace {
__global__ void store_zeros(float *s, size_t count, size_t stride, size_t ncols) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) {
    const size_t r = ncols ? i / ncols : i;
    const size_t c = ncols ? i - r * ncols : 0;
    s[ncols ? r * stride + c : i] = 0.0f;
  }
}

}  // namespace

namespace tcrv_host {

int zero_outputs(float *s, size_t count, size_t stride, size_t ncols, void *stream) {
  if (count == 0)
    return TCRV_HIP_OK;
  if (!s)
    return TCRV_HIP_ERR_NULL_POINTER;
  const size_t grid = (count + 255) / 256;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  store_zeros<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, as_stream(stream)>>>(
      s, count, stride, ncols);
  return launch_status();
}

template <DotFmt F>
int rows_direct(size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx, const uint8_t *vy,
                size_t by, size_t npairs, void *stream) {
  if (nb % 2 != 0 || !aligned4(vx) || !aligned4(vy) || bx % 4 != 0 || by % 4 != 0)
    return TCRV_HIP_ERR_UNSUPPORTED;
  return launch_direct_pairs<F>(nb, s, os, vx, bx, vy, by, npairs, as_stream(stream));
}

int q8_0_rows_direct(size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx,
                     const uint8_t *vy, size_t by, size_t npairs, void *stream) {
  return rows_direct<DotFmt::kQ8Q8>(nb, s, os, vx, bx, vy, by, npairs, stream);
}

int q4_0_rows_direct(size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx,
                     const uint8_t *vy, size_t by, size_t npairs, void *stream) {
  return rows_direct<DotFmt::kQ4Q8>(nb, s, os, vx, bx, vy, by, npairs, stream);
}

int q4_0_grid(size_t n, float *s, const uint8_t *vx, size_t bx, const uint8_t *vy, size_t by,
              size_t nr, size_t nc, size_t bs, void *stream) {
  if (n / tcrv::kQK == 0)
    return zero_outputs(s, nr * nc, bs, nc, stream);
  if (!s)
    return TCRV_HIP_ERR_NULL_POINTER;
  return launch_pairs<tcrv::DotFmt::kQ4Q8>(n, s, nullptr, vx, bx, vy, by, nr * nc, nc, bs,
                                           stream);
}

}  // namespace tcrv_host

using tcrv_host::zero_outputs;

extern "C" {

int tcrv_hip_q8_0_q8_0_block_dot(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                 void *stream) {
  if (n / tcrv::kQK == 0)
    return zero_outputs(s, 1, 0, 0, stream);
  if (!s)
    return TCRV_HIP_ERR_NULL_POINTER;
  return tcrv_host::launch_pairs<tcrv::DotFmt::kQ8Q8>(n, s, nullptr, vx, 0, vy, 0, 1, 0, 0,
                                                      stream);
}

int tcrv_hip_q8_0_q8_0_block_dot_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                      const uint8_t *vy, size_t by, size_t nrows,
                                      void *stream) {
  if (n / tcrv::kQK == 0)
    return zero_outputs(s, nrows, 0, 0, stream);
  if (!s)
    return TCRV_HIP_ERR_NULL_POINTER;
  return tcrv_host::launch_pairs<tcrv::DotFmt::kQ8Q8>(n, s, nullptr, vx, bx, vy, by, nrows,
                                                      0, 0, stream);
}

int tcrv_hip_q4_0_q8_0_block_dot(size_t n, float *s, size_t bs, const uint8_t *vx,
                                 size_t bx, const uint8_t *vy, size_t by, int32_t nrc,
                                 void *stream) {
  (void)bs;
  (void)bx;
  (void)by;
  (void)nrc;  // read by neither the reference emitter nor this entry
  if (n / tcrv::kQK == 0)
    return zero_outputs(s, 1, 0, 0, stream);
  if (!s)
    return TCRV_HIP_ERR_NULL_POINTER;
  return tcrv_host::launch_pairs<tcrv::DotFmt::kQ4Q8>(n, s, nullptr, vx, 0, vy, 0, 1, 0, 0,
                                                      stream);
}

int tcrv_hip_q4_0_q8_0_block_dot_rows(size_t n, float *s, const uint8_t *vx, size_t bx,
                                      const uint8_t *vy, size_t by, size_t nrows,
                                      void *stream) {
  if (n / tcrv::kQK == 0)
    return zero_outputs(s, nrows, 0, 0, stream);
  if (!s)
    return TCRV_HIP_ERR_NULL_POINTER;
  return tcrv_host::launch_pairs<tcrv::DotFmt::kQ4Q8>(n, s, nullptr, vx, bx, vy, by, nrows,
                                                      0, 0, stream);
}

int tcrv_hip_q8_0_q8_0_block_sums(size_t n, int32_t *sumi, const uint8_t *vx, size_t bx,
                                  const uint8_t *vy, size_t by, size_t nrows, void *stream) {
  if (n / tcrv::kQK == 0 || nrows == 0)
    return TCRV_HIP_OK;
  if (!sumi)
    return TCRV_HIP_ERR_NULL_POINTER;
  return tcrv_host::launch_pairs<tcrv::DotFmt::kQ8Q8>(n, nullptr, sumi, vx, bx, vy, by, nrows,
                                                      0, 0, stream);
}

int tcrv_hip_q4_0_q8_0_block_sums(size_t n, int32_t *sumi, const uint8_t *vx, size_t bx,
                                  const uint8_t *vy, size_t by, size_t nrows, void *stream) {
  if (n / tcrv::kQK == 0 || nrows == 0)
    return TCRV_HIP_OK;
  if (!sumi)
    return TCRV_HIP_ERR_NULL_POINTER;
  return tcrv_host::launch_pairs<tcrv::DotFmt::kQ4Q8>(n, nullptr, sumi, vx, bx, vy, by, nrows,
                                                      0, 0, stream);
}

}  // extern "C"
