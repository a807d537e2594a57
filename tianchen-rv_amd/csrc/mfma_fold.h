// mfma_fold.h -- pieces shared by the MFMA GEMMs (gemm.hip, gemm_tiled.hip):
// the XCD-aware tile order, the Q8_0 fold of tcrv::gemm_wide<false>, the
// repack GEMM and the tiled GEMM, and the Q4_0 fold of the tiled Q4_0 GEMM,
// parametrized by their staging layouts.
//
// Per 32x32 output tile and Q8_0 block b, the reference fold is
//   acc = fma((float)sumi, d_x * d_y, acc)
// (RVVToEmitCBlockQuantLinear.cpp:7538-7575, the product of the two scales
// rounded first -- it is exact, two fp16 significands -- then one fma), in
// ascending block order.  Here:
//   v_mfma_i32_32x32x32_i8  -> sumi(row, col) (exact int32 block sums; K = 32 is
//                              exactly one block)
//   v_mfma_f32_32x32x8_f16  -> d_x(row) * d_y(col): k-slot 0 carries the two fp16
//                              scales, every other k-slot is zero, so each output
//                              is one product of two fp16 values, exact in fp32
//                              (32 matrix cycles per block, measured on gfx950:
//                              per block what the 2-block f32 outer product
//                              costs, with no VALU to build its operands)
//   VALU: 16 conversions and 16 fmas per lane, in order.
// Scales are staged as fp16 bit patterns, [block][row], followed by 32 zero
// rows: lanes 32-63 (k-slots 4-7 of the f16 MFMA) point there, so building an
// operand costs one 16-bit LDS read and no VALU.
#pragma once

#include "tcrv_hip_internal.h"

namespace tcrv {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// XCD-aware tile order: work-groups are dispatched round-robin over the 8
// XCDs (id % 8), so id is first remapped so that each XCD owns one contiguous
// range of tiles, and that range is walked in groups of kGroupM tile rows so
// that concurrently running work-groups share weight and activation panels in
// their XCD's L2.
__device__ __forceinline__ void tile_of(unsigned id, unsigned tiles_m, unsigned tiles_n,
                                        unsigned &tm, unsigned &tn) {
  constexpr unsigned kXcds = 8, kGroupM = 8;
  const unsigned total = tiles_m * tiles_n;
  if (total % kXcds == 0)
    id = (id % kXcds) * (total / kXcds) + id / kXcds;
  const unsigned per_group = kGroupM * tiles_n;
  const unsigned group = id / per_group;
  const unsigned first_m = group * kGroupM;
  const unsigned gm = min(tiles_m - first_m, kGroupM);
  const unsigned in_group = id - group * per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// The operands of one (tile, block) step: qa/qb point at this lane's 16 quant
// bytes of block 0 in the staged A (weight) and B (token) rows, block b
// kBlockStride bytes further; hx/hy at this lane's fp16 scale slot of block 0
// (a zero row for lanes 32-63), block b kScaleRow scales further.  The two
// tiles of a wave share the B operand and d_y, read once per block.
template <int kBlockStride>
__device__ __forceinline__ v4i q8_frag(const int8_t *q, int b) {
  return *reinterpret_cast<const v4i *>(q + b * kBlockStride);
}

template <int kScaleRow>
__device__ __forceinline__ uint32_t q8_scale(const uint16_t *h, int b) {
  return h[b * kScaleRow];
}

// The block-sum MFMA (exact int32 sums of one 32x32 tile and block).
__device__ __forceinline__ v16i q8_sumi(const v4i &a, const v4i &bq) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, v16i{}, 0, 0, 0);
}

// The scale MFMA: d_x * d_y of one tile and block, from the lane's two fp16
// scale bit patterns (k-slot 0; the zero k-slots of lanes 32-63 come from the
// zero rows).
// The operands are the zero-extended 16-bit reads taken whole as the low two
// halves (k-slots 0, 1 = the scale, 0): built half by half, the compiler masks
// each read again (one VALU instruction and a hazard wait before the MFMA).
__device__ __forceinline__ v16f q8_dxy(uint32_t ux, uint32_t uy) {
  const v2h z = {};
  const v4h ax = __builtin_shufflevector(__builtin_bit_cast(v2h, ux), z, 0, 1, 2, 3);
  const v4h by = __builtin_shufflevector(__builtin_bit_cast(v2h, uy), z, 0, 1, 2, 3);
  return __builtin_amdgcn_mfma_f32_32x32x8f16(ax, by, v16f{}, 0, 0, 0);
}

// The fold of one step.  The empty asm pins the folded accumulators at this
// point of the instruction stream: instruction selection otherwise sinks the
// pure VALU work past every scheduling fence to the end of the chunk, where
// all the steps' MFMA results are then live at once.  kConvertFirst: all 16
// conversions (in place) before the first fma, which then reads a scale
// product whose MFMA was issued ~16 conversions earlier instead of ~4 (with
// two waves per SIMD the other wave hides less of that wait: the 256 x 256
// tiled kernel 154.3 -> 151.3 us at 4096^3; the four-wave kernels gain
// nothing).  The same operations in the same order per element either way.
template <bool kConvertFirst = false>
__device__ __forceinline__ void q8_fold(float (&acc)[16], const v16i &sumi, const v16f &dxy) {
  if constexpr (kConvertFirst) {
    float f[16];
#pragma unroll
    for (int e = 0; e < 16; ++e)
      f[e] = static_cast<float>(sumi[e]);
    asm volatile("" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                 "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]),
                 "+v"(f[12]), "+v"(f[13]), "+v"(f[14]), "+v"(f[15]));
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[e] = fmaf(f[e], dxy[e], acc[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[e] = fmaf(static_cast<float>(sumi[e]), dxy[e], acc[e]);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e)
    asm volatile("" : "+v"(acc[e]));
}

// One chunk of kBlocks blocks for a wave's two tiles (tile 1's A operand is
// kTileStride bytes after tile 0's, its scales 32 rows after), steps
// s = 2b + i in ascending block order, so each tile's blocks are folded in
// ascending order.
// kPipe: the block-sum MFMA of step s+1 is issued in step s, beside the fold of
// step s, and the scale MFMA of step s at its start (ready once the fold's 16
// conversions have run).  Otherwise each step issues both MFMAs and folds, and
// the other waves of the SIMD fill the wait.  Every step is fenced
// (`sched_barrier`) and ordered within (`sched_group_barrier`: LDS reads,
// MFMAs, VALU), and the next step's sums are pinned in the step that issues
// them.  `after_step(s)` runs after step s (a staging store, or nothing).
template <bool kPipe, int kBlocks, int kBlockStride, int kTileStride, int kScaleRow,
          typename AfterStep>
__device__ __forceinline__ void fold_chunk_q8(float (&acc)[2][16], const int8_t *qa,
                                              const int8_t *qb, const uint16_t *hx0,
                                              const uint16_t *hx1, const uint16_t *hy,
                                              AfterStep &&after_step) {
  if constexpr (kPipe) {
    v4i bq = q8_frag<kBlockStride>(qb, 0);
    v16i cur = q8_sumi(q8_frag<kBlockStride>(qa, 0), bq);
    uint32_t uy = 0;
#pragma unroll
    for (int s = 0; s < 2 * kBlocks; ++s) {
      const int i = s & 1, b = s >> 1;
      v16i nxt;
      if (s + 1 < 2 * kBlocks) {
        const int i1 = (s + 1) & 1, b1 = (s + 1) >> 1;
        if (i1 == 0)  // a new block: its B operand
          bq = q8_frag<kBlockStride>(qb, b1);
        nxt = q8_sumi(q8_frag<kBlockStride>(qa + i1 * kTileStride, b1), bq);
      }
      if (i == 0)
        uy = q8_scale<kScaleRow>(hy, b);
      const v16f dxy = q8_dxy(q8_scale<kScaleRow>(i ? hx1 : hx0, b), uy);
      q8_fold(acc[i], cur, dxy);
      if (s + 1 < 2 * kBlocks) {
        asm volatile("" : "+v"(nxt));
        cur = nxt;
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // LDS reads
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMAs
      __builtin_amdgcn_sched_group_barrier(0x002, 40, 0); // VALU
      __builtin_amdgcn_sched_barrier(0);
      after_step(s);
    }
  } else {
    v4i bq;
    uint32_t uy = 0;
#pragma unroll
    for (int s = 0; s < 2 * kBlocks; ++s) {
      const int i = s & 1, b = s >> 1;
      if (i == 0) {
        bq = q8_frag<kBlockStride>(qb, b);
        uy = q8_scale<kScaleRow>(hy, b);
      }
      const v16i sumi = q8_sumi(q8_frag<kBlockStride>(qa + i * kTileStride, b), bq);
      const v16f dxy = q8_dxy(q8_scale<kScaleRow>(i ? hx1 : hx0, b), uy);
      q8_fold(acc[i], sumi, dxy);
      __builtin_amdgcn_sched_barrier(0);
      after_step(s);
    }
  }
}

// A trailing partial chunk of nbc < the chunk's blocks, one step at a time.
template <int kBlockStride, int kTileStride, int kScaleRow>
__device__ __forceinline__ void fold_tail_q8(float (&acc)[2][16], const int8_t *qa,
                                             const int8_t *qb, const uint16_t *hx0,
                                             const uint16_t *hx1, const uint16_t *hy, int nbc) {
  for (int b = 0; b < nbc; ++b) {
    const v4i bq = q8_frag<kBlockStride>(qb, b);
    const uint32_t uy = q8_scale<kScaleRow>(hy, b);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const v16i sumi = q8_sumi(q8_frag<kBlockStride>(qa + i * kTileStride, b), bq);
      const v16f dxy = q8_dxy(q8_scale<kScaleRow>(i ? hx1 : hx0, b), uy);
      q8_fold(acc[i], sumi, dxy);
    }
  }
}

// ---- the Q8_0 fold over 2 x 4 tiles per wave ------------------------------
// One chunk of kBlocks blocks for a wave's two weight tiles (A operand at
// qa + i * kTile bytes, d_x at hx + 32 i) and four token tiles (B operand at
// qb + j * kTile, d_y at hy + 32 j); block b is kBlockStride bytes and
// kScaleRow scales further.  Steps s = 8b + 2j + i, so every tile's blocks are
// folded in ascending order.  As in fold_chunk_q8 the block-sum MFMA of step
// s+1 is issued in step s; here every LDS read also lands a whole step before
// the MFMA that takes it (two waves per SIMD hide less latency than four): the
// token operand and d_y of tile j+1 are read in step (b, j, 0), the next
// block's weight operands and d_x in steps (b, 3, 0), (b, 3, 1) and
// (b+1, 0, 0), each into the registers of an operand whose last MFMA has been
// issued (two weight and two token fragments, two d_x and two d_y words).
template <int kBlocks, int kBlockStride, int kTile, int kScaleRow, typename AfterStep>
__device__ __forceinline__ void fold_chunk_q8_2x4(float (&acc)[2][4][16], const int8_t *qa,
                                                  const int8_t *qb, const uint16_t *hx,
                                                  const uint16_t *hy, AfterStep &&after_step) {
  v4i w[2], t[2];
  uint32_t ux[2], uy[2];
  w[0] = q8_frag<kBlockStride>(qa, 0);
  w[1] = q8_frag<kBlockStride>(qa + kTile, 0);
  t[0] = q8_frag<kBlockStride>(qb, 0);
  ux[0] = q8_scale<kScaleRow>(hx, 0);
  ux[1] = q8_scale<kScaleRow>(hx + 32, 0);
  uy[0] = q8_scale<kScaleRow>(hy, 0);
  v16i cur = q8_sumi(w[0], t[0]);
#pragma unroll
  for (int s = 0; s < 8 * kBlocks; ++s) {
    const int b = s >> 3, j = (s >> 1) & 3, i = s & 1;
    if (i == 0) {
      if (j < 3) {
        t[(j + 1) & 1] = q8_frag<kBlockStride>(qb + (j + 1) * kTile, b);
        uy[(j + 1) & 1] = q8_scale<kScaleRow>(hy + 32 * (j + 1), b);
      } else if (b + 1 < kBlocks) {
        t[0] = q8_frag<kBlockStride>(qb, b + 1);
        uy[0] = q8_scale<kScaleRow>(hy, b + 1);
        w[0] = q8_frag<kBlockStride>(qa, b + 1);
      }
      if (j == 0 && b > 0)
        ux[1] = q8_scale<kScaleRow>(hx + 32, b);
    } else if (j == 3 && b + 1 < kBlocks) {
      w[1] = q8_frag<kBlockStride>(qa + kTile, b + 1);
      ux[0] = q8_scale<kScaleRow>(hx, b + 1);
    }
    v16i nxt;
    if (s + 1 < 8 * kBlocks)
      nxt = q8_sumi(w[(s + 1) & 1], t[((s + 1) >> 1) & 1]);
    const v16f dxy = q8_dxy(ux[i], uy[j & 1]);
    q8_fold<true>(acc[i][j], cur, dxy);
    if (s + 1 < 8 * kBlocks) {
      asm volatile("" : "+v"(nxt));
      cur = nxt;
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // LDS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMAs
    __builtin_amdgcn_sched_group_barrier(0x002, 40, 0); // VALU
    __builtin_amdgcn_sched_barrier(0);
    after_step(s);
  }
}

// A trailing partial chunk of nbc blocks over the 2 x 4 tiles, one step at a time.
template <int kBlockStride, int kTile, int kScaleRow>
__device__ __forceinline__ void fold_tail_q8_2x4(float (&acc)[2][4][16], const int8_t *qa,
                                                 const int8_t *qb, const uint16_t *hx,
                                                 const uint16_t *hy, int nbc) {
  for (int b = 0; b < nbc; ++b) {
    const v4i w0 = q8_frag<kBlockStride>(qa, b), w1 = q8_frag<kBlockStride>(qa + kTile, b);
    const uint32_t ux0 = q8_scale<kScaleRow>(hx, b), ux1 = q8_scale<kScaleRow>(hx + 32, b);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4i t = q8_frag<kBlockStride>(qb + j * kTile, b);
      const uint32_t uy = q8_scale<kScaleRow>(hy + 32 * j, b);
      q8_fold(acc[0][j], q8_sumi(w0, t), q8_dxy(ux0, uy));
      q8_fold(acc[1][j], q8_sumi(w1, t), q8_dxy(ux1, uy));
    }
  }
}

// ---- the Q4_0 x Q8_0 fold ----------------------------------------------
// Per tile and block the reference folds acc = fma(fl((float)sumi * d_x), d_y,
// acc) (RVVToEmitCBlockQuantLinear.cpp:322-356): the product with d_x is
// rounded first, so the scales cannot be multiplied ahead.
//
// The tile is computed transposed: the block-sum MFMA takes the tokens as its
// A operand and the weights as B, so lane (c = lane % 32, h = lane / 32) holds
// weight row c and tokens 8g + 4h + j (g, j < 4) of the tile.  d_x is then one
// value per lane and tile-block (a 16-bit LDS read) and d_y one per element,
// read as fp32 (a 128-bit LDS read gives four) from a row the staging widened
// once per chunk.
//
// The MFMA's accumulator input is the integer bit pattern of M = 1.5 * 2^23
// (0x4B400000) in every element, so its results read as floats are
// F = M + sumi exactly: |sumi| <= 32 * 8 * 128 < 2^22 keeps F in M's binade,
// whose spacing is 1.  Then fma(F, d_x, -M * d_x) = fl(sumi * d_x): the exact
// F * d_x - M * d_x = sumi * d_x is rounded once, and -M * d_x is itself exact
// (an fp16 significand times 1.5).  That fma (v_fma_f32) and fma(t, d_y, acc)
// (v_fmac_f32 on d_y widened to fp32) are the fold's two VALU instructions per
// element; d_x and -M * d_x are one each per lane and tile-block.  (With the
// fp16 d_y read in place by v_fma_mix_f32 instead, a register-only copy of the
// step ran 309 against 243 cycles per two tile-blocks at four waves per SIMD.)
// An infinite d_x makes -M * d_x infinite, and the fast form NaN where the
// reference has +-inf: a chunk with a non-finite d_x among the wave's weight
// rows (q4_chunk_nonfinite, one test per chunk) is folded in the exact
// three-instruction form instead (sumi = F - M, exact; fl(sumi * d_x); the
// fma), so the steps themselves carry no branch.
constexpr int kSeedBits = 0x4B400000;
constexpr float kSeed = 12582912.0f;

// The seeded block-sum MFMA of one tile and block: F = M + sumi.  The whole
// vector is bit-cast: __builtin_bit_cast of one subscripted element of an
// int vector reads element 0 with this compiler.
__device__ __forceinline__ v16f q4_seeded_sums(const v4i &tokens, const v4i &weights) {
  v16i seed;
#pragma unroll
  for (int e = 0; e < 16; ++e)
    seed[e] = kSeedBits;
  return __builtin_bit_cast(v16f,
                            __builtin_amdgcn_mfma_i32_32x32x32_i8(tokens, weights, seed, 0, 0, 0));
}

// fp16 bit pattern (low 16 bits of u) -> fp32, exact.
__device__ __forceinline__ float f16_bits(uint32_t u) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u)));
}

// Whether any d_x of the wave's 64 weight rows in the chunk's nbc blocks is
// non-finite (exponent field all ones; NaN is included, which only costs the
// exact form): lane 8b + k reads rows 8k..8k+7 of block b as one 128-bit LDS
// read, and (h & 0x7C00) + 0x0400 reaches bit 15 exactly when h's exponent is
// 0x1F (no carry crosses into the other half).  hx: the wave's row 0, block 0.
template <int kScaleRow>
__device__ __forceinline__ bool q4_chunk_nonfinite(const uint16_t *hx, int nbc, int lane) {
  const int b = lane >> 3, k = lane & 7;
  uint32_t top = 0;
  if (b < nbc) {
    const uint4 w = *reinterpret_cast<const uint4 *>(hx + b * kScaleRow + 8 * k);
    top = ((w.x & 0x7C007C00u) + 0x04000400u) | ((w.y & 0x7C007C00u) + 0x04000400u) |
          ((w.z & 0x7C007C00u) + 0x04000400u) | ((w.w & 0x7C007C00u) + 0x04000400u);
  }
  return __builtin_amdgcn_ballot_w64((top & 0x80008000u) != 0) != 0;
}

// The fold of one tile and block: F the seeded sums, ux the lane's d_x bits,
// fy d_y of its tokens 4h.. of the block as fp32 (tokens 8g + 4h + 0..3 at
// fy + 8g, 16-byte aligned); kExact: the three-instruction form.
template <bool kExact>
__device__ __forceinline__ void q4_fold(float (&acc)[16], const v16f &F, uint32_t ux,
                                        const float *fy) {
  // Plain fp32 arithmetic (the compiler inserts the wait states a VALU read of
  // a matrix-core result needs).  d_x is widened once and hidden from
  // instruction selection, which would otherwise re-read it as fp16 in every
  // product (v_fma_mix_f32 issues slower than v_fma_f32).
  float dx = f16_bits(ux);
  asm volatile("" : "+v"(dx));
  const float c = -kSeed * dx;  // -M * d_x, exact (unused by the exact form)
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 dy = *reinterpret_cast<const float4 *>(fy + 8 * g);
    // fl(sumi * d_x) of four rows, from F directly or from sumi = F - M
    // (exact), all four before the fmas that take them (each product a few
    // instructions ahead of its use).
    float t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      t[j] = kExact ? (F[4 * g + j] - kSeed) * dx : fmaf(F[4 * g + j], dx, c);
    asm volatile("" : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]));
    acc[4 * g + 0] = fmaf(t[0], dy.x, acc[4 * g + 0]);
    acc[4 * g + 1] = fmaf(t[1], dy.y, acc[4 * g + 1]);
    acc[4 * g + 2] = fmaf(t[2], dy.z, acc[4 * g + 2]);
    acc[4 * g + 3] = fmaf(t[3], dy.w, acc[4 * g + 3]);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e)
    asm volatile("" : "+v"(acc[e]));
}

// One chunk of kBlocks blocks for a wave's two tiles with the Q4_0 fold, steps
// s = 2b + i in ascending block order, the seeded MFMA of step s+1 issued in
// step s (as fold_chunk_q8 with kPipe).  qw: this lane's weight quants of tile
// 0, block 0 (tile 1 kTileStride bytes on); qt: its token quants; hx: its
// weight row's d_x slot of tile 0, block 0 (tile 1 is 32 rows on); fy: the
// fp32 d_y of its tokens 4h.. of block 0, block b kFyRow floats on (q4_fold).
template <bool kExact, int kBlocks, int kBlockStride, int kTileStride, int kScaleRow,
          int kFyRow, typename AfterStep>
__device__ __forceinline__ void fold_chunk_q4(float (&acc)[2][16], const int8_t *qw,
                                              const int8_t *qt, const uint16_t *hx,
                                              const float *fy, AfterStep &&after_step) {
  v4i tq = q8_frag<kBlockStride>(qt, 0);
  v16f cur = q4_seeded_sums(tq, q8_frag<kBlockStride>(qw, 0));
#pragma unroll
  for (int s = 0; s < 2 * kBlocks; ++s) {
    const int i = s & 1, b = s >> 1;
    v16f nxt;
    if (s + 1 < 2 * kBlocks) {
      const int i1 = (s + 1) & 1, b1 = (s + 1) >> 1;
      if (i1 == 0)  // a new block: its token operand
        tq = q8_frag<kBlockStride>(qt, b1);
      nxt = q4_seeded_sums(tq, q8_frag<kBlockStride>(qw + i1 * kTileStride, b1));
    }
    q4_fold<kExact>(acc[i], cur, q8_scale<kScaleRow>(hx + 32 * i, b), fy + b * kFyRow);
    if (s + 1 < 2 * kBlocks) {
      asm volatile("" : "+v"(nxt));
      cur = nxt;
    }
    __builtin_amdgcn_sched_barrier(0);
    after_step(s);
  }
}

// A trailing partial chunk of nbc blocks with the Q4_0 fold.
template <bool kExact, int kBlockStride, int kTileStride, int kScaleRow, int kFyRow>
__device__ __forceinline__ void fold_tail_q4(float (&acc)[2][16], const int8_t *qw,
                                             const int8_t *qt, const uint16_t *hx,
                                             const float *fy, int nbc) {
  for (int b = 0; b < nbc; ++b) {
    const v4i tq = q8_frag<kBlockStride>(qt, b);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      q4_fold<kExact>(acc[i], q4_seeded_sums(tq, q8_frag<kBlockStride>(qw + i * kTileStride, b)),
                      q8_scale<kScaleRow>(hx + 32 * i, b), fy + b * kFyRow);
  }
}

// ---- the Q4_0 fold over 2 x 4 tiles per wave ------------------------------
// The fold of one tile and block with d_y already in registers (dy[e]: the
// token of accumulator element e); every fl(sumi * d_x) of the step is formed
// before the first fma that takes one, so the d_y reads issued at the step's
// start have landed by then.  The same operations per element as q4_fold.
template <bool kExact>
__device__ __forceinline__ void q4_fold_dy(float (&acc)[16], const v16f &F, uint32_t ux,
                                           const float (&dy)[16]) {
  float dx = f16_bits(ux);
  asm volatile("" : "+v"(dx));
  const float c = -kSeed * dx;
  float t[16];
#pragma unroll
  for (int e = 0; e < 16; ++e)
    t[e] = kExact ? (F[e] - kSeed) * dx : fmaf(F[e], dx, c);
  asm volatile("" : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]),
               "+v"(t[6]), "+v"(t[7]), "+v"(t[8]), "+v"(t[9]), "+v"(t[10]), "+v"(t[11]),
               "+v"(t[12]), "+v"(t[13]), "+v"(t[14]), "+v"(t[15]));
#pragma unroll
  for (int e = 0; e < 16; ++e)
    acc[e] = fmaf(t[e], dy[e], acc[e]);
#pragma unroll
  for (int e = 0; e < 16; ++e)
    asm volatile("" : "+v"(acc[e]));
}

// d_y of a lane's 16 tokens of one token tile and block (tokens 8g + 4h + j at
// fy + 8g, four 128-bit LDS reads).
__device__ __forceinline__ void q4_read_dy(float (&dy)[16], const float *fy) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 v = *reinterpret_cast<const float4 *>(fy + 8 * g);
    dy[4 * g + 0] = v.x;
    dy[4 * g + 1] = v.y;
    dy[4 * g + 2] = v.z;
    dy[4 * g + 3] = v.w;
  }
}

// One chunk of kBlocks blocks for a wave's two weight tiles (B operand at
// qw + i * kTile, d_x at hx + 32 i) and four token tiles (A operand at
// qt + j * kTile, fp32 d_y at fy + 32 j, block b kFyRow floats on) on
// transposed 32 x 32 tiles, steps s = 8b + 2j + i: every tile's blocks in
// ascending order.  The seeded MFMA of step s+1 is issued in step s; the
// operand reads follow fold_chunk_q8_2x4's schedule (token tile j+1 in step
// (b, j, 0), the next block's weight operands in steps (b, 3, 0) and
// (b, 3, 1)); a token tile's d_y is read once per block, in its step i = 0,
// and serves both weight tiles.
template <bool kExact, int kBlocks, int kBlockStride, int kTile, int kScaleRow, int kFyRow,
          typename AfterStep>
__device__ __forceinline__ void fold_chunk_q4_2x4(float (&acc)[2][4][16], const int8_t *qw,
                                                  const int8_t *qt, const uint16_t *hx,
                                                  const float *fy, AfterStep &&after_step) {
  v4i w[2], t[2];
  uint32_t ux[2];
  float dy[16];
  w[0] = q8_frag<kBlockStride>(qw, 0);
  w[1] = q8_frag<kBlockStride>(qw + kTile, 0);
  t[0] = q8_frag<kBlockStride>(qt, 0);
  ux[0] = q8_scale<kScaleRow>(hx, 0);
  ux[1] = q8_scale<kScaleRow>(hx + 32, 0);
  // the seed, hidden from instruction selection: as a known constant it is
  // rebuilt from scalar registers (24 instructions) each time register
  // pressure evicts it
  v16i seed;
#pragma unroll
  for (int e = 0; e < 16; ++e)
    seed[e] = kSeedBits;
  asm volatile("" : "+v"(seed));
  auto sums = [&](const v4i &tk, const v4i &wt) {
    return __builtin_bit_cast(v16f, __builtin_amdgcn_mfma_i32_32x32x32_i8(tk, wt, seed, 0, 0, 0));
  };
  v16f cur = sums(t[0], w[0]);
#pragma unroll
  for (int s = 0; s < 8 * kBlocks; ++s) {
    const int b = s >> 3, j = (s >> 1) & 3, i = s & 1;
    if (i == 0) {
      q4_read_dy(dy, fy + b * kFyRow + 32 * j);
      if (j < 3) {
        t[(j + 1) & 1] = q8_frag<kBlockStride>(qt + (j + 1) * kTile, b);
      } else if (b + 1 < kBlocks) {
        t[0] = q8_frag<kBlockStride>(qt, b + 1);
        w[0] = q8_frag<kBlockStride>(qw, b + 1);
      }
    } else if (j == 3 && b + 1 < kBlocks) {
      w[1] = q8_frag<kBlockStride>(qw + kTile, b + 1);
    }
    v16f nxt;
    if (s + 1 < 8 * kBlocks)
      nxt = sums(t[((s + 1) >> 1) & 1], w[(s + 1) & 1]);
    q4_fold_dy<kExact>(acc[i][j], cur, ux[i], dy);
    if (j == 3 && b + 1 < kBlocks)  // this block's last use of d_x of tile i
      ux[i] = q8_scale<kScaleRow>(hx + 32 * i, b + 1);
    if (s + 1 < 8 * kBlocks) {
      asm volatile("" : "+v"(nxt));
      cur = nxt;
    }
    __builtin_amdgcn_sched_barrier(0);
    after_step(s);
  }
}

// A trailing partial chunk of nbc blocks over the 2 x 4 transposed tiles.
template <bool kExact, int kBlockStride, int kTile, int kScaleRow, int kFyRow>
__device__ __forceinline__ void fold_tail_q4_2x4(float (&acc)[2][4][16], const int8_t *qw,
                                                 const int8_t *qt, const uint16_t *hx,
                                                 const float *fy, int nbc) {
  for (int b = 0; b < nbc; ++b) {
    const v4i w0 = q8_frag<kBlockStride>(qw, b), w1 = q8_frag<kBlockStride>(qw + kTile, b);
    const uint32_t ux0 = q8_scale<kScaleRow>(hx, b), ux1 = q8_scale<kScaleRow>(hx + 32, b);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4i tq = q8_frag<kBlockStride>(qt + j * kTile, b);
      float dy[16];
      q4_read_dy(dy, fy + b * kFyRow + 32 * j);
      q4_fold_dy<kExact>(acc[0][j], q4_seeded_sums(tq, w0), ux0, dy);
      q4_fold_dy<kExact>(acc[1][j], q4_seeded_sums(tq, w1), ux1, dy);
    }
  }
}

}  // namespace tcrv
