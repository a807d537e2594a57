// mfma_fold.h -- pieces shared by the MFMA GEMMs (gemm.hip, gemm_tiled.hip):
// the XCD-aware tile order and the Q8_0 fold of tcrv::gemm_wide<false>, the
// repack GEMM and the tiled GEMM, parametrized by their staging layouts.
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
//                              (16 matrix cycles per block, half the per-block cost
//                              of the 2-block f32 outer product)
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
__device__ __forceinline__ v16f q8_dxy(uint32_t ux, uint32_t uy) {
  const v4h ax = __builtin_bit_cast(v4h, make_uint2(ux, 0u));
  const v4h by = __builtin_bit_cast(v4h, make_uint2(uy, 0u));
  return __builtin_amdgcn_mfma_f32_32x32x8f16(ax, by, v16f{}, 0, 0, 0);
}

// The fold of one step.  The empty asm pins the folded accumulators at this
// point of the instruction stream: instruction selection otherwise sinks the
// pure VALU work past every scheduling fence to the end of the chunk, where
// all the steps' MFMA results are then live at once.
__device__ __forceinline__ void q8_fold(float (&acc)[16], const v16i &sumi, const v16f &dxy) {
#pragma unroll
  for (int e = 0; e < 16; ++e)
    acc[e] = fmaf(static_cast<float>(sumi[e]), dxy[e], acc[e]);
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

}  // namespace tcrv
