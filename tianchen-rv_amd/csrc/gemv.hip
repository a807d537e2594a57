// gemv.hip -- a7: tcrv_rvv.q4_0_q8_0_gemm (G2) and its decode GEMV (nc = 1).
//
// The reference loops weight rows ir < nr and columns col < nc, and every
// output s[ir*bs + col] is the independent ggml_vec_dot_q4_0_q8_0 of weight
// row ir and activation column col (RVVToEmitCBlockQuantLinear.cpp:1691-2121;
// RVVOps.td:4147-4151).  The decode GEMV kernel below keeps that per-element
// definition and its fold order, fma(fl((float)sumi*d_x), d_y, sumf) in
// ascending block order, while mapping the work onto gfx950:
//   - a work-group of 4 waves owns 4*R consecutive weight rows; each wave
//     stages its R rows (2304 B each at n = 4096) in LDS with 128-bit loads,
//     all issued before the first use;
//   - the activation chunk (shared by every row) is staged once per
//     work-group and its quants for blocks 2l, 2l+1 are held in registers by
//     lane l across the wave's rows;
//   - lane l computes the integer sums of blocks 2l and 2l+1 of every row
//     (v_dot4_i32_i8 on in-register nibble decode), writes fl(sumi*d_x) to LDS,
//     and lanes r < R then run the R serial per-row folds side by side.
#include "tcrv_hip_internal.h"

namespace tcrv {

constexpr int kGvWaves = 4;
constexpr int kGvChunk = 128;  // blocks per chunk (as the block-dot kernels)

template <int kParity>
__device__ __forceinline__ void gv_read_q8(const uint8_t *chunk, int b, uint32_t q[8],
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

template <int kParity>
__device__ __forceinline__ float gv_q4_term(const uint8_t *chunk, int b, const uint32_t qy[8]) {
  const uint32_t *w = reinterpret_cast<const uint32_t *>(chunk) + ((b * kQ4Bytes) >> 2);
  uint32_t r[5];
#pragma unroll
  for (int k = 0; k < 5; ++k)
    r[k] = w[k];
  uint32_t q[4], d_bits;
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
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    acc = sdot4(nibbles_to_i8x4(q[k]), qy[k], acc);
    acc = sdot4(nibbles_to_i8x4(q[k] >> 4), qy[k + 4], acc);
  }
  return static_cast<float>(acc) * fp16_bits_to_f32(d_bits);
}

template <int R>
__global__ __launch_bounds__(kGvWaves * 64) void gemv_q4_0_q8_0_kernel(
    size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx, const uint8_t *vy,
    size_t nr) {
  constexpr int kXRow = kGvChunk * kQ4Bytes + 16;  // 2320: 16-B multiple, +16 over-read pad
  __shared__ __align__(16) uint8_t yl[kGvChunk * kQ8Bytes + 16];
  __shared__ __align__(16) uint8_t xl[kGvWaves][R][kXRow];
  __shared__ float tl[kGvWaves][R][kGvChunk + 1];
  __shared__ float dyl[kGvChunk];

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int l = tid & 63;
  const size_t row0 = (static_cast<size_t>(blockIdx.x) * kGvWaves + w) * R;
  float sumf = 0.0f;  // lane r < R: running fold of row row0 + r

  for (size_t c0 = 0; c0 < nb; c0 += kGvChunk) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kGvChunk), nb - c0));
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t row = min(row0 + r, nr - 1);  // rows past nr recompute row nr-1, unstored
      copy_span_to_lds(xl[w][r], vx + row * bx + c0 * kQ4Bytes, nbc * kQ4Bytes, l, 64);
    }
    copy_span_to_lds(yl, vy + c0 * kQ8Bytes, nbc * kQ8Bytes, tid, kGvWaves * 64);
    __syncthreads();
    for (int b = tid; b < nbc; b += kGvWaves * 64)
      dyl[b] = fp16_bits_to_f32(reinterpret_cast<const uint16_t *>(yl)[b * (kQ8Bytes / 2)]);
    const int b0 = 2 * l, b1 = 2 * l + 1;
    uint32_t qy0[8], qy1[8], dbits;
    if (b0 < nbc)
      gv_read_q8<0>(yl, b0, qy0, dbits);
    if (b1 < nbc)
      gv_read_q8<1>(yl, b1, qy1, dbits);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (b0 < nbc)
        tl[w][r][b0] = gv_q4_term<0>(xl[w][r], b0, qy0);
      if (b1 < nbc)
        tl[w][r][b1] = gv_q4_term<1>(xl[w][r], b1, qy1);
    }
    __syncthreads();
    if (l < R) {
      const float *t = tl[w][l];
#pragma unroll 8
      for (int b = 0; b < nbc; ++b)
        sumf = fmaf(t[b], dyl[b], sumf);
    }
    __syncthreads();
  }
  if (l < R && row0 + l < nr)
    s[(row0 + l) * os] = sumf;
}


// ---------------------------------------------------------------------------
// Register-direct decode GEMV (the fast path: nb even, rows 4-byte aligned).
//
// Lane l of a wave owns blocks 2l and 2l+1 of each 128-block chunk: 36
// contiguous weight bytes per row (two 128-bit loads and one 32-bit load, all
// issued for the wave's kR rows before the first use) and 68 contiguous
// activation bytes, which stay in registers for every row of the wave.
//
// Integer core: with n the raw nibble (0..15) and y the Q8_0 quant,
//   sumi = sum_j (n_j - 8) y_j = sum_j n_j y_j - 8 sum_j y_j,
// so the decode is a mask (low nibbles) or a shift and a mask (high nibbles)
// and the -8 offset enters once per activation block as the accumulator's
// start value; both forms are exact int32 arithmetic, so sumi is bit-identical
// to the reference's offset-binary decode (RVVToEmitC.cpp:2524-2589).
//
// Fold: t_b = fl((float)sumi_b * d_x) per block goes to the wave's LDS rows;
// after a wave-scope sync each row's serial fold sumf = fma(t_b, d_y, sumf),
// b ascending, runs as one chain across a group of fold lanes (fold_chain) --
// the reference's per-row serial fold (RVVToEmitCBlockQuantLinear.cpp:322-356).
// ---------------------------------------------------------------------------
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ void load36(const uint8_t *p, uint32_t w[9]) {
  const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
  const u32x4a4 a = *reinterpret_cast<const u32x4a4 *>(q);
  const u32x4a4 b = *reinterpret_cast<const u32x4a4 *>(q + 4);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  w[8] = q[8];
}

// Activation blocks 2l, 2l+1 (68 bytes, dword aligned) -> quants of each block
// as 8 aligned dwords, fp32 scales and the -8*sum(q) accumulator seeds.
struct ActPair {
  uint32_t q0[8], q1[8];
  float d0, d1;
  int c0, c1;
};

__device__ __forceinline__ void load_act_pair(const uint8_t *p, ActPair &a) {
  const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
  uint32_t r[17];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(q + 4 * k);
    r[4 * k + 0] = v.x; r[4 * k + 1] = v.y; r[4 * k + 2] = v.z; r[4 * k + 3] = v.w;
  }
  r[16] = q[16];
  // block 2l: d at bytes 0-1, quants at bytes 2..33; block 2l+1: d at 34-35,
  // quants at 36..67 (dwords 9..16)
  a.d0 = fp16_bits_to_f32(r[0] & 0xffffu);
  a.d1 = fp16_bits_to_f32(r[8] >> 16);
  int s0 = 0, s1 = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    a.q0[k] = funnel16(r[k], r[k + 1]);
    a.q1[k] = r[k + 9];
    s0 = sdot4(a.q0[k], 0x01010101u, s0);
    s1 = sdot4(a.q1[k], 0x01010101u, s1);
  }
  a.c0 = -8 * s0;
  a.c1 = -8 * s1;
}

// sum_j n_j y_j + seed over one block: quants q[0..3] (16 bytes = 32 nibbles).
__device__ __forceinline__ int nibble_dot(const uint32_t q[4], const uint32_t y[8], int seed) {
  int acc = seed;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    acc = sdot4(q[k] & 0x0F0F0F0Fu, y[k], acc);
    acc = sdot4((q[k] >> 4) & 0x0F0F0F0Fu, y[k + 4], acc);
  }
  return acc;
}

// kOneChunk: nb == kGvChunk exactly (n = 4096), so every lane owns a whole
// block pair, there is one chunk and no carry between chunks.
// kSoA: the weights are in the split layout (tcrv_hip_pack_q4_0_to_soa): for
// nr rows of nb blocks, the 16 quant bytes of row r block b at (r*nb + b)*16
// and its fp16 scale at nr*nb*16 + (r*nb + b)*2, so a lane's block pair is two
// aligned 128-bit loads and one dword (bx is unused).
template <int kWaves, int kR, bool kOneChunk, bool kSoA = false>
__global__ __launch_bounds__(kWaves * 64) void gemv_q4_0_q8_0_direct(
    size_t nb_arg, float *s, size_t os, const uint8_t *vx, size_t bx, const uint8_t *vy,
    size_t nr) {
  const size_t nb = kOneChunk ? static_cast<size_t>(kGvChunk) : nb_arg;
  // fold lanes per row: half a DPP row (8 lanes, 16 terms each) for 4 or 8
  // rows per wave -- 7 lane hops on the fold's dependency chain instead of 15
  // (4096^2: 3.92 against 3.98 us with 16 lanes; 4 lanes, 4.00 us) -- and a
  // whole DPP row for fewer rows.  Lanes past the last row fold copies of it,
  // which are never stored.
  constexpr int kLanes = kR >= 4 ? 8 : 16;
  constexpr int kTerms = kGvChunk / kLanes;    // blocks per fold lane
  static_assert(kLanes == 8 || kLanes == 16, "fold groups live inside one DPP row");
  __shared__ __align__(16) float tl[kWaves][kR][kGvChunk + 4];
  __shared__ __align__(16) float dyl[kWaves][kGvChunk];

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int l = tid & 63;
  const size_t row0 = (static_cast<size_t>(blockIdx.x) * kWaves + w) * kR;
  const int fr = min(l / kLanes, kR - 1);  // row of this lane in the fold
  const int fp = l & (kLanes - 1);    // position of this lane in its row's chain
  float sumf = 0.0f;

  if constexpr (kOneChunk) {
    // one chunk, and every lane owns a whole block pair.  Kept in the form of
    // a loop of one pass: the compiler schedules the straight-line form's
    // loads differently, and that measured slower (us, interleaved runs:
    // 128256 x 4096 50.65 against 47.47, 14336 x 4096 8.09 against 7.94)
    for (size_t c0 = 0; c0 < nb; c0 += kGvChunk) {
      const int b0 = 2 * l;
      uint32_t wr[kR][9];
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        const size_t row = min(row0 + r, nr - 1);  // rows past nr: computed, never stored
        if constexpr (kSoA) {
          const size_t blk = row * nb + c0 + b0;
          const uint4 *q = reinterpret_cast<const uint4 *>(vx + blk * 16);
          const uint4 qa4 = q[0], qb4 = q[1];
          wr[r][0] = qa4.x; wr[r][1] = qa4.y; wr[r][2] = qa4.z; wr[r][3] = qa4.w;
          wr[r][4] = qb4.x; wr[r][5] = qb4.y; wr[r][6] = qb4.z; wr[r][7] = qb4.w;
          wr[r][8] = *reinterpret_cast<const uint32_t *>(vx + nr * nb * 16 + blk * 2);
        } else {
          load36(vx + row * bx + (c0 + b0) * kQ4Bytes, wr[r]);
        }
      }
      ActPair ap;
      load_act_pair(vy + (c0 + b0) * kQ8Bytes, ap);
      dyl[w][b0] = ap.d0;
      dyl[w][b0 + 1] = ap.d1;
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        // block 2l: d = bytes 0-1, quants bytes 2..17 (shift by 2 bytes);
        // block 2l+1: d = bytes 18-19, quants bytes 20..35 (dwords 5..8)
        uint32_t qa[4], qb[4];
        float dx0, dx1;
        if constexpr (kSoA) {  // quants dwords 0-3 and 4-7, the two scales in dword 8
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            qa[k] = wr[r][k];
            qb[k] = wr[r][k + 4];
          }
          dx0 = fp16_bits_to_f32(wr[r][8] & 0xffffu);
          dx1 = fp16_bits_to_f32(wr[r][8] >> 16);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            qa[k] = funnel16(wr[r][k], wr[r][k + 1]);
            qb[k] = wr[r][k + 5];
          }
          dx0 = fp16_bits_to_f32(wr[r][0] & 0xffffu);
          dx1 = fp16_bits_to_f32(wr[r][4] >> 16);
        }
        float2 t;
        t.x = static_cast<float>(nibble_dot(qa, ap.q0, ap.c0)) * dx0;
        t.y = static_cast<float>(nibble_dot(qb, ap.q1, ap.c1)) * dx1;
        *reinterpret_cast<float2 *>(&tl[w][r][b0]) = t;
      }
      wave_lds_sync();  // the LDS rows are this wave's own
      float t[kTerms], dy[kTerms];
#pragma unroll
      for (int k = 0; k < kTerms; k += 4) {
        const float4 tv = *reinterpret_cast<const float4 *>(&tl[w][fr][fp * kTerms + k]);
        const float4 dv = *reinterpret_cast<const float4 *>(&dyl[w][fp * kTerms + k]);
        t[k] = tv.x; t[k + 1] = tv.y; t[k + 2] = tv.z; t[k + 3] = tv.w;
        dy[k] = dv.x; dy[k + 1] = dv.y; dy[k + 2] = dv.z; dy[k + 3] = dv.w;
      }
      sumf = fold_chain<kLanes, kTerms>(t, dy, 0.0f);
    }
  } else {
    const int b0 = 2 * l;

    // this lane's block pair of chunk c0 for the wave's rows (36 bytes each)
    auto load_rows = [&](size_t c0, uint32_t (&wr)[kR][9]) {
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        const size_t row = min(row0 + r, nr - 1);  // rows past nr: computed, never stored
        if constexpr (kSoA) {
          const size_t blk = row * nb + c0 + b0;
          const uint4 *q = reinterpret_cast<const uint4 *>(vx + blk * 16);
          const uint4 qa4 = q[0], qb4 = q[1];
          wr[r][0] = qa4.x; wr[r][1] = qa4.y; wr[r][2] = qa4.z; wr[r][3] = qa4.w;
          wr[r][4] = qb4.x; wr[r][5] = qb4.y; wr[r][6] = qb4.z; wr[r][7] = qb4.w;
          wr[r][8] = *reinterpret_cast<const uint32_t *>(vx + nr * nb * 16 + blk * 2);
        } else {
          load36(vx + row * bx + (c0 + b0) * kQ4Bytes, wr[r]);
        }
      }
    };
    // the terms fl(sumi * d_x) of the pair for every row, and d_y, to the wave's LDS
    auto terms = [&](const uint32_t (&wr)[kR][9], const ActPair &ap) {
      dyl[w][b0] = ap.d0;
      dyl[w][b0 + 1] = ap.d1;
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        // block 2l: d = bytes 0-1, quants bytes 2..17 (shift by 2 bytes);
        // block 2l+1: d = bytes 18-19, quants bytes 20..35 (dwords 5..8)
        uint32_t qa[4], qb[4];
        float dx0, dx1;
        if constexpr (kSoA) {  // quants dwords 0-3 and 4-7, the two scales in dword 8
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            qa[k] = wr[r][k];
            qb[k] = wr[r][k + 4];
          }
          dx0 = fp16_bits_to_f32(wr[r][8] & 0xffffu);
          dx1 = fp16_bits_to_f32(wr[r][8] >> 16);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            qa[k] = funnel16(wr[r][k], wr[r][k + 1]);
            qb[k] = wr[r][k + 5];
          }
          dx0 = fp16_bits_to_f32(wr[r][0] & 0xffffu);
          dx1 = fp16_bits_to_f32(wr[r][4] >> 16);
        }
        float2 t;
        t.x = static_cast<float>(nibble_dot(qa, ap.q0, ap.c0)) * dx0;
        t.y = static_cast<float>(nibble_dot(qb, ap.q1, ap.c1)) * dx1;
        *reinterpret_cast<float2 *>(&tl[w][r][b0]) = t;
      }
    };
    // blocks past the chunk: t = dy = 0, and fma(0, 0, sumf) == sumf (sumf is never -0)
    auto no_terms = [&] {
      dyl[w][b0] = 0.0f;
      dyl[w][b0 + 1] = 0.0f;
#pragma unroll
      for (int r = 0; r < kR; ++r)
        *reinterpret_cast<float2 *>(&tl[w][r][b0]) = make_float2(0.0f, 0.0f);
    };
    // each row's chain over the chunk's terms, seeded with `seed` in lane 0
    auto fold = [&](float seed) {
      wave_lds_sync();  // the LDS rows are this wave's own
      float t[kTerms], dy[kTerms];
#pragma unroll
      for (int k = 0; k < kTerms; k += 4) {
        const float4 tv = *reinterpret_cast<const float4 *>(&tl[w][fr][fp * kTerms + k]);
        const float4 dv = *reinterpret_cast<const float4 *>(&dyl[w][fp * kTerms + k]);
        t[k] = tv.x; t[k + 1] = tv.y; t[k + 2] = tv.z; t[k + 3] = tv.w;
        dy[k] = dv.x; dy[k + 1] = dv.y; dy[k + 2] = dv.z; dy[k + 3] = dv.w;
      }
      return fold_chain<kLanes, kTerms>(t, dy, seed);
    };

    // the loads of chunk c0 + kGvChunk are issued before chunk c0's terms and
    // fold, so a long row's chunks do not wait for each other's loads
    uint32_t wr[kR][9];
    ActPair ap;
    bool have = b0 < static_cast<int>(min(static_cast<size_t>(kGvChunk), nb));
    if (have) {
      load_rows(0, wr);
      load_act_pair(vy + b0 * kQ8Bytes, ap);
    }
    for (size_t c0 = 0; c0 < nb; c0 += kGvChunk) {
      const size_t c1 = c0 + kGvChunk;
      // nbc is even: a lane's pair is whole or absent
      const bool have1 =
          c1 < nb && b0 < static_cast<int>(min(static_cast<size_t>(kGvChunk), nb - c1));
      uint32_t wn[kR][9];
      ActPair an;
      if (have1) {
        load_rows(c1, wn);
        load_act_pair(vy + (c1 + b0) * kQ8Bytes, an);
      }
      if (have)
        terms(wr, ap);
      else
        no_terms();
      // the previous chunk's sum sits in the last lane of the group: seed lane 0
      const float carry = __shfl(sumf, (l & ~(kLanes - 1)) + kLanes - 1);
      sumf = fold(fp == 0 ? carry : 0.0f);
      wave_lds_sync();  // the LDS rows are this wave's own
      if (have1) {
#pragma unroll
        for (int r = 0; r < kR; ++r)
#pragma unroll
          for (int k = 0; k < 9; ++k)
            wr[r][k] = wn[r][k];
        ap = an;
      }
      have = have1;
    }
  }
  if (fp == kLanes - 1 && l / kLanes < kR && row0 + fr < nr)
    s[(row0 + fr) * os] = sumf;
}

// Rows of exactly 128 / kSplit blocks (n = 2048 for kSplit = 2, 1024 for 4):
// the register-direct GEMV with the wave cut into kSplit lane groups, group g
// on rows g*kR .. g*kR + kR - 1 of the wave, lane l owning blocks 2(l % G),
// 2(l % G) + 1 (G = 64 / kSplit lanes a group), so no lane idles (the chunked
// kernel would leave all but the first group without a block).  The kSplit*kR
// rows fold on 64 / (kSplit*kR) lanes each: the same chain per row as the
// chunked kernel, bit for bit.
template <int kWaves, int kR, int kSplit = 2>
__global__ __launch_bounds__(kWaves * 64) void gemv_q4_0_q8_0_half(float *s, size_t os,
                                                                  const uint8_t *vx, size_t bx,
                                                                  const uint8_t *vy, size_t nr) {
  constexpr int kNb = kGvChunk / kSplit;  // blocks a row
  constexpr int kGroup = 64 / kSplit;     // lanes a group
  constexpr int kRows = kSplit * kR;      // rows a wave
  constexpr int kLanes = 64 / kRows;      // fold lanes per row
  constexpr int kTerms = kNb / kLanes;    // blocks per fold lane
  static_assert(kRows * kLanes == 64 && kTerms % 4 == 0 && kLanes <= 16,
                "every lane folds, whole float4 reads, groups inside one DPP row");
  __shared__ __align__(16) float tl[kWaves][kRows][kNb + 4];
  __shared__ __align__(16) float dyl[kWaves][kNb];

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int l = tid & 63;
  const int hw = l / kGroup;            // lane group: rows hw*kR .. hw*kR + kR - 1
  const int b0 = 2 * (l % kGroup);      // this lane's block pair
  const size_t rowb = (static_cast<size_t>(blockIdx.x) * kWaves + w) * kRows;
  const int fr = l / kLanes;     // row of this lane in the fold
  const int fp = l & (kLanes - 1);
  uint32_t wr[kR][9];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const size_t row = min(rowb + hw * kR + r, nr - 1);  // rows past nr: computed, never stored
    load36(vx + row * bx + b0 * kQ4Bytes, wr[r]);
  }
  ActPair ap;
  load_act_pair(vy + b0 * kQ8Bytes, ap);
  if (hw == 0) {
    dyl[w][b0] = ap.d0;
    dyl[w][b0 + 1] = ap.d1;
  }
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    // block 2l: d = bytes 0-1, quants bytes 2..17; block 2l+1: d = bytes 18-19,
    // quants bytes 20..35 (dwords 5..8)
    uint32_t qa[4], qb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      qa[k] = funnel16(wr[r][k], wr[r][k + 1]);
      qb[k] = wr[r][k + 5];
    }
    const float dx0 = fp16_bits_to_f32(wr[r][0] & 0xffffu);
    const float dx1 = fp16_bits_to_f32(wr[r][4] >> 16);
    float2 t;
    t.x = static_cast<float>(nibble_dot(qa, ap.q0, ap.c0)) * dx0;
    t.y = static_cast<float>(nibble_dot(qb, ap.q1, ap.c1)) * dx1;
    *reinterpret_cast<float2 *>(&tl[w][hw * kR + r][b0]) = t;
  }
  wave_lds_sync();  // the LDS rows are this wave's own
  float t[kTerms], dy[kTerms];
#pragma unroll
  for (int k = 0; k < kTerms; k += 4) {
    const float4 tv = *reinterpret_cast<const float4 *>(&tl[w][fr][fp * kTerms + k]);
    const float4 dv = *reinterpret_cast<const float4 *>(&dyl[w][fp * kTerms + k]);
    t[k] = tv.x; t[k + 1] = tv.y; t[k + 2] = tv.z; t[k + 3] = tv.w;
    dy[k] = dv.x; dy[k + 1] = dv.y; dy[k + 2] = dv.z; dy[k + 3] = dv.w;
  }
  const float sumf = fold_chain<kLanes, kTerms>(t, dy, 0.0f);
  if (fp == kLanes - 1 && rowb + fr < nr)
    s[(rowb + fr) * os] = sumf;
}

// Multi-column form of the register-direct GEMV, for the a7 GEMM with a few
// tokens (batched decode, nc = 2..kGemvColsMax): each wave loads its 4 weight
// rows' block pairs once and dots them with kCols activation columns (ncols of
// them present; absent ones re-read the last and are not stored).  Per (row,
// column) the terms fl((float)sumi * d_x) and the column's d_y go through the
// wave's LDS and fold on 64 / (4 kCols) lanes -- one chain per row and column,
// 128 fmas in ascending block order, as the GEMV's.
template <int kCols, bool kOneChunk>
__global__ __launch_bounds__(256) void gemv_q4_0_q8_0_cols(size_t nb_arg, float *s, size_t bs,
                                                           const uint8_t *vx, size_t bx,
                                                           const uint8_t *vy, size_t by,
                                                           size_t nr, int ncols) {
  constexpr int kWaves = 4, kR = 4;
  constexpr int kChains = kR * kCols;
  constexpr int kLanes = 64 / kChains;       // 8 lanes for 2 columns, 4 for 4, 2 for 8
  constexpr int kTerms = kGvChunk / kLanes;  // blocks per fold lane
  static_assert(kLanes == 8 || kLanes == 4 || kLanes == 2, "fold groups inside one DPP row");
  const size_t nb = kOneChunk ? static_cast<size_t>(kGvChunk) : nb_arg;
  __shared__ __align__(16) float tl[kWaves][kChains][kGvChunk + 4];
  __shared__ __align__(16) float dyl[kWaves][kCols][kGvChunk];

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int l = tid & 63;
  const size_t row0 = (static_cast<size_t>(blockIdx.x) * kWaves + w) * kR;
  const int ch = l / kLanes;                  // chain: row ch / kCols, column ch % kCols
  const int fr = ch / kCols, fc = ch % kCols;
  const int fp = l & (kLanes - 1);            // position of this lane in its chain
  float sumf = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kGvChunk) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kGvChunk), nb - c0));
    const int b0 = 2 * l;
    if (kOneChunk || b0 < nbc) {  // nbc is even: the pair is whole or absent
      uint32_t wr[kR][9];
#pragma unroll
      for (int r = 0; r < kR; ++r)
        load36(vx + min(row0 + r, nr - 1) * bx + (c0 + b0) * kQ4Bytes, wr[r]);
      ActPair ap[kCols];
#pragma unroll
      for (int c = 0; c < kCols; ++c) {
        load_act_pair(vy + static_cast<size_t>(min(c, ncols - 1)) * by + (c0 + b0) * kQ8Bytes,
                      ap[c]);
        dyl[w][c][b0] = ap[c].d0;
        dyl[w][c][b0 + 1] = ap[c].d1;
      }
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        // block 2l: d = bytes 0-1, quants bytes 2..17; block 2l+1: d = bytes
        // 18-19, quants bytes 20..35 (dwords 5..8)
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          qa[k] = funnel16(wr[r][k], wr[r][k + 1]);
          qb[k] = wr[r][k + 5];
        }
        const float dx0 = fp16_bits_to_f32(wr[r][0] & 0xffffu);
        const float dx1 = fp16_bits_to_f32(wr[r][4] >> 16);
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
          float2 t;
          t.x = static_cast<float>(nibble_dot(qa, ap[c].q0, ap[c].c0)) * dx0;
          t.y = static_cast<float>(nibble_dot(qb, ap[c].q1, ap[c].c1)) * dx1;
          *reinterpret_cast<float2 *>(&tl[w][r * kCols + c][b0]) = t;
        }
      }
    } else {
      // blocks past the chunk: t = dy = 0, and fma(0, 0, sumf) == sumf (sumf is never -0)
#pragma unroll
      for (int c = 0; c < kCols; ++c) {
        dyl[w][c][b0] = 0.0f;
        dyl[w][c][b0 + 1] = 0.0f;
      }
#pragma unroll
      for (int q = 0; q < kChains; ++q)
        *reinterpret_cast<float2 *>(&tl[w][q][b0]) = make_float2(0.0f, 0.0f);
    }
    wave_lds_sync();  // the LDS rows are this wave's own
    float t[kTerms], dy[kTerms];
#pragma unroll
    for (int k = 0; k < kTerms; k += 4) {
      const float4 tv = *reinterpret_cast<const float4 *>(&tl[w][ch][fp * kTerms + k]);
      const float4 dv = *reinterpret_cast<const float4 *>(&dyl[w][fc][fp * kTerms + k]);
      t[k] = tv.x; t[k + 1] = tv.y; t[k + 2] = tv.z; t[k + 3] = tv.w;
      dy[k] = dv.x; dy[k + 1] = dv.y; dy[k + 2] = dv.z; dy[k + 3] = dv.w;
    }
    if constexpr (kOneChunk) {
      sumf = fold_chain<kLanes, kTerms>(t, dy, 0.0f);
    } else {
      // the previous chunk's sum sits in the last lane of the chain: seed lane 0
      const float carry = __shfl(sumf, (l & ~(kLanes - 1)) + kLanes - 1);
      sumf = fold_chain<kLanes, kTerms>(t, dy, fp == 0 ? carry : 0.0f);
      wave_lds_sync();  // the LDS rows are this wave's own
    }
  }
  if (fp == kLanes - 1 && row0 + fr < nr && fc < ncols)
    s[(row0 + fr) * bs + fc] = sumf;
}

// Q8_0 block pair 2l, 2l+1 (68 bytes, dword aligned) -> quants of each block as
// 8 aligned dwords and the fp32 scales.
struct Q8Pair {
  uint32_t q0[8], q1[8];
  float d0, d1;
};

__device__ __forceinline__ void load_q8_pair(const uint8_t *p, Q8Pair &a) {
  const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
  uint32_t r[17];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(q + 4 * k);
    r[4 * k + 0] = v.x; r[4 * k + 1] = v.y; r[4 * k + 2] = v.z; r[4 * k + 3] = v.w;
  }
  r[16] = q[16];
  a.d0 = fp16_bits_to_f32(r[0] & 0xffffu);
  a.d1 = fp16_bits_to_f32(r[8] >> 16);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    a.q0[k] = funnel16(r[k], r[k + 1]);
    a.q1[k] = r[k + 9];
  }
}

// The a9 (Q8_0 x Q8_0) GEMM with a few tokens, as gemv_q4_0_q8_0_cols: each
// wave loads its 4 weight rows' block pairs once and dots them with kCols
// activation columns; the a5 fold of each (row, column) is fma((float)sumi,
// d_x * d_y, acc) with the scale product exact in fp32, so (float)sumi and
// d_x * d_y go through the wave's LDS and fold on 64 / (4 kCols) lanes in
// ascending block order.
template <int kCols, bool kOneChunk>
__global__ __launch_bounds__(256) void gemv_q8_0_q8_0_cols(size_t nb_arg, float *s, size_t bs,
                                                           const uint8_t *vx, size_t bx,
                                                           const uint8_t *vy, size_t by,
                                                           size_t nr, int ncols) {
  constexpr int kWaves = 4, kR = 4;
  constexpr int kChains = kR * kCols;
  constexpr int kLanes = 64 / kChains;       // 8 lanes for 2 columns, 4 for 4, 2 for 8
  constexpr int kTerms = kGvChunk / kLanes;  // blocks per fold lane
  static_assert(kLanes == 8 || kLanes == 4 || kLanes == 2, "fold groups inside one DPP row");
  const size_t nb = kOneChunk ? static_cast<size_t>(kGvChunk) : nb_arg;
  __shared__ __align__(16) float2 tl[kWaves][kChains][kGvChunk + 2];  // ((float)sumi, d_x*d_y)

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int l = tid & 63;
  const size_t row0 = (static_cast<size_t>(blockIdx.x) * kWaves + w) * kR;
  const int ch = l / kLanes;                  // chain: row ch / kCols, column ch % kCols
  const int fr = ch / kCols, fc = ch % kCols;
  const int fp = l & (kLanes - 1);            // position of this lane in its chain
  float sumf = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kGvChunk) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kGvChunk), nb - c0));
    const int b0 = 2 * l;
    if (kOneChunk || b0 < nbc) {  // nbc is even: the pair is whole or absent
      Q8Pair wp[kR], ap[kCols];
#pragma unroll
      for (int r = 0; r < kR; ++r)
        load_q8_pair(vx + min(row0 + r, nr - 1) * bx + (c0 + b0) * kQ8Bytes, wp[r]);
#pragma unroll
      for (int c = 0; c < kCols; ++c)
        load_q8_pair(vy + static_cast<size_t>(min(c, ncols - 1)) * by + (c0 + b0) * kQ8Bytes,
                     ap[c]);
#pragma unroll
      for (int r = 0; r < kR; ++r)
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
          int s0 = 0, s1 = 0;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            s0 = sdot4(wp[r].q0[k], ap[c].q0[k], s0);
            s1 = sdot4(wp[r].q1[k], ap[c].q1[k], s1);
          }
          *reinterpret_cast<float4 *>(&tl[w][r * kCols + c][b0]) =
              make_float4(static_cast<float>(s0), wp[r].d0 * ap[c].d0, static_cast<float>(s1),
                          wp[r].d1 * ap[c].d1);
        }
    } else {
      // blocks past the chunk: fma(0, 0, sumf) == sumf (sumf is never -0)
#pragma unroll
      for (int q = 0; q < kChains; ++q)
        *reinterpret_cast<float4 *>(&tl[w][q][b0]) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    wave_lds_sync();  // the LDS rows are this wave's own
    float t[kTerms], dxy[kTerms];
#pragma unroll
    for (int k = 0; k < kTerms; k += 2) {
      const float4 v = *reinterpret_cast<const float4 *>(&tl[w][ch][fp * kTerms + k]);
      t[k] = v.x; dxy[k] = v.y; t[k + 1] = v.z; dxy[k + 1] = v.w;
    }
    if constexpr (kOneChunk) {
      sumf = fold_chain<kLanes, kTerms>(t, dxy, 0.0f);
    } else {
      // the previous chunk's sum sits in the last lane of the chain: seed lane 0
      const float carry = __shfl(sumf, (l & ~(kLanes - 1)) + kLanes - 1);
      sumf = fold_chain<kLanes, kTerms>(t, dxy, fp == 0 ? carry : 0.0f);
      wave_lds_sync();  // the LDS rows are this wave's own
    }
  }
  if (fp == kLanes - 1 && row0 + fr < nr && fc < ncols)
    s[(row0 + fr) * bs + fc] = sumf;
}

}  // namespace tcrv

namespace tcrv_host {

// Rows per wave of the LDS-staged decode GEMV (odd nb or 2-byte aligned rows).
constexpr int kGemvRows = 2;
// Shape of the register-direct GEMV: waves per work-group, rows per wave
// (4096^2, us: 1x4 4.16, 2x4 4.46, 4x4 4.00, 8x2 4.13, 8x4 5.06, 2x8 4.80, 4x2 4.28).
constexpr int kDirectWaves = 4;
constexpr int kDirectRows = 4;
// Up to this many rows the shape-free entries run two rows per wave: four
// leave too few work-groups to cover the chip (us, 2 against 4 rows per wave:
// 256 x 4096 2.52/2.95, 1024 x 4096 2.70/3.07, 2048 x 4096 3.08/3.25,
// 1024 x 14336 7.53/8.28; past it, 3072 x 4096 3.80/3.37, 4096^2 3.94/3.70).
constexpr size_t kDirectSmallRows = 2048;
inline int direct_rows(size_t nr) { return nr <= kDirectSmallRows ? 2 : kDirectRows; }

// Rows of 64 blocks (n = 2048) run the half-wave kernel: with 8 rows per wave
// from this many rows, where its work-groups fill the chip (us, against the
// chunked kernel: 8192 rows 4.06/4.25, 11008 rows 4.92/5.58; at 4096 rows
// 3.62/3.32), else with 4 rows per wave, as many work-groups as the chunked
// kernel (2560 rows 2.95/3.11, 4096 rows 3.20/3.33, 5632 rows 3.77/4.10).
constexpr size_t kHalfMinRows = 8192;
// Rows of 32 blocks (n = 1024) run it with four lane groups, 2 rows each (us,
// against the chunked kernel: 2560 rows 2.65/2.96, 4096 rows 2.75/3.07, 8192
// rows 3.10/3.93, 14336 rows 3.75/6.35).

// The register-direct GEMV with kR rows per wave (kDirectWaves waves per
// work-group); every shape computes the same per-row fold, bit for bit.
template <int kR>
int launch_direct(size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx,
                  const uint8_t *vy, size_t nr, hipStream_t st) {
  constexpr int kW = kDirectWaves;
  const size_t rows_per_wg = static_cast<size_t>(kW) * kR;
  const size_t grid = (nr + rows_per_wg - 1) / rows_per_wg;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (nb == static_cast<size_t>(tcrv::kGvChunk))
    tcrv::gemv_q4_0_q8_0_direct<kW, kR, true>
        <<<dim3(static_cast<unsigned>(grid)), dim3(kW * 64), 0, st>>>(nb, s, os, vx, bx, vy, nr);
  else if (kR == 4 && nb == static_cast<size_t>(tcrv::kGvChunk / 2) && nr >= kHalfMinRows) {
    const size_t grid_half = (nr + 2 * rows_per_wg - 1) / (2 * rows_per_wg);
    tcrv::gemv_q4_0_q8_0_half<kW, 4>
        <<<dim3(static_cast<unsigned>(grid_half)), dim3(kW * 64), 0, st>>>(s, os, vx, bx, vy, nr);
  } else if (kR == 4 && nb == static_cast<size_t>(tcrv::kGvChunk / 2)) {
    tcrv::gemv_q4_0_q8_0_half<kW, 2>
        <<<dim3(static_cast<unsigned>(grid)), dim3(kW * 64), 0, st>>>(s, os, vx, bx, vy, nr);
  } else if (kR == 4 && nb == static_cast<size_t>(tcrv::kGvChunk / 4)) {
    const size_t grid_q = (nr + 2 * rows_per_wg - 1) / (2 * rows_per_wg);  // 8 rows a wave
    tcrv::gemv_q4_0_q8_0_half<kW, 2, 4>
        <<<dim3(static_cast<unsigned>(grid_q)), dim3(kW * 64), 0, st>>>(s, os, vx, bx, vy, nr);
  } else
    tcrv::gemv_q4_0_q8_0_direct<kW, kR, false>
        <<<dim3(static_cast<unsigned>(grid)), dim3(kW * 64), 0, st>>>(nb, s, os, vx, bx, vy, nr);
  return launch_status();
}

int gemv_q4_0_q8_0(size_t n, float *s, size_t os, const uint8_t *vx, size_t bx,
                   const uint8_t *vy, size_t nr, void *stream, int rows_per_wave) {
  const size_t nb = n / tcrv::kQK;
  if (nr == 0)
    return TCRV_HIP_OK;
  if (!s || !vx || !vy)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(vx) || !aligned2(vy) || (nr > 1 && (bx & 1u)))
    return TCRV_HIP_ERR_MISALIGNED;
  if (nb == 0)
    return TCRV_HIP_ERR_BAD_SIZE;  // handled by the caller (zero fill)
  if (nr > 1 && bx < nb * tcrv::kQ4Bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  hipStream_t st = as_stream(stream);
  if (nb % 2 == 0 && aligned4(vx) && aligned4(vy) && (nr == 1 || bx % 4 == 0)) {
    switch (rows_per_wave) {
    case 2: return launch_direct<2>(nb, s, os, vx, bx, vy, nr, st);
    case 8: return launch_direct<8>(nb, s, os, vx, bx, vy, nr, st);
    default: return launch_direct<kDirectRows>(nb, s, os, vx, bx, vy, nr, st);
    }
  }
  const size_t rows_per_wg = static_cast<size_t>(tcrv::kGvWaves) * kGemvRows;
  const size_t grid = (nr + rows_per_wg - 1) / rows_per_wg;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::gemv_q4_0_q8_0_kernel<kGemvRows>
      <<<dim3(static_cast<unsigned>(grid)), dim3(tcrv::kGvWaves * 64), 0, st>>>(
          nb, s, os, vx, bx, vy, nr);
  return launch_status();
}

template <bool kQ4, int kCols>
int launch_cols(size_t nb, float *s, size_t bs, const uint8_t *vx, size_t bx, const uint8_t *vy,
                size_t by, size_t nr, int ncols, hipStream_t st) {
  const size_t grid = (nr + 15) / 16;  // 4 waves x 4 rows
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  const dim3 g(static_cast<unsigned>(grid)), b(256);
  const bool one = nb == static_cast<size_t>(tcrv::kGvChunk);
  if constexpr (kQ4) {
    if (one)
      tcrv::gemv_q4_0_q8_0_cols<kCols, true><<<g, b, 0, st>>>(nb, s, bs, vx, bx, vy, by, nr, ncols);
    else
      tcrv::gemv_q4_0_q8_0_cols<kCols, false><<<g, b, 0, st>>>(nb, s, bs, vx, bx, vy, by, nr, ncols);
  } else {
    if (one)
      tcrv::gemv_q8_0_q8_0_cols<kCols, true><<<g, b, 0, st>>>(nb, s, bs, vx, bx, vy, by, nr, ncols);
    else
      tcrv::gemv_q8_0_q8_0_cols<kCols, false><<<g, b, 0, st>>>(nb, s, bs, vx, bx, vy, by, nr, ncols);
  }
  return launch_status();
}

// Columns in groups: eight while five or more are left (five to seven present
// in the last), then four (three or four present), two, and a single column
// through the decode GEMV (Q4_0) or the block dots (Q8_0).
template <bool kQ4>
int gemv_cols(size_t nb, float *s, size_t bs, const uint8_t *vx, size_t bx, const uint8_t *vy,
              size_t by, size_t nr, size_t nc, void *stream) {
  if (nb % 2 != 0 || !aligned4(vx) || !aligned4(vy) || (nr > 1 && bx % 4 != 0) || by % 4 != 0)
    return TCRV_HIP_ERR_UNSUPPORTED;
  hipStream_t st = as_stream(stream);
  for (size_t c0 = 0; c0 < nc;) {
    const size_t rem = nc - c0;
    float *sc = s + c0;
    const uint8_t *yc = vy + c0 * by;
    const size_t take = rem >= 5 ? (rem < 8 ? rem : 8) : rem;  // rem <= 4: one last group
    int rc;
    if (rem >= 5)
      rc = launch_cols<kQ4, 8>(nb, sc, bs, vx, bx, yc, by, nr, static_cast<int>(take), st);
    else if (rem >= 3)
      rc = launch_cols<kQ4, 4>(nb, sc, bs, vx, bx, yc, by, nr, static_cast<int>(take), st);
    else if (rem == 2)
      rc = launch_cols<kQ4, 2>(nb, sc, bs, vx, bx, yc, by, nr, 2, st);
    else if constexpr (kQ4)
      rc = nr <= kDirectSmallRows ? launch_direct<2>(nb, sc, bs, vx, bx, yc, nr, st)
                                  : launch_direct<kDirectRows>(nb, sc, bs, vx, bx, yc, nr, st);
    else
      rc = q8_0_rows_direct(nb, sc, bs, vx, bx, yc, 0, nr, stream);
    if (rc != TCRV_HIP_OK)
      return rc;
    c0 += take;
  }
  return TCRV_HIP_OK;
}

int gemv_cols_q4_0_q8_0(size_t nb, float *s, size_t bs, const uint8_t *vx, size_t bx,
                        const uint8_t *vy, size_t by, size_t nr, size_t nc, void *stream) {
  return gemv_cols<true>(nb, s, bs, vx, bx, vy, by, nr, nc, stream);
}

int gemv_cols_q8_0_q8_0(size_t nb, float *s, size_t bs, const uint8_t *vx, size_t bx,
                        const uint8_t *vy, size_t by, size_t nr, size_t nc, void *stream) {
  return gemv_cols<false>(nb, s, bs, vx, bx, vy, by, nr, nc, stream);
}

int gemv_q4_0_soa_q8_0(size_t nb, float *s, const uint8_t *vx, const uint8_t *vy, size_t nr,
                       void *stream) {
  if (!s || !vx || !vy)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (nb % 2 != 0)
    return TCRV_HIP_ERR_UNSUPPORTED;  // a lane owns whole block pairs
  if (!aligned16(vx) || !aligned4(vy))
    return TCRV_HIP_ERR_MISALIGNED;
  constexpr int kW = kDirectWaves, kR = kDirectRows;
  const size_t rows_per_wg = static_cast<size_t>(kW) * kR;
  const size_t grid = (nr + rows_per_wg - 1) / rows_per_wg;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  hipStream_t st = as_stream(stream);
  if (nb == static_cast<size_t>(tcrv::kGvChunk))
    tcrv::gemv_q4_0_q8_0_direct<kW, kR, true, true>
        <<<dim3(static_cast<unsigned>(grid)), dim3(kW * 64), 0, st>>>(nb, s, 1, vx, 0, vy, nr);
  else
    tcrv::gemv_q4_0_q8_0_direct<kW, kR, false, true>
        <<<dim3(static_cast<unsigned>(grid)), dim3(kW * 64), 0, st>>>(nb, s, 1, vx, 0, vy, nr);
  return launch_status();
}

}  // namespace tcrv_host

namespace tcrv {

// Q4_0 rows -> the split layout: thread t moves block t (row t / nb, block
// t % nb): its 16 quant bytes to (t*16) and its fp16 scale to nr*nb*16 + t*2.
__global__ __launch_bounds__(256) void pack_q4_0_soa(size_t nrows, size_t nb, const uint8_t *src,
                                                     size_t bx, uint8_t *dst) {
  const size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= nrows * nb)
    return;
  const size_t r = t / nb, b = t - r * nb;
  const uint16_t *blk = reinterpret_cast<const uint16_t *>(src + r * bx + b * kQ4Bytes);
  uint32_t q[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    q[k] = static_cast<uint32_t>(blk[1 + 2 * k]) | (static_cast<uint32_t>(blk[2 + 2 * k]) << 16);
  reinterpret_cast<uint4 *>(dst)[t] = make_uint4(q[0], q[1], q[2], q[3]);
  reinterpret_cast<uint16_t *>(dst + nrows * nb * 16)[t] = blk[0];
}

}  // namespace tcrv

extern "C" {

int tcrv_hip_pack_q4_0_to_soa(size_t nrows, size_t nb, const uint8_t *src, size_t bx,
                              uint8_t *dst, void *stream) {
  using namespace tcrv_host;
  if (nrows == 0 || nb == 0)
    return TCRV_HIP_OK;
  if (!src || !dst)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(src) || (nrows > 1 && (bx & 1u)) || !aligned16(dst))
    return TCRV_HIP_ERR_MISALIGNED;
  if (nrows > 1 && bx < nb * tcrv::kQ4Bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  const size_t grid = (nrows * nb + 255) / 256;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::pack_q4_0_soa<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, as_stream(stream)>>>(
      nrows, nb, src, bx, dst);
  return launch_status();
}

int tcrv_hip_gemv_q4_0_soa_q8_0(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                size_t nr, void *stream) {
  if (nr == 0)
    return TCRV_HIP_OK;
  if (n / tcrv::kQK == 0)
    return tcrv_host::zero_outputs(s, nr, 1, 1, stream);
  return tcrv_host::gemv_q4_0_soa_q8_0(n / tcrv::kQK, s, vx, vy, nr, stream);
}

int tcrv_hip_gemv_q4_0_q8_0(size_t n, float *s, const uint8_t *vx, size_t bx,
                            const uint8_t *vy, size_t nr, void *stream) {
  if (nr == 0)
    return TCRV_HIP_OK;
  if (n / tcrv::kQK == 0)
    return tcrv_host::zero_outputs(s, nr, 1, 1, stream);
  return tcrv_host::gemv_q4_0_q8_0(n, s, 1, vx, bx, vy, nr, stream, tcrv_host::direct_rows(nr));
}

int tcrv_hip_gemv_q4_0_q8_0_shaped(size_t n, float *s, const uint8_t *vx, size_t bx,
                                   const uint8_t *vy, size_t nr, int rows_per_wave,
                                   void *stream) {
  if (rows_per_wave != 2 && rows_per_wave != 4 && rows_per_wave != 8)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (nr == 0)
    return TCRV_HIP_OK;
  if (n / tcrv::kQK == 0)
    return tcrv_host::zero_outputs(s, nr, 1, 1, stream);
  return tcrv_host::gemv_q4_0_q8_0(n, s, 1, vx, bx, vy, nr, stream, rows_per_wave);
}

int tcrv_hip_q4_0_q8_0_gemm(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                            size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                            void *stream) {
  if (nr == 0 || nc == 0)
    return TCRV_HIP_OK;
  if (nr > 1 && bs < nc)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (n / tcrv::kQK == 0)
    return tcrv_host::zero_outputs(s, nr * nc, bs, nc, stream);
  if (nc == 1)
    return tcrv_host::gemv_q4_0_q8_0(n, s, bs, vx, bx, vy, nr, stream, tcrv_host::direct_rows(nr));
  if (!s || !vx || !vy)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!tcrv_host::aligned2(vx) || !tcrv_host::aligned2(vy) || (nr > 1 && (bx & 1u)) || (by & 1u))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t nb = n / tcrv::kQK;
  if ((nr > 1 && bx < nb * tcrv::kQ4Bytes) || by < nb * tcrv::kQ8Bytes)
    return TCRV_HIP_ERR_BAD_SIZE;
  if (nr == 1) {  // one weight row against nc columns: bandwidth-bound block dots
    const int st = tcrv_host::q4_0_rows_direct(nb, s, 1, vx, 0, vy, by, nc, stream);
    if (st != TCRV_HIP_ERR_UNSUPPORTED)
      return st;
  } else {
    if (!tcrv_host::cols_first(nr, nc)) {  // few output tiles: one 32 x 32 tile a wave
      const int st = tcrv_host::gemm_rows_few(true, nb, s, vx, bx, vy, by, nr, nc, bs, stream);
      if (st != TCRV_HIP_ERR_UNSUPPORTED)
        return st;
    }
    if (nc <= tcrv_host::kGemvColsMax) {
      // a few tokens: the weights are read once per group of up to eight
      // columns (the MFMA GEMM would run only nr / 256 work-groups)
      const int st = tcrv_host::gemv_cols_q4_0_q8_0(nb, s, bs, vx, bx, vy, by, nr, nc, stream);
      if (st != TCRV_HIP_ERR_UNSUPPORTED)
        return st;
    }
  }
  const int st = tcrv_host::q4_0_gemm_mfma(nb, s, vx, bx, vy, by, nr, nc, bs, stream);
  if (st != TCRV_HIP_ERR_UNSUPPORTED)
    return st;
  return tcrv_host::q4_0_grid(n, s, vx, bx, vy, by, nr, nc, bs, stream);
}

int tcrv_hip_q4_0_q8_0_gemm_tile(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                 size_t by, size_t m, void *stream) {
  // one weight row times m activation columns, outputs s[0..m-1] contiguous:
  // the G2 GEMM with nr = 1 (its bx and bs are then unused)
  return tcrv_hip_q4_0_q8_0_gemm(n, s, vx, vy, by, 1, m, 0, m, stream);
}

}  // extern "C"
