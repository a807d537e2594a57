// gemm.hip -- a9: Q8_0 x Q8_0 prefill GEMM on v_mfma_i32_32x32x32_i8.
//
// Semantics (the reference's GEMM loop nest, RVVToEmitCBlockQuantLinear.cpp:
// 1691-2121, with the Q8_0 block dot of :7264-7671 as the element):
//   s[ir*bs + col] = sum over blocks b ascending of
//                    fma((float)sumi(ir,col,b), d_x(ir,b)*d_y(col,b), .)
// where x = weight rows (vx, stride bx) and y = activation rows (vy, stride by).
//
// Mapping: K = 32 of the MFMA is exactly one Q8_0 block, so every MFMA yields
// the int32 block sums of a 32x32 output tile for one block; the fp32 fold of
// that block is applied to the tile right away, in ascending block order, so
// every output element sees the reference's sequence of roundings.
//   work-group: 128 weight rows x 128 activation rows, 4 waves as 2x2, each
//               wave 2x2 MFMA tiles (64x64 outputs);
//   K loop:     chunks of 8 blocks (272 B per row, 17 x 128-bit loads) staged
//               through LDS; the fp16 scales are widened once per chunk into
//               fp32 LDS arrays.
#include "tcrv_hip_internal.h"

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
// The fast path.  Per 32x32 output tile and Q8_0 block b:
//   v_mfma_i32_32x32x32_i8   -> sumi(row, col, b) for the tile (K = one block)
//   v_mfma_f32_32x32x16_f16  -> dx(row, b) * dy(col, b) for the tile: the A
//                               operand carries dx in k-slot 0 only, the B
//                               operand dy in k-slot 0 only, so the product is
//                               a rank-1 outer product, exact in fp32 (two
//                               11-bit significands)
//   VALU: acc = fma((float)sumi, dxy, acc)   -- the reference fold, in order.
// Staging splits each 34-byte block into its 32 quants (row-major, 16-byte
// aligned, row stride 272 bytes so 16-byte LDS reads of 32 consecutive rows hit
// distinct banks) and its fp16 scale.
// Work-group: 128 weight rows x 128 activation rows, 4 waves as 2x2, each wave
// 2x2 tiles of 32x32; K chunk of kFbKB blocks, single-buffered, two
// work-groups per CU overlap one's staging with the other's MFMAs.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kFbBM = 128;
constexpr int kFbBN = 128;
constexpr int kFbKB = 8;                      // blocks per K chunk
constexpr int kFbQRow = kFbKB * kQK + 16;     // 272: quant bytes per staged row (+16 pad)
constexpr int kFbThreads = 256;

// Splits one staged block pair (68 bytes, dword aligned, at q) of one row into
// LDS: quants of blocks 2m and 2m+1 at qrow[64m..64m+63], fp16 scales into
// drow[2m*stride], drow[(2m+1)*stride].  `two` == false: only block 2m exists
// (34 bytes are read).
__device__ __forceinline__ void stage_pair(const uint8_t *q, bool two, int8_t *qrow,
                                           uint16_t *d0, uint16_t *d1) {
  const uint32_t *g = reinterpret_cast<const uint32_t *>(q);
  uint32_t r[17];
  if (two) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(g + 4 * k);
      r[4 * k + 0] = v.x; r[4 * k + 1] = v.y; r[4 * k + 2] = v.z; r[4 * k + 3] = v.w;
    }
    r[16] = g[16];
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(g + 4 * k);
      r[4 * k + 0] = v.x; r[4 * k + 1] = v.y; r[4 * k + 2] = v.z; r[4 * k + 3] = v.w;
    }
    r[8] = *reinterpret_cast<const uint16_t *>(q + 32);  // bytes 32-33: last two quants
#pragma unroll
    for (int k = 9; k < 17; ++k)
      r[k] = 0;
  }
  uint4 *dst = reinterpret_cast<uint4 *>(qrow);
  dst[0] = make_uint4(funnel16(r[0], r[1]), funnel16(r[1], r[2]), funnel16(r[2], r[3]),
                      funnel16(r[3], r[4]));
  dst[1] = make_uint4(funnel16(r[4], r[5]), funnel16(r[5], r[6]), funnel16(r[6], r[7]),
                      funnel16(r[7], r[8]));
  *d0 = static_cast<uint16_t>(r[0] & 0xffffu);
  if (two) {
    dst[2] = make_uint4(r[9], r[10], r[11], r[12]);
    dst[3] = make_uint4(r[13], r[14], r[15], r[16]);
    *d1 = static_cast<uint16_t>(r[8] >> 16);
  }
}

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

// One block's MFMA operands for a wave's 2x2 tiles: int8 quants of the two
// 32-row weight tiles and two 32-row activation tiles, and the fp16 scales as
// k-slot 0 of 4-element f16 operands (every other k-slot, and every slot of
// lanes 32..63, is zero), so the f16 MFMA yields the outer product dx*dy.
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

struct Frags {
  v4i a[2], b[2];
  v2i ax[2], by[2];
};

struct TileOut {
  v16i sumi;
  v16f dxy;
};

__device__ __forceinline__ void read_frags(Frags &f, const int8_t *qa, const int8_t *qb,
                                           const uint16_t (*da)[kFbBM],
                                           const uint16_t (*db)[kFbBN], int b, int wm, int wn,
                                           int li, int h) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = wm * 64 + i * 32 + li;
    f.a[i] = *reinterpret_cast<const v4i *>(qa + r * kFbQRow + b * kQK + 16 * h);
    const uint32_t d = da[b][r];
    f.ax[i] = v2i{h == 0 ? static_cast<int>(d) : 0, 0};
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = wn * 64 + j * 32 + li;
    f.b[j] = *reinterpret_cast<const v4i *>(qb + c * kFbQRow + b * kQK + 16 * h);
    const uint32_t d = db[b][c];
    f.by[j] = v2i{h == 0 ? static_cast<int>(d) : 0, 0};
  }
}

__device__ __forceinline__ void mfma_tile(TileOut &o, const Frags &f, int i, int j) {
  const v16i izero = {};
  const v16f fzero = {};
  o.sumi = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[i], f.b[j], izero, 0, 0, 0);
  o.dxy = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, f.ax[i]),
                                               __builtin_bit_cast(v4h, f.by[j]), fzero, 0, 0, 0);
}

// The reference fold for one block of one tile: acc = fma((float)sumi, dx*dy, acc).
__device__ __forceinline__ void fold_tile(float acc[16], const TileOut &o) {
#pragma unroll
  for (int e = 0; e < 16; ++e)
    acc[e] = fmaf(static_cast<float>(o.sumi[e]), o.dxy[e], acc[e]);
}

// Orders one pipeline step as: both MFMAs of the new tile, then the 32 VALU
// ops (16 cvt + 16 fma) of the previous tile's fold, which no longer waits on
// an MFMA issued in this step.
__device__ __forceinline__ void step_order() {
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // MFMA
  __builtin_amdgcn_sched_group_barrier(0x002, 32, 0);  // VALU
  __builtin_amdgcn_sched_barrier(0);
}

// One block for the wave's four tiles; `pend` carries tile (1,1) between
// blocks.  Each step issues a tile's MFMA pair and folds the tile issued one
// step earlier.
__device__ __forceinline__ void gemm_block(float (&acc)[2][2][16], TileOut &pend,
                                           const Frags &f) {
  TileOut t0, t1;
  mfma_tile(t0, f, 0, 0);
  fold_tile(acc[1][1], pend);
  step_order();
  mfma_tile(t1, f, 0, 1);
  fold_tile(acc[0][0], t0);
  step_order();
  mfma_tile(t0, f, 1, 0);
  fold_tile(acc[0][1], t1);
  step_order();
  mfma_tile(pend, f, 1, 1);
  fold_tile(acc[1][0], t0);
  step_order();
}

__global__ __launch_bounds__(kFbThreads, 2) void gemm_q8_0_q8_0_mfma(
    size_t nb, float *s, const uint8_t *vx, const uint8_t *vy, size_t by, size_t nr,
    size_t nc, size_t bx, size_t bs) {
  __shared__ __align__(16) int8_t qa[kFbBM * kFbQRow];
  __shared__ __align__(16) int8_t qb[kFbBN * kFbQRow];
  __shared__ __align__(16) uint16_t da[kFbKB][kFbBM];
  __shared__ __align__(16) uint16_t db[kFbKB][kFbBN];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, h = lane >> 5;
  const unsigned tiles_m = static_cast<unsigned>((nr + kFbBM - 1) / kFbBM);
  const unsigned tiles_n = static_cast<unsigned>((nc + kFbBN - 1) / kFbBN);
  unsigned tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const size_t m0 = static_cast<size_t>(tm) * kFbBM;
  const size_t n0 = static_cast<size_t>(tn) * kFbBN;

  float acc[2][2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[i][j][e] = 0.0f;

  // Results of the last tile of the previous block, folded at the start of the
  // next block; zero sums and zero scales make the first fold a no-op
  // (fma(0, 0, acc) == acc, and acc is never -0).
  TileOut pend;
  pend.sumi = v16i{};
  pend.dxy = v16f{};
  for (size_t c0 = 0; c0 < nb; c0 += kFbKB) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kFbKB), nb - c0));
    const int npairs = (nbc + 1) >> 1;
    __syncthreads();  // the previous chunk's fragments have been read
    for (int t = tid; t < kFbBM * (kFbKB / 2); t += kFbThreads) {
      const int r = t / (kFbKB / 2), m = t - r * (kFbKB / 2);
      if (m < npairs) {
        const size_t gr = min(m0 + r, nr - 1);  // rows past nr reuse row nr-1, never stored
        stage_pair(vx + gr * bx + (c0 + 2 * m) * kQ8Bytes, 2 * m + 1 < nbc,
                   qa + r * kFbQRow + 64 * m, &da[2 * m][r], &da[(2 * m + 1) & (kFbKB - 1)][r]);
      }
    }
    for (int t = tid; t < kFbBN * (kFbKB / 2); t += kFbThreads) {
      const int r = t / (kFbKB / 2), m = t - r * (kFbKB / 2);
      if (m < npairs) {
        const size_t gc = min(n0 + r, nc - 1);
        stage_pair(vy + gc * by + (c0 + 2 * m) * kQ8Bytes, 2 * m + 1 < nbc,
                   qb + r * kFbQRow + 64 * m, &db[2 * m][r], &db[(2 * m + 1) & (kFbKB - 1)][r]);
      }
    }
    __syncthreads();
    // Software pipeline: within a block each tile's MFMA pair is issued
    // before the previous tile's fold, the last tile's fold is carried into
    // the next block, and the next block's fragments are read from LDS while
    // the current block computes (two fragment sets, loop unrolled by two).
    Frags f0, f1;
    read_frags(f0, qa, qb, da, db, 0, wm, wn, li, h);
    for (int b = 0; b < nbc; b += 2) {
      if (b + 1 < nbc)
        read_frags(f1, qa, qb, da, db, b + 1, wm, wn, li, h);
      gemm_block(acc, pend, f0);
      if (b + 1 >= nbc)
        break;
      if (b + 2 < nbc)
        read_frags(f0, qa, qb, da, db, b + 2, wm, wn, li, h);
      gemm_block(acc, pend, f1);
    }
  }
  fold_tile(acc[1][1], pend);

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const size_t col = n0 + wn * 64 + j * 32 + li;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const size_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < nr && col < nc)
          s[row * bs + col] = acc[i][j][e];
      }
    }
}

}  // namespace tcrv

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
  const int rows16 = aligned16(vx) && aligned16(vy) && (nr == 1 || bx % 16 == 0) &&
                     (nc == 1 || by % 16 == 0);
  if (aligned4(vx) && aligned4(vy) && (nr == 1 || bx % 4 == 0) && (nc == 1 || by % 4 == 0)) {
    const size_t tiles = ((nr + tcrv::kFbBM - 1) / tcrv::kFbBM) * ((nc + tcrv::kFbBN - 1) / tcrv::kFbBN);
    if (tiles > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    tcrv::gemm_q8_0_q8_0_mfma<<<dim3(static_cast<unsigned>(tiles)), dim3(tcrv::kFbThreads), 0,
                                as_stream(stream)>>>(nb, s, vx, vy, by, nr, nc, bx, bs);
    return launch_status();
  }
  const size_t gx = (nc + tcrv::kGmBN - 1) / tcrv::kGmBN;
  const size_t gy = (nr + tcrv::kGmBM - 1) / tcrv::kGmBM;
  if (gx > 0x7fffffffu || gy > 65535u)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::gemm_q8_0_q8_0_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                                dim3(tcrv::kGmThreads), 0, as_stream(stream)>>>(
      nb, s, vx, vy, by, nr, nc, bx, bs, rows16);
  return launch_status();
}
