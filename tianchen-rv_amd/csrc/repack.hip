// repack.hip -- a8: the x16 block-as-lane weight layout.
//   tcrv_hip_pack_q4_0_to_q4_0x16   make_block_q4_0x16 (tcrv_rvv.pack_q4_0_to_q4_0x16)
//   tcrv_hip_pack_q8_0_to_q8_0x16   the layout tcrv_rvv.repack_gemv_q8_0_q8_0 reads
//   tcrv_hip_repack_gemv_q4_0_q8_0  tcrv_rvv.repack_gemv_q4_0_q8_0
//   tcrv_hip_repack_gemv_q8_0_q8_0  tcrv_rvv.repack_gemv_q8_0_q8_0
//
// Layouts (include/TianChenRV/Dialect/RVV/IR/RVVOps.td:4551-4577, :4846-4857):
//   block_q4_0x16  288 B: fp16 d[16] @0, qs[256] @32, qs[i*16 + r] = byte i of
//                  source block r, XOR 0x88 (both nibbles offset-binary biased)
//   block_q8_0x16  544 B: fp16 d[16] @0, qs[512] @32, qs[i*16 + r] = quant i of
//                  source block r
// Repacked GEMV over nc/16 groups of 16 weight rows (group x at vx + x*nb*stride),
// one plain block_q8_0 activation stream, output s[x*16 + r]; the fold of both
// emitters (RVVToEmitCBlockQuantLinear.cpp:3245-3290, :4258-4330) is
//   acc_r = fma((float)sumi_r, d_w[r]*d_a, acc_r)   (vfwmul exact, vfmacc fused)
// in ascending block order.
#include "tcrv_hip_internal.h"

namespace tcrv {

constexpr int kQ4x16Bytes = 288;
constexpr int kQ8x16Bytes = 544;

// ---------------------------------------------------------------------------
// Packs.  The output's quant bytes are a 16 x 16 (Q4_0) or 16 x 32 (Q8_0)
// byte transpose of the 16 source blocks' quants: out[32 + 16i + r] = quant
// byte i of source block r.  One lane per source block: lane r of a 16-lane group loads its block's
// quant bytes into registers (2-byte aligned source: the aligned dwords over
// them, realigned with v_perm; no load leaves the block), as dwords X_k =
// quant bytes 4k..4k+3.
// Within each lane quad (rows 4q..4q+3, j = r % 4) a 4x4 byte transpose of X_k
// -- two DPP quad moves and two v_perm -- leaves lane r holding bytes 4k+j of
// rows 4q..4q+3, i.e. output dword 8 + 4(4k+j) + q; for each k the group's 16
// lanes store 16 consecutive dwords.  The scale d of source block r is the
// output's fp16 d[r]: one 16-bit store per lane, 32 contiguous bytes per group.
// Ordinary loads and stores: with 64 rotating weight sets (past the 256 MB
// Infinity Cache), nontemporal stores measured 5.43 against 5.27 us; they gain
// only where the source stays cached.  Nontemporal loads lose outright, since
// a 16-lane group's loads share cache lines across its instructions.
// ---------------------------------------------------------------------------
template <bool kQ4>
__global__ __launch_bounds__(256) void pack_x16_quad(size_t nblocks, const uint8_t *src,
                                                     uint8_t *dst) {
  constexpr int kSrc = kQ4 ? kQ4Bytes : kQ8Bytes;
  constexpr int kDst = kQ4 ? kQ4x16Bytes : kQ8x16Bytes;
  constexpr int kQw = (kSrc - 2) / 4;  // quant dwords per source block: 4 or 8
  const size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  const size_t o = t >> 4;  // output block; its 16 lanes are a whole DPP row
  if (o >= nblocks)
    return;
  const int r = static_cast<int>(t & 15), j = r & 3, q = r >> 2;
  const uint8_t *in = src + o * kDst + r * kSrc;  // source block r (16 blocks = kDst bytes)
  const uint8_t *qs = in + 2;
  const int sh = static_cast<int>(reinterpret_cast<uintptr_t>(qs) & 2u);  // 0 or 2
  const uint32_t *w = reinterpret_cast<const uint32_t *>(qs - sh);
  uint32_t raw[kQw + 1];
#pragma unroll
  for (int k = 0; k < kQw; ++k)
    raw[k] = w[k];  // ends at the block's last byte (sh = 0) or 2 bytes before it
  // the quants' last 2 bytes, read on their own (the dword holding them when
  // sh = 2 would run 2 bytes past the block); unused when sh = 0
  raw[kQw] = *reinterpret_cast<const uint16_t *>(qs + 4 * kQw - 2);
  const uint32_t d = *reinterpret_cast<const uint16_t *>(in);
  // X_k = quant bytes 4k..4k+3: {raw[k+1]:raw[k]} >> 8*sh
  const uint32_t sel_align = sh ? 0x05040302u : 0x03020100u;
  // 4x4 byte transpose within the quad: stage 1 pairs lanes j, j^1, stage 2
  // j, j^2 (v_perm: selector bytes 0-3 pick the lane's own dword, 4-7 the
  // partner's)
  const uint32_t sel1 = (j & 1) ? 0x03070105u : 0x06020400u;
  const uint32_t sel2 = (j & 2) ? 0x03020706u : 0x05040100u;
  uint32_t *out = reinterpret_cast<uint32_t *>(dst + o * kDst);
#pragma unroll
  for (int k = 0; k < kQw; ++k) {
    uint32_t x = __builtin_amdgcn_perm(raw[k + 1], raw[k], sel_align);
    if constexpr (kQ4)
      x ^= 0x88888888u;  // both nibbles offset-binary biased
    const uint32_t p1 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
        0, static_cast<int>(x), 0xB1 /* quad_perm:[1,0,3,2] */, 0xf, 0xf, false));
    const uint32_t tq = __builtin_amdgcn_perm(p1, x, sel1);
    const uint32_t p2 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
        0, static_cast<int>(tq), 0x4E /* quad_perm:[2,3,0,1] */, 0xf, 0xf, false));
    out[8 + 4 * (4 * k + j) + q] = __builtin_amdgcn_perm(p2, tq, sel2);
  }
  reinterpret_cast<uint16_t *>(out)[r] = static_cast<uint16_t>(d);
}

// Quant bytes 4k..4k+3 of activation block b staged raw (34-byte blocks) in
// LDS: an even block starts on a dword (its quants sit 2 bytes in), an odd
// block 2 bytes into one (its quants are dword aligned).
__device__ __forceinline__ uint32_t act_dword(const uint8_t *act, int b, int k) {
  if ((b & 1) == 0) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(act + b * kQ8Bytes);
    return funnel16(w[k], w[k + 1]);
  }
  const uint32_t *w = reinterpret_cast<const uint32_t *>(act + b * kQ8Bytes - 2);
  return w[k + 1];
}

// ---------------------------------------------------------------------------
// Repacked GEMV, wave-staged.  Work-group = 8 waves for one group of 16
// weight rows, each wave a share of kRwBlocks blocks per chunk.  A group's x16
// blocks are contiguous, so each wave's share of a chunk -- kRwBlocks blocks,
// 4608 or 8704 bytes -- is one span: the wave copies it into its own LDS
// region with consecutive 128-bit loads (dword loads for a group that is only
// 4-byte aligned), each block at a 16-byte padded stride (kW + 16: 76 or 140
// dwords, 12 banks apart, so the wave's 16 blocks x 4 row quads read 64
// different banks), with its share of the activation beside it.  Lane (block
// b, row quad g) then reads position dword 4i + g of block b for every
// position i, turns each 4x4 group row-major with v_perm and dots it with the
// activation; exact (float)sumi and d_w*d_a go to LDS.  Only the fold needs
// every wave's terms: after one work-group barrier DPP row fr of wave w
// (w < 4) folds weight row 4w + fr with fold_chain.
// ---------------------------------------------------------------------------
constexpr int kRwWaves = 8, kRwBlocks = 16;
constexpr int kRwChunk = kRwWaves * kRwBlocks;  // x16 blocks per chunk

// Piece u = tid + k*kThreads (k < kPer) of a span of np 16-byte pieces, loaded
// into v[k].  Lanes past the span re-read its last piece (and store_pieces
// re-stores it: the same bytes to the same place), so no lane branches and
// every load is issued before the first store waits.
template <int kPer, int kThreads>
__device__ __forceinline__ void load_pieces(uint4 v[kPer], const uint8_t *src, int np, int tid) {
  const uint4 *s4 = reinterpret_cast<const uint4 *>(src);
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    v[k] = s4[min(tid + k * kThreads, np - 1)];
}

// Stores the pieces to LDS, piece u of a run of kRun at (u / kRun) * kStride +
// 16 * (u % kRun): a padded stride per block of kRun pieces.
template <int kPer, int kThreads, int kRun, int kStride>
__device__ __forceinline__ void store_pieces(const uint4 v[kPer], uint8_t *dst, int np, int tid) {
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int u = min(tid + k * kThreads, np - 1);
    const int b = u / kRun;
    *reinterpret_cast<uint4 *>(dst + b * kStride + 16 * (u - b * kRun)) = v[k];
  }
}

template <bool kQ4>
__global__ __launch_bounds__(64 * kRwWaves) void repack_gemv_waves(size_t nb, float *s,
                                                                   const uint8_t *vx,
                                                                   const uint8_t *vy) {
  constexpr int kW = kQ4 ? kQ4x16Bytes : kQ8x16Bytes;
  constexpr int kLw = kW + 16;          // LDS bytes per staged block
  constexpr int kPieces = kW / 16;      // 128-bit pieces per block
  constexpr int kWords = kW / 4;
  constexpr int kPos = kQ4 ? 16 : 32;   // quant-byte positions per block
  constexpr int kPer = (kRwBlocks * kPieces + 63) / 64;
  constexpr int kFoldLanes = 16, kFoldTerms = kRwChunk / kFoldLanes;
  constexpr int kTermRow = kRwChunk + 4;  // float2 per terms row (264 dwords)
  constexpr int kActPieces = kRwBlocks * kQ8Bytes / 16;  // a wave's activation share
  static_assert(kRwBlocks * 4 == 64, "one (block, row quad) item per lane");
  static_assert((kRwBlocks * kQ8Bytes) % 16 == 0 && kActPieces <= 64, "one piece per lane");
  __shared__ __align__(16) uint8_t wq[kRwChunk * kLw];
  __shared__ __align__(16) uint8_t act[kRwChunk * kQ8Bytes + 16];
  __shared__ __align__(16) float2 terms[16][kTermRow];  // [row][block]

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63;
  const int fr = l >> 4, fp = l & (kFoldLanes - 1);
  const uint8_t *group = vx + static_cast<size_t>(blockIdx.x) * nb * kW;
  const bool wide = (reinterpret_cast<uintptr_t>(vx) & 15u) == 0;  // every group then is
  const bool act16 = (reinterpret_cast<uintptr_t>(vy) & 15u) == 0;  // every wave's share then is
  const int wb0 = w * kRwBlocks;  // this wave's first block of a chunk
  float acc = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kRwChunk) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kRwChunk), nb - c0));
    const int wnb = max(0, min(kRwBlocks, nbc - wb0));  // this wave's blocks
    if (wnb > 0) {
      const uint8_t *src = group + (c0 + wb0) * kW;
      const uint8_t *asrc = vy + (c0 + wb0) * kQ8Bytes;
      if (wide && act16 && wnb == kRwBlocks) {
        // weights and activation in flight together (no lane branches)
        uint4 av[1], v[kPer];
        load_pieces<1, 64>(av, asrc, kActPieces, l);
        load_pieces<kPer, 64>(v, src, kRwBlocks * kPieces, l);
        store_pieces<kPer, 64, kPieces, kLw>(v, wq + wb0 * kLw, kRwBlocks * kPieces, l);
        store_pieces<1, 64, kActPieces, 16 * kActPieces>(av, act + wb0 * kQ8Bytes, kActPieces, l);
      } else if (wide) {
        copy_span_to_lds(act + wb0 * kQ8Bytes, asrc, wnb * kQ8Bytes, l, 64);
        uint4 v[kPer];
        load_pieces<kPer, 64>(v, src, wnb * kPieces, l);
        store_pieces<kPer, 64, kPieces, kLw>(v, wq + wb0 * kLw, wnb * kPieces, l);
      } else {
        copy_span_to_lds(act + wb0 * kQ8Bytes, asrc, wnb * kQ8Bytes, l, 64);
        const uint32_t *s1 = reinterpret_cast<const uint32_t *>(src);
        for (int u = l; u < wnb * kWords; u += 64) {
          const int b = u / kWords;
          *reinterpret_cast<uint32_t *>(wq + (wb0 + b) * kLw + 4 * (u - b * kWords)) = s1[u];
        }
      }
      wave_lds_sync();  // the wave reads only its own region
    }
    const int b = wb0 + (l >> 2), g = l & 3;
    float2 t[4] = {make_float2(0.0f, 0.0f), make_float2(0.0f, 0.0f), make_float2(0.0f, 0.0f),
                   make_float2(0.0f, 0.0f)};  // absent blocks: fma(0, 0, acc) == acc
    if (b < nbc) {
      const uint8_t *blk = wq + b * kLw;
      uint32_t raw[kPos];
#pragma unroll
      for (int i = 0; i < kPos; ++i)
        raw[i] = *reinterpret_cast<const uint32_t *>(blk + 32 + 16 * i + 4 * g);
      const uint2 dq = *reinterpret_cast<const uint2 *>(blk + 8 * g);  // d[4g..4g+3]
      uint32_t a[8];  // the block's 32 activation quants
#pragma unroll
      for (int k = 0; k < 8; ++k)
        a[k] = act_dword(act, b, k);
      const float da = fp16_bits_to_f32(*reinterpret_cast<const uint16_t *>(act + b * kQ8Bytes));
      int part[4] = {0, 0, 0, 0};
#pragma unroll
      for (int q = 0; q < kPos / 4; ++q) {
        uint32_t rows[4];
        transpose4x4(&raw[4 * q], rows);  // positions 4q..4q+3 of rows 4g..4g+3
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (kQ4) {
            // byte = (n_lo ^ 8) | (n_hi ^ 8) << 4: as signed bytes the masked
            // nibbles are 16 * (n - 8); low nibbles pair with quants 4q..,
            // high nibbles with 16+4q..
            part[r] = sdot4((rows[r] << 4) & 0xF0F0F0F0u, a[q], part[r]);
            part[r] = sdot4(rows[r] & 0xF0F0F0F0u, a[q + 4], part[r]);
          } else {
            part[r] = sdot4(rows[r], a[q], part[r]);
          }
        }
      }
      const uint32_t dw[4] = {dq.x & 0xffffu, dq.x >> 16, dq.y & 0xffffu, dq.y >> 16};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int sumi = kQ4 ? (part[r] >> 4) : part[r];  // Q4_0: exact division by 16
        t[r] = make_float2(static_cast<float>(sumi), fp16_bits_to_f32(dw[r]) * da);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      terms[4 * g + r][b] = t[r];
    __syncthreads();
    if (w < 4) {
      float ta[kFoldTerms], tb[kFoldTerms];
#pragma unroll
      for (int k = 0; k < kFoldTerms; k += 2) {
        const float4 v =
            *reinterpret_cast<const float4 *>(&terms[4 * w + fr][fp * kFoldTerms + k]);
        ta[k] = v.x; tb[k] = v.y; ta[k + 1] = v.z; tb[k + 1] = v.w;
      }
      // the previous chunk's sum sits in the last lane of the fold row: seed lane 0
      const float carry = __shfl(acc, (l & ~(kFoldLanes - 1)) + kFoldLanes - 1);
      acc = fold_chain<kFoldLanes, kFoldTerms>(ta, tb, fp == 0 ? carry : 0.0f);
    }
    __syncthreads();  // the next chunk rewrites terms
  }
  if (w < 4 && fp == kFoldLanes - 1)
    s[static_cast<size_t>(blockIdx.x) * 16 + 4 * w + fr] = acc;
}

// ---------------------------------------------------------------------------
// Repacked Q4_0 GEMV, register-direct (x16 weights 16-byte aligned).  Work-group
// = kRdWaves waves for one group of 16 weight rows, chunks of 128 blocks, 16
// blocks per wave and pass (8 waves: one pass; 4 waves and two passes measured
// 5.4 against 4.8 us at 4096 x 4096, the wave-staged kernel 4.9-5.0 us).  Lane
// (block b = 16(w*passes + pass) + l/4, quarter k = l%4) loads the 64
// contiguous bytes that hold positions 4k..4k+3 of block b for all 16 rows
// (four 128-bit loads straight into registers, no LDS staging) and reads its
// eight activation quants 4k.. and 16+4k.. from the chunk the work-group
// copied into LDS, turns each row
// quad row-major with v_perm (transpose4x4), dots the masked nibbles (16 times
// the signed quant, as in repack_gemv_waves) with the activation, and a quad
// reduce-scatter (two DPP stages) leaves lane k the sums of rows 4k..4k+3 over
// the block's 16 positions.  The terms go to LDS as in repack_gemv_waves; each
// of waves 0-3 folds four rows on 8 lanes of 16 terms (7 hand-offs per chunk).
// ---------------------------------------------------------------------------
constexpr int kRdWaves = 8;
constexpr int kRdChunk = 128;  // x16 blocks per chunk: kRdChunk / (16 kRdWaves) passes per wave

// keep + (send of the quad lane selected by kCtrl)
template <int kCtrl>
__device__ __forceinline__ int quad_add(int keep, int send) {
  return keep + __builtin_amdgcn_update_dpp(0, send, kCtrl, 0xf, 0xf, false);
}

__global__ __launch_bounds__(64 * kRdWaves) void repack_gemv_q4_direct(size_t nb, float *s,
                                                                       const uint8_t *vx,
                                                                       const uint8_t *vy) {
  constexpr int kW = kQ4x16Bytes;
  constexpr int kPasses = kRdChunk / (kRdWaves * 16);  // 16-block passes per wave and chunk
  constexpr int kFoldLanes = 8, kFoldTerms = kRdChunk / kFoldLanes;
  // [row][block + 2 * (block / 16)]: a fold lane's 16 terms are 144 bytes after
  // the previous lane's, so the 8 lanes' 128-bit reads start 4 banks apart
  constexpr int kTermRow = kRdChunk + 2 * (kRdChunk / 16) + 4;
  static_assert(kFoldTerms == 16 && kRdWaves >= 4, "waves 0-3 fold 16 rows, one run per lane");
  static_assert(kPasses * kRdWaves * 16 == kRdChunk, "whole passes");
  __shared__ __align__(16) float2 terms[16][kTermRow];
  __shared__ __align__(16) uint8_t yl[kRdChunk * kQ8Bytes];  // the activation chunk

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63;
  const int fr = (l >> 3) & 3, fp = l & (kFoldLanes - 1);  // fold row of the wave, fold lane
  const int k = l & 3;  // positions 4k..4k+3 of the block
  const uint8_t *group = vx + static_cast<size_t>(blockIdx.x) * nb * kW;
  float acc = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kRdChunk) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kRdChunk), nb - c0));
    // every pass's loads first; absent blocks re-read the chunk's last block
    // (their terms are zero)
    uint4 qv[kPasses][4];
    uint2 dq[kPasses];
    uint32_t ylo[kPasses], yhi[kPasses];
    uint16_t dah[kPasses];
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int bc = min((w * kPasses + ps) * 16 + (l >> 2), nbc - 1);
      const uint8_t *blk = group + (c0 + bc) * kW;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        qv[ps][i] = reinterpret_cast<const uint4 *>(blk + 32 + 64 * k)[i];
      dq[ps] = *reinterpret_cast<const uint2 *>(blk + 8 * k);  // d of rows 4k..4k+3
    }
    // The activation chunk is copied into LDS once per work-group with
    // coalesced loads, after the weight loads are in flight; read per lane from
    // global memory its quants are 2-byte misaligned pieces of 16 different
    // blocks (up to five small loads a lane): 4.79 -> 4.70 us at 4096^2.
    copy_span_to_lds(yl, vy + c0 * kQ8Bytes, nbc * kQ8Bytes, tid, 64 * kRdWaves);
    __syncthreads();
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int bc = min((w * kPasses + ps) * 16 + (l >> 2), nbc - 1);
      const uint16_t *a16 = reinterpret_cast<const uint16_t *>(yl + bc * kQ8Bytes);
      ylo[ps] = a16[1 + 2 * k] | (static_cast<uint32_t>(a16[2 + 2 * k]) << 16);
      yhi[ps] = a16[9 + 2 * k] | (static_cast<uint32_t>(a16[10 + 2 * k]) << 16);
      dah[ps] = a16[0];
    }
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int b = (w * kPasses + ps) * 16 + (l >> 2);
      int part[16];  // rows 0..15, positions 4k..4k+3
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        auto comp = [g](const uint4 &v) {
          return g == 0 ? v.x : g == 1 ? v.y : g == 2 ? v.z : v.w;
        };
        const uint32_t in[4] = {comp(qv[ps][0]), comp(qv[ps][1]), comp(qv[ps][2]),
                                comp(qv[ps][3])};
        uint32_t rows[4];
        transpose4x4(in, rows);  // positions 4k..4k+3 of rows 4g..4g+3
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int lo = sdot4((rows[r] << 4) & 0xF0F0F0F0u, ylo[ps], 0);
          part[4 * g + r] = sdot4(rows[r] & 0xF0F0F0F0u, yhi[ps], lo);
        }
      }
      // reduce-scatter over the quad: lanes k, k^2 exchange halves (rows 0-7 /
      // 8-15), then lanes k, k^1 quarters; lane k keeps rows 4k..4k+3
      int h8[8];
      const bool up2 = (k & 2) != 0, up1 = (k & 1) != 0;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        h8[i] = quad_add<0x4E>(up2 ? part[8 + i] : part[i], up2 ? part[i] : part[8 + i]);
      int h4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        h4[i] = quad_add<0xB1>(up1 ? h8[4 + i] : h8[i], up1 ? h8[i] : h8[4 + i]);
      const float da = fp16_bits_to_f32(dah[ps]);
      const uint32_t dw[4] = {dq[ps].x & 0xffffu, dq[ps].x >> 16, dq[ps].y & 0xffffu,
                              dq[ps].y >> 16};
#pragma unroll
      for (int r = 0; r < 4; ++r)  // sums of 16 * quants: exact division by 16
        terms[4 * k + r][b + 2 * (b >> 4)] =
            b < nbc ? make_float2(static_cast<float>(h4[r] >> 4), fp16_bits_to_f32(dw[r]) * da)
                    : make_float2(0.0f, 0.0f);  // fma(0, 0, acc) == acc
    }
    __syncthreads();
    if (w < 4 && l < 32) {
      float ta[kFoldTerms], tb[kFoldTerms];
#pragma unroll
      for (int j = 0; j < kFoldTerms; j += 2) {
        const float4 v =
            *reinterpret_cast<const float4 *>(&terms[4 * w + fr][fp * (kFoldTerms + 2) + j]);
        ta[j] = v.x; tb[j] = v.y; ta[j + 1] = v.z; tb[j + 1] = v.w;
      }
      // the previous chunk's sum sits in the last lane of the fold group: seed lane 0
      const float carry = __shfl(acc, (l & ~(kFoldLanes - 1)) + kFoldLanes - 1);
      acc = fold_chain<kFoldLanes, kFoldTerms>(ta, tb, fp == 0 ? carry : 0.0f);
    }
    __syncthreads();  // the next chunk rewrites terms
  }
  if (w < 4 && l < 32 && fp == kFoldLanes - 1)
    s[static_cast<size_t>(blockIdx.x) * 16 + 4 * w + fr] = acc;
}

}  // namespace tcrv

namespace {

template <bool kQ4>
int launch_pack(size_t nblocks, const uint8_t *src, uint8_t *dst, void *stream) {
  using namespace tcrv_host;
  if (nblocks == 0)
    return TCRV_HIP_OK;
  if (!src || !dst)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(src) || !aligned4(dst))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t grid = (nblocks * 16 + 255) / 256;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::pack_x16_quad<kQ4><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                             as_stream(stream)>>>(nblocks, src, dst);
  return launch_status();
}

template <bool kQ4>
int launch_repack_gemv(size_t n, float *s, const uint8_t *vx, const uint8_t *vy, size_t nc,
                       void *stream) {
  using namespace tcrv_host;
  const size_t groups = nc / 16;  // like the reference, a partial group is not written
  const size_t nb = n / tcrv::kQK;
  if (groups == 0)
    return TCRV_HIP_OK;
  if (!s)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (nb == 0)
    return zero_outputs(s, groups * 16, 0, 0, stream);
  if (!vx || !vy)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned4(vx) || !aligned2(vy))
    return TCRV_HIP_ERR_MISALIGNED;
  if (groups > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (kQ4 && aligned16(vx))
    tcrv::repack_gemv_q4_direct<<<dim3(static_cast<unsigned>(groups)),
                                  dim3(64 * tcrv::kRdWaves), 0, as_stream(stream)>>>(nb, s, vx, vy);
  else
    tcrv::repack_gemv_waves<kQ4><<<dim3(static_cast<unsigned>(groups)),
                                   dim3(64 * tcrv::kRwWaves), 0, as_stream(stream)>>>(nb, s, vx, vy);
  return launch_status();
}

}  // namespace

extern "C" {

int tcrv_hip_pack_q4_0_to_q4_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst,
                                  void *stream) {
  return launch_pack<true>(nblocks, src, dst, stream);
}

int tcrv_hip_pack_q8_0_to_q8_0x16(size_t nblocks, const uint8_t *src, uint8_t *dst,
                                  void *stream) {
  return launch_pack<false>(nblocks, src, dst, stream);
}

int tcrv_hip_repack_gemv_q4_0_q8_0(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                   size_t nc, void *stream) {
  return launch_repack_gemv<true>(n, s, vx, vy, nc, stream);
}

int tcrv_hip_repack_gemv_q8_0_q8_0(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                   size_t nc, void *stream) {
  return launch_repack_gemv<false>(n, s, vx, vy, nc, stream);
}

}  // extern "C"
