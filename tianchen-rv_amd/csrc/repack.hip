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
// Packs, 16-byte aligned spans: the 16 source blocks of an x16 block are
// contiguous and as long as it (16 x 18 = 288, 16 x 34 = 544 bytes), so a
// work-group copies kPkBlocks of them into LDS with coalesced 128-bit loads,
// gathers each output dword from LDS and writes the output span with
// consecutive dword stores.
// ---------------------------------------------------------------------------
constexpr int kPkBlocks = 16;  // x16 blocks per work-group

template <bool kQ4>
__global__ __launch_bounds__(256) void pack_x16_lds(size_t nblocks, const uint8_t *src,
                                                    uint8_t *dst) {
  constexpr int kSrc = kQ4 ? kQ4Bytes : kQ8Bytes;
  constexpr int kDst = kQ4 ? kQ4x16Bytes : kQ8x16Bytes;  // 16 * kSrc, a multiple of 16
  constexpr int kDwords = kDst / 4;
  __shared__ __align__(16) uint8_t in[kPkBlocks * kDst];
  const size_t o0 = static_cast<size_t>(blockIdx.x) * kPkBlocks;
  const int nblk = static_cast<int>(min(static_cast<size_t>(kPkBlocks), nblocks - o0));
  const uint4 *s4 = reinterpret_cast<const uint4 *>(src + o0 * kDst);
  uint4 *l4 = reinterpret_cast<uint4 *>(in);
  for (int c = threadIdx.x; c < nblk * (kDst / 16); c += 256)
    l4[c] = s4[c];
  __syncthreads();
  uint32_t *d = reinterpret_cast<uint32_t *>(dst + o0 * kDst);
  for (int t = threadIdx.x; t < nblk * kDwords; t += 256) {
    const int o = t / kDwords, k = t - o * kDwords;
    const uint8_t *b = in + o * kDst;  // the output block's 16 source blocks
    uint32_t v;
    if (k < 8) {  // scales d[2k], d[2k+1]
      const uint32_t d0 = *reinterpret_cast<const uint16_t *>(b + (2 * k) * kSrc);
      const uint32_t d1 = *reinterpret_cast<const uint16_t *>(b + (2 * k + 1) * kSrc);
      v = d0 | (d1 << 16);
    } else {  // qs bytes 4q .. 4q+3: byte i -> source block i % 16, offset i / 16
      const int q = k - 8;
      const int off = 2 + q / 4;
      const int r0 = 4 * (q % 4);
      v = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v |= static_cast<uint32_t>(b[(r0 + j) * kSrc + off]) << (8 * j);
      if constexpr (kQ4)
        v ^= 0x88888888u;
    }
    d[t] = v;
  }
}

// ---------------------------------------------------------------------------
// Packs: one thread per output dword (8 scale dwords + 64 or 128 quant dwords).
// ---------------------------------------------------------------------------
template <bool kQ4>
__global__ __launch_bounds__(256) void pack_x16(size_t nblocks, const uint8_t *src,
                                                uint8_t *dst) {
  constexpr int kSrc = kQ4 ? kQ4Bytes : kQ8Bytes;
  constexpr int kDst = kQ4 ? kQ4x16Bytes : kQ8x16Bytes;
  constexpr int kDwords = kDst / 4;
  const size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= nblocks * kDwords)
    return;
  const size_t o = t / kDwords;
  const int k = static_cast<int>(t - o * kDwords);
  const uint8_t *in = src + o * 16 * kSrc;
  uint32_t v;
  if (k < 8) {  // scales d[2k], d[2k+1]
    const uint32_t d0 = *reinterpret_cast<const uint16_t *>(in + (2 * k) * kSrc);
    const uint32_t d1 = *reinterpret_cast<const uint16_t *>(in + (2 * k + 1) * kSrc);
    v = d0 | (d1 << 16);
  } else {  // qs bytes 4q .. 4q+3: byte i -> source block i % 16, offset i / 16
    const int q = k - 8;
    const int off = 2 + q / 4;
    const int r0 = 4 * (q % 4);
    v = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v |= static_cast<uint32_t>(in[(r0 + j) * kSrc + off]) << (8 * j);
    if constexpr (kQ4)
      v ^= 0x88888888u;
  }
  reinterpret_cast<uint32_t *>(dst + o * kDst)[k] = v;
}

// ---------------------------------------------------------------------------
// Repacked GEMV.  Work-group = 4 waves for one group of 16 weight rows; each
// wave step covers 4 blocks with 16 lanes per block: lane (rq = l & 3,
// pq = (l >> 2) & 3) owns rows 4rq..4rq+3 and positions 4pq..4pq+3 (Q4_0; the
// high nibbles are positions 16+4pq..) or 8pq..8pq+7 (Q8_0).  It loads one dword
// per position (4 rows of it), turns the 4x4 bytes row-major with v_perm, and
// takes v_dot4_i32_i8 against the activation; the four position lanes of a row
// are summed with two shuffles.  All weight loads of a chunk are issued before
// the first use.  Exact (float)sumi and d_w*d_a per (row, block) go to LDS;
// then DPP row fr of wave w folds weight row 4w+fr with fold_chain (8
// consecutive blocks per lane), so no LDS access sits on the serial chain.
// ---------------------------------------------------------------------------
constexpr int kRgChunk = 128;   // blocks per LDS chunk

// 4x4 byte transpose: in[i] holds rows 0..3 of position i; out[r] holds
// positions 0..3 of row r.
__device__ __forceinline__ void transpose4x4(const uint32_t in[4], uint32_t out[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // i0r0 i1r0 i0r1 i1r1
  const uint32_t t1 = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);  // i2r0 i3r0 i2r1 i3r1
  const uint32_t t2 = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // i0r2 i1r2 i0r3 i1r3
  const uint32_t t3 = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);  // i2r2 i3r2 i2r3 i3r3
  out[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
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

template <bool kQ4>
__global__ __launch_bounds__(256) void repack_gemv(size_t nb, float *s, const uint8_t *vx,
                                                   const uint8_t *vy) {
  constexpr int kW = kQ4 ? kQ4x16Bytes : kQ8x16Bytes;
  constexpr int kDw = kQ4 ? 4 : 8;          // quant dwords per lane and block
  constexpr int kSteps = kRgChunk / 16;     // blocks per lane and chunk
  constexpr int kFoldLanes = 16, kFoldTerms = kRgChunk / kFoldLanes;
  __shared__ __align__(16) uint8_t act[kRgChunk * kQ8Bytes + 16];
  __shared__ __align__(16) float2 terms[16][kRgChunk + 8];  // [row][block]

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63;
  const int jb = l >> 4, pq = (l >> 2) & 3, rq = l & 3;
  const int fr = l >> 4, fp = l & (kFoldLanes - 1);  // fold: DPP row fr folds row 4w+fr
  const uint8_t *group = vx + static_cast<size_t>(blockIdx.x) * nb * kW;
  float acc = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kRgChunk) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kRgChunk), nb - c0));
    uint32_t raw[kSteps][kDw], dsc[kSteps][2];
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
      const int b = 16 * k + 4 * w + jb;
      if (b < nbc) {
        const uint8_t *blk = group + (c0 + b) * kW;
        const uint32_t *qd = reinterpret_cast<const uint32_t *>(blk + 32);
#pragma unroll
        for (int i = 0; i < kDw; ++i)
          raw[k][i] = qd[4 * (kDw * pq + i) + rq];  // position kDw*pq+i, rows 4rq..4rq+3
        const uint32_t *dq = reinterpret_cast<const uint32_t *>(blk + 8 * rq);  // d[4rq..4rq+3]
        dsc[k][0] = dq[0];
        dsc[k][1] = dq[1];
      }
    }
    copy_span_to_lds(act, vy + c0 * kQ8Bytes, nbc * kQ8Bytes, tid, 256);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
      const int b = 16 * k + 4 * w + jb;
      if (b < nbc) {
        int part[4];
        if constexpr (kQ4) {
          uint32_t rows[4];
          transpose4x4(raw[k], rows);
          // activation positions 4pq..4pq+3 (low nibbles) and 16+4pq.. (high)
          const uint32_t alo = act_dword(act, b, pq);
          const uint32_t ahi = act_dword(act, b, pq + 4);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            // byte = (n_lo ^ 8) | (n_hi ^ 8) << 4; as a signed byte, the nibble
            // moved to the high half is 16 * sext4(n ^ 8) = 16 * (n - 8)
            const uint32_t lo16 = (rows[r] << 4) & 0xF0F0F0F0u;
            const uint32_t hi16 = rows[r] & 0xF0F0F0F0u;
            part[r] = sdot4(hi16, ahi, sdot4(lo16, alo, 0));
          }
        } else {
          uint32_t rows[8];
          transpose4x4(raw[k], rows);
          transpose4x4(raw[k] + 4, rows + 4);
          const uint32_t a0 = act_dword(act, b, 2 * pq);
          const uint32_t a1 = act_dword(act, b, 2 * pq + 1);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            part[r] = sdot4(rows[4 + r], a1, sdot4(rows[r], a0, 0));
        }
        // sum over the four position lanes (lane bits 2..3)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          part[r] += __shfl_xor(part[r], 4);
          part[r] += __shfl_xor(part[r], 8);
        }
        if (pq == 0) {
          const float da =
              fp16_bits_to_f32(*reinterpret_cast<const uint16_t *>(act + b * kQ8Bytes));
          const uint32_t dw[4] = {dsc[k][0] & 0xffffu, dsc[k][0] >> 16, dsc[k][1] & 0xffffu,
                                  dsc[k][1] >> 16};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int sumi = kQ4 ? (part[r] >> 4) : part[r];  // Q4_0: exact division by 16
            terms[4 * rq + r][b] =
                make_float2(static_cast<float>(sumi), fp16_bits_to_f32(dw[r]) * da);
          }
        }
      } else if (pq == 0 && b < kRgChunk) {
        // blocks past the chunk: fma(0, 0, acc) == acc (acc is never -0)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          terms[4 * rq + r][b] = make_float2(0.0f, 0.0f);
      }
    }
    __syncthreads();
    float ta[kFoldTerms], tb[kFoldTerms];
#pragma unroll
    for (int k = 0; k < kFoldTerms; k += 2) {
      const float4 v = *reinterpret_cast<const float4 *>(&terms[4 * w + fr][fp * kFoldTerms + k]);
      ta[k] = v.x; tb[k] = v.y; ta[k + 1] = v.z; tb[k + 1] = v.w;
    }
    // the previous chunk's sum sits in the last lane of the fold row: seed lane 0
    const float carry = __shfl(acc, (l & ~(kFoldLanes - 1)) + kFoldLanes - 1);
    acc = fold_chain<kFoldLanes, kFoldTerms>(ta, tb, fp == 0 ? carry : 0.0f);
    __syncthreads();
  }
  if (fp == kFoldLanes - 1)
    s[static_cast<size_t>(blockIdx.x) * 16 + 4 * w + fr] = acc;
}


// ---------------------------------------------------------------------------
// Wave-per-row-quad form (activation 4-byte aligned; the LDS-staged form above
// serves 2-byte aligned activations).  Wave w of the group's work-group owns
// rows 4w..4w+3 and folds them itself, so no work-group barrier is needed:
// lane l takes blocks 2l, 2l+1 of the chunk; per block it loads the dword at
// position i of its row quad for every position i (the x16 interleave puts
// rows 4w..4w+3 of position i in dword 4i + w), turns each 4x4 group
// row-major with v_perm and dots it with the activation, which the lane loads
// straight from global memory (68 bytes, like the plain GEMV).  Exact
// (float)sumi and d_w*d_a go to the wave's own LDS rows; DPP row r then folds
// weight row 4w + r with fold_chain.
// ---------------------------------------------------------------------------
template <bool kQ4>
__global__ __launch_bounds__(256) void repack_gemv_rows(size_t nb, float *s, const uint8_t *vx,
                                                        const uint8_t *vy) {
  constexpr int kW = kQ4 ? kQ4x16Bytes : kQ8x16Bytes;
  constexpr int kPos = kQ4 ? 16 : 32;  // quant-byte positions per block
  constexpr int kFoldLanes = 16, kFoldTerms = kRgChunk / kFoldLanes;
  __shared__ __align__(16) float2 terms[4][4][kRgChunk + 8];  // [wave][row][block]

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63;
  const int fr = l >> 4, fp = l & (kFoldLanes - 1);
  const uint8_t *group = vx + static_cast<size_t>(blockIdx.x) * nb * kW;
  float acc = 0.0f;

  for (size_t c0 = 0; c0 < nb; c0 += kRgChunk) {
    const int nbc = static_cast<int>(min(static_cast<size_t>(kRgChunk), nb - c0));
    const int b0 = 2 * l;
    uint32_t raw[2][kPos], dq[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (b0 + j < nbc) {
        const uint8_t *blk = group + (c0 + b0 + j) * kW;
        const uint32_t *qd = reinterpret_cast<const uint32_t *>(blk + 32);
#pragma unroll
        for (int i = 0; i < kPos; ++i)
          raw[j][i] = qd[4 * i + w];
        const uint32_t *d = reinterpret_cast<const uint32_t *>(blk + 8 * w);  // d[4w..4w+3]
        dq[j][0] = d[0];
        dq[j][1] = d[1];
      }
    }
    // activation blocks 2l, 2l+1: 68 bytes from a dword-aligned start (34 when
    // only block 2l exists)
    uint32_t ar[17];
    const uint32_t *ag = reinterpret_cast<const uint32_t *>(vy + (c0 + b0) * kQ8Bytes);
    if (b0 + 1 < nbc) {
#pragma unroll
      for (int k = 0; k < 17; ++k)
        ar[k] = ag[k];
    } else if (b0 < nbc) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        ar[k] = ag[k];
      ar[8] = *reinterpret_cast<const uint16_t *>(ag + 8);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float2 t[4] = {make_float2(0.0f, 0.0f), make_float2(0.0f, 0.0f), make_float2(0.0f, 0.0f),
                     make_float2(0.0f, 0.0f)};  // absent blocks: fma(0, 0, acc) == acc
      if (b0 + j < nbc) {
        uint32_t a[8];  // the block's 32 activation quants, dword aligned
#pragma unroll
        for (int k = 0; k < 8; ++k)
          a[k] = j == 0 ? funnel16(ar[k], ar[k + 1]) : ar[k + 9];
        const float da = fp16_bits_to_f32(j == 0 ? (ar[0] & 0xffffu) : (ar[8] >> 16));
        int part[4] = {0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < kPos / 4; ++g) {
          uint32_t rows[4];
          transpose4x4(&raw[j][4 * g], rows);  // positions 4g..4g+3 of rows 4w..4w+3
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if constexpr (kQ4) {
              // byte = (n_lo ^ 8) | (n_hi ^ 8) << 4: as signed bytes the masked
              // nibbles are 16 * (n - 8); low nibbles pair with quants 4g..,
              // high nibbles with 16+4g..
              part[r] = sdot4((rows[r] << 4) & 0xF0F0F0F0u, a[g], part[r]);
              part[r] = sdot4(rows[r] & 0xF0F0F0F0u, a[g + 4], part[r]);
            } else {
              part[r] = sdot4(rows[r], a[g], part[r]);
            }
          }
        }
        const uint32_t dw[4] = {dq[j][0] & 0xffffu, dq[j][0] >> 16, dq[j][1] & 0xffffu,
                                dq[j][1] >> 16};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int sumi = kQ4 ? (part[r] >> 4) : part[r];  // Q4_0: exact division by 16
          t[r] = make_float2(static_cast<float>(sumi), fp16_bits_to_f32(dw[r]) * da);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
        terms[w][r][b0 + j] = t[r];
    }
    wave_lds_sync();  // the LDS rows are this wave's own
    float ta[kFoldTerms], tb[kFoldTerms];
#pragma unroll
    for (int k = 0; k < kFoldTerms; k += 2) {
      const float4 v = *reinterpret_cast<const float4 *>(&terms[w][fr][fp * kFoldTerms + k]);
      ta[k] = v.x; tb[k] = v.y; ta[k + 1] = v.z; tb[k + 1] = v.w;
    }
    // the previous chunk's sum sits in the last lane of the fold row: seed lane 0
    const float carry = __shfl(acc, (l & ~(kFoldLanes - 1)) + kFoldLanes - 1);
    acc = fold_chain<kFoldLanes, kFoldTerms>(ta, tb, fp == 0 ? carry : 0.0f);
    wave_lds_sync();
  }
  if (fp == kFoldLanes - 1)
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
  if (aligned16(src) && aligned16(dst)) {
    const size_t grid = (nblocks + tcrv::kPkBlocks - 1) / tcrv::kPkBlocks;
    if (grid > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    tcrv::pack_x16_lds<kQ4><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                              as_stream(stream)>>>(nblocks, src, dst);
    return launch_status();
  }
  const size_t dwords = nblocks * ((kQ4 ? tcrv::kQ4x16Bytes : tcrv::kQ8x16Bytes) / 4);
  const size_t grid = (dwords + 255) / 256;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::pack_x16<kQ4><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, as_stream(stream)>>>(
      nblocks, src, dst);
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
  if (aligned4(vy))
    tcrv::repack_gemv_rows<kQ4><<<dim3(static_cast<unsigned>(groups)), dim3(256), 0,
                                  as_stream(stream)>>>(nb, s, vx, vy);
  else
    tcrv::repack_gemv<kQ4><<<dim3(static_cast<unsigned>(groups)), dim3(256), 0,
                             as_stream(stream)>>>(nb, s, vx, vy);
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
