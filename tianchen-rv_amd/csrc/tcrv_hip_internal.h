// tcrv_hip_internal.h -- device helpers shared by the gfx950 kernels of
// libtcrv_hip.  Block formats are ggml's (pinned by the reference verifiers,
// lib/Dialect/RVV/IR/RVVDialectWideningOps.cpp:3358-3372, RVVOps.td:3893-3897):
//   block_q8_0  34 B : fp16 d @0, int8  qs[32] @2
//   block_q4_0  18 B : fp16 d @0, uint8 qs[16] @2 (element j = lo nibble - 8,
//                      element j+16 = hi nibble - 8)
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "tcrv_hip.h"

namespace tcrv {

constexpr int kQK = 32;
constexpr int kQ8Bytes = 34;
constexpr int kQ4Bytes = 18;

// Exact widening of an fp16 bit pattern (the reference's
// (float)*(const _Float16 *) read, RVVToEmitCBlockQuantLinear.cpp:117,140).
__device__ __forceinline__ float fp16_bits_to_f32(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// v_dot4_i32_i8: c + sum of the four signed byte products (exact in int32).
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// Four packed offset-binary nibbles (raw value n in 0..15, meaning n - 8, held
// in the low nibble of each byte of u after masking) -> four signed bytes.
// (n + 0x78) ^ 0x80 == (n - 8) as a byte and never carries into the next byte.
__device__ __forceinline__ uint32_t nibbles_to_i8x4(uint32_t u) {
  return ((u & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
}

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

// Bytes 2..5 of the 8-byte little-endian value hi:lo (v_alignbyte_b32).
__device__ __forceinline__ uint32_t funnel16(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// Copies `nbytes` (even) bytes from global `src` (2-byte aligned, as every
// ggml block is) into LDS `dst` (16-byte aligned); every thread of the
// work-group (nthreads of them) takes part.  A 16-byte aligned source (every
// row of a 4096-wide matrix) moves with 128-bit loads plus a 16-bit tail; other
// sources fall back to 32-bit or 16-bit loads.  Reads stay inside
// [src, src + nbytes).
__device__ __forceinline__ void copy_span_to_lds(uint8_t *dst, const uint8_t *src,
                                                 int nbytes, int tid, int nthreads) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(src);
  if ((a & 15u) == 0) {
    const int nchunks = nbytes >> 4;
    const uint4 *s4 = reinterpret_cast<const uint4 *>(src);
    uint4 *d4 = reinterpret_cast<uint4 *>(dst);
    for (int c = tid; c < nchunks; c += nthreads)
      d4[c] = s4[c];
    const int tail_halves = (nbytes - (nchunks << 4)) >> 1;
    if (tid < tail_halves) {
      const uint16_t *s2 = reinterpret_cast<const uint16_t *>(src + (nchunks << 4));
      uint16_t *d2 = reinterpret_cast<uint16_t *>(dst + (nchunks << 4));
      d2[tid] = s2[tid];
    }
  } else if ((a & 3u) == 0) {
    const int nwords = nbytes >> 2;
    const uint32_t *s1 = reinterpret_cast<const uint32_t *>(src);
    uint32_t *d1 = reinterpret_cast<uint32_t *>(dst);
    for (int c = tid; c < nwords; c += nthreads)
      d1[c] = s1[c];
    if ((nbytes & 2) && tid == 0)
      reinterpret_cast<uint16_t *>(dst)[nwords * 2] =
          reinterpret_cast<const uint16_t *>(src)[nwords * 2];
  } else {
    const int nhalves = nbytes >> 1;
    const uint16_t *s2 = reinterpret_cast<const uint16_t *>(src);
    uint16_t *d2 = reinterpret_cast<uint16_t *>(dst);
    for (int c = tid; c < nhalves; c += nthreads)
      d2[c] = s2[c];
  }
}

// The reverse copy: `nbytes` (even) bytes from LDS `src` (16-byte aligned) to
// global `dst` (2-byte aligned), widest stores the destination allows.
__device__ __forceinline__ void copy_lds_to_span(uint8_t *dst, const uint8_t *src, int nbytes,
                                                 int tid, int nthreads) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(dst);
  if ((a & 15u) == 0) {
    const int nchunks = nbytes >> 4;
    for (int c = tid; c < nchunks; c += nthreads)
      reinterpret_cast<uint4 *>(dst)[c] = reinterpret_cast<const uint4 *>(src)[c];
    const int tail_halves = (nbytes - (nchunks << 4)) >> 1;
    if (tid < tail_halves)
      reinterpret_cast<uint16_t *>(dst + (nchunks << 4))[tid] =
          reinterpret_cast<const uint16_t *>(src + (nchunks << 4))[tid];
  } else {
    const int nhalves = nbytes >> 1;
    for (int c = tid; c < nhalves; c += nthreads)
      reinterpret_cast<uint16_t *>(dst)[c] = reinterpret_cast<const uint16_t *>(src)[c];
  }
}

// Orders this wave's LDS writes before its later LDS reads by other lanes of
// the same wave (for data no other wave touches): the LDS executes one wave's
// accesses in order, so a wave-scope fence plus a scheduling barrier suffice
// where a work-group barrier would also wait for the other waves.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Serial fold of one row spread over the kLanes lanes of a lane group (a
// 16-lane DPP row, or half of one): lane p of the group holds the two fold
// operands t[k], dy[k] of kTerms consecutive blocks, p*kTerms + k, and each
// step is sumf = fmaf(t[k], dy[k], sumf).
// Phase ph runs the kTerms fmas of lane ph from the running sum it received,
// then hands the sum to lane ph+1 with one DPP row shift (v_mov_b32 row_shr:1)
// and a select; every lane executes every phase, and what the other lanes
// compute is discarded.  The sum therefore sees the terms in ascending block
// order, one fmaf each, exactly as a single scalar loop would.  The group's
// result ends in lane kLanes-1; `sumf` seeds lane 0.
template <int kLanes, int kTerms>
__device__ __forceinline__ float fold_chain(const float t[kTerms], const float dy[kTerms],
                                           float sumf) {
  const int p = threadIdx.x & (kLanes - 1);
#pragma unroll
  for (int ph = 0; ph < kLanes; ++ph) {
#pragma unroll
    for (int k = 0; k < kTerms; ++k)
      sumf = fmaf(t[k], dy[k], sumf);
    if (ph + 1 < kLanes) {
      const float moved = __builtin_bit_cast(
          float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sumf), 0x111 /* row_shr:1 */,
                                             0xf, 0xf, false));
      sumf = (p == ph + 1) ? moved : sumf;
    }
  }
  return sumf;
}

}  // namespace tcrv

// Host-side helpers shared by the entry points.
namespace tcrv_host {

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
inline bool aligned2(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TCRV_HIP_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void *stream) { return reinterpret_cast<hipStream_t>(stream); }

// Stores 0.0f to `count` outputs: s[i] when ncols == 0, else
// s[(i / ncols) * stride + i % ncols] (what the reference writes when nb == 0).
int zero_outputs(float *s, size_t count, size_t stride, size_t ncols, void *stream);

// Q4_0 x Q8_0 GEMM for nc > 1 on MFMA (gemm.hip); TCRV_HIP_ERR_UNSUPPORTED when
// rows are not 4-byte aligned.
int q4_0_gemm_mfma(size_t nb, float *s, const uint8_t *vx, size_t bx, const uint8_t *vy,
                   size_t by, size_t nr, size_t nc, size_t bs, void *stream);

// npairs register-direct block dots (block_dot.hip): s[p * os] = dot(vx + p*bx,
// vy + p*by); a stride of 0 pairs every row of the other operand with one row
// (the GEMM's nc = 1 and nr = 1 shapes).  TCRV_HIP_ERR_UNSUPPORTED for an odd
// block count or operands/strides that are not 4-byte aligned.
int q8_0_rows_direct(size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx,
                     const uint8_t *vy, size_t by, size_t npairs, void *stream);
int q4_0_rows_direct(size_t nb, float *s, size_t os, const uint8_t *vx, size_t bx,
                     const uint8_t *vy, size_t by, size_t npairs, void *stream);

// Q4_0 x Q8_0 GEMM for nc > 1 as one wave per output element (block_dot.hip).
int q4_0_grid(size_t n, float *s, const uint8_t *vx, size_t bx, const uint8_t *vy, size_t by,
              size_t nr, size_t nc, size_t bs, void *stream);

// The GEMMs with 2..kGemvColsMax tokens (batched decode) run as multi-column
// GEMVs over groups of up to eight activation columns, the weights read once
// per group (gemv.hip); an MFMA GEMM would run only nr / 256 work-groups.
// TCRV_HIP_ERR_UNSUPPORTED for an odd block count or operands/strides that are
// not 4-byte aligned.
constexpr size_t kGemvColsMax = 64;
// The multi-column GEMVs run first up to kColsFirstMax tokens; past it the
// one-tile-a-wave GEMMs (gemm_rows_few from plain rows, gemm_tiled.hip) where
// they serve the shape, then the GEMVs up to kGemvColsMax.  A GEMV launch
// serves 8 tokens at ~6 us for K 4096 whatever the weight rows (it is bound by
// its K loop at few rows: 256 x 40 x 4096 Q8_0 32 us as five launches against
// 18-27 us on the tiles), so the switch depends on the tokens only.
constexpr size_t kColsFirstMax = 24;
inline bool cols_first(size_t nr, size_t nc) {
  (void)nr;
  return nc <= kColsFirstMax;
}
// The GEMM of few output tiles straight from plain rows (16-byte aligned rows
// and strides, n a multiple of 256); TCRV_HIP_ERR_UNSUPPORTED otherwise.
int gemm_rows_few(bool q4, size_t nb, float *s, const uint8_t *vx, size_t bx, const uint8_t *vy,
                  size_t by, size_t nr, size_t nc, size_t bs, void *stream);
int gemv_cols_q4_0_q8_0(size_t nb, float *s, size_t bs, const uint8_t *vx, size_t bx,
                        const uint8_t *vy, size_t by, size_t nr, size_t nc, void *stream);
int gemv_cols_q8_0_q8_0(size_t nb, float *s, size_t bs, const uint8_t *vx, size_t bx,
                        const uint8_t *vy, size_t by, size_t nr, size_t nc, void *stream);

// tcrv_hip_q8_0_q8_0_gemm_ws packs into its workspace and runs the tiled
// kernels for this call (otherwise it runs the plain GEMM and reads no
// workspace); gemm_tiled.hip.
bool gemm_ws_uses_workspace(size_t n, const uint8_t *vx, size_t bx, const uint8_t *vy,
                            size_t by, size_t nr, size_t nc);

}  // namespace tcrv_host
