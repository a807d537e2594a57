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

}  // namespace tcrv

namespace tcrv_host {

// Rows per wave of the decode GEMV.
constexpr int kGemvRows = 2;

int gemv_q4_0_q8_0(size_t n, float *s, size_t os, const uint8_t *vx, size_t bx,
                   const uint8_t *vy, size_t nr, void *stream) {
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
  const size_t rows_per_wg = static_cast<size_t>(tcrv::kGvWaves) * kGemvRows;
  const size_t grid = (nr + rows_per_wg - 1) / rows_per_wg;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::gemv_q4_0_q8_0_kernel<kGemvRows>
      <<<dim3(static_cast<unsigned>(grid)), dim3(tcrv::kGvWaves * 64), 0, as_stream(stream)>>>(
          nb, s, os, vx, bx, vy, nr);
  return launch_status();
}

}  // namespace tcrv_host

extern "C" {

int tcrv_hip_gemv_q4_0_q8_0(size_t n, float *s, const uint8_t *vx, size_t bx,
                            const uint8_t *vy, size_t nr, void *stream) {
  if (nr == 0)
    return TCRV_HIP_OK;
  if (n / tcrv::kQK == 0)
    return tcrv_host::zero_outputs(s, nr, 1, 1, stream);
  return tcrv_host::gemv_q4_0_q8_0(n, s, 1, vx, bx, vy, nr, stream);
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
    return tcrv_host::gemv_q4_0_q8_0(n, s, bs, vx, bx, vy, nr, stream);
  return tcrv_host::q4_0_grid(n, s, vx, bx, vy, by, nr, nc, bs, stream);
}

}  // extern "C"
