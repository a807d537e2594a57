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
  const size_t gx = (nc + tcrv::kGmBN - 1) / tcrv::kGmBN;
  const size_t gy = (nr + tcrv::kGmBM - 1) / tcrv::kGmBM;
  if (gx > 0x7fffffffu || gy > 65535u)
    return TCRV_HIP_ERR_TOO_LARGE;
  tcrv::gemm_q8_0_q8_0_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                                dim3(tcrv::kGmThreads), 0, as_stream(stream)>>>(
      nb, s, vx, vy, by, nr, nc, bx, bs, rows16);
  return launch_status();
}
