// int_core.hip -- a4: tcrv_rvv.packed_i4_offset_binary_x_i8_product as the
// standalone kernel the reference emits for it
// (test/Conversion/RVV/rvv-to-emitc-packed-i4-offset-binary-x-i8-product-
// reduce.mlir:22-27; op RVVOps.td:3814-3871):
//   out[0] = acc[0] + sum_{i<n} ( lo(w[i]) * qlo[i] + hi(w[i]) * qhi[i] )
// with lo/hi the offset-binary nibble decode of the weight byte (v = w ^ 0x88,
// lo = (int8)(v << 4) >> 4, hi = (int8)v >> 4, i.e. nibble - 8;
// emitOffsetBinaryDecodeValue RVVToEmitC.cpp:2524-2561) and the plain int8
// activations.  The reference sums in i16 lanes (vwmul + vwmacc; each pair is
// at most 2048 in magnitude) and reduces with vwredsum into the int32 cell,
// which wraps modulo 2^32; the integer sum is order-free, so any grouping gives
// the same int32.
//
// GPU: one launch seeds out[0] = acc[0] (acc may alias out), a second sums the
// products with v_dot4_i32_i8 on decoded bytes, reduces each wave across its
// lanes and adds the wave's sum to out[0] with one atomic add (wrapping int32,
// so the result does not depend on the order of the adds).
#include "tcrv_hip_internal.h"

namespace {

constexpr int kThreads = 256;

__global__ void seed_out(const int32_t *acc, int32_t *out) { out[0] = acc[0]; }

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
    v += __shfl_xor(v, m, 64);
  return v;
}

// kVec: w, qlo and qhi are 16-byte aligned; 16 elements per uint4.
template <bool kVec>
__global__ __launch_bounds__(kThreads) void int_core_sum(const int8_t *w, const int8_t *qlo,
                                                         const int8_t *qhi, int32_t *out,
                                                         size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  int sum = 0;
  if constexpr (kVec) {
    const size_t n16 = n / 16;
    for (; i < n16; i += stride) {
      const uint4 wv = reinterpret_cast<const uint4 *>(w)[i];
      const uint4 lo = reinterpret_cast<const uint4 *>(qlo)[i];
      const uint4 hi = reinterpret_cast<const uint4 *>(qhi)[i];
      const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
      const uint32_t ls[4] = {lo.x, lo.y, lo.z, lo.w};
      const uint32_t hs[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        sum = tcrv::sdot4(tcrv::nibbles_to_i8x4(ws[k]), ls[k], sum);
        sum = tcrv::sdot4(tcrv::nibbles_to_i8x4(ws[k] >> 4), hs[k], sum);
      }
    }
    i = n16 * 16 + static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;  // the tail
  }
  for (; i < n; i += stride) {
    const int v = static_cast<int>(static_cast<uint8_t>(w[i]) ^ 0x88u);
    const int lo = static_cast<int8_t>(static_cast<uint8_t>(v << 4)) >> 4;
    const int hi = static_cast<int8_t>(static_cast<uint8_t>(v)) >> 4;
    sum = static_cast<int>(static_cast<uint32_t>(sum) +
                           static_cast<uint32_t>(lo * qlo[i] + hi * qhi[i]));
  }
  sum = wave_sum(sum);
  if ((threadIdx.x & 63) == 0)
    atomicAdd(out, sum);
}

}  // namespace

extern "C" int tcrv_hip_packed_i4_offset_binary_x_i8_product_reduce(const int8_t *w,
                                                                    const int8_t *qlo,
                                                                    const int8_t *qhi,
                                                                    const int32_t *acc,
                                                                    int32_t *out, size_t n,
                                                                    void *stream) {
  using namespace tcrv_host;
  if (!acc || !out || (n > 0 && (!w || !qlo || !qhi)))
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned4(acc) || !aligned4(out))
    return TCRV_HIP_ERR_MISALIGNED;
  hipStream_t st = as_stream(stream);
  seed_out<<<1, 1, 0, st>>>(acc, out);
  if (n > 0) {
    const bool vec = aligned16(w) && aligned16(qlo) && aligned16(qhi);
    const size_t per = static_cast<size_t>(kThreads) * (vec ? 16 : 1);
    const size_t grid = min((n + per - 1) / per, static_cast<size_t>(1024));
    if (vec)
      int_core_sum<true><<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st>>>(
          w, qlo, qhi, out, n);
    else
      int_core_sum<false><<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st>>>(
          w, qlo, qhi, out, n);
  }
  return launch_status();
}
