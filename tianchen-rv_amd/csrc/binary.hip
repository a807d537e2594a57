// binary.hip -- tcrv_rvv.binary {kind = add | sub | mul} over the element
// types of the reference's vector grid (RVVToEmitC.cpp:1873-1911, :4976-4993,
// :5040-5075): out[i] = lhs[i] <kind> rhs[i].
//
// Integer kinds run on unsigned types (wrap-around is the RVV vadd/vsub/vmul
// result for signed and unsigned elements alike); float kinds are single IEEE
// operations (the library is built with -ffp-contract=off).  Each thread moves
// kUnroll 16-byte vectors per operand, all loads issued before the arithmetic;
// a scalar kernel covers the tail and pointers that are not 16-byte aligned.
#include <type_traits>

#include "tcrv_hip_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 2;  // as add_f32: two 16-byte vectors per operand measured fastest

// Integer elements narrower than 32 bits would be promoted to (signed) int by
// C++, where 0xFFFF * 0xFFFF overflows; they are computed in uint32_t, whose
// arithmetic wraps by definition, and narrowed back (the low bits are the RVV
// result).
template <typename T>
using wide_t = typename std::conditional<std::is_integral<T>::value && (sizeof(T) < 4),
                                         uint32_t, T>::type;

template <typename T, int kKind>
__device__ __forceinline__ T apply(T a, T b) {
  const wide_t<T> x = static_cast<wide_t<T>>(a), y = static_cast<wide_t<T>>(b);
  if constexpr (kKind == TCRV_HIP_BINARY_ADD)
    return static_cast<T>(x + y);
  else if constexpr (kKind == TCRV_HIP_BINARY_SUB)
    return static_cast<T>(x - y);
  else
    return static_cast<T>(x * y);
}

template <typename T, int kKind>
__global__ __launch_bounds__(kThreads) void binary_vec(const uint4 *lhs, const uint4 *rhs,
                                                       uint4 *out, size_t n16) {
  constexpr int kLanes = 16 / sizeof(T);
  typedef T vec __attribute__((ext_vector_type(kLanes)));
  const size_t base = static_cast<size_t>(blockIdx.x) * (kThreads * kUnroll) + threadIdx.x;
  uint4 a[kUnroll], b[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const size_t i = base + static_cast<size_t>(u) * kThreads;
    if (i < n16) {
      a[u] = lhs[i];
      b[u] = rhs[i];
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const size_t i = base + static_cast<size_t>(u) * kThreads;
    if (i < n16) {
      vec r;
      const vec va = __builtin_bit_cast(vec, a[u]);
      const vec vb = __builtin_bit_cast(vec, b[u]);
#pragma unroll
      for (int k = 0; k < kLanes; ++k)
        r[k] = apply<T, kKind>(va[k], vb[k]);
      out[i] = __builtin_bit_cast(uint4, r);
    }
  }
}

template <typename T, int kKind>
__global__ __launch_bounds__(kThreads) void binary_scalar(const T *lhs, const T *rhs, T *out,
                                                          size_t begin, size_t n) {
  const size_t i = begin + static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n)
    out[i] = apply<T, kKind>(lhs[i], rhs[i]);
}

template <typename T, int kKind>
int launch(const void *lhs, const void *rhs, void *out, size_t n, hipStream_t st) {
  using namespace tcrv_host;
  const uintptr_t mask = sizeof(T) - 1;
  if ((reinterpret_cast<uintptr_t>(lhs) | reinterpret_cast<uintptr_t>(rhs) |
       reinterpret_cast<uintptr_t>(out)) & mask)
    return TCRV_HIP_ERR_MISALIGNED;
  size_t done = 0;
  if (aligned16(lhs) && aligned16(rhs) && aligned16(out)) {
    const size_t n16 = n * sizeof(T) / 16;
    if (n16 > 0) {
      const size_t per = static_cast<size_t>(kThreads) * kUnroll;
      const size_t grid = (n16 + per - 1) / per;
      if (grid > 0x7fffffffu)
        return TCRV_HIP_ERR_TOO_LARGE;
      binary_vec<T, kKind><<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st>>>(
          static_cast<const uint4 *>(lhs), static_cast<const uint4 *>(rhs),
          static_cast<uint4 *>(out), n16);
      done = n16 * 16 / sizeof(T);
    }
  }
  if (done < n) {
    const size_t grid = (n - done + kThreads - 1) / kThreads;
    if (grid > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    binary_scalar<T, kKind><<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st>>>(
        static_cast<const T *>(lhs), static_cast<const T *>(rhs), static_cast<T *>(out), done, n);
  }
  return launch_status();
}

template <typename T>
int by_kind(int kind, const void *lhs, const void *rhs, void *out, size_t n, hipStream_t st) {
  switch (kind) {
  case TCRV_HIP_BINARY_ADD: return launch<T, TCRV_HIP_BINARY_ADD>(lhs, rhs, out, n, st);
  case TCRV_HIP_BINARY_SUB: return launch<T, TCRV_HIP_BINARY_SUB>(lhs, rhs, out, n, st);
  case TCRV_HIP_BINARY_MUL: return launch<T, TCRV_HIP_BINARY_MUL>(lhs, rhs, out, n, st);
  default: return TCRV_HIP_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" {

int tcrv_hip_binary(int kind, int elem, const void *lhs, const void *rhs, void *out, size_t n,
                    void *stream) {
  if (kind < TCRV_HIP_BINARY_ADD || kind > TCRV_HIP_BINARY_MUL || elem < TCRV_HIP_ELEM_I8 ||
      elem > TCRV_HIP_ELEM_F64)
    return TCRV_HIP_ERR_UNSUPPORTED;
  if (n == 0)
    return TCRV_HIP_OK;
  if (!lhs || !rhs || !out)
    return TCRV_HIP_ERR_NULL_POINTER;
  hipStream_t st = tcrv_host::as_stream(stream);
  switch (elem) {
  case TCRV_HIP_ELEM_I8:
  case TCRV_HIP_ELEM_U8: return by_kind<uint8_t>(kind, lhs, rhs, out, n, st);
  case TCRV_HIP_ELEM_I16:
  case TCRV_HIP_ELEM_U16: return by_kind<uint16_t>(kind, lhs, rhs, out, n, st);
  case TCRV_HIP_ELEM_I32:
  case TCRV_HIP_ELEM_U32: return by_kind<uint32_t>(kind, lhs, rhs, out, n, st);
  case TCRV_HIP_ELEM_I64: return by_kind<uint64_t>(kind, lhs, rhs, out, n, st);
  case TCRV_HIP_ELEM_F32: return by_kind<float>(kind, lhs, rhs, out, n, st);
  default: return by_kind<double>(kind, lhs, rhs, out, n, st);
  }
}

int tcrv_hip_add_i32(const int32_t *lhs, const int32_t *rhs, int32_t *out, size_t n,
                     void *stream) {
  return tcrv_hip_binary(TCRV_HIP_BINARY_ADD, TCRV_HIP_ELEM_I32, lhs, rhs, out, n, stream);
}

}  // extern "C"
