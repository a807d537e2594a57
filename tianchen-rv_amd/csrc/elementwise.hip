// elementwise.hip -- the HBM-streaming kernels of libtcrv_hip:
//   a1  add_f32                (tcrv_rvv.binary{kind="add"})
//   a3  dequantize_row_q8_0    (ggml block dequant)
//   a3b dequantize_row_q4_0    (ggml block dequant)
//   a10 quantize_row_q8_0      (tcrv_rvv.quantize_row_q8_0)
// plus the library's status/version/synchronize entry points.
#include "tcrv_hip_internal.h"

namespace {

using namespace tcrv;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 128-bit streaming store (the output is not re-read by this kernel).
__device__ __forceinline__ void store_stream(float4 v, float4 *p) {
  const f32x4 x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<f32x4 *>(p));
}

// 128-bit streaming load (the input is read once).
__device__ __forceinline__ float4 load_stream(const float *p) {
  const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
  return make_float4(x.x, x.y, x.z, x.w);
}

// copy_lds_to_span with streaming 128-bit stores when dst is 16-byte aligned.
__device__ __forceinline__ void copy_lds_to_span_stream(uint8_t *dst, const uint8_t *src,
                                                        int nbytes, int tid, int nthreads) {
  if ((reinterpret_cast<uintptr_t>(dst) & 15u) != 0) {
    copy_lds_to_span(dst, src, nbytes, tid, nthreads);
    return;
  }
  const int nchunks = nbytes >> 4;
  for (int c = tid; c < nchunks; c += nthreads)
    __builtin_nontemporal_store(reinterpret_cast<const f32x4 *>(src)[c],
                                reinterpret_cast<f32x4 *>(dst) + c);
  const int tail_halves = (nbytes - (nchunks << 4)) >> 1;
  if (tid < tail_halves)
    reinterpret_cast<uint16_t *>(dst + (nchunks << 4))[tid] =
        reinterpret_cast<const uint16_t *>(src + (nchunks << 4))[tid];
}

// ---------------------------------------------------------------------------
// a1: out[i] = lhs[i] + rhs[i].  The reference emits a VL strip loop of
// vle32/vfadd/vse32 (lib/Conversion/RVV/RVVToEmitC.cpp:605, :1873-1911); here
// each thread moves kAddUnroll 128-bit vectors per operand, all loads issued
// before the adds (2 measured fastest for n = 2^24 over 2 rotating sets: 27.8
// us against 28.0, 28.7 and 29.1 us for 1, 4 and 8).  Loads and stores are nontemporal: over 3-6
// rotating sets (past the Infinity Cache) 31.7-32.4 against 34.6-35.0 us with
// ordinary loads.  IEEE binary32 addition is correctly rounded, so the result
// is bit-identical to the scalar loop.
// ---------------------------------------------------------------------------
constexpr int kAddThreads = 256;
constexpr int kAddUnroll = 2;

__global__ __launch_bounds__(kAddThreads) void add_f32_vec4(const float4 *lhs,
                                                            const float4 *rhs, float4 *out,
                                                            size_t n4) {
  const size_t base =
      static_cast<size_t>(blockIdx.x) * (kAddThreads * kAddUnroll) + threadIdx.x;
  float4 a[kAddUnroll], b[kAddUnroll];
#pragma unroll
  for (int u = 0; u < kAddUnroll; ++u) {
    const size_t i = base + static_cast<size_t>(u) * kAddThreads;
    if (i < n4) {
      a[u] = load_stream(reinterpret_cast<const float *>(lhs + i));
      b[u] = load_stream(reinterpret_cast<const float *>(rhs + i));
    }
  }
#pragma unroll
  for (int u = 0; u < kAddUnroll; ++u) {
    const size_t i = base + static_cast<size_t>(u) * kAddThreads;
    if (i < n4) {
      float4 r;
      r.x = a[u].x + b[u].x;
      r.y = a[u].y + b[u].y;
      r.z = a[u].z + b[u].z;
      r.w = a[u].w + b[u].w;
      store_stream(r, &out[i]);
    }
  }
}

__global__ __launch_bounds__(kAddThreads) void add_f32_scalar(const float *lhs, const float *rhs,
                                                              float *out, size_t begin,
                                                              size_t n) {
  const size_t i = begin + static_cast<size_t>(blockIdx.x) * kAddThreads + threadIdx.x;
  if (i < n)
    out[i] = lhs[i] + rhs[i];
}

// ---------------------------------------------------------------------------
// a3: y[32b+j] = qs_b[j] * d_b.  A work-group stages kDqBlocks contiguous
// 34-byte blocks (a 16-byte multiple: 64*34 = 2176) through LDS with 128-bit
// loads, then writes 128-bit float4 rows of the output, one per thread.
// int8 * fp16-valued float is exact in binary32, so the result is bit-exact.
// One float4 per thread measured fastest: 64 blocks per 512 threads 12.8 us
// for 4096^2, 32 per 256 13.0 us, 16 per 128 13.4 us; 128 blocks per 256
// threads 13.9 us and 256-1024 blocks per 256 threads 14.0-15.5 us.  The
// quantizer's nontemporal loads do not pay here: over 8 rotating sets (past the
// Infinity Cache) 19.4 against 12.5 us.
// ---------------------------------------------------------------------------
constexpr int kDqThreads = 512;
constexpr int kDqBlocks = 64;

template <bool kVecOut>
__global__ __launch_bounds__(kDqThreads) void dequantize_q8_0(const uint8_t *vx, float *y,
                                                              size_t nb) {
  __shared__ __align__(16) uint8_t lds[kDqBlocks * kQ8Bytes];
  const size_t blk0 = static_cast<size_t>(blockIdx.x) * kDqBlocks;
  const int nblk = static_cast<int>(min(static_cast<size_t>(kDqBlocks), nb - blk0));
  copy_span_to_lds(lds, vx + blk0 * kQ8Bytes, nblk * kQ8Bytes, threadIdx.x, kDqThreads);
  __syncthreads();
  const uint16_t *l16 = reinterpret_cast<const uint16_t *>(lds);
  float4 *dst = reinterpret_cast<float4 *>(y + blk0 * kQK);
  const int nf4 = nblk * (kQK / 4);
  for (int f = threadIdx.x; f < nf4; f += kDqThreads) {
    const int b = f >> 3;
    const int j = (f & 7) * 4;
    const int h = (b * kQ8Bytes) >> 1;  // block start in halfwords
    const float d = fp16_bits_to_f32(l16[h]);
    const uint32_t q01 = l16[h + 1 + (j >> 1)];
    const uint32_t q23 = l16[h + 2 + (j >> 1)];
    float4 r;
    r.x = static_cast<float>(static_cast<int8_t>(q01 & 0xffu)) * d;
    r.y = static_cast<float>(static_cast<int8_t>(q01 >> 8)) * d;
    r.z = static_cast<float>(static_cast<int8_t>(q23 & 0xffu)) * d;
    r.w = static_cast<float>(static_cast<int8_t>(q23 >> 8)) * d;
    if constexpr (kVecOut) {
      store_stream(r, &dst[f]);
    } else {
      float *d1 = y + blk0 * kQK + 4 * f;
      d1[0] = r.x;
      d1[1] = r.y;
      d1[2] = r.z;
      d1[3] = r.w;
    }
  }
}

// ---------------------------------------------------------------------------
// a3b: y[32b+j] = (lo(qs_b[j]) - 8) * d_b, y[32b+16+j] = (hi(qs_b[j]) - 8) * d_b
// (ggml dequantize_row_q4_0; the offset-binary nibble decode of RVVOps.td:
// 3837-3842, layout :3893-3897).  The same shape as the Q8_0 kernel: a
// work-group stages kDq4Blocks contiguous 18-byte blocks (64*18 = 1152 bytes,
// a 16-byte multiple) through LDS with 128-bit loads, and each thread writes one
// float4 of the output: lanes 8b..8b+3 the low nibbles of block b's bytes
// 0-15, lanes 8b+4..8b+7 the high ones.  (n - 8) is exact in binary32 and a
// 4-bit integer times an fp16-valued float is exact, so the result is
// bit-exact.
// ---------------------------------------------------------------------------
constexpr int kDq4Threads = 512;
constexpr int kDq4Blocks = kDq4Threads / 8;

template <bool kVecOut>
__global__ __launch_bounds__(kDq4Threads) void dequantize_q4_0(const uint8_t *vx, float *y,
                                                               size_t nb) {
  __shared__ __align__(16) uint8_t lds[kDq4Blocks * kQ4Bytes];
  const size_t blk0 = static_cast<size_t>(blockIdx.x) * kDq4Blocks;
  const int nblk = static_cast<int>(min(static_cast<size_t>(kDq4Blocks), nb - blk0));
  copy_span_to_lds(lds, vx + blk0 * kQ4Bytes, nblk * kQ4Bytes, threadIdx.x, kDq4Threads);
  __syncthreads();
  const int nf4 = nblk * (kQK / 4);
  for (int f = threadIdx.x; f < nf4; f += kDq4Threads) {
    const int b = f >> 3;
    const int part = f & 7;
    const uint16_t *l16 = reinterpret_cast<const uint16_t *>(lds) + b * (kQ4Bytes / 2);
    const float d = fp16_bits_to_f32(l16[0]);
    const int j = (part & 3) * 4;  // first of the four packed bytes this lane decodes
    const uint32_t u = static_cast<uint32_t>(l16[1 + (j >> 1)]) |
                       (static_cast<uint32_t>(l16[2 + (j >> 1)]) << 16);
    const uint32_t nib = (part < 4 ? u : u >> 4) & 0x0F0F0F0Fu;
    float4 r;
    r.x = (static_cast<float>(nib & 0xffu) - 8.0f) * d;
    r.y = (static_cast<float>((nib >> 8) & 0xffu) - 8.0f) * d;
    r.z = (static_cast<float>((nib >> 16) & 0xffu) - 8.0f) * d;
    r.w = (static_cast<float>(nib >> 24) - 8.0f) * d;
    // output element of this lane's r.x: 32b + j (low) or 32b + 16 + j (high)
    const size_t e = (blk0 + b) * kQK + (part < 4 ? 0 : kQK / 2) + j;
    if constexpr (kVecOut) {
      store_stream(r, reinterpret_cast<float4 *>(y + e));
    } else {
      y[e] = r.x;
      y[e + 1] = r.y;
      y[e + 2] = r.z;
      y[e + 3] = r.w;
    }
  }
}

// ---------------------------------------------------------------------------
// a10: f32 -> block_q8_0 (RVVOps.td:8345-8431; ggml riscv/quants.c RVV path).
// Eight lanes own one 32-float block (one float4 each):
//   amax = max|x|; d = amax/127.0f; id = d ? 1/d : 0; y.d = (_Float16)d (RNE);
//   q = (int8)(int16)sat_rne(x*id)   (vfncvt_x_f_w_i16 then vncvt_x_x_w_i8).
// Division and reciprocal are the correctly rounded IEEE operations, as the
// reference's scalar `amax / 127.0f` and `1.0f/d` are.  A work-group stages
// its kQzBlocks output blocks (64*34 = 2176 bytes, a 16-byte multiple) in LDS
// and writes them with 128-bit stores.  Loads and stores are nontemporal
// (4096^2 over 5 rotating sets, past the Infinity Cache, interleaved runs:
// 14.89 against 16.05-16.19 us with ordinary ones).
// ---------------------------------------------------------------------------
constexpr int kQzThreads = 256;
// blocks per 8-lane group (streaming, 4096^2: 1/2/4 15.81/14.89/15.59 us; 128
// threads with 2 15.64, 512 slower also without streaming)
constexpr int kQzPer = 2;
constexpr int kQzBlocks = kQzPer * kQzThreads / 8;

// Branch-free: the clamp to the i16 range (v_med3_f32) commutes with the
// rounding, as both bounds are integers; NaN is selected afterwards, since the
// clamp would map it to a bound.  (Written with branches the compiler gave
// every element its own exec-mask block: 340 instructions against 271.)
__device__ __forceinline__ uint32_t quant_byte(float x, float id) {
  const float v = x * id;
  const float r = fminf(fmaxf(__builtin_rintf(v), -32768.0f), 32767.0f);  // rint: nearest-even
  // RVV float->int conversion of NaN gives the largest value
  const int w = v != v ? 32767 : static_cast<int>(r);
  return static_cast<uint32_t>(w) & 0xffu;  // narrowing keeps the low byte
}

// max of v over the 8 lanes of its group: quad_perm [1,0,3,2] and [2,3,0,1]
// give each quad's max, row_half_mirror pairs lane i with lane 7-i of the
// other quad (fmaxf is exact and order-free)
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                  0xB1, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                  0x4E, 0xf, 0xf, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                  0x141, 0xf, 0xf, false)));
  return v;
}

// kVec: x is 16-byte aligned (128-bit loads); otherwise 4-byte loads.  Each
// thread quantizes kQzPer blocks' parts; all its loads are issued first
// (lanes of absent blocks re-read the last block and store nothing).
template <bool kVec>
__global__ __launch_bounds__(kQzThreads) void quantize_q8_0(const float *x, uint8_t *vy,
                                                            size_t nb) {
  __shared__ __align__(16) uint8_t lds[kQzBlocks * kQ8Bytes];
  const size_t blk0 = static_cast<size_t>(blockIdx.x) * kQzBlocks;
  const int nblk = static_cast<int>(min(static_cast<size_t>(kQzBlocks), nb - blk0));
  const int part = threadIdx.x & 7;  // float4 within the block
  float4 v[kQzPer];
#pragma unroll
  for (int k = 0; k < kQzPer; ++k) {
    const int lb = (threadIdx.x >> 3) + k * (kQzThreads / 8);  // block within the work-group
    const float *xp = x + (blk0 + min(lb, nblk - 1)) * kQK + 4 * part;
    if constexpr (kVec)
      v[k] = load_stream(xp);
    else
      v[k] = make_float4(xp[0], xp[1], xp[2], xp[3]);
  }
#pragma unroll
  for (int k = 0; k < kQzPer; ++k) {
    const int lb = (threadIdx.x >> 3) + k * (kQzThreads / 8);
    // seeded with 0.0f as the reference's reduction is: NaN elements are
    // skipped, and an all-NaN block has amax = 0 (d = 0, id = 0)
    const float amax = fmaxf(max8(fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)),
                                        fmaxf(fabsf(v[k].z), fabsf(v[k].w)))),
                             0.0f);
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __frcp_rn(d) : 0.0f;
    if (lb < nblk) {
      uint16_t *l16 = reinterpret_cast<uint16_t *>(lds + lb * kQ8Bytes);
      const uint32_t b0 = quant_byte(v[k].x, id), b1 = quant_byte(v[k].y, id);
      const uint32_t b2 = quant_byte(v[k].z, id), b3 = quant_byte(v[k].w, id);
      l16[1 + part * 2] = static_cast<uint16_t>(b0 | (b1 << 8));
      l16[2 + part * 2] = static_cast<uint16_t>(b2 | (b3 << 8));
      if (part == 0)
        l16[0] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(d));
    }
  }
  __syncthreads();
  copy_lds_to_span_stream(vy + blk0 * kQ8Bytes, lds, nblk * kQ8Bytes, threadIdx.x, kQzThreads);
}

}  // namespace

extern "C" {

const char *tcrv_hip_status_string(int status) {
  switch (status) {
  case TCRV_HIP_OK:
    return "ok";
  case TCRV_HIP_ERR_NULL_POINTER:
    return "null pointer argument";
  case TCRV_HIP_ERR_BAD_SIZE:
    return "size or stride violates the kernel contract";
  case TCRV_HIP_ERR_MISALIGNED:
    return "pointer or stride is not aligned as required";
  case TCRV_HIP_ERR_TOO_LARGE:
    return "size exceeds the kernel's index range";
  case TCRV_HIP_ERR_UNSUPPORTED:
    return "argument combination not supported";
  case TCRV_HIP_ERR_SCRATCH_LIMIT:
    return "the call needs more than the entry's fixed device scratch";
  default:
    break;
  }
  if (status > 0)
    return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

const char *tcrv_hip_version(void) { return "tcrv_hip 0.1.0 gfx950"; }

int tcrv_hip_stream_synchronize(void *stream) {
  return static_cast<int>(hipStreamSynchronize(tcrv_host::as_stream(stream)));
}

int tcrv_hip_add_f32(const float *lhs, const float *rhs, float *out, size_t n, void *stream) {
  using namespace tcrv_host;
  if (n == 0)
    return TCRV_HIP_OK;
  if (!lhs || !rhs || !out)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned4(lhs) || !aligned4(rhs) || !aligned4(out))
    return TCRV_HIP_ERR_MISALIGNED;
  hipStream_t st = as_stream(stream);
  size_t done = 0;
  if (aligned16(lhs) && aligned16(rhs) && aligned16(out)) {
    const size_t n4 = n / 4;
    if (n4 > 0) {
      const size_t per = static_cast<size_t>(kAddThreads) * kAddUnroll;
      const size_t grid = (n4 + per - 1) / per;
      if (grid > 0x7fffffffu)
        return TCRV_HIP_ERR_TOO_LARGE;
      add_f32_vec4<<<dim3(static_cast<unsigned>(grid)), dim3(kAddThreads), 0, st>>>(
          reinterpret_cast<const float4 *>(lhs), reinterpret_cast<const float4 *>(rhs),
          reinterpret_cast<float4 *>(out), n4);
      done = n4 * 4;
    }
  }
  if (done < n) {
    const size_t rest = n - done;
    const size_t grid = (rest + kAddThreads - 1) / kAddThreads;
    if (grid > 0x7fffffffu)
      return TCRV_HIP_ERR_TOO_LARGE;
    add_f32_scalar<<<dim3(static_cast<unsigned>(grid)), dim3(kAddThreads), 0, st>>>(
        lhs, rhs, out, done, n);
  }
  return launch_status();
}

int tcrv_hip_dequantize_row_q8_0(const uint8_t *vx, float *y, size_t n, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / kQK;
  if (nb == 0)
    return TCRV_HIP_OK;
  if (!vx || !y)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(vx) || !aligned4(y))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t grid = (nb + kDqBlocks - 1) / kDqBlocks;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (aligned16(y))
    dequantize_q8_0<true><<<dim3(static_cast<unsigned>(grid)), dim3(kDqThreads), 0,
                            as_stream(stream)>>>(vx, y, nb);
  else
    dequantize_q8_0<false><<<dim3(static_cast<unsigned>(grid)), dim3(kDqThreads), 0,
                             as_stream(stream)>>>(vx, y, nb);
  return launch_status();
}

int tcrv_hip_dequantize_row_q4_0(const uint8_t *vx, float *y, size_t n, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / kQK;
  if (nb == 0)
    return TCRV_HIP_OK;
  if (!vx || !y)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned2(vx) || !aligned4(y))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t grid = (nb + kDq4Blocks - 1) / kDq4Blocks;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (aligned16(y))
    dequantize_q4_0<true><<<dim3(static_cast<unsigned>(grid)), dim3(kDq4Threads), 0,
                            as_stream(stream)>>>(vx, y, nb);
  else
    dequantize_q4_0<false><<<dim3(static_cast<unsigned>(grid)), dim3(kDq4Threads), 0,
                             as_stream(stream)>>>(vx, y, nb);
  return launch_status();
}

int tcrv_hip_quantize_row_q8_0(size_t n, const float *x, uint8_t *vy, void *stream) {
  using namespace tcrv_host;
  const size_t nb = n / kQK;
  if (nb == 0)
    return TCRV_HIP_OK;
  if (!x || !vy)
    return TCRV_HIP_ERR_NULL_POINTER;
  if (!aligned4(x) || !aligned2(vy))
    return TCRV_HIP_ERR_MISALIGNED;
  const size_t grid = (nb + kQzBlocks - 1) / kQzBlocks;
  if (grid > 0x7fffffffu)
    return TCRV_HIP_ERR_TOO_LARGE;
  if (aligned16(x))
    quantize_q8_0<true><<<dim3(static_cast<unsigned>(grid)), dim3(kQzThreads), 0,
                          as_stream(stream)>>>(x, vy, nb);
  else
    quantize_q8_0<false><<<dim3(static_cast<unsigned>(grid)), dim3(kQzThreads), 0,
                           as_stream(stream)>>>(x, vy, nb);
  return launch_status();
}

}  // extern "C"
