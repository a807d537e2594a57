// hw_probes.hip -- microbenchmarks behind the design limits quoted for the
// GEMV and GEMM (not part of libtcrv_hip.so):
//   mix<kMode>: per iteration two v_mfma_i32_32x32x32_i8 (independent
//     accumulator chains) and/or 64 independent v_fma_f32, to see whether the
//     matrix core and the fp32 VALU overlap on one SIMD.
//       0: MFMA only   1: VALU only   2: both in every wave
//       3: waves 0-3 of a 512-thread work-group MFMA only, waves 4-7 VALU only
//   fold<kMode>: the GEMM's per-tile inner loop with its operands resident in
//     LDS (16 waves per CU, 4 per SIMD, no global memory), parts switched on
//     one at a time, to price each against the full loop:
//       0: i8 MFMA + 2-block f32 MFMA (d_x*d_y) + cvt/fma fold (the GEMM loop)
//       1: MFMAs only   2: i8 MFMA only
//       3: VALU only, 48 instructions per tile and block (xor, cvt, fma)
//   empty: the cost of one launch with no work (launch floor in a HIP graph)
//   read_only: streams `n16` 16-byte chunks, one 128-bit load per chunk (the
//     floor for a kernel that reads the GEMV's 9.4 MB once)
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <int kMode>
__global__ __launch_bounds__(512) void mix(const int *in, float *out, int iters) {
  const v4i a = *reinterpret_cast<const v4i *>(in + 4 * (threadIdx.x & 255));
  const v4i b = *reinterpret_cast<const v4i *>(in + 4 * (threadIdx.x & 255) + 1024);
  v16i c0 = {}, c1 = {};
  float acc[32];
  const float x = in[threadIdx.x & 7] * 1e-3f, y = in[(threadIdx.x + 3) & 7] * 1e-3f;
  for (int i = 0; i < 32; ++i)
    acc[i] = static_cast<float>(in[i]);
  const int w = threadIdx.x >> 6;
  const bool do_mfma = kMode == 0 || kMode == 2 || (kMode == 3 && w < 4);
  const bool do_valu = kMode == 1 || kMode == 2 || (kMode == 3 && w >= 4);
  for (int it = 0; it < iters; ++it) {
    if (do_mfma) {
      c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
    }
    if (do_valu) {
#pragma unroll
      for (int k = 0; k < 32; ++k)
        acc[k] = fmaf(acc[k], x, y);
#pragma unroll
      for (int k = 0; k < 32; ++k)
        acc[k] = fmaf(acc[k], y, x);
    }
  }
  float r = 0.0f;
  for (int e = 0; e < 16; ++e)
    r += static_cast<float>(c0[e] + c1[e]);
  for (int i = 0; i < 32; ++i)
    r += acc[i];
  out[blockIdx.x * 512 + threadIdx.x] = r;
}

typedef float v32f __attribute__((ext_vector_type(32)));

template <int kMode, bool kClock = false>
__global__ __launch_bounds__(1024, 1) void fold(const int *in, float *out, int iters,
                                                long long *clk = nullptr) {
  __shared__ __align__(16) int8_t q[256 * 272];
  __shared__ __align__(16) float dsc[8][256];
  const int tid = threadIdx.x;
  for (int i = tid; i < 256 * 272 / 4; i += 1024)
    reinterpret_cast<int *>(q)[i] = in[i & 1023];
  for (int i = tid; i < 8 * 256; i += 1024)
    (&dsc[0][0])[i] = 1.0f / static_cast<float>(1 + (in[i & 1023] & 7));
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63, wm = wave >> 2, wn = wave & 3;
  const int li = lane & 31, h = lane >> 5;
  const int8_t *qa = q + (wm * 32 + li) * 272 + 16 * h;
  const int8_t *qb = q + (128 + wn * 32 + li) * 272 + 16 * h;
  const float *sx = &dsc[h][wm * 32 + li];
  const float *sy = &dsc[h][128 + wn * 32 + li];
  float acc[16];
  for (int e = 0; e < 16; ++e)
    acc[e] = 0.0f;
  v16i iacc = {};
  long long c0 = 0, w0 = 0;
  if (kClock && blockIdx.x == 0 && tid == 0) {
    c0 = clock64();
    w0 = wall_clock64();
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int b = 0; b < 8; b += 2) {
      v32f dxy = {};
      if constexpr (kMode == 0 || kMode == 1)
        dxy = __builtin_amdgcn_mfma_f32_32x32x1f32(sx[b * 256], sy[b * 256], v32f{}, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v4i a = *reinterpret_cast<const v4i *>(qa + (b + j) * 32);
        const v4i bq = *reinterpret_cast<const v4i *>(qb + (b + j) * 32);
        if constexpr (kMode == 0) {
          const v16i sumi = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, v16i{}, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 16; ++e)
            acc[e] = fmaf(static_cast<float>(sumi[e]), dxy[16 * j + e], acc[e]);
        } else if constexpr (kMode == 1 || kMode == 2) {
          iacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, iacc, 0, 0, 0);
        } else {
          const float d = sx[(b + j) * 256];
#pragma unroll
          for (int e = 0; e < 16; ++e)
            acc[e] = fmaf(static_cast<float>(a[e & 3] ^ bq[e >> 2]), d, acc[e]);
        }
      }
      if constexpr (kMode == 1)
        acc[b] += dxy[b] + dxy[31 - b];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (kClock && blockIdx.x == 0 && tid == 0) {
    clk[0] = clock64() - c0;       // shader-clock cycles of this wave's loop
    clk[1] = wall_clock64() - w0;  // constant-rate ticks over the same span
  }
  float r = 0.0f;
  for (int e = 0; e < 16; ++e)
    r += acc[e] + static_cast<float>(iacc[e]);
  out[blockIdx.x * 1024 + tid] = r;
}

__global__ void empty_kernel() {}

// read_wide<kU>: every thread loads kU 16-byte chunks, each wave instruction a
// contiguous 1 KB, one pass over the buffer (grid = n16 / (256 * kU)): the
// streaming-read rate of a large buffer, the roofline of a read-only kernel.
template <int kU>
__global__ __launch_bounds__(256) void read_wide(const uint4 *p, size_t n16, uint32_t *out) {
  const size_t base = static_cast<size_t>(blockIdx.x) * (256 * kU) + threadIdx.x;
  uint4 v[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const size_t i = base + static_cast<size_t>(u) * 256;
    v[u] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < kU; ++u)
    acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (acc == 0x9e3779b9u)  // data-dependent store keeps the loads alive
    out[threadIdx.x] = acc;
}

__global__ __launch_bounds__(256) void read_only(const uint4 *p, size_t n16, uint32_t *out) {
  uint32_t acc = 0;
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * 256) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u)  // data-dependent store keeps the loads alive
    out[threadIdx.x] = acc;
}

extern "C" __attribute__((visibility("default"))) int probe_mix(int mode, const int *in, float *out, int iters, int grid, void *st) {
  hipStream_t s = static_cast<hipStream_t>(st);
  switch (mode) {
  case 0: mix<0><<<grid, 512, 0, s>>>(in, out, iters); break;
  case 1: mix<1><<<grid, 512, 0, s>>>(in, out, iters); break;
  case 2: mix<2><<<grid, 512, 0, s>>>(in, out, iters); break;
  case 3: mix<3><<<grid, 512, 0, s>>>(in, out, iters); break;
  default: return -1;
  }
  return hipGetLastError();
}

extern "C" __attribute__((visibility("default"))) int probe_fold(int mode, const int *in, float *out, int iters, int grid, void *st) {
  hipStream_t s = static_cast<hipStream_t>(st);
  switch (mode) {
  case 0: fold<0><<<grid, 1024, 0, s>>>(in, out, iters); break;
  case 1: fold<1><<<grid, 1024, 0, s>>>(in, out, iters); break;
  case 2: fold<2><<<grid, 1024, 0, s>>>(in, out, iters); break;
  case 3: fold<3><<<grid, 1024, 0, s>>>(in, out, iters); break;
  default: return -1;
  }
  return hipGetLastError();
}

extern "C" __attribute__((visibility("default"))) int probe_empty(void *st) {
  empty_kernel<<<1, 64, 0, static_cast<hipStream_t>(st)>>>();
  return hipGetLastError();
}

extern "C" __attribute__((visibility("default"))) int probe_read(const void *p, size_t nbytes, uint32_t *out, int grid, void *st) {
  read_only<<<grid, 256, 0, static_cast<hipStream_t>(st)>>>(static_cast<const uint4 *>(p),
                                                            nbytes / 16, out);
  return hipGetLastError();
}

extern "C" __attribute__((visibility("default"))) int probe_read_wide(const void *p, size_t nbytes, uint32_t *out, int unroll, void *st) {
  const size_t n16 = nbytes / 16;
  hipStream_t s = static_cast<hipStream_t>(st);
  switch (unroll) {
  case 1: read_wide<1><<<(n16 + 255) / 256, 256, 0, s>>>(static_cast<const uint4 *>(p), n16, out); break;
  case 2: read_wide<2><<<(n16 + 511) / 512, 256, 0, s>>>(static_cast<const uint4 *>(p), n16, out); break;
  case 4: read_wide<4><<<(n16 + 1023) / 1024, 256, 0, s>>>(static_cast<const uint4 *>(p), n16, out); break;
  default: return -1;
  }
  return hipGetLastError();
}

// The shader clock during the GEMM inner loop (fold mode 0): wave 0 of
// work-group 0 records its loop's clock64 and wall_clock64 deltas in clk[0..1].
extern "C" __attribute__((visibility("default"))) int probe_fold_clock(const int *in, float *out, long long *clk, int iters, int grid, void *st) {
  fold<0, true><<<grid, 1024, 0, static_cast<hipStream_t>(st)>>>(in, out, iters, clk);
  return hipGetLastError();
}
