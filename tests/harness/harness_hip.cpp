// harness_hip.cpp -- a C++ host program driving libtcrv_hip the way the
// reference's qemu harness drives its generated kernel
// (examples/qemu/harness_add.cpp:13-33): declare the entry, supply inputs,
// call, check every element against a scalar reference.  TEST INFRASTRUCTURE:
// the scalar references here are the oracle library (oracle/tcrv_oracle.h).
//
//   1. the reference's own add proof (i32, n = 1031, lhs = 3i - 17,
//      rhs = 41 - 2i) through tcrv_hip_add_i32;
//   2. the route provider's selection for every combination of typed facts;
//   3. routed decode GEMVs and prefill GEMMs (Q4_0 and Q8_0 weights, and the
//      repack GEMM over x16 Q4_0 weights) on
//      quantized synthetic rows, each output compared bit for bit with the
//      oracle.
// Prints one line per step and "harness ok" last; exits non-zero on any
// mismatch or failed call.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "tcrv_hip.h"
#include "tcrv_hip_route.h"
#include "tcrv_oracle.h"

namespace {

int fail(const char *what, int status) {
  std::printf("FAIL %s: %d (%s)\n", what, status, tcrv_hip_status_string(status));
  return 1;
}

#define HIP_OK(call)                                                        \
  do {                                                                      \
    hipError_t e_ = (call);                                                 \
    if (e_ != hipSuccess) {                                                 \
      std::printf("FAIL %s: %s\n", #call, hipGetErrorString(e_));          \
      return 1;                                                             \
    }                                                                       \
  } while (0)

// splitmix64 -> uniform (-1, 1)
struct Rng {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  float uniform() { return static_cast<float>((next() >> 40) * (2.0 / 16777216.0) - 1.0); }
};

template <typename T>
struct DeviceBuffer {
  T *p = nullptr;
  explicit DeviceBuffer(size_t n) {
    if (hipMalloc(reinterpret_cast<void **>(&p), n * sizeof(T)) != hipSuccess)
      p = nullptr;
  }
  ~DeviceBuffer() {
    if (p)
      (void)hipFree(p);
  }
};

int add_proof() {
  const size_t n = 1031;  // not a multiple of any vector width: the tail path
  std::vector<int32_t> lhs(n), rhs(n), out(n), want(n);
  for (size_t i = 0; i < n; ++i) {
    lhs[i] = static_cast<int32_t>(i * 3 - 17);
    rhs[i] = static_cast<int32_t>(41 - static_cast<int32_t>(i * 2));
  }
  tcrv_oracle_add_i32(lhs.data(), rhs.data(), want.data(), n);
  DeviceBuffer<int32_t> dl(n), dr(n), dout(n);
  if (!dl.p || !dr.p || !dout.p) {
    std::printf("FAIL hipMalloc (is a GPU visible?)\n");
    return 1;
  }
  HIP_OK(hipMemcpy(dl.p, lhs.data(), n * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dr.p, rhs.data(), n * 4, hipMemcpyHostToDevice));
  const int st = tcrv_hip_add_i32(dl.p, dr.p, dout.p, n, nullptr);
  if (st != TCRV_HIP_OK)
    return fail("tcrv_hip_add_i32", st);
  HIP_OK(hipMemcpy(out.data(), dout.p, n * 4, hipMemcpyDeviceToHost));
  for (size_t i = 0; i < n; ++i)
    if (out[i] != want[i] || out[i] != lhs[i] + rhs[i]) {
      std::printf("FAIL add mismatch at %zu: got %d expected %d\n", i, out[i], want[i]);
      return 1;
    }
  std::printf("add proof ok: %zu elements checked\n", n);
  return 0;
}

int route_matrix() {
  const char *quant[] = {"q4_0", "q8_0", "q4_K"};
  const char *regime[] = {"decode", "prefill"};
  const char *layout[] = {"plain", "x16"};
  for (int q = 0; q < 3; ++q)
    for (int m = 0; m < 2; ++m)
      for (int l = 0; l < 2; ++l) {
        int algo = -1;
        const char *reason = nullptr, *entry = nullptr;
        const int st = tcrv_hip_route_select(q, m, l, &algo, &reason, &entry);
        if (st != TCRV_HIP_OK)
          return fail("tcrv_hip_route_select", st);
        std::printf("route %s %s %s -> %d %s %s\n", quant[q], regime[m], layout[l], algo, reason,
                    entry ? entry : "-");
      }
  return 0;
}

// nrows rows of n floats quantized to Q8_0 (q8 = true) or Q4_0, scale `amp`.
std::vector<uint8_t> quantized_rows(size_t nrows, size_t n, uint64_t seed, float amp, bool q8) {
  Rng rng{seed};
  std::vector<float> x(n);
  const size_t rb = (n / 32) * (q8 ? 34 : 18);
  std::vector<uint8_t> out(nrows * rb);
  for (size_t r = 0; r < nrows; ++r) {
    for (auto &v : x)
      v = amp * rng.uniform();
    if (q8)
      tcrv_oracle_quantize_row_q8_0(n, x.data(), out.data() + r * rb);
    else
      tcrv_oracle_quantize_row_q4_0(n, x.data(), out.data() + r * rb);
  }
  return out;
}

int routed_contraction(const char *name, int quant, size_t nr, size_t nc, size_t n,
                       int want_algo) {
  const bool q4 = quant == TCRV_HIP_QUANT_Q4_0;
  const size_t nb = n / 32, wb = nb * (q4 ? 18 : 34), ab = nb * 34;
  const std::vector<uint8_t> w = quantized_rows(nr, n, 1006 + nr, 0.02f, !q4);
  const std::vector<uint8_t> a = quantized_rows(nc, n, 1007 + nc, 1.0f, true);
  std::vector<float> got(nr * nc), want(nr * nc);
  if (q4)
    tcrv_oracle_gemm_q4_0_q8_0(n, want.data(), w.data(), a.data(), ab, nr, nc, wb, nc, 1);
  else
    tcrv_oracle_gemm_q8_0_q8_0(n, want.data(), w.data(), a.data(), ab, nr, nc, wb, nc, 1);
  DeviceBuffer<uint8_t> dw(w.size()), da(a.size());
  DeviceBuffer<float> ds(got.size());
  if (!dw.p || !da.p || !ds.p) {
    std::printf("FAIL hipMalloc (is a GPU visible?)\n");
    return 1;
  }
  HIP_OK(hipMemcpy(dw.p, w.data(), w.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(da.p, a.data(), a.size(), hipMemcpyHostToDevice));
  int algo = -1;
  const int st = tcrv_hip_route_contraction(quant, TCRV_HIP_LAYOUT_PLAIN, n, ds.p, dw.p, da.p,
                                            ab, nr, nc, wb, nc, nullptr, &algo);
  if (st != TCRV_HIP_OK)
    return fail(name, st);
  if (algo != want_algo) {
    std::printf("FAIL %s: routed to algorithm %d, expected %d\n", name, algo, want_algo);
    return 1;
  }
  HIP_OK(hipMemcpy(got.data(), ds.p, got.size() * 4, hipMemcpyDeviceToHost));
  for (size_t i = 0; i < got.size(); ++i)
    if (std::memcmp(&got[i], &want[i], 4) != 0) {
      std::printf("FAIL %s mismatch at %zu: got %.9g expected %.9g\n", name, i, got[i], want[i]);
      return 1;
    }
  std::printf("%s ok: %zu x %zu x %zu bit-identical to the oracle (algorithm %d)\n", name, nr, nc,
              n, algo);
  return 0;
}

// Prefill over x16 Q4_0 weights: the route runs the repack GEMM in its own
// contract (activations in block_q8_0x4, output activation-row major); both
// layouts are built here with the oracle's packs.
int routed_repack_gemm(size_t nr, size_t nc, size_t n) {
  const char *name = "routed q4_0 x16 prefill";
  const size_t nb = n / 32;
  const std::vector<uint8_t> w = quantized_rows(nr, n, 1006 + nr, 0.02f, false);
  const std::vector<uint8_t> a = quantized_rows(nc, n, 1007 + nc, 1.0f, true);
  // group x, block b of the x16 source: block b of rows 16x .. 16x+15
  std::vector<uint8_t> src(w.size()), wx16(nr / 16 * nb * 288), ax4(nc / 4 * nb * 136);
  for (size_t x = 0; x < nr / 16; ++x)
    for (size_t b = 0; b < nb; ++b)
      for (size_t r = 0; r < 16; ++r)
        std::memcpy(&src[((x * nb + b) * 16 + r) * 18], &w[(16 * x + r) * nb * 18 + b * 18], 18);
  tcrv_oracle_pack_q4_0_to_q4_0x16(nr / 16 * nb, src.data(), wx16.data());
  tcrv_oracle_pack_q8_0_to_q8_0x4(nc, nb, a.data(), nb * 34, ax4.data());
  std::vector<float> got(nc * nr), want(nc * nr);
  tcrv_oracle_repack_gemm_q4_0_q8_0(n, want.data(), wx16.data(), ax4.data(), nc, nr, nr);
  DeviceBuffer<uint8_t> dw(wx16.size()), da(ax4.size());
  DeviceBuffer<float> ds(got.size());
  if (!dw.p || !da.p || !ds.p) {
    std::printf("FAIL hipMalloc (is a GPU visible?)\n");
    return 1;
  }
  HIP_OK(hipMemcpy(dw.p, wx16.data(), wx16.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(da.p, ax4.data(), ax4.size(), hipMemcpyHostToDevice));
  int algo = -1;
  const int st = tcrv_hip_route_contraction(TCRV_HIP_QUANT_Q4_0, TCRV_HIP_LAYOUT_X16, n, ds.p,
                                            dw.p, da.p, 0, nr, nc, 0, nr, nullptr, &algo);
  if (st != TCRV_HIP_OK)
    return fail(name, st);
  if (algo != TCRV_HIP_ALGO_REPACK_GEMM) {
    std::printf("FAIL %s: routed to algorithm %d\n", name, algo);
    return 1;
  }
  HIP_OK(hipMemcpy(got.data(), ds.p, got.size() * 4, hipMemcpyDeviceToHost));
  for (size_t i = 0; i < got.size(); ++i)
    if (std::memcmp(&got[i], &want[i], 4) != 0) {
      std::printf("FAIL %s mismatch at %zu: got %.9g expected %.9g\n", name, i, got[i], want[i]);
      return 1;
    }
  std::printf("%s ok: %zu x %zu x %zu bit-identical to the oracle (algorithm %d)\n", name, nr, nc,
              n, algo);
  return 0;
}

}  // namespace

int main() {
  std::printf("%s\n", tcrv_hip_version());
  if (add_proof() || route_matrix() ||
      routed_contraction("routed q4_0 decode", TCRV_HIP_QUANT_Q4_0, 256, 1, 1024,
                         TCRV_HIP_ALGO_DECODE_GEMV) ||
      routed_contraction("routed q8_0 decode", TCRV_HIP_QUANT_Q8_0, 96, 1, 512,
                         TCRV_HIP_ALGO_DECODE_GEMV) ||
      routed_contraction("routed q8_0 prefill", TCRV_HIP_QUANT_Q8_0, 160, 72, 512,
                         TCRV_HIP_ALGO_MFMA_GEMM) ||
      routed_contraction("routed q4_0 prefill", TCRV_HIP_QUANT_Q4_0, 130, 40, 256,
                         TCRV_HIP_ALGO_MFMA_GEMM) ||
      routed_repack_gemm(272, 44, 352))
    return 1;
  std::printf("harness ok\n");
  return 0;
}
