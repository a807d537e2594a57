// harness_hip.cpp -- a C++ host program driving libtcrv_hip the way the
// reference's qemu harness drives its generated kernel
// (examples/qemu/harness_add.cpp:13-33): declare the entry, supply inputs,
// call, check every element against a scalar reference.  TEST INFRASTRUCTURE:
// the scalar references here are the oracle library (oracle/tcrv_oracle.h).
//
//   1. the reference's own add proof (i32, n = 1031, lhs = 3i - 17,
//      rhs = 41 - 2i) through the exported fixture function
//      tcrv_emitc_explicit_selected_body_add_kernel_explicit_selected_body_rvv_i32_add;
//   2. every other exported fixture function (_gen/tcrv_emitc_fixtures.cpp,
//      generated from emitc_fixtures.manifest by the package's export tool),
//      called by its name on synthetic inputs, each output compared bit for bit
//      with the oracle;
//   3. the route provider's selection for every combination of typed facts;
//   4. routed decode GEMVs and prefill GEMMs (Q4_0 and Q8_0 weights) on
//      quantized synthetic rows, and the x16 Q4_0 prefill, whose selected
//      repack GEMM runs in its own ABI, each output compared bit for bit with
//      the oracle.
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
// the generated prototypes, then the fixtures' own: g++ rejects the build if
// any two differ
#include "tcrv_emitc_fixtures.h"
#include "emitc_fixture_prototypes.h"

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
  const int st = tcrv_emitc_explicit_selected_body_add_kernel_explicit_selected_body_rvv_i32_add(
      dl.p, dr.p, dout.p, n, nullptr);
  if (st != TCRV_HIP_OK)
    return fail("exported add", st);
  HIP_OK(hipMemcpy(out.data(), dout.p, n * 4, hipMemcpyDeviceToHost));
  for (size_t i = 0; i < n; ++i)
    if (out[i] != want[i] || out[i] != lhs[i] + rhs[i]) {
      std::printf("FAIL add mismatch at %zu: got %d expected %d\n", i, out[i], want[i]);
      return 1;
    }
  std::printf("add proof ok: %zu elements checked (exported add)\n", n);
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

// ---- the exported fixture functions -------------------------------------

template <typename T>
bool upload(DeviceBuffer<T> &d, const std::vector<T> &h) {
  return d.p && hipMemcpy(d.p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) == hipSuccess;
}

template <typename T>
bool download(std::vector<T> &h, const DeviceBuffer<T> &d) {
  return hipMemcpy(h.data(), d.p, h.size() * sizeof(T), hipMemcpyDeviceToHost) == hipSuccess;
}

// Compares got with want byte for byte and prints the step's line.
template <typename T>
int same(const char *name, const std::vector<T> &got, const std::vector<T> &want,
         const char *shape) {
  for (size_t i = 0; i < got.size(); ++i)
    if (std::memcmp(&got[i], &want[i], sizeof(T)) != 0) {
      std::printf("FAIL exported %s mismatch at element %zu\n", name, i);
      return 1;
    }
  std::printf("exported %s ok: %s bit-identical to the oracle\n", name, shape);
  return 0;
}

std::vector<uint8_t> random_bytes(size_t n, uint64_t seed) {
  Rng rng{seed};
  std::vector<uint8_t> v(n);
  for (auto &b : v)
    b = static_cast<uint8_t>(rng.next() >> 56);
  return v;
}

// x16 source order of nrows plain rows (nb blocks of `bytes` each): group x,
// block b holds block b of rows 16x .. 16x+15.
std::vector<uint8_t> x16_source(const std::vector<uint8_t> &w, size_t nrows, size_t nb,
                                size_t bytes) {
  std::vector<uint8_t> src(w.size());
  for (size_t x = 0; x < nrows / 16; ++x)
    for (size_t b = 0; b < nb; ++b)
      for (size_t r = 0; r < 16; ++r)
        std::memcpy(&src[((x * nb + b) * 16 + r) * bytes], &w[(16 * x + r) * nb * bytes + b * bytes],
                    bytes);
  return src;
}

#define EXPORTED_OK(name, call)              \
  do {                                       \
    const int st_ = (call);                  \
    if (st_ != TCRV_HIP_OK)                  \
      return fail("exported " name, st_);    \
  } while (0)

int exported_variants() {
  const size_t n = 1024, nb = n / 32;
  // Q8_0 . Q8_0 and Q4_0 . Q8_0 block dots (one row pair each)
  {
    const std::vector<uint8_t> x8 = quantized_rows(1, n, 2001, 0.5f, true);
    const std::vector<uint8_t> x4 = quantized_rows(1, n, 2002, 0.5f, false);
    const std::vector<uint8_t> y8 = quantized_rows(1, n, 2003, 1.0f, true);
    DeviceBuffer<uint8_t> dx8(x8.size()), dx4(x4.size()), dy8(y8.size());
    DeviceBuffer<float> ds(1);
    if (!upload(dx8, x8) || !upload(dx4, x4) || !upload(dy8, y8) || !ds.p)
      return fail("upload", -1);
    std::vector<float> got(1), want(1);
    EXPORTED_OK("q8_0 block dot", tcrv_emitc_ggml_vec_dot_q8_0_q8_0_kernel_ggml_vec_dot_q8_0_q8_0(
                                      n, ds.p, dx8.p, dy8.p, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, ds))
      return fail("download", -1);
    tcrv_oracle_vec_dot_q8_0_q8_0(n, want.data(), x8.data(), y8.data());
    if (same("q8_0 block dot", got, want, "K 1024"))
      return 1;
    EXPORTED_OK("q4_0 block dot", tcrv_emitc_ggml_vec_dot_q4_0_q8_0_kernel_ggml_vec_dot_q4_0_q8_0(
                                      n, ds.p, 0, dx4.p, 0, dy8.p, 0, 1, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, ds))
      return fail("download", -1);
    tcrv_oracle_vec_dot_q4_0_q8_0(n, want.data(), 0, x4.data(), 0, y8.data(), 0, 1);
    if (same("q4_0 block dot", got, want, "K 1024"))
      return 1;
  }
  // the Q4_0 GEMM (ragged 37 x 11) and its one-row tile (activation_cols = 4)
  {
    const size_t nr = 37, nc = 11, wb = nb * 18, ab = nb * 34;
    const std::vector<uint8_t> w = quantized_rows(nr, n, 2004, 0.02f, false);
    const std::vector<uint8_t> a = quantized_rows(nc, n, 2005, 1.0f, true);
    DeviceBuffer<uint8_t> dw(w.size()), da(a.size());
    DeviceBuffer<float> ds(nr * nc);
    if (!upload(dw, w) || !upload(da, a) || !ds.p)
      return fail("upload", -1);
    std::vector<float> got(nr * nc), want(nr * nc);
    EXPORTED_OK("q4_0 gemm", tcrv_emitc_ggml_q4_0_q8_0_gemm_kernel_ggml_q4_0_q8_0_gemm(
                                 n, ds.p, dw.p, da.p, ab, nr, nc, wb, nc, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, ds))
      return fail("download", -1);
    tcrv_oracle_gemm_q4_0_q8_0(n, want.data(), w.data(), a.data(), ab, nr, nc, wb, nc, 1);
    if (same("q4_0 gemm", got, want, "37 x 11 x 1024"))
      return 1;
    std::vector<float> tile(4), tile_want(4);
    EXPORTED_OK("q4_0 gemm tile", tcrv_emitc_ggml_q4_0_q8_0_gemm_tile_kernel_ggml_q4_0_q8_0_gemm_tile(
                                      n, ds.p, dw.p, da.p, ab, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(tile, ds))
      return fail("download", -1);
    tcrv_oracle_gemm_q4_0_q8_0(n, tile_want.data(), w.data(), a.data(), ab, 1, 4, wb, 4, 1);
    if (same("q4_0 gemm tile", tile, tile_want, "1 x 4 x 1024"))
      return 1;
  }
  // x16 pack and the repack GEMVs (64 weight rows)
  {
    const size_t rows = 64, groups = rows / 16;
    const std::vector<uint8_t> w4 = quantized_rows(rows, n, 2006, 0.02f, false);
    const std::vector<uint8_t> w8 = quantized_rows(rows, n, 2007, 0.02f, true);
    const std::vector<uint8_t> a = quantized_rows(1, n, 2008, 1.0f, true);
    const std::vector<uint8_t> src4 = x16_source(w4, rows, nb, 18);
    const std::vector<uint8_t> src8 = x16_source(w8, rows, nb, 34);
    std::vector<uint8_t> p4(groups * nb * 288), p4_want(p4.size()), p8(groups * nb * 544);
    tcrv_oracle_pack_q4_0_to_q4_0x16(groups * nb, src4.data(), p4_want.data());
    tcrv_oracle_pack_q8_0_to_q8_0x16(groups * nb, src8.data(), p8.data());
    DeviceBuffer<uint8_t> dsrc(src4.size()), dp4(p4.size()), dp8(p8.size()), da(a.size());
    DeviceBuffer<float> ds(rows);
    if (!upload(dsrc, src4) || !upload(dp8, p8) || !upload(da, a) || !dp4.p || !ds.p)
      return fail("upload", -1);
    EXPORTED_OK("x16 pack", tcrv_emitc_ggml_pack_q4_0_to_q4_0x16_kernel_ggml_pack_q4_0_to_q4_0x16(
                                groups * nb, dsrc.p, dp4.p, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(p4, dp4))
      return fail("download", -1);
    if (same("x16 pack", p4, p4_want, "128 block_q4_0x16"))
      return 1;
    std::vector<float> got(rows), want(rows);
    EXPORTED_OK("q4_0 repack gemv",
                tcrv_emitc_ggml_repack_gemv_q4_0_q8_0_kernel_ggml_repack_gemv_q4_0_q8_0(
                    n, ds.p, dp4.p, da.p, rows, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, ds))
      return fail("download", -1);
    tcrv_oracle_repack_gemv_q4_0_q8_0(n, want.data(), p4_want.data(), a.data(), rows);
    if (same("q4_0 repack gemv", got, want, "64 x 1024"))
      return 1;
    EXPORTED_OK("q8_0 repack gemv",
                tcrv_emitc_ggml_repack_gemv_q8_0_q8_0_kernel_ggml_repack_gemv_q8_0_q8_0(
                    n, ds.p, dp8.p, da.p, rows, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, ds))
      return fail("download", -1);
    tcrv_oracle_repack_gemv_q8_0_q8_0(n, want.data(), p8.data(), a.data(), rows);
    if (same("q8_0 repack gemv", got, want, "64 x 1024"))
      return 1;
  }
  // the repack GEMM: 48 x16 weight rows x 12 x4 activation rows
  {
    const size_t wrows = 48, arows = 12;
    const std::vector<uint8_t> w = quantized_rows(wrows, n, 2009, 0.02f, false);
    const std::vector<uint8_t> a = quantized_rows(arows, n, 2010, 1.0f, true);
    const std::vector<uint8_t> src = x16_source(w, wrows, nb, 18);
    std::vector<uint8_t> wx16(wrows / 16 * nb * 288), ax4(arows / 4 * nb * 136);
    tcrv_oracle_pack_q4_0_to_q4_0x16(wrows / 16 * nb, src.data(), wx16.data());
    tcrv_oracle_pack_q8_0_to_q8_0x4(arows, nb, a.data(), nb * 34, ax4.data());
    DeviceBuffer<uint8_t> dw(wx16.size()), da(ax4.size());
    DeviceBuffer<float> ds(wrows * arows);
    if (!upload(dw, wx16) || !upload(da, ax4) || !ds.p)
      return fail("upload", -1);
    std::vector<float> got(wrows * arows), want(wrows * arows);
    EXPORTED_OK("repack gemm",
                tcrv_emitc_ggml_repack_gemm_q4_0_q8_0_kernel_ggml_repack_gemm_q4_0_q8_0(
                    n, ds.p, dw.p, da.p, arows, wrows, wrows, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, ds))
      return fail("download", -1);
    tcrv_oracle_repack_gemm_q4_0_q8_0(n, want.data(), wx16.data(), ax4.data(), arows, wrows, wrows);
    if (same("repack gemm", got, want, "48 x 12 x 1024"))
      return 1;
  }
  // quantize_row_q8_0 over 97 blocks
  {
    const size_t nq = 97 * 32;
    Rng rng{2011};
    std::vector<float> x(nq);
    for (auto &v : x)
      v = 3.0f * rng.uniform();
    std::vector<uint8_t> got(97 * 34), want(97 * 34);
    tcrv_oracle_quantize_row_q8_0(nq, x.data(), want.data());
    DeviceBuffer<float> dx(nq);
    DeviceBuffer<uint8_t> dy(got.size());
    if (!upload(dx, x) || !dy.p)
      return fail("upload", -1);
    EXPORTED_OK("quantize", tcrv_emitc_quantize_row_q8_0_kernel_quantize_row_q8_0(nq, dx.p, dy.p,
                                                                               nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, dy))
      return fail("download", -1);
    if (same("quantize", got, want, "97 blocks"))
      return 1;
  }
  // both block dequants over 97 blocks of one row (finite scales)
  {
    const size_t nd = 97 * 32;
    const std::vector<uint8_t> q8 = quantized_rows(1, nd, 2015, 0.7f, true);
    const std::vector<uint8_t> q4 = quantized_rows(1, nd, 2016, 0.7f, false);
    std::vector<float> got(nd), want(nd);
    DeviceBuffer<uint8_t> d8(q8.size()), d4(q4.size());
    DeviceBuffer<float> dy(nd);
    if (!upload(d8, q8) || !upload(d4, q4) || !dy.p)
      return fail("upload", -1);
    EXPORTED_OK("q8_0 dequant",
                tcrv_emitc_ggml_dequantize_row_q8_0_kernel_ggml_dequantize_row_q8_0(
                    d8.p, dy.p, nd, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, dy))
      return fail("download", -1);
    tcrv_oracle_dequantize_row_q8_0(nd, want.data(), q8.data());
    if (same("q8_0 dequant", got, want, "97 blocks"))
      return 1;
    EXPORTED_OK("q4_0 dequant",
                tcrv_emitc_ggml_dequantize_row_q4_0_kernel_ggml_dequantize_row_q4_0(
                    d4.p, dy.p, nd, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, dy))
      return fail("download", -1);
    tcrv_oracle_dequantize_row_q4_0(nd, want.data(), q4.data());
    if (same("q4_0 dequant", got, want, "97 blocks"))
      return 1;
  }
  // the integer core over 1003 bytes (the vector and the tail paths)
  {
    const size_t ni = 1003;
    const std::vector<uint8_t> wb = random_bytes(ni, 2012), lb = random_bytes(ni, 2013),
                               hb = random_bytes(ni, 2014);
    std::vector<int8_t> w(wb.begin(), wb.end()), lo(lb.begin(), lb.end()), hi(hb.begin(), hb.end());
    const std::vector<int32_t> acc = {12345};
    std::vector<int32_t> got(1), want(1);
    tcrv_oracle_packed_i4_offset_binary_x_i8_product_reduce(w.data(), lo.data(), hi.data(),
                                                            acc.data(), want.data(), ni);
    DeviceBuffer<int8_t> dw(ni), dlo(ni), dhi(ni);
    DeviceBuffer<int32_t> dacc(1), dout(1);
    if (!upload(dw, w) || !upload(dlo, lo) || !upload(dhi, hi) || !upload(dacc, acc) || !dout.p)
      return fail("upload", -1);
    EXPORTED_OK("integer core",
                tcrv_emitc_rvv_q4_0_q8_0_integer_core_kernel_rvv_q4_0_q8_0_integer_core(
                    dw.p, dlo.p, dhi.p, dacc.p, dout.p, ni, nullptr));
    HIP_OK(hipDeviceSynchronize());
    if (!download(got, dout))
      return fail("download", -1);
    if (same("integer core", got, want, "1003 bytes"))
      return 1;
  }
  return 0;
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

// Prefill over x16 Q4_0 weights: the selection names the repack GEMM, whose
// contract (activations in block_q8_0x4, output activation-row major) is not
// the reference GEMM ABI, so the routed GEMM-ABI call refuses it untouched and
// the caller runs the selected entry in its own ABI; both layouts are built
// here with the oracle's packs.
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
  std::vector<float> got(nc * nr, -5.0f), want(nc * nr);
  tcrv_oracle_repack_gemm_q4_0_q8_0(n, want.data(), wx16.data(), ax4.data(), nc, nr, nr);
  DeviceBuffer<uint8_t> dw(wx16.size()), da(ax4.size());
  DeviceBuffer<float> ds(got.size());
  if (!dw.p || !da.p || !ds.p) {
    std::printf("FAIL hipMalloc (is a GPU visible?)\n");
    return 1;
  }
  HIP_OK(hipMemcpy(dw.p, wx16.data(), wx16.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(da.p, ax4.data(), ax4.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(ds.p, got.data(), got.size() * 4, hipMemcpyHostToDevice));
  int algo = -1;
  int st = tcrv_hip_route_contraction(TCRV_HIP_QUANT_Q4_0, TCRV_HIP_LAYOUT_X16, n, ds.p, dw.p,
                                      da.p, 0, nr, nc, 0, nr, nullptr, &algo);
  if (st != TCRV_HIP_ERR_UNSUPPORTED || algo != TCRV_HIP_ALGO_REPACK_GEMM) {
    std::printf("FAIL %s: the GEMM-ABI call returned %d (algorithm %d), expected a refusal\n",
                name, st, algo);
    return 1;
  }
  const char *reason = nullptr, *entry = nullptr;
  st = tcrv_hip_route_select(TCRV_HIP_QUANT_Q4_0, TCRV_HIP_M_PREFILL, TCRV_HIP_LAYOUT_X16, &algo,
                             &reason, &entry);
  if (st != TCRV_HIP_OK || !entry || std::strcmp(entry, "tcrv_hip_repack_gemm_q4_0_q8_0") != 0)
    return fail("tcrv_hip_route_select (x16 prefill)", st);
  HIP_OK(hipMemcpy(got.data(), ds.p, got.size() * 4, hipMemcpyDeviceToHost));
  for (float v : got)
    if (v != -5.0f) {
      std::printf("FAIL %s: the refused call wrote its output\n", name);
      return 1;
    }
  st = tcrv_hip_repack_gemm_q4_0_q8_0(n, ds.p, dw.p, da.p, nc, nr, nr, nullptr);
  if (st != TCRV_HIP_OK)
    return fail(entry, st);
  HIP_OK(hipMemcpy(got.data(), ds.p, got.size() * 4, hipMemcpyDeviceToHost));
  for (size_t i = 0; i < got.size(); ++i)
    if (std::memcmp(&got[i], &want[i], 4) != 0) {
      std::printf("FAIL %s mismatch at %zu: got %.9g expected %.9g\n", name, i, got[i], want[i]);
      return 1;
    }
  std::printf("%s ok: %zu x %zu x %zu bit-identical to the oracle (selected entry %s, %s)\n",
              name, nr, nc, n, entry, reason);
  return 0;
}

}  // namespace

int main() {
  std::printf("%s\n", tcrv_hip_version());
  if (add_proof() || exported_variants() || route_matrix() ||
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
