// gemm_noalloc.hip -- tcrv_hip_q8_0_q8_0_gemm_noalloc: the Q8_0 x Q8_0 GEMM of
// tcrv_hip_q8_0_q8_0_gemm_ws with its workspace (the two operands in the
// GEMM-tile layout) in a file-scope device array instead of caller memory, for
// callers that cannot allocate device memory (code under HIP graph capture,
// serving loops that forbid hipMalloc).
//
// The array, `scratch`, is kScratchBytes on every GPU the entry runs on, held
// until the process ends.  It lives in this translation unit alone, so its
// code object (and the array) is loaded on a device only when the entry is
// first called there.  Host code never uses the array's name as an address
// (on the host it names a stand-in): the device address comes from
// hipGetSymbolAddress, once per device, with that device current, and is kept
// per device.
//
// Every call on one GPU shares that GPU's array; the pack kernels rewrite
// every byte the GEMM reads, so no call depends on what an earlier one left.
// Calls that overlap in time on one GPU (two streams, two host threads) race
// on it; the caller orders them.
#include <mutex>

#include "tcrv_hip_internal.h"

constexpr size_t kScratchBytes = static_cast<size_t>(64) << 20;  // 64 MiB

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mutex;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the device `st` runs on (looked up on
// the first call there).  Returns TCRV_HIP_OK or a HIP error.
int scratch_of(hipStream_t st, uint8_t **out) {
  int dev = 0, cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess)
    e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess)
    return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices)
    return TCRV_HIP_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
      return static_cast<int>(e);
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = dev != cur ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess)
      return static_cast<int>(e);
    if (back != hipSuccess)
      return static_cast<int>(back);
    if (!p)
      return static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = static_cast<uint8_t *>(p);
  }
  *out = g_scratch_ptr[dev];
  return TCRV_HIP_OK;
}

}  // namespace

extern "C" {

size_t tcrv_hip_q8_0_q8_0_gemm_noalloc_max_bytes(void) { return kScratchBytes; }

int tcrv_hip_q8_0_q8_0_gemm_noalloc(size_t n, float *s, const uint8_t *vx, const uint8_t *vy,
                                    size_t by, size_t nr, size_t nc, size_t bx, size_t bs,
                                    void *stream) {
  using namespace tcrv_host;
  // the shapes tcrv_hip_q8_0_q8_0_gemm_ws runs without its workspace (the
  // plain GEMM) need no scratch, and do not look its address up (the lookup
  // is the call that must stay outside a graph capture)
  if (!gemm_ws_uses_workspace(n, vx, bx, vy, by, nr, nc))
    return tcrv_hip_q8_0_q8_0_gemm_ws(n, s, vx, vy, by, nr, nc, bx, bs, nullptr, 0, stream);
  if (tcrv_hip_q8_0_q8_0_gemm_workspace_bytes(n, nr, nc) > kScratchBytes)
    return TCRV_HIP_ERR_SCRATCH_LIMIT;
  uint8_t *ws = nullptr;
  const int rc = scratch_of(as_stream(stream), &ws);
  if (rc != TCRV_HIP_OK)
    return rc;
  return tcrv_hip_q8_0_q8_0_gemm_ws(n, s, vx, vy, by, nr, nc, bx, bs, ws, kScratchBytes, stream);
}

}  // extern "C"
