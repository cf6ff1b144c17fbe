// No-allocation variant of the routed layer/block entry point, for callers
// that cannot call hipMalloc (code under HIP graph capture, tight serving
// loops, harnesses that forbid allocation).  It has no counterpart in the
// reference.
//
// Its workspace (pair table, h, per-pair w2 rows, router scores, the
// official requantised x, route completion counters, x and h exponent
// windows: the same layout a context allocates) is the file-scope
// device array `scratch`, one copy per GPU, held until the process ends.  In
// host code `scratch` names a host-side stand-in, not a device address, so
// host code never passes it to a kernel: the first call on a device, with
// that device current, looks up its device address with hipGetSymbolAddress
// and keeps it per device, and every launch uses that pointer.  Only a
// successful set-up is kept: a call whose set-up fails returns the error and
// the next call on that device tries again.  The set-up also enqueues, on
// the caller's stream, a kernel that zeroes the route completion counters
// and the status line (the array starts zeroed as static storage; every
// route launch leaves the counters at zero again).  When the caller is
// capturing that stream into a graph, the lookup runs with this thread's
// capture mode relaxed (it is no stream operation) and the clear is
// recorded into the graph, where it runs ahead of the captured route on
// every replay.
//
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// (different streams or threads) race on it.  Bad routes and non-resident
// pages are reported only as NaN outputs of the affected tokens: the status
// bits the launches leave in the array have no reader here.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "s14_device.hpp"
#include "s14_internal.hpp"

namespace {

static __device__ __align__(256) uint8_t scratch[s14::kWorkspaceBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::mutex mu;
  std::atomic<void *> ptr{nullptr};  // device address of this GPU's `scratch`, once set up
};
DeviceScratch g_devices[kMaxDevices];

// The device address of the calling thread's current device's `scratch`,
// set up on the first successful call.
int device_scratch(int device, hipStream_t stream, void **out) {
  DeviceScratch &d = g_devices[device];
  if (void *p = d.ptr.load(std::memory_order_acquire)) {
    *out = p;
    return S14_OK;
  }
  std::lock_guard<std::mutex> lock(d.mu);
  if (void *p = d.ptr.load(std::memory_order_relaxed)) {
    *out = p;
    return S14_OK;
  }
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  hipError_t e = hipThreadExchangeStreamCaptureMode(&mode);
  if (e != hipSuccess) return s14::fail(S14_ERR_HIP, "hipThreadExchangeStreamCaptureMode: %s", hipGetErrorString(e));
  void *p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  const hipError_t r = hipThreadExchangeStreamCaptureMode(&mode);  // the caller's mode again
  if (e != hipSuccess || !p)
    return s14::fail(S14_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  if (r != hipSuccess) return s14::fail(S14_ERR_HIP, "hipThreadExchangeStreamCaptureMode: %s", hipGetErrorString(r));
  const hipError_t c = s14::launch_clear_route_counters(stream, s14::workspace_carve(p));
  if (c != hipSuccess) return s14::fail(S14_ERR_HIP, "route counter clear: %s", hipGetErrorString(c));
  d.ptr.store(p, std::memory_order_release);
  *out = p;
  return S14_OK;
}

}  // namespace

extern "C" uint64_t s14_noalloc_scratch_bytes(void) { return s14::kWorkspaceBytes; }

extern "C" int s14_moe_block_route_noalloc(void *stream, uint32_t tokens, const s14_router *router,
                                          const uint64_t *expert_pages_dev, const uint8_t *shared_page,
                                          int shared_format, const float *x, float *y, uint16_t *ids_out,
                                          float *weights_out, int mode) {
  // sizes beyond the scratch array's capacity (more than kMaxTokens tokens)
  // are rejected here, with the other argument checks
  if (int rc = s14::block_route_validate(tokens, router, expert_pages_dev, shared_page, shared_format, x, y, mode))
    return rc;
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return s14::fail(S14_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (device < 0 || device >= kMaxDevices)
    return s14::fail(S14_ERR_INVALID, "device %d outside the %d devices this entry point serves", device, kMaxDevices);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void *base = nullptr;
  if (int rc = device_scratch(device, st, &base)) return rc;
  return s14::block_route_launch(st, s14::workspace_carve(base), tokens, router, expert_pages_dev, shared_page,
                                 shared_format, x, y, ids_out, weights_out, mode, nullptr, nullptr);
}
