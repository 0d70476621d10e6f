// kd_attn_bwd_noalloc: the whole backward (kd_attn_bwd) with its workspace in
// library-owned device memory, for callers that cannot allocate (code under
// HIP graph capture, serving loops, harnesses that forbid hipMalloc).
//
// The workspace kd_attn_bwd takes in a->delta -- -Delta and -LSE / c, 2 B H T
// floats, fully written by the dQ kernel before the dK/dV kernel reads it --
// lives here in a file-scope __device__ array of KD_NOALLOC_WORKSPACE_FLOATS.
// Every GPU the library runs on holds its own copy of the array until the
// process ends.  Its address on a device comes from hipGetSymbolAddress, once
// per device, with that device current; host code uses only that address,
// never the array's name (a host-side stand-in).  Nothing here allocates.
//
// All calls on one GPU share its array: calls that overlap on one GPU (two
// streams, two threads) race on it and must be ordered by the caller.
#include <mutex>

#include "kd_internal.h"

namespace {

__device__ __align__(256) float scratch[KD_NOALLOC_WORKSPACE_FLOATS];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_ptr[kMaxDevices] = {};

// The array's device address on the current device (resolved on first use).
int scratch_ptr(float** out, const char** err) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *err = "no current HIP device (or device index >= 64)";
    return KD_ERR_LAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      *err = "hipGetSymbolAddress of the workspace array failed";
      return KD_ERR_LAUNCH;
    }
    g_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_ptr[dev];
  return KD_OK;
}

}  // namespace

namespace kd {

int noalloc_workspace(float** out, const char** err) { return scratch_ptr(out, err); }

}  // namespace kd
