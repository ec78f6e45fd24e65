// The library's static device scratch: the workspace of mtk_gemm_run_noalloc, for callers that
// cannot allocate device memory (code under HIP graph capture, serving loops, harnesses that
// forbid hipMalloc). One file-scope device array; each GPU the library is initialised on holds
// its own copy (MTK_NOALLOC_MAX_WORKSPACE bytes) until the process ends.
//
// In host code the array's name is a host-side stand-in, not a device address: the device
// address is taken once per device with hipGetSymbolAddress (scratch_setup, called by mtk_init
// with that device current) and only that address is used afterwards.
#include "scratch.h"

#include <hip/hip_runtime.h>
#include <stdio.h>

#include <mutex>

#include "../../include/mtk.h"

static __device__ __align__(256) unsigned char scratch[MTK_NOALLOC_MAX_WORKSPACE];

namespace mtk_scratch {
namespace {

constexpr int kMaxDevices = 64;

struct Slot {
  bool done = false;     // hipGetSymbolAddress was called for this device
  hipError_t status = hipSuccess;
  void *ptr = nullptr;   // the device address of this device's copy of the array
};

std::mutex g_mu;
Slot g_slots[kMaxDevices];

}  // namespace

int setup(int device) {
  if (device < 0 || device >= kMaxDevices) return -1;
  std::lock_guard<std::mutex> lock(g_mu);
  Slot &s = g_slots[device];
  if (s.done) return s.status == hipSuccess ? 0 : -1;
  void *p = nullptr;
  s.status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (s.status != hipSuccess) (void)hipGetLastError();  // no sticky error for the caller's next call
  s.ptr = s.status == hipSuccess ? p : nullptr;
  s.done = true;
  return s.status == hipSuccess ? 0 : -1;
}

int address(int device, void **out, char *err, size_t errlen) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) {
    snprintf(err, errlen, "device %d is beyond the %d devices the static scratch tracks", device, kMaxDevices);
    return -1;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  const Slot &s = g_slots[device];
  if (!s.done) {
    snprintf(err, errlen, "the static scratch of device %d was not set up (no mtk_init on it)", device);
    return -1;
  }
  if (s.status != hipSuccess || !s.ptr) {
    snprintf(err, errlen, "hipGetSymbolAddress of the static scratch failed on device %d: %s", device,
             hipGetErrorString(s.status));
    return -1;
  }
  *out = s.ptr;
  return 0;
}

}  // namespace mtk_scratch
