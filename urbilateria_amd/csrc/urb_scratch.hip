// urb_scratch.hip -- the device scratch of the allocation-free layer call
// (urb_moe_forward_noalloc): a file-scope device array each GPU holds for the life of the
// process, resolved to a device address once per device.
#include <hip/hip_runtime.h>

#include <mutex>

#include "urb_kernels.hpp"

namespace urb {

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void* g_ptr[kMaxDevices] = {};
}  // namespace

// The current device's copy of `scratch`.  In host code the array's name is a host-side
// stand-in, not a device address: the address comes from hipGetSymbolAddress, called once per
// device with that device current, and only that address is ever handed to kernels.
hipError_t scratch_region(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return hipSuccess;
}

}  // namespace urb
