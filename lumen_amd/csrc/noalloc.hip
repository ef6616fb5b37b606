// Scratch memory of lumen_sampler_sample_batch_noalloc: one file-scope
// device array per GPU, so that entry point never allocates.
//
// In host code `scratch` names a host-side stand-in for the symbol, not a
// device address: its device address on the current GPU comes from
// hipGetSymbolAddress, taken once per device (lumen_sampler_create takes it
// for its device) and kept here. Every use passes that address.
#include <hip/hip_runtime.h>

#include <mutex>

#include "noalloc.h"

namespace {

static __device__ __align__(256) unsigned char scratch[lumen::kNoAllocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];

}  // namespace

namespace lumen {

// The scratch array's device address on the current device (taken once per
// device). Returns hipSuccess or the error of hipGetSymbolAddress.
hipError_t noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return hipSuccess;
}

}  // namespace lumen
