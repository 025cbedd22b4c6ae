// The fixed scratch array of kdn_delta_scan_fwd_noalloc, in a translation unit of its own with no kernels:
// its code object (and with it the array's KDN_NOALLOC_SCRATCH_BYTES of device memory) is loaded on a GPU
// only when the array's address is first looked up there, that is on the first noalloc call on that
// device, not when any scan kernel loads.
//
// In host code the name `scratch` is only a host-side stand-in: its device address (one copy per GPU) is
// looked up with hipGetSymbolAddress, with that device current, and every use goes through that address.
#include <hip/hip_runtime.h>
#include <mutex>
#include "kdn_internal.hpp"

namespace kdn {

static __device__ __align__(256) unsigned char scratch[KDN_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES] = {};

int noalloc_scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return KDN_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return KDN_ERR_DEVICE;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KDN_OK;
}

}  // namespace kdn
