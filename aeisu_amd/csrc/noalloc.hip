// Static device scratch for the allocation-free entry point (aeisu_upscale_noalloc).
//
// The default frame path needs device memory beyond its inputs, outputs and weights: the FP16 work
// tensor between the fused body and the fused refine + tail + head kernel (and, for the FP16 policy,
// the skip tensor the project kernel writes), plus the non-finite flag.  aeisu_upscale_async takes
// them from buffers allocated by aeisu_configure; the allocation-free variant takes them from this
// file-scope array, so a caller that cannot allocate (code under HIP graph capture, tight serving
// loops) needs only the weights uploaded by aeisu_create_*.
//
// `scratch` names a host-side stand-in in host code; the array's device address is looked up once
// per device with hipGetSymbolAddress (noalloc_scratch_init, called from the library's create path
// with that device current) and only that address is handed to kernels.  Every GPU holds its own
// copy for the life of the process; calls that overlap on one GPU share it and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kernels.hpp"

namespace aeisu {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];
}  // namespace

hipError_t noalloc_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_ptr[device]) return hipSuccess;
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return e;
  if (current != device) return hipErrorInvalidDevice;   // the caller makes `device` current
  void* ptr = nullptr;
  e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  g_ptr[device] = ptr;
  return hipSuccess;
}

void* noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  return g_ptr[device];
}

}  // namespace aeisu
