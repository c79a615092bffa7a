// The device scratch of dh_gemm_nt_noalloc: a file-scope device array that
// every GPU the library runs on holds from the library's first context on
// that GPU until the process ends, so that entry point never allocates.
//
// In host code `scratch` names a host-side stand-in, not device memory: the
// only way to its device address is hipGetSymbolAddress, called once per
// device (with that device current) by noalloc_scratch below, from
// dh_ctx_create. Everything else uses the pointer it returns.
#include <hip/hip_runtime.h>

#include <mutex>

#include "dh_kernels.h"

namespace dh {

static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_lock;
float* g_ptr[kMaxDevices] = {};
}  // namespace

hipError_t noalloc_scratch(int device, float** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_lock);
  if (!g_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_ptr[device] = (float*)p;
  }
  *out = g_ptr[device];
  return hipSuccess;
}

}  // namespace dh
