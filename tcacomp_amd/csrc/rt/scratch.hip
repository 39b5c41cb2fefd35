// scratch.hip — the device-resident scratch buffer behind
// tca_program_launch_noalloc: a file-scope device array that the HIP runtime
// places in device memory when this library's code object is loaded on a
// GPU, so launches that use it allocate nothing.
//
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, taken once per device (with
// that device current) by ScratchInit, and only that address is ever handed
// to kernels. Every GPU holds its own copy at its own address until the
// process ends.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>

#include "scratch.h"

static __device__ __align__(256) unsigned char scratch[tca::rt::kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

}  // namespace

namespace tca {
namespace rt {

hipError_t ScratchInit(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ptr[device] != nullptr) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (p == nullptr) return hipErrorInvalidSymbol;
  g_ptr[device] = p;
  return hipSuccess;
}

void* ScratchPtr(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  return g_ptr[device];
}

}  // namespace rt
}  // namespace tca
