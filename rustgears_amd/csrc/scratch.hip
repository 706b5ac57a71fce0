// scratch.hip -- device memory of rgnpu_program_run_device_noalloc.
//
// Callers that cannot allocate device memory (code under HIP graph capture,
// serving loops that must not call hipMalloc) run a program through that
// entry point; every intermediate buffer of such a run -- activations
// between ops, the i8 / binary16 GEMM operands, absmax slots, scales,
// coverage masks, split-K partial sums -- is a view into `scratch`, one
// file-scope array per device, which lives until the process ends.
//
// In host code `scratch` names a host-side stand-in, not the device copy:
// the address kernels and copies use is the one hipGetSymbolAddress returns
// with the device current, looked up once per device and cached here.
#include <hip/hip_runtime.h>

#include <mutex>

#include "rgnpu_internal.h"

namespace rgnpu {

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];
}  // namespace

hipError_t scratch_address(int device, void** out) {
  if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

}  // namespace rgnpu
