// The library's own scratch for rmoe_moe_block_noalloc: callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops)
// get the block's workspace from a file-scope device array instead of a
// caller-provided buffer.
//
// Each GPU the library runs on holds one copy of the array, at its own
// address, until the process ends.  Host code never uses the array's name
// as an address (in host code it names a host-side stand-in): the device
// address comes from hipGetSymbolAddress, once per device with that device
// current, and is kept per device.  Static storage starts zero-filled, which
// is the state a fresh workspace must have; the kernels leave their
// counters at zero when a call completes, and the hand-over words carry
// per-call tags, so every later call finds the array in a valid state.
// Calls that overlap on one GPU share the array and race.
#include <mutex>

#include "kernels.h"

namespace rmoe {

namespace {

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];  // device address of `scratch`, per device

// Copies the status word into the caller's output (when given) and clears
// it, so that each call reports its own outcome (the word is sticky
// otherwise).
__global__ void take_status_kernel(uint32_t* word, uint32_t* out) {
  if (threadIdx.x == 0) {
    if (out) *out = *word;
    *word = 0u;
  }
}

}  // namespace

hipError_t static_scratch(hipStream_t stream, void** out) {
  // the copy of the device the stream runs on, resolved with that device
  // current
  int dev = 0, cur = 0;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return hipSuccess;
}

hipError_t launch_take_status(uint32_t* word, uint32_t* out, hipStream_t s) {
  hipLaunchKernelGGL(take_status_kernel, dim3(1), dim3(64), 0, s, word, out);
  return hipGetLastError();
}

}  // namespace rmoe
