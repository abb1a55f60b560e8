// scratch.hip -- the device-resident scratch array behind fa_decode_noalloc.
//
// fa_decode splits a long KV cache across workgroups and merges the splits' fp32 partial O and LSE
// in a second kernel; those partials live in a caller-provided workspace. Callers that cannot
// allocate (code under HIP graph capture, serving loops that forbid hipMalloc) use
// fa_decode_noalloc instead, whose partials live here: one fixed array in the code object, which
// the loader places in each GPU's memory when the library's code is loaded there and which stays
// until the process ends.
//
// In host code the name `scratch` is a host-side shadow symbol, not a device address; the device
// address of each GPU's copy comes from hipGetSymbolAddress, looked up once per device (with that
// device current) and cached. Only that address is ever handed to a kernel.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

#include "fa_internal.h"

namespace fa {
namespace {

static_assert(FA_DECODE_SCRATCH_BYTES % 256 == 0, "the scratch size is a whole number of 256 B");

static __device__ __align__(256) unsigned char scratch[FA_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
// Device address of `scratch` on each device (0 = not looked up yet).
std::atomic<std::uintptr_t> g_scratch_addr[kMaxDevices];

}  // namespace

int decode_scratch(void** out) {
  if (out == nullptr) return static_cast<int>(hipErrorInvalidValue);
  int dev = 0;
  FA_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  std::uintptr_t addr = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (addr == 0) {
    // First call on this device: resolve this device's copy (the current device is `dev`).
    void* p = nullptr;
    FA_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
    addr = reinterpret_cast<std::uintptr_t>(p);
    // Concurrent first calls resolve the same address; whichever store lands is correct.
    g_scratch_addr[dev].store(addr, std::memory_order_release);
  }
  *out = reinterpret_cast<void*>(addr);
  return static_cast<int>(hipSuccess);
}

}  // namespace fa
