// Statically allocated device scratch for fa_paged_decode_noalloc.
//
// Callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc) get the decode split-KV
// workspace (partial O, partial LSE, the split used) from a file-scope
// device array instead of a caller-provided buffer.  Each GPU the library
// runs on holds its own copy of the array, at its own address, until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the symbol); the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
#include <hip/hip_runtime.h>

#include <mutex>

#include "fa355.h"
#include "fa_internal.h"

namespace fa {

static __device__ __align__(256) char scratch[FA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];
}  // namespace

hipError_t noalloc_scratch(void** ptr) {
  *ptr = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(g_once[dev], [dev] {
    void* p = nullptr;
    g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
  });
  *ptr = g_ptr[dev];
  return g_err[dev];
}

}  // namespace fa
